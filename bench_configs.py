"""Measurements of the BASELINE configurations other than the headline decode line.

`bench.py` prints the one JSON line the driver reads (Q4 7B-shape decode tok/s).
This script measures the remaining configurations on one MI355X, one JSON line
per case, each against the HBM roofline (8 TB/s) with its algorithmic bytes:

  c2  single decoder layer at Llama-7B shapes (RMSNorm, QKV, O, gate/up + SwiGLU,
      down; MARLIN Q4 G64 re-tiled for the matrix cores) at M = 1, 4, 16 tokens
  c3  split-K decode attention, B 8, 32 query / 8 KV heads, hd 128, INT4 and FP8
      KV at 1k / 8k / 32k keys, and the 4096-slot ring buffer after 10k tokens
  c4  BitNet ternary, affine 2-bit and GGUF Q2_K GEMVs at the FFN shapes
      (4096 -> 11008, 11008 -> 4096), batch 1 (GGUF also 4 tokens)
  c5  speculative tree verification, 7B shape, FP8 KV, prefix 2048, a 64-node
      tree (depth 6, branching 4,4,2,2,1,1): one runner.verify_tree_step; the
      128-step greedy-acceptance loop (verify, greedy walk, KV compaction) with
      seeded random drafts and with drafts that follow the model's own greedy
      continuation along the first-child chain; this runner's t(N) latency
      profile and the Sequoia tree it selects
  modes  the 7B decode step with q4_k_m, q8 and fp16 weights (the runner's other formats)

Kernels are timed from a captured HIP graph of back-to-back calls (no host
launch gaps), rotating over enough weight / cache copies that the stream does
not sit in the 256 MB last-level cache.  Weights are random-init N(0, 0.02),
activations and KV N(0, 1).

    python bench_configs.py [c2 c3 c4 c5]
"""

from __future__ import annotations

import argparse
import json
import sys
import time

import bench

HBM_PEAK_GBS = bench.HBM_PEAK_GBS
MFMA_PEAK_F16_TFLOPS = 2500.0
COLD_POOL_BYTES = 600 << 20  # > 2x the 256 MB last-level cache


def _graph_time_us(fn, n_calls: int, replays: int = 5) -> float:
    """Average device time of fn(i) over n_calls calls captured in one graph."""
    import torch

    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_calls):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / (replays * n_calls)


def _line(config, case, avg_us, nbytes, extra=None):
    gbs = nbytes / (avg_us * 1e-6) / 1e9
    out = {"config": config, "case": case, "avg_us": round(avg_us, 3), "algorithmic_bytes": int(nbytes),
           "achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if extra:
        out.update(extra)
    print(json.dumps(out), flush=True)


def run_c2(dev):
    import torch

    from axiomlm_amd.kernels import (fused_rmsnorm, pack_linear_q4_marlin, qmv_q4_tile16, qmv_q4_tile16_swiglu,
                                     repack_q4_marlin_tile16)

    c = bench.CFG_7B
    d, H = c["d"], c["hidden"]
    qkv_rows = (c["n_head"] + 2 * c["n_kv_head"]) * c["hd"]
    g = torch.Generator(device=dev)
    g.manual_seed(1)

    def packed(n, k):
        w = (torch.randn(n, k, generator=g, device=dev) * 0.02).half()
        p, s = pack_linear_q4_marlin(w, clip_search=False)
        return repack_q4_marlin_tile16(p, s, n, k)

    layer_bytes = bench.layer_weight_bytes(c)
    n_copies = max(2, COLD_POOL_BYTES // layer_bytes + 1)
    layers = [dict(qkv=packed(qkv_rows, d), o=packed(d, d), gu=packed(2 * H, d), dn=packed(d, H),
                   ln1=(1 + 0.1 * torch.randn(d, generator=g, device=dev)).half(),
                   ln2=(1 + 0.1 * torch.randn(d, generator=g, device=dev)).half()) for _ in range(n_copies)]
    for M in (1, 4, 16):
        x = torch.randn(M, d, generator=g, device=dev).half()

        def layer(i):
            L = layers[i % n_copies]
            xn = fused_rmsnorm(x, L["ln1"], 1e-5)
            q = qmv_q4_tile16(xn, *L["qkv"], qkv_rows)
            o = qmv_q4_tile16(q[:, :d].contiguous(), *L["o"], d)
            h = qmv_q4_tile16_swiglu(x + o, L["ln2"], 1e-5, *L["gu"], H)
            return qmv_q4_tile16(h, *L["dn"], d)

        us = _graph_time_us(layer, 2 * n_copies)
        nbytes = layer_bytes + M * (d + qkv_rows + d + d + d + 2 * H + H + d) * 2
        _line("C2", f"layer M={M}", us, nbytes, {"tokens_per_s_per_layer": round(M / (us * 1e-6), 1),
                                                 "weight_copies": n_copies})


def run_c3(dev):
    import torch

    from axiomlm_amd.kernels import gqa_flash_decode_mps, quantize_kv_fp8, quantize_kv_int4

    B, Hq, Hkv, hd = 8, 32, 8, 128
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    per_key = {"int4": 136, "fp8": 264}
    cases = [(L, L) for L in (1024, 8192, 32768)] + [(4096, "ring")]
    for kind in ("int4", "fp8"):
        quant = quantize_kv_int4 if kind == "int4" else quantize_kv_fp8
        for L, label in cases:
            nbytes = B * Hkv * L * per_key[kind] + 2 * B * Hq * hd * 2
            n_copies = max(1, min(16, COLD_POOL_BYTES // (B * Hkv * L * per_key[kind]) + 1))
            caches = []
            for _ in range(n_copies):
                k = torch.randn(B, Hkv, L, hd, generator=g, device=dev).half()
                v = torch.randn(B, Hkv, L, hd, generator=g, device=dev).half()
                kc, ks, vc, vs = quant(k, v)
                del k, v
                caches.append((kc, vc, ks, vs))
            q = torch.randn(B, Hq, 1, hd, generator=g, device=dev).half()

            def attn(i):
                kc, vc, ks, vs = caches[i % n_copies]
                return gqa_flash_decode_mps(q, kc, vc, L, 0, ks, vs, kind)

            us = _graph_time_us(attn, max(8, 2 * n_copies))
            case = f"{kind} L={L}" if label != "ring" else f"{kind} ring S=4096 after 10k tokens (all slots valid)"
            _line("C3", case, us, nbytes, {"cache_copies": n_copies})
            del caches
            torch.cuda.empty_cache()


def run_c4(dev):
    import torch

    from axiomlm_amd.kernels import pack_linear_q2_k, pack_linear_ternary, qmv_q2_k, qmv_ternary

    g = torch.Generator(device=dev)
    g.manual_seed(0)
    for fmt in ("ternary", "q2"):
        for N, K in ((11008, 4096), (4096, 11008)):
            if fmt == "ternary":
                codes = torch.multinomial(torch.tensor([0.25, 0.5, 0.25], device=dev), N * K, replacement=True,
                                          generator=g).view(N, K).to(torch.float16) - 1
                w = codes * 0.02
                packs = [pack_linear_ternary(w) for _ in range(1)]
                fn, per_w = qmv_ternary, 0.28125
            else:
                w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
                packs = [pack_linear_q2_k(w) for _ in range(1)]
                fn, per_w = qmv_q2_k, 0.3125
            wb = int(N * K * per_w)
            n_copies = max(2, COLD_POOL_BYTES // wb + 1)
            packs = [tuple(t.clone() for t in packs[0]) for _ in range(n_copies)]
            for M in (1, 4):  # one token (the C4 workload), four (the several-token MFMA form)
                x = torch.randn(M, K, generator=g, device=dev).half()

                def gemv(i):
                    p, s = packs[i % n_copies]
                    return fn(x, p, s)

                us = _graph_time_us(gemv, 2 * n_copies)
                _line("C4", f"{fmt} {K}->{N} M={M}", us, wb + M * (K + N) * 2, {"weight_copies": n_copies})
            del packs
            torch.cuda.empty_cache()
    from axiomlm_amd.kernels import pack_linear_q2_k_gguf, qmv_q2_k_gguf

    for N, K in ((11008, 4096), (4096, 11008)):
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
        blocks = pack_linear_q2_k_gguf(w)
        del w
        wb = blocks.numel()  # 84 bytes per 256 weights
        n_copies = max(2, COLD_POOL_BYTES // wb + 1)
        pool = [blocks.clone() for _ in range(n_copies)]
        for M in (1, 4):
            x = torch.randn(M, K, generator=g, device=dev).half()
            us = _graph_time_us(lambda i: qmv_q2_k_gguf(x, pool[i % n_copies]), 2 * n_copies)
            _line("C4", f"GGUF Q2_K {K}->{N} M={M}", us, wb + M * (K + N) * 2, {"weight_copies": n_copies})
        del pool, blocks
        torch.cuda.empty_cache()


def run_c5(dev, quick=False):
    import torch

    from axiomlm_amd.cache import StaticKVCache
    from axiomlm_amd.kernels import pack_linear_q4_marlin, pack_linear_q8_g64, quantize_kv_fp8
    from axiomlm_amd.runner import QuantizedDecodeRunner
    from axiomlm_amd.tree import build_branching_tree

    c = bench.CFG_7B
    d, H, L, hd = c["d"], c["hidden"], c["n_layer"], c["hd"]
    prefix, T, loop_steps = 2048, 64, 128
    S = prefix + loop_steps * 7 + T + 64  # room for 7 tokens per loop step
    g = torch.Generator(device=dev)
    g.manual_seed(0)

    def randn(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * std).half()

    def q4(n, k):
        return pack_linear_q4_marlin(randn(n, k), clip_search=False)

    qkv_rows = (c["n_head"] + 2 * c["n_kv_head"]) * hd
    lay = {k: [] for k in ("ln1", "ln2", "qkv", "o", "gu", "dn")}
    for _ in range(L):
        lay["ln1"].append((1 + randn(d, std=0.1).float()).half())
        lay["ln2"].append((1 + randn(d, std=0.1).float()).half())
        lay["qkv"].append(q4(qkv_rows, d))
        lay["o"].append(q4(d, d))
        lay["gu"].append(q4(2 * H, d))
        lay["dn"].append(q4(d, H))
    lmh_p, lmh_s = q4(c["vocab"], d)
    wte_p, wte_s = pack_linear_q8_g64(randn(c["vocab"], d))
    lnf = (1 + randn(d, std=0.1).float()).half()
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    fr = torch.outer(torch.arange(4 * S, dtype=torch.float32), inv)
    freqs = torch.stack([fr.cos(), fr.sin()], dim=-1).to(dev)
    cache = StaticKVCache(1, S, L, c["n_kv_head"], hd, device=dev, cache_dtype="fp8")
    for li in range(L):
        k = torch.randn(1, c["n_kv_head"], S, hd, generator=g, device=dev).half()
        v = torch.randn(1, c["n_kv_head"], S, hd, generator=g, device=dev).half()
        kc, ks, vc, vs = quantize_kv_fp8(k, v)
        cache.cache[li, 0].copy_(kc)
        cache.cache[li, 1].copy_(vc)
        cache.scales[li, 0].copy_(ks)
        cache.scales[li, 1].copy_(vs)
    runner = QuantizedDecodeRunner(
        None, lmh_p, lmh_s, freqs, lay["ln1"], [p for p, _ in lay["qkv"]], [s for _, s in lay["qkv"]],
        [p for p, _ in lay["o"]], [s for _, s in lay["o"]], lay["ln2"], [p for p, _ in lay["gu"]],
        [s for _, s in lay["gu"]], [p for p, _ in lay["dn"]], [s for _, s in lay["dn"]], lnf, cache.k_caches,
        cache.v_caches, c["n_head"], c["n_kv_head"], hd, True, 1e-5, [], c["vocab"], wte_p=wte_p, wte_s=wte_s,
        k_scales=cache.k_scales, v_scales=cache.v_scales, kv_dtype="fp8", max_tokens=T)
    tree = build_branching_tree([4, 4, 2, 2, 1, 1], max_nodes=T)
    assert tree["num_nodes"] == T
    toks = torch.randint(0, c["vocab"], (1, T), generator=g, device=dev)
    depths, masks = tree["tree_depths"], tree["tree_mask"]

    def verify():
        return runner.verify_tree_step(toks, prefix, prefix, prefix, depths, masks)

    for _ in range(3):
        verify()
    torch.cuda.synchronize()
    reps = 10
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        verify()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps
    us = e0.elapsed_time(e1) * 1000.0 / reps
    w_bytes = L * bench.layer_weight_bytes(c) + bench.q4_bytes(c["vocab"], d)
    kv_bytes = L * 2 * c["n_kv_head"] * (prefix + T) * (hd + 2 * (hd // 64))
    flops = 2.0 * T * (L * (qkv_rows * d + d * d + 2 * H * d + d * H) + c["vocab"] * d)
    _line("C5", f"verify_tree_step T={T} prefix={prefix} fp8 KV", us, w_bytes + kv_bytes,
          {"mfma_frac_f16": round(flops / (us * 1e-6) / 1e12 / MFMA_PEAK_F16_TFLOPS, 4),
           "tree_nodes_per_s": round(T / (us * 1e-6), 1), "host_wall_us": round(wall * 1e6, 1)})
    if not quick:
        _c5_loops(runner, cache, tree, prefix, loop_steps, c["vocab"], dev, g)


def _loop_line(case, T, r, cont):
    n_tok = len(r["tokens"])
    match = sum(int(a == b) for a, b in zip(r["tokens"], cont))
    print(json.dumps({"config": "C5", "case": case, "tree_nodes": T, "steps": r["model_calls"], "tokens": n_tok,
                      "mean_accepted_per_step": round(sum(r["accepted"]) / len(r["accepted"]), 3),
                      "ms_per_step": round(r["seconds"] * 1e3 / r["model_calls"], 3),
                      "tokens_per_s": round(n_tok / r["seconds"], 1),
                      "tokens_equal_to_reference_continuation": f"{match}/{n_tok}"}), flush=True)


def _c5_loops(runner, cache, tree, prefix, n_steps, vocab, dev, g):
    """The 128-step tree loop of medusa.py:278-363 (greedy acceptance) on the C5 model, then
    the runner's t(N) profile and the Sequoia tree chosen with it."""
    import torch

    from axiomlm_amd.sequoia import SequoiaDPOptimizer, measure_tree_latency
    from axiomlm_amd.speculative import tree_decode_greedy

    T = tree["num_nodes"]
    chain = []
    u = 0
    while tree["children"][u]:
        u = tree["children"][u][0]
        chain.append(u)
    root = int(torch.randint(0, vocab, (1,), generator=g, device=dev))
    rng = torch.Generator().manual_seed(1)

    def reset():
        cache.total_seen_tokens[:] = [prefix] * cache.n_layer
        cache.layer_seq_lens[:] = [prefix] * cache.n_layer

    def random_draft(step, last, seen):
        return torch.randint(0, vocab, (T - 1,), generator=rng).tolist()

    # Random drafts are never accepted, so this run emits the model's greedy continuation
    # one token per step, computed by the same verify path as the loop below.
    reset()
    tree_decode_greedy(runner, cache, root, tree, random_draft, 2)  # warm-up
    reset()
    n_ref = n_steps * (len(chain) + 1)
    r = tree_decode_greedy(runner, cache, root, tree, random_draft, n_ref)
    cont = r["tokens"]  # cont[i] = greedy token at position prefix + 1 + i
    _loop_line(f"{n_ref}-step tree loop, seeded random drafts", T, r, cont)

    def chain_draft(step, last, seen):
        nodes = torch.randint(0, vocab, (T,), generator=rng).tolist()
        for k, node in enumerate(chain, start=1):
            i = seen - prefix + k - 1
            nodes[node] = cont[i] if i < len(cont) else 0
        return nodes[1:]

    reset()
    r = tree_decode_greedy(runner, cache, root, tree, chain_draft, n_steps)
    _loop_line(f"{n_steps}-step tree loop, drafts = the greedy continuation on the first-child chain", T, r, cont)
    reset()
    prof = measure_tree_latency(runner, cache, budgets=(2, 3, 4, 6, 8, 16, 24, 32, 48, 64))
    opt = SequoiaDPOptimizer(num_heads=6, max_branches=4, max_budget=64, latency_profile=prof)
    res = opt.solve_optimal_tree()
    print(json.dumps({"config": "C5", "case": "t(N) = verify_tree_step(N) / step, 7B Q4 FP8 prefix 2048",
                      "t_of_N": prof, "sequoia_N": res.optimal_N, "sequoia_depth": res.max_depth,
                      "sequoia_expected_tokens": res.expected_accepted_tokens,
                      "sequoia_speedup": res.speedup}), flush=True)


def run_modes(dev):
    """The 7B decode step in the runner's other weight formats: "q4_k_m" (MARLIN Q4 with Q8_G64
    w_down and lm_head), "q8" (Q8_G64 everywhere) and the fp16 runner (every matrix fp16),
    fp16 KV cache, context 128; tokens fed from device memory (no greedy feedback, which
    needs the MARLIN lm_head)."""
    import torch

    from axiomlm_amd.cache import StaticKVCache
    from axiomlm_amd.kernels import pack_linear_q4_marlin, pack_linear_q8_g64
    from axiomlm_amd.runner import DecodeRunner, QuantizedDecodeRunner

    c = bench.CFG_7B
    d, H, L, hd, V = c["d"], c["hidden"], c["n_layer"], c["hd"], c["vocab"]
    qkv_rows = (c["n_head"] + 2 * c["n_kv_head"]) * hd
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    fr = torch.outer(torch.arange(bench.MAX_SEQ * 4, dtype=torch.float32), inv)
    freqs = torch.stack([fr.cos(), fr.sin()], dim=-1).to(dev)
    shapes = {"qkv": (qkv_rows, d), "o": (d, d), "gu": (2 * H, d), "dn": (d, H)}
    bpw = {"q4": 0.5625, "q8": 1.0625, "fp16": 2.0}
    for mode in ("q4_k_m", "q8", "fp16"):
        g = torch.Generator(device=dev)
        g.manual_seed(0)

        def randn(*shape, std=0.02):
            return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std).to(torch.float16)

        def fmt_of(kind):
            if mode == "fp16":
                return "fp16"
            return "q8" if (mode == "q8" or kind in ("dn", "lm")) else "q4"

        def pack(kind, rows, k):
            w = randn(rows, k)
            f = fmt_of(kind)
            if f == "fp16":
                return w, None
            return pack_linear_q8_g64(w) if f == "q8" else pack_linear_q4_marlin(w, clip_search=False)

        lay = {k: [] for k in ("ln1", "ln2", "qkv", "o", "gu", "dn")}
        for _ in range(L):
            lay["ln1"].append((1 + randn(d, std=0.1).float()).half())
            lay["ln2"].append((1 + randn(d, std=0.1).float()).half())
            for k, (n, kk) in shapes.items():
                lay[k].append(pack(k, n, kk))
        lnf = (1 + randn(d, std=0.1).float()).half()
        cache = StaticKVCache(1, bench.MAX_SEQ, L, c["n_kv_head"], hd, device=dev)
        cache.cache.normal_(generator=g)
        P = lambda k: [p for p, _ in lay[k]]  # noqa: E731
        S = lambda k: [s for _, s in lay[k]]  # noqa: E731
        if mode == "fp16":
            wte = randn(V, d)
            runner = DecodeRunner(wte, freqs, lay["ln1"], P("qkv"), P("o"), lay["ln2"], P("gu"), P("dn"), lnf,
                                  cache.k_caches, cache.v_caches, c["n_head"], c["n_kv_head"], hd, 1e-5,
                                  lm_head_w=randn(V, d))
        else:
            lmh_p, lmh_s = pack("lm", V, d)
            wte_p, wte_s = pack_linear_q8_g64(randn(V, d))
            runner = QuantizedDecodeRunner(None, lmh_p, lmh_s, freqs, lay["ln1"], P("qkv"), S("qkv"), P("o"), S("o"),
                                           lay["ln2"], P("gu"), S("gu"), P("dn"), S("dn"), lnf, cache.k_caches,
                                           cache.v_caches, c["n_head"], c["n_kv_head"], hd, mode != "q8", 1e-5, [],
                                           V, wte_p=wte_p, wte_s=wte_s)
        tok = torch.zeros((1, 1), dtype=torch.int64, device=dev)
        pos = bench.CTX0
        for i in range(10):
            runner.step(tok, pos + i, pos + i, pos + i + 1)
        torch.cuda.synchronize()
        steps = 100
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            p = pos + 10 + i
            runner.step(tok, p, p, p + 1)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        w_bytes = sum(L * n * kk * bpw[fmt_of(k)] for k, (n, kk) in shapes.items()) + V * d * bpw[fmt_of("lm")]
        active = pos + 10 + steps // 2
        b = w_bytes + L * 2 * c["n_kv_head"] * active * hd * 2
        print(json.dumps({"config": "modes", "case": f"7B decode, {mode} weights ({runner.layer_formats})",
                          "ms_per_token": round(ms, 4), "tokens_per_s": round(1000.0 / ms, 1),
                          "algorithmic_bytes_per_token": int(b),
                          "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)
        del runner, cache, lay
        torch.cuda.empty_cache()


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("configs", nargs="*", default=["c2", "c3", "c4", "c5"])
    ap.add_argument("--quick", action="store_true",
                    help="c5: time the single verify step only (short runs under counter collection)")
    args = ap.parse_args()
    import torch

    dev = torch.device("cuda", 0)
    runs = {"c2": run_c2, "c3": run_c3, "c4": run_c4, "c5": run_c5, "modes": run_modes}
    for name in args.configs:
        if name not in runs:
            sys.exit(f"unknown config {name!r}; choose from {sorted(runs)}")
        print(f"[bench_configs] {name}", file=sys.stderr, flush=True)
        runs[name](dev, quick=args.quick) if name == "c5" else runs[name](dev)
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
