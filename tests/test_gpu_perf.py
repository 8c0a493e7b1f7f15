"""Performance assertions of the reference's test suite, restated for this build.

* The multi-token tile16 GEMM must sustain at least 1.25x the bandwidth of the
  reference-layout MARLIN kernel at M = 8 and 16 rows (the reference's
  "MARLIN beats naive Q4 by >= 1.25x in tree regimes",
  tests/test_phase1_task13_bandwidth_saturation.py:42-85: N = K = 2048, pools of 16
  weight copies, 5 trials of 8 calls).
* Tree verification must scale sub-linearly: t(N) / N < 0.6 for N = 4, 8, 16 with
  t(N) = latency(forward_tree_verify over N nodes) / latency(one node), on the
  reference's 4-layer model (tests/test_phase2_task21_verification_latency.py:133-209).
* The runner's one-launch step (its captured graph, the reference's single command
  buffer) must cost at most 1 / 1.2 of the host dispatch time of the same step issued
  kernel by kernel (tests/test_phase1_task14_single_command_buffer.py:136-173: "CPU
  dispatch overhead").  The host time of one call is measured with the device idle
  before it; the device time of these small steps is the same in both modes.
"""
import time

import numpy as np
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu


def _median_call_us(fn, pool, steps_per_trial=8, num_trials=5):
    """Median over trials of the mean device time of one call, each trial a replay of one
    captured graph of max(steps_per_trial, len(pool)) back-to-back calls rotating over the
    pool (the reference's run_latency_trials, with the host dispatch cost taken out: these
    launches take a few microseconds, less than the Python wrappers' dispatch)."""
    n_calls = max(steps_per_trial, len(pool))
    for i in range(3):
        fn(pool[i % len(pool)])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_calls):
            fn(pool[i % len(pool)])
    graph.replay()
    torch.cuda.synchronize()
    trials = []
    for _ in range(num_trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        trials.append(e0.elapsed_time(e1) * 1000.0 / n_calls)
    return sorted(trials)[num_trials // 2]


def test_tile16_gemm_bandwidth_over_marlin_layout(dev):
    from axiomlm_amd.kernels import pack_linear_q4_marlin, qmm_q4_tile16, qmv_q4_marlin, repack_q4_marlin_tile16

    N = K = 2048
    g = torch.Generator(device=dev)
    g.manual_seed(2026)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
    pm, sbm = pack_linear_q4_marlin(w, clip_search=False)
    w16, sb16 = repack_q4_marlin_tile16(pm, sbm, N, K)
    pool_marlin = [(pm.clone(), sbm.clone()) for _ in range(16)]
    pool_t16 = [(w16.clone(), sb16.clone()) for _ in range(16)]
    weight_bytes = N * (K // 2) + N * (K // 64) * 4
    for M in (8, 16):
        print(f"[perf_bandwidth] M={M} N={N} K={K}", flush=True)
        x = torch.randn(1, M, K, generator=g, device=dev).half()
        total = weight_bytes + M * K * 2 + M * N * 2
        t_marlin = _median_call_us(lambda ws: qmv_q4_marlin(x, ws[0], ws[1], N), pool_marlin)
        t_t16 = _median_call_us(lambda ws: qmm_q4_tile16(x, ws[0], ws[1], N), pool_t16)
        bw_marlin = total / (t_marlin * 1e-6) / 1e9
        bw_t16 = total / (t_t16 * 1e-6) / 1e9
        print(f"[perf_bandwidth] M={M}: MARLIN layout {t_marlin:.2f} us ({bw_marlin:.0f} GB/s), tile16 GEMM "
              f"{t_t16:.2f} us ({bw_t16:.0f} GB/s)", flush=True)
        # Same product (the GEMM is checked against the oracle elsewhere): the two layouts agree.
        a = qmv_q4_marlin(x, pm, sbm, N).float()
        b = qmm_q4_tile16(x, w16, sb16, N).float()
        assert torch.allclose(a, b, atol=2e-2, rtol=2e-2)
        assert bw_t16 > 1.25 * bw_marlin, f"M={M}: {bw_t16:.1f} GB/s vs {bw_marlin:.1f} GB/s"


def _model4(dev):
    """The reference's 4-layer latency model (8 heads, GQA 4:1, d 512, SwiGLU 1024, vocab
    1024), Q4 MARLIN, with a 256-slot cache."""
    from axiomlm_amd.cache import StaticKVCache
    from axiomlm_amd.transformer import ModelConfig, Transformer

    c = om.OracleConfig(n_layer=4, n_head=8, n_kv_head=2, d_model=512, hidden=1024, vocab=1024, eps=1e-5,
                        block_size=256)
    W = om.make_float_weights(c, seed=3)
    sd = {"transformer.wte.weight": W["wte"], "lm_head.weight": W["lm_head"], "transformer.ln_f.weight": W["lnf"]}
    for i, lw in enumerate(W["layers"]):
        pre = f"transformer.h.{i}."
        for k_sd, k_w in (("ln_1.weight", "ln1"), ("ln_2.weight", "ln2"), ("attn.c_attn.weight", "c_attn"),
                          ("attn.c_proj.weight", "c_proj"), ("mlp.w_gate.weight", "w_gate"),
                          ("mlp.w_up.weight", "w_up"), ("mlp.w_down.weight", "w_down")):
            sd[pre + k_sd] = lw[k_w]
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}
    cfg = ModelConfig(block_size=c.block_size, vocab_size=c.vocab, n_layer=c.n_layer, n_head=c.n_head,
                      n_embd=c.d_model, n_kv_head=c.n_kv_head, intermediate_size=c.hidden, rms_norm_eps=c.eps,
                      tie_word_embeddings=False)
    model = Transformer(cfg, sd, device=dev).quantize("q4")
    cache = StaticKVCache(1, 256, cfg.n_layer, cfg.kv_heads, cfg.head_dim, device=dev)
    return model, cfg, cache


def test_tree_verify_latency_is_sublinear(dev):
    from axiomlm_amd.tree import build_candidate_tree

    print("[perf_tree_sublinear]", flush=True)
    model, cfg, cache = _model4(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1337)
    prefix = torch.randint(0, cfg.vocab_size, (1, 32), generator=g, device=dev)
    model.forward(prefix, kv_caches=cache)
    lat = {}
    for n in (1, 4, 8, 16):
        depths, masks = build_candidate_tree(n)
        cand = torch.randint(0, cfg.vocab_size, (1, n), generator=g, device=dev)
        for _ in range(3):
            model.forward_tree_verify(cand, cache, depths, masks, return_medusa=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            model.forward_tree_verify(cand, cache, depths, masks, return_medusa=False)
        e1.record()
        torch.cuda.synchronize()
        lat[n] = e0.elapsed_time(e1) / 10.0
    print("[perf_tree_sublinear] latency ms " + " ".join(f"N={n}: {v:.3f}" for n, v in lat.items()), flush=True)
    # The tree slots lie past the prefix: the verify calls leave the counters alone.
    assert cache.total_seen_tokens == [32] * cfg.n_layer
    for n in (4, 8, 16):
        t_n = lat[n] / lat[1]
        assert t_n / n < 0.60, f"t({n}) / {n} = {t_n / n:.3f}"


def test_runner_graph_dispatch_faster_than_eager(dev):
    print("[perf_dispatch]", flush=True)
    model, cfg, cache = _model4(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    model.forward(torch.randint(0, cfg.vocab_size, (1, 32), generator=g, device=dev), kv_caches=cache)
    runner = model.get_decode_runner(cache)
    idx = torch.tensor([55], dtype=torch.int64, device=dev)

    def host_us(n_trials=50):
        """Median host time of one step call, issued onto an idle device."""
        for _ in range(5):
            runner.step(idx, 40, 40, 41)
        times = []
        for _ in range(n_trials):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            runner.step(idx, 40, 40, 41)
            times.append((time.perf_counter() - t0) * 1e6)
        torch.cuda.synchronize()
        return sorted(times)[n_trials // 2]

    try:
        runner.set_mode("graph")
        logits_graph = runner.step(idx, 40, 40, 41).float().clone()
        t_graph = host_us()
        runner.set_mode("eager")
        logits_eager = runner.step(idx, 40, 40, 41).float().clone()
        t_eager = host_us()
    finally:
        runner.set_mode("graph")
    print(f"[perf_dispatch] host dispatch per step: graph {t_graph:.1f} us, eager {t_eager:.1f} us", flush=True)
    assert torch.equal(logits_graph, logits_eager)
    assert t_eager / t_graph >= 1.20, f"{t_eager:.1f} us eager vs {t_graph:.1f} us graph"
