"""Benchmark: Q4 7B-shape batch-1 decode on one MI355X.

Workload (BASELINE.json metric "Q4 7B-shape decode tok/s (bs=1, 1 GPU); achieved
HBM GB/s as % of peak", on the configuration it names: Q4 MARLIN-interleaved
weights of group 128 with fp16 scales): a Llama-7B-shape decoder (32 layers,
d 4096, 32 heads x 128, SwiGLU 11008, vocab 32000) with random-init N(0, 0.02)
weights packed to MARLIN Q4 group 128 (one fp16 scale + bias per 128 columns,
round-to-nearest), a Q8_G64 embedding table, an fp16 KV cache of 4096 slots whose
first CTX0 slots hold synthetic N(0,1) context.  One step = one greedy decode token
through the captured whole-step hipGraph (the argmax of step t feeds step t+1 on
the device).

Printed JSON line: value = tokens/s; roofline = the runner's fused RMSNorm +
gate/up GEMV + SwiGLU kernel (tile16 matrix-core layout; the largest per-launch
weight stream, 47.6 MB at group 128) timed live with HIP events on its stream, beside
its average inside the decode graph from the committed rocprofv3 summary;
decode_kernels = every launch group of the step (QKV, attention, O, gate/up, down,
lm_head) timed the same way, with its algorithmic bytes and fraction of the peak;
cpu_baseline = the reference's CPU path restated with torch on the host cores
(dequantize every weight on every call, then F.linear in fp16) on a bounded sample
of the same step, extrapolated to tokens/s, plus C1 end to end and a C2 layer on the
CPU (group-64 packs: the reference's CPU dequantizer has no other group size);
group64_decode = the same decode with the reference's own group-64 packs (0.56
instead of 0.53 bytes per weight), reported beside the headline.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
CFG_7B = dict(n_layer=32, d=4096, n_head=32, n_kv_head=32, hd=128, hidden=11008, vocab=32000)
CTX0 = 128
MAX_SEQ = 4096
HEADLINE_GROUP = 128  # BASELINE configs[1] / north_star: MARLIN Q4, group 128, fp16 scales
def q4_bytes(n_rows: int, k: int, group: int = 64) -> int:
    """MARLIN Q4 bytes: group/2 bytes of nibbles + an fp16 (scale, bias) pair per group."""
    return ((n_rows + 7) // 8) * 8 * (k // group) * (group // 2 + 4)


def layer_weight_bytes(c, group: int = 64) -> int:
    qkv = (c["n_head"] + 2 * c["n_kv_head"]) * c["hd"]
    return (q4_bytes(qkv, c["d"], group) + q4_bytes(c["d"], c["n_head"] * c["hd"], group)
            + q4_bytes(2 * c["hidden"], c["d"], group) + q4_bytes(c["d"], c["hidden"], group))


def step_bytes(c, active_len: int, group: int = 64) -> int:
    """Algorithmic HBM bytes of one decode token at context `active_len` (weights once,
    KV prefix once, embedding row, plus the small activation vectors)."""
    w = c["n_layer"] * layer_weight_bytes(c, group) + q4_bytes(c["vocab"], c["d"], group)
    kv = c["n_layer"] * 2 * c["n_kv_head"] * active_len * c["hd"] * 2
    emb = c["d"] + (c["d"] // 64) * 4
    return w + kv + emb


def build_model(c, dev, seed=0, group_size=64):
    import torch

    from axiomlm_amd.cache import StaticKVCache
    from axiomlm_amd.kernels import pack_linear_q4_marlin, pack_linear_q8_g64
    from axiomlm_amd.runner import QuantizedDecodeRunner

    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def randn(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std).to(torch.float16)

    def q4(rows, k):
        w = randn(rows, k)
        p = pack_linear_q4_marlin(w, clip_search=False, group_size=group_size)
        del w
        return p

    d, H = c["d"], c["hidden"]
    qkv_rows = (c["n_head"] + 2 * c["n_kv_head"]) * c["hd"]
    L = c["n_layer"]
    layers = {k: [] for k in ("ln1", "ln2", "qkv_p", "qkv_s", "o_p", "o_s", "gu_p", "gu_s", "dn_p", "dn_s")}
    for _ in range(L):
        layers["ln1"].append((1 + randn(d, std=0.1).float()).half())
        layers["ln2"].append((1 + randn(d, std=0.1).float()).half())
        p, s = q4(qkv_rows, d)
        layers["qkv_p"].append(p)
        layers["qkv_s"].append(s)
        p, s = q4(d, c["n_head"] * c["hd"])
        layers["o_p"].append(p)
        layers["o_s"].append(s)
        p, s = q4(2 * H, d)
        layers["gu_p"].append(p)
        layers["gu_s"].append(s)
        p, s = q4(d, H)
        layers["dn_p"].append(p)
        layers["dn_s"].append(s)
    lmh_p, lmh_s = q4(c["vocab"], d)
    wte_p, wte_s = pack_linear_q8_g64(randn(c["vocab"], d))
    lnf = (1 + randn(d, std=0.1).float()).half()
    inv = 1.0 / (10000.0 ** (torch.arange(0, c["hd"], 2, dtype=torch.float32) / c["hd"]))
    fr = torch.outer(torch.arange(MAX_SEQ * 4, dtype=torch.float32), inv)
    freqs = torch.stack([fr.cos(), fr.sin()], dim=-1).to(dev)
    cache = StaticKVCache(1, MAX_SEQ, L, c["n_kv_head"], c["hd"], device=dev)
    cache.cache.normal_(generator=g)  # synthetic context for the first CTX0 slots (and beyond)
    runner = QuantizedDecodeRunner(
        None, lmh_p, lmh_s, freqs, layers["ln1"], layers["qkv_p"], layers["qkv_s"], layers["o_p"], layers["o_s"],
        layers["ln2"], layers["gu_p"], layers["gu_s"], layers["dn_p"], layers["dn_s"], lnf, cache.k_caches,
        cache.v_caches, c["n_head"], c["n_kv_head"], c["hd"], True, 1e-5, [], c["vocab"], wte_p=wte_p, wte_s=wte_s)
    return runner, cache, layers, lnf


def set_mode(runner, mode: str) -> str:
    """Select the step execution ("graph" or "persistent")."""
    runner.set_mode(mode)
    return runner.mode


def time_decode(runner, cache, steps, warmup, dev, ctx0=CTX0):
    """Greedy decode: argmax of step t (device) is the token of step t+1."""
    import torch

    pos = ctx0
    runner.step(torch.zeros(1, dtype=torch.int64, device=dev), pos - 1, pos - 1, pos)

    def one(p):
        runner.step_greedy(p, p, p + 1)

    for i in range(warmup):
        one(pos + i)
    torch.cuda.synchronize()
    pos0 = pos + warmup
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        one(pos0 + i)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop)
    return ms, wall, pos0


KERNEL_NAMES = {
    "qkv": "t16_gemv_kernel<1,1,3,12,2,G128,256>: RMSNorm + QKV Q4 GEMV + RoPE + fp16 KV slot write",
    "attention": "attn_split_kernel<0,1,false,4,4>: split-KV flash decode, partials for the O projection",
    "o": "t16_gemv_kernel<1,1,16,12,2,G128,512>: O Q4 GEMV merging the attention partials + residual",
    "gate_up": "t16_gemv_kernel<1,2,2,12,2,G128,256>: RMSNorm + gate|up Q4 GEMV + SwiGLU",
    "down": "t16_gemv_kernel<1,1,1,12,2,G128,512>: down Q4 GEMV + residual",
    "lm_head": "t16_gemv_kernel<1,1,0,12,2,G128,512>: final RMSNorm + lm_head Q4 GEMV + argmax keys",
}


def kernel_bytes(c, active_len: int, group: int) -> dict:
    """Algorithmic HBM bytes of each launch group of one decode token (one layer's kernel;
    the lm_head once): every weight byte (codes + scale + bias) once, the KV prefix once,
    the activation vectors read and written.  The attention split partials are this
    build's intermediate and not counted."""
    d, H, hd = c["d"], c["hidden"], c["hd"]
    qd, kvd = c["n_head"] * hd, c["n_kv_head"] * hd
    return {
        "qkv": q4_bytes(qd + 2 * kvd, d, group) + 2 * d * 2 + (qd + 2 * kvd) * 2,
        "attention": 2 * c["n_kv_head"] * active_len * hd * 2 + qd * 2 + qd * 2,
        "o": q4_bytes(d, qd, group) + qd * 2 + 2 * d * 2,
        "gate_up": q4_bytes(2 * H, d, group) + 2 * d * 2 + H * 2,
        "down": q4_bytes(d, H, group) + H * 2 + 2 * d * 2,
        "lm_head": q4_bytes(c["vocab"], d, group) + 2 * d * 2 + c["vocab"] * 2 + d * 2,
    }


def time_step_kernels(runner, c, position: int, active_len: int, group: int, reps: int = 200) -> dict:
    """Each launch group of the decode step timed live with HIP events on the runner's stream
    (QuantizedDecodeRunner.time_kernels: the runner's own launches, `reps` back to back over
    the 32 layers' weights in turn, 3.6 GB, past the 256 MB last-level cache, replayed as one
    captured graph), with its algorithmic bytes and fraction of the HBM peak."""
    us = runner.time_kernels(position, active_len, reps)
    nb = kernel_bytes(c, active_len, group)
    out = {}
    for k, t in us.items():
        gbs = nb[k] / (t * 1e-6) / 1e9
        out[k] = {"kernel": KERNEL_NAMES[k].replace("G128", "true" if group == 128 else "false"),
                  "avg_launch_us": round(t, 3), "algorithmic_bytes": nb[k], "achieved_gbs": round(gbs, 1),
                  "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def in_graph_profile(group=HEADLINE_GROUP):
    """Per-kernel average durations inside the captured decode graph from the committed rocprofv3
    kernel-trace summary (profiles/decode_7b_q4_g128_kernel_stats.json; its fields name the
    command and the commit it was measured at).  None when absent or for group 64."""
    path = os.path.join(ROOT, "profiles", "decode_7b_q4_g128_kernel_stats.json")
    if group != 128 or not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def gate_up_traffic(group=HEADLINE_GROUP):
    """HBM bytes per gate/up launch measured with rocprofv3 FETCH_SIZE and WRITE_SIZE counters
    (profiles/gate_up_g128_traffic.json for group 128, gate_up_traffic.json for group 64,
    written from two counter runs and a copy-kernel calibration; the JSON names the commands
    and the commit).  (bytes, provenance) or (None, None) when absent."""
    path = os.path.join(ROOT, "profiles", "gate_up_g128_traffic.json" if group == 128 else "gate_up_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        j = json.load(f)
    prov = {k: j[k] for k in ("measured_at_commit", "source", "commands") if k in j}
    return j.get("hbm_bytes_per_launch"), prov


# (group, name patterns): the profiler prints some kernels demangled and others (those
# with fp16 pointer arguments) mangled, so each GEMV group carries both forms.
TRACE_GROUPS = (("qkv", ("t16_gemv_kernel<1, 1, 3,", "t16_gemv_kernelILi1ELi1ELi3E")),
                ("attention", ("attn_split_kernel",)),
                ("o", ("t16_gemv_kernel<1, 1, 16,", "t16_gemv_kernelILi1ELi1ELi16E")),
                ("gate_up", ("t16_gemv_kernel<1, 2, 2,", "t16_gemv_kernelILi1ELi2ELi2E")),
                ("down", ("t16_gemv_kernel<1, 1, 1,", "t16_gemv_kernelILi1ELi1ELi1E")),
                ("lm_head", ("t16_gemv_kernel<1, 1, 0,", "t16_gemv_kernelILi1ELi1ELi0E")),
                ("set_params", ("set_params_kernel",)))


def summarize_trace(csv_path: str, n_steps: int, n_layer: int = CFG_7B["n_layer"]) -> dict:
    """In-graph per-kernel averages from a rocprofv3 --kernel-trace CSV of this benchmark: the
    decode steps run first, so each layer kernel's first n_steps * n_layer launches (the lm_head's
    and the parameter kernel's first n_steps) are the graph's; later launches of the same kernels
    are time_kernels' stand-alone ones."""
    import csv

    rows = []
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    out = {}
    for key, pats in TRACE_GROUPS:
        durs = [(e - b) / 1000.0 for b, e, name in rows if any(p in name for p in pats)]
        n = n_steps * (1 if key in ("lm_head", "set_params") else n_layer)
        if len(durs) < n:
            continue
        g = durs[:n]
        out[key] = {"avg_us": round(sum(g) / n, 3), "min_us": round(min(g), 3), "max_us": round(max(g), 3),
                    "calls": n}
    return out


def _cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(layers, lnf, c, budget_s=20.0):
    """The reference's CPU path restated with torch on the host cores (oracle/torch_cpu.py:
    quantized linears dequantize the MARLIN codes to fp16 on every call, then F.linear in
    fp16, as quant.py:656-661 does), torch.set_num_threads = every core this process may use.

    value: 7B-shape tokens/s from whole decoder layers (T = 1, fp16 cache of CTX0 tokens) run
    for about budget_s, extrapolated to 32 layers + lm_head (by weight bytes).  Also: C1 end
    to end (32-token prompt as one prefill, then 64 greedy steps) and one C2 layer at
    M = 1, 4, 16 tokens."""
    import numpy as np
    import torch

    from oracle import model as om
    from oracle import torch_cpu as tc

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    d, H, hd = c["d"], c["hidden"], c["hd"]
    cfg7 = om.OracleConfig(n_layer=1, n_head=c["n_head"], n_kv_head=c["n_kv_head"], d_model=d, hidden=H,
                           vocab=c["vocab"], eps=1e-5, block_size=CTX0 + 64)
    cos, sin = om.rope_tables(hd, CTX0 + 64)
    lay = [{"ln1": layers["ln1"][0], "ln2": layers["ln2"][0], "qkv_p": layers["qkv_p"][0],
            "qkv_s": layers["qkv_s"][0], "o_p": layers["o_p"][0], "o_s": layers["o_s"][0],
            "gu_p": layers["gu_p"][0], "gu_s": layers["gu_s"][0], "dn_p": layers["dn_p"][0],
            "dn_s": layers["dn_s"][0]}]
    m = tc.TorchCpuModel.from_tensors(cfg7, lay, lnf, lay[0]["qkv_p"], lay[0]["qkv_s"], lay[0]["qkv_p"],
                                      lay[0]["qkv_s"], cos, sin)
    gen = torch.Generator().manual_seed(0)

    def fresh_cache():
        cache = m.new_cache(CTX0 + 32)
        cache["k"][:, :, :, :CTX0] = torch.randn(cache["k"][:, :, :, :CTX0].shape, generator=gen).half()
        cache["v"][:, :, :, :CTX0] = torch.randn(cache["v"][:, :, :, :CTX0].shape, generator=gen).half()
        cache["seen"] = CTX0
        return cache

    x = torch.randn(1, 1, d, generator=gen).half()
    n_done = 0
    t0 = time.perf_counter()
    with torch.no_grad():
        while True:
            cache = fresh_cache()
            x = m.layer(0, x, cache, CTX0)
            n_done += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        per_layer = (time.perf_counter() - t0) / n_done
        c2 = {}
        for M in (1, 4, 16):
            cache = fresh_cache()
            xm = torch.randn(1, M, d, generator=gen).half()
            t1 = time.perf_counter()
            m.layer(0, xm, cache, CTX0)
            c2[str(M)] = round((time.perf_counter() - t1) * 1e6, 1)
        # C1 end to end (MLP 688 zero-padded to 704 for the group-64 packer)
        c1 = om.OracleConfig(n_layer=4, n_head=4, n_kv_head=4, d_model=256, hidden=704, vocab=1024, eps=1e-5,
                             block_size=256)
        c1m = tc.TorchCpuModel(c1, om.pack_model_rtn(c1, om.make_float_weights(c1, seed=0)),
                               *om.rope_tables(c1.head_dim, c1.block_size))
        prompt = np.random.default_rng(0).integers(0, c1.vocab, 32).tolist()
        cache = c1m.new_cache(128)
        t1 = time.perf_counter()
        tok = int(torch.argmax(c1m.forward(prompt, cache)[-1].float()))
        t2 = time.perf_counter()
        for _ in range(64):
            tok = int(torch.argmax(c1m.forward([tok], cache)[-1].float()))
        t3 = time.perf_counter()
    lm_frac = q4_bytes(c["vocab"], d) / layer_weight_bytes(c)
    per_token = per_layer * (c["n_layer"] + lm_frac)
    return {
        "value": 1.0 / per_token,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n_done} x one 7B-shape decoder layer (torch CPU: MARLIN Q4 group-64 packs, the reference "
                   f"CPU dequantizer's only group size, dequantized to fp16 every call, "
                   f"then F.linear; SDPA over {CTX0} fp16 keys) in {per_layer * n_done:.1f} s, extrapolated to "
                   f"32 layers + lm_head"),
        "cpu_model": _cpu_model_name(),
        "torch": torch.__version__,
        "c1_end_to_end": {"prefill_32_ms": round((t2 - t1) * 1e3, 2),
                          "decode_tokens_per_s": round(64 / (t3 - t2), 2)},
        "c2_layer_us": c2,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--group", type=int, choices=(64, 128), default=HEADLINE_GROUP,
                    help="MARLIN group size of the headline decode and the gate/up roofline (default %(default)s)")
    ap.add_argument("--mode", choices=("graph", "persistent"), default="graph",
                    help="decode step execution: the captured per-op graph (the faster on MI355X) or the one-launch "
                         "persistent step (default %(default)s)")
    ap.add_argument("--no-other-group", action="store_true",
                    help="skip the decode line of the other group size")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--context", type=int, default=CTX0,
                    help="tokens of synthetic context before the first timed step (default %(default)s)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 plain device copies of 256 MiB (calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only build the model and time each decode kernel 20 times (short runs under counter "
                         "collection)")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print the in-graph per-kernel averages (JSON) of a rocprofv3 kernel trace of a run of this "
                         "benchmark with the same --steps / --warmup, then exit (no GPU use)")
    args = ap.parse_args()
    if args.summarize_trace:
        print(json.dumps(summarize_trace(args.summarize_trace, 1 + args.warmup + args.steps), indent=1))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs the decode step on one GPU only (no sharding across GPUs), "
                                   "so --gpus must be 1"}))
        sys.exit(2)

    if not 1 <= args.context or args.context + args.warmup + args.steps + 1 > MAX_SEQ:
        print(json.dumps({"error": f"--context + --warmup + --steps must stay within the {MAX_SEQ}-slot cache"}))
        sys.exit(2)

    import torch

    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        n = 256 << 20
        src = torch.ones(n // 2, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_copy": n}), flush=True)
        return
    c = CFG_7B
    G = args.group
    other = 64 if G == 128 else 128
    t_build = time.perf_counter()
    runner, cache, layers, lnf = build_model(c, dev, group_size=G)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t_build
    mode = set_mode(runner, args.mode)
    print(f"[bench] model built and packed in {t_build:.1f} s", file=sys.stderr, flush=True)
    if args.kernel_only:
        runner.step(torch.zeros(1, dtype=torch.int64, device=dev), args.context - 1, args.context - 1, args.context)
        ks = time_step_kernels(runner, c, args.context, args.context + 1, G, reps=20)
        print(json.dumps({k: v["avg_launch_us"] for k, v in ks.items()}), flush=True)
        return
    ms, wall, pos0 = time_decode(runner, cache, args.steps, args.warmup, dev, args.context)
    ms_per_step = ms / args.steps
    tok_s = 1000.0 / ms_per_step
    mean_active = pos0 + (args.steps + 1) / 2.0
    bytes_tok = step_bytes(c, int(round(mean_active)), G)
    gbs = bytes_tok / (ms_per_step * 1e-3) / 1e9
    print(f"[bench] decode {ms_per_step:.3f} ms/token, {tok_s:.1f} tok/s, {gbs:.0f} GB/s step-level", file=sys.stderr,
          flush=True)
    # Each decode kernel timed live after the timed region (the last step's context).
    last = pos0 + args.steps
    ks = time_step_kernels(runner, c, last, last + 1, G)
    prof = in_graph_profile(G)
    if prof is not None:
        for k, v in ks.items():
            pk = prof.get("kernels", {}).get(k)
            if pk:
                v["in_graph_avg_us"] = pk["avg_us"]
                v["in_graph_frac"] = round(v["algorithmic_bytes"] / (pk["avg_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    gu = ks["gate_up"]
    avg_us, bpl, ach = gu["avg_launch_us"], gu["algorithmic_bytes"], gu["achieved_gbs"]
    print("[bench] kernels (us): " + ", ".join(f"{k} {v['avg_launch_us']:.2f}" for k, v in ks.items()),
          file=sys.stderr, flush=True)
    print(f"[bench] gate/up kernel {avg_us:.2f} us, {ach:.0f} GB/s", file=sys.stderr, flush=True)
    traffic, traffic_src = gate_up_traffic(G)
    cpu = None
    second = None
    # The CPU baseline runs on group-64 packs (the reference's CPU dequantizer's format).
    if G == 64 and not args.no_cpu_baseline:
        cpu = cpu_baseline(layers, lnf, c, args.cpu_budget)
    if not args.no_other_group or (other == 64 and not args.no_cpu_baseline):
        del runner, cache, layers, lnf
        torch.cuda.empty_cache()
        runner, cache, layers, lnf = build_model(c, dev, group_size=other)
        set_mode(runner, args.mode)
        if not args.no_other_group:
            ms2, _, p2 = time_decode(runner, cache, args.steps, args.warmup, dev, args.context)
            ms2 /= args.steps
            b2 = step_bytes(c, int(round(p2 + (args.steps + 1) / 2.0)), other)
            second = {"weights": (f"MARLIN Q4 group {other}" + (" (the reference's pack format)" if other == 64 else "")
                                  + ", RTN"),
                      "tokens_per_s": round(1000.0 / ms2, 2), "ms_per_step": round(ms2, 4),
                      "algorithmic_bytes_per_token": b2,
                      "step_hbm_frac_of_peak": round(b2 / (ms2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            print(f"[bench] group-{other} decode {ms2:.3f} ms/token", file=sys.stderr, flush=True)
        if other == 64 and not args.no_cpu_baseline:
            cpu = cpu_baseline(layers, lnf, c, args.cpu_budget)
    line = {
        "metric": "Q4 7B-shape decode tok/s (bs=1, 1 GPU); achieved HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 activations, int4 weights (fp32 accumulation)",
        "data": "synthetic (random-init N(0,0.02) weights, N(0,1) context KV)",
        "config": {
            "workload": "Llama-7B-shape quantized decode step, batch 1 (BASELINE configs[1] shapes, full 32-layer model)",
            "layers": c["n_layer"], "d_model": c["d"], "heads": c["n_head"], "head_dim": c["hd"],
            "mlp_hidden": c["hidden"], "vocab": c["vocab"], "weights": f"MARLIN Q4 group {G} (fp16 scale+bias), RTN",
            "embedding": "Q8_G64", "kv_cache": f"fp16, {MAX_SEQ} slots, context {pos0}..{pos0 + args.steps}",
            "algorithmic_bytes_per_token": bytes_tok,
            "step_hbm_gbs": round(gbs, 1),
            "step_hbm_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "kernel": (f"t16_gemv_kernel<1,2,2,12,2,{'true' if G == 128 else 'false'},256> (fused RMSNorm + gate/up "
                       f"Q4 G{G} GEMV on matrix cores + SwiGLU, 22016x4096, 256-thread workgroups)"),
            "bound": "hbm",
            "achieved": round(ach, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "avg_launch_us": round(avg_us, 3),
            "algorithmic_bytes_per_launch": bpl,
            "method": ("achieved / frac: algorithmic bytes / average launch duration by HIP events on the "
                       "runner's stream around a captured graph of 200 launches back to back over the 32 layers' "
                       "weights, after the timed decode; in_graph_*: the same kernel inside the captured decode "
                       "graph, from the committed rocprofv3 kernel-trace summary"),
            "in_graph_avg_us": gu.get("in_graph_avg_us"),
            "in_graph_frac": gu.get("in_graph_frac"),
            "in_graph_source": (None if prof is None else
                                {k: prof[k] for k in ("source", "measured_at_commit", "command") if k in prof}),
            "traffic_source": traffic_src,
        },
        "decode_kernels": ks,
        "cpu_baseline": cpu,
        f"group{other}_decode": second,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
