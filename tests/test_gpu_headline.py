"""The headline configuration (BASELINE configs[1] / north_star: MARLIN Q4 group 128 with
fp16 scales, the 7B layer shape) through the runner's captured decode step, against the
oracle, plus full-depth property checks on the 32-layer model that ``bench.py`` times.

* One 7B-shape layer (d 4096, 32 heads x 128, SwiGLU 11008) with a 32000-row group-128
  lm_head and a Q8_G64 embedding, fp16 KV with 140 keys of context: the same kernel
  instantiations as the benchmark's step (QKV + RoPE + cache write, short-split
  attention, O with the split merge + residual, gate/up + SwiGLU on 256-thread
  workgroups, down + residual, lm_head + argmax keys, the parameter kernel), greedy
  tokens fed back on the device, logits <= 1e-2 from the oracle, the greedy choices the
  oracle's (apart from near-ties); ``get_last_norm`` after a step and after a verify
  chain against the oracle's final normed hidden state (mps_kernels.mm:3731-3736).
* The 32-layer model of ``bench.py`` (group 128): a verify chain of k tokens equals k
  consecutive decode steps (the reference's cross-path check, tests/test_speculative.py:
  210-218), for k = 2, 3, 8, 32.
* C5 at full depth (32 layers, vocab 32000, FP8 prefix of 2048): the first-child chain of
  the 64-node tree (branching 4, 4, 2, 2, 1, 1) verified in one ``verify_tree_step``
  equals the same chain decoded step by step.
  Both full-depth bounds are the larger of the reference's 0.02 (set for a two-layer
  model) and 1.5 x the fp16 noise floor of 32 layers, measured in the test as the
  difference between two kernel families computing the same decode steps (tile16
  group-128 kernels vs MARLIN-layout kernels on the bit-identical group-64 twin).

Weights are packed on the GPU (the group-64 and group-128 packers are bit-identical to
the oracle's, test_gpu_kernels.py / test_gpu_g128.py) and copied to the host for the
oracle where one is used.
"""

import numpy as np
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32
TOL = 1e-2
CROSS_TOL = 0.02  # verify vs step on the same runner (tests/test_speculative.py:213-218)


def _packs(dev, cfg, group, seed):
    """Group-`group` MARLIN packs of a random N(0, 0.02) model made on the GPU, as host
    OracleWeights (Q8_G64 embedding, MARLIN lm_head)."""
    from axiomlm_amd.kernels import pack_linear_q4_marlin, pack_linear_q8_g64

    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def randn(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * std).half()

    def q4(n, k):
        p, s = pack_linear_q4_marlin(randn(n, k), clip_search=False, group_size=group)
        return p.cpu().numpy(), s.cpu().numpy()

    d, H, V = cfg.d_model, cfg.hidden, cfg.vocab
    qkv_rows = (cfg.n_head + 2 * cfg.n_kv_head) * cfg.head_dim
    wte_p, wte_s = pack_linear_q8_g64(randn(V, d))
    lmh_p, lmh_s = q4(V, d)
    ow = om.OracleWeights(wte_p.cpu().numpy().view(np.uint8).reshape(V, d), wte_s.cpu().numpy(), lmh_p, lmh_s,
                          [], [], (1 + randn(d, std=0.1).float()).half().cpu().numpy(), [], [], [], [], [], [], [],
                          [])
    for _ in range(cfg.n_layer):
        ow.ln1.append((1 + randn(d, std=0.1).float()).half().cpu().numpy())
        ow.ln2.append((1 + randn(d, std=0.1).float()).half().cpu().numpy())
        for (pl, sl), (n, k) in (((ow.c_attn_p, ow.c_attn_s), (qkv_rows, d)), ((ow.c_proj_p, ow.c_proj_s), (d, d)),
                                 ((ow.gu_p, ow.gu_s), (2 * H, d)), ((ow.wd_p, ow.wd_s), (d, H))):
            p, s = q4(n, k)
            pl.append(p)
            sl.append(s)
    return ow


def _fill_context(cache, ctx, seed):
    """N(0, 1) fp16 rows in slots [0, ctx) of every layer (the benchmark's synthetic context)."""
    g = torch.Generator(device=cache.cache.device)
    g.manual_seed(seed)
    cache.cache[..., :ctx, :].normal_(generator=g)
    cache.total_seen_tokens[:] = [ctx] * cache.n_layer
    cache.layer_seq_lens[:] = [ctx] * cache.n_layer


@pytest.mark.parametrize("mode", ["graph", "persistent"])
def test_headline_g128_7b_layer_step_greedy_and_last_norm(dev, mode):
    """One 7B-shape group-128 layer + 32000-row group-128 lm_head through the decode step
    (graph: the benchmark's kernel instantiations; persistent: the one-launch step), 140
    keys of fp16 context, one step with a given token then seven device-fed greedy steps,
    a 4-token verify chain; logits, greedy choices and get_last_norm against the oracle."""
    from test_gpu_runner import _load_gpu_cache, build_runner

    cfg = om.OracleConfig(n_layer=1, n_head=32, n_kv_head=32, d_model=4096, hidden=11008, vocab=32000, eps=1e-5,
                          block_size=4096)
    S, ctx = 4096, 140
    print(f"[headline_g128] mode={mode} d={cfg.d_model} heads={cfg.n_head} V={cfg.vocab} ctx={ctx}", flush=True)
    ow = _packs(dev, cfg, 128, seed=11)
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size, 10000.0)
    model = om.OracleModel(cfg, ow, cos, sin)
    runner, cache = build_runner(cfg, ow, cos, sin, dev, S, "fp16", mode=mode)
    assert runner.group_size == 128 and runner.mode == mode
    _fill_context(cache, ctx, seed=12)
    ocache = om.OracleKVCache(S, cfg.n_layer, cfg.n_kv_head, cfg.head_dim, "fp16")
    _load_gpu_cache(ocache, cache)
    ocache.total_seen_tokens[:] = [ctx] * cfg.n_layer
    ocache.layer_seq_lens[:] = [ctx] * cfg.n_layer

    def check_norm(T, ref_norm, what):
        got = runner.get_last_norm(T)[0].float().cpu().numpy()
        ref = ref_norm.astype(F32)
        assert got.shape == ref.shape
        err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
        print(f"[headline_g128] {what}: max rel |norm diff| {err.max():.2e}", flush=True)
        assert err.max() <= TOL, what

    pos = ctx
    tok = 1234
    got = runner.step(torch.tensor([[tok]], device=dev), pos, pos, pos + 1)[0, 0].float().cpu().numpy()
    ref, ref_norm = model.forward([tok], ocache, return_norm=True)
    ref = ref[-1].astype(F32)
    err = np.abs(got - ref).max()
    print(f"[headline_g128] step 0 tok={tok} max |logit diff| {err:.2e}", flush=True)
    assert err <= TOL
    check_norm(1, ref_norm, "step 0")
    pos += 1
    for i in range(1, 8):
        want = om.argmax_first(ref)
        got = runner.step_greedy(pos, pos, pos + 1)[0, 0].float().cpu().numpy()
        used = int(runner.last_token().item())
        # the device's argmax of the previous logits; another token only at a near-tie
        assert used == want or ref[want] - ref[used] <= 2 * TOL, (i, used, want)
        ref, ref_norm = model.forward([used], ocache, return_norm=True)
        ref = ref[-1].astype(F32)
        err = np.abs(got - ref).max()
        print(f"[headline_g128] greedy step {i} tok={used} max |logit diff| {err:.2e}", flush=True)
        assert err <= TOL
        pos += 1
    check_norm(1, ref_norm, "greedy step 7")
    cache.total_seen_tokens[:] = [pos] * cfg.n_layer
    cache.layer_seq_lens[:] = [pos] * cfg.n_layer
    chain = [7, 31999, 0, 4242]
    g = runner.verify_step(torch.tensor([chain], device=dev), pos, pos, pos + 4)[0].float().cpu().numpy()
    ref, ref_norm = model.forward(chain, ocache, return_all_logits=True, return_norm=True)
    for t in range(4):
        err = np.abs(g[t] - ref[t].astype(F32)).max()
        assert err <= TOL, (t, err)
    check_norm(4, ref_norm, "verify chain of 4")
    runner.check()


def _full_packs(dev, group=128, seed=0):
    """The benchmark's 32-layer 7B-shape model: random N(0, 0.02) weights packed to MARLIN Q4
    of the given group on the GPU, Q8_G64 embedding."""
    import bench
    from axiomlm_amd.kernels import pack_linear_q4_marlin, pack_linear_q8_g64

    c = bench.CFG_7B
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def randn(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * std).half()

    def q4(n, k):
        return pack_linear_q4_marlin(randn(n, k), clip_search=False, group_size=group)

    d, H, L, hd = c["d"], c["hidden"], c["n_layer"], c["hd"]
    qkv_rows = (c["n_head"] + 2 * c["n_kv_head"]) * hd
    lay = {k: [] for k in ("ln1", "ln2", "qkv", "o", "gu", "dn")}
    for _ in range(L):
        lay["ln1"].append((1 + randn(d, std=0.1).float()).half())
        lay["ln2"].append((1 + randn(d, std=0.1).float()).half())
        lay["qkv"].append(q4(qkv_rows, d))
        lay["o"].append(q4(d, c["n_head"] * hd))
        lay["gu"].append(q4(2 * H, d))
        lay["dn"].append(q4(d, H))
    lay["lmh"] = q4(c["vocab"], d)
    lay["wte"] = pack_linear_q8_g64(randn(c["vocab"], d))
    lay["lnf"] = (1 + randn(d, std=0.1).float()).half()
    return c, lay


def _g64_twin(pack):
    """The group-64 form of a group-128 pack: the same codes with each (scale, bias) pair
    repeated over its two 64-column halves; it dequantizes bit-identically
    (test_gpu_g128.py::test_g128_gemv_gemm_match_group64_and_oracle)."""
    p, s = pack
    return p, s.repeat_interleave(2, dim=1).contiguous()


def _full_runner(dev, c, lay, kv, S, layout="tile16", twin=False, max_tokens=32):
    from axiomlm_amd.cache import StaticKVCache
    from axiomlm_amd.runner import QuantizedDecodeRunner

    hd, L = c["hd"], c["n_layer"]
    cos, sin = om.rope_tables(hd, 4 * S, 10000.0)
    freqs = torch.from_numpy(np.stack([cos, sin], -1).astype(F32)).to(dev)
    cache = StaticKVCache(1, S, L, c["n_kv_head"], hd, device=dev, cache_dtype=kv)
    m = _g64_twin if twin else (lambda x: x)
    P = lambda k: [m(x)[0] for x in lay[k]]  # noqa: E731
    Sc = lambda k: [m(x)[1] for x in lay[k]]  # noqa: E731
    lmh_p, lmh_s = m(lay["lmh"])
    runner = QuantizedDecodeRunner(
        None, lmh_p, lmh_s, freqs, lay["ln1"], P("qkv"), Sc("qkv"), P("o"), Sc("o"), lay["ln2"], P("gu"), Sc("gu"),
        P("dn"), Sc("dn"), lay["lnf"], cache.k_caches, cache.v_caches, c["n_head"], c["n_kv_head"], hd, True, 1e-5,
        [], c["vocab"], wte_p=lay["wte"][0], wte_s=lay["wte"][1], k_scales=cache.k_scales, v_scales=cache.v_scales,
        kv_dtype=kv, max_tokens=max_tokens, layout=layout)
    return runner, cache


def _decode_chain(runner, toks, pos0, dev):
    out = []
    for t, tok in enumerate(toks):
        lg = runner.step(torch.tensor([[tok]], device=dev), pos0 + t, pos0 + t, pos0 + t + 1)
        out.append(lg[0, 0].float().cpu().numpy().copy())
    return out


def _assert_within_floor(what, cross, floor, a, b):
    """The cross-path difference must sit within the fp16 noise floor of the depth: max(0.02,
    1.5 x the difference between two kernel families computing the same decode steps)."""
    bound = max(CROSS_TOL, 1.5 * floor)
    print(f"[{what}] max |cross-path diff| {cross:.3e}, noise floor (tile16 G128 vs MARLIN-layout G64 twin) "
          f"{floor:.3e}, bound {bound:.3e}", flush=True)
    assert floor < 0.15, f"{what}: the two step implementations differ by {floor}"
    assert cross <= bound, f"{what}: {cross} > {bound}"
    for x, y in zip(a, b):
        i, j = int(np.argmax(x)), int(np.argmax(y))
        assert i == j or abs(float(x[i]) - float(x[j])) <= 2 * bound, (i, j)


def test_full_depth_verify_chain_equals_steps(dev):
    """32 layers, group 128, fp16 cache with 128 keys of context: verify_step over k tokens
    gives the logits of k consecutive decode steps for k = 2, 3, 8, 32 (both paths write the
    same cache slots, so every k starts from the same prefix).  At this depth fp16 rounding
    alone moves logits by a few hundredths, so the bound is the larger of the reference's
    0.02 (tests/test_speculative.py:213-218, a two-layer model) and 1.5 x the difference
    between two implementations of the same decode steps: the tile16 group-128 kernels and
    the MARLIN-layout kernels on the group-64 twin of the same packs."""
    print("[full_depth_chain] building the 32-layer model", flush=True)
    c, lay = _full_packs(dev)
    runner, cache = _full_runner(dev, c, lay, "fp16", 4096)
    twin, tcache = _full_runner(dev, c, lay, "fp16", 4096, layout="marlin", twin=True)
    ctx = 128
    _fill_context(cache, ctx, seed=1)
    _fill_context(tcache, ctx, seed=1)
    assert torch.equal(cache.cache, tcache.cache)
    rng = np.random.default_rng(2)
    for k in (2, 3, 8, 32):
        chain = rng.integers(0, c["vocab"], k).tolist()
        steps = _decode_chain(runner, chain, ctx, dev)
        other = _decode_chain(twin, chain, ctx, dev)
        ver = runner.verify_step(torch.tensor([chain], device=dev), ctx, ctx, ctx + k)[0].float().cpu().numpy()
        cross = max(float(np.abs(ver[t] - steps[t]).max()) for t in range(k))
        floor = max(float(np.abs(other[t] - steps[t]).max()) for t in range(k))
        _assert_within_floor(f"full_depth_chain k={k}", cross, floor, ver, steps)


def test_c5_full_depth_tree_first_child_chain_equals_steps(dev):
    """C5 at full size: 32 layers, vocab 32000, group 128, FP8 cache with a 2048-token prefix.
    The 64-node tree (branching 4, 4, 2, 2, 1, 1) is verified in one call; the logits of its
    first-child chain (one node per depth) equal the chain decoded step by step, within the
    same noise-floor bound as the verify chain, and every node's logits are finite."""
    from axiomlm_amd.kernels import quantize_kv_fp8
    from axiomlm_amd.tree import build_branching_tree

    prefix, T = 2048, 64
    print(f"[c5_full_depth] building the 32-layer model, fp8 prefix {prefix}", flush=True)
    c, lay = _full_packs(dev)
    S = prefix + 2 * T
    runner, cache = _full_runner(dev, c, lay, "fp8", S, max_tokens=T)
    twin, tcache = _full_runner(dev, c, lay, "fp8", S, layout="marlin", twin=True, max_tokens=T)
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    for li in range(c["n_layer"]):
        k = torch.randn(1, c["n_kv_head"], prefix, c["hd"], generator=g, device=dev).half()
        v = torch.randn(1, c["n_kv_head"], prefix, c["hd"], generator=g, device=dev).half()
        kc, ks, vc, vs = quantize_kv_fp8(k, v)
        for cc in (cache, tcache):
            cc.cache[li, 0, :, :, :prefix].copy_(kc)
            cc.cache[li, 1, :, :, :prefix].copy_(vc)
            cc.scales[li, 0, :, :, :prefix].copy_(ks)
            cc.scales[li, 1, :, :, :prefix].copy_(vs)
    tree = build_branching_tree((4, 4, 2, 2, 1, 1), max_nodes=T)
    assert tree["num_nodes"] == T
    children = tree["children"]
    path = [0]
    while children[path[-1]]:
        path.append(children[path[-1]][0])
    rng = np.random.default_rng(7)
    nodes = rng.integers(0, c["vocab"], T).tolist()
    chain = [nodes[u] for u in path]
    steps = _decode_chain(runner, chain, prefix, dev)
    other = _decode_chain(twin, chain, prefix, dev)
    got = runner.verify_tree_step(torch.tensor([nodes], device=dev), prefix, prefix, prefix, tree["tree_depths"],
                                  tree["tree_mask"])[0].float().cpu().numpy()
    assert np.isfinite(got).all()
    cross = max(float(np.abs(got[u] - steps[j]).max()) for j, u in enumerate(path))
    floor = max(float(np.abs(other[j] - steps[j]).max()) for j in range(len(path)))
    _assert_within_floor(f"c5_full_depth chain {path}", cross, floor, [got[u] for u in path], steps)
