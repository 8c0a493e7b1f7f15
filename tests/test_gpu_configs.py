"""BASELINE configurations at their own sizes against the oracle.

* C3: decode attention for batch 8, 32 query / 8 KV heads of 128, over INT4 and
  FP8 caches of 1k, 8k and 32k keys, and over the 4096-slot ring after 10,000 tokens
  written in chunks that wrap the ring (attention over all slots = the last
  4096 tokens).
* C5: the speculative tree-verification loop at the 7B layer shape (d 4096,
  32 heads of 128, SwiGLU 11008; one layer and a 2048-token vocabulary keep
  the oracle affordable) with an FP8 cache holding a 2048-token prefix: a
  64-node tree (branching 4, 4, 2, 2, 1, 1) verified in one step, the greedy
  walk, the compaction of the accepted slots and the next step, three times,
  then a decode step.

Inputs are made on the GPU (seeded torch generators) where the oracle would
take minutes to make them; the oracle then checks the GPU's quantization on
the same rows (bit for bit) and its arithmetic on the GPU's own codes.
"""

import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import model as om

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32


def _quant_fns(kind):
    if kind == "fp8":
        return fm.quantize_kv_fp8_single, fm.dequantize_kv_fp8
    return fm.quantize_kv_int4_single, fm.dequantize_kv_int4


def _attention_reference(q, kc, vc, ks, vs, kind, n_rep):
    """SDPA per (sequence, KV head) over the dequantized codes; q (B, Hq, hd) fp16."""
    _, deq = _quant_fns(kind)
    B, Hkv = kc.shape[:2]
    out = np.zeros(q.shape, F32)
    for b in range(B):
        for h in range(Hkv):
            kd = deq(kc[b, h], ks[b, h])[None]
            vd = deq(vc[b, h], vs[b, h])[None]
            qq = q[b, h * n_rep:(h + 1) * n_rep][:, None, :]
            out[b, h * n_rep:(h + 1) * n_rep] = om.sdpa_fp16(qq, kd, vd)[:, 0].astype(F32)
    return out


@pytest.mark.parametrize("kind,L", [("int4", 32768), ("fp8", 32768), ("int4", 8192), ("fp8", 8192),
                                    ("int4", 1024), ("fp8", 1024)])
def test_c3_decode_attention(dev, kind, L):
    """B 8, 32 q / 8 kv heads, hd 128, L keys (the C3 lengths 1k / 8k / 32k): the quantizer
    on sampled rows (bit for bit) and the attention output against SDPA over the GPU's
    codes (<= 2e-3)."""
    from axiomlm_amd.kernels import gqa_flash_decode_mps, quantize_kv_fp8, quantize_kv_int4

    B, Hq, Hkv, hd = 8, 32, 8, 128
    print(f"[c3] kind={kind} B={B} L={L}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(3 + L)
    k = torch.randn((B, Hkv, L, hd), generator=g, device=dev).half()
    v = torch.randn((B, Hkv, L, hd), generator=g, device=dev).half()
    kq, ks, vq, vs = (quantize_kv_fp8 if kind == "fp8" else quantize_kv_int4)(k, v)
    rng = np.random.default_rng(4)
    rows = rng.choice(B * Hkv * L, min(2048, B * Hkv * L), replace=False)
    qf, _ = _quant_fns(kind)
    for src, codes, scales in ((k, kq, ks), (v, vq, vs)):
        x = src.view(-1, hd)[torch.from_numpy(rows).to(dev)].cpu().numpy()
        rc, rs = qf(x)
        assert np.array_equal(codes.view(-1, codes.shape[-1])[torch.from_numpy(rows).to(dev)].cpu().numpy(), rc)
        assert np.array_equal(scales.view(-1, 2)[torch.from_numpy(rows).to(dev)].cpu().numpy().view(np.uint16),
                              rs.view(np.uint16))
    del k, v
    q = torch.randn((B, Hq, 1, hd), generator=g, device=dev).half()
    got = gqa_flash_decode_mps(q, kq, vq, L, 0, ks, vs, kind)[:, :, 0].float().cpu().numpy()
    ref = _attention_reference(q[:, :, 0].cpu().numpy(), kq.cpu().numpy(), vq.cpu().numpy(), ks.cpu().numpy(),
                               vs.cpu().numpy(), kind, Hq // Hkv)
    err = np.abs(got - ref).max()
    print(f"[c3] kind={kind} L={L} max |out - SDPA| = {err:.2e}", flush=True)
    assert err <= 2e-3


@pytest.mark.parametrize("kind", ["int4", "fp8"])
def test_c3_ring_window_after_10k_tokens(dev, kind):
    """A 4096-slot ring after 10,000 tokens (write_pos 1808), written in chunks of 1000
    rows whose slots wrap: every slot holds the newest token of its residue, coded bit for
    bit like the oracle's quantizer; attention over all 4096 slots equals SDPA over the
    last 4096 tokens."""
    from axiomlm_amd import _lib
    from axiomlm_amd.kernels import gqa_flash_decode_mps
    from axiomlm_amd.kernels.ops import KV_CODES

    B, Hq, Hkv, hd, S, n_tok, chunk = 8, 32, 8, 128, 4096, 10000, 1000
    print(f"[c3_ring] kind={kind} S={S} after {n_tok}", flush=True)
    width = hd if kind == "fp8" else hd // 2
    kc = torch.zeros((B, Hkv, S, width), dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((B, Hkv, S, hd // 64), dtype=torch.float16, device=dev)
    vs = torch.zeros_like(ks)
    g = torch.Generator(device=dev)
    g.manual_seed(10)
    qf, _ = _quant_fns(kind)
    want_k = np.zeros((B, Hkv, S, width), np.uint8)
    want_v = np.zeros_like(want_k)
    want_ks = np.zeros((B, Hkv, S, hd // 64), F16)
    want_vs = np.zeros_like(want_ks)
    for b in range(B):
        rows_k = torch.randn((n_tok, Hkv * hd), generator=g, device=dev).half()
        rows_v = torch.randn((n_tok, Hkv * hd), generator=g, device=dev).half()
        for n0 in range(0, n_tok, chunk):
            kr, vr = rows_k[n0:n0 + chunk], rows_v[n0:n0 + chunk]
            _lib.check(_lib.lib().axm_kv_cache_write(
                _lib.ptr(kr), _lib.ptr(vr), Hkv * hd, chunk, _lib.ptr(kc[b]), _lib.ptr(vc[b]), _lib.ptr(ks[b]),
                _lib.ptr(vs[b]), KV_CODES[kind], Hkv, hd, S, n0 % S, _lib.stream_of(dev)), "kv_cache_write")
        slots = np.arange(n_tok - S, n_tok) % S
        for rows, wc, wsc in ((rows_k, want_k, want_ks), (rows_v, want_v, want_vs)):
            x = rows[n_tok - S:].cpu().numpy().reshape(S, Hkv, hd).transpose(1, 0, 2)
            c, s = qf(np.ascontiguousarray(x))
            wc[b][:, slots] = c
            wsc[b][:, slots] = s
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().numpy(), want_k) and np.array_equal(vc.cpu().numpy(), want_v)
    assert np.array_equal(ks.cpu().numpy().view(np.uint16), want_ks.view(np.uint16))
    assert np.array_equal(vs.cpu().numpy().view(np.uint16), want_vs.view(np.uint16))
    q = torch.randn((B, Hq, 1, hd), generator=g, device=dev).half()
    got = gqa_flash_decode_mps(q, kc, vc, S, 0, ks, vs, kind)[:, :, 0].float().cpu().numpy()
    ref = _attention_reference(q[:, :, 0].cpu().numpy(), want_k, want_v, want_ks, want_vs, kind, Hq // Hkv)
    err = np.abs(got - ref).max()
    print(f"[c3_ring] kind={kind} max |out - SDPA| = {err:.2e}", flush=True)
    assert err <= 2e-3


# ---------------------------------------------------------------------------
# C5
# ---------------------------------------------------------------------------
def _c5_layer_model(dev, cfg):
    """RTN packs made on the GPU (bit-identical to the oracle's packer, test_gpu_kernels.py::
    test_q4_rtn_pack_bit_exact), copied to the host for the oracle."""
    from axiomlm_amd.kernels import pack_linear_q4_marlin, pack_linear_q8_g64

    g = torch.Generator(device=dev)
    g.manual_seed(5)

    def randn(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * std).half()

    def q4(n, k):
        p, s = pack_linear_q4_marlin(randn(n, k), clip_search=False)
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


def test_c5_tree_verify_loop_7b_layer(dev):
    """Three iterations of tree_decode_greedy at the C5 shapes.  Per iteration: logits of all
    64 nodes within 1e-2 of the oracle's bitmask tree attention over the GPU's FP8 codes,
    the codes the GPU wrote for the 64 tree slots against the oracle's quantization of its
    own rows, the greedy walk equal to the oracle's (apart from near-ties), the compacted
    cache equal to the oracle's compaction of the same contents (bit for bit).  The drafter
    puts the model's greedy continuation on the first-child path so that drafts are
    accepted; the other nodes are seeded random ids."""
    from axiomlm_amd.cache import StaticKVCache  # noqa: F401
    from axiomlm_amd.kernels import quantize_kv_fp8
    from axiomlm_amd.speculative import tree_decode_greedy
    from axiomlm_amd.tree import build_branching_tree, greedy_tree_walk
    from test_gpu_runner import _check_codes, _code_diffs, _load_gpu_cache, build_runner

    cfg = om.OracleConfig(n_layer=1, n_head=32, n_kv_head=32, d_model=4096, hidden=11008, vocab=2048, eps=1e-5,
                          block_size=4096)
    prefix, T, kv = 2048, 64, "fp8"
    S = prefix + 4 * T
    print(f"[c5_loop] d={cfg.d_model} heads={cfg.n_head} prefix={prefix} T={T} kv={kv}", flush=True)
    ow = _c5_layer_model(dev, cfg)
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size, 10000.0)
    model = om.OracleModel(cfg, ow, cos, sin)
    runner, cache = build_runner(cfg, ow, cos, sin, dev, S, kv, max_tokens=T)
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    for li in range(cfg.n_layer):
        k = torch.randn(1, cfg.n_kv_head, prefix, cfg.head_dim, generator=g, device=dev).half()
        v = torch.randn(1, cfg.n_kv_head, prefix, cfg.head_dim, generator=g, device=dev).half()
        kc, ks, vc, vs = quantize_kv_fp8(k, v)
        cache.cache[li, 0, :, :, :prefix].copy_(kc)
        cache.cache[li, 1, :, :, :prefix].copy_(vc)
        cache.scales[li, 0, :, :, :prefix].copy_(ks)
        cache.scales[li, 1, :, :, :prefix].copy_(vs)
    cache.total_seen_tokens[:] = [prefix] * cfg.n_layer
    cache.layer_seq_lens[:] = [prefix] * cfg.n_layer
    tree = build_branching_tree((4, 4, 2, 2, 1, 1), max_nodes=T)
    assert tree["num_nodes"] == T
    children = tree["children"]
    first_path = [0]
    while children[first_path[-1]]:
        first_path.append(children[first_path[-1]][0])
    rng = np.random.default_rng(7)
    ocache = om.OracleKVCache(S, cfg.n_layer, cfg.n_kv_head, cfg.head_dim, kv)
    ocache.frozen = True
    expected = {}

    def draft(step, root, seen):
        # the model's greedy continuation of root (decode steps whose slots the tree overwrites)
        toks = rng.integers(0, cfg.vocab, T).tolist()
        tok = root
        for j, u in enumerate(first_path[1:]):
            lg = runner.step(torch.tensor([[tok]], device=dev), seen + j, seen + j, seen + j + 1)
            tok = int(torch.argmax(lg[0, 0].float()).item())
            toks[u] = tok
        return toks[1:]

    def on_verify(step, seen, nodes, logits, preds, accepted, emitted):
        if "cache" in expected:
            # the committed prefix after the previous iteration's compaction, bit for bit (the
            # slots from `seen` on were since rewritten by the drafter and this tree)
            assert np.array_equal(cache.cache[..., :seen, :].cpu().numpy(), expected["cache"][..., :seen, :])
            assert np.array_equal(cache.scales[..., :seen, :].cpu().numpy().view(np.uint16),
                                  expected["scales"][..., :seen, :])
        got = logits[0].float().cpu().numpy()
        _load_gpu_cache(ocache, cache)
        ocache.total_seen_tokens[:] = [seen] * cfg.n_layer
        ref = model.forward_tree(nodes, ocache, tree["tree_depths"], tree["tree_mask"]).astype(F32)
        err = np.abs(got - ref).max()
        print(f"[c5_loop] step {step}: seen={seen} max |logit diff| {err:.2e} accepted={accepted}", flush=True)
        assert err <= 1e-2
        _check_codes(kv, _code_diffs(kv, ocache), f"c5 step {step}")
        assert preds == [int(np.argmax(r)) for r in got]
        o_acc, o_em = greedy_tree_walk([int(np.argmax(r)) for r in ref], nodes, children, 10 ** 6)
        if (o_acc, o_em) != (accepted, emitted):
            # the walks may part only at a node whose top-2 oracle logits are within the tolerance
            i = 0
            while i < min(len(accepted), len(o_acc)) and accepted[i] == o_acc[i]:
                i += 1
            node = accepted[i - 1]
            top = np.sort(ref[node])[::-1]
            assert top[0] - top[1] <= 2e-2, f"walk differs at node {node}: {accepted} vs {o_acc}"
        ocache.frozen = False
        ocache.compact_tree_path(seen, accepted, seen + len(accepted))
        ocache.frozen = True
        c = cache.cache.cpu().numpy()
        c[:, 0, 0] = ocache.k
        c[:, 1, 0] = ocache.v
        sc = cache.scales.cpu().numpy()
        sc[:, 0, 0] = ocache.ks
        sc[:, 1, 0] = ocache.vs
        expected["cache"], expected["scales"] = c, sc.view(np.uint16)

    last = int(rng.integers(0, cfg.vocab))
    res = tree_decode_greedy(runner, cache, last, tree, draft, 3, on_verify=on_verify)
    assert np.array_equal(cache.cache.cpu().numpy(), expected["cache"])
    assert np.array_equal(cache.scales.cpu().numpy().view(np.uint16), expected["scales"])
    print(f"[c5_loop] accepted per step {res['accepted']} tokens {res['tokens']}", flush=True)
    assert res["model_calls"] == 3 and len(res["tokens"]) == sum(res["accepted"]) + 3
    assert sum(res["accepted"]) >= 1
    seen = cache.total_seen_tokens[0]
    assert seen == prefix + sum(res["accepted"]) + 3
    tok = res["tokens"][-1]
    got = runner.step(torch.tensor([[tok]], device=dev), seen, seen, seen + 1)[0, 0].float().cpu().numpy()
    _load_gpu_cache(ocache, cache)
    ocache.total_seen_tokens[:] = [seen] * cfg.n_layer
    ocache.layer_seq_lens[:] = [seen] * cfg.n_layer
    ref = model.forward([tok], ocache)[-1].astype(F32)
    assert np.abs(got - ref).max() <= 1e-2
