"""MARLIN Q4 group 128 on the GPU (this build's variant: the reference's 64-column code
layout with one (scale, bias) per 128 columns).

* packer and dequantization bit for bit against the oracle (oracle/formats.py, pinned
  against the group-64 format and the RTN closed form in test_oracle_formats.py);
* the tile16 copy keeps every scale (host decode of the buffer);
* GEMV / multi-token GEMM: bit-identical to the group-64 kernels on the same codes with
  each 128-group's (scale, bias) duplicated over its two 64-groups (same arithmetic),
  and within 2e-3 relative of the oracle's dequantize-then-matmul;
* the runner with group-128 weights against the oracle (decode steps, a verify chain,
  a tree), logits <= 1e-2.
"""

import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import model as om

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def N(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("N_,K,src", [(64, 128, F16), (13, 256, F16), (100, 384, F32), (12288, 4096, F16)])
def test_g128_pack_and_dequant_bit_exact(dev, N_, K, src):
    from axiomlm_amd.kernels import dequantize_q4_marlin, pack_linear_q4_marlin

    print(f"[g128_pack] N={N_} K={K} src={src.__name__}", flush=True)
    rng = np.random.default_rng(N_ + K)
    w = (rng.standard_normal((N_, K)) * 0.02).astype(src)
    wm_ref, sb_ref = fm.pack_linear_q4_marlin_g128(w)
    wm, sb = pack_linear_q4_marlin(T(w, dev), clip_search=False, group_size=128)
    assert tuple(sb.shape) == ((N_ + 7) // 8, K // 128, 8, 2)
    assert np.array_equal(N(wm), wm_ref)
    assert np.array_equal(N(sb).view(np.uint16), sb_ref.view(np.uint16))
    deq = N(dequantize_q4_marlin(wm, sb, K, N_))
    assert np.array_equal(deq.view(np.uint16), fm.dequantize_q4_marlin_g128(wm_ref, sb_ref, K, N_).view(np.uint16))


def test_g128_tile16_keeps_scales(dev):
    from axiomlm_amd.kernels import repack_q4_marlin_tile16

    N_, K = 40, 384
    rng = np.random.default_rng(3)
    wm, sb = fm.pack_linear_q4_marlin_g128((rng.standard_normal((N_, K)) * 0.02).astype(F16))
    w16, sb16 = repack_q4_marlin_tile16(T(wm, dev), T(sb, dev), N_, K)
    w16_64, _ = repack_q4_marlin_tile16(T(wm, dev), T(np.repeat(sb, 2, axis=1), dev), N_, K)
    assert torch.equal(w16, w16_64)  # codes re-tile exactly as for group 64
    N16, KB = (N_ + 15) // 16, K // 128
    got = N(sb16).view(F16).reshape(N16, KB, 16, 2)
    sbr = sb.transpose(0, 2, 1, 3).reshape(-1, KB, 2)
    for r in range(N16 * 16):
        want = sbr[r] if r < sbr.shape[0] else np.zeros((KB, 2), F16)
        assert np.array_equal(got[r // 16, :, r % 16].view(np.uint16), want.view(np.uint16)), r


@pytest.mark.parametrize("M,N_,K", [(1, 12288, 4096), (1, 4096, 11008), (3, 768, 256), (16, 1024, 1024),
                                    (40, 4096, 4096), (64, 384, 640)])
def test_g128_gemv_gemm_match_group64_and_oracle(dev, M, N_, K):
    from axiomlm_amd.kernels import qmv_q4_tile16, repack_q4_marlin_tile16

    print(f"[g128_gemv] M={M} N={N_} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N_)
    w = (rng.standard_normal((N_, K)) * 0.02).astype(F16)
    x = rng.standard_normal((M, K)).astype(F16)
    wm, sb = fm.pack_linear_q4_marlin_g128(w)
    w16, sb16 = repack_q4_marlin_tile16(T(wm, dev), T(sb, dev), N_, K)
    w16b, sb16b = repack_q4_marlin_tile16(T(wm, dev), T(np.repeat(sb, 2, axis=1), dev), N_, K)
    y = N(qmv_q4_tile16(T(x, dev), w16, sb16, N_))
    y64 = N(qmv_q4_tile16(T(x, dev), w16b, sb16b, N_))
    assert np.array_equal(y.view(np.uint16), y64.view(np.uint16))
    ref = fm.linear_fp16(x, fm.dequantize_q4_marlin_g128(wm, sb, K, N_)).astype(F32)
    err = np.abs(y.astype(F32) - ref)
    assert np.all(err <= 2e-3 * np.maximum(1.0, np.abs(ref))), float(err.max())


@pytest.mark.parametrize("M", [1, 3, 20])
def test_g128_swiglu_matches_group64(dev, M):
    from axiomlm_amd.kernels import qmv_q4_tile16_swiglu, repack_q4_marlin_tile16

    K, H = 4096, 11008
    rng = np.random.default_rng(M)
    w = (rng.standard_normal((2 * H, K)) * 0.02).astype(F16)
    x = T(rng.standard_normal((M, K)).astype(F16), dev)
    ln = T((1 + 0.1 * rng.standard_normal(K)).astype(F16), dev)
    wm, sb = fm.pack_linear_q4_marlin_g128(w)
    a = qmv_q4_tile16_swiglu(x, ln, 1e-5, *repack_q4_marlin_tile16(T(wm, dev), T(sb, dev), 2 * H, K), H)
    b = qmv_q4_tile16_swiglu(x, ln, 1e-5, *repack_q4_marlin_tile16(T(wm, dev), T(np.repeat(sb, 2, axis=1), dev),
                                                                    2 * H, K), H)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_g128_runner_matches_oracle(dev):
    """Decode steps, a 6-token verify chain and a 9-node tree with group-128 layer and
    lm_head weights (d 1024, 8 heads of 128, 2 KV heads, SwiGLU 2816)."""
    from test_gpu_runner import _check_logits, build_runner, run_steps

    print("[g128_runner]", flush=True)
    cfg = om.OracleConfig(n_layer=2, n_head=8, n_kv_head=2, d_model=1024, hidden=2816, vocab=2048, eps=1e-5,
                          block_size=256)
    ow = om.pack_model(cfg, om.make_float_weights(cfg, seed=4), "q4_g128")
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size)
    model = om.OracleModel(cfg, ow, cos, sin)
    runner, cache = build_runner(cfg, ow, cos, sin, dev, 128)
    assert runner.group_size == 128
    ocache = om.OracleKVCache(128, cfg.n_layer, cfg.n_kv_head, cfg.head_dim)
    rng = np.random.default_rng(8)
    toks = rng.integers(0, cfg.vocab, 12).tolist()
    got = run_steps(runner, cache, toks, dev)
    for i, t in enumerate(toks):
        _check_logits(got[i], model.forward([t], ocache)[-1], f"g128 step {i}")
    seen = cache.total_seen_tokens[0]
    chain = rng.integers(0, cfg.vocab, 6).tolist()
    g = runner.verify_step(torch.tensor([chain], device=dev), seen, seen, seen + 6)[0].float().cpu().numpy()
    ref = model.forward(chain, ocache, return_all_logits=True)
    for t in range(6):
        _check_logits(g[t], ref[t], f"g128 verify {t}")
    seen += 6
    cache.total_seen_tokens[:] = [seen] * cfg.n_layer
    cache.layer_seq_lens[:] = [seen] * cfg.n_layer
    parents = [-1, 0, 0, 1, 1, 2, 3, 5, 5]
    depths, masks = [], []
    for u, p in enumerate(parents):
        depths.append(0 if p < 0 else depths[p] + 1)
        masks.append((0 if p < 0 else masks[p]) | (1 << u))
    tree = rng.integers(0, cfg.vocab, len(parents)).tolist()
    g = runner.verify_tree_step(torch.tensor([tree], device=dev), seen, seen, seen, depths, masks)[0].float()
    ref = model.forward_tree(tree, ocache, depths, masks)
    for t in range(len(tree)):
        _check_logits(g[t].cpu().numpy(), ref[t], f"g128 tree {t}")


def test_g128_runner_rejects_mixed_groups(dev):
    from test_gpu_runner import build_runner

    cfg = om.OracleConfig(n_layer=1, n_head=4, n_kv_head=4, d_model=256, hidden=256, vocab=256, eps=1e-5,
                          block_size=64)
    W = om.make_float_weights(cfg, seed=2)
    ow = om.pack_model(cfg, W, "q4_g128")
    ow.lmh_p, ow.lmh_sb = fm.pack_linear_q4_marlin(W["lm_head"], clip_search=False)
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size)
    with pytest.raises(RuntimeError, match="mixed MARLIN group sizes"):
        build_runner(cfg, ow, cos, sin, dev, 32)
