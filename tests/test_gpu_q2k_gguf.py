"""GGUF Q2_K super-blocks on the GPU against the numpy oracle (oracle/formats.py):
packer and dequantization bit for bit, GEMV within 2e-3 relative of x times the
oracle's fp32 dequantized weights (float64 product, one fp16 rounding) at the C4
shapes, ragged row counts, 1-5 tokens, bias, the largest K, and on weights that
sit exactly on the lattice; and the rounding of the one-token and several-token
kernels against the float64 product."""

import numpy as np
import pytest
import torch

from oracle import formats as fm

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("N,K,src", [(16, 256, F16), (37, 512, F32), (1024, 4096, F16), (64, 11008, F16)])
def test_q2k_pack_and_dequant_bit_exact(dev, N, K, src):
    from axiomlm_amd.kernels import dequantize_q2_k_gguf, pack_linear_q2_k_gguf

    print(f"[q2k_pack] N={N} K={K} src={src.__name__}", flush=True)
    rng = np.random.default_rng(N + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(src)
    w[0, :16] = 0.0  # an all-zero sub-block (scale code 0 where the block max allows)
    want = fm.pack_q2_k_gguf(w)
    got = pack_linear_q2_k_gguf(T(w, dev))
    assert tuple(got.shape) == (N, K // 256, 84)
    g = got.cpu().numpy()
    assert np.array_equal(g, want), f"{int((g != want).any(-1).sum())} blocks differ"
    deq = dequantize_q2_k_gguf(got).cpu().numpy()
    assert np.array_equal(deq.view(np.uint16), fm.dequantize_q2_k_gguf(want).view(np.uint16))


def _check_gemv(dev, M, N, K, bias, w=None, seed=0):
    from axiomlm_amd.kernels import qmv_q2_k_gguf

    rng = np.random.default_rng(seed)
    if w is None:
        w = (rng.standard_normal((N, K)) * 0.02).astype(F16)
    blocks = fm.pack_q2_k_gguf(w)
    x = rng.standard_normal((M, K)).astype(F16)
    b = (rng.standard_normal(N) * 0.1).astype(F16) if bias else None
    got = qmv_q2_k_gguf(T(x, dev), T(blocks, dev), None if b is None else T(b, dev)).cpu().numpy().astype(F32)
    # the published decoder yields fp32 weights; reference product in float64, one fp16 rounding
    ref = x.astype(np.float64) @ fm.dequantize_q2_k_gguf(blocks, F32).astype(np.float64).T
    if b is not None:
        ref = ref + b.astype(np.float64)
    ref = ref.astype(F16).astype(F32)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 * np.maximum(1.0, np.abs(ref))), float(err.max())


@pytest.mark.parametrize("M,N,K,bias", [(1, 11008, 4096, False), (1, 4096, 11008, False), (1, 13, 256, True),
                                        (2, 300, 768, False), (3, 129, 4096, True), (4, 4096, 4096, False),
                                        (5, 200, 1024, False), (4, 64, 16384, False), (1, 32000, 4096, False),
                                        (2, 13, 256, True), (4, 40, 512, False),
                                        # 8 and 16 tokens per launch; 7 + 2 at K = 11008 (LDS holds seven rows)
                                        (8, 300, 4096, True), (16, 100, 2048, False), (9, 64, 11008, False)])
def test_q2k_gemv_matches_oracle(dev, M, N, K, bias):
    print(f"[q2k_gemv] M={M} N={N} K={K} bias={bias}", flush=True)
    _check_gemv(dev, M, N, K, bias, seed=M * 31 + N)


def _ulps(a, b):
    """Distance in fp16 ulps between fp16 arrays (through zero: both distances)."""
    ua, ub = a.view(np.uint16).astype(np.int32), b.view(np.uint16).astype(np.int32)
    ma, mb = ua & 0x7FFF, ub & 0x7FFF  # magnitudes, ordered like the values of one sign
    return np.where((ua >> 15) == (ub >> 15), np.abs(ma - mb), ma + mb)


@pytest.mark.parametrize("M,N,K", [(4, 11008, 4096), (4, 4096, 11008), (2, 300, 768), (3, 64, 16384),
                                   (16, 512, 4096)])
def test_q2k_gemv_rounding(dev, M, N, K):
    """Two to sixteen tokens per launch run the MFMA kernel, which multiplies the exact
    code products sc q and the min codes and applies d and dmin in fp32: at least 99 %
    of its outputs are the fp16 rounding of the float64 product and the rest one ulp
    away (at the C4 shapes 99.8-99.9 %; a kernel that rounded each dequantized weight to
    fp16 gets about 58 % at 4096 x 2048, a plant on the CPU).  The one-token
    dot-product kernel is checked on the same rows at its own bar: its per-sub-block
    sum acc - 64 S cancels a term of about 64 |S| in fp32, so about 88 % of its outputs
    are correctly rounded and the rest one ulp or up to 2e-4 (at K = 4096) away."""
    from axiomlm_amd.kernels import qmv_q2_k_gguf

    print(f"[q2k_rounding] M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F16)
    blocks = fm.pack_q2_k_gguf(w)
    xn = rng.standard_normal((M, K)).astype(F16)
    ref = xn.astype(np.float64) @ fm.dequantize_q2_k_gguf(blocks, F32).astype(np.float64).T
    rr = ref.astype(F16)
    bd, x = T(blocks, dev), T(xn, dev)
    many = qmv_q2_k_gguf(x, bd).cpu().numpy()
    one = np.concatenate([qmv_q2_k_gguf(x[m:m + 1], bd).cpu().numpy() for m in range(M)])
    grow = np.sqrt(K / 4096.0)  # accumulation error grows like the square root of K
    u = _ulps(many, rr)
    assert np.all((u <= 1) | (np.abs(many - ref) <= 2e-5 * grow)), int(u.max())
    assert np.mean(u == 0) >= 0.99, float(np.mean(u == 0))
    u1 = _ulps(one, rr)
    assert np.all((u1 <= 1) | (np.abs(one - ref) <= 2.5e-4 * grow)), int(u1.max())
    assert np.mean(u1 == 0) >= 0.8, float(np.mean(u1 == 0))


def test_q2k_gemv_on_lattice_weights(dev):
    import sys

    sys.path.insert(0, __file__.rsplit("/", 1)[0])
    from test_oracle_formats import _q2k_lattice

    w, *_ = _q2k_lattice(np.random.default_rng(3), 512, 16)
    _check_gemv(dev, 1, 512, 4096, False, w=w.astype(F32), seed=4)


def test_q2k_rejects_bad_shapes(dev):
    from axiomlm_amd.kernels import qmv_q2_k_gguf

    blocks = torch.zeros((8, 2, 84), dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError):
        qmv_q2_k_gguf(torch.zeros((1, 256), dtype=torch.float16, device=dev), blocks)
    with pytest.raises(RuntimeError):
        qmv_q2_k_gguf(torch.zeros((1, 512), dtype=torch.float16, device=dev), blocks[:, :, :80])
