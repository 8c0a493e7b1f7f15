"""numpy restatement of the reference weight / KV formats (TEST INFRASTRUCTURE).

All arithmetic reproduces torch CPU semantics: fp16 tensors are computed in
fp32 and rounded to fp16 after every op; ``torch.round`` is round-half-even
(``np.rint``); fp32 division is IEEE.

Pinning (see tests/test_oracle_*.py):
  * MARLIN layout: reference KAT of the fp16 magic-exponent nibble decode
    (tests/test_phase1_task11_disassembly.py:71-98), the lane maps of
    quant.py:573-576 checked against the kernel-side equations
    (metal_kernels.metal:2159-2161, 2183-2185) on all 32 lanes, and the
    reference invariant "RTN-MARLIN dequant == Q4_G64 dequant bit for bit"
    (quant.py:462-463) on random matrices.
  * RTN codes: brute-force optimality (each code is the nearest lattice point)
    and closed-form scale/bias on hand-built groups.
  * MSE clip search (quant.py:495-571): SHA-256 of every C1 pack written by
    tests/golden/make_golden_c1.py from the reference implementation
    (tests/test_oracle_golden.py).
  * Ternary / Q2: reference KATs (tests/test_phase3_task33_bitnet_q2k.py:62-129)
    and byte-per-weight constants (:321-324).
  * FP8 E4M3FN: all 65536 fp16 inputs against torch's own cast (the library
    the reference calls, quant.py:719, 766).
  * INT4 KV: closed form, exact round trip on lattice inputs, and torch's own
    round / clamp / int8 cast (quant.py:789-803) on exact .5 ties, all-zero
    (NaN-code) groups, subnormal groups and every fp16 quotient in [-8.5, 8.5]
    (tests/test_oracle_model.py).
  * GGUF Q2_K (ggml block_q2_K; not in the reference's code, not vendored, no
    gguf library here): the decoder against a hand-assembled block and an
    element-by-element loop over the published formula, lattice round trips,
    0.328125 B/w.  The encoder is this build's round-to-nearest: parity
    unpinned against ggml's quantize_row_q2_K (iterative scale search).
"""

from __future__ import annotations

import numpy as np

F16 = np.float16
F32 = np.float32


def _h(x):
    """Round an fp32 array to fp16 (RNE) and return it as fp32."""
    return np.asarray(x, dtype=F32).astype(F16).astype(F32)


# ---------------------------------------------------------------------------
# MARLIN Q4 (group 64, fp16 scale + bias) -- quant.py:447-634
# ---------------------------------------------------------------------------
def marlin_lane_maps():
    """(r, c0) of each of the 32 reference lanes, quant.py:573-576."""
    lanes = np.arange(32)
    r = ((lanes & 16) >> 2) | ((lanes & 6) >> 1)
    c0 = ((lanes & 8) >> 1) | ((lanes & 1) << 1)
    return r, c0


def _rtn_scale_bias(wg: np.ndarray, src_fp16: bool):
    """RTN scale/bias per group, quant.py:483-487 (wg: [..., 64])."""
    w_min = wg.min(axis=-1, keepdims=True)
    w_max = wg.max(axis=-1, keepdims=True)
    if src_fp16:
        # fp16 subtraction; clamp(min=1e-8) casts the bound to fp16 (0) -> no-op
        denom = _h(w_max.astype(F32) - w_min.astype(F32))
        scale = _h(denom / F32(15.0))
    else:
        denom = np.maximum(w_max.astype(F32) - w_min.astype(F32), F32(1e-8))
        scale = _h(denom / F32(15.0))
    bias = _h(w_min)
    return scale.astype(F32), bias.astype(F32)


def _codes(wg32: np.ndarray, scale: np.ndarray, bias: np.ndarray, qmax: float):
    """clamp(round((w - bias) / clamp(scale, 1e-8)), 0, qmax), quant.py:488-494."""
    q = np.rint((wg32 - bias) / np.maximum(scale, F32(1e-8)))
    return np.clip(q, 0.0, qmax).astype(np.int32)


def linspace_f32(start: float, end: float, steps: int) -> np.ndarray:
    """torch.linspace in fp32 (quant.py:512 uses the default fp32 dtype): step computed
    in fp32, first half counted up from start, second half down from end."""
    s0, s1 = F32(start), F32(end)
    step = (s1 - s0) / F32(steps - 1)
    i = np.arange(steps)
    lo = s0 + step * i.astype(F32)
    hi = s1 - step * (steps - 1 - i).astype(F32)
    return np.where(i < steps // 2, lo, hi).astype(F32)


def _mse_clip_search(wg: np.ndarray, col_importance: np.ndarray | None, grid_steps: int, min_shrink: float):
    """Importance-weighted two-pass clip search, quant.py:495-571 (fp32)."""
    Np, KG, _ = wg.shape
    wg = wg.astype(F32)
    if col_importance is not None:
        ig = col_importance.astype(F32).reshape(1, KG, 64)
        ig = ig * ig
        ig = ig / np.maximum(ig.mean(axis=-1, keepdims=True), F32(1e-8))
    else:
        ig = None
    alphas = linspace_f32(1.0, min_shrink, max(2, grid_steps))
    mn0 = wg.min(axis=-1, keepdims=True)
    mx0 = wg.max(axis=-1, keepdims=True)
    mu = (wg * ig).mean(axis=-1, keepdims=True) if ig is not None else wg.mean(axis=-1, keepdims=True)

    def err_of(sc, bi):
        qc = np.clip(np.rint((wg - bi) / np.maximum(sc, F32(1e-8))), 0.0, 15.0)
        diff = wg - (qc * sc + bi)
        e = diff * diff
        if ig is not None:
            e = ig * e
        return e.sum(axis=-1, dtype=F32)

    best = np.full((Np, KG), np.inf, dtype=F32)
    cur_mn = mn0.copy()
    for a in alphas:
        cand_mn = mu + a * (mn0 - mu)
        sc = _h(np.maximum(mx0 - cand_mn, F32(1e-8)) / F32(15.0))
        bi = _h(cand_mn)
        e = err_of(sc, bi)
        better = e < best
        best = np.where(better, e, best)
        cur_mn = np.where(better[..., None], cand_mn, cur_mn)

    best[:] = np.inf
    best_sc = _h(np.maximum(mx0 - cur_mn, F32(1e-8)) / F32(15.0))
    best_bi = _h(cur_mn)
    for a in alphas:
        cand_mx = mu + a * (mx0 - mu)
        sc = _h(np.maximum(cand_mx - cur_mn, F32(1e-8)) / F32(15.0))
        bi = _h(cur_mn)
        e = err_of(sc, bi)
        better = e < best
        best = np.where(better, e, best)
        best_sc = np.where(better[..., None], sc, best_sc)
        best_bi = np.where(better[..., None], bi, best_bi)
    q = _codes(wg, best_sc, best_bi, 15.0)
    return best_sc, best_bi, q


def interleave_marlin(q: np.ndarray, scale: np.ndarray, bias: np.ndarray):
    """Lane interleave of codes q [N_pad, KG, 64] -> (w_marlin, sb_marlin), quant.py:573-593."""
    Np, KG, _ = q.shape
    nt = Np // 8
    r_idx, c0_idx = marlin_lane_maps()
    # (tile, c, g, word, s, r) -> (tile, g, c, r, word, s)
    q_cr = q.reshape(nt, 8, KG, 2, 4, 8).transpose(0, 2, 1, 5, 3, 4)
    q_c0 = q_cr[:, :, c0_idx, r_idx]  # (nt, KG, 32, 2, 4)
    q_c1 = q_cr[:, :, c0_idx + 1, r_idx]
    shifts = np.array([0, 4, 8, 12], dtype=np.int64)
    lo = ((q_c0.astype(np.int64) & 0xF) << shifts).sum(-1)
    hi = ((q_c1.astype(np.int64) & 0xF) << shifts).sum(-1) << 16
    w_marlin = (lo | hi).astype(np.uint32).view(np.int32)
    sb = np.stack([scale[..., 0], bias[..., 0]], axis=-1).astype(F16)  # (Np, KG, 2)
    sb_marlin = sb.reshape(nt, 8, KG, 2).transpose(0, 2, 1, 3).copy()
    return np.ascontiguousarray(w_marlin), np.ascontiguousarray(sb_marlin)


def pack_linear_q4_marlin(weight: np.ndarray, clip_search: bool = True, col_importance=None, grid_steps: int = 13,
                          min_shrink: float = 0.72):
    """quant.py:447-594.  weight: fp16 or fp32 [N, K], K % 64 == 0."""
    N, K = weight.shape
    assert K % 64 == 0
    nt = (N + 7) // 8
    Np = nt * 8
    src_fp16 = weight.dtype == F16
    w = np.zeros((Np, K), dtype=weight.dtype)
    w[:N] = weight
    wg = w.reshape(Np, K // 64, 64)
    if not clip_search and col_importance is None:
        scale, bias = _rtn_scale_bias(wg, src_fp16)
        q = _codes(wg.astype(F32), scale, bias, 15.0)
    else:
        scale, bias, q = _mse_clip_search(wg, col_importance, grid_steps, min_shrink)
    return interleave_marlin(q, scale, bias)


def _marlin_group_order():
    """Position in a group's 512 (lane, word, half, s) nibbles of each (row c, column k) code:
    the nibble at bits 16*half + 4*s of word j of lane l holds row c0(l) + half, column
    32 j + 8 s + r(l) (quant.py:573-593)."""
    r_idx, c0_idx = marlin_lane_maps()
    order = np.empty((8, 64), dtype=np.int64)
    for lane in range(32):
        for j in range(2):
            for half in range(2):
                for s in range(4):
                    order[c0_idx[lane] + half, 32 * j + 8 * s + r_idx[lane]] = ((lane * 2 + j) * 2 + half) * 4 + s
    return order.reshape(-1)


_MARLIN_ORDER = _marlin_group_order()


def pack_linear_q4_marlin_g128(weight: np.ndarray):
    """MARLIN Q4 with one (scale, bias) per 128 columns (this build's group-128 variant of
    quant.py:447-594; round to nearest): the codes keep the group-64 lane interleave of every
    64-column block, the scales become sb_marlin [N/8][K/128][8][2].  The reference has no
    group-128 packer; scale and bias follow its RTN rule (quant.py:483-494) over 128 columns."""
    N, K = weight.shape
    assert K % 128 == 0
    nt = (N + 7) // 8
    Np = nt * 8
    w = np.zeros((Np, K), dtype=weight.dtype)
    w[:N] = weight
    wg = w.reshape(Np, K // 128, 128)
    scale, bias = _rtn_scale_bias(wg, weight.dtype == F16)
    q = _codes(wg.astype(F32), scale, bias, 15.0).reshape(Np, K // 64, 64)
    wm, _ = interleave_marlin(q, np.zeros((Np, K // 64, 1), F32), np.zeros((Np, K // 64, 1), F32))
    sb = np.stack([scale[..., 0], bias[..., 0]], axis=-1).astype(F16)  # (Np, K/128, 2)
    return wm, np.ascontiguousarray(sb.reshape(nt, 8, K // 128, 2).transpose(0, 2, 1, 3))


def dequantize_q4_marlin_g128(w_marlin: np.ndarray, sb128: np.ndarray, K: int, out_features: int | None = None):
    """fp16 [N, K] = fp16(q * scale + bias) with the (scale, bias) of column k's 128-group."""
    nt = w_marlin.shape[0]
    q = unpack_marlin_codes(w_marlin).astype(F32).reshape(nt * 8, K // 128, 128)
    sb = sb128.transpose(0, 2, 1, 3).reshape(nt * 8, K // 128, 2).astype(F32)
    w = (q * sb[..., 0:1] + sb[..., 1:2]).reshape(nt * 8, K).astype(F16)
    return w[:out_features] if out_features is not None and out_features < w.shape[0] else w


def unpack_marlin_codes(w_marlin: np.ndarray):
    """Inverse interleave: codes [N_pad, K] (uint8), quant.py:597-625."""
    nt, KG, _, _ = w_marlin.shape
    w = w_marlin.view(np.uint32)
    # nibbles as (tile, group, lane, word, half, s)
    nib = np.empty((nt, KG, 32, 2, 2, 4), dtype=np.uint8)
    for half in range(2):
        for s in range(4):
            nib[..., half, s] = (w >> np.uint32(16 * half + 4 * s)) & np.uint32(0xF)
    q = nib.reshape(nt, KG, 512)[:, :, _MARLIN_ORDER].reshape(nt, KG, 8, 64)
    return np.ascontiguousarray(q.transpose(0, 2, 1, 3)).reshape(nt * 8, KG * 64)


def dequantize_q4_marlin(w_marlin: np.ndarray, sb_marlin: np.ndarray, K: int, out_features: int | None = None):
    """fp16 [N, K] = fp16(q * scale + bias) computed in fp32, quant.py:597-634."""
    nt, KG, _, _ = w_marlin.shape
    assert KG * 64 == K
    q = unpack_marlin_codes(w_marlin).astype(F32).reshape(nt * 8, KG, 64)
    sb = sb_marlin.transpose(0, 2, 1, 3).reshape(nt * 8, KG, 2).astype(F32)
    w = (q * sb[..., 0:1] + sb[..., 1:2]).reshape(nt * 8, K).astype(F16)
    if out_features is not None and out_features < w.shape[0]:
        w = w[:out_features]
    return w


def linear_fp16(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None):
    """F.linear on fp16 CPU tensors: fp32 accumulation, one fp16 rounding (+ fp16 bias add)."""
    y = (x.astype(F32) @ w.astype(F32).T).astype(F16)
    if bias is not None:
        y = (y.astype(F32) + bias.astype(F32)).astype(F16)
    return y


def qmv_q4_marlin(x, w_marlin, sb_marlin, out_features=None, bias=None):
    """CPU fallback of qmv/qmm_q4_marlin: dequantize, then F.linear, quant.py:637-684."""
    K = x.shape[-1]
    w = dequantize_q4_marlin(w_marlin, sb_marlin, K, out_features)
    return linear_fp16(x, w, bias)


# ---------------------------------------------------------------------------
# Legacy Q4_G64 (quant.py:17-69) -- used only by the RTN-MARLIN invariant.
# ---------------------------------------------------------------------------
def pack_linear_q4_g64(weight: np.ndarray):
    N, K = weight.shape
    wg = weight.reshape(N, K // 64, 64)
    scale, bias = _rtn_scale_bias(wg, weight.dtype == F16)
    q = _codes(wg.astype(F32), scale, bias, 15.0)
    q_sub = q.reshape(N, K // 8, 8).astype(np.int64)
    packed = np.zeros((N, K // 8), dtype=np.int64)
    for i in range(8):
        packed |= (q_sub[:, :, i] & 0xF) << (4 * i)
    sb = np.stack([scale[..., 0], bias[..., 0]], axis=-1).astype(F16)
    return packed.astype(np.uint32).view(np.int32), sb


def dequantize_q4_g64(w_packed: np.ndarray, sb: np.ndarray, K: int):
    N = w_packed.shape[0]
    w = w_packed.view(np.uint32).astype(np.int64)
    q = np.stack([(w >> (4 * i)) & 0xF for i in range(8)], axis=-1).reshape(N, K // 64, 64).astype(F32)
    return (q * sb[..., 0:1].astype(F32) + sb[..., 1:2].astype(F32)).reshape(N, K).astype(F16)


# ---------------------------------------------------------------------------
# Q8_G64 -- quant.py:72-163
# ---------------------------------------------------------------------------
def pack_linear_q8_g64(weight: np.ndarray):
    """-> (packed uint8 [N, K] == int32 [N, K/4] little-endian bytes, sb fp16 [N, K/64, 2])."""
    N, K = weight.shape
    wg = weight.reshape(N, K // 64, 64)
    w_min = wg.min(axis=-1, keepdims=True)
    w_max = wg.max(axis=-1, keepdims=True)
    if weight.dtype == F16:
        denom = _h(w_max.astype(F32) - w_min.astype(F32))  # fp16 clamp bound rounds to 0
    else:
        denom = np.maximum(w_max.astype(F32) - w_min.astype(F32), F32(1e-8))
    sc = _h(denom.astype(F32) / F32(255.0))
    bi = _h(w_min)
    q = _codes(wg.astype(F32), sc, bi, 255.0)
    packed = q.reshape(N, K).astype(np.uint8)
    sb = np.stack([sc[..., 0], bi[..., 0]], axis=-1).astype(F16)
    return packed, sb


def dequantize_q8_g64(packed_u8: np.ndarray, sb: np.ndarray, K: int):
    N = packed_u8.shape[0]
    q = packed_u8.reshape(N, K // 64, 64).astype(F32)
    return (q * sb[..., 0:1].astype(F32) + sb[..., 1:2].astype(F32)).reshape(N, K).astype(F16)


def dequant_q8_rows(idx: np.ndarray, packed_u8: np.ndarray, sb: np.ndarray):
    K = packed_u8.shape[1]
    flat = np.asarray(idx).reshape(-1)
    return dequantize_q8_g64(packed_u8[flat], sb[flat], K).reshape(*np.shape(idx), K)


# ---------------------------------------------------------------------------
# Ternary (BitNet 1.58) -- quant.py:236-296
# ---------------------------------------------------------------------------
def pack_linear_ternary(weight: np.ndarray):
    N, K = weight.shape
    wg = weight.reshape(N, K // 64, 64)
    if weight.dtype == F16:
        # abs (exact) -> mean accumulated in fp32 then one fp16 rounding; clamp(1e-5) in fp16
        m = _h(np.abs(wg.astype(F32)).mean(axis=-1, keepdims=True, dtype=F32))
        scale = np.maximum(m, _h(F32(1e-5)))
    else:
        m = np.abs(wg.astype(F32)).mean(axis=-1, keepdims=True, dtype=F32)
        scale = _h(np.maximum(m, F32(1e-5)))
    scale = scale.astype(F32)
    q = np.clip(np.rint(wg.astype(F32) / np.maximum(scale, F32(1e-5))), -1.0, 1.0).astype(np.int8)
    code = np.where(q == 1, 1, np.where(q == -1, 2, 0)).astype(np.uint8).reshape(N, K // 4, 4)
    packed = code[..., 0] | (code[..., 1] << 2) | (code[..., 2] << 4) | (code[..., 3] << 6)
    return packed.astype(np.uint8), scale[..., 0].astype(F16)


def ternary_decode_bytes(packed: np.ndarray):
    """(b >> 2j & 1) - (b >> (2j+1) & 1) for j = 0..3 (quant.py:287-293): [..., 4] int8."""
    b = packed.astype(np.int32)[..., None]
    j = np.arange(4)
    return (((b >> (2 * j)) & 1) - ((b >> (2 * j + 1)) & 1)).astype(np.int8)


def dequantize_ternary(packed: np.ndarray, scales: np.ndarray, K: int | None = None):
    N = packed.shape[0]
    K = K or packed.shape[1] * 4
    q = ternary_decode_bytes(packed).reshape(N, K // 64, 64).astype(F32)
    # q.to(scales.dtype) * scales in fp16 (one rounding)
    return (q * scales[..., None].astype(F32)).reshape(N, K).astype(F16)


# ---------------------------------------------------------------------------
# Reference "Q2_K" (affine 2-bit, group 64) -- quant.py:339-403
# ---------------------------------------------------------------------------
def pack_linear_q2_k(weight: np.ndarray):
    N, K = weight.shape
    wg = weight.reshape(N, K // 64, 64)
    w_min = wg.min(axis=-1, keepdims=True)
    w_max = wg.max(axis=-1, keepdims=True)
    if weight.dtype == F16:
        denom = _h(w_max.astype(F32) - w_min.astype(F32))
        scale = _h(denom / F32(3.0))
    else:
        denom = np.maximum(w_max.astype(F32) - w_min.astype(F32), F32(1e-8))
        scale = _h(denom / F32(3.0))
    bias = _h(w_min)
    q = _codes(wg.astype(F32), scale, bias, 3.0).astype(np.uint8).reshape(N, K // 4, 4)
    packed = (q[..., 0] & 3) | ((q[..., 1] & 3) << 2) | ((q[..., 2] & 3) << 4) | ((q[..., 3] & 3) << 6)
    sb = np.stack([scale[..., 0], bias[..., 0]], axis=-1).astype(F16)
    return packed.astype(np.uint8), sb


def dequantize_q2_k(packed: np.ndarray, sb: np.ndarray, K: int | None = None):
    N = packed.shape[0]
    K = K or packed.shape[1] * 4
    b = packed.astype(np.int32)[..., None]
    q = ((b >> (2 * np.arange(4))) & 3).reshape(N, K // 64, 64).astype(F32)
    # q.to(fp16) * sc + bi: two fp16 roundings (torch fp16 ops)
    t = _h(q * sb[..., 0:1].astype(F32))
    return _h(t + sb[..., 1:2].astype(F32)).reshape(N, K).astype(F16)


# ---------------------------------------------------------------------------
# GGUF Q2_K super-blocks: ggml's block_q2_K (QK_K = 256, 84 bytes) and its
# published decoder dequantize_row_q2_K (llama.cpp ggml-quants.c); the format is
# not part of the reference's code (its "Q2_K" above is affine group-64).
# ---------------------------------------------------------------------------
Q2K_BLOCK_BYTES = 84  # scales[16] | qs[64] | d fp16 | dmin fp16


def q2k_element_maps():
    """For element e of a block: (qs byte index, bit shift, sub-block index):
    e = 128h + 32j + l -> qs[32h + l] >> 2j, sub-block e // 16."""
    e = np.arange(256)
    h, j, l = e // 128, (e // 32) % 4, e % 32
    return 32 * h + l, 2 * j, e // 16


def pack_q2_k_gguf(weight: np.ndarray) -> np.ndarray:
    """(N, K) -> uint8 (N, K/256, 84), round to nearest (this build's encoder): per
    16-element sub-block m = min(0, min w), scale = (max w - m) / 3; d = fp16(max
    scale / 15), dmin = fp16(max(-m) / 15); 4-bit codes rint(scale / d), rint(-m / dmin)
    clamped to [0, 15]; 2-bit codes rint((w + dmin mc) / (d sc)) clamped to [0, 3]
    (0 where d sc == 0).  fp32, one rounding per operation, rint = half to even."""
    N, K = weight.shape
    assert K % 256 == 0
    NB = K // 256
    w = weight.astype(F32).reshape(N, NB, 16, 16)
    mn = np.minimum(w.min(-1), F32(0))
    mx = w.max(-1)
    sub_scale = ((mx - mn).astype(F32) / F32(3)).astype(F32)
    sub_min = (-mn).astype(F32)
    d = (sub_scale.max(-1) / F32(15)).astype(F32).astype(F16).astype(F32)  # (N, NB)
    dmin = (sub_min.max(-1) / F32(15)).astype(F32).astype(F16).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[..., None] > 0, np.clip(np.rint(sub_scale / d[..., None]), 0, 15), 0).astype(F32)
        mc = np.where(dmin[..., None] > 0, np.clip(np.rint(sub_min / dmin[..., None]), 0, 15), 0).astype(F32)
        dl = (d[..., None] * sc).astype(F32)
        dm = (dmin[..., None] * mc).astype(F32)
        num = (w + dm[..., None]).astype(F32)
        q = np.where(dl[..., None] > 0, np.clip(np.rint(num / dl[..., None]), 0, 3), 0).astype(np.uint8)
    q = q.reshape(N, NB, 256)
    byte_idx, shift, _ = q2k_element_maps()
    qs = np.zeros((N, NB, 64), np.uint8)
    for e in range(256):
        qs[:, :, byte_idx[e]] |= (q[:, :, e] << shift[e]).astype(np.uint8)
    out = np.zeros((N, NB, Q2K_BLOCK_BYTES), np.uint8)
    out[:, :, :16] = (sc.astype(np.uint8) | (mc.astype(np.uint8) << 4))
    out[:, :, 16:80] = qs
    out[:, :, 80:82] = d.astype(F16).view(np.uint8).reshape(N, NB, 2)
    out[:, :, 82:84] = dmin.astype(F16).view(np.uint8).reshape(N, NB, 2)
    return out


def dequantize_q2_k_gguf(blocks: np.ndarray, out_dtype=F16) -> np.ndarray:
    """uint8 (N, K/256, 84) -> (N, K): w = d * (sc & 15) * q - dmin * (sc >> 4) in fp32
    (dl = d * scale and ml = dmin * min first, as the published decoder forms them),
    rounded once to out_dtype."""
    N, NB, _ = blocks.shape
    byte_idx, shift, sub = q2k_element_maps()
    qs = blocks[:, :, 16:80]
    q = ((qs[:, :, byte_idx] >> shift) & 3).astype(F32)  # (N, NB, 256)
    scb = blocks[:, :, :16][:, :, sub]
    d = blocks[:, :, 80:82].copy().view(F16).astype(F32)  # (N, NB, 1)
    dmin = blocks[:, :, 82:84].copy().view(F16).astype(F32)
    dl = (d * (scb & 15).astype(F32)).astype(F32)
    ml = (dmin * (scb >> 4).astype(F32)).astype(F32)
    w = ((dl * q).astype(F32) - ml).astype(F32)
    return w.reshape(N, NB * 256).astype(out_dtype)


# ---------------------------------------------------------------------------
# KV cache quantization -- quant.py:692-852
# ---------------------------------------------------------------------------
def fp8_e4m3fn_from_f32(x: np.ndarray) -> np.ndarray:
    """torch's float -> float8_e4m3fn cast (c10 fp8e4m3fn_from_fp32_value), bitwise."""
    f = np.ascontiguousarray(x, dtype=F32)
    u = f.view(np.uint32).astype(np.uint64)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & 0x7FFFFFFF
    out = np.zeros(f.shape, dtype=np.uint8)
    nan_or_big = a >= 0x43F00000
    normal = (a >= 0x3C800000) & ~nan_or_big
    sub = ~(nan_or_big | normal)
    out[nan_or_big] = 0x7F
    an = a[normal]
    odd = (an >> 20) & 1
    an = an + 0x7FFFF + odd - (120 << 23)
    out[normal] = (an >> 20).astype(np.uint8)
    af = a[sub].astype(np.uint32).view(F32)
    out[sub] = np.rint(af * F32(512.0)).astype(np.uint8)
    return out | sign


def fp8_e4m3fn_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint32)
    sign = np.where(b & 0x80, -1.0, 1.0).astype(F32)
    e = (b >> 3) & 0xF
    m = (b & 7).astype(F32)
    val = np.where(e == 0, m * F32(2.0 ** -9), (1.0 + m / 8.0) * np.exp2(e.astype(F32) - 7.0)).astype(F32)
    val = np.where((b & 0x7F) == 0x7F, np.nan, val).astype(F32)
    return sign * val


def _kv_scale(x16: np.ndarray, div: float):
    """fp16 amax / div rounded to fp16; clamp(min=1e-8) is a no-op in fp16 (quant.py:713-715, 792-794)."""
    xg = x16.reshape(*x16.shape[:-1], -1, 64).astype(F32)
    amax = np.abs(xg).max(axis=-1, keepdims=True)
    return _h(amax / F32(div)), xg


def _fp16_div(xg: np.ndarray, scale: np.ndarray):
    with np.errstate(divide="ignore", invalid="ignore"):
        q = _h(xg / scale)
    # x86 produces a negative quiet NaN for 0/0
    zz = (scale == 0) & (xg == 0)
    q = np.where(zz, np.float32(-np.nan), q).astype(F32)
    if np.any(zz):
        q = q.copy()
        q.view(np.uint32)[zz] = np.uint32(0xFFC00000)
    return q


def quantize_kv_fp8_single(x16: np.ndarray):
    """-> (codes uint8 [..., hd], scales fp16 [..., hd/64]), quant.py:710-720."""
    scale, xg = _kv_scale(x16, 448.0)
    q = _fp16_div(xg, scale)
    return fp8_e4m3fn_from_f32(q).reshape(x16.shape), scale[..., 0].astype(F16)


def dequantize_kv_fp8(codes: np.ndarray, scales: np.ndarray):
    """fp8 -> fp16 (exact) then * fp16 scale (one rounding), quant.py:760-768."""
    cg = codes.reshape(*codes.shape[:-1], -1, 64)
    v = fp8_e4m3fn_to_f32(cg)
    return _h(v * scales[..., None].astype(F32)).reshape(codes.shape).astype(F16)


def quantize_kv_int4_single(x16: np.ndarray):
    """-> (packed uint8 [..., hd/2], scales fp16 [..., hd/64]), quant.py:789-803."""
    scale, xg = _kv_scale(x16, 7.0)
    q = _fp16_div(xg, scale)
    with np.errstate(invalid="ignore"):
        qi = np.clip(np.rint(q), -8, 7)
    qi = np.where(np.isnan(qi), 0, qi).astype(np.int32)
    pairs = qi.reshape(*qi.shape[:-1], 32, 2)
    packed = ((pairs[..., 0] & 0xF) | ((pairs[..., 1] & 0xF) << 4)).astype(np.uint8)
    hd = x16.shape[-1]
    return packed.reshape(*x16.shape[:-1], hd // 2), scale[..., 0].astype(F16)


def dequantize_kv_int4(packed: np.ndarray, scales: np.ndarray):
    """((nib ^ 8) - 8) * scale in fp16, quant.py:843-852."""
    c = packed.reshape(*packed.shape[:-1], -1, 32).astype(np.int32)
    q0 = ((c & 0xF) ^ 8) - 8
    q1 = (((c >> 4) & 0xF) ^ 8) - 8
    q = np.stack([q0, q1], axis=-1).astype(F32)
    out = _h(q * scales[..., None, None].astype(F32))
    return out.reshape(*packed.shape[:-1], packed.shape[-1] * 2).astype(F16)
