"""Pins the numpy oracle's formats against the reference's own known-answer tests,
closed forms, invariants and (for torch-defined arithmetic) torch itself.

CPU only.  Reference citations are paths in the AxiomLM source tree.
"""

import struct

import numpy as np
import pytest
import torch

from oracle import formats as fm

F16, F32 = np.float16, np.float32


def test_marlin_magic_nibble_kat():
    # tests/test_phase1_task11_disassembly.py:71-98: (n | 0x6400) - 1024 == n, ((n << 4) | 0x5400) - 64 == n
    for n in range(16):
        lo = struct.unpack("e", struct.pack("<H", n | 0x6400))[0] - 1024.0
        hi = struct.unpack("e", struct.pack("<H", (n << 4) | 0x5400))[0] - 64.0
        assert lo == n and hi == n


def test_marlin_lane_maps_match_kernel_equations():
    # quant.py:573-576 vs the kernel's lane decode (metal_kernels.metal:2159-2161): every (r, c0) pair
    # with c0 in {0,2,4,6} and r in 0..7 appears exactly once over the 32 lanes.
    r, c0 = fm.marlin_lane_maps()
    pairs = set(zip(r.tolist(), c0.tolist()))
    assert len(pairs) == 32
    assert pairs == {(rr, cc) for rr in range(8) for cc in (0, 2, 4, 6)}
    # explicit spot values
    assert (r[0], c0[0]) == (0, 0) and (r[1], c0[1]) == (0, 2) and (r[2], c0[2]) == (1, 0)
    assert (r[8], c0[8]) == (0, 4) and (r[16], c0[16]) == (4, 0) and (r[31], c0[31]) == (7, 6)


def _hand_marlin_code(w_marlin, row, k):
    """Read the code of (row, k) straight from the bit equations of the layout."""
    r_map, c0_map = fm.marlin_lane_maps()
    tile, c = divmod(row, 8)
    g, kk = divmod(k, 64)
    j, rest = divmod(kk, 32)
    s, r = divmod(rest, 8)
    lane = [l for l in range(32) if r_map[l] == r and c0_map[l] in (c, c - 1) and c0_map[l] % 2 == 0][0]
    half = c - c0_map[lane]
    word = int(w_marlin.view(np.uint32)[tile, g, lane, j])
    return (word >> (16 * half + 4 * s)) & 0xF


@pytest.mark.parametrize("N,K", [(16, 128), (13, 192), (8, 704)])
def test_marlin_pack_unpack_bit_equations(N, K):
    rng = np.random.default_rng(N * 1000 + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F16)
    wm, sb = fm.pack_linear_q4_marlin(w, clip_search=False)
    assert wm.shape == ((N + 7) // 8, K // 64, 32, 2) and wm.dtype == np.int32
    assert sb.shape == ((N + 7) // 8, K // 64, 8, 2) and sb.dtype == F16
    codes = fm.unpack_marlin_codes(wm)
    for _ in range(200):
        row, k = int(rng.integers(0, N)), int(rng.integers(0, K))
        assert codes[row, k] == _hand_marlin_code(wm, row, k)


@pytest.mark.parametrize("src", [F16, F32])
def test_rtn_marlin_equals_q4_g64(src):
    # Reference invariant (quant.py:462-463): RTN MARLIN is bit-for-bit the Q4_G64 quantization.
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((40, 256)) * 0.05).astype(src)
    wm, sbm = fm.pack_linear_q4_marlin(w, clip_search=False)
    wq, sbq = fm.pack_linear_q4_g64(w)
    a = fm.dequantize_q4_marlin(wm, sbm, 256, out_features=40)
    b = fm.dequantize_q4_g64(wq, sbq, 256)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_rtn_codes_are_nearest_lattice_points():
    # Brute force: each RTN code minimizes |w - (q*s + b)| over q in 0..15 (ties resolved to even).
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((8, 64)) * 0.03).astype(F32)
    wm, sb = fm.pack_linear_q4_marlin(w, clip_search=False)
    codes = fm.unpack_marlin_codes(wm)[:8].astype(np.int64)
    s = sb[0, 0, :, 0].astype(F32)[:, None]
    b = sb[0, 0, :, 1].astype(F32)[:, None]
    err = np.abs((w[..., None] - b[..., None]) / s[..., None] - np.arange(16, dtype=F32))
    best = err.argmin(-1)
    # where the exact quotient is not a .5 tie the brute-force minimizer must match
    frac = np.abs(((w - b) / s) % 1.0 - 0.5)
    ok = frac > 1e-4
    inside = ((w - b) / s >= -0.5) & ((w - b) / s <= 15.5)
    assert np.array_equal(codes[ok & inside], best[ok & inside])


def test_rtn_scale_bias_closed_form():
    # A group spanning exactly [-0.75, 0.75]: scale = fp16(1.5 / 15) = fp16(0.1), bias = -0.75, codes exact.
    q = np.arange(64) % 16
    w = (-0.75 + q * (1.5 / 15)).astype(F32)[None, :].repeat(8, 0)
    w[:, 0], w[:, 1] = -0.75, 0.75
    wm, sb = fm.pack_linear_q4_marlin(w, clip_search=False)
    assert sb[0, 0, 0, 0] == F16(F32(1.5) / F32(15.0))
    assert sb[0, 0, 0, 1] == F16(-0.75)
    codes = fm.unpack_marlin_codes(wm)[0]
    assert codes[0] == 0 and codes[1] == 15


def test_mse_clip_never_worse_than_rtn():
    # The search includes the full-range candidate (alpha = 1), so its weighted error is <= RTN's.
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((16, 128)) * 0.02).astype(F16)
    imp = np.abs(rng.standard_normal(128)).astype(F32) + 0.1
    wr, sr = fm.pack_linear_q4_marlin(w, clip_search=False)
    wc, sc = fm.pack_linear_q4_marlin(w, clip_search=True, col_importance=imp)
    ig = (imp ** 2).reshape(2, 64)
    ig = ig / ig.mean(-1, keepdims=True)
    ig = ig.reshape(128)
    e_r = (ig * (w.astype(F32) - fm.dequantize_q4_marlin(wr, sr, 128).astype(F32)) ** 2).reshape(16, 2, 64).sum(-1)
    e_c = (ig * (w.astype(F32) - fm.dequantize_q4_marlin(wc, sc, 128).astype(F32)) ** 2).reshape(16, 2, 64).sum(-1)
    assert np.all(e_c <= e_r * (1 + 1e-3) + 1e-12)


def test_mse_alphas_match_torch_linspace():
    # The product passes torch.linspace(1.0, 0.72, 13) (quant.py:512); the oracle's grid must be identical.
    for steps, lo in [(13, 0.72), (2, 0.5), (7, 0.81), (20, 0.6)]:
        assert np.array_equal(fm.linspace_f32(1.0, lo, steps), torch.linspace(1.0, lo, steps=steps).numpy())


def test_ternary_byte_table_and_roundtrips():
    # tests/test_phase3_task33_bitnet_q2k.py:62-108
    dec = fm.ternary_decode_bytes(np.arange(256, dtype=np.uint8))
    assert set(np.unique(dec).tolist()) <= {-1, 0, 1}
    assert dec[0b01].tolist() == [1, 0, 0, 0] and dec[0b10].tolist() == [-1, 0, 0, 0]
    assert dec[0b11].tolist() == [0, 0, 0, 0] and dec[0b10_01_00_10].tolist() == [-1, 0, 1, -1]
    rng = np.random.default_rng(42)
    q = np.where(rng.standard_normal((64, 256)) > 0, 1.0, -1.0).astype(F16)
    w = (q.astype(F32) * 0.75).astype(F16)
    p, s = fm.pack_linear_ternary(w)
    assert p.shape == (64, 64) and p.dtype == np.uint8 and s.shape == (64, 4)
    assert np.array_equal(fm.dequantize_ternary(p, s, 256), w)
    g = rng.standard_normal((64, 256)).astype(F16)
    p, s = fm.pack_linear_ternary(g)
    r = fm.dequantize_ternary(p, s, 256).astype(F32).reshape(64, 4, 64)
    sg = s.astype(F32)[..., None]
    assert np.max(np.abs(r - np.rint(r / sg) * sg)) == 0.0


def test_q2_roundtrip_and_bytes_per_weight():
    # tests/test_phase3_task33_bitnet_q2k.py:110-129 and :321-324
    rng = np.random.default_rng(5)
    q = rng.integers(0, 4, (64, 256)).astype(F32)
    w = (q * 0.5 - 1.0).astype(F16)
    p, sb = fm.pack_linear_q2_k(w)
    assert p.shape == (64, 64) and sb.shape == (64, 4, 2)
    assert np.max(np.abs(fm.dequantize_q2_k(p, sb, 256).astype(F32) - w.astype(F32))) < 1e-3
    N, K = 4096, 11008
    tern = N * K // 4 + N * (K // 64) * 2
    q2 = N * K // 4 + N * (K // 64) * 4
    assert tern / (N * K) == 0.28125 and q2 / (N * K) == 0.3125


def test_q8_pack_closed_form():
    rng = np.random.default_rng(9)
    w = rng.standard_normal((4, 128)).astype(F32)
    p, sb = fm.pack_linear_q8_g64(w)
    d = fm.dequantize_q8_g64(p, sb, 128).astype(F32)
    # error bounded by half a quantization step (+ fp16 rounding of the result)
    step = sb[..., 0].astype(F32).repeat(64, axis=1)
    assert np.all(np.abs(d - w) <= 0.5 * step + np.abs(w) * 2 ** -10 + 1e-6)
    assert p.min() == 0 and p.max() == 255


def test_fp8_encode_matches_torch_on_all_fp16():
    # quant.py:719: float(fp16(x / s)).to(float8_e4m3fn) -- pin the oracle to torch's cast bitwise.
    allh = np.arange(65536, dtype=np.uint16).view(F16).astype(F32)
    ours = fm.fp8_e4m3fn_from_f32(allh)
    ref = torch.from_numpy(allh).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    nan_in = np.isnan(allh)
    assert np.array_equal(ours[~nan_in], ref[~nan_in])
    assert np.all((ours[nan_in] & 0x7F) == 0x7F)


def test_fp8_encode_matches_torch_random_f32():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200000) * np.exp2(rng.integers(-12, 10, 200000))).astype(F32)
    x = np.concatenate([x, np.array([448, 464, 464.01, 479.9, 480, -464, 2 ** -9, 1.5 * 2 ** -10], F32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fm.fp8_e4m3fn_from_f32(x), ref)


def test_fp8_decode_matches_torch():
    b = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(b).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    ours = fm.fp8_e4m3fn_to_f32(b)
    finite = ~np.isnan(ref)
    assert np.array_equal(ours[finite], ref[finite]) and np.all(np.isnan(ours[~finite]))


def test_int4_kv_closed_form_and_lattice_roundtrip():
    # symmetric scale amax/7 per 64 (quant.py:771-807); lattice inputs round-trip exactly
    rng = np.random.default_rng(2)
    q = rng.integers(-7, 8, (3, 5, 128)).astype(F32)
    q[..., 0] = 7
    q[..., 64] = -7
    x = (q * 0.25).astype(F16)  # scale = 1.75 / 7 = 0.25 exactly
    packed, sc = fm.quantize_kv_int4_single(x)
    assert packed.shape == (3, 5, 64) and sc.shape == (3, 5, 2)
    assert np.all(sc == F16(0.25))
    assert np.array_equal(fm.dequantize_kv_int4(packed, sc), x)
    # nibble order: element 2i in the low nibble, 2i+1 in the high nibble, two's complement
    lo = (packed[..., 0] & 0xF).astype(np.int32)
    assert np.array_equal(np.where(lo >= 8, lo - 16, lo), q[..., 0].astype(np.int32))


def test_fp8_kv_scale_and_sqnr():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 4, 128)).astype(F16)
    codes, sc = fm.quantize_kv_fp8_single(x)
    amax = np.abs(x.astype(F32).reshape(8, 4, 2, 64)).max(-1)
    assert np.array_equal(sc, (amax / F32(448.0)).astype(F16))
    d = fm.dequantize_kv_fp8(codes, sc).astype(F32)
    sqnr = 10 * np.log10((x.astype(F32) ** 2).sum() / ((x.astype(F32) - d) ** 2).sum())
    assert sqnr > 30.0  # tests/test_phase3_task31_kv_quantization.py:46-121


def test_kv_zero_group_gives_nan_codes():
    # fp16 clamp(min=1e-8) rounds the bound to 0, so an all-zero group has scale 0 and 0/0 = NaN codes.
    x = np.zeros((1, 64), F16)
    codes, sc = fm.quantize_kv_fp8_single(x)
    assert sc[0, 0] == 0 and np.all(codes == 0xFF)
    t = torch.zeros(1, 64, dtype=torch.float16)
    s_t = torch.clamp(t.abs().amax(dim=-1, keepdim=True) / 448.0, min=1e-8).to(torch.float16)
    assert float(s_t) == 0.0


# ---------------------------------------------------------------------------
# MARLIN Q4 group 128 (the build's variant: group-64 code layout, one scale per 128)
# ---------------------------------------------------------------------------
def test_g128_equals_g64_with_shared_pair_scales():
    # Duplicating each 128-group's (scale, bias) over its two 64-groups gives a group-64 pack
    # that must dequantize bit for bit like the group-128 one (the scale of column k is the
    # one of group k // 128, not k // 64).
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((24, 384)) * 0.03).astype(F16)
    wm, sb128 = fm.pack_linear_q4_marlin_g128(w)
    assert wm.shape == (3, 6, 32, 2) and sb128.shape == (3, 3, 8, 2)
    sb64 = np.repeat(sb128, 2, axis=1)
    a = fm.dequantize_q4_marlin_g128(wm, sb128, 384)
    b = fm.dequantize_q4_marlin(wm, sb64, 384)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    # a matrix whose 64-groups already share (min, max) per 128 packs to the same codes in G64
    w2 = w.copy().reshape(24, 3, 2, 64)
    w2[:, :, :, 0] = w2.reshape(24, 3, 128).min(-1)[:, :, None]
    w2[:, :, :, 1] = w2.reshape(24, 3, 128).max(-1)[:, :, None]
    w2 = w2.reshape(24, 384)
    g64m, g64s = fm.pack_linear_q4_marlin(w2, clip_search=False)
    g128m, g128s = fm.pack_linear_q4_marlin_g128(w2)
    assert np.array_equal(g64m, g128m)
    assert np.array_equal(g64s.view(np.uint16), np.repeat(g128s, 2, axis=1).view(np.uint16))


def test_g128_rtn_closed_form_and_nearest_codes():
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((8, 128)) * 0.05).astype(np.float32)
    wm, sb = fm.pack_linear_q4_marlin_g128(w)
    mn, mx = w.min(-1), w.max(-1)
    assert np.array_equal(sb[0, 0, :, 0], ((mx - mn) / np.float32(15.0)).astype(F16))
    assert np.array_equal(sb[0, 0, :, 1], mn.astype(F16))
    codes = fm.unpack_marlin_codes(wm)[:8].astype(np.int64)
    s = sb[0, 0, :, 0].astype(F32)[:, None]
    b = sb[0, 0, :, 1].astype(F32)[:, None]
    t = (w - b) / s
    best = np.abs(t[..., None] - np.arange(16)).argmin(-1)
    ok = (np.abs(t % 1.0 - 0.5) > 1e-4) & (t > -0.5) & (t < 15.5)
    assert np.array_equal(codes[ok], best[ok])
    # bytes per weight: 4-bit codes + one fp16 scale and bias per 128
    N, K = 4096, 4096
    assert (wm.nbytes / w.size, sb.nbytes / w.size) == (0.5, 4 / 128)
    assert (N * K // 2 + N * K // 128 * 4) / (N * K) == 0.53125


# ---------------------------------------------------------------------------
# GGUF Q2_K super-blocks (ggml block_q2_K)
# ---------------------------------------------------------------------------
def _published_q2k_decode(block: bytes) -> list:
    """ggml's dequantize_row_q2_K for one block, written as its nested loops: two
    halves of 128 elements, each reading 32 qs bytes at shifts 0, 2, 4, 6, sixteen
    elements per scale byte."""
    sc, qs = block[:16], block[16:80]
    d = float(np.frombuffer(block[80:82], np.float16)[0])
    dmin = float(np.frombuffer(block[82:84], np.float16)[0])
    out, is_ = [], 0
    for n in (0, 128):
        q = qs[n // 4:n // 4 + 32]
        for shift in (0, 2, 4, 6):
            for half in (0, 16):
                s = sc[is_]
                is_ += 1
                dl, ml = np.float32(d) * np.float32(s & 0xF), np.float32(dmin) * np.float32(s >> 4)
                for l in range(16):
                    out.append(np.float32(dl * np.float32((q[half + l] >> shift) & 3)) - ml)
    return out


def test_q2k_decoder_matches_published_loop_on_a_hand_assembled_block():
    rng = np.random.default_rng(7)
    blk = bytearray(84)
    blk[:16] = bytes((s % 16) | (((7 * s + 3) % 16) << 4) for s in range(16))
    blk[16:80] = rng.integers(0, 256, 64, dtype=np.uint8).tobytes()
    blk[80:82] = np.float16(0.0371).tobytes()
    blk[82:84] = np.float16(0.0113).tobytes()
    want = np.array(_published_q2k_decode(bytes(blk)), np.float32)
    got = fm.dequantize_q2_k_gguf(np.frombuffer(bytes(blk), np.uint8).reshape(1, 1, 84), np.float32)[0]
    assert np.array_equal(got, want)
    # element 0 is bits 0-1 of qs[0] with scale byte 0; element 37 = 32 * 1 + 5 is bits 2-3 of qs[5]
    # with scale byte 2; element 200 = 128 + 32 * 2 + 8 is bits 4-5 of qs[40] with scale byte 12
    d16, m16 = np.float32(np.float16(0.0371)), np.float32(np.float16(0.0113))
    for e, byte, shift, s in ((0, 0, 0, 0), (37, 5, 2, 2), (200, 40, 4, 12)):
        q = (blk[16 + byte] >> shift) & 3
        val = np.float32(d16 * np.float32(blk[s] & 15)) * np.float32(q) - np.float32(m16 * np.float32(blk[s] >> 4))
        assert got[e] == val, e


def test_q2k_element_map_planted_mistake_is_caught():
    """A decoder that swaps the roles of j and l (element 128h + 4l + j) differs from the
    published loop on a random block."""
    rng = np.random.default_rng(8)
    blk = np.zeros(84, np.uint8)
    blk[:16] = rng.integers(0, 256, 16)
    blk[16:80] = rng.integers(0, 256, 64)
    blk[80:82] = np.frombuffer(np.float16(0.05).tobytes(), np.uint8)
    want = np.array(_published_q2k_decode(blk.tobytes()), np.float32)
    e = np.arange(256)
    wrong_q = (blk[16 + 32 * (e // 128) + (e % 128) // 4] >> (2 * (e % 4))) & 3
    wrong = np.float32(0.05) * (blk[:16][e // 16] & 15).astype(np.float32) * wrong_q
    assert not np.allclose(wrong.astype(np.float32), want)


def _q2k_lattice(rng, N, NB):
    """Weights that sit exactly on a Q2_K lattice the encoder must reproduce: every block has
    a sub-block with scale code 15 and one with min code 15, every sub-block holds codes 0 and 3."""
    d = rng.uniform(2.0 ** -8, 2.0 ** -7, (N, NB)).astype(F16).astype(F32)
    dmin = rng.uniform(2.0 ** -8, 2.0 ** -7, (N, NB)).astype(F16).astype(F32)
    sc = rng.integers(1, 16, (N, NB, 16))
    mc = rng.integers(0, 16, (N, NB, 16))
    sc[..., 0] = 15
    mc[..., 1] = 15
    q = rng.integers(0, 4, (N, NB, 16, 16))
    q[..., 0] = 0
    q[..., 1] = 3
    w = (d[..., None, None] * sc[..., None] * q - (dmin[..., None] * mc)[..., None]).astype(F32)
    return w.reshape(N, NB * 256), d, dmin, sc, mc, q


def test_q2k_lattice_round_trip_and_bytes_per_weight():
    rng = np.random.default_rng(9)
    w, d, dmin, sc, mc, q = _q2k_lattice(rng, 6, 3)
    blocks = fm.pack_q2_k_gguf(w)
    assert blocks.shape == (6, 3, 84) and blocks.nbytes / w.size == 0.328125
    assert np.array_equal(blocks[..., 80:82].copy().view(F16)[..., 0].astype(F32), d)
    assert np.array_equal(blocks[..., 82:84].copy().view(F16)[..., 0].astype(F32), dmin)
    assert np.array_equal(blocks[..., :16], (sc | (mc << 4)).astype(np.uint8))
    assert np.array_equal(fm.dequantize_q2_k_gguf(blocks, F32), w)
    # the C4 shapes: 11008 x 4096 and 4096 x 11008 hold 14,794,752 bytes each
    assert 11008 * (4096 // 256) * 84 == 4096 * (11008 // 256) * 84 == 14794752


def test_q2k_rtn_codes_are_nearest_with_the_quantized_scales():
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((4, 512)) * 0.02).astype(F16)
    blocks = fm.pack_q2_k_gguf(w)
    deq = fm.dequantize_q2_k_gguf(blocks, F32).reshape(4, 2, 16, 16)
    scb = blocks[..., :16]
    d = blocks[..., 80:82].copy().view(F16).astype(F32)
    dmin = blocks[..., 82:84].copy().view(F16).astype(F32)
    dl = d * (scb & 15)
    ml = dmin * (scb >> 4)
    # every weight decodes to a lattice point of its sub-block no farther than any other code's
    lattice = dl[..., None] * np.arange(4, dtype=F32) - ml[..., None]  # (4, 2, 16, 4)
    err = np.abs(w.astype(F32).reshape(4, 2, 16, 16)[..., None] - lattice[..., None, :])
    best = err.min(-1)
    got = np.abs(w.astype(F32).reshape(4, 2, 16, 16) - deq)
    assert np.all(got <= best + 1e-6)
    # the super-block scales are the fp16 maxima over sub-blocks / 15
    wr = w.astype(F32).reshape(4, 2, 16, 16)
    mn = np.minimum(wr.min(-1), 0)
    assert np.array_equal(d[..., 0], (((wr.max(-1) - mn) / F32(3)).astype(F32).max(-1) / F32(15)).astype(F16)
                          .astype(F32))
