"""Packed weight formats and quantized GEMV/GEMM entry points (MI355X).

Drop-in mirror of ``axiomlm.kernels.quant`` (axiomlm/kernels/quant.py): same
function names, argument meaning, packed layouts and return shapes.  Packers
and products run as HIP kernels on the ROCm device; CPU inputs are moved to
the current device, packed there and returned on the caller's device.  There
is no CPU fallback: without libaxm.so every call raises.
"""

from __future__ import annotations

import torch

from .. import _lib

__all__ = [
    "pack_linear_q4_marlin",
    "dequantize_q4_marlin",
    "qmv_q4_marlin",
    "qmm_q4_marlin",
    "repack_q4_marlin_tile16",
    "qmv_q4_tile16",
    "qmv_ternary",
    "qmm_ternary",
    "qmv_q2_k",
    "qmm_q2_k",
    "qmv_q4_marlin_swiglu",
    "qmv_q4_tile16_swiglu",
    "pack_linear_q8_g64",
    "dequantize_q8_g64",
    "dequant_q8_rows",
    "qmv_q8_g64",
    "qmm_q8_g64",
    "pack_linear_ternary",
    "dequantize_ternary",
    "pack_linear_q2_k",
    "dequantize_q2_k",
    "compute_quantization_metrics",
]


def _gpu_src(weight: torch.Tensor, what: str):
    if weight.ndim != 2:
        raise AssertionError(f"Expected 2D weight matrix, got shape {tuple(weight.shape)}")
    N, K = weight.shape
    if K % 64 != 0:
        raise AssertionError(f"K ({K}) must be an exact multiple of group size 64")
    dev = weight.device if weight.device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
    if not torch.cuda.is_available():
        raise RuntimeError(f"{what}: no ROCm device available (the MI355X build has no CPU path)")
    src = weight.detach().to(dev)
    if src.dtype not in (torch.float16, torch.float32):
        src = src.float()
    return src.contiguous(), dev, int(N), int(K)


# ---------------------------------------------------------------------------
# MARLIN Q4  (quant.py:447-684)
# ---------------------------------------------------------------------------
def pack_linear_q4_marlin(
    weight: torch.Tensor,
    clip_search: bool = True,
    col_importance: torch.Tensor | None = None,
    grid_steps: int = 13,
    min_shrink: float = 0.72,
    group_size: int = 64,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K) -> w_marlin int32 (ceil(N/8), K/64, 32, 2), sb_marlin fp16 (ceil(N/8), K/64, 8, 2).

    clip_search=False and no importance: round-to-nearest (quant.py:482-494);
    otherwise the importance-weighted MSE clip search (quant.py:495-571).
    group_size=128 (this build's extension, round to nearest only): the same code
    layout with one (scale, bias) per 128 columns, sb fp16 (ceil(N/8), K/128, 8, 2)."""
    if group_size not in (64, 128):
        raise ValueError(f"pack_linear_q4_marlin: group_size must be 64 or 128, got {group_size}")
    if group_size == 128 and (clip_search or col_importance is not None):
        raise ValueError("pack_linear_q4_marlin: group_size=128 packs by round to nearest (clip_search=False)")
    src, dev, N, K = _gpu_src(weight, "pack_linear_q4_marlin")
    if K % group_size != 0:
        raise AssertionError(f"K ({K}) must be an exact multiple of group size {group_size}")
    nt, KG = (N + 7) // 8, K // 64
    w_m = torch.empty((nt, KG, 32, 2), dtype=torch.int32, device=dev)
    sb_m = torch.empty((nt, K // group_size, 8, 2), dtype=torch.float16, device=dev)
    s = _lib.stream_of(dev)
    is16 = int(src.dtype == torch.float16)
    if group_size == 128:
        _lib.check(_lib.lib().axm_pack_q4_marlin_rtn_g128(_lib.ptr(src), is16, N, K, _lib.ptr(w_m), _lib.ptr(sb_m),
                                                          s), "pack_linear_q4_marlin")
    elif not clip_search and col_importance is None:
        _lib.check(_lib.lib().axm_pack_q4_marlin_rtn(_lib.ptr(src), is16, N, K, _lib.ptr(w_m), _lib.ptr(sb_m), s),
                   "pack_linear_q4_marlin")
    else:
        imp = None
        if col_importance is not None:
            if col_importance.numel() != K:
                raise AssertionError(f"Expected col_importance of length {K}, got {col_importance.numel()}")
            imp = col_importance.detach().to(device=dev, dtype=torch.float32).reshape(K).contiguous()
        # fp32 shrink grid exactly as torch.linspace produces it (quant.py:512)
        alphas = torch.linspace(1.0, min_shrink, steps=max(2, grid_steps)).to(dev)
        _lib.check(
            _lib.lib().axm_pack_q4_marlin_mse(_lib.ptr(src), is16, N, K, _lib.ptr(imp), _lib.ptr(alphas),
                                              int(alphas.numel()), _lib.ptr(w_m), _lib.ptr(sb_m), s),
            "pack_linear_q4_marlin",
        )
    if weight.device.type != "cuda":
        return w_m.to(weight.device), sb_m.to(weight.device)
    return w_m, sb_m


def marlin_group_size(w_marlin, sb_marlin) -> int:
    """64 (reference layout) or 128 (one (scale, bias) per 128 columns), from the packed shapes."""
    KG64, KGs = int(w_marlin.shape[1]), int(sb_marlin.shape[1])
    if KGs == KG64:
        return 64
    if 2 * KGs == KG64:
        return 128
    raise ValueError(f"MARLIN scales cover {KGs} groups for {KG64} 64-column blocks")


def dequantize_q4_marlin(w_marlin, sb_marlin, K: int, out_features: int | None = None) -> torch.Tensor:
    """Packed MARLIN -> fp16 (N, K), quant.py:597-634 (group 64 or, from the scale shape, 128)."""
    _lib.require_gpu(w_marlin, "dequantize_q4_marlin")
    nt, KG = int(w_marlin.shape[0]), int(w_marlin.shape[1])
    if KG * 64 != K:
        raise AssertionError(f"Expected K={KG * 64}, got {K}")
    N = nt * 8
    out = torch.empty((N, K), dtype=torch.float16, device=w_marlin.device)
    fn = (_lib.lib().axm_dequantize_q4_marlin_g128 if marlin_group_size(w_marlin, sb_marlin) == 128
          else _lib.lib().axm_dequantize_q4_marlin)
    _lib.check(fn(_lib.ptr(w_marlin.contiguous()), _lib.ptr(sb_marlin.contiguous()), _lib.ptr(out), K, N,
                  _lib.stream_of(w_marlin.device)), "dequantize_q4_marlin")
    if out_features is not None and out_features < N:
        out = out[:out_features]
    return out


def qmv_q4_marlin(x, w_marlin, sb_marlin, out_features: int | None = None, bias=None) -> torch.Tensor:
    """y = x @ W^T (+ bias) for fp16 x (..., K); M > 1 rows are batched (quant.py:637-661)."""
    _lib.require_gpu(x, "qmv_q4_marlin")
    if x.dtype != torch.float16:
        raise RuntimeError("qmv_q4_marlin: x must be float16")
    K = x.size(-1)
    M = x.numel() // K
    nt, KG = int(w_marlin.shape[0]), int(w_marlin.shape[1])
    if KG * 64 != K:
        raise RuntimeError(f"qmv_q4_marlin: K={K} does not match packed K={KG * 64}")
    N = nt * 8 if (out_features is None or out_features < 0) else int(out_features)
    if N > nt * 8:
        raise RuntimeError(f"qmv_q4_marlin: out_features={N} exceeds packed rows {nt * 8}")
    if marlin_group_size(w_marlin, sb_marlin) != 64:
        raise RuntimeError("qmv_q4_marlin: group-128 packs run on the tile16 copy (repack_q4_marlin_tile16, "
                           "qmv_q4_tile16)")
    xc = x.contiguous()
    y = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=x.device)
    b = None
    if bias is not None:
        b = bias.to(device=x.device, dtype=torch.float16).contiguous()
    _lib.check(_lib.lib().axm_qmv_q4_marlin(_lib.ptr(xc), _lib.ptr(w_marlin.contiguous()),
                                            _lib.ptr(sb_marlin.contiguous()), _lib.ptr(b), _lib.ptr(y), M, K, N,
                                            _lib.stream_of(x.device)),
               "qmv_q4_marlin")
    return y


def qmm_q4_marlin(x, w_marlin, sb_marlin, out_features: int | None = None, bias=None) -> torch.Tensor:
    """Batched form of :func:`qmv_q4_marlin` (quant.py:664-684)."""
    return qmv_q4_marlin(x, w_marlin, sb_marlin, out_features, bias)


def repack_q4_marlin_tile16(w_marlin, sb_marlin, N: int, K: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Bit-exact re-tiling of a MARLIN matrix for the matrix-core GEMV (the layout
    the decode runner streams); returns (w16 int32, sb16 fp16) flat buffers.  A
    group-128 pack keeps one (scale, bias) per row and 128 columns (half the sb16)."""
    _lib.require_gpu(w_marlin, "repack_q4_marlin_tile16")
    L = _lib.lib()
    g128 = marlin_group_size(w_marlin, sb_marlin) == 128
    w16 = torch.empty(L.axm_tile16_bytes(N, K, 0) // 4, dtype=torch.int32, device=w_marlin.device)
    sb16 = torch.empty(L.axm_tile16_bytes(N, K, 2 if g128 else 1) // 2, dtype=torch.float16, device=w_marlin.device)
    fn = L.axm_repack_q4_marlin_g128_tile16 if g128 else L.axm_repack_q4_marlin_tile16
    _lib.check(fn(_lib.ptr(w_marlin.contiguous()), _lib.ptr(sb_marlin.contiguous()), N, K, _lib.ptr(w16),
                  _lib.ptr(sb16), _lib.stream_of(w_marlin.device)), "repack_q4_marlin_tile16")
    return w16, sb16


def tile16_group_size(w16, sb16) -> int:
    """64 or 128, from the byte ratio of a tile16 copy's codes to its scales: every
    (16-row tile, 128-column block) holds 1024 code bytes and 128 (group 64) or 64
    (group 128) scale bytes, whatever the number of tiles the copy was made for."""
    wb = w16.numel() * w16.element_size()
    sbb = sb16.numel() * sb16.element_size()
    if wb > 0 and wb == 8 * sbb:
        return 64
    if wb > 0 and wb == 16 * sbb:
        return 128
    raise ValueError(f"tile16 copy: {wb} code bytes and {sbb} scale bytes match neither group size")


def _qmm_workspace(K: int, N: int, swiglu: bool, device):
    n = _lib.lib().axm_qmm_q4_tile16_workspace_bytes(K, N, int(swiglu))
    return (torch.empty(n, dtype=torch.uint8, device=device) if n else None), n


# Rows from which the tile16 entry points run the multi-token GEMM instead of the decode
# GEMV, as the runner's verify steps do (a 7B layer of these calls at three rows: GEMV
# 53.0 us, GEMM 60.7 us; at four: GEMV 62.5 us, GEMM 60.5 us).
TILE16_GEMM_MIN_ROWS = 4


def qmv_q4_tile16(x, w16, sb16, out_features: int, bias=None) -> torch.Tensor:
    """y = x @ W^T (+ bias) on a tile16 copy made by :func:`repack_q4_marlin_tile16`: the
    decode GEMV for up to three rows, the multi-token GEMM (up to 64 rows per weight pass)
    from four."""
    _lib.require_gpu(x, "qmv_q4_tile16")
    K = x.size(-1)
    M = x.numel() // K
    N = int(out_features)
    y = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=x.device)
    b = None if bias is None else bias.to(device=x.device, dtype=torch.float16).contiguous()
    xc = x.contiguous()
    gs = tile16_group_size(w16, sb16)
    if M < TILE16_GEMM_MIN_ROWS:
        _lib.check(_lib.lib().axm_qmv_q4_tile16(_lib.ptr(xc), _lib.ptr(w16), _lib.ptr(sb16), _lib.ptr(b),
                                                _lib.ptr(y), M, K, N, gs, _lib.stream_of(x.device)),
                   "qmv_q4_tile16")
        return y
    ws, n = _qmm_workspace(K, N, False, x.device)
    _lib.check(_lib.lib().axm_qmm_q4_tile16(_lib.ptr(xc), _lib.ptr(w16), _lib.ptr(sb16), _lib.ptr(b), _lib.ptr(y),
                                            M, K, N, gs, _lib.ptr(ws), n, _lib.stream_of(x.device)),
               "qmm_q4_tile16")
    return y


def qmm_q4_tile16(x, w16, sb16, out_features: int, bias=None) -> torch.Tensor:
    """Multi-token form of :func:`qmv_q4_tile16` (the qmm_q4_marlin role, quant.py:664-684)."""
    return qmv_q4_tile16(x, w16, sb16, out_features, bias)


def _swiglu_call(fn, name, x, ln_w, eps, w, sb, H, group_size=None):
    _lib.require_gpu(x, name)
    K = x.size(-1)
    M = x.numel() // K
    if x.dtype != torch.float16 or not 1 <= M <= 4:
        raise RuntimeError(f"{name}: x must be float16 with 1..4 rows")
    y = torch.empty((*x.shape[:-1], int(H)), dtype=torch.float16, device=x.device)
    lw = None if ln_w is None else ln_w.to(device=x.device, dtype=torch.float16).contiguous()
    extra = () if group_size is None else (int(group_size),)
    _lib.check(fn(_lib.ptr(x.contiguous()), _lib.ptr(lw), float(eps), _lib.ptr(w.contiguous()),
                  _lib.ptr(sb.contiguous()), _lib.ptr(y), M, K, int(H), *extra, _lib.stream_of(x.device)), name)
    return y


def qmv_q4_marlin_swiglu(x, ln_w, eps: float, gu_w, gu_sb, H: int) -> torch.Tensor:
    """silu(g) * u of [g | u] = rmsnorm(x) @ [W_gate; W_up]^T, one launch (the MLP input of a
    decoder layer, transformer.py:1178-1189); ``ln_w`` None skips the norm."""
    return _swiglu_call(_lib.lib().axm_qmv_q4_marlin_swiglu, "qmv_q4_marlin_swiglu", x, ln_w, eps, gu_w, gu_sb, H)


def qmv_q4_tile16_swiglu(x, ln_w, eps: float, gu16, gusb16, H: int) -> torch.Tensor:
    """:func:`qmv_q4_marlin_swiglu` on the tile16 copy of the packed [W_gate; W_up] (H % 16 == 0);
    from four rows on they are normalized first and go through the multi-token GEMM."""
    K = x.size(-1)
    M = x.numel() // K
    gs = tile16_group_size(gu16, gusb16)
    if M < TILE16_GEMM_MIN_ROWS:
        return _swiglu_call(_lib.lib().axm_qmv_q4_tile16_swiglu, "qmv_q4_tile16_swiglu", x, ln_w, eps, gu16, gusb16,
                            H, gs)
    from .ops import fused_rmsnorm

    _lib.require_gpu(x, "qmv_q4_tile16_swiglu")
    if x.dtype != torch.float16:
        raise RuntimeError("qmv_q4_tile16_swiglu: x must be float16")
    xn = (fused_rmsnorm(x.reshape(M, K), ln_w, eps) if ln_w is not None else x.reshape(M, K)).contiguous()
    y = torch.empty((*x.shape[:-1], int(H)), dtype=torch.float16, device=x.device)
    ws, n = _qmm_workspace(K, int(H), True, x.device)
    _lib.check(_lib.lib().axm_qmm_q4_tile16_swiglu(_lib.ptr(xn), _lib.ptr(gu16.contiguous()),
                                                   _lib.ptr(gusb16.contiguous()), _lib.ptr(y), M, K, int(H), gs,
                                                   _lib.ptr(ws), n, _lib.stream_of(x.device)),
               "qmm_q4_tile16_swiglu")
    return y


# ---------------------------------------------------------------------------
# Q8_G64  (quant.py:72-233)
# ---------------------------------------------------------------------------
def pack_linear_q8_g64(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K) -> packed int32 (N, K/4) (little-endian bytes), scales_biases fp16 (N, K/64, 2)."""
    src, dev, N, K = _gpu_src(weight, "pack_linear_q8_g64")
    packed = torch.empty((N, K // 4), dtype=torch.int32, device=dev)
    sb = torch.empty((N, K // 64, 2), dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().axm_pack_q8_g64(_lib.ptr(src), int(src.dtype == torch.float16), N, K, _lib.ptr(packed),
                                          _lib.ptr(sb), _lib.stream_of(dev)),
               "pack_linear_q8_g64")
    if weight.device.type != "cuda":
        return packed.to(weight.device), sb.to(weight.device)
    return packed, sb


def dequantize_q8_g64(w_packed, scales_biases, K: int) -> torch.Tensor:
    """fp16(q * scale + bias) in fp32 (quant.py:114-129)."""
    N = w_packed.shape[0]
    q = w_packed.contiguous().view(torch.uint8).view(N, K // 64, 64).float()
    sb = scales_biases.float()
    return (q * sb[..., 0:1] + sb[..., 1:2]).view(N, K).to(torch.float16)


def dequant_q8_rows(indices, w_packed, scales_biases) -> torch.Tensor:
    """Gather + dequantize token rows (quant.py:132-163) with the HIP gather kernel."""
    _lib.require_gpu(w_packed, "dequant_q8_rows")
    K = w_packed.shape[1] * 4
    flat = indices.reshape(-1).to(device=w_packed.device, dtype=torch.int64).contiguous()
    out = torch.empty((flat.numel(), K), dtype=torch.float16, device=w_packed.device)
    _lib.check(_lib.lib().axm_embed_q8_g64(_lib.ptr(w_packed.contiguous()), _lib.ptr(scales_biases.contiguous()),
                                           _lib.ptr(flat), _lib.ptr(out), int(flat.numel()), K,
                                           int(w_packed.shape[0]), _lib.stream_of(w_packed.device)),
               "dequant_q8_rows")
    return out.view(*indices.shape, K)


def qmv_q8_g64(x, w_packed, scales_biases, bias=None) -> torch.Tensor:
    """y = x @ W^T (+ bias, this build's addition) with Q8_G64 weights (quant.py:201-218)."""
    _lib.require_gpu(x, "qmv_q8_g64")
    K = x.size(-1)
    M = x.numel() // K
    N = w_packed.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=x.device)
    b = None if bias is None else bias.to(device=x.device, dtype=torch.float16).contiguous()
    _lib.check(_lib.lib().axm_qmv_q8_g64(_lib.ptr(x.contiguous()), _lib.ptr(w_packed.contiguous()),
                                         _lib.ptr(scales_biases.contiguous()), _lib.ptr(b), _lib.ptr(y), M, K, N,
                                         _lib.stream_of(x.device)),
               "qmv_q8_g64")
    return y


def qmm_q8_g64(x, w_packed, scales_biases) -> torch.Tensor:
    return qmv_q8_g64(x, w_packed, scales_biases)


# ---------------------------------------------------------------------------
# Ternary / reference Q2_K packers  (quant.py:236-403)
# ---------------------------------------------------------------------------
def pack_linear_ternary(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K) -> packed uint8 (N, K/4), scales fp16 (N, K/64)."""
    src, dev, N, K = _gpu_src(weight, "pack_linear_ternary")
    packed = torch.empty((N, K // 4), dtype=torch.uint8, device=dev)
    scales = torch.empty((N, K // 64), dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().axm_pack_ternary(_lib.ptr(src), int(src.dtype == torch.float16), N, K, _lib.ptr(packed),
                                           _lib.ptr(scales), _lib.stream_of(dev)),
               "pack_linear_ternary")
    if weight.device.type != "cuda":
        return packed.to(weight.device), scales.to(weight.device)
    return packed, scales


def dequantize_ternary(w_packed, scales, K: int | None = None) -> torch.Tensor:
    N = w_packed.shape[0]
    K = K or w_packed.shape[1] * 4
    b = w_packed.unsqueeze(-1).to(torch.int32)
    shifts = torch.arange(4, device=w_packed.device, dtype=torch.int32) * 2
    q = ((b >> shifts) & 1) - ((b >> (shifts + 1)) & 1)
    q = q.view(N, K // 64, 64).to(scales.dtype)
    return (q * scales.unsqueeze(-1)).view(N, K).to(torch.float16)


def pack_linear_q2_k(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K) -> packed uint8 (N, K/4), scales_biases fp16 (N, K/64, 2)."""
    src, dev, N, K = _gpu_src(weight, "pack_linear_q2_k")
    packed = torch.empty((N, K // 4), dtype=torch.uint8, device=dev)
    sb = torch.empty((N, K // 64, 2), dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().axm_pack_q2_k(_lib.ptr(src), int(src.dtype == torch.float16), N, K, _lib.ptr(packed),
                                        _lib.ptr(sb), _lib.stream_of(dev)),
               "pack_linear_q2_k")
    if weight.device.type != "cuda":
        return packed.to(weight.device), sb.to(weight.device)
    return packed, sb


def dequantize_q2_k(w_packed, scales_biases, K: int | None = None) -> torch.Tensor:
    N = w_packed.shape[0]
    K = K or w_packed.shape[1] * 4
    b = w_packed.unsqueeze(-1).to(torch.int32)
    shifts = torch.arange(4, device=w_packed.device, dtype=torch.int32) * 2
    q = ((b >> shifts) & 3).view(N, K // 64, 64).to(scales_biases.dtype)
    return (q * scales_biases[..., 0:1] + scales_biases[..., 1:2]).view(N, K).to(torch.float16)


def _lowbit_qmv(fn, name, x, w_packed, s, bias):
    _lib.require_gpu(x, name)
    if x.dtype != torch.float16:
        raise RuntimeError(f"{name}: x must be float16")
    K = x.size(-1)
    M = x.numel() // K
    N = int(w_packed.shape[0])
    if int(w_packed.shape[1]) * 4 != K:
        raise RuntimeError(f"{name}: K={K} does not match packed K={int(w_packed.shape[1]) * 4}")
    y = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=x.device)
    b = None if bias is None else bias.to(device=x.device, dtype=torch.float16).contiguous()
    _lib.check(fn(_lib.ptr(x.contiguous()), _lib.ptr(w_packed.contiguous()), _lib.ptr(s.contiguous()), _lib.ptr(b),
                  _lib.ptr(y), M, K, N, _lib.stream_of(x.device)), name)
    return y


def qmv_ternary(x, w_packed, scales, bias=None) -> torch.Tensor:
    """y = x @ W^T (+ bias) on BitNet 1.58 ternary rows (quant.py:298-318); M > 1 rows batched."""
    return _lowbit_qmv(_lib.lib().axm_qmv_ternary, "qmv_ternary", x, w_packed, scales, bias)


def qmm_ternary(x, w_packed, scales, bias=None) -> torch.Tensor:
    """Batched form of :func:`qmv_ternary` (quant.py:321-336)."""
    return qmv_ternary(x, w_packed, scales, bias)


def qmv_q2_k(x, w_packed, scales_biases, bias=None) -> torch.Tensor:
    """y = x @ W^T (+ bias) on reference affine 2-bit rows (quant.py:406-426)."""
    return _lowbit_qmv(_lib.lib().axm_qmv_q2_k, "qmv_q2_k", x, w_packed, scales_biases, bias)


def qmm_q2_k(x, w_packed, scales_biases, bias=None) -> torch.Tensor:
    """Batched form of :func:`qmv_q2_k` (quant.py:429-444)."""
    return qmv_q2_k(x, w_packed, scales_biases, bias)


# ---------------------------------------------------------------------------
# GGUF Q2_K super-blocks (ggml block_q2_K; no counterpart in the reference)
# ---------------------------------------------------------------------------
Q2K_GGUF_BLOCK_BYTES = 84


def pack_linear_q2_k_gguf(weight: torch.Tensor) -> torch.Tensor:
    """(N, K) fp16/fp32, K % 256 == 0 -> uint8 (N, K/256, 84) GGUF Q2_K blocks (round to nearest)."""
    src, dev, N, K = _gpu_src(weight, "pack_linear_q2_k_gguf")
    if K % 256:
        raise RuntimeError(f"pack_linear_q2_k_gguf: K={K} is not a multiple of 256")
    blocks = torch.empty((N, K // 256, Q2K_GGUF_BLOCK_BYTES), dtype=torch.uint8, device=dev)
    _lib.check(_lib.lib().axm_pack_q2_k_gguf(_lib.ptr(src), int(src.dtype == torch.float16), N, K, _lib.ptr(blocks),
                                             _lib.stream_of(dev)),
               "pack_linear_q2_k_gguf")
    return blocks.to(weight.device) if weight.device.type != "cuda" else blocks


def _q2k_shape(blocks, name):
    if blocks.dtype != torch.uint8 or blocks.dim() != 3 or blocks.shape[2] != Q2K_GGUF_BLOCK_BYTES:
        raise RuntimeError(f"{name}: blocks must be uint8 (N, K/256, 84)")
    return int(blocks.shape[0]), int(blocks.shape[1]) * 256


def dequantize_q2_k_gguf(blocks) -> torch.Tensor:
    """GGUF Q2_K blocks -> fp16 (N, K): d * (sc & 15) * q - dmin * (sc >> 4) in fp32."""
    _lib.require_gpu(blocks, "dequantize_q2_k_gguf")
    N, K = _q2k_shape(blocks, "dequantize_q2_k_gguf")
    out = torch.empty((N, K), dtype=torch.float16, device=blocks.device)
    _lib.check(_lib.lib().axm_dequantize_q2_k_gguf(_lib.ptr(blocks.contiguous()), N, K, _lib.ptr(out),
                                                   _lib.stream_of(blocks.device)),
               "dequantize_q2_k_gguf")
    return out


def qmv_q2_k_gguf(x, blocks, bias=None) -> torch.Tensor:
    """y = x @ W^T (+ bias) on GGUF Q2_K blocks; x fp16 (..., K), any number of rows."""
    _lib.require_gpu(x, "qmv_q2_k_gguf")
    if x.dtype != torch.float16:
        raise RuntimeError("qmv_q2_k_gguf: x must be float16")
    N, K = _q2k_shape(blocks, "qmv_q2_k_gguf")
    if x.size(-1) != K:
        raise RuntimeError(f"qmv_q2_k_gguf: x has K={x.size(-1)}, blocks hold K={K}")
    M = x.numel() // K
    y = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=x.device)
    b = None if bias is None else bias.to(device=x.device, dtype=torch.float16).contiguous()
    _lib.check(_lib.lib().axm_qmv_q2_k_gguf(_lib.ptr(x.contiguous()), _lib.ptr(blocks.contiguous()), _lib.ptr(b),
                                            _lib.ptr(y), M, K, N, _lib.stream_of(x.device)),
               "qmv_q2_k_gguf")
    return y


def compute_quantization_metrics(orig, dequant, quant_bytes: int | None = None) -> dict:
    """SQNR / cosine / MSE / L_inf / compression ratio (quant.py:855-893)."""
    o = orig.flatten().float()
    d = dequant.flatten().float()
    noise = o - d
    sig = o.pow(2).sum()
    npow = noise.pow(2).sum().clamp(min=1e-12)
    ob = orig.numel() * orig.element_size()
    return {
        "sqnr_db": float(10.0 * torch.log10(sig / npow)),
        "cosine_similarity": float(torch.cosine_similarity(o, d, dim=0)),
        "mse": float(noise.pow(2).mean()),
        "max_abs_error": float(noise.abs().max()),
        "orig_bytes": ob,
        "quant_bytes": quant_bytes or ob,
        "compression_ratio": float(ob) / float(quant_bytes) if quant_bytes else 1.0,
    }
