"""Decode-path operators (MI355X): KV quantization, split-KV decode attention,
bitmask tree attention, RMSNorm / SwiGLU / argmax.

Mirrors the names and argument meaning of ``axiomlm.kernels.ops`` and the KV
helpers of ``axiomlm.kernels.quant`` (axiomlm/kernels/ops.py:552-797,
axiomlm/kernels/quant.py:692-1008).  All compute runs in libaxm.so.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib

KV_CODES = {"fp16": 0, "fp8": 1, "int4": 2}


def _kv_code(kv_dtype: str) -> int:
    try:
        return KV_CODES[kv_dtype.lower()]
    except KeyError:
        raise ValueError(f"unsupported kv_dtype {kv_dtype!r}") from None


def _check_head_dim(head_dim: int, who: str) -> None:
    # Same argument checks as the reference entry points (ops.py:564-569).
    if head_dim > 128:
        raise ValueError(f"{who} requires head_dim <= 128, got {head_dim}")
    if head_dim % 2 != 0:
        raise ValueError(f"{who} requires even head_dim, got {head_dim}")


# ---------------------------------------------------------------------------
# KV quantization (quant.py:692-852)
# ---------------------------------------------------------------------------
def _quantize_rows(k: torch.Tensor, v: torch.Tensor, code: int):
    _lib.require_gpu(k, "quantize_kv")
    hd = k.size(-1)
    if hd % 64 != 0:
        raise ValueError(f"quantize_kv requires head_dim % 64 == 0, got {hd}")
    R = k.numel() // hd
    kr = k.reshape(R, hd).to(torch.float16).contiguous()
    vr = v.reshape(R, hd).to(torch.float16).contiguous()
    width = hd if code == 1 else hd // 2
    kq = torch.empty((R, width), dtype=torch.uint8, device=k.device)
    vq = torch.empty_like(kq)
    ks = torch.empty((R, hd // 64), dtype=torch.float16, device=k.device)
    vs = torch.empty_like(ks)
    # Rows as slots 0..R-1 of a single-head cache.
    _lib.check(_lib.lib().axm_kv_cache_write(_lib.ptr(kr), _lib.ptr(vr), hd, R, _lib.ptr(kq), _lib.ptr(vq),
                                             _lib.ptr(ks), _lib.ptr(vs), code, 1, hd, R, 0,
                                             _lib.stream_of(k.device)),
               "quantize_kv")
    lead = k.shape[:-1]
    return kq.view(*lead, width), ks.view(*lead, hd // 64), vq.view(*lead, width), vs.view(*lead, hd // 64)


def quantize_kv_fp8(k: torch.Tensor, v: torch.Tensor):
    """-> (k_fp8, k_scales, v_fp8, v_scales): E4M3FN codes + fp16 scales per 64 elements."""
    return _quantize_rows(k, v, 1)


def quantize_kv_int4(k: torch.Tensor, v: torch.Tensor):
    """-> (k_int4, k_scales, v_int4, v_scales): packed signed nibbles + fp16 scales per 64."""
    return _quantize_rows(k, v, 2)


def _dequantize_rows(codes: torch.Tensor, scales: torch.Tensor, hd: int, code: int, who: str) -> torch.Tensor:
    _lib.require_gpu(codes, who)
    c = codes.contiguous()
    sc = scales.to(device=codes.device, dtype=torch.float16).contiguous()
    width = hd if code == 1 else hd // 2
    rows = c.numel() // width
    if sc.numel() != rows * (hd // 64):
        raise ValueError(f"{who}: {sc.numel()} scales for {rows} rows of head_dim {hd}")
    out = torch.empty((*c.shape[:-1], hd), dtype=torch.float16, device=codes.device)
    _lib.check(_lib.lib().axm_dequantize_kv(_lib.ptr(c), _lib.ptr(sc), code, rows, hd, _lib.ptr(out),
                                            _lib.stream_of(codes.device)), who)
    return out


def dequantize_kv_fp8(cache_fp8: torch.Tensor, scales: torch.Tensor, head_dim: int | None = None) -> torch.Tensor:
    """E4M3FN bytes -> fp16 (exact), times the fp16 scale with one rounding (quant.py:727-768)."""
    hd = head_dim or cache_fp8.size(-1)
    return _dequantize_rows(cache_fp8, scales, hd, 1, "dequantize_kv_fp8")


def dequantize_kv_int4(cache_int4: torch.Tensor, scales: torch.Tensor, head_dim: int | None = None) -> torch.Tensor:
    """Packed nibbles ((n ^ 8) - 8) times the fp16 scale (quant.py:810-852)."""
    hd = head_dim or cache_int4.size(-1) * 2
    return _dequantize_rows(cache_int4, scales, hd, 2, "dequantize_kv_int4")


# ---------------------------------------------------------------------------
# Fused bias + RoPE + KV-cache write (quant.py:896-1008; rope_kv_cache_write*_mps,
# rope_tree_kv_*_mps, mps_kernels.mm:788-929, 1005-1140, 3961-3998)
# ---------------------------------------------------------------------------
def _rope_kv_write(who, qkv, freqs_cis, k_cache, v_cache, k_scales, v_scales, q_dim, kv_dim, head_dim, start_pos,
                   write_pos, kv_dtype, qkv_bias, depths):
    _lib.require_gpu(qkv, who)
    code = _kv_code(kv_dtype)
    if qkv.dtype != torch.float16 or not qkv.is_contiguous():
        raise ValueError(f"{who}: qkv must be a contiguous fp16 tensor (updated in place)")
    width = int(q_dim) + 2 * int(kv_dim)
    if qkv.numel() % width:
        raise ValueError(f"{who}: qkv has {qkv.numel()} elements, not a multiple of q_dim + 2 kv_dim = {width}")
    T = qkv.numel() // width
    if depths is not None and len(depths) != T:
        raise ValueError(f"{who}: {len(depths)} tree depths for {T} tokens")
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("k_scales", k_scales), ("v_scales", v_scales)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{who}: {name} must be contiguous (written in place)")
    if code and (k_scales is None or v_scales is None):
        raise ValueError(f"{who}: quantized KV cache needs k_scales and v_scales")
    fr = torch.view_as_real(freqs_cis) if freqs_cis.is_complex() else freqs_cis
    fr = fr.to(device=qkv.device, dtype=torch.float32).contiguous()
    S = k_cache.size(-2)
    bias = qkv_bias.to(device=qkv.device, dtype=torch.float16).contiguous() if qkv_bias is not None else None
    arr = (ctypes.c_int * T)(*[int(d) for d in depths]) if depths is not None else None
    _lib.check(_lib.lib().axm_rope_kv_cache_write(
        _lib.ptr(qkv), T, _lib.ptr(fr), fr.size(0), int(start_pos), arr, _lib.ptr(bias), _lib.ptr(k_cache),
        _lib.ptr(v_cache), _lib.ptr(k_scales if code else None), _lib.ptr(v_scales if code else None), code,
        int(q_dim), int(kv_dim), int(head_dim), S, int(write_pos), _lib.stream_of(qkv.device)), who)


def rope_kv_cache_write_quantized(qkv: torch.Tensor, freqs_cis: torch.Tensor, k_cache: torch.Tensor,
                                  v_cache: torch.Tensor, k_scales: torch.Tensor | None, v_scales: torch.Tensor | None,
                                  q_dim: int, kv_dim: int, head_dim: int, start_pos: int, write_pos: int,
                                  kv_dtype: str = "fp16", qkv_bias: torch.Tensor | None = None) -> None:
    """Fused RoPE + KV-cache write of the qkv rows (1, T, q_dim + 2 kv_dim) (quant.py:896-1008):
    the query part of qkv is biased and rotated in place; token t is rotated at
    start_pos + t and its key / value land at slot write_pos + t of batch 0 (quantized
    per 64-element group for "fp8" / "int4").  freqs_cis: complex (rope_len, hd/2) or its
    real view (rope_len, hd/2, 2)."""
    _rope_kv_write("rope_kv_cache_write_quantized", qkv, freqs_cis, k_cache, v_cache, k_scales, v_scales, q_dim,
                   kv_dim, head_dim, start_pos, write_pos, kv_dtype, qkv_bias, None)


def rope_kv_cache_write(qkv: torch.Tensor, freqs_cis: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        q_dim: int, kv_dim: int, head_dim: int, start_pos: int, write_pos: int,
                        qkv_bias: torch.Tensor | None = None) -> None:
    """fp16-cache form (rope_kv_cache_write_mps, mps_kernels.mm:788-815)."""
    rope_kv_cache_write_quantized(qkv, freqs_cis, k_cache, v_cache, None, None, q_dim, kv_dim, head_dim, start_pos,
                                  write_pos, "fp16", qkv_bias)


def rope_tree_kv_cache_write(qkv: torch.Tensor, freqs_cis: torch.Tensor, k_cache: torch.Tensor,
                             v_cache: torch.Tensor, tree_depths, q_dim: int, kv_dim: int, head_dim: int,
                             start_pos: int, write_pos: int, qkv_bias: torch.Tensor | None = None,
                             k_scales: torch.Tensor | None = None, v_scales: torch.Tensor | None = None,
                             kv_dtype: str = "fp16") -> None:
    """Tree form (rope_tree_kv_cache_write_mps / rope_tree_kv_write_{fp8,int4}_mps,
    mps_kernels.mm:3961-3998, 1005-1140): node t is rotated at start_pos + tree_depths[t]
    and written at slot write_pos + t; up to 64 nodes."""
    _rope_kv_write("rope_tree_kv_cache_write", qkv, freqs_cis, k_cache, v_cache, k_scales, v_scales, q_dim, kv_dim,
                   head_dim, start_pos, write_pos, kv_dtype, qkv_bias, list(tree_depths))


# ---------------------------------------------------------------------------
# Attention (ops.py:552-797)
# ---------------------------------------------------------------------------
def _cache_dims(k_cache: torch.Tensor, code: int):
    kc = k_cache if k_cache.dim() == 4 else k_cache.unsqueeze(0)
    B, Hkv, S, last = kc.shape
    hd = last * 2 if code == 2 else last
    return B, Hkv, S, hd


def gqa_flash_decode_mps(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    active_len: int,
    num_splits: int = 0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
    kv_dtype: str = "fp16",
) -> torch.Tensor:
    """Split-KV GQA decode attention over slots [0, active_len) (ops.py:552-654).

    q: (B, Hq, 1, hd) / (B, Hq, hd) / (Hq, hd) fp16; caches (B, Hkv, S, *) or (Hkv, S, *)."""
    head_dim = q.size(-1)
    _check_head_dim(head_dim, "gqa_flash_decode_mps")
    _lib.require_gpu(q, "gqa_flash_decode_mps")
    code = _kv_code(kv_dtype)
    B, Hkv, S, hd = _cache_dims(k_cache, code)
    n_head = q.numel() // (B * head_dim)
    if code and (k_scales is None or v_scales is None):
        raise ValueError("quantized KV cache needs k_scales and v_scales")
    splits = int(num_splits) if num_splits and num_splits > 0 else _lib.lib().axm_attention_num_splits(
        B, n_head, Hkv, head_dim, code, int(active_len))
    ws_bytes = _lib.lib().axm_attention_workspace_bytes(B, n_head, head_dim, splits)
    ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=q.device) if ws_bytes else None
    qc = q.to(torch.float16).contiguous()
    out = torch.empty_like(qc)
    _lib.check(
        _lib.lib().axm_gqa_flash_decode(
            _lib.ptr(qc), _lib.ptr(k_cache.contiguous()), _lib.ptr(v_cache.contiguous()),
            _lib.ptr(k_scales.contiguous() if code else None), _lib.ptr(v_scales.contiguous() if code else None),
            code, _lib.ptr(out), B, n_head, Hkv, head_dim, S, int(active_len), splits, _lib.ptr(ws), ws_bytes,
            _lib.stream_of(q.device)),
        "gqa_flash_decode_mps",
    )
    return out.view(q.shape)


def _masks_tensor(tree_mask, T: int, device) -> torch.Tensor:
    if isinstance(tree_mask, torch.Tensor) and tree_mask.device == device and tree_mask.dtype == torch.int64:
        # uint64 bit patterns already on the device (no host round trip)
        if tree_mask.numel() != T:
            raise ValueError(f"tree_mask has {tree_mask.numel()} entries for {T} nodes")
        return tree_mask.contiguous()
    if isinstance(tree_mask, torch.Tensor):
        vals = [int(x) for x in tree_mask.cpu().tolist()]
    else:
        vals = [int(x) for x in tree_mask]
    if len(vals) != T:
        raise ValueError(f"tree_mask has {len(vals)} entries for {T} nodes")
    # uint64 bit patterns carried in an int64 tensor
    signed = [v - (1 << 64) if v >= (1 << 63) else v for v in vals]
    return torch.tensor(signed, dtype=torch.int64).to(device)


def gqa_tree_verify_mps(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    tree_mask,
    prefix_len: int,
    write_pos: int,
    n_head: int,
    num_splits: int = 0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
    kv_dtype: str = "fp16",
) -> torch.Tensor:
    """Bitmask tree attention (ops.py:657-797); T <= 64 nodes, uint64 ancestor masks."""
    q_dim = (n_head * q.size(-1)) if q.dim() == 4 else q.size(-1)
    head_dim = q_dim // n_head
    _check_head_dim(head_dim, "gqa_tree_verify_mps")
    _lib.require_gpu(q, "gqa_tree_verify_mps")
    code = _kv_code(kv_dtype)
    B, Hkv, S, hd = _cache_dims(k_cache, code)
    T = len(tree_mask) if not isinstance(tree_mask, torch.Tensor) else tree_mask.numel()
    if q.dim() == 4:  # (1, Hq, T, hd) -> (T, Hq, hd)
        qc = q[0].transpose(0, 1).contiguous()
    else:
        qc = q.reshape(T, n_head, head_dim).contiguous()
    qc = qc.to(torch.float16)
    masks = _masks_tensor(tree_mask, T, q.device)
    splits = int(num_splits) if num_splits and num_splits > 0 else _lib.lib().axm_tree_attention_num_splits(
        T, n_head, Hkv, int(prefix_len) + T)
    ws_bytes = _lib.lib().axm_attention_workspace_bytes(T, n_head, head_dim, splits)
    ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=q.device) if ws_bytes else None
    out = torch.empty_like(qc)
    _lib.check(
        _lib.lib().axm_gqa_tree_verify(
            _lib.ptr(qc), _lib.ptr(k_cache.contiguous()), _lib.ptr(v_cache.contiguous()),
            _lib.ptr(k_scales.contiguous() if code else None), _lib.ptr(v_scales.contiguous() if code else None),
            code, _lib.ptr(out), T, n_head, Hkv, head_dim, S, int(prefix_len), int(write_pos), _lib.ptr(masks),
            splits, _lib.ptr(ws), ws_bytes, _lib.stream_of(q.device)),
        "gqa_tree_verify_mps",
    )
    if q.dim() == 4:
        return out.transpose(0, 1).unsqueeze(0)
    return out.view(q.shape)


# ---------------------------------------------------------------------------
# Tree-path KV compaction (compact_tree_kv{,_quant}_mps, mps_kernels.mm:4066-4110, 4251-4295)
# ---------------------------------------------------------------------------
def compact_tree_kv(cache: torch.Tensor, scales: torch.Tensor | None, write_pos: int, accepted_indices) -> None:
    """Move slot (write_pos + a[m]) % S to (write_pos + m) % S in every (layer, k|v, batch,
    head) row block of a 6-D StaticKVCache tensor (L, 2, B, Hkv, S, width) and, for FP8 /
    INT4 caches, of its scales (L, 2, B, Hkv, S, hd/64); one race-free pass, up to 64
    accepted nodes."""
    acc = [int(a) for a in accepted_indices]
    n = len(acc)
    if n == 0 or all(a == m for m, a in enumerate(acc)):
        return
    _lib.require_gpu(cache, "compact_tree_kv")
    if cache.dim() != 6 or not cache.is_contiguous():
        raise ValueError("compact_tree_kv expects a contiguous 6-D StaticKVCache tensor")
    if scales is not None and (scales.dim() != 6 or not scales.is_contiguous() or
                               tuple(scales.shape[:5]) != tuple(cache.shape[:5])):
        raise ValueError("compact_tree_kv: scales must be a contiguous 6-D tensor over the same slots")
    L, two, B, H, S = cache.shape[:5]
    slot_bytes = cache.shape[5] * cache.element_size()
    halves = scales.shape[5] if scales is not None else 0
    arr = (ctypes.c_int * n)(*acc)
    _lib.check(_lib.lib().axm_compact_tree_kv(_lib.ptr(cache), _lib.ptr(scales), L * two * B * H, S, slot_bytes,
                                              halves, int(write_pos), arr, n, _lib.stream_of(cache.device)),
               "compact_tree_kv")


# ---------------------------------------------------------------------------
# Norms / activations / argmax
# ---------------------------------------------------------------------------
def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Inference RMSNorm on fp16 rows (modules.py:41-43; rmsnorm_infer_mps)."""
    _lib.require_gpu(x, "fused_rmsnorm")
    D = x.size(-1)
    xc = x.to(torch.float16).contiguous()
    w = weight.to(device=x.device, dtype=torch.float16).contiguous()
    y = torch.empty_like(xc)
    _lib.check(_lib.lib().axm_rmsnorm(_lib.ptr(xc), _lib.ptr(w), _lib.ptr(y), xc.numel() // D, D, float(eps),
                                      _lib.stream_of(x.device)), "fused_rmsnorm")
    return y


def add_rmsnorm_infer(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x += residual (in place, fp16); returns RMSNorm(x) (add_rmsnorm_infer_mps)."""
    _lib.require_gpu(x, "add_rmsnorm_infer")
    D = x.size(-1)
    y = torch.empty_like(x)
    _lib.check(_lib.lib().axm_add_rmsnorm(_lib.ptr(x), _lib.ptr(residual.contiguous()),
                                          _lib.ptr(weight.to(torch.float16).contiguous()), _lib.ptr(y),
                                          x.numel() // D, D, float(eps), _lib.stream_of(x.device)),
               "add_rmsnorm_infer")
    return y


def swiglu_gate_up(gu: torch.Tensor) -> torch.Tensor:
    """silu(g) * u over the concatenated [g || u] last dimension (swiglu_gate_up_mps)."""
    _lib.require_gpu(gu, "swiglu_gate_up")
    H = gu.size(-1) // 2
    rows = gu.numel() // (2 * H)
    y = torch.empty((*gu.shape[:-1], H), dtype=torch.float16, device=gu.device)
    _lib.check(_lib.lib().axm_swiglu_gate_up(_lib.ptr(gu.contiguous()), _lib.ptr(y), rows, H,
                                             _lib.stream_of(gu.device)), "swiglu_gate_up")
    return y


def argmax_last_token(logits: torch.Tensor) -> torch.Tensor:
    """Row argmax (lowest index on ties) over the last dim, int64."""
    _lib.require_gpu(logits, "argmax_last_token")
    V = logits.size(-1)
    rows = logits.numel() // V
    out = torch.empty(logits.shape[:-1], dtype=torch.int64, device=logits.device)
    _lib.check(_lib.lib().axm_argmax(_lib.ptr(logits.to(torch.float16).contiguous()), rows, V, _lib.ptr(out),
                                     _lib.stream_of(logits.device)), "argmax_last_token")
    return out
