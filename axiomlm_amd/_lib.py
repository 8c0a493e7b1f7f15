"""ctypes binding of libaxm.so (the C ABI declared in include/axm.h).

torch is imported first so that the library binds to the HIP runtime torch
already loaded (same SONAME), sharing device memory and streams with it.
There is no fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading libaxm.so)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaxm.so")

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_float = ctypes.c_float
c_size_t = ctypes.c_size_t
c_long = ctypes.c_long
c_int64 = ctypes.c_int64

_SIGNATURES = {
    "axm_last_error": (ctypes.c_char_p, []),
    "axm_version": (c_int, []),
    "axm_qmv_q4_marlin": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "axm_qmv_q4_marlin_swiglu": (
        c_int, [c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]
    ),
    "axm_tile16_bytes": (c_size_t, [c_int, c_int, c_int]),
    "axm_repack_q4_marlin_tile16": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_qmv_q4_tile16": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]
    ),
    "axm_repack_q4_marlin_g128_tile16": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_pack_q4_marlin_rtn_g128": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_dequantize_q4_marlin_g128": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "axm_compact_tree_kv": (
        c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(c_int), c_int, c_void_p]
    ),
    "axm_qmv_ternary": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "axm_qmv_q2_k": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "axm_pack_q2_k_gguf": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "axm_dequantize_q2_k_gguf": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "axm_qmv_q2_k_gguf": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "axm_qmv_q4_tile16_swiglu": (
        c_int, [c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]
    ),
    "axm_qmm_q4_tile16_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "axm_qmm_q4_tile16": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_size_t, c_void_p],
    ),
    "axm_qmm_q4_tile16_swiglu": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_size_t, c_void_p]
    ),
    "axm_dequantize_q4_marlin": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "axm_pack_q4_marlin_rtn": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_pack_q4_marlin_mse": (
        c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p]
    ),
    "axm_pack_q8_g64": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_pack_q2_k": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_pack_ternary": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "axm_qmv_q8_g64": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "axm_embed_q8_g64": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "axm_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "axm_add_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "axm_swiglu_gate_up": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "axm_argmax": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "axm_kv_cache_write": (
        c_int,
        [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
         c_void_p],
    ),
    "axm_dequantize_kv": (c_int, [c_void_p, c_void_p, c_int, c_long, c_int, c_void_p, c_void_p]),
    "axm_rope_kv_cache_write": (
        c_int,
        [c_void_p, c_int, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
         c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "axm_attention_num_splits": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "axm_attention_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "axm_tree_attention_num_splits": (c_int, [c_int, c_int, c_int, c_int]),
    "axm_gqa_flash_decode": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_void_p, c_size_t, c_void_p],
    ),
    "axm_gqa_flash_decode_noalloc": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_void_p],
    ),
    "axm_gqa_tree_verify": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_void_p, c_int, c_void_p, c_size_t, c_void_p],
    ),
    "axm_runner_create": (c_int, [c_void_p, c_void_p]),
    "axm_runner_destroy": (None, [c_void_p]),
    "axm_runner_step": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_void_p, c_void_p]),
    "axm_runner_verify_step": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "axm_runner_verify_tree_step": (
        c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, ctypes.POINTER(c_int),
                ctypes.POINTER(ctypes.c_uint64), c_void_p, c_void_p]
    ),
    "axm_runner_speculative_decode": (
        c_int, [c_void_p, ctypes.POINTER(c_int64), c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(c_int64), c_int,
                ctypes.POINTER(c_int64), c_void_p]
    ),
    "axm_runner_last_norm": (c_int, [c_void_p, c_void_p]),
    "axm_runner_persistent_words": (c_int, [c_void_p, c_void_p, c_void_p]),
    "axm_runner_token_slot": (c_int, [c_void_p, c_void_p]),
    "axm_runner_time_kernels": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, ctypes.POINTER(c_float)]),
    "axm_runner_set_graph": (c_int, [c_void_p, c_int]),
    "axm_runner_set_mode": (c_int, [c_void_p, c_int]),
    "axm_runner_get_mode": (c_int, [c_void_p]),
    "axm_runner_check": (c_int, [c_void_p]),
}


class RunnerDesc(ctypes.Structure):
    """Mirror of axm_runner_desc (include/axm.h)."""

    _fields_ = [
        ("n_layer", c_int), ("n_head", c_int), ("n_kv_head", c_int), ("head_dim", c_int), ("d_model", c_int),
        ("hidden_dim", c_int), ("vocab_size", c_int), ("max_seq_len", c_int), ("rope_len", c_int),
        ("eps", c_float), ("kv_dtype", c_int),
        ("wte_format", c_int), ("wte", c_void_p), ("wte_sb", c_void_p),
        ("lm_head_format", c_int), ("lm_head_w", c_void_p), ("lm_head_sb", c_void_p),
        ("freqs", c_void_p), ("lnf_w", c_void_p),
        ("ln1_w", ctypes.POINTER(c_void_p)), ("ln2_w", ctypes.POINTER(c_void_p)),
        ("qkv_w", ctypes.POINTER(c_void_p)), ("qkv_sb", ctypes.POINTER(c_void_p)),
        ("qkv_bias", ctypes.POINTER(c_void_p)),
        ("o_w", ctypes.POINTER(c_void_p)), ("o_sb", ctypes.POINTER(c_void_p)),
        ("gu_w", ctypes.POINTER(c_void_p)), ("gu_sb", ctypes.POINTER(c_void_p)),
        ("down_w", ctypes.POINTER(c_void_p)), ("down_sb", ctypes.POINTER(c_void_p)),
        ("k_cache", ctypes.POINTER(c_void_p)), ("v_cache", ctypes.POINTER(c_void_p)),
        ("k_scales", ctypes.POINTER(c_void_p)), ("v_scales", ctypes.POINTER(c_void_p)),
        ("max_tokens", c_int), ("layout", c_int), ("group_size", c_int),
        ("qkv_format", c_int), ("o_format", c_int), ("gu_format", c_int), ("down_format", c_int),
    ]


_LIB = None


def lib():
    """Load libaxm.so once; raises RuntimeError when it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m axiomlm_amd.build` "
                "(the MI355X path has no CPU fallback)"
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def exported_symbols():
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().axm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t) -> c_void_p | None:
    return None if t is None else c_void_p(t.data_ptr())


def stream_of(device=None) -> c_void_p:
    return c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(t, what: str) -> None:
    if not (isinstance(t, torch.Tensor) and t.device.type == "cuda"):
        raise RuntimeError(f"{what}: expected a tensor on a ROCm (cuda) device, got {getattr(t, 'device', type(t))}")
