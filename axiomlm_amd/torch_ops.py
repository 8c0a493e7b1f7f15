"""PyTorch custom operators over libaxm.so: ``torch.ops.axiomlm.<name>``.

The reference binds its kernels as pybind functions taking and returning
torch tensors (axiomlm/kernels/mps_kernels.mm:4300-4641).  Here the same
operations are registered with ``torch.library.custom_op``, so they carry
schemas, go through the dispatcher (``torch.ops.axiomlm.*``) and have fake
(meta) implementations for tracing; each one calls the C ABI of libaxm.so
through the ctypes layer of ``axiomlm_amd.kernels``.  Operators that write
caches in place declare those arguments as mutated.

Tree masks are int64 tensors holding uint64 bit patterns (up to 64 nodes), since
a schema ``int`` is signed 64-bit; ``tree_mask_tensor`` converts a list of
Python ints.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor
from torch.library import custom_op

from .kernels import ops as _ops
from .kernels import quant as _q


def tree_mask_tensor(tree_mask, device) -> Tensor:
    """uint64 ancestor masks -> int64 device tensor with the same bit patterns."""
    vals = [int(x) & 0xFFFFFFFFFFFFFFFF for x in tree_mask]
    signed = [v - (1 << 64) if v >= (1 << 63) else v for v in vals]
    return torch.tensor(signed, dtype=torch.int64).to(device)


def _linear_fake(x: Tensor, n: int) -> Tensor:
    return x.new_empty((*x.shape[:-1], n), dtype=torch.float16)


# ---------------------------------------------------------------------------
# Quantized linear layers
# ---------------------------------------------------------------------------
@custom_op("axiomlm::qmv_q4_marlin", mutates_args=())
def qmv_q4_marlin(x: Tensor, w_marlin: Tensor, sb_marlin: Tensor, out_features: int = -1,
                  bias: Optional[Tensor] = None) -> Tensor:
    """qmv_q4_marlin_mps / qmm_q4_marlin_mps (mps_kernels.mm:3927-3960)."""
    return _q.qmv_q4_marlin(x, w_marlin, sb_marlin, None if out_features < 0 else out_features, bias)


@qmv_q4_marlin.register_fake
def _(x, w_marlin, sb_marlin, out_features=-1, bias=None):
    return _linear_fake(x, w_marlin.shape[0] * 8 if out_features < 0 else out_features)


@custom_op("axiomlm::qmv_q8_g64", mutates_args=())
def qmv_q8_g64(x: Tensor, w_packed: Tensor, scales_biases: Tensor) -> Tensor:
    """qmv_q8_g64_mps / qmm_q8_g64_mps (mps_kernels.mm:3853-3861)."""
    return _q.qmv_q8_g64(x, w_packed, scales_biases)


@qmv_q8_g64.register_fake
def _(x, w_packed, scales_biases):
    return _linear_fake(x, w_packed.shape[0])


@custom_op("axiomlm::qmv_ternary", mutates_args=())
def qmv_ternary(x: Tensor, w_packed: Tensor, scales: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """qmv_ternary_mps / qmm_ternary_mps (metal_kernels.metal:3990-4160)."""
    return _q.qmv_ternary(x, w_packed, scales, bias)


@qmv_ternary.register_fake
def _(x, w_packed, scales, bias=None):
    return _linear_fake(x, w_packed.shape[0])


@custom_op("axiomlm::qmv_q2_k", mutates_args=())
def qmv_q2_k(x: Tensor, w_packed: Tensor, scales_biases: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """qmv_q2_k_mps / qmm_q2_k_mps (metal_kernels.metal:4167-4334)."""
    return _q.qmv_q2_k(x, w_packed, scales_biases, bias)


@qmv_q2_k.register_fake
def _(x, w_packed, scales_biases, bias=None):
    return _linear_fake(x, w_packed.shape[0])


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
@custom_op("axiomlm::gqa_flash_decode", mutates_args=())
def gqa_flash_decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, active_len: int, num_splits: int = 0,
                     k_scales: Optional[Tensor] = None, v_scales: Optional[Tensor] = None,
                     kv_dtype: str = "fp16") -> Tensor:
    """gqa_flash_decode{,_fp8,_int4}_mps (ops.py:552-654)."""
    return _ops.gqa_flash_decode_mps(q, k_cache, v_cache, active_len, num_splits, k_scales, v_scales, kv_dtype)


@gqa_flash_decode.register_fake
def _(q, k_cache, v_cache, active_len, num_splits=0, k_scales=None, v_scales=None, kv_dtype="fp16"):
    return torch.empty_like(q, dtype=torch.float16)


@custom_op("axiomlm::gqa_tree_verify", mutates_args=())
def gqa_tree_verify(q: Tensor, k_cache: Tensor, v_cache: Tensor, tree_mask: Tensor, prefix_len: int,
                    write_pos: int, n_head: int, num_splits: int = 0, k_scales: Optional[Tensor] = None,
                    v_scales: Optional[Tensor] = None, kv_dtype: str = "fp16") -> Tensor:
    """gqa_tree_verify{,_fp8,_int4}_mps (ops.py:657-797); tree_mask: int64 tensor of uint64 masks."""
    return _ops.gqa_tree_verify_mps(q, k_cache, v_cache, tree_mask, prefix_len, write_pos, n_head, num_splits,
                                    k_scales, v_scales, kv_dtype)


@gqa_tree_verify.register_fake
def _(q, k_cache, v_cache, tree_mask, prefix_len, write_pos, n_head, num_splits=0, k_scales=None, v_scales=None,
      kv_dtype="fp16"):
    return torch.empty_like(q, dtype=torch.float16)


# ---------------------------------------------------------------------------
# KV cache writes, compaction, dequantization
# ---------------------------------------------------------------------------
@custom_op("axiomlm::rope_kv_cache_write", mutates_args=("qkv", "k_cache", "v_cache", "k_scales", "v_scales"))
def rope_kv_cache_write(qkv: Tensor, freqs_cis: Tensor, k_cache: Tensor, v_cache: Tensor,
                        k_scales: Optional[Tensor], v_scales: Optional[Tensor], q_dim: int, kv_dim: int,
                        head_dim: int, start_pos: int, write_pos: int, kv_dtype: str = "fp16",
                        qkv_bias: Optional[Tensor] = None, tree_depths: Optional[list[int]] = None) -> None:
    """rope_kv_cache_write{,_fp8,_int4}_mps and the tree forms rope_tree_kv_cache_write_mps /
    rope_tree_kv_write_{fp8,int4}_mps (mps_kernels.mm:788-929, 1005-1140, 3961-3998)."""
    if tree_depths is None:
        _ops.rope_kv_cache_write_quantized(qkv, freqs_cis, k_cache, v_cache, k_scales, v_scales, q_dim, kv_dim,
                                           head_dim, start_pos, write_pos, kv_dtype, qkv_bias)
    else:
        _ops.rope_tree_kv_cache_write(qkv, freqs_cis, k_cache, v_cache, tree_depths, q_dim, kv_dim, head_dim,
                                      start_pos, write_pos, qkv_bias, k_scales, v_scales, kv_dtype)


@custom_op("axiomlm::compact_tree_kv", mutates_args=("cache", "scales"))
def compact_tree_kv(cache: Tensor, scales: Optional[Tensor], write_pos: int, accepted_indices: list[int]) -> None:
    """compact_tree_kv_mps / compact_tree_kv_quant_mps (mps_kernels.mm:4066-4110, 4251-4295)."""
    _ops.compact_tree_kv(cache, scales, write_pos, accepted_indices)


@custom_op("axiomlm::dequantize_kv", mutates_args=())
def dequantize_kv(codes: Tensor, scales: Tensor, head_dim: int, kv_dtype: str) -> Tensor:
    """dequantize_kv_cache_{fp8,int4}_mps (mps_kernels.mm:931-1003)."""
    if kv_dtype == "fp8":
        return _ops.dequantize_kv_fp8(codes, scales, head_dim)
    if kv_dtype == "int4":
        return _ops.dequantize_kv_int4(codes, scales, head_dim)
    raise ValueError(f"dequantize_kv: kv_dtype must be 'fp8' or 'int4', got {kv_dtype!r}")


@dequantize_kv.register_fake
def _(codes, scales, head_dim, kv_dtype):
    return codes.new_empty((*codes.shape[:-1], head_dim), dtype=torch.float16)


# ---------------------------------------------------------------------------
# Norms, SwiGLU, argmax
# ---------------------------------------------------------------------------
@custom_op("axiomlm::rmsnorm_infer", mutates_args=())
def rmsnorm_infer(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """rmsnorm_infer_mps (mps_kernels.mm:398-403)."""
    return _ops.fused_rmsnorm(x, weight, eps)


@rmsnorm_infer.register_fake
def _(x, weight, eps):
    return torch.empty_like(x, dtype=torch.float16)


@custom_op("axiomlm::add_rmsnorm_infer", mutates_args=("x_inout",))
def add_rmsnorm_infer(x_inout: Tensor, residual: Tensor, weight: Tensor, eps: float) -> Tensor:
    """add_rmsnorm_infer_mps (mps_kernels.mm:427-432): x_inout += residual, returns RMSNorm."""
    return _ops.add_rmsnorm_infer(x_inout, residual, weight, eps)


@add_rmsnorm_infer.register_fake
def _(x_inout, residual, weight, eps):
    return torch.empty_like(x_inout)


@custom_op("axiomlm::swiglu_gate_up", mutates_args=())
def swiglu_gate_up(gate_up: Tensor) -> Tensor:
    """swiglu_gate_up_mps (mps_kernels.mm:452-460)."""
    return _ops.swiglu_gate_up(gate_up)


@swiglu_gate_up.register_fake
def _(gate_up):
    return gate_up.new_empty((*gate_up.shape[:-1], gate_up.shape[-1] // 2), dtype=torch.float16)


@custom_op("axiomlm::argmax_rows", mutates_args=())
def argmax_rows(logits: Tensor) -> Tensor:
    """Argmax of every row over the last dimension, lowest index on ties
    (argmax_multi_half_kernel, metal_kernels.metal:455-510)."""
    return _ops.argmax_last_token(logits)


@argmax_rows.register_fake
def _(logits):
    return logits.new_empty(logits.shape[:-1], dtype=torch.int64)
