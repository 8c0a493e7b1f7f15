"""The native module object AxiomLM probes, backed by libaxm.so.

AxiomLM reaches its native decode path through one module object
(``_METAL_MOD``, axiomlm/kernels/ops.py:25, quant.py:14) and feature-probes it
with ``hasattr`` (transformer.py:1234, ops.py:575-611, 690-760,
paged_cache.py:407-430).  ``load_rocm_module()`` returns an object with the
attribute names and argument order of the reference's pybind module
(mps_kernels.mm:4300-4641) for every operation of the decode path, each one
calling a ``torch.ops.axiomlm`` custom operator (``axiomlm_amd.torch_ops``)
or, for the runners, ``QuantizedDecodeRunner`` and the fp16 ``DecodeRunner``.

The fp16 ``MPSDecodeRunner`` is provided by ``DecodeRunner`` (same constructor
and methods).  Names of the reference module that belong to training (backward
kernels, cross entropy, flash attention forward) or to the legacy Q4_G64 layout
are not part of this path and are absent, so the reference's probes fall back
for them as they do on any non-Metal device.
"""

from __future__ import annotations

import types


def _build():
    import torch

    from . import torch_ops  # noqa: F401  (registers torch.ops.axiomlm)
    from .runner import DecodeRunner, QuantizedDecodeRunner

    A = torch.ops.axiomlm

    def _masks(tree_mask, q):
        if isinstance(tree_mask, torch.Tensor) and tree_mask.dtype == torch.int64 and tree_mask.device == q.device:
            return tree_mask
        return torch_ops.tree_mask_tensor(list(tree_mask), q.device)

    def _depths(tree_depths):
        if isinstance(tree_depths, torch.Tensor):
            return [int(d) for d in tree_depths.cpu().tolist()]
        return [int(d) for d in tree_depths]

    # -- quantized linear layers (mps_kernels.mm:4470-4480, 4620-4641) --------
    def qmv_q4_marlin_mps(x, w_marlin, sb_marlin, out_features=-1, bias=None):
        return A.qmv_q4_marlin(x, w_marlin, sb_marlin, int(out_features), bias)

    def qmm_q4_marlin_mps(x, w_marlin, sb_marlin, out_features=-1, bias=None):
        return A.qmv_q4_marlin(x, w_marlin, sb_marlin, int(out_features), bias)

    def qmv_q8_g64_mps(x, w_packed, scales_biases):
        return A.qmv_q8_g64(x, w_packed, scales_biases)

    def qmm_q8_g64_mps(x, w_packed, scales_biases):
        return A.qmv_q8_g64(x, w_packed, scales_biases)

    def qmv_ternary_mps(x, w_packed, scales, bias=None):
        return A.qmv_ternary(x, w_packed, scales, bias)

    def qmm_ternary_mps(x, w_packed, scales, bias=None):
        return A.qmv_ternary(x, w_packed, scales, bias)

    def qmv_q2_k_mps(x, w_packed, scales_biases, bias=None):
        return A.qmv_q2_k(x, w_packed, scales_biases, bias)

    def qmm_q2_k_mps(x, w_packed, scales_biases, bias=None):
        return A.qmv_q2_k(x, w_packed, scales_biases, bias)

    # -- attention (mps_kernels.mm:4481-4490, 4577-4618) -------------------------
    def gqa_flash_decode_mps(q, k_cache, v_cache, active_len, num_splits=0):
        return A.gqa_flash_decode(q, k_cache, v_cache, int(active_len), int(num_splits))

    def gqa_flash_decode_fp8_mps(q, k_cache, v_cache, k_scales, v_scales, active_len, num_splits=0):
        return A.gqa_flash_decode(q, k_cache, v_cache, int(active_len), int(num_splits), k_scales, v_scales, "fp8")

    def gqa_flash_decode_int4_mps(q, k_cache, v_cache, k_scales, v_scales, active_len, num_splits=0):
        return A.gqa_flash_decode(q, k_cache, v_cache, int(active_len), int(num_splits), k_scales, v_scales, "int4")

    def gqa_tree_verify_mps(q, k_cache, v_cache, tree_mask, prefix_len, write_pos, n_head, num_splits=0):
        return A.gqa_tree_verify(q, k_cache, v_cache, _masks(tree_mask, q), int(prefix_len), int(write_pos),
                                 int(n_head), int(num_splits))

    def gqa_tree_verify_fp8_mps(q, k_cache, v_cache, k_scales, v_scales, tree_mask, prefix_len, write_pos, n_head,
                                num_splits=0):
        return A.gqa_tree_verify(q, k_cache, v_cache, _masks(tree_mask, q), int(prefix_len), int(write_pos),
                                 int(n_head), int(num_splits), k_scales, v_scales, "fp8")

    def gqa_tree_verify_int4_mps(q, k_cache, v_cache, k_scales, v_scales, tree_mask, prefix_len, write_pos, n_head,
                                 num_splits=0):
        return A.gqa_tree_verify(q, k_cache, v_cache, _masks(tree_mask, q), int(prefix_len), int(write_pos),
                                 int(n_head), int(num_splits), k_scales, v_scales, "int4")

    # -- fused RoPE + KV-cache writes (mps_kernels.mm:788-929, 1005-1140, 3961-3998) --
    def rope_kv_cache_write_mps(qkv, freqs_cis, k_cache, v_cache, q_dim, kv_dim, head_dim, start_pos, write_pos,
                                qkv_bias=None):
        A.rope_kv_cache_write(qkv, freqs_cis, k_cache, v_cache, None, None, int(q_dim), int(kv_dim), int(head_dim),
                              int(start_pos), int(write_pos), "fp16", qkv_bias, None)

    def rope_kv_cache_write_fp8_mps(qkv, freqs_cis, k_cache_fp8, v_cache_fp8, k_scales, v_scales, q_dim, kv_dim,
                                    head_dim, start_pos, write_pos, qkv_bias=None):
        A.rope_kv_cache_write(qkv, freqs_cis, k_cache_fp8, v_cache_fp8, k_scales, v_scales, int(q_dim), int(kv_dim),
                              int(head_dim), int(start_pos), int(write_pos), "fp8", qkv_bias, None)

    def rope_kv_cache_write_int4_mps(qkv, freqs_cis, k_cache_int4, v_cache_int4, k_scales, v_scales, q_dim, kv_dim,
                                     head_dim, start_pos, write_pos, qkv_bias=None):
        A.rope_kv_cache_write(qkv, freqs_cis, k_cache_int4, v_cache_int4, k_scales, v_scales, int(q_dim),
                              int(kv_dim), int(head_dim), int(start_pos), int(write_pos), "int4", qkv_bias, None)

    def rope_tree_kv_cache_write_mps(qkv, freqs_cis, k_cache, v_cache, tree_depths, q_dim, kv_dim, head_dim,
                                     start_pos, write_pos, qkv_bias=None):
        A.rope_kv_cache_write(qkv, freqs_cis, k_cache, v_cache, None, None, int(q_dim), int(kv_dim), int(head_dim),
                              int(start_pos), int(write_pos), "fp16", qkv_bias, _depths(tree_depths))

    def rope_tree_kv_write_fp8_mps(qkv, freqs_cis, k_cache_fp8, v_cache_fp8, k_scales, v_scales, tree_depths, q_dim,
                                   kv_dim, head_dim, start_pos, write_pos, T, qkv_bias=None):
        A.rope_kv_cache_write(qkv, freqs_cis, k_cache_fp8, v_cache_fp8, k_scales, v_scales, int(q_dim), int(kv_dim),
                              int(head_dim), int(start_pos), int(write_pos), "fp8", qkv_bias,
                              _depths(tree_depths)[:int(T)])

    def rope_tree_kv_write_int4_mps(qkv, freqs_cis, k_cache_int4, v_cache_int4, k_scales, v_scales, tree_depths,
                                    q_dim, kv_dim, head_dim, start_pos, write_pos, T, qkv_bias=None):
        A.rope_kv_cache_write(qkv, freqs_cis, k_cache_int4, v_cache_int4, k_scales, v_scales, int(q_dim),
                              int(kv_dim), int(head_dim), int(start_pos), int(write_pos), "int4", qkv_bias,
                              _depths(tree_depths)[:int(T)])

    # -- compaction and dequantization (mps_kernels.mm:4066-4110, 4251-4295, 931-1003) --
    def compact_tree_kv_mps(cache, write_pos, accepted_indices):
        A.compact_tree_kv(cache, None, int(write_pos), [int(a) for a in accepted_indices])

    def compact_tree_kv_quant_mps(cache, scales, write_pos, accepted_indices, cache_dtype="fp8"):
        if cache_dtype not in ("fp8", "int4"):
            raise ValueError(f"compact_tree_kv_quant_mps: cache_dtype must be 'fp8' or 'int4', got {cache_dtype!r}")
        A.compact_tree_kv(cache, scales, int(write_pos), [int(a) for a in accepted_indices])

    def dequantize_kv_cache_fp8_mps(cache_fp8, scales, n_kv_head, seq_len, head_dim):
        return A.dequantize_kv(cache_fp8, scales, int(head_dim), "fp8")

    def dequantize_kv_cache_int4_mps(cache_int4, scales, n_kv_head, seq_len, head_dim):
        return A.dequantize_kv(cache_int4, scales, int(head_dim), "int4")

    # -- norms, SwiGLU, argmax (mps_kernels.mm:292-304, 398-460) -----------------
    def rmsnorm_infer_mps(x, weight, eps):
        return A.rmsnorm_infer(x, weight, float(eps))

    def add_rmsnorm_infer_mps(x_inout, residual, weight, eps):
        return A.add_rmsnorm_infer(x_inout, residual, weight, float(eps))

    def swiglu_gate_up_mps(gate_up):
        return A.swiglu_gate_up(gate_up)

    def argmax_last_token_mps(logits):
        """Greedy token of the last row, (1, 1) int64."""
        last = logits.reshape(-1, logits.size(-1))[-1:]
        return A.argmax_rows(last).view(1, 1)

    names = {k: v for k, v in locals().items() if k.endswith("_mps")}
    return types.SimpleNamespace(MPSQuantizedDecodeRunner=QuantizedDecodeRunner, MPSDecodeRunner=DecodeRunner,
                                 **names)


def load_rocm_module(require_device: bool = True):
    """The module object, or None when no ROCm device is present (``require_device``)."""
    import torch

    if require_device and (getattr(torch.version, "hip", None) is None or not torch.cuda.is_available()):
        return None
    return _build()
