"""``axiomlm.kernels``-compatible operator surface backed by libaxm.so (MI355X).

Names, argument order and packed layouts follow axiomlm/kernels/__init__.py:83-129
for the decode path; training-only operators of the reference are not part of
this package.
"""

from .ops import (  # noqa: F401
    add_rmsnorm_infer,
    argmax_last_token,
    dequantize_kv_fp8,
    dequantize_kv_int4,
    fused_rmsnorm,
    gqa_flash_decode_mps,
    gqa_tree_verify_mps,
    quantize_kv_fp8,
    quantize_kv_int4,
    rope_kv_cache_write,
    rope_kv_cache_write_quantized,
    rope_tree_kv_cache_write,
    swiglu_gate_up,
)
from .quant import (  # noqa: F401
    compute_quantization_metrics,
    dequant_q8_rows,
    dequantize_q2_k,
    dequantize_q2_k_gguf,
    dequantize_q4_marlin,
    dequantize_q8_g64,
    dequantize_ternary,
    pack_linear_q2_k,
    pack_linear_q2_k_gguf,
    pack_linear_q4_marlin,
    pack_linear_q8_g64,
    pack_linear_ternary,
    qmm_q4_marlin,
    qmm_q4_tile16,
    qmm_q8_g64,
    qmv_q4_marlin,
    qmv_q8_g64,
    qmv_q4_tile16,
    qmv_ternary,
    qmm_ternary,
    qmv_q2_k,
    qmv_q2_k_gguf,
    qmm_q2_k,
    qmv_q4_tile16_swiglu,
    qmv_q4_marlin_swiglu,
    repack_q4_marlin_tile16,
)
