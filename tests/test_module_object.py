"""The drop-in module object (axiomlm_amd.rocm_module) and the torch custom operators
it calls (axiomlm_amd.torch_ops), on the CPU: every name the reference probes or
calls on its native module is present with the reference's parameter names and
order, and the custom operators are registered with shape-correct fake kernels.

Reference names and parameters: the pybind module of
axiomlm/kernels/mps_kernels.mm:4300-4641 (pybind11::arg lists, else the C++
parameter names of the bound function).
"""

import inspect

import pytest
import torch

# name -> parameters, in order (extra trailing parameters of ours must have defaults)
REFERENCE_SIGNATURES = {
    "qmv_q4_marlin_mps": ["x", "w_marlin", "sb_marlin", "out_features", "bias"],  # :4470-4474
    "qmm_q4_marlin_mps": ["x", "w_marlin", "sb_marlin", "out_features", "bias"],  # :4475-4480
    "qmv_q8_g64_mps": ["x", "w_packed", "scales_biases"],  # :3853
    "qmm_q8_g64_mps": ["x", "w_packed", "scales_biases"],
    "qmv_ternary_mps": ["x", "w_packed", "scales", "bias"],  # :4617-4622
    "qmm_ternary_mps": ["x", "w_packed", "scales", "bias"],
    "qmv_q2_k_mps": ["x", "w_packed", "scales_biases", "bias"],  # :4629-4641
    "qmm_q2_k_mps": ["x", "w_packed", "scales_biases", "bias"],
    "gqa_flash_decode_mps": ["q", "k_cache", "v_cache", "active_len", "num_splits"],  # :1633-1638
    "gqa_flash_decode_fp8_mps": ["q", "k_cache", "v_cache", "k_scales", "v_scales", "active_len", "num_splits"],
    "gqa_flash_decode_int4_mps": ["q", "k_cache", "v_cache", "k_scales", "v_scales", "active_len", "num_splits"],
    "gqa_tree_verify_mps": ["q", "k_cache", "v_cache", "tree_mask", "prefix_len", "write_pos", "n_head",
                            "num_splits"],  # :4482-4490
    "gqa_tree_verify_fp8_mps": ["q", "k_cache", "v_cache", "k_scales", "v_scales", "tree_mask", "prefix_len",
                                "write_pos", "n_head", "num_splits"],  # :4594-4605
    "gqa_tree_verify_int4_mps": ["q", "k_cache", "v_cache", "k_scales", "v_scales", "tree_mask", "prefix_len",
                                 "write_pos", "n_head", "num_splits"],
    "rope_kv_cache_write_mps": ["qkv", "freqs_cis", "k_cache", "v_cache", "q_dim", "kv_dim", "head_dim",
                                "start_pos", "write_pos"],  # :788-797
    "rope_kv_cache_write_fp8_mps": ["qkv", "freqs_cis", "k_cache_fp8", "v_cache_fp8", "k_scales", "v_scales",
                                    "q_dim", "kv_dim", "head_dim", "start_pos", "write_pos", "qkv_bias"],
    "rope_kv_cache_write_int4_mps": ["qkv", "freqs_cis", "k_cache_int4", "v_cache_int4", "k_scales", "v_scales",
                                     "q_dim", "kv_dim", "head_dim", "start_pos", "write_pos", "qkv_bias"],
    "rope_tree_kv_cache_write_mps": ["qkv", "freqs_cis", "k_cache", "v_cache", "tree_depths", "q_dim", "kv_dim",
                                     "head_dim", "start_pos", "write_pos", "qkv_bias"],
    "rope_tree_kv_write_fp8_mps": ["qkv", "freqs_cis", "k_cache_fp8", "v_cache_fp8", "k_scales", "v_scales",
                                   "tree_depths", "q_dim", "kv_dim", "head_dim", "start_pos", "write_pos", "T",
                                   "qkv_bias"],
    "rope_tree_kv_write_int4_mps": ["qkv", "freqs_cis", "k_cache_int4", "v_cache_int4", "k_scales", "v_scales",
                                    "tree_depths", "q_dim", "kv_dim", "head_dim", "start_pos", "write_pos", "T",
                                    "qkv_bias"],
    "compact_tree_kv_mps": ["cache", "write_pos", "accepted_indices"],  # :4066-4069
    "compact_tree_kv_quant_mps": ["cache", "scales", "write_pos", "accepted_indices", "cache_dtype"],
    "dequantize_kv_cache_fp8_mps": ["cache_fp8", "scales", "n_kv_head", "seq_len", "head_dim"],
    "dequantize_kv_cache_int4_mps": ["cache_int4", "scales", "n_kv_head", "seq_len", "head_dim"],
    "rmsnorm_infer_mps": ["x", "weight", "eps"],  # :398
    "add_rmsnorm_infer_mps": ["x_inout", "residual", "weight", "eps"],  # :427
    "swiglu_gate_up_mps": ["gate_up"],  # :452
    "argmax_last_token_mps": ["logits"],  # :292
}

# hasattr probes on the module: ops.py:575, 590, 603, 693, 711, 727; transformer.py:1234;
# paged_cache.py:410; quant.py:747, 830
PROBED = ["gqa_flash_decode_fp8_mps", "gqa_flash_decode_int4_mps", "gqa_flash_decode_mps",
          "gqa_tree_verify_fp8_mps", "gqa_tree_verify_int4_mps", "gqa_tree_verify_mps",
          "MPSQuantizedDecodeRunner", "compact_tree_kv_quant_mps", "dequantize_kv_cache_fp8_mps",
          "dequantize_kv_cache_int4_mps"]


@pytest.fixture(scope="module")
def mod():
    from axiomlm_amd.rocm_module import load_rocm_module

    return load_rocm_module(require_device=False)


def test_every_probed_name_is_present(mod):
    missing = [n for n in PROBED if not hasattr(mod, n)]
    assert not missing, missing


@pytest.mark.parametrize("name", sorted(REFERENCE_SIGNATURES))
def test_parameters_follow_the_reference(mod, name):
    params = list(inspect.signature(getattr(mod, name)).parameters.values())
    want = REFERENCE_SIGNATURES[name]
    assert [p.name for p in params[:len(want)]] == want
    assert all(p.default is not inspect.Parameter.empty for p in params[len(want):])


def test_runner_class_signature(mod):
    params = list(inspect.signature(mod.MPSQuantizedDecodeRunner.__init__).parameters)[1:]
    # the 26 constructor arguments of mps_kernels.mm:4404-4456, then keyword extensions
    assert params[:26] == ["wte_emb", "lmh_packed", "lmh_sb", "freqs_r", "ln1_ws", "c_attn_p", "c_attn_s",
                           "c_proj_p", "c_proj_s", "ln2_ws", "gate_up_p", "gate_up_s", "w_down_p", "w_down_s",
                           "lnf_w", "k_cs", "v_cs", "n_h", "n_kvh", "hd", "use_q4", "epsilon", "c_attn_bs",
                           "vocab_sz", "wte_p", "wte_s"]
    for meth in ("step", "verify_step", "verify_tree_step", "speculative_decode", "get_last_norm"):
        assert callable(getattr(mod.MPSQuantizedDecodeRunner, meth))


def test_fp16_runner_class_signature(mod):
    params = list(inspect.signature(mod.MPSDecodeRunner.__init__).parameters)[1:]
    # MPSDecodeRunner's constructor (mps_kernels.mm:4328-4373): 15 positional arguments, then
    # lm_head_w and c_attn_bs
    assert params[:17] == ["wte_w", "freqs_r", "ln1_ws", "c_attn_ws", "c_proj_ws", "ln2_ws", "gate_up_ws",
                           "w_down_ws", "lnf_w", "k_cs", "v_cs", "n_h", "n_kvh", "hd", "epsilon", "lm_head_w",
                           "c_attn_bs"]
    for meth in ("step", "verify_step", "verify_tree_step", "speculative_decode", "get_last_norm"):
        assert callable(getattr(mod.MPSDecodeRunner, meth))


def test_no_device_means_no_module():
    from axiomlm_amd.rocm_module import load_rocm_module

    if not torch.cuda.is_available():
        assert load_rocm_module() is None


def test_custom_ops_registered_with_fake_shapes(mod):
    from torch._subclasses.fake_tensor import FakeTensorMode

    A = torch.ops.axiomlm
    for op in ("qmv_q4_marlin", "qmv_q8_g64", "qmv_ternary", "qmv_q2_k", "gqa_flash_decode", "gqa_tree_verify",
               "rope_kv_cache_write", "compact_tree_kv", "dequantize_kv", "rmsnorm_infer", "add_rmsnorm_infer",
               "swiglu_gate_up", "argmax_rows"):
        assert hasattr(A, op), op
    schema = str(A.rope_kv_cache_write.default._schema)
    assert "Tensor(a0!) qkv" in schema and "Tensor(a2!) k_cache" in schema
    with FakeTensorMode():
        x = torch.empty(3, 256, dtype=torch.float16)
        w = torch.empty(13, 4, 32, 2, dtype=torch.int32)  # 104 packed rows
        sb = torch.empty(13, 4, 8, 2, dtype=torch.float16)
        assert tuple(A.qmv_q4_marlin(x, w, sb).shape) == (3, 104)
        assert tuple(A.qmv_q4_marlin(x, w, sb, 100).shape) == (3, 100)
        assert tuple(A.qmv_q8_g64(x, torch.empty(40, 64, dtype=torch.int32),
                                  torch.empty(40, 4, 2, dtype=torch.float16)).shape) == (3, 40)
        assert tuple(A.swiglu_gate_up(torch.empty(2, 5, 64, dtype=torch.float16)).shape) == (2, 5, 32)
        assert tuple(A.argmax_rows(torch.empty(4, 7, dtype=torch.float16)).shape) == (4,)
        codes = torch.empty(2, 9, 64, dtype=torch.uint8)
        assert tuple(A.dequantize_kv(codes, torch.empty(2, 9, 2, dtype=torch.float16), 128, "int4").shape) == (2, 9,
                                                                                                             128)


def test_tree_mask_tensor_keeps_64_bit_patterns():
    from axiomlm_amd.torch_ops import tree_mask_tensor

    masks = [1, (1 << 63) | 1, (1 << 64) - 1]
    t = tree_mask_tensor(masks, torch.device("cpu"))
    assert t.dtype == torch.int64
    assert [int(v) & 0xFFFFFFFFFFFFFFFF for v in t.tolist()] == masks
