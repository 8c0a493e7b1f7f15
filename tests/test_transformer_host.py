"""Host side of the decode driver on the CPU: RoPE tables and config rules.

``precompute_rope_frequencies`` (modules.py:46-92) is pinned against the oracle's
closed form for plain RoPE and against the independent implementations of Llama-3
and linear scaling in ``transformers.modeling_rope_utils``."""

import numpy as np
import pytest
import torch

from axiomlm_amd.transformer import ModelConfig, Transformer, precompute_rope_frequencies
from oracle import model as om


def _inv_freq(fr):
    # Row t=1 of the table is (cos w, sin w) for every frequency w.
    return torch.atan2(fr[1, :, 1], fr[1, :, 0])


def test_plain_rope_matches_oracle_tables():
    fr = precompute_rope_frequencies(64, 256, 10000.0)
    assert fr.shape == (256, 32, 2) and fr.dtype == torch.float32 and fr.is_contiguous()
    cos, sin = om.rope_tables(64, 256, 10000.0)
    # The fp32 pow of torch and numpy may differ by an ulp in inv_freq, which moves the angle
    # at position t by up to t ulp: 255 * 2^-24 * 2 ~ 3e-5 rad at most.
    assert np.max(np.abs(fr[..., 0].numpy() - cos)) <= 3e-5
    assert np.max(np.abs(fr[..., 1].numpy() - sin)) <= 3e-5
    assert np.max(np.abs(fr[:8].numpy() - np.stack([cos, sin], -1)[:8])) <= 1e-6
    assert np.all(fr[0, :, 0].numpy() == 1.0) and np.all(fr[0, :, 1].numpy() == 0.0)


@pytest.mark.parametrize(
    "scaling,theta",
    [({"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
       "original_max_position_embeddings": 8192}, 500000.0),
     ({"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
       "original_max_position_embeddings": 8192}, 500000.0),
     ({"type": "linear", "factor": 4.0}, 10000.0)],
)
def test_scaled_rope_matches_transformers(scaling, theta):
    from transformers import LlamaConfig
    import transformers.modeling_rope_utils as ru

    hd = 128
    fr = precompute_rope_frequencies(hd, 4, theta, scaling)
    hf_scaling = dict(scaling)
    hf_scaling["rope_type"] = hf_scaling.pop("type", hf_scaling.get("rope_type"))
    c = LlamaConfig(hidden_size=hd * 4, num_attention_heads=4, rope_theta=theta, rope_scaling=hf_scaling,
                    max_position_embeddings=131072)
    fn = ru._compute_llama3_parameters if hf_scaling["rope_type"] == "llama3" else ru._compute_linear_scaling_rope_parameters
    inv, _ = fn(c, "cpu")
    got = _inv_freq(fr).double()
    assert torch.allclose(got, inv.double(), rtol=2e-6, atol=1e-12)


def test_config_rules():
    c = ModelConfig(n_embd=4096, n_head=32, n_kv_head=8)
    assert c.head_dim == 128 and c.kv_heads == 8
    assert c.hidden == 10944  # int(8/3 * 4096) = 10922 rounded up to 64 (modules.py:151-152)
    assert ModelConfig(n_embd=256, n_head=4, intermediate_size=704).hidden == 704
    assert ModelConfig(n_embd=768, n_head=12).kv_heads == 12
    with pytest.raises(ValueError):
        precompute_rope_frequencies(63)


def test_quantize_modes_and_tied_head():
    c = ModelConfig(n_layer=1, n_embd=64, n_head=1, vocab_size=128, intermediate_size=128)
    sd = {"transformer.wte.weight": torch.zeros(128, 64, dtype=torch.float16)}
    m = Transformer(c, sd, device="cpu")
    assert m.w["lm_head.weight"] is m.w["transformer.wte.weight"]  # tied by default
    for mode in ("q4", "q4_rtn", "q4_k_m", "q8", None):
        m.quantize(mode)
    for mode in ("q4_legacy", "q2_k", "ternary", "int4"):  # not modes of the decode runner
        with pytest.raises(ValueError):
            m.quantize(mode)
    m.quantize("q4_rtn")
    with pytest.raises(RuntimeError):
        Transformer(c, sd, device="cpu").forward(torch.zeros(1, 1, dtype=torch.long), kv_caches=None)
