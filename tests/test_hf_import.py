"""HuggingFace safetensors import (axiomlm_amd/hf_import.py) against HuggingFace's own models.

The pins are independent of the reference: tiny LlamaForCausalLM / Qwen2ForCausalLM models
built by `transformers` (random init, no download) are saved with ``save_pretrained``; the
imported weights, run through the oracle's CPU decode path (oracle/model.py, fp16 weights),
must reproduce the logits of the HuggingFace model itself, which uses the half-split RoPE
convention, so a wrong row permutation, q/k/v order or gate/up order fails.  The
permutation is also checked directly: interleaved RoPE of the permuted projection equals
the permuted half-split RoPE (transformers' ``apply_rotary_pos_emb``), and the inverse
permutation restores the input.
"""

import numpy as np
import pytest
import torch

from axiomlm_amd.hf_import import (build_model_config_from_hf, load_hf_safetensors, permute_hf_rope_bias,
                                   permute_hf_rope_weight, unpermute_hf_rope_weight)
from oracle import model as om

transformers = pytest.importorskip("transformers")


def test_permutation_round_trip_and_closed_form():
    w = torch.arange(2 * 8 * 3, dtype=torch.float32).reshape(16, 3)
    p = permute_hf_rope_weight(w, 2, 8)
    assert torch.equal(unpermute_hf_rope_weight(p, 2, 8), w)
    # head 0 rows 0, 4, 1, 5, 2, 6, 3, 7; head 1 the same + 8
    assert p[:, 0].tolist() == [3 * r for r in (0, 4, 1, 5, 2, 6, 3, 7, 8, 12, 9, 13, 10, 14, 11, 15)]
    b = torch.arange(16.0)
    assert torch.equal(permute_hf_rope_bias(b, 2, 8), p[:, 0] / 3)


def test_interleaved_rope_of_permuted_rows_equals_half_split_rope():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    torch.manual_seed(0)
    H, hd, K, pos = 3, 16, 24, 37
    W = torch.randn(H * hd, K, dtype=torch.float64)
    x = torch.randn(K, dtype=torch.float64)
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    ang = pos * inv
    emb = torch.cat([ang, ang])  # HF cos/sin layout [hd]
    q_hf = (W @ x).view(1, H, 1, hd)
    rot_hf, _ = apply_rotary_pos_emb(q_hf, q_hf, emb.cos().view(1, 1, hd), emb.sin().view(1, 1, hd))
    q_il = (permute_hf_rope_weight(W, H, hd) @ x).view(H, hd // 2, 2)
    c, s = ang.cos(), ang.sin()
    rot_il = torch.stack([q_il[..., 0] * c - q_il[..., 1] * s, q_il[..., 0] * s + q_il[..., 1] * c], -1).view(-1)
    want = permute_hf_rope_weight(rot_hf.reshape(H * hd, 1), H, hd).view(-1)
    assert torch.allclose(rot_il, want, atol=1e-12)


def _oracle_from(model):
    """The imported state dict as oracle fp16 weights."""
    c, w = model.config, model.w
    cfg = om.OracleConfig(n_layer=c.n_layer, n_head=c.n_head, n_kv_head=c.kv_heads, d_model=c.n_embd,
                          hidden=c.hidden, vocab=c.vocab_size, eps=c.rms_norm_eps, block_size=c.block_size)
    f = lambda k: w[k].to(torch.float16).cpu().numpy()  # noqa: E731
    ow = om.OracleWeights(f("transformer.wte.weight"), None, f("lm_head.weight"), None, [], [], f("transformer.ln_f.weight"),
                          [], [], [], [], [], [], [], [])
    for i in range(c.n_layer):
        p = f"transformer.h.{i}."
        ow.ln1.append(f(p + "ln_1.weight"))
        ow.ln2.append(f(p + "ln_2.weight"))
        ow.c_attn_p.append(f(p + "attn.c_attn.weight"))
        ow.c_proj_p.append(f(p + "attn.c_proj.weight"))
        ow.gu_p.append(np.concatenate([f(p + "mlp.w_gate.weight"), f(p + "mlp.w_up.weight")], 0))
        ow.wd_p.append(f(p + "mlp.w_down.weight"))
        for lst in (ow.c_attn_s, ow.c_proj_s, ow.gu_s, ow.wd_s):
            lst.append(None)
        if p + "attn.c_attn.bias" in w:
            ow.c_attn_b.append(f(p + "attn.c_attn.bias"))
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size, c.rope_theta)
    return cfg, om.OracleModel(cfg, ow, cos, sin)


def tiny_hf_checkpoint(tmp_path, family, tie, hidden=128, inter=256):
    """A random-init tiny HuggingFace model saved as safetensors; returns (dir, hf model)."""
    torch.manual_seed(3)
    kw = dict(hidden_size=hidden, intermediate_size=inter, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=2, vocab_size=256, rms_norm_eps=1e-5, max_position_embeddings=128,
              tie_word_embeddings=tie, initializer_range=0.05)
    if family == "llama":
        cfg = transformers.LlamaConfig(rope_theta=10000.0, **kw)
        m = transformers.LlamaForCausalLM(cfg)
    else:
        cfg = transformers.Qwen2Config(rope_theta=10000.0, **kw)
        m = transformers.Qwen2ForCausalLM(cfg)
        with torch.no_grad():  # non-zero q/k/v biases so that the bias permutation matters
            for layer in m.model.layers:
                for proj in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj):
                    proj.bias.normal_(0.0, 0.2)
    m = m.eval()
    m.save_pretrained(str(tmp_path), safe_serialization=True)
    return tmp_path, m


@pytest.mark.parametrize("family,tie", [("llama", False), ("llama", True), ("qwen2", False)])
def test_imported_model_reproduces_huggingface_logits(tmp_path, family, tie):
    path, hf = tiny_hf_checkpoint(tmp_path, family, tie)
    model = load_hf_safetensors(path, device="cpu")
    assert model.config.qkv_bias == (family == "qwen2") and model.config.tie_word_embeddings == tie
    cfg, oracle = _oracle_from(model)
    ids = [5, 77, 200, 3, 141, 9, 64, 250]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0].float().numpy()
    got = oracle.forward(ids, None, return_all_logits=True).astype(np.float32)
    err = np.abs(got - want).max()
    assert err <= 2e-2 * max(1.0, float(np.abs(want).max())), err
    assert (got.argmax(-1) == want.argmax(-1)).mean() >= 0.75


def test_planted_permutation_mistake_is_caught(tmp_path, monkeypatch):
    """Without the row reorder the imported model's logits miss HuggingFace's by far more
    than the bound above (measured about 10x)."""
    import axiomlm_amd.hf_import as hi

    path, hf = tiny_hf_checkpoint(tmp_path, "llama", False)
    monkeypatch.setattr(hi, "permute_hf_rope_weight", lambda w, n, hd: w.contiguous())
    _, oracle = _oracle_from(hi.load_hf_safetensors(path, device="cpu"))
    ids = [5, 77, 200, 3, 141, 9, 64, 250]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0].float().numpy()
    got = oracle.forward(ids, None, return_all_logits=True).astype(np.float32)
    assert np.abs(got - want).max() > 5 * 2e-2 * max(1.0, float(np.abs(want).max()))


def test_config_translation_and_sharded_reader(tmp_path):
    hf_cfg = {"num_attention_heads": 32, "num_key_value_heads": 8, "hidden_size": 4096, "num_hidden_layers": 32,
              "vocab_size": 128256, "intermediate_size": 14336, "rms_norm_eps": 1e-5, "rope_theta": 500000.0,
              "max_position_embeddings": 131072, "tie_word_embeddings": False,
              "rope_scaling": {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                               "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}}
    c = build_model_config_from_hf(hf_cfg)
    assert (c.n_head, c.kv_heads, c.head_dim, c.hidden, c.block_size) == (32, 8, 128, 14336, 4096)
    assert c.rope_theta == 500000.0 and c.rope_scaling["rope_type"] == "llama3" and not c.qkv_bias
    # a two-shard checkpoint with an index file
    path, hf = tiny_hf_checkpoint(tmp_path, "llama", False)
    from safetensors.torch import load_file, save_file
    import json

    full = load_file(str(path / "model.safetensors"))
    keys = sorted(full)
    shards = {"model-00001-of-00002.safetensors": keys[: len(keys) // 2],
              "model-00002-of-00002.safetensors": keys[len(keys) // 2:]}
    for name, ks in shards.items():
        save_file({k: full[k] for k in ks}, str(path / name))
    (path / "model.safetensors").unlink()
    with open(path / "model.safetensors.index.json", "w") as f:
        json.dump({"weight_map": {k: n for n, ks in shards.items() for k in ks}}, f)
    model = load_hf_safetensors(path, device="cpu")
    assert torch.equal(model.w["transformer.h.1.mlp.w_down.weight"],
                       full["model.layers.1.mlp.down_proj.weight"].to(torch.float16))


def test_missing_checkpoint_is_a_clear_error(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_hf_safetensors(tmp_path / "nope-not-a-repo-xyz", device="cpu")
