"""HuggingFace safetensors checkpoints (Llama / Llama-3 / SmolLM2 / Qwen2 layouts) into the
decode driver: the interface of axiomlm/utils/hf_importer.py (``permute_hf_rope_weight``,
``unpermute_hf_rope_weight``, ``permute_hf_rope_bias``, ``build_model_config_from_hf``,
``load_hf_safetensors``).

HuggingFace's Llama attention rotates the pairs (i, i + hd/2) of every head ("rotate half"),
the AxiomLM RoPE the interleaved pairs (2i, 2i + 1) (modules.py:95-121).  Reordering the q
and k projection rows of each head as 0, hd/2, 1, hd/2 + 1, ... makes the interleaved
rotation of the reordered rows equal the reordered half-split rotation, and q . k is
unchanged, so the imported model computes the same attention (hf_importer.py:23-63).
Tensors are read one at a time from the (possibly sharded) safetensors files and moved to
the device as they are read, so a checkpoint is never held twice in host memory.

Only local directories (or a snapshot already in the HuggingFace cache) are read: this
build does not download.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any

import torch

from .transformer import ModelConfig, Transformer


def _pair_order(head_dim: int) -> torch.Tensor:
    """Row order within one head: half-split index of interleaved row r."""
    half = head_dim // 2
    r = torch.arange(head_dim)
    return (r // 2) + (r % 2) * half


def permute_hf_rope_weight(w: torch.Tensor, n_heads: int, head_dim: int) -> torch.Tensor:
    """Half-split RoPE rows [0..hd/2 | hd/2..hd] of each head -> interleaved pairs
    [0, hd/2, 1, hd/2+1, ...] (hf_importer.py:23-35); w is [n_heads * head_dim, K]."""
    idx = (torch.arange(n_heads)[:, None] * head_dim + _pair_order(head_dim)[None, :]).reshape(-1)
    return w.index_select(0, idx.to(w.device)).contiguous()


def unpermute_hf_rope_weight(w: torch.Tensor, n_heads: int, head_dim: int) -> torch.Tensor:
    """Inverse of :func:`permute_hf_rope_weight` (hf_importer.py:38-50)."""
    inv = torch.argsort(_pair_order(head_dim))
    idx = (torch.arange(n_heads)[:, None] * head_dim + inv[None, :]).reshape(-1)
    return w.index_select(0, idx.to(w.device)).contiguous()


def permute_hf_rope_bias(b: torch.Tensor, n_heads: int, head_dim: int) -> torch.Tensor:
    """The same row reorder for a q / k bias vector (Qwen2; hf_importer.py:53-63)."""
    return permute_hf_rope_weight(b.reshape(-1, 1), n_heads, head_dim).reshape(-1)


def resolve_hf_model_dir(repo_id_or_path: str | Path, token: str | None = None) -> Path:
    """A local checkpoint directory, or the cached snapshot of a hub repository id
    (hf_importer.py:66-93 without the download)."""
    candidate = Path(repo_id_or_path).expanduser()
    if candidate.is_dir():
        return candidate
    try:
        from huggingface_hub import snapshot_download

        return Path(snapshot_download(repo_id=str(repo_id_or_path), token=token, local_files_only=True,
                                      allow_patterns=["*.json", "*.safetensors", "*.txt", "*.model"]))
    except Exception as exc:  # not cached, or huggingface_hub missing
        raise FileNotFoundError(f"{repo_id_or_path!r} is neither a local directory nor a cached HuggingFace "
                                f"snapshot (this build does not download checkpoints)") from exc


def build_model_config_from_hf(hf_cfg: dict[str, Any], has_qkv_bias: bool = False,
                               max_seq_len: int | None = None) -> ModelConfig:
    """LlamaConfig / Qwen2Config ``config.json`` -> ModelConfig (hf_importer.py:96-153)."""
    n_head = int(hf_cfg["num_attention_heads"])
    rope_params = hf_cfg.get("rope_parameters") or {}
    rope_theta = float(hf_cfg.get("rope_theta", rope_params.get("rope_theta", 10000.0)))
    rope_scaling = hf_cfg.get("rope_scaling")
    if rope_scaling is None and isinstance(rope_params, dict) and rope_params.get("rope_type") not in (None, "default"):
        rope_scaling = rope_params
    block = max_seq_len if max_seq_len is not None else min(int(hf_cfg.get("max_position_embeddings", 4096)), 4096)
    return ModelConfig(
        block_size=block, vocab_size=int(hf_cfg["vocab_size"]), n_layer=int(hf_cfg["num_hidden_layers"]),
        n_head=n_head, n_embd=int(hf_cfg["hidden_size"]), n_kv_head=int(hf_cfg.get("num_key_value_heads", n_head)),
        rope_theta=rope_theta, intermediate_size=int(hf_cfg["intermediate_size"]),
        rms_norm_eps=float(hf_cfg.get("rms_norm_eps", 1e-6)),
        tie_word_embeddings=bool(hf_cfg.get("tie_word_embeddings", True)),
        qkv_bias=bool(has_qkv_bias or hf_cfg.get("attention_bias", False) or hf_cfg.get("qkv_bias", False)),
        rope_scaling=rope_scaling)


class SafetensorsReader:
    """Lazy tensor access over ``model.safetensors``, a sharded checkpoint with
    ``model.safetensors.index.json``, or any ``*.safetensors`` files of a directory."""

    def __init__(self, model_dir: Path):
        from safetensors import safe_open

        self._open = lambda p: safe_open(str(p), framework="pt", device="cpu")
        self.model_dir = Path(model_dir)
        self._handles: dict[str, Any] = {}
        self.weight_map: dict[str, str] = {}
        index = self.model_dir / "model.safetensors.index.json"
        if index.exists():
            with open(index, encoding="utf-8") as f:
                self.weight_map = dict(json.load(f)["weight_map"])
            return
        files = [self.model_dir / "model.safetensors"]
        if not files[0].exists():
            files = sorted(self.model_dir.glob("*.safetensors"))
        if not files:
            raise FileNotFoundError(f"no .safetensors files in {self.model_dir}")
        for f in files:
            h = self._handles[f.name] = self._open(f)
            for k in h.keys():
                self.weight_map[k] = f.name

    def __contains__(self, key: str) -> bool:
        return key in self.weight_map

    def get(self, key: str, dtype: torch.dtype, device) -> torch.Tensor:
        shard = self.weight_map[key]
        if shard not in self._handles:
            self._handles[shard] = self._open(self.model_dir / shard)
        return self._handles[shard].get_tensor(key).to(device=device, dtype=dtype)


def load_hf_safetensors(repo_id_or_path: str | Path, device: str | torch.device = "cuda",
                        dtype: torch.dtype = torch.float16, max_seq_len: int | None = None,
                        token: str | None = None) -> Transformer:
    """A HuggingFace LlamaForCausalLM / Qwen2ForCausalLM checkpoint as a decode-driver
    Transformer (hf_importer.py:199-305): q / k rows (and biases) reordered for the
    interleaved RoPE, [q; k; v] fused into c_attn, gate / up / down and the norms under the
    reference's state-dict names, the lm_head tied unless the checkpoint has its own."""
    model_dir = resolve_hf_model_dir(repo_id_or_path, token=token)
    with open(model_dir / "config.json", encoding="utf-8") as f:
        hf_cfg = json.load(f)
    rd = SafetensorsReader(model_dir)
    if "lm_head.weight" in rd and not bool(hf_cfg.get("tie_word_embeddings", True)):
        hf_cfg["tie_word_embeddings"] = False
    cfg = build_model_config_from_hf(hf_cfg, "model.layers.0.self_attn.q_proj.bias" in rd, max_seq_len)
    dev = torch.device(device)
    hd, nq, nkv = cfg.head_dim, cfg.n_head, cfg.kv_heads

    def get(key):
        return rd.get(key, dtype, dev)

    sd = {"transformer.wte.weight": get("model.embed_tokens.weight"), "transformer.ln_f.weight": get("model.norm.weight")}
    if not cfg.tie_word_embeddings and "lm_head.weight" in rd:
        sd["lm_head.weight"] = get("lm_head.weight")
    for i in range(cfg.n_layer):
        src, dst = f"model.layers.{i}.", f"transformer.h.{i}."
        sd[dst + "ln_1.weight"] = get(src + "input_layernorm.weight")
        sd[dst + "ln_2.weight"] = get(src + "post_attention_layernorm.weight")
        a = src + "self_attn."
        sd[dst + "attn.c_attn.weight"] = torch.cat([
            permute_hf_rope_weight(get(a + "q_proj.weight"), nq, hd),
            permute_hf_rope_weight(get(a + "k_proj.weight"), nkv, hd),
            get(a + "v_proj.weight")], dim=0)
        if a + "q_proj.bias" in rd:
            sd[dst + "attn.c_attn.bias"] = torch.cat([
                permute_hf_rope_bias(get(a + "q_proj.bias"), nq, hd),
                permute_hf_rope_bias(get(a + "k_proj.bias"), nkv, hd),
                get(a + "v_proj.bias")], dim=0)
        sd[dst + "attn.c_proj.weight"] = get(a + "o_proj.weight")
        sd[dst + "mlp.w_gate.weight"] = get(src + "mlp.gate_proj.weight")
        sd[dst + "mlp.w_up.weight"] = get(src + "mlp.up_proj.weight")
        sd[dst + "mlp.w_down.weight"] = get(src + "mlp.down_proj.weight")
    return Transformer(cfg, sd, device=dev)
