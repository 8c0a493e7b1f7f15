"""Quantized decode driver: the part of ``Transformer`` that feeds the decode runner.

Mirrors, for a Llama-style decoder (RMSNorm, RoPE, SwiGLU, no linear bias except an
optional QKV bias), the reference's

* ``ModelConfig`` fields the quantized decode step reads
  (axiomlm/models/transformer.py:44-99);
* ``precompute_rope_frequencies`` -> ``freqs_real`` (modules.py:46-92, transformer.py:234-248);
* ``quantize`` / ``_ensure_quant_weights`` packing choices (transformer.py:276-320, 822-1008):
  MARLIN Q4 layers (MSE clip search with the reference importance vectors in mode "q4",
  round-to-nearest in "q4_rtn"), gate|up packed as one matrix, Q8_G64 embedding table,
  lm_head Q8_G64 when tied (or ``lm_head_q8``) else MARLIN Q4;
* ``get_decode_runner`` (transformer.py:1202-1308) and the ``forward`` fast path
  (transformer.py:1437-1473): positions, runner ``step`` / ``verify_step`` and the cache
  counters; ``forward_tree_verify`` through ``verify_tree_step``.

Weights are plain tensors named as in the reference ``state_dict`` (``transformer.wte.weight``,
``transformer.h.{i}.attn.c_attn.weight``, ...), so a reference checkpoint's tensors load
unchanged.  Every kernel runs on the GPU; there is no CPU fallback: sequences longer than
the runner's multi-token capacity are fed as consecutive ``verify_step`` chunks.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch

from .cache import StaticKVCache
from .kernels import pack_linear_q4_marlin, pack_linear_q8_g64
from .runner import DecodeRunner, QuantizedDecodeRunner


@dataclass
class ModelConfig:
    block_size: int = 1024
    vocab_size: int = 50304
    n_layer: int = 12
    n_head: int = 12
    n_embd: int = 768
    n_kv_head: int | None = None
    rope_theta: float = 10000.0
    intermediate_size: int | None = None
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = True
    qkv_bias: bool = False
    rope_scaling: dict[str, Any] | None = None

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    @property
    def kv_heads(self) -> int:
        return self.n_kv_head if self.n_kv_head is not None else self.n_head

    @property
    def hidden(self) -> int:
        """SwiGLU width: ``intermediate_size`` or 8/3 d rounded up to 64 (modules.py:147-152)."""
        if self.intermediate_size:
            return self.intermediate_size
        return 64 * ((int(2 * (4 * self.n_embd) / 3) + 63) // 64)


def precompute_rope_frequencies(head_dim: int, max_seq_len: int = 2048, theta: float = 10000.0,
                                rope_scaling: dict[str, Any] | None = None) -> torch.Tensor:
    """(max_seq_len, head_dim/2, 2) fp32 (cos, sin), the ``freqs_real`` buffer (modules.py:46-92)."""
    if head_dim % 2:
        raise ValueError(f"head_dim ({head_dim}) must be even for RoPE")
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    if rope_scaling is not None:
        rope_type = rope_scaling.get("rope_type", rope_scaling.get("type", "default"))
        if rope_type == "llama3":
            factor = float(rope_scaling["factor"])
            lo = float(rope_scaling.get("low_freq_factor", 1.0))
            hi = float(rope_scaling.get("high_freq_factor", 4.0))
            old = float(rope_scaling.get("original_max_position_embeddings", 8192))
            wavelen = 2.0 * math.pi / inv_freq
            inv_l = torch.where(wavelen > old / lo, inv_freq / factor, inv_freq)
            smooth = (old / wavelen - lo) / (hi - lo)
            smoothed = (1.0 - smooth) * inv_l / factor + smooth * inv_l
            medium = ~(wavelen < old / hi) & ~(wavelen > old / lo)
            inv_freq = torch.where(medium, smoothed, inv_l)
        elif rope_type == "linear" and "factor" in rope_scaling:
            inv_freq = inv_freq / float(rope_scaling["factor"])
    t = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.view_as_real(torch.polar(torch.ones_like(freqs), freqs)).contiguous()


class Transformer:
    """Decode-side view of an AxiomLM ``Transformer`` over a reference-named state dict."""

    def __init__(self, config: ModelConfig, state_dict: dict[str, torch.Tensor], device=None):
        self.config = config
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.w = {k: v.detach() for k, v in state_dict.items()}
        if config.tie_word_embeddings and "lm_head.weight" not in self.w:
            self.w["lm_head.weight"] = self.w["transformer.wte.weight"]
        self.freqs_real = precompute_rope_frequencies(config.head_dim, config.block_size, config.rope_theta,
                                                      config.rope_scaling)
        self._quant_mode: str | None = None
        self._lm_head_q8: bool | None = None
        self._quant_weights_cache: dict[str, Any] | None = None
        self._runner: QuantizedDecodeRunner | None = None
        self._runner_key = None

    # -- transformer.py:276-320 ---------------------------------------------
    def quantize(self, mode: str | None = "q4", lm_head_q8: bool | None = None,
                 release_fp16: bool = False) -> "Transformer":
        """Modes of the quantized decode runner (transformer.py:282-289): "q4" (MARLIN Q4 with the
        importance-weighted MSE clip search), "q4_rtn" (round to nearest), "q4_k_m" ("q4" with
        Q8_G64 w_down and lm_head), "q8" (Q8_G64 everywhere); None runs the fp16 weights on the
        fp16 runner.  The reference's "q4_legacy", "q2_k" and "ternary" modes do not run through
        its decode runner and are not modes here.

        release_fp16 (transformer.py:321-351): pack now, then drop the fp16 copies of every
        packed matrix (layer projections, lm_head, embedding table), keeping only the packs and
        the norms; the model cannot be unquantized or repacked in another mode afterwards."""
        if mode not in (None, "q4", "q4_rtn", "q4_k_m", "q8"):
            raise ValueError(f"quant mode {mode!r} is not on the MI355X decode path (q4, q4_rtn, q4_k_m, q8)")
        if getattr(self, "_fp16_released", False) and (mode, lm_head_q8) != (self._quant_mode, self._lm_head_q8):
            raise RuntimeError("the fp16 weights were released by quantize(..., release_fp16=True); the model cannot "
                               "be unquantized or packed in another mode")
        if not getattr(self, "_fp16_released", False):
            self._quant_weights_cache = None
            self._runner = None
        self._quant_mode = mode
        self._lm_head_q8 = lm_head_q8
        if release_fp16 and mode is not None:
            self._ensure_quant_weights()
            names = ["lm_head.weight", "transformer.wte.weight"]
            for i in range(self.config.n_layer):
                pre = f"transformer.h.{i}."
                names += [pre + n for n in ("attn.c_attn.weight", "attn.c_proj.weight", "mlp.w_gate.weight",
                                            "mlp.w_up.weight", "mlp.w_down.weight")]
            for n in names:
                if n in self.w:
                    self.w[n] = torch.empty(0, dtype=torch.float16, device=self.w[n].device)
            self._fp16_released = True
            if self.device.type == "cuda":
                torch.cuda.empty_cache()
        return self

    def _t(self, name: str) -> torch.Tensor:
        return self.w[name].to(self.device)

    # -- transformer.py:822-1008 ----------------------------------------------
    def _ensure_quant_weights(self) -> dict[str, Any]:
        key = (self._quant_mode, self._lm_head_q8, str(self.device))
        if self._quant_weights_cache is not None and self._quant_weights_cache["key"] == key:
            return self._quant_weights_cache
        if self._quant_mode is None:
            raise RuntimeError("call quantize() first")
        c = self.config
        mode = self._quant_mode
        mse = mode in ("q4", "q4_k_m")
        # transformer.py:840-847: Q8 lm_head for q4_k_m / q8 or tied embeddings unless overridden
        use_q8_lm = (bool(self._lm_head_q8) if self._lm_head_q8 is not None
                     else (mode in ("q4_k_m", "q8") or bool(c.tie_word_embeddings)))
        use_q8_down = mode in ("q4_k_m", "q8")

        def pack(w, imp=None, q8=False):
            w = w.to(self.device)
            if q8 or mode == "q8":
                return pack_linear_q8_g64(w)
            if not mse:
                return pack_linear_q4_marlin(w, clip_search=False)
            return pack_linear_q4_marlin(w, clip_search=True, col_importance=imp)

        absf = lambda t: t.to(self.device).float().abs()  # noqa: E731
        lmh_p, lmh_sb = pack(self.w["lm_head.weight"], absf(self.w["transformer.ln_f.weight"]) if mse else None,
                             use_q8_lm)
        if c.tie_word_embeddings and use_q8_lm:
            wte_p, wte_sb = lmh_p, lmh_sb
        else:
            wte_p, wte_sb = pack(self.w["transformer.wte.weight"], q8=True)
        q = {"key": key, "hidden_dim": c.hidden, "wte_p": wte_p, "wte_sb": wte_sb, "lmh_p": lmh_p, "lmh_sb": lmh_sb}
        for name in ("c_attn_p", "c_attn_s", "c_attn_b", "c_proj_p", "c_proj_s", "gu_p", "gu_s", "wd_p", "wd_s"):
            q[name] = []
        for i in range(c.n_layer):
            pre = f"transformer.h.{i}."
            ln1 = absf(self.w[pre + "ln_1.weight"]) if mse else None
            ln2 = absf(self.w[pre + "ln_2.weight"]) if mse else None
            p, s = pack(self.w[pre + "attn.c_attn.weight"], ln1)
            q["c_attn_p"].append(p)
            q["c_attn_s"].append(s)
            b = self.w.get(pre + "attn.c_attn.bias")
            q["c_attn_b"].append(b.to(self.device, torch.float16) if b is not None else None)
            p, s = pack(self.w[pre + "attn.c_proj.weight"])
            q["c_proj_p"].append(p)
            q["c_proj_s"].append(s)
            wg, wu = self._t(pre + "mlp.w_gate.weight"), self._t(pre + "mlp.w_up.weight")
            p, s = pack(torch.cat([wg, wu], dim=0), ln2)
            q["gu_p"].append(p)
            q["gu_s"].append(s)
            imp_sw = (wg.float().norm(dim=1) * wu.float().norm(dim=1)) if (mse and not use_q8_down) else None
            p, s = pack(self.w[pre + "mlp.w_down.weight"], imp_sw, use_q8_down)
            q["wd_p"].append(p)
            q["wd_s"].append(s)
        self._quant_weights_cache = q
        return q

    # -- transformer.py:1202-1308 ---------------------------------------------
    def get_decode_runner(self, cache: StaticKVCache) -> QuantizedDecodeRunner:
        cache0 = cache[0] if isinstance(cache, list) else cache
        if cache0.max_batch_size != 1:
            raise RuntimeError("the decode runner drives a batch-1 StaticKVCache")
        key = (id(cache0), cache0.k_caches[0].data_ptr(), self._quant_mode, self._lm_head_q8)
        if self._runner is not None and self._runner_key == key:
            return self._runner
        if self._quant_mode is None:
            self._runner = self._fp16_runner(cache0)
            self._runner_key = key
            return self._runner
        qw = self._ensure_quant_weights()
        c = self.config
        h16 = lambda t: t.to(self.device, torch.float16).contiguous()  # noqa: E731
        ln1 = [h16(self.w[f"transformer.h.{i}.ln_1.weight"]) for i in range(c.n_layer)]
        ln2 = [h16(self.w[f"transformer.h.{i}.ln_2.weight"]) for i in range(c.n_layer)]
        lnf = h16(self.w["transformer.ln_f.weight"])
        biases = [b if b is not None else torch.empty(0, device=self.device) for b in qw["c_attn_b"]]
        self._runner = QuantizedDecodeRunner(
            None, qw["lmh_p"], qw["lmh_sb"], self.freqs_real.to(self.device), ln1, qw["c_attn_p"], qw["c_attn_s"],
            qw["c_proj_p"], qw["c_proj_s"], ln2, qw["gu_p"], qw["gu_s"], qw["wd_p"], qw["wd_s"], lnf,
            cache0.k_caches, cache0.v_caches, c.n_head, c.kv_heads, c.head_dim, self._quant_mode != "q8",
            c.rms_norm_eps, biases,
            c.vocab_size, wte_p=qw["wte_p"], wte_s=qw["wte_sb"], k_scales=cache0.k_scales, v_scales=cache0.v_scales,
            kv_dtype=cache0.cache_dtype, max_tokens=64)
        self._runner_key = key
        return self._runner

    def _fp16_runner(self, cache0: StaticKVCache) -> DecodeRunner:
        """The unquantized model on the fp16 runner (transformer.py:1310-1380, MPSDecodeRunner):
        fp16 weights as given, gate|up stacked [W_gate; W_up]."""
        c = self.config
        h16 = lambda name: self.w[name].to(self.device, torch.float16).contiguous()  # noqa: E731
        pre = [f"transformer.h.{i}." for i in range(c.n_layer)]
        bias = [self.w.get(p + "attn.c_attn.bias") for p in pre]
        return DecodeRunner(
            h16("transformer.wte.weight"), self.freqs_real.to(self.device), [h16(p + "ln_1.weight") for p in pre],
            [h16(p + "attn.c_attn.weight") for p in pre], [h16(p + "attn.c_proj.weight") for p in pre],
            [h16(p + "ln_2.weight") for p in pre],
            [torch.cat([h16(p + "mlp.w_gate.weight"), h16(p + "mlp.w_up.weight")], dim=0) for p in pre],
            [h16(p + "mlp.w_down.weight") for p in pre], h16("transformer.ln_f.weight"), cache0.k_caches,
            cache0.v_caches, c.n_head, c.kv_heads, c.head_dim, c.rms_norm_eps, lm_head_w=h16("lm_head.weight"),
            c_attn_bs=[b.to(self.device, torch.float16) if b is not None else torch.empty(0, device=self.device)
                       for b in bias],
            k_scales=cache0.k_scales, v_scales=cache0.v_scales, kv_dtype=cache0.cache_dtype, max_tokens=64)

    def _positions(self, cache0: StaticKVCache, T: int):
        seen = cache0.total_seen_tokens[0]
        S = cache0.max_seq_len
        write_pos = (seen % S) if (cache0.ring_buffer or seen >= S) else seen
        return seen, write_pos, min(seen + T, S), seen % self.freqs_real.shape[0]

    # -- transformer.py:1437-1473 ---------------------------------------------
    @torch.no_grad()
    def forward(self, idx: torch.Tensor, targets=None, kv_caches=None, return_all_logits: bool = False):
        """Decode / verify tokens ``idx`` (1, T) into the cache; returns ``(logits, None, kv_caches)``
        with logits (1, 1, V), or (1, T, V) with ``return_all_logits``, as the reference does."""
        if targets is not None:
            raise RuntimeError("training forward (targets) is not on the quantized decode path")
        if kv_caches is None:
            raise RuntimeError("the quantized decode path needs a StaticKVCache")
        if not isinstance(kv_caches, (list, tuple)):
            kv_caches = [kv_caches] * self.config.n_layer
        cache0 = kv_caches[0]
        if idx.dim() != 2 or idx.shape[0] != 1:
            raise RuntimeError("forward expects idx of shape (1, T)")
        runner = self.get_decode_runner(cache0)
        T = idx.shape[1]
        chunk = 32
        outs = []
        for t0 in range(0, T, chunk):
            part = idx[:, t0:t0 + chunk]
            Tc = part.shape[1]
            seen, write_pos, active, rope_pos = self._positions(cache0, Tc)
            if Tc == 1:
                logits = runner.step(part.to(self.device), rope_pos, write_pos, active)
            else:
                logits = runner.verify_step(part, rope_pos, write_pos, active)
            outs.append(logits.clone() if (return_all_logits and T > chunk) else logits)
            cache0.total_seen_tokens[:] = [seen + Tc] * cache0.n_layer
            cache0.layer_seq_lens[:] = [active] * cache0.n_layer
        logits = torch.cat(outs, dim=1) if len(outs) > 1 else outs[0]
        return (logits if return_all_logits else logits[:, -1:, :]), None, kv_caches

    @torch.no_grad()
    def forward_tree_verify(self, idx: torch.Tensor, kv_caches, tree_depths, tree_mask, return_medusa: bool = True):
        """Tree verification over the draft tree ``idx`` (1, T) (transformer.py:580-636): node u is
        rotated at seen + depth[u] and attends to the cached prefix plus the nodes set in
        ``tree_mask[u]``; its K/V rows land at slot write_pos + u.  Returns
        ``(logits (1, T, V), [], kv_caches)`` (no Medusa heads on this path).  Counters are left to
        the caller, which commits the accepted path with ``compact_tree_path``."""
        if not isinstance(kv_caches, (list, tuple)):
            kv_caches = [kv_caches] * self.config.n_layer
        cache0 = kv_caches[0]
        B, T = idx.shape
        if B != 1 or not 1 <= T <= 64:
            raise RuntimeError(f"Expected B=1 and T in [1, 64], got {(B, T)}")
        if len(tree_depths) != T or len(tree_mask) != T:
            raise RuntimeError("tree_depths and tree_mask need one entry per node")
        seen, write_pos, _, rope_pos = self._positions(cache0, T)
        if not (write_pos + T <= cache0.max_seq_len and seen == write_pos):
            raise RuntimeError(f"Tree verification requires contiguous tail capacity: write_pos={write_pos}, "
                               f"T={T}, max_seq={cache0.max_seq_len}")
        runner = self.get_decode_runner(cache0)
        logits = runner.verify_tree_step(idx, rope_pos, write_pos, seen, [int(d) for d in tree_depths],
                                         [int(m) for m in tree_mask])
        self._last_verify_norm = runner.get_last_norm(T)
        return logits, [], kv_caches

    @torch.no_grad()
    def generate(self, prompt: list[int], max_new_tokens: int, cache: StaticKVCache) -> list[int]:
        """Greedy decoding: prompt through ``forward`` then one token per step."""
        logits = self.forward(torch.tensor([prompt], device=self.device), kv_caches=cache)[0]
        out = []
        tok = int(torch.argmax(logits[0, -1].float()))
        for _ in range(max_new_tokens):
            out.append(tok)
            logits = self.forward(torch.tensor([[tok]], device=self.device), kv_caches=cache)[0]
            tok = int(torch.argmax(logits[0, -1].float()))
        return out
