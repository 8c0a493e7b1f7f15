"""Write the C1 golden vectors from the reference's own Python CPU path.

Run in the development container only (the reference tree is not present on
the GPU box); the output ``c1_q4.npz`` is committed and the tests read it.

What is recorded, for the BASELINE configs[0] model (4 layers, d 256, 4 heads x
64, SwiGLU 704, vocab 1024, eps 1e-5, RoPE theta 1e4) with the weights of
``oracle.model.make_float_weights(cfg, seed=0)`` loaded into the reference
``Transformer``:

* the SHA-256 of every packed matrix of ``Transformer._ensure_quant_weights``
  in mode "q4" (MSE clip search with the reference importance vectors,
  axiomlm/models/transformer.py:822-1008, axiomlm/kernels/quant.py:447-594),
  Q8_G64 embedding, untied Q4 lm_head (the packs themselves are re-made by
  the packer under test and compared through the hash);
* the logits of ``_forward_quantized_sequence`` (transformer.py:1036-1200)
  decoding a 32-token prompt one token at a time into a reference
  ``StaticKVCache(1, 128, 4, 4, 64)`` (engine/paged_cache.py:122-361), then 64
  greedy steps (argmax, lowest index on ties);
* the logits of the same 32-token prompt run as one sequence (prefill).

Hidden size: BASELINE's 688 is not a multiple of the packer's group 64
(quant.py:467 asserts K % 64 == 0 for w_down), so C1 uses 704.

The reference package's ``__init__`` imports the tokenizer stack (tiktoken is
not installed); the modules used here are loaded through empty package
objects whose ``__path__`` points into the reference tree, so only the
reference files named above (and what they import) execute.
"""

from __future__ import annotations

import hashlib
import os
import sys
import types

import numpy as np
import torch

REF = os.environ.get("AXIOMLM_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import model as om  # noqa: E402


def _ref_packages():
    for name, sub in (("axiomlm", "axiomlm"), ("axiomlm.engine", "axiomlm/engine")):
        m = types.ModuleType(name)
        m.__path__ = [os.path.join(REF, sub)]
        sys.modules[name] = m
    from axiomlm.engine.paged_cache import StaticKVCache
    from axiomlm.models.transformer import ModelConfig, Transformer

    return ModelConfig, Transformer, StaticKVCache


def pack_digest(a: np.ndarray) -> str:
    """SHA-256 over the little-endian bytes of a packed array (codes as stored, fp16 as bits)."""
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_config():
    return om.OracleConfig(n_layer=4, n_head=4, n_kv_head=4, d_model=256, hidden=704, vocab=1024, eps=1e-5,
                           block_size=256)


def build_reference_model(Transformer, ModelConfig, cfg, W):
    mc = ModelConfig(block_size=cfg.block_size, vocab_size=cfg.vocab, n_layer=cfg.n_layer, n_head=cfg.n_head,
                     n_embd=cfg.d_model, n_kv_head=cfg.n_kv_head, norm_type="rmsnorm", pos_emb="rope",
                     mlp_type="swiglu", bias=False, rope_theta=cfg.rope_theta, intermediate_size=cfg.hidden,
                     rms_norm_eps=cfg.eps, tie_word_embeddings=False)
    model = Transformer(mc)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).float()  # noqa: E731
    with torch.no_grad():
        model.transformer.wte.weight.copy_(t(W["wte"]))
        model.lm_head.weight.copy_(t(W["lm_head"]))
        model.transformer.ln_f.weight.copy_(t(W["lnf"]))
        for blk, L in zip(model.transformer.h, W["layers"]):
            blk.ln_1.weight.copy_(t(L["ln1"]))
            blk.ln_2.weight.copy_(t(L["ln2"]))
            blk.attn.c_attn.weight.copy_(t(L["c_attn"]))
            blk.attn.c_proj.weight.copy_(t(L["c_proj"]))
            blk.mlp.w_gate.weight.copy_(t(L["w_gate"]))
            blk.mlp.w_up.weight.copy_(t(L["w_up"]))
            blk.mlp.w_down.weight.copy_(t(L["w_down"]))
    model = model.half().eval()
    model.quantize("q4")
    return model


def main(out_path=os.path.join(HERE, "c1_q4.npz")):
    ModelConfig, Transformer, StaticKVCache = _ref_packages()
    cfg = c1_config()
    W = om.make_float_weights(cfg, seed=0)
    model = build_reference_model(Transformer, ModelConfig, cfg, W)
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, cfg.vocab, 32).tolist()
    out = {"prompt": np.array(prompt, np.int64)}
    with torch.no_grad():
        qw = model._ensure_quant_weights(torch.device("cpu"))
        names, digests = [], []
        for key in ("wte_p", "wte_sb", "lmh_p", "lmh_sb"):
            names.append(key)
            digests.append(pack_digest(qw[key].numpy()))
        for key in ("c_attn_p", "c_attn_s", "c_proj_p", "c_proj_s", "gu_p", "gu_s", "wd_p", "wd_s"):
            for i, tsr in enumerate(qw[key]):
                names.append(f"{key}{i}")
                digests.append(pack_digest(tsr.numpy()))
        out["pack_names"] = np.array(names)
        out["pack_sha256"] = np.array(digests)
        # Token-by-token decode through the reference cache, then greedy.
        cache = StaticKVCache(1, 128, cfg.n_layer, cfg.n_kv_head, cfg.head_dim, dtype=torch.float16,
                              device=torch.device("cpu"))
        logits = []
        for tok in prompt:
            lg, _, _ = model(torch.tensor([[tok]]), kv_caches=cache)
            logits.append(lg[0, -1].numpy().copy())
        tokens = []
        tok = int(torch.argmax(torch.from_numpy(logits[-1]).float()))
        for _ in range(64):
            tokens.append(tok)
            lg, _, _ = model(torch.tensor([[tok]]), kv_caches=cache)
            logits.append(lg[0, -1].numpy().copy())
            tok = int(torch.argmax(lg[0, -1].float()))
        out["decode_logits"] = np.stack(logits).astype(np.float16)
        out["greedy_tokens"] = np.array(tokens, np.int64)
        # One-sequence prefill of the prompt (no cache).
        lg = model(torch.tensor([prompt]), return_all_logits=True)[0]
        out["prefill_logits"] = lg[0].numpy().astype(np.float16)
    np.savez_compressed(out_path, **out)
    print(f"wrote {out_path}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in out.items()))


if __name__ == "__main__":
    main(*sys.argv[1:])
