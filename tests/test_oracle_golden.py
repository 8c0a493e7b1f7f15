"""The oracle against vectors the reference's own CPU path wrote (tests/golden/c1_q4.npz):
the MSE clip-search packer bit for bit, the decode step to fp16 op-order noise."""

import numpy as np

from c1_golden import c1_config, golden, named_packs, oracle_packs, pack_digest
from oracle import model as om

F32 = np.float32


def test_q4_mse_packs_match_reference_bit_for_bit():
    """Every matrix of _ensure_quant_weights(mode "q4") (transformer.py:822-1008,
    quant.py:447-594): codes, scales and biases identical to the reference's."""
    g = golden()
    mine = named_packs(oracle_packs())
    want = dict(zip(g["pack_names"].tolist(), g["pack_sha256"].tolist()))
    assert sorted(mine) == sorted(want)
    bad = [k for k in want if pack_digest(mine[k]) != want[k]]
    assert not bad, f"packs differ from the reference: {bad}"


def _oracle_model():
    cfg = c1_config()
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size, cfg.rope_theta)
    return cfg, om.OracleModel(cfg, oracle_packs(), cos, sin)


def test_decode_and_greedy_match_reference():
    """32 prompt tokens fed one at a time into a 128-slot fp16 cache, then 64 greedy
    steps (transformer.py:1437-1473 CPU branch).  Measured max |diff| 1.95e-3 (the
    reference rounds torch-CPU fp16 matmul / SDPA internally in its own order)."""
    g = golden()
    cfg, m = _oracle_model()
    cache = om.OracleKVCache(128, cfg.n_layer, cfg.n_kv_head, cfg.head_dim)
    outs = [m.forward([t], cache)[-1] for t in g["prompt"].tolist()]
    toks = []
    tok = int(np.argmax(outs[-1].astype(F32)))
    for _ in range(64):
        toks.append(tok)
        outs.append(m.forward([tok], cache)[-1])
        tok = int(np.argmax(outs[-1].astype(F32)))
    d = np.abs(np.stack(outs).astype(F32) - g["decode_logits"].astype(F32))
    assert d.max() <= 4e-3, f"max |logit diff| {d.max()}"
    assert toks == g["greedy_tokens"].tolist()


def test_prefill_matches_reference():
    """The 32-token prompt as one causal sequence (no cache)."""
    g = golden()
    cfg, m = _oracle_model()
    lg = m.forward(g["prompt"].tolist(), om.OracleKVCache(128, cfg.n_layer, cfg.n_kv_head, cfg.head_dim),
                   return_all_logits=True)
    d = np.abs(lg.astype(F32) - g["prefill_logits"].astype(F32))
    assert d.max() <= 4e-3, f"max |logit diff| {d.max()}"
