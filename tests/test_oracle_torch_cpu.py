"""The torch-CPU restatement of the reference CPU path (oracle/torch_cpu.py), which
bench.py times as its CPU baseline: its MARLIN / Q8 dequantization bit for bit
against the numpy oracle, and the C1 decode and prefill against the golden logits
written from the reference (same bar as the numpy oracle's)."""

import numpy as np
import torch

from c1_golden import c1_config, golden, oracle_packs
from oracle import formats as fm
from oracle import model as om
from oracle import torch_cpu as tc

F32 = np.float32


def test_dequantize_matches_numpy_oracle_bit_for_bit():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((104, 320)) * 0.02).astype(np.float16)
    p, s = fm.pack_linear_q4_marlin(w, clip_search=False)
    a = tc.dequantize_q4_marlin(torch.from_numpy(p), torch.from_numpy(s), 320, 100).numpy()
    b = fm.dequantize_q4_marlin(p, s, 320, 100)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    q8, sb = fm.pack_linear_q8_g64(w)
    a = tc.dequantize_q8_g64(torch.from_numpy(q8.view("<i4").reshape(104, -1).copy()), torch.from_numpy(sb),
                             320).numpy()
    assert np.array_equal(a.view(np.uint16), fm.dequantize_q8_g64(q8, sb, 320).view(np.uint16))


def _c1_model():
    cfg = c1_config()
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size, cfg.rope_theta)
    return cfg, tc.TorchCpuModel(cfg, oracle_packs(), cos, sin)


def test_c1_decode_and_greedy_match_reference():
    g = golden()
    cfg, m = _c1_model()
    cache = m.new_cache(128)
    with torch.no_grad():
        outs = [m.forward([t], cache)[-1].float().numpy() for t in g["prompt"].tolist()]
        toks = []
        tok = int(np.argmax(outs[-1]))
        for _ in range(64):
            toks.append(tok)
            outs.append(m.forward([tok], cache)[-1].float().numpy())
            tok = int(np.argmax(outs[-1]))
    d = np.abs(np.stack(outs) - g["decode_logits"].astype(F32))
    assert d.max() <= 4e-3, f"max |logit diff| {d.max()}"
    assert toks == g["greedy_tokens"].tolist()


def test_c1_prefill_matches_reference():
    g = golden()
    cfg, m = _c1_model()
    with torch.no_grad():
        lg = m.forward(g["prompt"].tolist(), m.new_cache(128), all_logits=True).float().numpy()
    d = np.abs(lg - g["prefill_logits"].astype(F32))
    assert d.max() <= 4e-3, f"max |logit diff| {d.max()}"
