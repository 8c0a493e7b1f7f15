"""Shared loader for the C1 golden vectors written by tests/golden/make_golden_c1.py
from the reference's own CPU path (see that script for what was recorded)."""

from __future__ import annotations

import functools
import hashlib
import os

import numpy as np

from oracle import formats as fm
from oracle import model as om

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c1_q4.npz")


def c1_config():
    return om.OracleConfig(n_layer=4, n_head=4, n_kv_head=4, d_model=256, hidden=704, vocab=1024, eps=1e-5,
                           block_size=256)


@functools.lru_cache(maxsize=1)
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@functools.lru_cache(maxsize=1)
def oracle_packs():
    """Mode "q4" packs of the seed-0 C1 weights made by the oracle packer."""
    cfg = c1_config()
    return om.pack_model(cfg, om.make_float_weights(cfg, seed=0), "q4")


def pack_digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def named_packs(ow: om.OracleWeights) -> dict:
    """Packed arrays of an OracleWeights under the fixture's names and storage views
    (the reference keeps the Q8 table as int32 [V, d/4])."""
    out = {"wte_p": ow.wte_p.view(np.int32).reshape(ow.wte_p.shape[0], -1), "wte_sb": ow.wte_sb,
           "lmh_p": ow.lmh_p, "lmh_sb": ow.lmh_sb}
    for key, lst in (("c_attn_p", ow.c_attn_p), ("c_attn_s", ow.c_attn_s), ("c_proj_p", ow.c_proj_p),
                     ("c_proj_s", ow.c_proj_s), ("gu_p", ow.gu_p), ("gu_s", ow.gu_s), ("wd_p", ow.wd_p),
                     ("wd_s", ow.wd_s)):
        for i, a in enumerate(lst):
            out[f"{key}{i}"] = a
    return out


def marlin_near_tie_fraction(wm: np.ndarray, sb: np.ndarray, ref_p: np.ndarray, ref_s: np.ndarray, K: int,
                             what: str = "") -> float:
    """Fraction of (row, group) entries whose (scale, bias) differ from the reference pack;
    asserts that wherever they agree the 4-bit codes agree bit for bit.  The MSE clip search
    may pick another candidate only where two candidates' weighted errors tie up to fp32
    summation order."""
    same = np.all(sb.view(np.uint16) == ref_s.view(np.uint16), axis=-1)  # [tile, g, row]
    agree = same.transpose(0, 2, 1).reshape(-1, K // 64)
    cg = fm.unpack_marlin_codes(wm).reshape(-1, K // 64, 64)
    cr = fm.unpack_marlin_codes(ref_p).reshape(-1, K // 64, 64)
    assert np.array_equal(cg[agree], cr[agree]), what
    return float(1.0 - same.mean())
