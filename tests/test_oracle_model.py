"""Pins the oracle's cache, tree-verification and ring-buffer functions
(oracle/model.py) on the CPU, independently of the functions themselves.

* ``OracleKVCache.update`` in ring mode, ``OracleModel.forward_tree`` and
  ``OracleModel.forward_verify_ring`` are checked against a brute-force model
  (``Brute``) that keeps every token's per-layer key / value rows in a flat
  history and lets each query attend an explicitly listed set of tokens: no
  slot arithmetic, no masks, no ring positions.  The sets come from the
  reference semantics: a ring of S slots holds the last S tokens
  (axiomlm/engine/paged_cache.py:289-331), a tree node attends the prefix, its
  ancestors and itself at RoPE position seen + depth
  (axiomlm/models/transformer.py:600-684), and the runner's wrap-around
  verify step attends all S slots unmasked
  (axiomlm/kernels/mps_kernels.mm:3380-3464).
* ``forward_tree`` is also checked node by node against ``forward`` over the
  node's own ancestor path, and on a chain against ``forward`` of the chain.
* ``compact_tree_path`` is checked against a gather from a snapshot, with
  source and destination slots overlapping and wrapping
  (paged_cache.py:376-462).
* ``quantize_kv_int4_single`` is checked against torch's own round / clamp /
  int8 cast on exact .5 ties and all-zero groups (quant.py:789-803).

Each brute-force comparison also checks that a plausible mistake (one extra
or one missing key, a position off by one) moves the result by far more than
the tolerance, so the tolerance cannot hide such a mistake.
"""

import copy

import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import model as om

F16, F32 = np.float16, np.float32
TOL = 1e-2  # a few fp16 ulps at |logit| <= 4.7 (fp32 summation order); planted mistakes move > 3
TOL_Q = 3e-2  # fp8 / int4 caches: a one-ulp hidden difference can flip a code over many steps


def _tol(cache_dtype):
    return TOL if cache_dtype == "fp16" else TOL_Q


# ---------------------------------------------------------------------------
# INT4 KV codes against torch (quant.py:789-803)
# ---------------------------------------------------------------------------
def _torch_int4(x16: np.ndarray):
    x = torch.from_numpy(np.ascontiguousarray(x16))
    G = max(1, x.shape[-1] // 64)
    xg = x.view(*x.shape[:-1], G, 64)
    s = torch.clamp(xg.abs().amax(dim=-1, keepdim=True) / 7.0, min=1e-8).to(torch.float16)
    q = torch.clamp(torch.round((xg / s).float()), -8, 7).to(torch.int8)
    qp = q.view(*x.shape[:-1], G, 32, 2)
    packed = ((qp[..., 0] & 0x0F) | ((qp[..., 1] & 0x0F) << 4)).to(torch.uint8)
    return packed.view(*x.shape[:-1], x.shape[-1] // 2).numpy(), s.squeeze(-1).numpy()


def test_int4_kv_ties_round_half_even_like_torch():
    # scale 1.75 / 7 = 0.25 exactly; (k + 0.5) * 0.25 / 0.25 = k + 0.5 exactly in fp16
    # (|quotient| <= 7 always, as the scale is amax / 7)
    halves = np.arange(-7, 7) + 0.5
    row = np.zeros(128, F32)
    row[0], row[64] = 1.75, -1.75
    row[1:1 + len(halves)] = halves * 0.25
    row[65:65 + len(halves)] = -halves * 0.25
    x = row.astype(F16)[None, :]
    ours_p, ours_s = fm.quantize_kv_int4_single(x)
    ref_p, ref_s = _torch_int4(x)
    assert np.array_equal(ours_s.view(np.uint16), ref_s.view(np.uint16))
    assert np.array_equal(ours_p, ref_p)
    # round-half-even, not half-away: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -0.5 -> 0, -1.5 -> -2
    dq = fm.dequantize_kv_int4(ours_p, ours_s).astype(F32)[0] / 0.25
    got = dict(zip(halves.tolist(), dq[1:1 + len(halves)].tolist()))
    assert got[0.5] == 0 and got[1.5] == 2 and got[2.5] == 2 and got[-0.5] == 0 and got[-1.5] == -2
    assert got[6.5] == 6 and got[-6.5] == -6 and got[3.5] == 4 and got[-4.5] == -4


def test_int4_kv_zero_groups_and_random_match_torch():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((6, 9, 128)).astype(F16)
    x[0, 0, :64] = 0  # all-zero group: scale 0, 0/0 = NaN -> torch's int8 cast of NaN
    x[1, 2, 64:] = 0
    x[2, 3, :64] = (rng.standard_normal(64) * 1e-6).astype(F16)  # subnormal amax / 7
    x[3, 4, 64:] = F16(6e-8)
    ours_p, ours_s = fm.quantize_kv_int4_single(x)
    ref_p, ref_s = _torch_int4(x)
    assert np.array_equal(ours_s.view(np.uint16), ref_s.view(np.uint16))
    assert np.array_equal(ours_p, ref_p)
    assert ours_s[0, 0, 0] == 0 and np.all(ours_p[0, 0, :32] == 0)


def test_int4_kv_exhaustive_quotients_match_torch():
    # every fp16 value in [-8.5, 8.5] as x with scale 1 (amax 7 in each group pins the scale)
    vals = np.arange(65536, dtype=np.uint16).view(F16)
    vals = vals[np.isfinite(vals) & (np.abs(vals.astype(F32)) <= 8.5)]
    n = (len(vals) + 62) // 63
    grid = np.zeros(n * 63, F16)
    grid[:len(vals)] = vals
    grid = grid.reshape(n, 63)
    x = np.concatenate([np.full((n, 1), 7.0, F16), grid], axis=1)  # amax 7 (and 8.5 -> scale 8.5/7)
    x = np.concatenate([x, x], axis=1)
    ours_p, ours_s = fm.quantize_kv_int4_single(x)
    ref_p, ref_s = _torch_int4(x)
    assert np.array_equal(ours_s.view(np.uint16), ref_s.view(np.uint16))
    assert np.array_equal(ours_p, ref_p)


# ---------------------------------------------------------------------------
# Brute-force model: explicit attention sets over a flat token history
# ---------------------------------------------------------------------------
def _tiny(n_kv_head=2, std=0.08, seed=3):
    cfg = om.OracleConfig(n_layer=2, n_head=4, n_kv_head=n_kv_head, d_model=256, hidden=256, vocab=256, eps=1e-5,
                          block_size=512)
    W = om.make_float_weights(cfg, seed=seed, std=std)
    ow = om.pack_model_rtn(cfg, W)
    cos, sin = om.rope_tables(cfg.head_dim, cfg.block_size)
    return cfg, om.OracleModel(cfg, ow, cos, sin)


class Brute:
    """Every token fed keeps its per-layer key / value rows as a cache read returns them
    (quantized, then dequantized); token ids number the history in feeding order."""

    def __init__(self, model: om.OracleModel, cache_dtype: str = "fp16"):
        self.m = model
        self.dtype = cache_dtype
        self.k = []  # k[token][layer] -> [Hkv, hd] fp16
        self.v = []
        self.k_codes = []  # codes of layer 0 as the cache stores them

    def _stored(self, x):
        if self.dtype == "fp8":
            c, s = fm.quantize_kv_fp8_single(x)
            return fm.dequantize_kv_fp8(c, s), (c, s)
        if self.dtype == "int4":
            c, s = fm.quantize_kv_int4_single(x)
            return fm.dequantize_kv_int4(c, s), (c, s)
        return x, (x, None)

    def feed(self, tokens, positions, attend):
        """tokens [T]; positions [T] (RoPE); attend[t]: history ids token t attends, where this
        call's tokens get ids len(history) + t.  Returns logits [T, V]."""
        m, c = self.m, self.m.cfg
        T = len(tokens)
        hd = c.head_dim
        qd, kvd = c.n_head * hd, c.n_kv_head * hd
        n_rep = c.n_head // c.n_kv_head
        base = len(self.k)
        new_k = [[None] * c.n_layer for _ in range(T)]
        new_v = [[None] * c.n_layer for _ in range(T)]
        codes0 = [None] * T
        pos = np.asarray(positions)
        cs, sn = m.cos[pos], m.sin[pos]
        x = fm.dequant_q8_rows(np.asarray(tokens), m.w.wte_p, m.w.wte_sb).astype(F16)
        for i in range(c.n_layer):
            h1 = om.rmsnorm_fp16(x, m.w.ln1[i], c.eps)
            qkv = om.qlin(h1, m.w.c_attn_p[i], m.w.c_attn_s[i], qd + 2 * kvd)
            q = om.apply_rope_fp16(qkv[:, :qd].reshape(T, c.n_head, hd).transpose(1, 0, 2), cs, sn)
            k = om.apply_rope_fp16(qkv[:, qd:qd + kvd].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2), cs, sn)
            v = qkv[:, qd + kvd:].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            for t in range(T):
                new_k[t][i], kc = self._stored(np.ascontiguousarray(k[:, t]))
                new_v[t][i], _ = self._stored(np.ascontiguousarray(v[:, t]))
                if i == 0:
                    codes0[t] = kc

            def row(store, new, j, h):
                return store[j][i][h] if j < base else new[j - base][i][h]

            y = np.zeros((T, qd), F16)
            for t in range(T):
                for h in range(c.n_head):
                    g = h // n_rep
                    K = np.stack([row(self.k, new_k, j, g) for j in attend[t]])
                    V = np.stack([row(self.v, new_v, j, g) for j in attend[t]])
                    y[t, h * hd:(h + 1) * hd] = om.sdpa_fp16(q[h, t:t + 1], K, V)[0]
            x = (x.astype(F32) + om.qlin(y, m.w.c_proj_p[i], m.w.c_proj_s[i], qd).astype(F32)).astype(F16)
            h2 = om.rmsnorm_fp16(x, m.w.ln2[i], c.eps)
            gu = om.qlin(h2, m.w.gu_p[i], m.w.gu_s[i], 2 * c.hidden)
            gg, uu = gu[:, :c.hidden].astype(F32), gu[:, c.hidden:].astype(F32)
            sw = (gg / (1 + np.exp(-gg))).astype(F16).astype(F32) * uu
            x = (x.astype(F32) + om.qlin(sw.astype(F16), m.w.wd_p[i], m.w.wd_s[i], qd).astype(F32)).astype(F16)
        self.k += new_k
        self.v += new_v
        self.k_codes += codes0
        xn = om.rmsnorm_fp16(x, m.w.lnf, c.eps)
        return om.qlin(xn, m.w.lmh_p, m.w.lmh_sb, c.vocab).astype(F32)


def _maxdiff(a, b):
    return float(np.max(np.abs(np.asarray(a, F32) - np.asarray(b, F32))))


def _prefill(model, brute, cache, toks, window=None, tol=TOL):
    """Feed tokens one at a time into the oracle cache and the brute force (causal, over
    the last ``window`` tokens when the cache is a ring of that many slots)."""
    for t in toks:
        n = len(brute.k)
        lo = 0 if window is None else max(0, n + 1 - window)
        want = brute.feed([t], [n], [list(range(lo, n + 1))])
        got = model.forward([t], cache)[-1]
        assert _maxdiff(got, want[0]) <= tol


# ---------------------------------------------------------------------------
# forward_tree
# ---------------------------------------------------------------------------
def _random_tree(rng, T):
    parents = [-1] + [int(rng.integers(-1, u)) for u in range(1, T)]
    depths, masks = [], []
    for u, p in enumerate(parents):
        depths.append(0 if p < 0 else depths[p] + 1)
        masks.append((1 << u) | (0 if p < 0 else masks[p]))
    return parents, depths, masks


def _ancestors(parents, u):
    path = []
    while u >= 0:
        path.append(u)
        u = parents[u]
    return path[::-1]


@pytest.mark.parametrize("cache_dtype", ["fp16", "fp8", "int4"])
def test_forward_tree_nodes_equal_their_ancestor_paths(cache_dtype):
    rng = np.random.default_rng(21)
    cfg, model = _tiny()
    prefix = rng.integers(0, cfg.vocab, 9).tolist()
    T = 14
    parents, depths, masks = _random_tree(rng, T)
    assert max(depths) >= 3 and parents.count(-1) >= 2
    toks = rng.integers(0, cfg.vocab, T).tolist()
    cache = om.OracleKVCache(64, cfg.n_layer, cfg.n_kv_head, cfg.head_dim, cache_dtype)
    brute = Brute(model, cache_dtype)
    _prefill(model, brute, cache, prefix, tol=_tol(cache_dtype))
    seen = len(prefix)
    base_cache = copy.deepcopy(cache)
    got = model.forward_tree(toks, cache, depths, masks).astype(F32)
    assert got.shape == (T, cfg.vocab)

    # (1) brute force: node u attends prefix + its ancestors + itself at position seen + depth
    attend = [list(range(seen)) + [seen + a for a in _ancestors(parents, u)] for u in range(T)]
    want = brute.feed(toks, [seen + d for d in depths], attend)
    assert _maxdiff(got, want) <= _tol(cache_dtype)
    # slots seen + j hold node j's layer-0 key codes (exact: they depend on token and position only)
    for j in range(T):
        kc, ks = brute.k_codes[seen + j]
        assert np.array_equal(cache.k[0][:, seen + j], kc)
        if ks is not None:
            assert np.array_equal(cache.ks[0][:, seen + j], ks)

    # (2) each node equals forward() over its own ancestor path after the same prefix
    for u in range(T):
        path = _ancestors(parents, u)
        c2 = copy.deepcopy(base_cache)
        ref = model.forward([toks[a] for a in path], c2)[-1]
        assert _maxdiff(got[u], ref) <= _tol(cache_dtype), u

    # a plausible mistake moves the logits well past the tolerance
    wrong_mask = Brute(model, cache_dtype)
    wrong_mask.k, wrong_mask.v = brute.k[:seen], brute.v[:seen]
    bad = [a + [seen + (u + 1) % T] if (seen + (u + 1) % T) not in a else a[:-1] for u, a in enumerate(attend)]
    assert _maxdiff(wrong_mask.feed(toks, [seen + d for d in depths], bad), want) > 20 * TOL_Q
    wrong_pos = Brute(model, cache_dtype)
    wrong_pos.k, wrong_pos.v = brute.k[:seen], brute.v[:seen]
    assert _maxdiff(wrong_pos.feed(toks, [seen + u for u in range(T)], attend), want) > 20 * TOL_Q


def test_forward_tree_chain_equals_forward():
    rng = np.random.default_rng(5)
    cfg, model = _tiny()
    prefix = rng.integers(0, cfg.vocab, 7).tolist()
    toks = rng.integers(0, cfg.vocab, 6).tolist()
    cache = om.OracleKVCache(32, cfg.n_layer, cfg.n_kv_head, cfg.head_dim)
    model.forward(prefix, cache)
    c2 = copy.deepcopy(cache)
    T = len(toks)
    got = model.forward_tree(toks, cache, list(range(T)), [(1 << (t + 1)) - 1 for t in range(T)])
    ref = model.forward(toks, c2, return_all_logits=True)
    assert _maxdiff(got, ref) <= TOL
    assert np.array_equal(cache.k, c2.k) and np.array_equal(cache.v, c2.v)


# ---------------------------------------------------------------------------
# Ring buffer: update (T = 1 past the end) and the wrap-around verify step
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("cache_dtype,ring", [("fp16", True), ("int4", True), ("fp8", False)])
def test_ring_update_is_a_sliding_window(cache_dtype, ring):
    S = 16
    rng = np.random.default_rng(8)
    cfg, model = _tiny(n_kv_head=4)
    toks = rng.integers(0, cfg.vocab, 3 + 2 * S + 5).tolist()
    cache = om.OracleKVCache(S, cfg.n_layer, cfg.n_kv_head, cfg.head_dim, cache_dtype, ring_buffer=ring)
    brute = Brute(model, cache_dtype)
    worst, worst_off = 0.0, 0.0
    for n, t in enumerate(toks):
        got = model.forward([t], cache)[-1]
        if n == S + 2:  # a window one token too wide must not pass
            w = copy.deepcopy(brute)
            off = w.feed([t], [n], [list(range(max(0, n - S), n + 1))])[0]
        want = brute.feed([t], [n], [list(range(max(0, n + 1 - S), n + 1))])[0]
        worst = max(worst, _maxdiff(got, want))
        if n == S + 2:
            worst_off = _maxdiff(off, want)
        # slot s holds the newest token congruent to s mod S (layer 0 codes are exact)
        for s in range(min(n + 1, S)):
            j = n - ((n - s) % S)
            assert np.array_equal(cache.k[0][:, s], brute.k_codes[j][0]), (n, s)
    assert worst <= _tol(cache_dtype)
    assert worst_off > 20 * TOL_Q
    # axiomlm tests/test_metal_boundary_and_tiling.py:125-130 (3 + 64 tokens, window 32): counters
    assert cache.total_seen_tokens == [len(toks)] * cfg.n_layer
    assert cache.layer_seq_lens == [S] * cfg.n_layer


def test_ring_counters_reference_case():
    # 3-token prompt then 64 single tokens through a 32-slot ring: 67 seen, 32 active.
    cache = om.OracleKVCache(32, 2, 2, 64, "fp16", ring_buffer=True)
    rng = np.random.default_rng(0)
    kv = lambda T: rng.standard_normal((2, T, 64)).astype(F16)  # noqa: E731
    cache.update(0, kv(3), kv(3))
    for _ in range(64):
        k, _ = cache.update(0, kv(1), kv(1))
        assert k.shape[1] <= 32
    assert cache.total_seen_tokens[0] == 67 and cache.layer_seq_lens[0] == 32
    # the int4 variant of the same check (test_phase3_task31_kv_quantization.py:630-650): 25 into 16
    c4 = om.OracleKVCache(16, 1, 2, 64, "int4", ring_buffer=True)
    for _ in range(25):
        k, _ = c4.update(0, kv(1), kv(1))
        assert k.shape[1] <= 16
    assert c4.layer_seq_lens[0] == 16 and c4.total_seen_tokens[0] == 25


@pytest.mark.parametrize("cache_dtype,n_before", [("fp16", 40), ("fp16", 14), ("fp8", 21)])
def test_verify_ring_attends_the_last_S_tokens(cache_dtype, n_before):
    S, T = 16, 5
    rng = np.random.default_rng(n_before)
    cfg, model = _tiny()
    toks = rng.integers(0, cfg.vocab, n_before).tolist()
    new = rng.integers(0, cfg.vocab, T).tolist()
    cache = om.OracleKVCache(S, cfg.n_layer, cfg.n_kv_head, cfg.head_dim, cache_dtype, ring_buffer=True)
    brute = Brute(model, cache_dtype)
    _prefill(model, brute, cache, toks, window=S, tol=_tol(cache_dtype))
    c_seq = copy.deepcopy(cache)
    got = model.forward_verify_ring(new, cache, n_before, n_before % S)
    total = n_before + T
    window = list(range(total - S, total))
    want = brute.feed(new, [n_before + t for t in range(T)], [window] * T)
    assert _maxdiff(got, want) <= _tol(cache_dtype)
    # the reference's sequence forward over a wrapped ring attends the same slots (mask all true)
    if n_before >= S:
        seq = model.forward(new, c_seq, return_all_logits=True)
        assert _maxdiff(seq, got) <= _tol(cache_dtype)
    # causal masking inside the batch would be a different (wrong) result
    causal = [window[:S - T + t + 1] for t in range(T)]
    w = Brute(model, cache_dtype)
    w.k, w.v = brute.k[:n_before], brute.v[:n_before]
    assert _maxdiff(w.feed(new, [n_before + t for t in range(T)], causal), want) > 20 * TOL_Q


# ---------------------------------------------------------------------------
# compact_tree_path
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("cache_dtype", ["fp16", "fp8", "int4"])
@pytest.mark.parametrize("write_pos,accepted", [(3, [0, 2, 3, 7]), (13, [1, 4, 5]), (2, [2, 0, 1]), (5, [0, 1, 2])])
def test_compact_tree_path_is_a_snapshot_gather(cache_dtype, write_pos, accepted):
    S = 16
    rng = np.random.default_rng(write_pos)
    cache = om.OracleKVCache(S, 3, 2, 64, cache_dtype, ring_buffer=True)
    if cache_dtype == "fp16":
        cache.k[:] = rng.standard_normal(cache.k.shape).astype(F16)
        cache.v[:] = rng.standard_normal(cache.v.shape).astype(F16)
    else:
        cache.k[:] = rng.integers(0, 256, cache.k.shape, dtype=np.uint8)
        cache.v[:] = rng.integers(0, 256, cache.v.shape, dtype=np.uint8)
        cache.ks[:] = rng.standard_normal(cache.ks.shape).astype(F16)
        cache.vs[:] = rng.standard_normal(cache.vs.shape).astype(F16)
    before = {n: (None if getattr(cache, n) is None else getattr(cache, n).copy()) for n in ("k", "v", "ks", "vs")}
    cache.compact_tree_path(write_pos, accepted, new_total_seen=40 + len(accepted))
    moved = {(write_pos + m) % S: (write_pos + a) % S for m, a in enumerate(accepted)}
    for name, arr in before.items():
        if arr is None:
            continue
        now = getattr(cache, name)
        for s in range(S):
            want = arr[:, :, moved.get(s, s)]
            assert np.array_equal(now[:, :, s], want), (name, s)
    assert cache.total_seen_tokens == [40 + len(accepted)] * 3
    assert cache.layer_seq_lens == [S] * 3
    # counters only below the ring size
    c2 = om.OracleKVCache(S, 1, 2, 64)
    c2.compact_tree_path(0, [0, 1], new_total_seen=7)
    assert c2.total_seen_tokens == [7] and c2.layer_seq_lens == [7]


# ---------------------------------------------------------------------------
# Primitives against closed forms
# ---------------------------------------------------------------------------
def test_rmsnorm_matches_float64_within_fp16_rounding():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((16, 512)) * 3).astype(F16)
    w = (1 + 0.1 * rng.standard_normal(512)).astype(F16)
    got = om.rmsnorm_fp16(x, w, 1e-5).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * w.astype(np.float64)
    # four fp16 roundings (square, mean, rsqrt, two products) bound the relative error by ~5 ulps
    assert np.all(np.abs(got - ref) <= 5 * 2.0 ** -11 * np.abs(ref) + 1e-6)
    # a dropped eps or a missing weight would be far outside that bound
    assert np.max(np.abs(got - xd / np.sqrt((xd * xd).mean(-1, keepdims=True)))) > 0.05


def test_sdpa_closed_forms():
    rng = np.random.default_rng(2)
    v = rng.standard_normal((2, 6, 64)).astype(F16)
    # equal scores -> the mean of the values
    q = np.zeros((2, 1, 64), F16)
    k = rng.standard_normal((2, 6, 64)).astype(F16)
    got = om.sdpa_fp16(q, k, v).astype(F32)
    assert np.allclose(got[:, 0], v.astype(F32).mean(1), atol=2e-3)
    # a dominant key -> its value
    k2 = np.zeros((2, 6, 64), F16)
    k2[:, 3, 0] = 60.0
    q2 = np.zeros((2, 1, 64), F16)
    q2[:, 0, 0] = 60.0
    assert np.array_equal(om.sdpa_fp16(q2, k2, v)[:, 0], v[:, 3])
    # a boolean mask removes keys exactly as gathering the kept ones does
    q3 = rng.standard_normal((2, 3, 64)).astype(F16)
    mask = np.array([[1, 0, 1, 1, 0, 0], [0, 1, 1, 0, 0, 1], [1, 1, 1, 1, 1, 1]], bool)
    masked = om.sdpa_fp16(q3, k, v, mask=mask).astype(F32)
    for r in range(3):
        keep = np.nonzero(mask[r])[0]
        alone = om.sdpa_fp16(q3[:, r:r + 1], k[:, keep], v[:, keep]).astype(F32)
        assert np.allclose(masked[:, r], alone[:, 0], atol=2e-3)
    # float64 softmax reference
    s = (q3.astype(np.float64) @ k.astype(np.float64).transpose(0, 2, 1)) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = (p / p.sum(-1, keepdims=True)) @ v.astype(np.float64)
    assert np.allclose(om.sdpa_fp16(q3, k, v).astype(np.float64), ref, atol=2e-3)


def test_rope_preserves_pair_norms_and_composes():
    cos, sin = om.rope_tables(64, 64)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 64)).astype(F16)
    pos = np.array([0, 1, 7, 33, 63])
    y = om.apply_rope_fp16(x, cos[pos], sin[pos]).astype(np.float64)
    xp = x.astype(np.float64).reshape(5, 32, 2)
    yp = y.reshape(5, 32, 2)
    assert np.allclose(np.hypot(xp[..., 0], xp[..., 1]), np.hypot(yp[..., 0], yp[..., 1]), rtol=2e-3, atol=2e-3)
    assert np.array_equal(y[0], x[0].astype(np.float64))  # position 0 is the identity
    # angle of pair i at position p is p * theta^(-2i/hd)
    inv = 10000.0 ** (-np.arange(0, 64, 2) / 64.0)
    assert np.allclose(cos, np.cos(np.outer(np.arange(64), inv)), atol=1e-5)
