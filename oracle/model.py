"""numpy restatement of the reference quantized decoder forward (TEST INFRASTRUCTURE).

Follows the CPU path of a half-precision AxiomLM model:
  * ``Transformer._forward_quantized_sequence`` (axiomlm/models/transformer.py:1036-1200)
  * ``RMSNorm.forward`` (axiomlm/models/modules.py:41-43), ``precompute_rope_frequencies``
    (:46-92, default scaling only), ``repeat_kv`` (:120-132)
  * ``StaticKVCache.update`` (axiomlm/engine/paged_cache.py:218-361), fp16 / fp8 / int4 and
    the ring-buffer mode; ``compact_tree_path`` (:376-462)
  * the boolean-mask tree verification fallback (transformer.py:639-784) and the
    decode / tree attention fallbacks (axiomlm/kernels/ops.py:612-654, 739-797)
  * greedy decoding: argmax with the lowest index on ties (torch.argmax).

Every fp16 op rounds to fp16; matmuls and SDPA accumulate in fp32 and round once.

This module is test infrastructure: only tests/, the smoke check and the CPU
baseline of bench.py use it, as the checker.

Pinning (tests/test_oracle_model.py unless noted):
  * RMSNorm against a float64 evaluation, SDPA against equal-score / dominant-key
    closed forms, a float64 softmax and key gathering, RoPE pair norms and angles;
  * ``forward`` (decode, 32-token prefill, 64 greedy tokens) against golden logits
    written from the reference by tests/golden/make_golden_c1.py
    (tests/test_oracle_golden.py);
  * ``OracleKVCache.update`` in ring mode, ``forward_tree`` and
    ``forward_verify_ring`` against a brute-force model with explicit per-query
    key sets over a flat token history (sliding window, prefix + ancestors at
    seen + depth, all S slots), ``forward_tree`` against ``forward`` over each
    node's ancestor path and over a chain, the reference ring counters 67 / 32
    and 25 / 16;
  * ``compact_tree_path`` against a gather from a snapshot (overlapping and
    wrapping slots, a non-monotonic accepted list).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import formats as fm

F16 = np.float16
F32 = np.float32


def _h(x):
    return np.asarray(x, dtype=F32).astype(F16).astype(F32)


# ---------------------------------------------------------------------------
# primitives
# ---------------------------------------------------------------------------
def rmsnorm_fp16(x16: np.ndarray, w16: np.ndarray, eps: float) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * w on fp16 tensors (modules.py:41-43)."""
    x = x16.astype(F32)
    sq = _h(x * x)
    mean = _h(sq.mean(axis=-1, keepdims=True, dtype=F32))
    t = _h(mean + F32(eps))
    r = _h(F32(1.0) / np.sqrt(t))
    return _h(_h(x * r) * w16.astype(F32)).astype(F16)


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0):
    """(cos, sin) fp32 [max_seq_len, head_dim/2] of precompute_rope_frequencies (modules.py:58-92)."""
    inv = (F32(1.0) / (F32(theta) ** (np.arange(0, head_dim, 2, dtype=np.int64).astype(F32) / F32(head_dim)))).astype(F32)
    t = np.arange(max_seq_len, dtype=F32)
    fr = np.outer(t, inv).astype(F32)
    return np.cos(fr).astype(F32), np.sin(fr).astype(F32)


def apply_rope_fp16(x16: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Interleaved-pair complex rotation in fp32, rounded to fp16.

    x16: [..., T, hd]; cos/sin: [T, hd/2] (already gathered per position)."""
    x = x16.astype(F32).reshape(*x16.shape[:-1], -1, 2)
    a, b = x[..., 0], x[..., 1]
    re = a * cos - b * sin
    im = a * sin + b * cos
    return np.stack([re, im], axis=-1).reshape(x16.shape).astype(F16)


def rope_kv_rows(qkv16: np.ndarray, cos: np.ndarray, sin: np.ndarray, positions, q_dim: int, kv_dim: int, hd: int,
                 bias: np.ndarray | None = None):
    """CPU fallback of ``rope_kv_cache_write_quantized`` (quant.py:960-1008) for T token rows
    qkv16 [T, q_dim + 2 kv_dim]: fp16 bias add, then query and key rotated at their
    positions.  Returns (q [T, q_dim], k [Hkv, T, hd], v [Hkv, T, hd]) fp16; the caller stores
    k / v with ``OracleKVCache.write`` (quantizing for fp8 / int4)."""
    x = qkv16.astype(F16)
    if bias is not None:
        x = _h(x.astype(F32) + bias.astype(F32)[None, :]).astype(F16)
    T = x.shape[0]
    pos = np.asarray(positions, dtype=np.int64)
    c, s_ = cos[pos], sin[pos]
    q = x[:, :q_dim].reshape(T, -1, hd).transpose(1, 0, 2)
    k = x[:, q_dim:q_dim + kv_dim].reshape(T, -1, hd).transpose(1, 0, 2)
    v = x[:, q_dim + kv_dim:].reshape(T, -1, hd).transpose(1, 0, 2)
    q = apply_rope_fp16(q, c, s_).transpose(1, 0, 2).reshape(T, q_dim)
    return q, apply_rope_fp16(k, c, s_), np.ascontiguousarray(v)


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    return x if n_rep == 1 else np.repeat(x, n_rep, axis=-3)


def sdpa_fp16(q16, k16, v16, mask=None, is_causal=False):
    """Scaled dot-product attention, fp32 math, fp16 output.

    q: [..., Tq, hd], k/v: [..., Tk, hd], mask: bool [Tq, Tk] (True = attend)."""
    q = q16.astype(F32)
    k = k16.astype(F32)
    v = v16.astype(F32)
    scale = F32(1.0 / math.sqrt(q.shape[-1]))
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    Tq, Tk = s.shape[-2], s.shape[-1]
    if is_causal:
        mask = np.tril(np.ones((Tq, Tk), dtype=bool))
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    den = p.sum(axis=-1, keepdims=True)
    out = (p @ v) / np.where(den > 0, den, 1.0)
    return out.astype(F16)


def argmax_first(x: np.ndarray) -> int:
    return int(np.argmax(x.astype(F32)))


# ---------------------------------------------------------------------------
# KV cache (StaticKVCache semantics)
# ---------------------------------------------------------------------------
class OracleKVCache:
    """paged_cache.py:122-462 for batch 1 (fp16 / fp8 / int4, monotonic or ring)."""

    def __init__(self, max_seq_len, n_layer, n_kv_head, head_dim, cache_dtype="fp16", ring_buffer=False):
        self.S = max_seq_len
        self.n_layer = n_layer
        self.Hkv = n_kv_head
        self.hd = head_dim
        self.dtype = cache_dtype
        self.ring = ring_buffer
        G = max(1, head_dim // 64)
        if cache_dtype == "fp16":
            self.k = np.zeros((n_layer, n_kv_head, max_seq_len, head_dim), F16)
            self.v = np.zeros_like(self.k)
            self.ks = self.vs = None
        else:
            width = head_dim if cache_dtype == "fp8" else head_dim // 2
            self.k = np.zeros((n_layer, n_kv_head, max_seq_len, width), np.uint8)
            self.v = np.zeros_like(self.k)
            self.ks = np.zeros((n_layer, n_kv_head, max_seq_len, G), F16)
            self.vs = np.zeros_like(self.ks)
        self.total_seen_tokens = [0] * n_layer
        self.layer_seq_lens = [0] * n_layer
        # When frozen, writes are skipped: the cache contents were loaded from
        # another implementation and attention must read exactly those codes.
        # The codes a write would have stored are kept in last_write[layer] as
        # (slots, k_codes, k_scales, v_codes, v_scales) for comparison.
        self.frozen = False
        self.last_write = [None] * n_layer

    def _quant(self, x16):
        if self.dtype == "fp8":
            return fm.quantize_kv_fp8_single(x16)
        if self.dtype == "int4":
            return fm.quantize_kv_int4_single(x16)
        return x16, None

    def _dequant(self, codes, scales):
        if self.dtype == "fp8":
            return fm.dequantize_kv_fp8(codes, scales)
        if self.dtype == "int4":
            return fm.dequantize_kv_int4(codes, scales)
        return codes

    def write(self, layer, slots, k16, v16):
        """Store rows k16/v16 [Hkv, T, hd] at the given slots."""
        kq, ks = self._quant(k16)
        vq, vs = self._quant(v16)
        if self.frozen:
            self.last_write[layer] = (slots, kq, ks, vq, vs)
            return
        self.k[layer][:, slots] = kq
        self.v[layer][:, slots] = vq
        if ks is not None:
            self.ks[layer][:, slots] = ks
            self.vs[layer][:, slots] = vs

    def view(self, layer, n):
        ks = self.ks[layer][:, :n] if self.ks is not None else None
        vs = self.vs[layer][:, :n] if self.vs is not None else None
        return self._dequant(self.k[layer][:, :n], ks), self._dequant(self.v[layer][:, :n], vs)

    def update(self, layer, k16, v16):
        """paged_cache.py:218-361: returns dequantized active k, v [Hkv, L, hd]."""
        T = k16.shape[1]
        seen = self.total_seen_tokens[layer]
        if not self.ring and seen + T <= self.S:
            self.write(layer, np.arange(seen, seen + T), k16, v16)
            self.layer_seq_lens[layer] = self.total_seen_tokens[layer] = seen + T
            return self.view(layer, seen + T)
        if T >= self.S:
            self.write(layer, np.arange(self.S), k16[:, -self.S:], v16[:, -self.S:])
        else:
            slots = (seen + np.arange(T)) % self.S
            self.write(layer, slots, k16, v16)
        active = min(seen + T, self.S)
        self.layer_seq_lens[layer] = active
        self.total_seen_tokens[layer] = seen + T
        return self.view(layer, active)

    def compact_tree_path(self, write_pos, accepted, new_total_seen=None):
        """paged_cache.py:376-462."""
        if accepted and any(a != i for i, a in enumerate(accepted)):
            src = [(write_pos + a) % self.S for a in accepted]
            dst = [(write_pos + m) % self.S for m in range(len(accepted))]
            for arr in (self.k, self.v, self.ks, self.vs):
                if arr is not None:
                    staged = arr[:, :, src].copy()
                    arr[:, :, dst] = staged
        if new_total_seen is not None:
            self.total_seen_tokens = [new_total_seen] * self.n_layer
            self.layer_seq_lens = [min(new_total_seen, self.S)] * self.n_layer


# ---------------------------------------------------------------------------
# Quantized model
# ---------------------------------------------------------------------------
@dataclass
class OracleConfig:
    n_layer: int
    n_head: int
    n_kv_head: int
    d_model: int
    hidden: int
    vocab: int
    eps: float = 1e-5
    rope_theta: float = 10000.0
    block_size: int = 1024

    @property
    def head_dim(self):
        return self.d_model // self.n_head


@dataclass
class OracleWeights:
    """Packed weights as produced by ``Transformer._ensure_quant_weights`` (transformer.py:822-1008)."""

    wte_p: np.ndarray  # Q8_G64 uint8 [V, d]
    wte_sb: np.ndarray
    lmh_p: np.ndarray  # MARLIN int32 [V/8, d/64, 32, 2] or Q8 uint8 [V, d]
    lmh_sb: np.ndarray
    ln1: list
    ln2: list
    lnf: np.ndarray
    c_attn_p: list
    c_attn_s: list
    c_proj_p: list
    c_proj_s: list
    gu_p: list
    gu_s: list
    wd_p: list
    wd_s: list
    c_attn_b: list = field(default_factory=list)


_DEQ_MEMO: dict = {}


def _dequantized(wp, wsb, K, out_features):
    """fp16 weights of a packed matrix, memoized per packed array (the entry keeps the
    arrays alive, so an id is never reused while its entry exists)."""
    key = (id(wp), id(wsb), K, out_features)
    hit = _DEQ_MEMO.get(key)
    if hit is not None and hit[0] is wp and hit[1] is wsb:
        return hit[2]
    if wsb is None:  # fp16 weights (the fp16 runner's layers)
        w = wp.astype(F16)
    elif wp.ndim == 4 and wsb.shape[1] * 2 == wp.shape[1]:
        w = fm.dequantize_q4_marlin_g128(wp, wsb, K, out_features)
    elif wp.ndim == 4:
        w = fm.dequantize_q4_marlin(wp, wsb, K, out_features)
    else:
        w = fm.dequantize_q8_g64(wp, wsb, K)
    if sum(e[2].nbytes for e in _DEQ_MEMO.values()) + w.nbytes > (1 << 30):
        _DEQ_MEMO.clear()
    _DEQ_MEMO[key] = (wp, wsb, w)
    return w


def qlin(x16, wp, wsb, out_features, bias=None):
    """Transformer._qlin (transformer.py:1010-1034): the CPU fallback dequantizes the
    packed weights to fp16 (quant.py:656-661, 597-634 / 72-129), then F.linear."""
    K = x16.shape[-1]
    w = _dequantized(wp, wsb, K, out_features)
    y = fm.linear_fp16(x16, w)
    if bias is not None:
        y = (y.astype(F32) + bias.astype(F32)).astype(F16)
    return y


class OracleModel:
    def __init__(self, cfg: OracleConfig, w: OracleWeights, cos: np.ndarray, sin: np.ndarray):
        self.cfg = cfg
        self.w = w
        self.cos = cos
        self.sin = sin

    def _embed(self, idx):
        """Token rows: the Q8_G64 gather (quant.py:132-163), or an fp16 table (the fp16 model)."""
        if self.w.wte_sb is None:
            return self.w.wte_p[idx].astype(F16)
        return fm.dequant_q8_rows(idx, self.w.wte_p, self.w.wte_sb).astype(F16)

    # -- transformer.py:1036-1200 ------------------------------------------
    def forward(self, idx, cache: OracleKVCache | None = None, return_all_logits=False, return_norm=False):
        c = self.cfg
        idx = np.asarray(idx).reshape(-1)
        T = idx.shape[0]
        hd = c.head_dim
        qd, kvd = c.n_head * hd, c.n_kv_head * hd
        n_rep = c.n_head // c.n_kv_head
        x = self._embed(idx)  # [T, d]
        for i in range(c.n_layer):
            start = cache.total_seen_tokens[i] if cache is not None else 0
            h1 = rmsnorm_fp16(x, self.w.ln1[i], c.eps)
            b_i = self.w.c_attn_b[i] if self.w.c_attn_b else None
            qkv = qlin(h1, self.w.c_attn_p[i], self.w.c_attn_s[i], qd + 2 * kvd, b_i)
            q = qkv[:, :qd].reshape(T, c.n_head, hd).transpose(1, 0, 2)
            k = qkv[:, qd:qd + kvd].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            v = qkv[:, qd + kvd:].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            pos = start + np.arange(T)
            cs, sn = self.cos[pos], self.sin[pos]
            q = apply_rope_fp16(q, cs, sn)
            k = apply_rope_fp16(k, cs, sn)
            if cache is not None:
                k, v = cache.update(i, k, v)
            mask = None
            is_causal = False
            if T > 1 and start > 0:
                qp = (start + np.arange(T))[:, None]
                kp = np.arange(k.shape[1])[None, :]
                mask = kp <= qp
            else:
                is_causal = T > 1 and start == 0
            y = sdpa_fp16(q, repeat_kv(k, n_rep), repeat_kv(v, n_rep), mask=mask, is_causal=is_causal)
            y = y.transpose(1, 0, 2).reshape(T, qd)
            attn_out = qlin(y, self.w.c_proj_p[i], self.w.c_proj_s[i], qd)
            x = (x.astype(F32) + attn_out.astype(F32)).astype(F16)
            h2 = rmsnorm_fp16(x, self.w.ln2[i], c.eps)
            gu = qlin(h2, self.w.gu_p[i], self.w.gu_s[i], 2 * c.hidden)
            g, u = gu[:, :c.hidden].astype(F32), gu[:, c.hidden:].astype(F32)
            sw = _h(_h(g / (F32(1.0) + np.exp(-g))) * u).astype(F16)
            mlp = qlin(sw, self.w.wd_p[i], self.w.wd_s[i], qd)
            x = (x.astype(F32) + mlp.astype(F32)).astype(F16)
        xt = x if (return_all_logits or cache is None) else x[-1:]
        xn = rmsnorm_fp16(xt, self.w.lnf, c.eps)
        logits = qlin(xn, self.w.lmh_p, self.w.lmh_sb, c.vocab)
        return (logits, xn) if return_norm else logits

    # -- transformer.py:639-784 (boolean-mask tree fallback) -------------------
    def forward_tree(self, idx, cache: OracleKVCache, depths, masks):
        c = self.cfg
        idx = np.asarray(idx).reshape(-1)
        T = idx.shape[0]
        hd = c.head_dim
        qd, kvd = c.n_head * hd, c.n_kv_head * hd
        n_rep = c.n_head // c.n_kv_head
        seen = cache.total_seen_tokens[0]
        S = cache.S
        write_pos = (seen % S) if (cache.ring or seen >= S) else seen
        assert write_pos + T <= S and seen == write_pos
        rope_pos = seen % self.cos.shape[0]
        attn_mask = np.zeros((T, seen + T), dtype=bool)
        attn_mask[:, :seen] = True
        for u in range(T):
            for j in range(T):
                if (int(masks[u]) >> j) & 1:
                    attn_mask[u, seen + j] = True
        pos = np.array([(rope_pos + int(d)) % self.cos.shape[0] for d in depths])
        cs, sn = self.cos[pos], self.sin[pos]
        x = self._embed(idx)
        for i in range(c.n_layer):
            h1 = rmsnorm_fp16(x, self.w.ln1[i], c.eps)
            b_i = self.w.c_attn_b[i] if self.w.c_attn_b else None
            qkv = qlin(h1, self.w.c_attn_p[i], self.w.c_attn_s[i], qd + 2 * kvd, b_i)
            q = qkv[:, :qd].reshape(T, c.n_head, hd).transpose(1, 0, 2)
            k = qkv[:, qd:qd + kvd].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            v = qkv[:, qd + kvd:].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            q = apply_rope_fp16(q, cs, sn)
            k = apply_rope_fp16(k, cs, sn)
            cache.write(i, np.arange(write_pos, write_pos + T), k, v)
            k_all, v_all = cache.view(i, seen + T)
            y = sdpa_fp16(q, repeat_kv(k_all, n_rep), repeat_kv(v_all, n_rep), mask=attn_mask)
            y = y.transpose(1, 0, 2).reshape(T, qd)
            x = (x.astype(F32) + qlin(y, self.w.c_proj_p[i], self.w.c_proj_s[i], qd).astype(F32)).astype(F16)
            h2 = rmsnorm_fp16(x, self.w.ln2[i], c.eps)
            gu = qlin(h2, self.w.gu_p[i], self.w.gu_s[i], 2 * c.hidden)
            g, u = gu[:, :c.hidden].astype(F32), gu[:, c.hidden:].astype(F32)
            sw = _h(_h(g / (F32(1.0) + np.exp(-g))) * u).astype(F16)
            x = (x.astype(F32) + qlin(sw, self.w.wd_p[i], self.w.wd_s[i], qd).astype(F32)).astype(F16)
        xn = rmsnorm_fp16(x, self.w.lnf, c.eps)
        return qlin(xn, self.w.lmh_p, self.w.lmh_sb, c.vocab)

    def forward_verify_ring(self, idx, cache: OracleKVCache, start_pos: int, write_pos: int):
        """verify_step of the reference runner when the T slots wrap around the ring
        (mps_kernels.mm:3380-3464): every token is rotated at start_pos + t and written to
        slot (write_pos + t) % S, then each token attends over all S slots, unmasked."""
        c = self.cfg
        idx = np.asarray(idx).reshape(-1)
        T = idx.shape[0]
        hd = c.head_dim
        qd, kvd = c.n_head * hd, c.n_kv_head * hd
        n_rep = c.n_head // c.n_kv_head
        S = cache.S
        pos = np.array([(start_pos + t) % self.cos.shape[0] for t in range(T)])
        cs, sn = self.cos[pos], self.sin[pos]
        slots = np.array([(write_pos + t) % S for t in range(T)])
        x = self._embed(idx)
        for i in range(c.n_layer):
            h1 = rmsnorm_fp16(x, self.w.ln1[i], c.eps)
            b_i = self.w.c_attn_b[i] if self.w.c_attn_b else None
            qkv = qlin(h1, self.w.c_attn_p[i], self.w.c_attn_s[i], qd + 2 * kvd, b_i)
            q = qkv[:, :qd].reshape(T, c.n_head, hd).transpose(1, 0, 2)
            k = qkv[:, qd:qd + kvd].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            v = qkv[:, qd + kvd:].reshape(T, c.n_kv_head, hd).transpose(1, 0, 2)
            q = apply_rope_fp16(q, cs, sn)
            k = apply_rope_fp16(k, cs, sn)
            cache.write(i, slots, k, v)
            k_all, v_all = cache.view(i, S)
            y = sdpa_fp16(q, repeat_kv(k_all, n_rep), repeat_kv(v_all, n_rep))
            y = y.transpose(1, 0, 2).reshape(T, qd)
            x = (x.astype(F32) + qlin(y, self.w.c_proj_p[i], self.w.c_proj_s[i], qd).astype(F32)).astype(F16)
            h2 = rmsnorm_fp16(x, self.w.ln2[i], c.eps)
            gu = qlin(h2, self.w.gu_p[i], self.w.gu_s[i], 2 * c.hidden)
            g, u = gu[:, :c.hidden].astype(F32), gu[:, c.hidden:].astype(F32)
            sw = _h(_h(g / (F32(1.0) + np.exp(-g))) * u).astype(F16)
            x = (x.astype(F32) + qlin(sw, self.w.wd_p[i], self.w.wd_s[i], qd).astype(F32)).astype(F16)
        xn = rmsnorm_fp16(x, self.w.lnf, c.eps)
        return qlin(xn, self.w.lmh_p, self.w.lmh_sb, c.vocab)

    def generate_greedy(self, prompt, n_new, cache: OracleKVCache):
        """Prefill the prompt then n_new greedy steps; returns (tokens, per-step logits)."""
        logits = self.forward(prompt, cache)
        out_tokens, out_logits = [], []
        tok = argmax_first(logits[-1])
        for _ in range(n_new):
            out_tokens.append(tok)
            logits = self.forward([tok], cache)
            out_logits.append(logits[-1])
            tok = argmax_first(logits[-1])
        return out_tokens, out_logits


# ---------------------------------------------------------------------------
# Synthetic model construction (shared by tests, smoke and the CPU baseline)
# ---------------------------------------------------------------------------
def make_float_weights(cfg: OracleConfig, seed: int = 0, std: float = 0.02):
    """N(0, std) fp16 weights for every linear / embedding, ln weights N(1, 0.1)."""
    rng = np.random.default_rng(seed)
    hd = cfg.head_dim
    qkv_rows = (cfg.n_head + 2 * cfg.n_kv_head) * hd

    def n(*shape, s=std):
        return (rng.standard_normal(shape, dtype=np.float32) * s).astype(F16)

    W = {
        "wte": n(cfg.vocab, cfg.d_model),
        "lm_head": n(cfg.vocab, cfg.d_model),
        "lnf": (1.0 + n(cfg.d_model, s=0.1).astype(F32)).astype(F16),
        "layers": [],
    }
    for _ in range(cfg.n_layer):
        W["layers"].append(
            {
                "ln1": (1.0 + n(cfg.d_model, s=0.1).astype(F32)).astype(F16),
                "ln2": (1.0 + n(cfg.d_model, s=0.1).astype(F32)).astype(F16),
                "c_attn": n(qkv_rows, cfg.d_model),
                "c_proj": n(cfg.d_model, cfg.n_head * hd),
                "w_gate": n(cfg.hidden, cfg.d_model),
                "w_up": n(cfg.hidden, cfg.d_model),
                "w_down": n(cfg.d_model, cfg.hidden),
            }
        )
    return W


def pack_model(cfg: OracleConfig, W, mode: str = "q4") -> OracleWeights:
    """``Transformer._ensure_quant_weights`` (transformer.py:822-1008) for an untied model:
    Q8_G64 embedding, MARLIN Q4 lm_head and layer matrices (gate|up rows stacked,
    :959-963).  mode "q4" = MSE clip search with the reference importance vectors
    (|ln_f| for lm_head, |ln_1| for c_attn, |ln_2| for gate|up, row-norm product of
    w_gate and w_up for w_down, none for c_proj; :876-948); "q4_rtn" = round to nearest;
    "q4_k_m" = "q4" with Q8_G64 w_down and lm_head (:840-847; no importance vector for
    w_down, :931-941); "q8" = every matrix Q8_G64; "q4_g128" = round to nearest with one
    (scale, bias) per 128 columns (this build's variant).  Q8_G64 packs are uint8 [N][K]."""
    if mode not in ("q4", "q4_rtn", "q4_g128", "q4_k_m", "q8"):
        raise ValueError(f"unsupported mode {mode!r}")
    mse = mode in ("q4", "q4_k_m")
    q8_down = mode in ("q4_k_m", "q8")

    def pack(w, imp, q8=False):
        if q8 or mode == "q8":
            return fm.pack_linear_q8_g64(w)
        if mode == "q4_g128":  # this build's group-128 variant (round to nearest)
            return fm.pack_linear_q4_marlin_g128(w)
        return fm.pack_linear_q4_marlin(w, clip_search=mse, col_importance=imp if mse else None)

    a = lambda v: np.abs(v.astype(F32))  # noqa: E731
    wte_p, wte_sb = fm.pack_linear_q8_g64(W["wte"])
    lmh_p, lmh_sb = pack(W["lm_head"], a(W["lnf"]), q8=mode in ("q4_k_m", "q8"))
    ow = OracleWeights(wte_p, wte_sb, lmh_p, lmh_sb, [], [], W["lnf"], [], [], [], [], [], [], [], [])
    for L in W["layers"]:
        ow.ln1.append(L["ln1"])
        ow.ln2.append(L["ln2"])
        p, s = pack(L["c_attn"], a(L["ln1"]))
        ow.c_attn_p.append(p)
        ow.c_attn_s.append(s)
        p, s = pack(L["c_proj"], None)
        ow.c_proj_p.append(p)
        ow.c_proj_s.append(s)
        p, s = pack(np.concatenate([L["w_gate"], L["w_up"]], axis=0), a(L["ln2"]))
        ow.gu_p.append(p)
        ow.gu_s.append(s)
        imp_sw = (np.linalg.norm(L["w_gate"].astype(F32), axis=1) * np.linalg.norm(L["w_up"].astype(F32), axis=1))
        p, s = pack(L["w_down"], imp_sw, q8=q8_down)
        ow.wd_p.append(p)
        ow.wd_s.append(s)
    return ow


def fp16_model(cfg: OracleConfig, W) -> OracleWeights:
    """The unquantized fp16 model the reference's fp16 runner executes: every matrix fp16
    [N][K] (gate|up rows stacked), an fp16 embedding table; scale arrays are None."""
    h = lambda a: np.ascontiguousarray(a.astype(F16))  # noqa: E731
    ow = OracleWeights(h(W["wte"]), None, h(W["lm_head"]), None, [], [], W["lnf"], [], [], [], [], [], [], [], [])
    for L in W["layers"]:
        ow.ln1.append(L["ln1"])
        ow.ln2.append(L["ln2"])
        for dst, w in ((ow.c_attn_p, L["c_attn"]), (ow.c_proj_p, L["c_proj"]),
                       (ow.gu_p, np.concatenate([L["w_gate"], L["w_up"]], axis=0)), (ow.wd_p, L["w_down"])):
            dst.append(h(w))
        for dst in (ow.c_attn_s, ow.c_proj_s, ow.gu_s, ow.wd_s):
            dst.append(None)
    return ow


def pack_model_rtn(cfg: OracleConfig, W) -> OracleWeights:
    """Round-to-nearest packing (mode "q4_rtn", untied lm_head kept in MARLIN Q4)."""
    return pack_model(cfg, W, "q4_rtn")
