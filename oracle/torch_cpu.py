"""torch-CPU restatement of the reference's CPU decode path (TEST INFRASTRUCTURE and
the CPU baseline of bench.py).

A half-precision AxiomLM model quantized with mode "q4" runs these torch
operations per call on a CPU, and so does this module:
  * ``_forward_quantized_sequence`` (axiomlm/models/transformer.py:1036-1200):
    Q8_G64 embedding rows (quant.py:132-163), RMSNorm in fp16
    (modules.py:41-43), fused QKV linear, RoPE as a complex product in fp32
    rounded to fp16 (ops.py:858-866), the fp16 ``StaticKVCache`` write
    (paged_cache.py:218-287), ``F.scaled_dot_product_attention`` (causal for a
    prompt, an explicit mask for a continuation), residual adds in fp16, SwiGLU
    as ``F.silu(g) * u``, the final norm and the lm_head;
  * every quantized linear layer is the CPU fallback of ``qmv_q4_marlin``
    (quant.py:637-661): the MARLIN codes are dequantized to fp16 on every call
    (quant.py:597-634), then ``F.linear`` in fp16.

The reference's own code cannot travel to the GPU box, so bench.py times this
restatement on the box's host cores.  tests/test_oracle_torch_cpu.py checks it
against the golden logits written from the reference (C1 decode and prefill)
and against the numpy oracle.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _lane_maps():
    lanes = torch.arange(32)
    r = ((lanes & 16) >> 2) | ((lanes & 6) >> 1)
    c0 = ((lanes & 8) >> 1) | ((lanes & 1) << 1)
    return r, c0


def dequantize_q4_marlin(w_marlin: torch.Tensor, sb_marlin: torch.Tensor, K: int, out_features: int | None = None):
    """MARLIN codes -> fp16 (N, K) = fp16(q * scale + bias) in fp32 (quant.py:597-634): every nibble
    is shifted out of its int32 word, scattered to (row, column) and scaled in fp32."""
    nt, KG = w_marlin.shape[0], w_marlin.shape[1]
    r, c0 = _lane_maps()
    w = w_marlin.unsqueeze(-1)
    lo = ((w >> torch.tensor([0, 4, 8, 12], dtype=torch.int32)) & 0xF).float()
    hi = ((w >> torch.tensor([16, 20, 24, 28], dtype=torch.int32)) & 0xF).float()
    q = torch.empty((nt, KG, 8, 8, 2, 4), dtype=torch.float32)  # (tile, group, row c, r, word, s)
    q[:, :, c0, r] = lo
    q[:, :, c0 + 1, r] = hi
    q = q.permute(0, 2, 1, 4, 5, 3).reshape(nt * 8, KG, 64)
    sb = sb_marlin.permute(0, 2, 1, 3).reshape(nt * 8, KG, 2).float()
    w16 = (q * sb[..., 0:1] + sb[..., 1:2]).reshape(nt * 8, K).to(torch.float16)
    return w16[:out_features] if out_features is not None and out_features < w16.shape[0] else w16


def dequantize_q8_g64(w_packed: torch.Tensor, sb: torch.Tensor, K: int) -> torch.Tensor:
    """Q8_G64 int32 [N, K/4] little-endian bytes -> fp16 (quant.py:115-129)."""
    N = w_packed.shape[0]
    b = (w_packed.unsqueeze(-1) >> torch.tensor([0, 8, 16, 24], dtype=torch.int32)) & 0xFF
    q = b.reshape(N, K // 64, 64).float()
    return (q * sb[..., 0:1].float() + sb[..., 1:2].float()).reshape(N, K).to(torch.float16)


def qlin(x: torch.Tensor, wp: torch.Tensor, wsb: torch.Tensor, out_features: int) -> torch.Tensor:
    """Transformer._qlin on the CPU: dequantize every call, then F.linear in fp16."""
    K = x.shape[-1]
    if wp.dim() == 4:
        w = dequantize_q4_marlin(wp, wsb, K, out_features)
    else:
        w = dequantize_q8_g64(wp, wsb, K)
    return F.linear(x, w)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward (modules.py:41-43) on fp16 tensors."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """Complex rotation of interleaved pairs in fp32, result in x's dtype (ops.py:858-866);
    x (B, H, T, hd), freqs complex (T, hd / 2)."""
    B, H, T, hd = x.shape
    xc = torch.view_as_complex(x.float().reshape(B, H, T, -1, 2))
    return torch.view_as_real(xc * freqs.view(1, 1, T, -1)).reshape(B, H, T, hd).to(x.dtype)


class TorchCpuModel:
    """The quantized decoder of one OracleWeights set (numpy packs) as torch CPU tensors."""

    def __init__(self, cfg, ow, cos, sin):
        t = lambda a: torch.from_numpy(a.copy())  # noqa: E731
        self.cfg = cfg
        self.wte_p = t(ow.wte_p.view("<i4").reshape(ow.wte_p.shape[0], -1))
        self.wte_sb = t(ow.wte_sb)
        self.lmh_p = t(ow.lmh_p.view("<i4").reshape(ow.lmh_p.shape[0], -1) if ow.lmh_p.ndim == 2 else ow.lmh_p)
        self.lmh_sb = t(ow.lmh_sb)
        self.lnf = t(ow.lnf)
        self.layers = []
        for i in range(cfg.n_layer):
            self.layers.append({
                "ln1": t(ow.ln1[i]), "ln2": t(ow.ln2[i]), "qkv_p": t(ow.c_attn_p[i]), "qkv_s": t(ow.c_attn_s[i]),
                "o_p": t(ow.c_proj_p[i]), "o_s": t(ow.c_proj_s[i]), "gu_p": t(ow.gu_p[i]), "gu_s": t(ow.gu_s[i]),
                "dn_p": t(ow.wd_p[i]), "dn_s": t(ow.wd_s[i])})
        # freqs_cis of precompute_rope_frequencies as a complex table (cos + i sin)
        self.freqs = torch.complex(torch.from_numpy(cos), torch.from_numpy(sin))

    @classmethod
    def from_tensors(cls, cfg, layers, lnf, lmh_p, lmh_sb, wte_p, wte_sb, cos, sin):
        """From torch tensors (any device): layers = list of dicts with ln1, ln2, qkv_p, qkv_s,
        o_p, o_s, gu_p, gu_s, dn_p, dn_s; Q8 tables as int32 [N, K/4]."""
        m = cls.__new__(cls)
        c = lambda t: t.detach().to("cpu").contiguous()  # noqa: E731
        m.cfg = cfg
        m.wte_p, m.wte_sb, m.lmh_p, m.lmh_sb, m.lnf = c(wte_p), c(wte_sb), c(lmh_p), c(lmh_sb), c(lnf)
        m.layers = [{k: c(v) for k, v in Ly.items()} for Ly in layers]
        m.freqs = torch.complex(torch.as_tensor(cos), torch.as_tensor(sin))
        return m

    def new_cache(self, max_seq_len: int):
        c = self.cfg
        k = torch.zeros((c.n_layer, 1, c.n_kv_head, max_seq_len, c.head_dim), dtype=torch.float16)
        return {"k": k, "v": torch.zeros_like(k), "seen": 0}

    def layer(self, i: int, x: torch.Tensor, cache, start: int) -> torch.Tensor:
        """One decoder layer on x (1, T, d) fp16 with the cache holding `start` tokens."""
        c, Ly = self.cfg, self.layers[i]
        T = x.shape[1]
        hd = c.head_dim
        qd, kvd = c.n_head * hd, c.n_kv_head * hd
        h1 = rmsnorm(x, Ly["ln1"], c.eps)
        qkv = qlin(h1, Ly["qkv_p"], Ly["qkv_s"], qd + 2 * kvd)
        q = qkv[:, :, :qd].view(1, T, c.n_head, hd).transpose(1, 2)
        k = qkv[:, :, qd:qd + kvd].view(1, T, c.n_kv_head, hd).transpose(1, 2)
        v = qkv[:, :, qd + kvd:].view(1, T, c.n_kv_head, hd).transpose(1, 2)
        fr = self.freqs[start:start + T]
        q, k = rope(q, fr), rope(k, fr)
        cache["k"][i, :, :, start:start + T] = k
        cache["v"][i, :, :, start:start + T] = v
        kk, vv = cache["k"][i, :, :, :start + T], cache["v"][i, :, :, :start + T]
        n_rep = c.n_head // c.n_kv_head
        if n_rep > 1:
            kk = kk[:, :, None].expand(1, c.n_kv_head, n_rep, start + T, hd).reshape(1, c.n_head, start + T, hd)
            vv = vv[:, :, None].expand(1, c.n_kv_head, n_rep, start + T, hd).reshape(1, c.n_head, start + T, hd)
        mask, causal = None, False
        if T > 1 and start > 0:
            mask = torch.arange(start + T)[None, :] <= (start + torch.arange(T))[:, None]
        else:
            causal = T > 1
        y = F.scaled_dot_product_attention(q, kk, vv, attn_mask=mask, is_causal=causal)
        y = y.transpose(1, 2).reshape(1, T, qd)
        x = x + qlin(y, Ly["o_p"], Ly["o_s"], qd)
        h2 = rmsnorm(x, Ly["ln2"], c.eps)
        gu = qlin(h2, Ly["gu_p"], Ly["gu_s"], 2 * c.hidden)
        g, u = gu.chunk(2, dim=-1)
        return x + qlin(F.silu(g) * u, Ly["dn_p"], Ly["dn_s"], qd)

    def forward(self, idx, cache, all_logits: bool = False) -> torch.Tensor:
        """Logits (T, V) (all_logits) or (1, V) of the last token; advances the cache."""
        c = self.cfg
        ids = torch.as_tensor(idx, dtype=torch.int64).reshape(-1)
        T = ids.numel()
        x = dequantize_q8_g64(self.wte_p[ids], self.wte_sb[ids], c.d_model).view(1, T, c.d_model)
        start = cache["seen"]
        for i in range(c.n_layer):
            x = self.layer(i, x, cache, start)
        cache["seen"] = start + T
        xt = x if all_logits else x[:, -1:]
        return qlin(rmsnorm(xt, self.lnf, c.eps), self.lmh_p, self.lmh_sb, c.vocab)[0]
