"""StaticKVCache for the MI355X decode path (axiomlm/engine/paged_cache.py:122-462).

Same constructor, tensor layout and counters as the reference:
  cache  (L, 2, B, Hkv, S, hd)      fp16, or uint8 (FP8 E4M3FN) / uint8 hd/2 (INT4)
  scales (L, 2, B, Hkv, S, hd/64)   fp16 for the quantized caches
``k_caches[i]`` / ``v_caches[i]`` are views of ``cache[i, 0]`` / ``cache[i, 1]``.
Writes of new rows (``update``) quantize on the GPU with the reference CPU
quantizer semantics; ``compact_tree_path`` moves accepted tree slots of every
layer with one HIP kernel per call.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kernels.ops import KV_CODES, compact_tree_kv, dequantize_kv_fp8, dequantize_kv_int4


class StaticKVCache:
    def __init__(
        self,
        max_batch_size: int,
        max_seq_len: int,
        n_layer: int,
        n_kv_head: int,
        head_dim: int,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str | None = None,
        ring_buffer: bool = False,
        cache_dtype: str = "fp16",
    ):
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        elif isinstance(device, str):
            device = torch.device(device)
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        self.n_layer = n_layer
        self.n_kv_head = n_kv_head
        self.head_dim = head_dim
        self.ring_buffer = ring_buffer
        self.cache_dtype = cache_dtype.lower()
        if self.cache_dtype not in KV_CODES:
            raise ValueError(f"unsupported cache_dtype {cache_dtype!r}")
        self.num_groups = max(1, head_dim // 64)
        shape5 = (n_layer, 2, max_batch_size, n_kv_head, max_seq_len)
        if self.cache_dtype == "fp8":
            self.cache = torch.zeros((*shape5, head_dim), dtype=torch.uint8, device=device)
        elif self.cache_dtype == "int4":
            self.cache = torch.zeros((*shape5, head_dim // 2), dtype=torch.uint8, device=device)
        else:
            self.cache = torch.empty((*shape5, head_dim), dtype=dtype, device=device)
        if self.cache_dtype == "fp16":
            self.scales = None
            self.k_scales = None
            self.v_scales = None
        else:
            self.scales = torch.zeros((*shape5, self.num_groups), dtype=torch.float16, device=device)
            self.k_scales = [self.scales[i, 0] for i in range(n_layer)]
            self.v_scales = [self.scales[i, 1] for i in range(n_layer)]
        self.k_caches = [self.cache[i, 0] for i in range(n_layer)]
        self.v_caches = [self.cache[i, 1] for i in range(n_layer)]
        self.layer_seq_lens = [0] * n_layer
        self.total_seen_tokens = [0] * n_layer

    @property
    def kv_code(self) -> int:
        return KV_CODES[self.cache_dtype]

    def get_memory_bytes(self) -> int:
        total = self.cache.numel() * self.cache.element_size()
        if self.scales is not None:
            total += self.scales.numel() * self.scales.element_size()
        return total

    @property
    def seq_len(self) -> int:
        return self.total_seen_tokens[0]

    def reset(self):
        for i in range(self.n_layer):
            self.layer_seq_lens[i] = 0
            self.total_seen_tokens[i] = 0

    # ---- writes ---------------------------------------------------------------
    def _write_rows(self, layer: int, k: torch.Tensor, v: torch.Tensor, write_pos: int) -> None:
        """Store k, v (1, Hkv, T, hd) at slots (write_pos + t) % S of batch 0."""
        T = k.shape[2]
        hd = self.head_dim
        kr = k[0].transpose(0, 1).reshape(T, self.n_kv_head * hd).to(torch.float16).contiguous()
        vr = v[0].transpose(0, 1).reshape(T, self.n_kv_head * hd).to(torch.float16).contiguous()
        ks = self.k_scales[layer] if self.scales is not None else None
        vs = self.v_scales[layer] if self.scales is not None else None
        _lib.check(
            _lib.lib().axm_kv_cache_write(
                _lib.ptr(kr), _lib.ptr(vr), self.n_kv_head * hd, T, _lib.ptr(self.k_caches[layer]),
                _lib.ptr(self.v_caches[layer]), _lib.ptr(ks), _lib.ptr(vs), self.kv_code, self.n_kv_head, hd,
                self.max_seq_len, int(write_pos) % self.max_seq_len, _lib.stream_of(self.cache.device)),
            "StaticKVCache.update",
        )

    def _active_views(self, layer: int, n: int):
        kb, vb = self.k_caches[layer][:1, :, :n], self.v_caches[layer][:1, :, :n]
        if self.cache_dtype == "fp8":
            return (dequantize_kv_fp8(kb, self.k_scales[layer][:1, :, :n], self.head_dim),
                    dequantize_kv_fp8(vb, self.v_scales[layer][:1, :, :n], self.head_dim))
        if self.cache_dtype == "int4":
            return (dequantize_kv_int4(kb, self.k_scales[layer][:1, :, :n], self.head_dim),
                    dequantize_kv_int4(vb, self.v_scales[layer][:1, :, :n], self.head_dim))
        return kb, vb

    def update(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        """In-place write of (1, Hkv, T, hd) rows; returns the active (dequantized) views.

        Monotonic and ring-buffer semantics of paged_cache.py:218-361 (batch 1)."""
        if k.shape[0] != 1:
            raise ValueError("the MI355X StaticKVCache path supports batch 1 writes")
        T = k.shape[2]
        seen = self.total_seen_tokens[layer_idx]
        S = self.max_seq_len
        if not self.ring_buffer and seen + T <= S:
            self._write_rows(layer_idx, k, v, seen)
            self.layer_seq_lens[layer_idx] = self.total_seen_tokens[layer_idx] = seen + T
            return self._active_views(layer_idx, seen + T)
        if T >= S:
            self._write_rows(layer_idx, k[:, :, -S:], v[:, :, -S:], 0)
        else:
            self._write_rows(layer_idx, k, v, seen % S)
        active = min(seen + T, S)
        self.layer_seq_lens[layer_idx] = active
        self.total_seen_tokens[layer_idx] = seen + T
        return self._active_views(layer_idx, active)

    def get_quantized_views(self, layer_idx: int):
        k_s = self.k_scales[layer_idx] if self.scales is not None else None
        v_s = self.v_scales[layer_idx] if self.scales is not None else None
        return self.k_caches[layer_idx], self.v_caches[layer_idx], k_s, v_s

    def compact_tree_path(self, write_pos: int, accepted_indices: list[int], new_total_seen: int | None = None):
        """Move accepted tree slots (write_pos + a[m]) % S to (write_pos + m) % S in every layer
        with one race-free HIP pass (paged_cache.py:376-462)."""
        if self.scales is not None and not self.scales.is_contiguous():
            raise RuntimeError("compact_tree_path: cache and scales must be contiguous")
        compact_tree_kv(self.cache, self.scales, write_pos, accepted_indices)
        if new_total_seen is not None:
            active = min(new_total_seen, self.max_seq_len)
            self.total_seen_tokens[:] = [new_total_seen] * self.n_layer
            self.layer_seq_lens[:] = [active] * self.n_layer
