"""QuantizedDecodeRunner: the MPSQuantizedDecodeRunner interface on MI355X.

Constructor arguments and methods follow the reference pybind class
(axiomlm/kernels/mps_kernels.mm:4373-4461, state at :2982-3738):

    QuantizedDecodeRunner(wte_emb, lmh_packed, lmh_sb, freqs_r, ln1_ws, c_attn_p, c_attn_s,
                          c_proj_p, c_proj_s, ln2_ws, gate_up_p, gate_up_s, w_down_p, w_down_s,
                          lnf_w, k_cs, v_cs, n_h, n_kvh, hd, use_q4, epsilon,
                          c_attn_bs=[], vocab_sz=-1, wte_p=None, wte_s=None,
                          k_scales=None, v_scales=None, kv_dtype="fp16")

Formats are detected from the packed tensors as the reference does
(mps_kernels.mm:3055-3068, 3149-3157): a 4-D pack is MARLIN Q4, a 2-D int32 one
(K/4 words per row) is Q8_G64 -- per kind of layer matrix and for the lm_head,
which covers the modes "q4", "q4_rtn", "q4_k_m" (Q8 w_down and lm_head) and "q8";
a 2-D int32 ``wte_p`` selects the Q8 embedding gather.  The
keyword arguments after ``wte_s`` are this build's additions: quantized (FP8 /
INT4) KV caches inside the captured step, and ``layout`` -- "tile16" (default)
re-tiles every MARLIN matrix once, bit-exactly, for the matrix-core GEMV;
"marlin" streams the reference layout as given.

The runner holds references to every tensor it was given (weights and the
caller's KV cache views); ``step`` returns a view of a persistent logits
buffer that is overwritten by the next call, like the reference.  ``set_mode``
selects how a step executes: "graph" (the default: the per-op kernels replayed
as one captured hipGraph), "eager" (the same kernels launched one by one) or
"persistent" (one cooperative launch per token, when the configuration allows it).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kernels.ops import KV_CODES


def _arr(ptrs):
    a = (ctypes.c_void_p * len(ptrs))()
    for i, p in enumerate(ptrs):
        a[i] = p
    return a


def _p(t):
    return None if t is None or (isinstance(t, torch.Tensor) and t.numel() == 0) else t.data_ptr()


def _packed_k(p) -> int:
    """Input width of a packed matrix: MARLIN Q4 int32 [N/8][K/64][32][2], or Q8_G64 codes as
    int32 [N][K/4] (the reference packer's view) or uint8 [N][K]."""
    if p.dim() == 4:
        return int(p.shape[1]) * 64
    if p.dim() == 2:
        return int(p.shape[1]) * (4 if p.element_size() == 4 else 1)
    raise RuntimeError(f"QuantizedDecodeRunner: unsupported packed weight of shape {tuple(p.shape)}")


def _matrix_format(p, K: int, name: str) -> int:
    """0 for MARLIN Q4, 1 for Q8_G64 (the shape test of mps_kernels.mm:3055-3068), 2 for an
    fp16 [N][K] matrix (the fp16 runner's weights)."""
    if p.dim() == 2 and p.dtype == torch.float16 and int(p.shape[1]) == K:
        return 2
    if p.dim() == 4 and _packed_k(p) == K:
        return 0
    if p.dim() == 2 and p.dtype != torch.float16 and _packed_k(p) == K:
        return 1
    raise RuntimeError(f"QuantizedDecodeRunner: the {name} pack of shape {tuple(p.shape)} is neither MARLIN Q4 nor "
                       f"Q8_G64 for K={K} (the legacy Q4_G64 layout of mode 'q4_legacy' is not on this runner)")


class QuantizedDecodeRunner:
    def __init__(self, wte_emb, lmh_packed, lmh_sb, freqs_r, ln1_ws, c_attn_p, c_attn_s, c_proj_p, c_proj_s,
                 ln2_ws, gate_up_p, gate_up_s, w_down_p, w_down_s, lnf_w, k_cs, v_cs, n_h, n_kvh, hd, use_q4,
                 epsilon, c_attn_bs=(), vocab_sz=-1, wte_p=None, wte_s=None, k_scales=None, v_scales=None,
                 kv_dtype="fp16", max_tokens: int = 32, layout: str = "tile16"):
        L = len(ln1_ws)
        dev = lmh_packed.device
        _lib.require_gpu(lmh_packed, "QuantizedDecodeRunner")
        h16 = lambda t: t.to(device=dev, dtype=torch.float16).contiguous()  # noqa: E731
        self._keep = []  # tensors whose storage the native runner points to

        def keep(t):
            if t is not None:
                self._keep.append(t)
            return t

        ln1 = [keep(h16(w)) for w in ln1_ws]
        ln2 = [keep(h16(w)) for w in ln2_ws]
        lnf = keep(h16(lnf_w))
        freqs = keep(freqs_r.to(device=dev, dtype=torch.float32).contiguous())
        mats = [c_attn_p, c_attn_s, c_proj_p, c_proj_s, gate_up_p, gate_up_s, w_down_p, w_down_s]
        mats = [[keep(t.contiguous()) if t is not None else None for t in m] for m in mats]
        biases = [keep(h16(b)) if (b is not None and b.numel() > 0) else None for b in (c_attn_bs or [])]
        biases = biases + [None] * (L - len(biases))

        if wte_p is not None and wte_p.numel() > 0 and wte_p.dim() == 2:
            wte_fmt, wte, wte_sb = 1, keep(wte_p.contiguous()), keep(wte_s.contiguous())
        elif wte_emb is not None and wte_emb.dtype == torch.int32 and wte_emb.dim() == 2:
            wte_fmt, wte, wte_sb = 1, keep(wte_emb.contiguous()), keep(lmh_sb.contiguous())
        else:
            wte_fmt, wte, wte_sb = 0, keep(h16(wte_emb)), None
        lmh_fmt = 0 if lmh_packed.dim() == 4 else (2 if lmh_packed.dtype == torch.float16 else 1)
        lmh = keep(lmh_packed.contiguous())
        lmh_s = keep(lmh_sb.contiguous()) if lmh_sb is not None else None
        if vocab_sz is None or vocab_sz <= 0:
            vocab_sz = wte.shape[0] if lmh_fmt == 0 else lmh_packed.shape[0]
        self.vocab_size = int(vocab_sz)
        self.d_model = int(n_h * hd)
        # MLP width from the gate|up rows (MARLIN packs hold N/8 tiles of 8 rows; Q8_G64 one
        # row per output); w_down's packed input width is checked against it below
        gu0 = gate_up_p[0]
        self.hidden_dim = int(gu0.shape[0]) * (8 if gu0.dim() == 4 else 1) // 2
        kv_code = KV_CODES[kv_dtype]
        self.kv_dtype = kv_dtype
        self.max_seq_len = int(k_cs[0].shape[-2])
        self.rope_len = int(freqs.shape[0])

        def first_batch(t):
            return keep(t[0] if t.dim() == 4 else t)

        kcs = [first_batch(t) for t in k_cs]
        vcs = [first_batch(t) for t in v_cs]
        kss = [first_batch(t) for t in k_scales] if kv_code else [None] * L
        vss = [first_batch(t) for t in v_scales] if kv_code else [None] * L

        self._arrays = [
            _arr([_p(t) for t in ln1]), _arr([_p(t) for t in ln2]),
            *[_arr([_p(t) for t in m]) for m in mats],
            _arr([_p(b) for b in biases]),
            _arr([_p(t) for t in kcs]), _arr([_p(t) for t in vcs]),
            _arr([_p(t) for t in kss]), _arr([_p(t) for t in vss]),
        ]
        a = self._arrays
        d = _lib.RunnerDesc()
        d.n_layer, d.n_head, d.n_kv_head, d.head_dim = L, int(n_h), int(n_kvh), int(hd)
        d.d_model, d.hidden_dim, d.vocab_size = self.d_model, self.hidden_dim, self.vocab_size
        d.max_seq_len, d.rope_len = self.max_seq_len, int(freqs.shape[0])
        d.eps, d.kv_dtype = float(epsilon), kv_code
        d.wte_format, d.wte, d.wte_sb = wte_fmt, _p(wte), _p(wte_sb)
        d.lm_head_format, d.lm_head_w, d.lm_head_sb = lmh_fmt, _p(lmh), _p(lmh_s)
        d.freqs, d.lnf_w = _p(freqs), _p(lnf)
        cv = ctypes.cast
        P = ctypes.POINTER(ctypes.c_void_p)
        d.ln1_w, d.ln2_w = cv(a[0], P), cv(a[1], P)
        d.qkv_w, d.qkv_sb, d.o_w, d.o_sb = cv(a[2], P), cv(a[3], P), cv(a[4], P), cv(a[5], P)
        d.gu_w, d.gu_sb, d.down_w, d.down_sb = cv(a[6], P), cv(a[7], P), cv(a[8], P), cv(a[9], P)
        d.qkv_bias = cv(a[10], P)
        d.k_cache, d.v_cache = cv(a[11], P), cv(a[12], P)
        d.k_scales, d.v_scales = (cv(a[13], P), cv(a[14], P)) if kv_code else (None, None)
        d.max_tokens = int(max_tokens)
        # group 64 (reference) or 128, from the packed scales; one size for every Q4 matrix
        from .kernels.quant import marlin_group_size

        # per kind of layer matrix: MARLIN Q4 (4-D pack) or Q8_G64 (2-D), as the reference runner
        # dispatches on the packed shape (mps_kernels.mm:3055-3068); one format per kind
        fmts = []
        for name, ps, K in (("c_attn", c_attn_p, self.d_model), ("c_proj", c_proj_p, self.d_model),
                            ("gate_up", gate_up_p, self.d_model), ("w_down", w_down_p, self.hidden_dim)):
            kinds = {_matrix_format(p, K, name) for p in ps}
            if len(kinds) != 1:
                raise RuntimeError(f"QuantizedDecodeRunner: {name} packs mix MARLIN Q4 and Q8_G64 layers")
            fmts.append(kinds.pop())
        d.qkv_format, d.o_format, d.gu_format, d.down_format = fmts
        self.layer_formats = tuple(("q4_marlin", "q8_g64", "fp16")[f] for f in fmts)
        packs, scales = [], []
        for f, ps, ss in zip(fmts, (c_attn_p, c_proj_p, gate_up_p, w_down_p), (c_attn_s, c_proj_s, gate_up_s, w_down_s)):
            if f == 0:
                packs += list(ps)
                scales += list(ss)
        groups = {marlin_group_size(p, s) for p, s in zip(packs, scales)}
        if lmh_fmt == 0:
            groups.add(marlin_group_size(lmh_packed, lmh_sb))
        if len(groups) > 1:
            raise RuntimeError(f"QuantizedDecodeRunner: mixed MARLIN group sizes {sorted(groups)}")
        self.group_size = groups.pop() if groups else 64
        d.group_size = self.group_size
        if layout not in ("tile16", "marlin"):
            raise ValueError(f"layout must be 'tile16' or 'marlin', got {layout!r}")
        d.layout = 0 if layout == "tile16" else 1
        self._desc = d
        h = ctypes.c_void_p()
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().axm_runner_create(ctypes.byref(d), ctypes.byref(h)), "QuantizedDecodeRunner")
        self._h = h
        self.device = dev
        self._logits = None
        self._norm = None

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                torch.cuda.synchronize(self.device)
            except Exception:
                pass
            try:
                _lib.lib().axm_runner_destroy(h)
            except Exception:  # interpreter shutdown: the library object may already be gone
                pass
            self._h = None

    MODES = {"graph": 0, "eager": 1, "persistent": 2}

    def set_graph(self, enable: bool) -> None:
        """True: replay the per-op kernels as a captured hipGraph; False: launch them eagerly."""
        _lib.check(_lib.lib().axm_runner_set_graph(self._h, int(bool(enable))), "set_graph")

    def set_mode(self, mode: str) -> None:
        """"graph" (default) or "eager" (five kernels per layer), or "persistent" (one cooperative
        launch per token)."""
        if mode not in self.MODES:
            raise ValueError(f"mode must be one of {sorted(self.MODES)}, got {mode!r}")
        _lib.check(_lib.lib().axm_runner_set_mode(self._h, self.MODES[mode]), "set_mode")

    @property
    def mode(self) -> str:
        m = _lib.lib().axm_runner_get_mode(self._h)
        return {v: k for k, v in self.MODES.items()}[m]

    def check(self) -> None:
        """Synchronize and raise if a persistent step gave up waiting for another workgroup."""
        _lib.check(_lib.lib().axm_runner_check(self._h), "QuantizedDecodeRunner.check")

    def step(self, idx, start_pos: int, write_pos: int, active_len: int) -> torch.Tensor:
        """One decode token -> logits (1, 1, V) (mps_kernels.mm:3195-3263)."""
        out = ctypes.c_void_p()
        if isinstance(idx, torch.Tensor) and idx.device.type == "cuda":
            t = idx.reshape(-1)[:1].to(torch.int64)
            rc = _lib.lib().axm_runner_step(self._h, _lib.ptr(t), 0, int(start_pos), int(write_pos),
                                            int(active_len), _lib.stream_of(self.device), ctypes.byref(out))
        else:
            tok = int(idx.reshape(-1)[0]) if isinstance(idx, torch.Tensor) else int(idx)
            rc = _lib.lib().axm_runner_step(self._h, None, tok, int(start_pos), int(write_pos), int(active_len),
                                            _lib.stream_of(self.device), ctypes.byref(out))
        _lib.check(rc, "QuantizedDecodeRunner.step")
        if self._logits is None:
            self._logits = _RawBuffer.view(out.value, self.vocab_size, self.device).view(1, 1, self.vocab_size)
        return self._logits

    def step_greedy(self, start_pos: int, write_pos: int, active_len: int) -> torch.Tensor:
        """Decode the greedy argmax of the previous step's logits without a host round trip
        (the device loop of mps_kernels.mm:3466-3527).  Returns the logits view."""
        out = ctypes.c_void_p()
        rc = _lib.lib().axm_runner_step(self._h, None, -1, int(start_pos), int(write_pos), int(active_len),
                                        _lib.stream_of(self.device), ctypes.byref(out))
        _lib.check(rc, "QuantizedDecodeRunner.step_greedy")
        if self._logits is None:
            self._logits = _RawBuffer.view(out.value, self.vocab_size, self.device).view(1, 1, self.vocab_size)
        return self._logits

    def _tokens(self, idx) -> torch.Tensor:
        t = idx if isinstance(idx, torch.Tensor) else torch.tensor(idx)
        return t.reshape(-1).to(device=self.device, dtype=torch.int64).contiguous()

    def verify_step(self, idx, start_pos: int, write_pos: int, active_len: int) -> torch.Tensor:
        """T tokens in one pass -> logits (1, T, V) (mps_kernels.mm:3359-3464); T == 1 is a step."""
        t = self._tokens(idx)
        T = int(t.numel())
        if T == 1:
            return self.step(t, start_pos, write_pos, active_len)
        out = ctypes.c_void_p()
        rc = _lib.lib().axm_runner_verify_step(self._h, _lib.ptr(t), T, int(start_pos), int(write_pos),
                                               int(active_len), _lib.stream_of(self.device), ctypes.byref(out))
        _lib.check(rc, "QuantizedDecodeRunner.verify_step")
        self._keep_tokens = t
        return _RawBuffer.view(out.value, T * self.vocab_size, self.device).view(1, T, self.vocab_size)

    def verify_tree_step(self, idx, start_pos: int, write_pos: int, prefix_len: int, depths, masks) -> torch.Tensor:
        """Tree verification -> logits (1, T, V) (mps_kernels.mm:3265-3357).  ``masks[u]`` has bit j set
        when tree node j is visible to node u (Python ints, up to 64 nodes)."""
        t = self._tokens(idx)
        T = int(t.numel())
        if len(depths) != T or len(masks) != T:
            raise RuntimeError("tree_depths and tree_mask must match T")
        d = (ctypes.c_int * T)(*[int(v) for v in depths])
        m = (ctypes.c_uint64 * T)(*[int(v) & 0xFFFFFFFFFFFFFFFF for v in masks])
        out = ctypes.c_void_p()
        rc = _lib.lib().axm_runner_verify_tree_step(self._h, _lib.ptr(t), T, int(start_pos), int(write_pos),
                                                    int(prefix_len), d, m, _lib.stream_of(self.device),
                                                    ctypes.byref(out))
        _lib.check(rc, "QuantizedDecodeRunner.verify_tree_step")
        self._keep_tokens = t
        return _RawBuffer.view(out.value, T * self.vocab_size, self.device).view(1, T, self.vocab_size)

    def speculative_decode(self, initial_tokens, max_new_tokens: int, ngram_size: int, max_spec_tokens: int,
                           start_pos: int):
        """Native prompt-lookup speculative decoding (mps_kernels.mm:3639-3730).  Returns
        (tokens, seen, model_forward_calls, drafted, accepted, seconds) like the reference."""
        init = [int(t) for t in initial_tokens]
        n = len(init)
        cap = n + int(max_new_tokens)
        a = (ctypes.c_int64 * n)(*init)
        out = (ctypes.c_int64 * cap)()
        stats = (ctypes.c_int64 * 6)()
        rc = _lib.lib().axm_runner_speculative_decode(self._h, a, n, int(max_new_tokens), int(ngram_size),
                                                      int(max_spec_tokens), int(start_pos), out, cap, stats,
                                                      _lib.stream_of(self.device))
        _lib.check(rc, "QuantizedDecodeRunner.speculative_decode")
        secs = ctypes.cast(ctypes.byref(stats, 5 * 8), ctypes.POINTER(ctypes.c_double))[0]
        return list(out[:stats[0]]), int(stats[1]), int(stats[2]), int(stats[3]), int(stats[4]), float(secs)

    def last_token(self) -> torch.Tensor:
        """int64 device view of the token id consumed by the latest step."""
        p = ctypes.c_void_p()
        _lib.check(_lib.lib().axm_runner_token_slot(self._h, ctypes.byref(p)), "last_token")
        return _RawBuffer.view(p.value, 4, self.device).view(torch.int64)

    KERNEL_GROUPS = ("qkv", "attention", "o", "gate_up", "down", "lm_head")

    def time_kernels(self, position: int, active_len: int, reps: int = 200) -> dict:
        """Average microseconds per launch of each of the one-token step's launch groups
        (KERNEL_GROUPS), each run `reps` times back to back over the layers in turn as one
        captured graph and timed with HIP events on the runner's stream.  A measurement call with no
        counterpart in the reference: it overwrites the runner's activations and the
        cache slot at `position`, which the next step recomputes."""
        out = (ctypes.c_float * 6)()
        rc = _lib.lib().axm_runner_time_kernels(self._h, int(position), int(active_len), int(reps),
                                                _lib.stream_of(self.device), out)
        _lib.check(rc, "QuantizedDecodeRunner.time_kernels")
        return {k: float(out[i]) for i, k in enumerate(self.KERNEL_GROUPS)}

    def persistent_words(self) -> torch.Tensor | None:
        """Copy of the persistent step's cross-workgroup words as int64 (payload in the low
        32 bits, phase tag in the high 32), or None when the mode is unavailable; a
        diagnostic view of the last layer's intermediate vectors."""
        p = ctypes.c_void_p()
        n = ctypes.c_int64()
        _lib.check(_lib.lib().axm_runner_persistent_words(self._h, ctypes.byref(p), ctypes.byref(n)),
                   "persistent_words")
        if n.value == 0:
            return None
        torch.cuda.synchronize(self.device)
        raw = _RawBuffer.view(p.value, 4 * n.value, self.device)
        return raw.view(torch.int64).clone()

    def get_last_norm(self, T: int = 1) -> torch.Tensor:
        """Clone of the final normalized hidden state (mps_kernels.mm:3732-3737)."""
        p = ctypes.c_void_p()
        _lib.check(_lib.lib().axm_runner_last_norm(self._h, ctypes.byref(p)), "get_last_norm")
        return _RawBuffer.view(p.value, T * self.d_model, self.device).view(1, T, self.d_model).clone()


class _RawBuffer:
    """fp16 torch view of device memory owned by the native runner."""

    @staticmethod
    def view(ptr_value: int, numel: int, device) -> torch.Tensor:
        class _Cai:
            __cuda_array_interface__ = {
                "shape": (numel,),
                "typestr": "<f2",
                "data": (ptr_value, False),
                "version": 3,
                "strides": None,
            }

        return torch.as_tensor(_Cai(), device=device)


class DecodeRunner(QuantizedDecodeRunner):
    """The reference's fp16 decode runner ``MPSDecodeRunner`` (mps_kernels.mm:2304-2980, binding
    :4328-4373) on MI355X:

        DecodeRunner(wte_w, freqs_r, ln1_ws, c_attn_ws, c_proj_ws, ln2_ws, gate_up_ws, w_down_ws,
                     lnf_w, k_cs, v_cs, n_h, n_kvh, hd, epsilon, lm_head_w=None, c_attn_bs=[])

    fp16 [N][K] weights (gate_up rows [W_gate; W_up]); the lm_head defaults to the embedding
    table (tied), and the vocabulary is its row count.  The same native runner as the
    quantized class with every matrix in the fp16 format (an HBM-bound fp16 GEMV), so the
    methods are the same: step, verify_step, verify_tree_step, speculative_decode,
    get_last_norm.  Keyword arguments after c_attn_bs are this build's (max_tokens, kv_dtype
    and layout of the quantized class)."""

    def __init__(self, wte_w, freqs_r, ln1_ws, c_attn_ws, c_proj_ws, ln2_ws, gate_up_ws, w_down_ws, lnf_w, k_cs,
                 v_cs, n_h, n_kvh, hd, epsilon, lm_head_w=None, c_attn_bs=(), **kw):
        L = len(ln1_ws)
        lm = wte_w if lm_head_w is None or lm_head_w.numel() == 0 else lm_head_w
        h16 = lambda ts: [t.to(torch.float16).contiguous() for t in ts]  # noqa: E731
        none = [None] * L
        super().__init__(wte_w.to(torch.float16), lm.to(torch.float16).contiguous(), None, freqs_r, ln1_ws,
                         h16(c_attn_ws), none, h16(c_proj_ws), none, ln2_ws, h16(gate_up_ws), none, h16(w_down_ws),
                         none, lnf_w, k_cs, v_cs, n_h, n_kvh, hd, False, epsilon, c_attn_bs, int(lm.shape[0]), **kw)
