"""The module object on the GPU: every function gives bit-identical results to the
direct operator it adapts (argument order of the reference's module, the torch
custom-operator dispatch in between)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mod():
    from axiomlm_amd.rocm_module import load_rocm_module

    m = load_rocm_module()
    assert m is not None
    return m


def _same(a, b):
    return torch.equal(a.view(torch.uint8) if a.dtype != torch.int64 else a,
                       b.view(torch.uint8) if b.dtype != torch.int64 else b)


def test_module_linear_layers(dev, mod):
    import axiomlm_amd.kernels as K

    print("[module_linear]", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(3, 256, generator=g, device=dev).half()
    w = (torch.randn(100, 256, generator=g, device=dev) * 0.02).half()
    p, s = K.pack_linear_q4_marlin(w, clip_search=False)
    b = torch.randn(100, generator=g, device=dev).half()
    assert _same(mod.qmv_q4_marlin_mps(x, p, s, 100, b), K.qmv_q4_marlin(x, p, s, 100, b))
    assert _same(mod.qmm_q4_marlin_mps(x, p, s), K.qmm_q4_marlin(x, p, s))
    p8, s8 = K.pack_linear_q8_g64(w)
    assert _same(mod.qmv_q8_g64_mps(x, p8, s8), K.qmv_q8_g64(x, p8, s8))
    assert _same(mod.qmm_q8_g64_mps(x, p8, s8), K.qmm_q8_g64(x, p8, s8))
    pt, st = K.pack_linear_ternary(w)
    assert _same(mod.qmv_ternary_mps(x, pt, st, b), K.qmv_ternary(x, pt, st, b))
    assert _same(mod.qmm_ternary_mps(x, pt, st), K.qmm_ternary(x, pt, st))
    p2, s2 = K.pack_linear_q2_k(w)
    assert _same(mod.qmv_q2_k_mps(x, p2, s2), K.qmv_q2_k(x, p2, s2))
    assert _same(mod.qmm_q2_k_mps(x, p2, s2, b), K.qmm_q2_k(x, p2, s2, b))


def _quant_cache(kind, B, H, S, hd, g, dev):
    import axiomlm_amd.kernels as K

    k = torch.randn(B, H, S, hd, generator=g, device=dev).half()
    v = torch.randn(B, H, S, hd, generator=g, device=dev).half()
    if kind == "fp16":
        return k, v, None, None
    kq, ks, vq, vs = (K.quantize_kv_fp8 if kind == "fp8" else K.quantize_kv_int4)(k, v)
    return kq, vq, ks, vs


@pytest.mark.parametrize("kind", ["fp16", "fp8", "int4"])
def test_module_attention(dev, mod, kind):
    import axiomlm_amd.kernels as K

    print(f"[module_attention] kv={kind}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    kc, vc, ks, vs = _quant_cache(kind, 1, 2, 256, 128, g, dev)
    q = torch.randn(1, 8, 1, 128, generator=g, device=dev).half()
    want = K.gqa_flash_decode_mps(q, kc, vc, 200, 0, ks, vs, kind)
    if kind == "fp16":
        got = mod.gqa_flash_decode_mps(q, kc, vc, 200)
    else:
        got = getattr(mod, f"gqa_flash_decode_{kind}_mps")(q, kc, vc, ks, vs, 200)
    assert _same(got, want)
    parents = [-1, 0, 0, 1, 2, 2]
    masks = []
    for u, p in enumerate(parents):
        masks.append((masks[p] if p >= 0 else 0) | (1 << u))
    qt = torch.randn(1, 6, 8 * 128, generator=g, device=dev).half()
    want = K.gqa_tree_verify_mps(qt, kc, vc, masks, 100, 100, 8, 0, ks, vs, kind)
    if kind == "fp16":
        got = mod.gqa_tree_verify_mps(qt, kc, vc, masks, 100, 100, 8)
    else:
        got = getattr(mod, f"gqa_tree_verify_{kind}_mps")(qt, kc, vc, ks, vs, masks, 100, 100, 8)
    assert _same(got, want)


@pytest.mark.parametrize("kind", ["fp16", "fp8", "int4"])
def test_module_cache_writes_compaction_dequant(dev, mod, kind):
    import axiomlm_amd.kernels as K
    from axiomlm_amd.cache import StaticKVCache

    print(f"[module_cache] kv={kind}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    hd, Hq, Hkv, S, T = 128, 4, 2, 64, 5
    qd, kd = Hq * hd, Hkv * hd
    freqs = torch.randn(128, hd // 2, 2, generator=g, device=dev)
    bias = torch.randn(qd + 2 * kd, generator=g, device=dev).half()
    caches = [StaticKVCache(1, S, 2, Hkv, hd, device=dev, cache_dtype=kind) for _ in range(2)]
    for c in caches:
        c.cache.zero_()  # an fp16 cache starts uninitialized; compare written slots only
    for tree in (False, True):
        qkv0 = torch.randn(1, T, qd + 2 * kd, generator=g, device=dev).half()
        qkv = [qkv0.clone(), qkv0.clone()]
        depths = [0, 1, 1, 2, 3]
        c0, c1 = caches
        ks0 = c0.k_scales[1] if kind != "fp16" else None
        vs0 = c0.v_scales[1] if kind != "fp16" else None
        ks1 = c1.k_scales[1] if kind != "fp16" else None
        vs1 = c1.v_scales[1] if kind != "fp16" else None
        if tree:
            K.rope_tree_kv_cache_write(qkv[0], freqs, c0.k_caches[1], c0.v_caches[1], depths, qd, kd, hd, 7, 20,
                                       bias, ks0, vs0, kind)
            if kind == "fp16":
                mod.rope_tree_kv_cache_write_mps(qkv[1], freqs, c1.k_caches[1], c1.v_caches[1], depths, qd, kd, hd,
                                                 7, 20, bias)
            else:
                getattr(mod, f"rope_tree_kv_write_{kind}_mps")(qkv[1], freqs, c1.k_caches[1], c1.v_caches[1], ks1,
                                                               vs1, torch.tensor(depths), qd, kd, hd, 7, 20, T, bias)
        else:
            K.rope_kv_cache_write_quantized(qkv[0], freqs, c0.k_caches[1], c0.v_caches[1], ks0, vs0, qd, kd, hd, 3,
                                            61, kind, bias)
            if kind == "fp16":
                mod.rope_kv_cache_write_mps(qkv[1], freqs, c1.k_caches[1], c1.v_caches[1], qd, kd, hd, 3, 61, bias)
            else:
                getattr(mod, f"rope_kv_cache_write_{kind}_mps")(qkv[1], freqs, c1.k_caches[1], c1.v_caches[1], ks1,
                                                                vs1, qd, kd, hd, 3, 61, bias)
        assert _same(qkv[0], qkv[1]) and _same(c0.cache, c1.cache)
        if kind != "fp16":
            assert _same(c0.scales, c1.scales)
    acc = [0, 2, 3]
    c0, c1 = caches
    c0.compact_tree_path(20, acc)
    if kind == "fp16":
        mod.compact_tree_kv_mps(c1.cache, 20, acc)
    else:
        mod.compact_tree_kv_quant_mps(c1.cache, c1.scales, 20, acc, kind)
        assert _same(c0.scales, c1.scales)
    assert _same(c0.cache, c1.cache)
    if kind != "fp16":
        want = (K.dequantize_kv_fp8 if kind == "fp8" else K.dequantize_kv_int4)(c0.k_caches[1], c0.k_scales[1], hd)
        got = getattr(mod, f"dequantize_kv_cache_{kind}_mps")(c1.k_caches[1], c1.k_scales[1], Hkv, S, hd)
        assert _same(got, want)


def test_module_norms_swiglu_argmax(dev, mod):
    import axiomlm_amd.kernels as K

    print("[module_norms]", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = torch.randn(3, 512, generator=g, device=dev).half()
    w = torch.randn(512, generator=g, device=dev).half()
    assert _same(mod.rmsnorm_infer_mps(x, w, 1e-5), K.fused_rmsnorm(x, w, 1e-5))
    r = torch.randn(3, 512, generator=g, device=dev).half()
    x1, x2 = x.clone(), x.clone()
    assert _same(mod.add_rmsnorm_infer_mps(x1, r, w, 1e-5), K.add_rmsnorm_infer(x2, r, w, 1e-5))
    assert _same(x1, x2)
    gu = torch.randn(2, 1, 2 * 704, generator=g, device=dev).half()
    assert _same(mod.swiglu_gate_up_mps(gu), K.swiglu_gate_up(gu))
    logits = torch.randn(1, 4, 1000, generator=g, device=dev).half()
    logits[0, 3, 17] = logits[0, 3, 900] = 50.0
    tok = mod.argmax_last_token_mps(logits)
    assert tuple(tok.shape) == (1, 1) and int(tok) == 17
    host = logits[0, 3].float().cpu().numpy()
    assert int(tok) == int(np.argmax(host))  # lowest index of the two maxima
