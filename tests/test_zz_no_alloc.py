"""axm_gqa_flash_decode_noalloc through the C ABI against axm_gqa_flash_decode with a
caller workspace: bit-identical outputs on two calls in a row (the second with a
smaller input, so stale partials of the first call sit in the shared array), for
fp16 / fp8 / int4 caches with split counts above one; and a size beyond the
fixed array rejected with an error before anything is launched."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cache(kind, B, H, S, hd, g, dev):
    import axiomlm_amd.kernels as K

    k = torch.randn(B, H, S, hd, generator=g, device=dev).half()
    v = torch.randn(B, H, S, hd, generator=g, device=dev).half()
    if kind == "fp16":
        return k, v, None, None
    kq, ks, vq, vs = (K.quantize_kv_fp8 if kind == "fp8" else K.quantize_kv_int4)(k, v)
    return kq, vq, ks, vs


def _call(fn_name, q, kc, vc, ks, vs, code, B, Hq, Hkv, hd, S, L, splits, ws=None):
    from axiomlm_amd import _lib

    out = torch.empty_like(q)
    lib = _lib.lib()
    args = [_lib.ptr(q), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(ks), _lib.ptr(vs), code, _lib.ptr(out), B, Hq, Hkv, hd,
            S, L, splits]
    if fn_name == "axm_gqa_flash_decode":
        args += [_lib.ptr(ws), ws.numel() if ws is not None else 0]
    rc = getattr(lib, fn_name)(*args, _lib.stream_of(q.device))
    return rc, out


@pytest.mark.parametrize("kind", ["fp16", "fp8", "int4"])
def test_noalloc_flash_decode_matches_workspace_entry_point(dev, kind):
    from axiomlm_amd import _lib
    from axiomlm_amd.kernels.ops import KV_CODES

    code = KV_CODES[kind]
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    lib = _lib.lib()
    # first a large call, then a smaller one: B, heads, length and splits all shrink
    for B, Hq, Hkv, hd, S, L in ((8, 32, 8, 128, 4096, 4000), (2, 8, 2, 64, 1024, 700)):
        print(f"[noalloc] kind={kind} B={B} Hq={Hq} Hkv={Hkv} hd={hd} L={L}", flush=True)
        kc, vc, ks, vs = _cache(kind, B, Hkv, S, hd, g, dev)
        q = torch.randn(B, Hq, hd, generator=g, device=dev).half()
        splits = lib.axm_attention_num_splits(B, Hq, Hkv, hd, code, L)
        if splits < 2:
            splits = 4
        need = lib.axm_attention_workspace_bytes(B, Hq, hd, splits)
        assert 0 < need <= 16 << 20
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        rc, want = _call("axm_gqa_flash_decode", q, kc, vc, ks, vs, code, B, Hq, Hkv, hd, S, L, splits, ws)
        assert rc == 0, lib.axm_last_error()
        rc, got = _call("axm_gqa_flash_decode_noalloc", q, kc, vc, ks, vs, code, B, Hq, Hkv, hd, S, L, splits)
        assert rc == 0, lib.axm_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_partials_beyond_the_array(dev):
    from axiomlm_amd import _lib

    lib = _lib.lib()
    B, Hq, Hkv, hd, S, L = 8, 64, 8, 128, 8192, 8192
    splits = 128  # 8 * 64 * 128 * 130 * 4 bytes = 34 MB > 16 MiB
    assert lib.axm_attention_workspace_bytes(B, Hq, hd, splits) > 16 << 20
    kc = torch.zeros(B, Hkv, S, hd, dtype=torch.float16, device=dev)
    q = torch.zeros(B, Hq, hd, dtype=torch.float16, device=dev)
    rc, _ = _call("axm_gqa_flash_decode_noalloc", q, kc, kc, None, None, 0, B, Hq, Hkv, hd, S, L, splits)
    assert rc == -1
    assert b"scratch" in lib.axm_last_error()
