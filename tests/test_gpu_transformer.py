"""The decode driver (axiomlm_amd.transformer.Transformer) end to end on the GPU against
the reference's own CPU path (tests/golden/c1_q4.npz, written by
tests/golden/make_golden_c1.py from the seed-0 C1 weights):

* quantize("q4") on the GPU packs every matrix as the reference's
  ``_ensure_quant_weights`` does (byte-identical up to near-tie groups of the
  MSE clip search);
* forward() token by token then greedy reproduces the reference decode logits
  (max |diff| <= 1e-2) and its 64 greedy tokens;
* forward() of the whole prompt (one verify pass) reproduces the reference
  prefill logits, and a 48-token sequence fed as 32 + 16 chunks matches the
  token-by-token logits;
* forward_tree_verify over a chain tree and over a branching tree of the golden
  continuation matches the golden logits on the golden path, leaves the counters
  alone, and after compact_tree_path decoding continues the golden run.
"""

import numpy as np
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu

F32 = np.float32
TOL = 1e-2


def _model(dev):
    from axiomlm_amd.transformer import ModelConfig, Transformer
    from c1_golden import c1_config

    c = c1_config()
    W = om.make_float_weights(c, seed=0)
    sd = {"transformer.wte.weight": W["wte"], "lm_head.weight": W["lm_head"], "transformer.ln_f.weight": W["lnf"]}
    for i, lw in enumerate(W["layers"]):
        pre = f"transformer.h.{i}."
        sd[pre + "ln_1.weight"] = lw["ln1"]
        sd[pre + "ln_2.weight"] = lw["ln2"]
        sd[pre + "attn.c_attn.weight"] = lw["c_attn"]
        sd[pre + "attn.c_proj.weight"] = lw["c_proj"]
        sd[pre + "mlp.w_gate.weight"] = lw["w_gate"]
        sd[pre + "mlp.w_up.weight"] = lw["w_up"]
        sd[pre + "mlp.w_down.weight"] = lw["w_down"]
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}
    cfg = ModelConfig(block_size=c.block_size, vocab_size=c.vocab, n_layer=c.n_layer, n_head=c.n_head,
                      n_embd=c.d_model, n_kv_head=c.n_kv_head, intermediate_size=c.hidden, rms_norm_eps=c.eps,
                      tie_word_embeddings=False)
    return Transformer(cfg, sd, device=dev).quantize("q4"), cfg


def _cache(cfg, dev, S=128):
    from axiomlm_amd.cache import StaticKVCache

    return StaticKVCache(1, S, cfg.n_layer, cfg.kv_heads, cfg.head_dim, device=dev)


def _check(got, ref, what):
    d = float(np.max(np.abs(got.astype(F32) - ref.astype(F32))))
    assert d <= TOL, f"{what}: max |diff| {d:.3e} > {TOL}"


def test_quantize_packs_match_reference(dev):
    """quantize("q4") packs every matrix with the reference's choices: the Q8_G64 table
    byte-identical to the reference's, each MARLIN Q4 matrix equal to the reference pack
    except near-tie groups of the MSE clip search (at most 1% of groups per matrix, codes
    identical wherever the group's (scale, bias) agree)."""
    from c1_golden import golden, marlin_near_tie_fraction, named_packs, oracle_packs, pack_digest

    print("[transformer_packs]", flush=True)
    m, cfg = _model(dev)
    qw = m._ensure_quant_weights()
    got = {"wte_p": qw["wte_p"], "wte_sb": qw["wte_sb"], "lmh_p": qw["lmh_p"], "lmh_sb": qw["lmh_sb"]}
    for key in ("c_attn_p", "c_attn_s", "c_proj_p", "c_proj_s", "gu_p", "gu_s", "wd_p", "wd_s"):
        for i, t in enumerate(qw[key]):
            got[f"{key}{i}"] = t
    got = {k: v.cpu().numpy() for k, v in got.items()}
    g = golden()
    want = dict(zip(g["pack_names"].tolist(), g["pack_sha256"].tolist()))
    assert set(want) == set(got)
    ref = named_packs(oracle_packs())
    assert all(pack_digest(ref[k]) == want[k] for k in want)
    assert pack_digest(got["wte_p"]) == want["wte_p"] and pack_digest(got["wte_sb"]) == want["wte_sb"]
    pairs = [("lmh_p", "lmh_sb", cfg.n_embd)]
    for i in range(cfg.n_layer):
        pairs += [(f"c_attn_p{i}", f"c_attn_s{i}", cfg.n_embd), (f"c_proj_p{i}", f"c_proj_s{i}", cfg.n_embd),
                  (f"gu_p{i}", f"gu_s{i}", cfg.n_embd), (f"wd_p{i}", f"wd_s{i}", cfg.hidden)]
    exact, report = 0, []
    for kp, ks, K in pairs:
        if pack_digest(got[kp]) == want[kp] and pack_digest(got[ks]) == want[ks]:
            exact += 1
            continue
        report.append((kp, marlin_near_tie_fraction(got[kp], got[ks], ref[kp], ref[ks], K, kp)))
    print(f"[transformer_packs] {exact}/{len(pairs)} bit-identical; near-tie groups: {report}", flush=True)
    assert all(frac <= 0.01 for _, frac in report), report


def test_forward_decode_and_greedy_match_reference(dev):
    from c1_golden import golden

    print("[transformer_decode]", flush=True)
    g = golden()
    m, cfg = _model(dev)
    cache = _cache(cfg, dev)
    ref = g["decode_logits"]
    prompt = g["prompt"].tolist()
    for i, tok in enumerate(prompt):
        lg, extra, kv = m.forward(torch.tensor([[tok]], device=dev), kv_caches=cache)
        assert extra is None and len(kv) == cfg.n_layer and kv[0] is cache
        assert lg.shape == (1, 1, cfg.vocab_size)
        _check(lg[0, 0].float().cpu().numpy(), ref[i], f"prompt step {i}")
    assert cache.total_seen_tokens == [32] * cfg.n_layer and cache.layer_seq_lens == [32] * cfg.n_layer
    toks = []
    tok = int(torch.argmax(lg[0, 0].float()))
    for i in range(64):
        toks.append(tok)
        lg = m.forward(torch.tensor([[tok]], device=dev), kv_caches=cache)[0]
        _check(lg[0, 0].float().cpu().numpy(), ref[32 + i], f"greedy step {i}")
        tok = int(torch.argmax(lg[0, 0].float()))
    assert toks == g["greedy_tokens"].tolist()


def test_forward_prefill_and_chunks_match_reference(dev):
    from c1_golden import golden

    print("[transformer_prefill]", flush=True)
    g = golden()
    m, cfg = _model(dev)
    prompt = g["prompt"].tolist()
    cache = _cache(cfg, dev)
    lg = m.forward(torch.tensor([prompt], device=dev), kv_caches=cache, return_all_logits=True)[0]
    assert lg.shape == (1, 32, cfg.vocab_size)
    _check(lg[0].float().cpu().numpy(), g["prefill_logits"], "prefill")
    # Teacher-forced continuation on the prefilled cache.
    greedy = g["greedy_tokens"].tolist()
    for i in range(16):
        lg = m.forward(torch.tensor([[greedy[i]]], device=dev), kv_caches=cache)[0]
        _check(lg[0, 0].float().cpu().numpy(), g["decode_logits"][32 + i], f"after-prefill step {i}")
    # 48 tokens in one call: chunks of 32 + 16 (the second with a cached prefix).
    seq = prompt + greedy[:16]
    cache2 = _cache(cfg, dev)
    lg = m.forward(torch.tensor([seq], device=dev), kv_caches=cache2, return_all_logits=True)[0]
    assert lg.shape == (1, 48, cfg.vocab_size)
    _check(lg[0, :32].float().cpu().numpy(), g["prefill_logits"], "chunk 0")
    _check(lg[0, 32:].float().cpu().numpy(), g["decode_logits"][32:48], "chunk 1")
    assert cache2.total_seen_tokens == [48] * cfg.n_layer
    last = m.forward(torch.tensor([seq], device=dev), kv_caches=_cache(cfg, dev))[0]
    assert last.shape == (1, 1, cfg.vocab_size)


def test_tree_verify_chain_matches_reference(dev):
    from c1_golden import golden

    print("[transformer_tree]", flush=True)
    g = golden()
    m, cfg = _model(dev)
    cache = _cache(cfg, dev)
    m.forward(torch.tensor([g["prompt"].tolist()], device=dev), kv_caches=cache)
    T = 8
    nodes = g["greedy_tokens"].tolist()[:T]
    depths = list(range(T))
    masks = [(1 << (u + 1)) - 1 for u in range(T)]
    lg, medusa, kv = m.forward_tree_verify(torch.tensor([nodes], device=dev), cache, depths, masks)
    assert medusa == [] and cache.total_seen_tokens == [32] * cfg.n_layer
    _check(lg[0].float().cpu().numpy(), g["decode_logits"][32:32 + T], "chain tree")
    assert m._last_verify_norm.shape == (1, T, cfg.n_embd)
    # A branching tree: node 1 is a wrong sibling of node 2; the golden path is 0 -> 2 -> 3.
    cache = _cache(cfg, dev)
    m.forward(torch.tensor([g["prompt"].tolist()], device=dev), kv_caches=cache)
    wrong = (nodes[1] + 1) % cfg.vocab_size
    tree = [nodes[0], wrong, nodes[1], nodes[2]]
    depths = [0, 1, 1, 2]
    masks = [0b0001, 0b0011, 0b0101, 0b1101]
    lg = m.forward_tree_verify(torch.tensor([tree], device=dev), cache, depths, masks)[0]
    ref = g["decode_logits"]
    for u, row in ((0, 32), (2, 33), (3, 34)):
        _check(lg[0, u].float().cpu().numpy(), ref[row], f"tree node {u}")
    # Commit the accepted path [0, 2, 3], then decode on: logits continue the golden run.
    cache.compact_tree_path(32, [0, 2, 3], 35)
    assert cache.total_seen_tokens == [35] * cfg.n_layer
    lg = m.forward(torch.tensor([[nodes[3]]], device=dev), kv_caches=cache)[0]
    _check(lg[0, 0].float().cpu().numpy(), ref[35], "after compaction")


def _host(p):
    """A pack on the host: Q8 packs as uint8 [N][K] like the oracle's; MARLIN packs unchanged."""
    a = p.cpu().numpy()
    return a.view(np.uint8).reshape(a.shape[0], -1) if a.ndim == 2 else a


def _oracle_on_packs(m, c):
    """The oracle model over the packs the GPU produced for Transformer m (and its fp16 norms)."""
    qw = m._ensure_quant_weights()
    h = lambda k: m.w[k].to(torch.float16).cpu().numpy()  # noqa: E731
    L = c.n_layer
    bias = [b.cpu().numpy() if b is not None else None for b in qw["c_attn_b"]]
    ow = om.OracleWeights(_host(qw["wte_p"]), qw["wte_sb"].cpu().numpy(), _host(qw["lmh_p"]),
                          qw["lmh_sb"].cpu().numpy(), [h(f"transformer.h.{i}.ln_1.weight") for i in range(L)],
                          [h(f"transformer.h.{i}.ln_2.weight") for i in range(L)], h("transformer.ln_f.weight"),
                          [_host(p) for p in qw["c_attn_p"]], [s.cpu().numpy() for s in qw["c_attn_s"]],
                          [_host(p) for p in qw["c_proj_p"]], [s.cpu().numpy() for s in qw["c_proj_s"]],
                          [_host(p) for p in qw["gu_p"]], [s.cpu().numpy() for s in qw["gu_s"]],
                          [_host(p) for p in qw["wd_p"]], [s.cpu().numpy() for s in qw["wd_s"]],
                          [] if all(b is None for b in bias) else bias)
    cos, sin = om.rope_tables(c.head_dim, c.block_size, m.config.rope_theta)
    return om.OracleModel(c, ow, cos, sin)


@pytest.mark.parametrize("mode", ["q4_k_m", "q8"])
def test_quantize_modes_decode_against_oracle(dev, mode):
    """quantize("q4_k_m") packs w_down and lm_head as Q8_G64 and the rest as MSE-clipped MARLIN
    Q4; quantize("q8") packs every matrix Q8_G64 (transformer.py:840-847).  The Q8 packs are
    byte-identical to the oracle's packer; forward() token by token matches the oracle model
    running on the packs the GPU produced (logits <= 1e-2)."""
    from oracle import formats as fm

    print(f"[transformer_modes] {mode}", flush=True)
    m, cfg = _model(dev)
    m.quantize(mode)
    qw = m._ensure_quant_weights()
    from c1_golden import c1_config

    c = c1_config()
    W = om.make_float_weights(c, seed=0)

    def q8_same(p, s, w):
        wp, wsb = fm.pack_linear_q8_g64(w)
        return np.array_equal(_host(p), wp) and np.array_equal(s.cpu().numpy().view(np.uint16), wsb.view(np.uint16))

    assert qw["lmh_p"].dim() == 2 and q8_same(qw["lmh_p"], qw["lmh_sb"], W["lm_head"])
    for i, lw in enumerate(W["layers"]):
        assert qw["wd_p"][i].dim() == 2 and q8_same(qw["wd_p"][i], qw["wd_s"][i], lw["w_down"])
        assert (qw["c_attn_p"][i].dim() == 2) == (mode == "q8")
    model = _oracle_on_packs(m, c)
    cache = _cache(cfg, dev)
    ocache = om.OracleKVCache(128, c.n_layer, c.n_kv_head, c.head_dim)
    rng = np.random.default_rng(21)
    for i, tok in enumerate(rng.integers(0, c.vocab, 10).tolist()):
        got = m.forward(torch.tensor([[tok]], device=dev), kv_caches=cache)[0][0, -1].float().cpu().numpy()
        _check(got, model.forward([tok], ocache)[-1], f"{mode} token {i}")


def test_unquantized_model_runs_on_the_fp16_runner(dev):
    """quantize(None) (the unquantized model) decodes through the fp16 runner
    (transformer.py:1310-1380) and matches the oracle on the same fp16 weights."""
    from c1_golden import c1_config

    from axiomlm_amd.runner import DecodeRunner

    print("[transformer_fp16]", flush=True)
    m, cfg = _model(dev)
    m.quantize(None)
    c = c1_config()
    W = om.make_float_weights(c, seed=0)
    cos, sin = om.rope_tables(c.head_dim, c.block_size)
    model = om.OracleModel(c, om.fp16_model(c, W), cos, sin)
    cache = _cache(cfg, dev)
    ocache = om.OracleKVCache(128, c.n_layer, c.n_kv_head, c.head_dim)
    rng = np.random.default_rng(22)
    for i, tok in enumerate(rng.integers(0, c.vocab, 10).tolist()):
        got = m.forward(torch.tensor([[tok]], device=dev), kv_caches=cache)[0][0, -1].float().cpu().numpy()
        _check(got, model.forward([tok], ocache)[-1], f"fp16 token {i}")
    assert isinstance(m.get_decode_runner(cache), DecodeRunner)


@pytest.mark.parametrize("family", ["llama", "qwen2"])
def test_hf_checkpoint_runs_on_the_gpu_runners(dev, tmp_path, family):
    """A HuggingFace safetensors checkpoint (tiny random-init Llama / Qwen2 written by
    transformers, head size 64) imported with load_hf_safetensors: on the fp16 runner its
    logits match HuggingFace's own forward; quantized ("q4_rtn", then release_fp16) it still
    decodes, with the fp16 copies of the packed matrices gone."""
    from test_hf_import import tiny_hf_checkpoint

    from axiomlm_amd.hf_import import load_hf_safetensors

    print(f"[hf_gpu] {family}", flush=True)
    path, hf = tiny_hf_checkpoint(tmp_path, family, False, hidden=256, inter=512)
    m = load_hf_safetensors(path, device=dev).quantize(None)
    ids = [5, 77, 200, 3, 141, 9, 64, 250]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0].float().numpy()
    cache = _cache(m.config, dev)
    got = np.stack([m.forward(torch.tensor([[t]], device=dev), kv_caches=cache)[0][0, -1].float().cpu().numpy()
                    for t in ids])
    err = float(np.abs(got - want).max())
    assert err <= 2e-2 * max(1.0, float(np.abs(want).max())), err
    m.quantize("q4_rtn", release_fp16=True)
    assert m.w["transformer.h.0.attn.c_attn.weight"].numel() == 0 and m.w["lm_head.weight"].numel() == 0
    with pytest.raises(RuntimeError):
        m.quantize(None)
    c = m.config
    oracle = _oracle_on_packs(m, om.OracleConfig(n_layer=c.n_layer, n_head=c.n_head, n_kv_head=c.kv_heads,
                                                 d_model=c.n_embd, hidden=c.hidden, vocab=c.vocab_size,
                                                 eps=c.rms_norm_eps, block_size=c.block_size))
    cache = _cache(m.config, dev)
    ocache = om.OracleKVCache(128, c.n_layer, c.kv_heads, c.head_dim)
    for i, t in enumerate(ids):
        q = m.forward(torch.tensor([[t]], device=dev), kv_caches=cache)[0][0, -1].float().cpu().numpy()
        _check(q, oracle.forward([t], ocache)[-1], f"{family} q4_rtn token {i}")
