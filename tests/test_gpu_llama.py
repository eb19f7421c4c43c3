"""GPU parity of the int8 Llama path against the CPU oracle on the same seeded
synthetic weights and prompt ids:
  - the quantize + repack layout step is bit-exact (every tensor, every scale);
  - logits agree within 1e-3 relative (max|g - c| / max|c|, fp32 accumulation);
  - greedy tokens are identical over the run.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32
LOGIT_TOL = 1e-3


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def configs(orc, hip):
    return orc, hip


def both(orc, hip, seed=0, quant_mode=0, keep_f32=False, **cfg):
    oc = orc.LlamaConfig(**cfg)
    hc = hip.LlamaConfig(**{k: v for k, v in cfg.items()})
    om = orc.Llama(oc, seed, quantize=True, keep_f32=keep_f32, block32=(quant_mode == 1))
    hm = hip.LlamaModel.new_random(hc, seed, quant_mode)
    return om, hm


TINY = dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
            n_kv_heads=6, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=True)
SMOKE = dict(vocab_size=32, hidden_size=16, intermediate_size=32, n_layers=2, n_heads=4,
             n_kv_heads=2, max_seq_len=64, rope_theta=500000.0, tie_word_embeddings=True)


@pytest.fixture(scope="module")
def tiny(orc, hip):
    print("[case] tiny model init (h288 L6 V32000, seed 0)", flush=True)
    orc.set_threads(8)
    om, hm = both(orc, hip, **TINY)
    yield om, hm
    hm.free()
    om.close()
    orc.set_threads(0)


def test_layout_step_bit_exact(tiny, orc, hip):
    om, hm = tiny
    assert (hm.embed() == om.tensor(orc.T_EMBED)).all()
    for layer in range(TINY["n_layers"]):
        for tid in (orc.T_QKV, orc.T_O, orc.T_GATE, orc.T_UP, orc.T_DOWN):
            qg, sg = hm.qtensor(tid, layer)
            qo, so = om.qtensor(tid, layer)
            assert sg == so, (layer, tid)
            assert (qg == qo).all(), (layer, tid)
    qg, sg = hm.qtensor(orc.T_LM_HEAD)
    qo, so = om.qtensor(orc.T_LM_HEAD)
    assert sg == so and (qg == qo).all()


def test_tiny_greedy_128_tokens(tiny, orc):
    """Config 1: 8 seeded prompt ids, 128 greedy tokens, identical tokens and
    per-step logits within 1e-3 relative."""
    om, hm = tiny
    prompt = orc.prompt_ids(1, 8, TINY["vocab_size"])
    print(f"[case] tiny greedy 128, prompt {prompt.tolist()}", flush=True)
    ref_toks, ref_lg = om.generate_greedy(prompt, 128, mode=1, want_logits=True)
    toks, lg = hm.generate_greedy(prompt, 128, want_logits=True)
    errs = [rel_err(lg[i], ref_lg[i]) for i in range(len(ref_toks))]
    print(f"[err] max step rel err {max(errs):.3e}", flush=True)
    assert max(errs) < LOGIT_TOL
    assert (toks == ref_toks).all()
    # the fast path (no logits readback, pure graph replays) gives the same ids
    assert (hm.generate_greedy(prompt, 128) == ref_toks).all()


def test_tiny_forward_with_cache_and_kv_contents(tiny, orc):
    om, hm = tiny
    prompt = [5, 17, 31999, 0, 123]
    oc = om.new_cache(16)
    hc = hm.new_llama_kv_cache(16)
    for pos, t in enumerate(prompt):
        ref = om.forward_with_cache(oc, t, pos, mode=1)
        lg, am = hm.forward_with_llama_cache(t, pos, hc)
        assert rel_err(lg, ref) < LOGIT_TOL
        assert am == orc.argmax(lg)
    assert hc.seq_len == len(prompt)
    for layer in (0, 5):
        kg, vg = hc.layer(layer)
        ko, vo = oc.layer(layer)
        assert rel_err(kg, ko) < 1e-4 and rel_err(vg, vo) < 1e-4
        n = len(prompt) * TINY["hidden_size"]
        assert (kg[n:] == 0).all()
    hc.free()


def test_generate_edge_cases(tiny, orc, hip):
    om, hm = tiny
    # max_tokens = 0 still yields the token after the prompt (generate.rs:68-75)
    t0 = hm.generate_greedy([7], 0)
    assert len(t0) == 1 and t0[0] == om.generate_greedy([7], 0, mode=1)[0]
    with pytest.raises(ValueError):
        hip.generate(hm, [], hip.SamplingConfig(temperature=0.0, max_tokens=4))
    with pytest.raises(hip.ScryHipError) as ei:
        hm.generate_greedy([32000], 4)
    assert ei.value.code == 5
    c = hm.new_llama_kv_cache(2)
    hm.forward_with_llama_cache(1, 0, c)
    hm.forward_with_llama_cache(2, 1, c)
    with pytest.raises(hip.ScryHipError) as ei:
        hm.forward_with_llama_cache(3, 2, c)  # cache full
    assert ei.value.code == 5
    c.free()


def test_smoke_cache_matches_full_forward(orc, hip):
    """tests/llama_smoke.rs:102-128 with the GPU cache path against the
    oracle's full (prefill) forward, int8 composition."""
    om, hm = both(orc, hip, seed=42, **SMOKE)
    toks = [3, 7, 1]
    full = om.forward(toks, mode=1)
    c = hm.new_llama_kv_cache(64)
    for pos, t in enumerate(toks):
        lg, _ = hm.forward_with_llama_cache(t, pos, c)
    assert np.abs(full[-1] - lg).max() < 1e-3
    c.free()
    hm.free()


@pytest.mark.parametrize("nh,nkv", [(4, 4), (4, 2), (4, 1), (8, 2)])
def test_gqa_ratios(orc, hip, nh, nkv):
    # tests/llama_smoke.rs:268-305 (head_dim 4)
    cfg = dict(vocab_size=16, hidden_size=nh * 4, intermediate_size=32, n_layers=1, n_heads=nh,
               n_kv_heads=nkv, max_seq_len=32, rope_theta=10000.0, tie_word_embeddings=True)
    om, hm = both(orc, hip, seed=42, **cfg)
    oc = om.new_cache(32)
    hc = hm.new_llama_kv_cache(32)
    for pos in range(12):
        t = pos % 16
        ref = om.forward_with_cache(oc, t, pos, mode=1)
        lg, _ = hm.forward_with_llama_cache(t, pos, hc)
        assert np.isfinite(lg).all()
        assert rel_err(lg, ref) < LOGIT_TOL, (nh, nkv, pos)
    hc.free()
    hm.free()


def test_gqa_head_dim_128_long_context(orc, hip):
    """Llama-3 head geometry (hd 128, 4 query heads per KV head) at a length
    that exercises every attention split."""
    cfg = dict(vocab_size=64, hidden_size=512, intermediate_size=256, n_layers=1, n_heads=4,
               n_kv_heads=1, max_seq_len=300, rope_theta=500000.0, tie_word_embeddings=False)
    om, hm = both(orc, hip, seed=3, **cfg)
    prompt = orc.prompt_ids(5, 200, 64)
    ref = om.generate_greedy(prompt, 40, mode=1, want_logits=True)
    got = hm.generate_greedy(prompt, 40, want_logits=True)
    assert max(rel_err(got[1][i], ref[1][i]) for i in range(40)) < LOGIT_TOL
    assert (got[0] == ref[0]).all()
    hm.free()


def test_block32_mode(orc, hip):
    om, hm = both(orc, hip, seed=1, quant_mode=1, **{**TINY, "n_layers": 2})
    for tid in (orc.T_QKV, orc.T_GATE, orc.T_UP, orc.T_DOWN):
        qg, _ = hm.qtensor(tid, 1)
        qo, _ = om.qtensor(tid, 1)
        assert qg.shape == qo.shape
    prompt = orc.prompt_ids(1, 8, TINY["vocab_size"])
    ref = om.generate_greedy(prompt, 16, mode=2, want_logits=True)
    got = hm.generate_greedy(prompt, 16, want_logits=True)
    assert max(rel_err(got[1][i], ref[1][i]) for i in range(16)) < LOGIT_TOL
    assert (got[0] == ref[0]).all()
    hm.free()


def test_llama2_7b_dims_two_layers(orc, hip):
    """Config-4 tensor shapes (h4096, 32 heads, ffn 11008, V32000, untied) with
    two layers: layout bit-exact, logits 1e-3, identical greedy tokens."""
    print("[case] 7B dims, 2 layers", flush=True)
    orc.set_threads(16)
    cfg = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, n_layers=2,
               n_heads=32, n_kv_heads=32, max_seq_len=2048, rope_theta=10000.0,
               tie_word_embeddings=False)
    om, hm = both(orc, hip, seed=0, **cfg)
    for tid in (orc.T_QKV, orc.T_O, orc.T_GATE, orc.T_UP, orc.T_DOWN):
        qg, sg = hm.qtensor(tid, 1)
        qo, so = om.qtensor(tid, 1)
        assert sg == so and (qg == qo).all(), tid
    qg, sg = hm.qtensor(orc.T_LM_HEAD)
    qo, so = om.qtensor(orc.T_LM_HEAD)
    assert sg == so and (qg == qo).all()
    prompt = orc.prompt_ids(1, 6, 32000)
    ref = om.generate_greedy(prompt, 10, mode=1, want_logits=True)
    got = hm.generate_greedy(prompt, 10, want_logits=True)
    err = max(rel_err(got[1][i], ref[1][i]) for i in range(10))
    print(f"[err] 7B-dims max step rel err {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    assert (got[0] == ref[0]).all()
    hm.free()
    om.close()
    orc.set_threads(0)
