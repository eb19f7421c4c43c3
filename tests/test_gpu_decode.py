"""The decode step (one replay of the captured per-kernel graph per token)
against the CPU oracle on the same seeded synthetic weights and prompts, at
long prompts (every attention split populated) and across GQA geometries.

Bars: identical greedy tokens; logits within 1e-3 relative of the oracle; a
repeated run reproduces the logits bit for bit (the attention merge and every
reduction run in a fixed order).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
LOGIT_TOL = 1e-3

TINY = dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
            n_kv_heads=6, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=True)


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def test_tiny_decode_deterministic(orc, hip):
    print("[case] tiny: decode vs oracle, 64 tokens, twice", flush=True)
    orc.set_threads(8)
    om = orc.Llama(orc.LlamaConfig(**TINY), 0, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**TINY), 0)
    prompt = orc.prompt_ids(1, 8, TINY["vocab_size"])
    ref_t, ref_l = om.generate_greedy(prompt, 64, mode=1, want_logits=True)
    kt, kl = hm.generate_greedy(prompt, 64, want_logits=True)
    err = max(rel_err(kl[i], ref_l[i]) for i in range(64))
    print(f"[err] tiny decode {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    assert (kt == ref_t).all()
    kt2, kl2 = hm.generate_greedy(prompt, 64, want_logits=True)
    assert (kt2 == kt).all() and np.array_equal(kl2, kl)
    hm.free()
    om.close()
    orc.set_threads(0)


def test_7b_dims_long_prompt_vs_oracle(orc, hip):
    """Config-4 shapes (h4096, 32 heads, hd 128, ffn 11008, V32000), 2 layers,
    a 300-token prompt (every attention split populated) and 24 greedy steps,
    token by token and with the batched prompt prefill."""
    print("[case] 7B dims, 2 layers, prompt 300, 24 greedy", flush=True)
    cfg = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, n_layers=2,
               n_heads=32, n_kv_heads=32, max_seq_len=2048, rope_theta=10000.0,
               tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 0, init_on_device=True)
    prompt = hip.synth.prompt_ids(1, 300, 32000)
    kt, kl = hm.generate_greedy(prompt, 24, want_logits=True)
    pt, pl = hm.generate_greedy(prompt, 24, want_logits=True, prefill=True)
    orc.set_threads(16)
    om = orc.Llama(orc.LlamaConfig(**cfg), None)
    for layer in range(2):
        for tid in (orc.T_QKV, orc.T_O, orc.T_GATE, orc.T_UP, orc.T_DOWN):
            q, s = hm.qtensor(tid, layer)
            om.set_qtensor(tid, layer, q, s)
    q, s = hm.qtensor(orc.T_LM_HEAD)
    om.set_qtensor(orc.T_LM_HEAD, 0, q, s)
    om.set_embed(hm.embed())
    hm.free()
    ref_t, ref_l = om.generate_greedy_fast(prompt, 24, want_logits=True)
    om.close()
    orc.set_threads(0)
    ek = max(rel_err(kl[i], ref_l[i]) for i in range(24))
    ep = max(rel_err(pl[i], ref_l[i]) for i in range(24))
    print(f"[err] token by token {ek:.3e}, prefill {ep:.3e}", flush=True)
    assert ek < LOGIT_TOL and ep < LOGIT_TOL
    assert (kt == ref_t).all() and (pt == ref_t).all()


def test_7b_dims_long_context_vs_oracle(orc, hip):
    """Config-4 shapes, 2 layers, a 1600-token prompt: with 16 splits per KV
    group each split walks 100 cached rows, more than one step of its
    workgroup (96 rows), so the split loop runs twice.  Token by token and
    with the batched prefill, 6 greedy steps, against the oracle on the GPU
    model's own weights."""
    print("[case] 7B dims, 2 layers, prompt 1600, 6 greedy", flush=True)
    cfg = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, n_layers=2,
               n_heads=32, n_kv_heads=32, max_seq_len=2048, rope_theta=10000.0,
               tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 0, init_on_device=True)
    prompt = hip.synth.prompt_ids(5, 1600, 32000)
    kt, kl = hm.generate_greedy(prompt, 6, want_logits=True)
    pt, pl = hm.generate_greedy(prompt, 6, want_logits=True, prefill=True)
    orc.set_threads(16)
    om = orc.Llama(orc.LlamaConfig(**cfg), None)
    for layer in range(2):
        for tid in (orc.T_QKV, orc.T_O, orc.T_GATE, orc.T_UP, orc.T_DOWN):
            q, s = hm.qtensor(tid, layer)
            om.set_qtensor(tid, layer, q, s)
    q, s = hm.qtensor(orc.T_LM_HEAD)
    om.set_qtensor(orc.T_LM_HEAD, 0, q, s)
    om.set_embed(hm.embed())
    hm.free()
    ref_t, ref_l = om.generate_greedy_fast(prompt, 6, want_logits=True)
    om.close()
    orc.set_threads(0)
    ek = max(rel_err(kl[i], ref_l[i]) for i in range(6))
    ep = max(rel_err(pl[i], ref_l[i]) for i in range(6))
    print(f"[err] token by token {ek:.3e}, prefill {ep:.3e}", flush=True)
    assert ek < LOGIT_TOL and ep < LOGIT_TOL
    assert (kt == ref_t).all() and (pt == ref_t).all()


@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 4), (4, 1, 128), (16, 4, 64)])
def test_gqa_decode_vs_oracle(orc, hip, nh, nkv, hd):
    print(f"[case] GQA nh={nh} nkv={nkv} hd={hd}", flush=True)
    cfg = dict(vocab_size=64, hidden_size=nh * hd, intermediate_size=256, n_layers=2,
               n_heads=nh, n_kv_heads=nkv, max_seq_len=160, rope_theta=500000.0,
               tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 7, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 7)
    prompt = orc.prompt_ids(3, 100, 64)
    ref_t, ref_l = om.generate_greedy(prompt, 20, mode=1, want_logits=True)
    kt, kl = hm.generate_greedy(prompt, 20, want_logits=True)
    assert max(rel_err(kl[i], ref_l[i]) for i in range(20)) < LOGIT_TOL
    assert (kt == ref_t).all()
    hm.free()
    om.close()
