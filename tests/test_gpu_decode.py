"""The two decode-step implementations -- the persistent decode kernel (one
launch per token) and the captured per-kernel graph -- against each other and
against the CPU oracle, on the same seeded synthetic weights and prompts.

Bars: identical greedy tokens; logits within 1e-3 relative of the oracle and
within 1e-4 relative of each other (same fp32 arithmetic, different summation
order); the persistent kernel is deterministic (bitwise-equal logits on a
repeated run).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
LOGIT_TOL = 1e-3
PATH_TOL = 1e-4

TINY = dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
            n_kv_heads=6, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=True)


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def run_both(hip, hm, prompt, n):
    """(tokens, logits) from the persistent kernel and from the per-kernel graph."""
    hip.set_decode_mode(hip.DECODE_PERSISTENT)
    try:
        assert hm.decode_persistent()
        p = hm.generate_greedy(prompt, n, want_logits=True)
    finally:
        hip.set_decode_mode(hip.DECODE_KERNELS)
    assert not hm.decode_persistent()
    k = hm.generate_greedy(prompt, n, want_logits=True)
    return p, k


def test_path_selection(hip):
    cfg = hip.LlamaConfig(**{**TINY, "n_layers": 1})
    m = hip.LlamaModel.new_random(cfg, 0)
    assert not m.decode_persistent()  # default: per-kernel graph
    hip.set_decode_mode(hip.DECODE_PERSISTENT)
    try:
        assert m.decode_persistent()
        b = hip.LlamaModel.new_random(cfg, 0, hip.QUANT_BLOCK32)
        assert not b.decode_persistent()  # block-32 scales: per-kernel graph
        b.free()
    finally:
        hip.set_decode_mode(hip.DECODE_KERNELS)
    m.free()


def test_tiny_paths_agree_with_oracle(orc, hip):
    print("[case] tiny: persistent vs per-kernel vs oracle, 64 tokens", flush=True)
    orc.set_threads(8)
    om = orc.Llama(orc.LlamaConfig(**TINY), 0, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**TINY), 0)
    prompt = orc.prompt_ids(1, 8, TINY["vocab_size"])
    ref_t, ref_l = om.generate_greedy(prompt, 64, mode=1, want_logits=True)
    (pt, pl), (kt, kl) = run_both(hip, hm, prompt, 64)
    ep = max(rel_err(pl[i], ref_l[i]) for i in range(64))
    ek = max(rel_err(kl[i], ref_l[i]) for i in range(64))
    epk = max(rel_err(pl[i], kl[i]) for i in range(64))
    print(f"[err] persistent {ep:.3e} kernels {ek:.3e} between {epk:.3e}", flush=True)
    assert ep < LOGIT_TOL and ek < LOGIT_TOL and epk < PATH_TOL
    assert (pt == ref_t).all() and (kt == ref_t).all()
    # deterministic: a second persistent run reproduces the logits bit for bit
    hip.set_decode_mode(hip.DECODE_PERSISTENT)
    try:
        pt2, pl2 = hm.generate_greedy(prompt, 64, want_logits=True)
    finally:
        hip.set_decode_mode(hip.DECODE_KERNELS)
    assert (pt2 == pt).all() and np.array_equal(pl2, pl)
    hm.free()
    om.close()
    orc.set_threads(0)


def test_7b_dims_paths_agree_long_prompt(hip):
    """Config-4 shapes (h4096, 32 heads, hd 128, ffn 11008, V32000), 2 layers,
    a 300-token prompt (every attention split populated) and 24 greedy steps."""
    print("[case] 7B dims, 2 layers, prompt 300: persistent vs per-kernel", flush=True)
    cfg = hip.LlamaConfig(vocab_size=32000, hidden_size=4096, intermediate_size=11008,
                          n_layers=2, n_heads=32, n_kv_heads=32, max_seq_len=2048,
                          rope_theta=10000.0, tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(cfg, 0)
    prompt = hip.synth.prompt_ids(1, 300, 32000)
    (pt, pl), (kt, kl) = run_both(hip, hm, prompt, 24)
    epk = max(rel_err(pl[i], kl[i]) for i in range(24))
    print(f"[err] between paths {epk:.3e}", flush=True)
    assert epk < PATH_TOL
    assert (pt == kt).all()
    hm.free()


@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 4), (4, 1, 128), (16, 4, 64)])
def test_gqa_paths_agree_with_oracle(orc, hip, nh, nkv, hd):
    print(f"[case] GQA nh={nh} nkv={nkv} hd={hd}", flush=True)
    cfg = dict(vocab_size=64, hidden_size=nh * hd, intermediate_size=256, n_layers=2,
               n_heads=nh, n_kv_heads=nkv, max_seq_len=160, rope_theta=500000.0,
               tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 7, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 7)
    prompt = orc.prompt_ids(3, 100, 64)
    ref_t, ref_l = om.generate_greedy(prompt, 20, mode=1, want_logits=True)
    (pt, pl), (kt, kl) = run_both(hip, hm, prompt, 20)
    assert max(rel_err(pl[i], ref_l[i]) for i in range(20)) < LOGIT_TOL
    assert max(rel_err(kl[i], ref_l[i]) for i in range(20)) < LOGIT_TOL
    assert (pt == ref_t).all() and (kt == ref_t).all()
    hm.free()
    om.close()
