"""Batched prefill on the matrix cores (LlamaModel::forward, llama.rs:683-700)
and the quantized GEMM behind it, against the CPU oracle on the same seeded
synthetic weights and token ids.

Bars: GEMM outputs within 1e-4 relative of the oracle's matmul_i8_f32 (the
activations enter the MFMAs as two bf16 terms, 2^-17 relative) and exact on
integer inputs; logits within 1e-3 relative per position; KV cache rows
written by the prefill within 1e-4 of the token-by-token decode path's;
greedy tokens identical with and without prefill.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32
LOGIT_TOL = 1e-3
GEMM_TOL = 1e-4
KV_TOL = 1e-4

TINY = dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
            n_kv_heads=6, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=True)


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def row_err(g, c):
    return max(rel_err(g[i], c[i]) for i in range(len(c)))


@pytest.mark.parametrize("m,k,n", [(17, 100, 300), (64, 288, 864), (130, 4096, 512),
                                   (300, 1000, 257), (257, 11008, 384)])
def test_gemm_matmul_i8_f32(hip, orc, m, k, n):
    """matmul_i8_f32 with m > 16 runs the MFMA GEMM: ragged M, N and K tails."""
    B = hip.HipBackend
    print(f"[case] gemm m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    q, s = orc.quantize_symmetric(w)
    orc.set_threads(8)
    ref = orc.matmul_i8_f32(a, q, s, m, k, n)
    orc.set_threads(0)
    out = B.matmul_i8_f32(B.from_vec(a), B.i8_from_vec(q), s, m, k, n).to_vec().reshape(m, n)
    err = rel_err(out, ref)
    print(f"[err] rel {err:.3e}", flush=True)
    assert err < GEMM_TOL


def test_gemm_exact_integers(hip):
    """A of small integers (exact in bf16, lo = 0), scale 1: integer sums exactly."""
    B = hip.HipBackend
    rng = np.random.default_rng(5)
    m, k, n = 96, 544, 300
    a = rng.integers(-3, 4, (m, k)).astype(F)
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    out = B.matmul_i8_f32(B.from_vec(a), B.i8_from_vec(q), 1.0, m, k, n).to_vec().reshape(m, n)
    ref = a.astype(np.int64) @ q.astype(np.int64)
    assert (out == ref).all()


def test_gemm_bias_and_block32(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(23)
    m, k, n = 40, 1024, 320
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    bias = rng.normal(0, 1, n).astype(F)
    q, s = orc.quantize_symmetric(w)
    ref = orc.matmul_i8_f32_bias(a, q, s, bias, m, k, n)
    out = B.matmul_i8_f32_bias(B.from_vec(a), B.i8_from_vec(q), s, B.from_vec(bias), m, k, n)
    assert rel_err(out.to_vec().reshape(m, n), ref) < GEMM_TOL
    q32, s32 = orc.quantize_block32(w, k, n)
    ref = orc.matmul_i8_f32_b32(a, q32, s32, m, k, n)
    out = B.matmul_i8_f32_block32(B.from_vec(a), B.i8_from_vec(q32), B.from_vec(s32), m, k, n)
    assert rel_err(out.to_vec().reshape(m, n), ref) < GEMM_TOL


def test_forward_tiny_vs_oracle(orc, hip):
    """Every position's logits of LlamaModel::forward (causal, no cache)."""
    print("[case] forward tiny seq 40", flush=True)
    orc.set_threads(8)
    om = orc.Llama(orc.LlamaConfig(**TINY), 0, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**TINY), 0)
    toks = orc.prompt_ids(1, 40, TINY["vocab_size"])
    ref = om.forward(toks)
    got = hm.forward(toks)
    err = row_err(got, ref)
    print(f"[err] forward rows {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    assert (got.argmax(1) == ref.argmax(1)).all()
    hm.free()
    om.close()
    orc.set_threads(0)


@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 4), (4, 1, 128), (16, 4, 64), (6, 6, 48), (8, 8, 32)])
def test_prefill_cache_matches_decode(orc, hip, nh, nkv, hd):
    """Prefill of 70 tokens: K/V rows equal the token-by-token path's, the last
    logits match the oracle's cache path."""
    print(f"[case] prefill vs decode nh={nh} nkv={nkv} hd={hd}", flush=True)
    cfg = dict(vocab_size=64, hidden_size=nh * hd, intermediate_size=256, n_layers=2, n_heads=nh,
               n_kv_heads=nkv, max_seq_len=160, rope_theta=500000.0, tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 7, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 7)
    toks = orc.prompt_ids(3, 70, 64)
    oc = om.new_cache(80)
    for p, t in enumerate(toks):
        ref_last = om.forward_with_cache(oc, t, p)
    cp = hm.new_llama_kv_cache(80)
    cd = hm.new_llama_kv_cache(80)
    last = hm.prefill([cp], toks[None, :])[0]
    for p, t in enumerate(toks):
        dec_last, _ = hm.forward_with_llama_cache(t, p, cd)
    assert cp.seq_len == 70 and cd.seq_len == 70
    n = 70 * nkv * hd
    for layer in range(2):
        kp, vp = cp.layer(layer)
        kd, vd = cd.layer(layer)
        assert rel_err(kp[:n], kd[:n]) < KV_TOL and rel_err(vp[:n], vd[:n]) < KV_TOL
    assert rel_err(last, ref_last) < LOGIT_TOL
    assert rel_err(last, dec_last) < LOGIT_TOL
    # decode continues from the prefilled cache like from the decoded one
    a, _ = hm.forward_with_llama_cache(5, 70, cp)
    b, _ = hm.forward_with_llama_cache(5, 70, cd)
    assert rel_err(a, b) < LOGIT_TOL
    cp.free()
    cd.free()
    hm.free()
    om.close()


def test_batched_prefill_ragged_starts(hip):
    """Two sequences in one prefill, one of them continuing a cache that already
    holds 9 rows, against each sequence prefilled alone."""
    cfg = hip.LlamaConfig(vocab_size=96, hidden_size=256, intermediate_size=512, n_layers=2,
                          n_heads=4, n_kv_heads=2, max_seq_len=128, rope_theta=10000.0,
                          tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(cfg, 11)
    rng = np.random.default_rng(2)
    head = rng.integers(0, 96, 9)
    seqs = rng.integers(0, 96, (2, 33))
    solo = []
    for i in range(2):
        c = hm.new_llama_kv_cache(64)
        if i == 1:
            hm.prefill([c], head[None, :], want_logits=False)
        solo.append(hm.prefill([c], seqs[i][None, :])[0])
        c.free()
    c0, c1 = hm.new_llama_kv_cache(64), hm.new_llama_kv_cache(64)
    hm.prefill([c1], head[None, :], want_logits=False)
    both = hm.prefill([c0, c1], seqs)
    assert c0.seq_len == 33 and c1.seq_len == 42
    assert rel_err(both[0], solo[0]) < 1e-5 and rel_err(both[1], solo[1]) < 1e-5
    c0.free()
    c1.free()
    hm.free()


def test_generate_with_prefill_tiny(orc, hip):
    """generate() with the prompt prefilled: the oracle's greedy tokens."""
    print("[case] generate tiny, 48-token prompt, prefill", flush=True)
    orc.set_threads(8)
    om = orc.Llama(orc.LlamaConfig(**TINY), 0, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**TINY), 0)
    prompt = orc.prompt_ids(1, 48, TINY["vocab_size"])
    ref_t, ref_l = om.generate_greedy(prompt, 32, mode=1, want_logits=True)
    pt, pl = hm.generate_greedy(prompt, 32, want_logits=True, prefill=True)
    kt, kl = hm.generate_greedy(prompt, 32, want_logits=True)
    e = max(rel_err(pl[i], ref_l[i]) for i in range(32))
    print(f"[err] prefill path vs oracle {e:.3e}", flush=True)
    assert e < LOGIT_TOL
    assert (pt == ref_t).all() and (kt == ref_t).all()
    hm.free()
    om.close()
    orc.set_threads(0)


def test_7b_dims_prefill_vs_decode(hip):
    """Config-4 shapes, 2 layers: a 300-token prefill (ragged M tile) against the
    token-by-token path: cache rows and the next 16 greedy tokens."""
    print("[case] 7B dims 2 layers prefill 300", flush=True)
    cfg = hip.LlamaConfig(vocab_size=32000, hidden_size=4096, intermediate_size=11008,
                          n_layers=2, n_heads=32, n_kv_heads=32, max_seq_len=2048,
                          rope_theta=10000.0, tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(cfg, 0)
    prompt = hip.synth.prompt_ids(1, 300, 32000)
    pt, pl = hm.generate_greedy(prompt, 16, want_logits=True, prefill=True)
    kt, kl = hm.generate_greedy(prompt, 16, want_logits=True)
    e = max(rel_err(pl[i], kl[i]) for i in range(16))
    print(f"[err] prefill vs token-by-token {e:.3e}", flush=True)
    assert e < LOGIT_TOL
    assert (pt == kt).all()
    hm.free()


def test_forward_block32_vs_oracle(orc, hip):
    """Block-32 scales through the prefill GEMM (the per-block scaled MFMA path)."""
    cfg = dict(TINY, n_layers=2)
    om = orc.Llama(orc.LlamaConfig(**cfg), 0, quantize=True, block32=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 0, hip.QUANT_BLOCK32)
    toks = orc.prompt_ids(2, 24, cfg["vocab_size"])
    orc.set_threads(8)
    ref = om.forward(toks, mode=2)  # mode 2: the oracle's block-32 arithmetic
    orc.set_threads(0)
    got = hm.forward(toks)
    err = row_err(got, ref)
    print(f"[err] block-32 forward {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    hm.free()
    om.close()


@pytest.mark.parametrize("seq", [1, 129])
def test_forward_single_and_ragged_rows(orc, hip, seq):
    """seq = 1 (one GEMM row) and 129 (one row past the 128-row tile)."""
    cfg = dict(vocab_size=96, hidden_size=256, intermediate_size=320, n_layers=2, n_heads=4,
               n_kv_heads=2, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 5, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 5)
    toks = orc.prompt_ids(4, seq, 96)
    assert row_err(hm.forward(toks), om.forward(toks)) < LOGIT_TOL
    hm.free()
    om.close()


def test_prefill_after_decode_positions(orc, hip):
    """A cache filled token by token for 5 positions, then 20 more by prefill:
    the last logits equal the oracle's all-token-by-token path."""
    cfg = dict(vocab_size=80, hidden_size=192, intermediate_size=256, n_layers=2, n_heads=6,
               n_kv_heads=3, max_seq_len=64, rope_theta=10000.0, tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 9, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 9)
    toks = orc.prompt_ids(6, 25, 80)
    oc = om.new_cache(32)
    for p, t in enumerate(toks):
        ref = om.forward_with_cache(oc, t, p)
    c = hm.new_llama_kv_cache(32)
    for p in range(5):
        hm.forward_with_llama_cache(int(toks[p]), p, c)
    last = hm.prefill([c], toks[None, 5:])[0]
    assert c.seq_len == 25
    assert rel_err(last, ref) < LOGIT_TOL
    c.free()
    hm.free()
    om.close()


def test_prefill_argument_errors(hip):
    cfg = hip.LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=128, n_layers=1,
                          n_heads=2, n_kv_heads=2, max_seq_len=32, rope_theta=10000.0,
                          tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(cfg, 1)
    c = hm.new_llama_kv_cache(16)
    with pytest.raises(hip.ScryHipError) as ei:  # past the cache capacity
        hm.prefill([c], np.zeros((1, 17), np.int64))
    assert "exceed" in str(ei.value)
    with pytest.raises(hip.ScryHipError):  # token id out of range
        hm.prefill([c], np.full((1, 4), 64, np.int64))
    with pytest.raises(hip.ScryHipError):  # the same cache twice
        hm.prefill([c, c], np.zeros((2, 4), np.int64))
    many = [hm.new_llama_kv_cache(8) for _ in range(17)]
    with pytest.raises(hip.ScryHipError):  # more sequences than one prefill takes
        hm.prefill(many, np.zeros((17, 2), np.int64))
    assert c.seq_len == 0  # failed calls leave the cache untouched
    for x in many:
        x.free()
    c.free()
    hm.free()


def test_generate_prefill_one_token_prompt(hip):
    """A one-token prompt has nothing to prefill: both paths are the same run."""
    cfg = hip.LlamaConfig(**TINY)
    hm = hip.LlamaModel.new_random(cfg, 0)
    a = hm.generate_greedy([17], 12, prefill=True)
    b = hm.generate_greedy([17], 12)
    assert (a == b).all()
    hm.free()


def test_llama3_rope_scaling_decode_and_forward(orc, hip):
    """Llama-3 RoPE frequency scaling (compute_rope_freqs, llama.rs:1035-1067)
    with GQA: greedy decode and the batched forward against the oracle."""
    cfg = dict(vocab_size=128, hidden_size=256, intermediate_size=384, n_layers=2, n_heads=4,
               n_kv_heads=1, max_seq_len=128, rope_theta=500000.0, tie_word_embeddings=False,
               rope_scaling=(8.0, 1.0, 4.0, 64))
    om = orc.Llama(orc.LlamaConfig(**cfg), 13, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 13)
    prompt = orc.prompt_ids(7, 40, 128)
    ref_t, ref_l = om.generate_greedy(prompt, 16, mode=1, want_logits=True)
    got_t, got_l = hm.generate_greedy(prompt, 16, want_logits=True, prefill=True)
    assert max(rel_err(got_l[i], ref_l[i]) for i in range(16)) < LOGIT_TOL
    assert (got_t == ref_t).all()
    assert row_err(hm.forward(prompt), om.forward(prompt)) < LOGIT_TOL
    hm.free()
    om.close()
