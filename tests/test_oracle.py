"""Pins the CPU oracle (oracle/oracle.c) to the reference: the reference's own
known-answer tests (cited file:line), hand-derived values that a plausible
transcription mistake would change, and mathematical properties.  CPU only."""
import math

import numpy as np
import pytest

F = np.float32
T24 = float(2 ** 24)


# ------------------------------------------------ quantize.rs:16-40, 46-83
def test_quantize_roundtrip_accuracy_kat(orc):
    # quantize.rs:46-65
    w = np.array([i * 0.1 for i in range(-100, 101)], F)
    q, s = orc.quantize_symmetric(w)
    r = orc.dequantize(q, s)
    tol = np.abs(w).max() / F(127)
    assert np.abs(w - r).max() <= tol + 1e-6


def test_quantize_zero_weights_kat(orc):
    # quantize.rs:67-73
    q, s = orc.quantize_symmetric(np.zeros(10, F))
    assert (q == 0).all() and s == 0.0


def test_quantize_clamps_kat(orc):
    # quantize.rs:75-83
    q, _ = orc.quantize_symmetric(np.array([1000.0, -1000.0, 0.0], F))
    assert q.tolist() == [127, -127, 0]


def test_quantize_round_half_away_from_zero(orc):
    # absmax 127 -> scale 1, inv 1: w*inv lands exactly on .5 (f32::round is
    # half-away-from-zero; banker's rounding would give 2, -2, 0, 0, 2, -2)
    w = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5], F)
    q, s = orc.quantize_symmetric(w)
    assert s == F(1.0)
    assert q.tolist() == [127, 3, -3, 1, -1, 2, -2]


def test_quantize_uses_multiply_by_inverse(orc):
    # quantize.rs:24-29 multiplies by inv = 1/scale; w/scale rounds differently
    # for some inputs.  Find such an input and check the oracle follows w*inv.
    rng = np.random.default_rng(0)
    found = 0
    for _ in range(200):
        w = rng.normal(0, 0.02, 4096).astype(F)
        absmax = np.abs(w).max()
        scale = F(absmax) / F(127)
        inv = F(1) / scale
        def half_away(x):  # x: f32 values, exact in f64
            x = x.astype(np.float64)
            return np.clip(np.sign(x) * np.floor(np.abs(x) + 0.5), -127, 127)

        mul = half_away((w * inv).astype(F))
        div = half_away((w / scale).astype(F))
        idx = np.nonzero(mul != div)[0]
        if len(idx):
            q, s = orc.quantize_symmetric(w)
            assert s == scale
            for i in idx:
                assert q[i] == mul[i] != div[i]
            found += len(idx)
        if found >= 3:
            break
    assert found >= 1


def test_quantize_nan_and_inf(orc):
    # f32::max ignores NaN in the absmax fold; `as i8` maps NaN to 0
    q, s = orc.quantize_symmetric(np.array([np.nan, 1.0, -0.5], F))
    assert s == F(1.0) / F(127)
    assert q.tolist() == [0, 127, -64]  # -0.5*127 = -63.5 -> -64 (half away)
    # absmax = inf -> scale inf, inv 0: inf*0 = NaN -> 0, finite*0 = 0
    q, s = orc.quantize_symmetric(np.array([np.inf, 1.0, -3.0], F))
    assert math.isinf(s) and q.tolist() == [0, 0, 0]


def test_quantize_properties(orc):
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, 10000).astype(F)
    q, s = orc.quantize_symmetric(w)
    qn, sn = orc.quantize_symmetric(-w)
    assert sn == s and (qn == -q).all()  # odd symmetry
    q4, s4 = orc.quantize_symmetric(w * F(4))
    assert s4 == s * F(4) and (q4 == q).all()  # power-of-two scale invariance
    assert np.abs(q).max() == 127  # the absmax element maps to +-127
    assert np.abs(orc.dequantize(q, s) - w).max() <= s / 2 * (1 + 1e-6)


def test_quantize_block32_is_per_block_symmetric(orc):
    rng = np.random.default_rng(2)
    k, n = 100, 7  # ragged last block
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    q, sc = orc.quantize_block32(w, k, n)
    q = q.reshape(k, n)
    nb = (k + 31) // 32
    sc = sc.reshape(n, nb)
    for j in range(n):
        for b in range(nb):
            blk = w[32 * b: 32 * b + 32, j]
            qb, sb = orc.quantize_symmetric(blk)
            assert sb == sc[j, b]
            assert (qb == q[32 * b: 32 * b + 32, j]).all()


# --------------------------------------- cpu.rs:1128-1160 matmul_i8_f32_tiled
def test_matmul_i8_matches_f32_kat(orc):
    # cpu.rs:1699-1728
    m, k, n = 4, 8, 3
    a = np.array([i * 0.1 - 1.5 for i in range(m * k)], F)
    b = np.array([i * 0.05 - 0.6 for i in range(k * n)], F)
    ref = orc.matmul_f32(a, b, m, k, n)
    q, s = orc.quantize_symmetric(b)
    c = orc.matmul_i8_f32(a, q, s, m, k, n)
    tol = np.abs(b).max() / 127 * k * 0.5
    assert np.abs(ref - c).max() < tol


def test_matmul_i8_bias_kat(orc):
    # cpu.rs:1730-1756
    m, k, n = 2, 4, 3
    a = np.array([i * 0.1 for i in range(m * k)], F)
    b = np.array([i * 0.05 for i in range(k * n)], F)
    bias = np.array([1.0, 2.0, 3.0], F)
    ref = orc.matmul_f32(a, b, m, k, n) + bias
    q, s = orc.quantize_symmetric(b)
    c = orc.matmul_i8_f32_bias(a, q, s, bias, m, k, n)
    assert np.abs(ref - c).max() < np.abs(b).max() / 127 * k * 0.5


def test_matmul_i8_exact_integer_cases(orc):
    rng = np.random.default_rng(3)
    k, n = 37, 11
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    # ones row -> column sums (exact in f32 for these magnitudes)
    c = orc.matmul_i8_f32(np.ones((1, k), F), q, 1.0, 1, k, n)
    assert (c[0] == q.astype(np.int64).sum(0)).all()
    # identity rows pick out rows of q (pins row/column indexing)
    c = orc.matmul_i8_f32(np.eye(k, dtype=F), q, 0.5, k, k, n)
    assert (c == q.astype(F) * F(0.5)).all()


def test_matmul_i8_sequential_f32_accumulation(orc):
    # per element the reference adds f32 products left to right in p:
    # 2^24 + 1 rounds back to 2^24, so the sum is 0 (an f64 accumulator gives 1)
    a = np.array([[T24, 1.0, -T24]], F)
    q = np.array([[1], [1], [1]], np.int8)
    assert orc.matmul_i8_f32(a, q, 1.0, 1, 3, 1)[0, 0] == 0.0
    assert orc.matmul_i8_f32(a, q, 1.0, 1, 3, 1, faithful=True)[0, 0] == 0.0
    # LM-head form (weights stored [n,k]) follows the same rule
    assert orc.matmul_i8_f32_tb(a, q.reshape(1, 3), 1.0, 1, 3, 1)[0, 0] == 0.0


def test_matmul_i8_product_rounded_once(orc):
    # c += f32(f64(a) * (f64(q) * f64(scale))): the product is formed in f64
    # and rounded once.  a = 1 + 2^-23, q = 3, scale = 1 + 2^-23:
    # exact product 3 * (1 + 2^-23)^2 = 3 + 6*2^-23 + 3*2^-46 -> f32 nearest is
    # 3 + 2^-21 * 3 (= 3 + 6*2^-23, spacing 2^-22 near 3).  Rounding q*scale to
    # f32 first (3 + 2^-21) and then multiplying gives 3 + 2^-20 instead.
    e = 2.0 ** -23
    a = np.array([[1 + e]], F)
    q = np.array([[3]], np.int8)
    c = orc.matmul_i8_f32(a, q, F(1 + e), 1, 1, 1)[0, 0]
    assert c == F(3 + 6 * e)
    assert c != F(3 + 2.0 ** -20)


def test_matmul_i8_brute_force_and_parallel_identity(orc):
    rng = np.random.default_rng(4)
    for (m, k, n) in [(1, 288, 864), (3, 100, 65), (5, 33, 17), (16, 70, 130)]:
        a = rng.normal(0, 1, (m, k)).astype(F)
        w = rng.normal(0, 0.02, (k, n)).astype(F)
        q, s = orc.quantize_symmetric(w)
        q = q.reshape(k, n)
        exact = a.astype(np.float64) @ (q.astype(np.float64) * float(s))
        orc.set_threads(0)
        c0 = orc.matmul_i8_f32(a, q, s, m, k, n, faithful=True)
        orc.set_threads(4)
        c1 = orc.matmul_i8_f32(a, q, s, m, k, n)
        orc.set_threads(0)
        assert (c0 == c1).all()  # tiled == column-parallel, bit for bit
        assert np.abs(c0 - exact).max() <= 1e-5 * np.abs(exact).max()
        # transposed storage gives the same numbers
        ct = orc.matmul_i8_f32_tb(a, np.ascontiguousarray(q.T), s, m, k, n)
        assert (ct == c0).all()


def test_matmul_i8_block32(orc):
    rng = np.random.default_rng(5)
    m, k, n = 2, 96, 10
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    q, sc = orc.quantize_block32(w, k, n)
    c = orc.matmul_i8_f32_b32(a, q, sc, m, k, n)
    deq = q.reshape(k, n).astype(np.float64) * np.repeat(sc.reshape(n, -1).T, 32, 0)[:k]
    exact = a.astype(np.float64) @ deq
    assert np.abs(c - exact).max() <= 1e-5 * np.abs(exact).max()
    # block-32 error is below per-tensor error on the same weights
    qt, st = orc.quantize_symmetric(w)
    ref = a.astype(np.float64) @ w.astype(np.float64)
    ct = orc.matmul_i8_f32(a, qt, st, m, k, n)
    assert np.abs(c - ref).max() < np.abs(ct - ref).max()


# ------------------------------------------------------ f32 GEMV order
def test_matmul_identity_kat(orc):
    # cpu.rs:1476-1481
    c = orc.matmul_f32(np.array([1, 0, 0, 1], F), np.array([1, 2, 3, 4], F), 2, 2, 2)
    assert c.ravel().tolist() == [1, 2, 3, 4]


def test_gemv_f32_left_to_right_groups(orc):
    # out += ((v0*r0 + v1*r1) + v2*r2) + v3*r3: 2^24 + 1 + 1 + 1 stays 2^24;
    # a pairwise grouping would give 2^24 + 2
    v = np.array([T24, 1, 1, 1], F)
    assert orc.gemv_f32(v, np.ones((4, 1), F), 4, 1)[0] == T24
    assert orc.gemv_into(v, np.ones((4, 1), F), 4, 1)[0] == T24


def test_gemv_trans_b_four_partials(orc):
    # cpu.rs:825-842: partial a0 takes p = 0, 4: 1 + 2^24 -> 2^24 (tie to even),
    # then ((a0 + a1) + a2) + a3 with a1..a3 = 1 stays 2^24.  A single
    # left-to-right sum would give 4 + 2^24.
    v = np.array([1, 1, 1, 1, T24, 0, 0, 0], F)
    assert orc.gemv_trans_b(v, np.ones(8, F), 8, 1)[0] == T24
    seq = F(0)
    for x in v:
        seq = F(seq + x)
    assert seq == F(T24 + 4)


def test_strided_batched_matches_per_head(orc):
    # cpu.rs:1633-1660 (batched == per-slice matmul)
    rng = np.random.default_rng(6)
    b, k, n = 3, 8, 5
    a = rng.normal(size=(b, 1, k)).astype(F)
    bt = rng.normal(size=(b, n, k)).astype(F)
    c = orc.matmul_strided_batched(a, bt, b, 1, k, n, trans_b=True).reshape(b, n)
    for i in range(b):
        assert (c[i] == orc.gemv_trans_b(a[i, 0], bt[i], k, n)).all()
        assert np.allclose(c[i], bt[i] @ a[i, 0], rtol=1e-5)


# ------------------------------------------------------------ glue ops
def test_rmsnorm_kat(orc):
    # cpu.rs:1500-1511
    out = orc.rmsnorm(np.array([1, 2, 3, 4], F), np.ones(4, F), 1, 4, 1e-5)
    rstd = 1.0 / math.sqrt(7.5 + 1e-5)
    assert np.abs(out - np.arange(1, 5) * rstd).max() < 1e-5
    # the weight multiplies element-wise; rows are independent
    w = np.array([1, 2, 0.5, -1], F)
    x = np.array([[1, 2, 3, 4], [0, 0, 0, 2]], F)
    out = orc.rmsnorm(x, w, 2, 4, 1e-5).reshape(2, 4)
    exp = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.abs(out - exp).max() < 1e-6


def test_rope_kat_and_textbook_rotation(orc):
    # cpu.rs:1538-1548: pair (1, 0) at pos 1 rotated by angle 1
    freqs = orc.compute_rope_freqs(4, 10000.0).astype(F)
    out = orc.rope_with_freqs_preloaded(np.array([1, 0, 1, 0], F), 1, 1, 4, 1, freqs)
    assert abs(out[0] - 0.5403) < 1e-3 and abs(out[1] - 0.8415) < 1e-3
    # interleaved pairs (2i, 2i+1) rotate as complex numbers by pos*freq_i
    rng = np.random.default_rng(7)
    seq, nh, hd, p0 = 3, 2, 8, 5
    freqs = orc.compute_rope_freqs(hd, 10000.0).astype(F)
    x = rng.normal(size=(seq, nh, hd)).astype(F)
    out = orc.rope_with_freqs_preloaded(x, seq, nh, hd, p0, freqs).reshape(seq, nh, hd // 2, 2)
    z = x.reshape(seq, nh, hd // 2, 2).astype(np.float64)
    zc = z[..., 0] + 1j * z[..., 1]
    ang = (p0 + np.arange(seq))[:, None, None] * freqs.astype(np.float64)[None, None, :]
    r = zc * np.exp(1j * ang)
    assert np.abs(out[..., 0] - r.real).max() < 1e-5
    assert np.abs(out[..., 1] - r.imag).max() < 1e-5


def test_rope_freqs(orc):
    f = orc.compute_rope_freqs(4, 10000.0)
    assert f[0] == 1.0 and abs(f[1] - 0.01) < 1e-15
    hd = 64
    plain = orc.compute_rope_freqs(hd, 500000.0)
    assert np.allclose(plain, 1.0 / 500000.0 ** (np.arange(0, hd, 2) / hd), rtol=1e-14)
    # Llama-3 scaling (llama.rs:37-44 preset): short wavelengths untouched,
    # long ones divided by the factor, monotone in between
    sc = orc.compute_rope_freqs(hd, 500000.0, (32.0, 1.0, 4.0, 8192))
    wl = 2 * np.pi / plain
    assert (sc[wl < 8192 / 4] == plain[wl < 8192 / 4]).all()
    assert np.allclose(sc[wl > 8192] * 32.0, plain[wl > 8192], rtol=1e-14)
    assert (np.diff(sc) < 0).all()


def test_softmax_kat(orc):
    # cpu.rs:1483-1492
    out = orc.softmax(np.array([1, 2, 3], F), 1, 3)
    assert abs(out.sum() - 1) < 1e-6 and out[2] > out[1] > out[0]
    x = np.array([[1000, 1001, -np.inf], [0, 0, 0]], F)
    out = orc.softmax(x, 2, 3).reshape(2, 3)
    e = np.exp(np.array([0, 1.0]))
    assert np.allclose(out[0, :2], e / e.sum(), rtol=1e-6) and out[0, 2] == 0
    assert np.allclose(out[1], 1 / 3, rtol=1e-6)


def test_silu_swiglu_kat(orc):
    # cpu.rs:1513-1522
    out = orc.swiglu(np.array([0, 1, -1], F), np.ones(3, F))
    assert abs(out[0]) < 1e-6 and abs(out[1] - 0.7311) < 1e-3 and abs(out[2] + 0.2689) < 1e-3
    assert abs(orc.silu(2.0) - 2.0 / (1.0 + math.exp(-2.0))) < 1e-7
    out = orc.swiglu(np.array([1.0, 2.0], F), np.array([2.0, -0.5], F))
    assert np.allclose(out, [2 * 0.7310586, -0.5 * 1.7615942], rtol=1e-6)


def test_repeat_kv_kats(orc):
    # cpu.rs:1524-1536
    x = np.array([1, 2, 3, 4], F)
    assert orc.repeat_kv(x, 1, 1, 2, 2).tolist() == [1, 2, 3, 4]
    assert orc.repeat_kv(x, 1, 2, 2, 2).tolist() == [1, 2, 3, 4, 1, 2, 3, 4]


def test_gather_reshape_repeat_kv_matches_three_step(orc):
    # cpu.rs:1662-1697: == gather_rows -> reshape_for_heads -> repeat_kv
    rng = np.random.default_rng(8)
    max_seq, L, nkv, nq, hd = 10, 6, 2, 8, 4
    cache = rng.normal(size=(max_seq, nkv * hd)).astype(F)
    out = orc.gather_reshape_repeat_kv(cache, max_seq, L, nkv, nq, hd).reshape(nq, L, hd)
    heads = cache[:L].reshape(L, nkv, hd).transpose(1, 0, 2)  # [nkv, L, hd]
    exp = np.repeat(heads, nq // nkv, axis=0)
    assert (out == exp).all()
    assert (orc.repeat_kv(heads, nkv, nq, L, hd).reshape(nq, L, hd) == exp).all()


def test_embedding(orc):
    w = np.arange(12, dtype=F).reshape(4, 3)
    assert orc.embedding(w, [2, 0], 4, 3).tolist() == [6, 7, 8, 0, 1, 2]
    with pytest.raises(IndexError):
        orc.embedding(w, [4], 4, 3)


def test_causal_mask_scale(orc):
    s = np.ones((2, 3, 3), F)
    out = orc.causal_mask_scale(s, 2, 3, 0.5, -np.inf).reshape(2, 3, 3)
    assert (np.isneginf(out) == np.triu(np.ones((3, 3), bool), 1)).all()
    assert (out[np.isfinite(out)] == 0.5).all()


def test_argmax_max_by_semantics(orc):
    # generate.rs:167-173: Iterator::max_by returns the LAST of equal maxima;
    # partial_cmp of NaN is mapped to Equal, which also hands over to the
    # later element
    assert orc.argmax([1, 3, 3, 2]) == 2
    assert orc.argmax([5]) == 0
    assert orc.argmax(np.array([], F)) == 0
    assert orc.argmax([1, np.nan, 0.5]) == 2
    assert orc.argmax([3, np.nan, 1, 2]) == 3
    assert orc.argmax([2, np.nan]) == 1
    assert orc.argmax([np.nan, np.nan]) == 1
    assert orc.argmax([-np.inf, -np.inf]) == 1


# ------------------------------------------- fastrand + Box-Muller (unpinned)
def test_rng_stream_properties(orc):
    """fastrand 2.3.0 parity is UNPINNED (no reference test fixes a value);
    this only checks the restatement is self-consistent and well formed."""
    u = orc.rng_f64(0, 0, 100000)
    assert (u >= 0).all() and (u < 1).all() and abs(u.mean() - 0.5) < 0.005
    assert orc.rng_u64(7, 10, 5).tolist() == [int(orc.lib().orc_rng_u64_at(7, 10 + i))
                                               for i in range(5)]
    seq = orc.normal_vec(0, 3, 200001)
    par = orc.normal_vec(0, 3, 200001, par=True)
    assert (seq == par).all()
    assert abs(seq.mean()) < 2e-4 and abs(seq.std() - 0.02) < 2e-4


# ------------------------------------------------- llama.rs invariants
SMOKE = dict(vocab_size=32, hidden_size=16, intermediate_size=32, n_layers=2, n_heads=4,
             n_kv_heads=2, max_seq_len=64, rope_theta=500000.0, tie_word_embeddings=True)


def _model(orc, seed=42, **kw):
    cfg = orc.LlamaConfig(**{**SMOKE, **kw})
    return orc.Llama(cfg, seed, quantize=True, keep_f32=True)


def test_llama_rng_order_consumes_every_parameter(orc):
    m = _model(orc)
    c = m.cfg
    hd = c.head_dim
    n = (c.vocab_size * c.hidden_size + c.n_layers * (
        c.hidden_size * (c.n_heads + 2 * c.n_kv_heads) * hd + c.n_heads * hd * c.hidden_size
        + 3 * c.hidden_size * c.intermediate_size))
    assert m.rng_calls == 2 * n
    # embed_tokens is the first tensor drawn (llama.rs:602-605)
    assert (m.tensor(orc.T_EMBED) == orc.normal_vec(42, 0, c.vocab_size * c.hidden_size)).all()


@pytest.mark.parametrize("mode", [0, 1])
def test_llama_cache_matches_full_forward(orc, mode):
    # tests/llama_smoke.rs:102-128 (1e-3 abs), for the f32 and int8 compositions
    m = _model(orc)
    toks = [3, 7, 1]
    full = m.forward(toks, mode=mode)
    c = m.new_cache(64)
    for pos, t in enumerate(toks):
        last = m.forward_with_cache(c, t, pos, mode=mode)
    assert np.abs(full[-1] - last).max() < 1e-3
    assert np.isfinite(full).all()


@pytest.mark.parametrize("nh,nkv", [(4, 4), (4, 2), (4, 1), (8, 2)])
def test_llama_gqa_ratios(orc, nh, nkv):
    # tests/llama_smoke.rs:268-305
    m = _model(orc, vocab_size=16, hidden_size=nh * 4, intermediate_size=32, n_layers=1,
               n_heads=nh, n_kv_heads=nkv, max_seq_len=32, rope_theta=10000.0)
    full = m.forward([0, 1, 2], mode=1)
    assert np.isfinite(full).all()
    c = m.new_cache(32)
    for pos in range(3):
        lg = m.forward_with_cache(c, pos, pos, mode=1)
        assert np.isfinite(lg).all()
    assert np.abs(full[-1] - lg).max() < 1e-3


def test_llama_greedy_determinism_and_quant_error(orc):
    # tests/llama_smoke.rs:149-169
    m = _model(orc)
    a = m.generate_greedy([0, 1], 8, mode=1)
    b = m.generate_greedy([0, 1], 8, mode=1)
    assert len(a) == 8 and (a == b).all()
    # max_tokens = 0 still returns the token sampled after the prompt
    assert len(m.generate_greedy([0, 1], 0, mode=1)) == 1
    # the int8 composition stays close to the f32 reference forward
    lf = m.forward([3, 7, 1], mode=0)
    lq = m.forward([3, 7, 1], mode=1)
    assert np.abs(lf - lq).max() < 0.05 * np.abs(lf).max()


def test_llama_loaded_norm_weights_and_eps(orc):
    """from_safetensors norms (llama.rs:880-914, 936-940): a final-norm weight
    of 2 doubles every logit exactly (x2 commutes with each rounding on the
    path: f64 RMSNorm product, f64 int8 products, f32 sums); eps and the
    per-layer weights are used (the logits move)."""
    m = _model(orc)
    h = m.cfg.hidden_size
    toks = [3, 7, 1, 9]
    base = m.forward(toks, mode=1)
    m.set_norm(2, 0, np.full(h, 2.0, np.float32), 1e-5)
    assert np.array_equal(m.forward(toks, mode=1), 2 * base)
    c = m.new_cache(16)
    step = [m.forward_with_cache(c, t, p, mode=1) for p, t in enumerate(toks)]
    assert np.abs(step[-1] - 2 * base[-1]).max() < 2e-3 * np.abs(base).max()
    m.set_norm(2, 0, np.ones(h, np.float32), 1e-5)
    assert np.array_equal(m.forward(toks, mode=1), base)
    m.set_norm(0, 1, np.linspace(0.5, 1.5, h, dtype=np.float32), 1e-5)
    moved = m.forward(toks, mode=1)
    assert not np.array_equal(moved, base)
    m.set_norm(0, 1, np.ones(h, np.float32), 0.25)  # eps alone
    assert not np.array_equal(m.forward(toks, mode=1), base)
    with pytest.raises(ValueError):
        m.set_norm(0, 5, np.ones(h, np.float32), 1e-5)


# ------------------------------------------------ sampling (generate.rs:92-186)
def _sample_py(logits, t, k, p, r):
    """generate.rs:92-186 in plain Python (f64, sequential sums), ties in the
    sorts broken by the smaller index."""
    n = len(logits)
    sc = [float(x) / float(np.float32(t)) for x in logits]
    if 0 < k < n:
        thr = sorted(sc, reverse=True)[k - 1]
        sc = [-math.inf if v < thr else v for v in sc]
    mx = max(sc)
    pr = [math.exp(v - mx) for v in sc]
    s = 0.0
    for v in pr:
        s += v
    pr = [v / s for v in pr] if s > 0 else [1.0 / n] * n
    pf = float(np.float32(p))
    if 0.0 < pf < 1.0:
        order = sorted(range(n), key=lambda i: (-pr[i], i))
        cum, cut = 0.0, n
        for j, i in enumerate(order):
            cum += pr[i]
            if cum >= pf:
                cut = j + 1
                break
        keep = set(order[:cut])
        pr = [v if i in keep else 0.0 for i, v in enumerate(pr)]
        s2 = 0.0
        for v in pr:
            s2 += v
        if s2 > 0:
            pr = [v / s2 for v in pr]
    cum = 0.0
    for i, v in enumerate(pr):
        cum += v
        if r < cum:
            return i
    return n - 1


@pytest.mark.parametrize("t,k,p", [(1.0, 0, 1.0), (0.7, 3, 1.0), (1.3, 0, 0.6), (0.9, 4, 0.8),
                                   (2.0, 7, 0.3), (1.0, 1, 1.0)])
def test_sample_token_matches_plain_restatement(orc, t, k, p):
    rng = np.random.default_rng(int(t * 100) + k)
    for seed in range(40):
        logits = rng.normal(0, 2, 9).astype(np.float32)
        logits[seed % 9] = logits[(seed + 4) % 9]  # a tie somewhere
        r = float(orc.rng_f64(seed, 0, 1)[0])
        tok, st = orc.sample_token(logits, t, k, p, seed)
        assert tok == _sample_py(logits, t, k, p, r), (seed, logits)
        assert st == (seed + 0x2D358DCCAA6C78A5) % 2**64  # one rng call per sample


def test_sample_token_edge_cases(orc):
    lg = np.array([0.5, 2.0, -1.0, 2.0, 1.5], np.float32)
    # temperature < 1e-8: argmax (last of equal maxima), no rng call
    assert orc.sample_token(lg, 0.0, 0, 1.0, 5) == (3, 5)
    assert orc.sample_token(lg, 9e-9, 3, 0.5, 5) == (3, 5)
    # top_k = 1 keeps every value equal to the largest: only 1 and 3 remain
    for seed in range(20):
        assert orc.sample_token(lg, 1.0, 1, 1.0, seed)[0] in (1, 3)
    # a tiny top_p keeps only the first entry of the descending order (index 1)
    for seed in range(20):
        assert orc.sample_token(lg, 1.0, 0, 1e-6, seed)[0] == 1
    # every scaled logit -inf: the sum is NaN, not > 0, so the draw is uniform
    ninf = np.full(4, -np.inf, np.float32)
    for seed in range(20):
        r = float(orc.rng_f64(seed, 0, 1)[0])
        assert orc.sample_token(ninf, 1.0, 0, 1.0, seed)[0] == min(int(r * 4), 3)


def test_f32_to_bf16_matches_torch_rounding(orc):
    """The bf16 feature's cast (kernels.rs:629-633) is round-to-nearest-even:
    torch's independent f32 -> bfloat16 conversion gives the same words for
    every non-NaN input (ties, subnormals, overflow to inf, signed zeros)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(17)
    bits = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2**16, 2000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000  # exact ties
    special = np.array([0, 0x80000000, 1, 0x807FFFFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F800000,
                        0xFF800000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x00008000, 0x00018000], np.uint32)
    x = np.concatenate([bits, ties, special]).view(np.float32)
    x = x[~np.isnan(x)]
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), want)
    # NaN inputs follow the reference's integer arithmetic (no NaN branch)
    nan = np.array([0x7FC00000, 0x7F800001, 0xFFFFFFFF, 0x7FFF0000], np.uint32).view(np.float32)
    assert orc.f32_to_bf16(nan).tolist() == [0x7FC0, 0x7F80, 0x0000, 0x7FFF]


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_matmul_bf16_oracle(orc, ta, tb):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3 + 2 * ta + tb)
    m, k, n = 5, 37, 11
    # bf16-representable integers: every product and sum exact
    ai = rng.integers(-100, 100, (m, k)).astype(np.float32)
    bi = rng.integers(-100, 100, (k, n)).astype(np.float32)
    A = ai.T.copy() if ta else ai
    Bm = bi.T.copy() if tb else bi
    assert np.array_equal(orc.matmul_bf16(A, Bm, m, k, n, ta, tb), ai @ bi)
    # random values: torch's bf16 rounding, then an f64 product
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1, (k, n)).astype(np.float32)
    ab = torch.from_numpy(a).to(torch.bfloat16).to(torch.float64).numpy()
    bb = torch.from_numpy(b).to(torch.bfloat16).to(torch.float64).numpy()
    want = (ab @ bb).astype(np.float32)
    got = orc.matmul_bf16(a.T.copy() if ta else a, b.T.copy() if tb else b, m, k, n, ta, tb)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    assert not np.array_equal(got, a @ b)  # the rounding of the operands is there


@pytest.mark.parametrize("m,k,n,tb", [(1, 300, 700, False), (3, 129, 257, False), (2, 64, 513, True),
                                      (5, 37, 11, True)])
def test_matmul_bf16_par_bit_identical(orc, m, k, n, tb):
    """The all-core bf16 matmul (forward mode 3) sums the same exact products
    in the same order as the pinned scalar one: equal bit for bit."""
    rng = np.random.default_rng(m * 1000 + k)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1, (n, k) if tb else (k, n)).astype(np.float32)
    orc.set_threads(4)
    try:
        got = orc.matmul_bf16_par(a, b, m, k, n, tb)
    finally:
        orc.set_threads(0)
    want = orc.matmul_bf16(a, b, m, k, n, False, tb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_forward_mode3_is_the_bf16_composition(orc):
    """Forward mode 3 (the bf16 feature) runs the mode-0 composition with
    every projection through matmul_bf16_par (pinned above and against
    torch's bf16 rounding): on a tiny model the two modes differ by the bf16
    rounding of the operands only."""
    cfg = orc.LlamaConfig(vocab_size=64, hidden_size=32, intermediate_size=64, n_layers=2, n_heads=4,
                          n_kv_heads=2, max_seq_len=16, rope_theta=10000.0, tie_word_embeddings=False)
    m = orc.Llama(cfg, 5, quantize=False)
    try:
        toks = np.array([1, 7, 3, 60], np.int64)
        l0 = m.forward(toks, mode=0)
        l3 = m.forward(toks, mode=3)
    finally:
        m.close()
    rel = np.abs(l3 - l0).max() / np.abs(l0).max()
    assert 1e-5 < rel < 3e-2, rel  # bf16 operands: ~2^-8 relative per product
    assert (np.argmax(l3, -1) == np.argmax(l0, -1)).mean() >= 0.75


# ------------------------------------------------- distribution of sample_token
def _closed_form_probs(logits, t, k, p):
    """generate.rs:92-165 written from its definition: keep the k largest of
    logits / t, softmax over the kept ones, then keep the smallest
    most-probable prefix whose mass reaches p and renormalise."""
    z = np.asarray(logits, np.float64) / np.float64(np.float32(t))
    order = np.argsort(-z, kind="stable")
    keep = np.zeros(z.size, bool)
    keep[order[: (k if 0 < k < z.size else z.size)]] = True
    e = np.where(keep, np.exp(z - z[keep].max()), 0.0)
    pr = e / e.sum()
    pf = float(np.float32(p))
    if 0.0 < pf < 1.0:
        o2 = np.argsort(-pr, kind="stable")
        cut = int(np.searchsorted(np.cumsum(pr[o2]), pf)) + 1
        pr2 = np.zeros_like(pr)
        pr2[o2[:cut]] = pr[o2[:cut]]
        pr = pr2 / pr2.sum()
    return pr


@pytest.mark.parametrize("t,k,p", [(0.8, 4, 1.0), (1.3, 0, 0.7), (0.9, 5, 0.85), (1.0, 0, 1.0)])
def test_sample_token_distribution_chi_square(orc, t, k, p):
    """Token frequencies over 100000 rng states against the closed-form
    kept-and-renormalised probabilities (Pearson chi-square).  A wrong
    temperature direction, an off-by-one in the top-k or top-p cut, or a
    missing renormalisation moves the frequencies far outside the test."""
    stats = pytest.importorskip("scipy.stats")
    logits = np.array([1.7, -0.3, 0.9, 2.4, 0.1, -1.2, 1.1, 0.5], np.float32)
    want = _closed_form_probs(logits, t, k, p)
    n = 100_000
    counts = np.zeros(logits.size, np.int64)
    for s in range(n):
        counts[orc.sample_token(logits, t, k, p, s * 7919 + 13)[0]] += 1
    kept = want > 0
    assert (counts[~kept] == 0).all(), (counts, want)
    chi2, pval = stats.chisquare(counts[kept], want[kept] * n)
    assert pval > 1e-4, (chi2, pval, counts, want)


# ------------------------------------------ f64 accumulation of the m > 1 path
def test_matmul_fallback_accumulates_in_f64(orc):
    """cpu.rs:964-999 matmul_tiled_fallback accumulates in f64 and rounds once:
    a row [2^24, 1, -2^24] against ones sums to 1 (in f32 the 1 is lost).  At
    m == 1 the dispatch (cpu.rs:924-945) takes the f32 GEMV instead: 0."""
    a = np.array([[2.0**24, 1.0, -(2.0**24)], [1.0, 2.0**24, -(2.0**24)]], np.float32)
    b = np.ones((3, 2), np.float32)
    assert orc.matmul_f32(a, b, 2, 3, 2).tolist() == [[1.0, 1.0], [1.0, 1.0]]
    assert orc.matmul_f32(a[:1], b, 1, 3, 2).tolist() == [[0.0, 0.0]]
    assert orc.matmul_f32(a.T.copy(), b, 2, 3, 2, trans_a=True).tolist() == [[1.0, 1.0], [1.0, 1.0]]


# ------------------------------------------------ layer-major cache path
FAST_CFGS = [
    dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
         n_kv_heads=6, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=True),
    dict(vocab_size=500, hidden_size=512, intermediate_size=300, n_layers=2, n_heads=4,
         n_kv_heads=1, max_seq_len=300, rope_theta=500000.0, tie_word_embeddings=False),
    dict(vocab_size=77, hidden_size=40, intermediate_size=52, n_layers=3, n_heads=5,
         n_kv_heads=5, max_seq_len=80, rope_theta=10000.0, tie_word_embeddings=False),
    dict(vocab_size=300, hidden_size=96, intermediate_size=70, n_layers=2, n_heads=8,
         n_kv_heads=2, max_seq_len=80, rope_theta=10000.0, tie_word_embeddings=True),
]


@pytest.mark.parametrize("ci", range(len(FAST_CFGS)))
def test_layer_major_cache_path_bit_identical(orc, ci):
    """orc_generate_greedy_fast / orc_llama_forward_cache_seq (the oracle's
    full-size parity mode) against the token-by-token cache path: the same
    tokens, bit-identical logits and KV cache rows, single- and multi-threaded
    (head dims 48, 128, 8 and 12; GQA 1:1, 4:1 and 4:1 with odd vocab)."""
    cfg = orc.LlamaConfig(**FAST_CFGS[ci])
    om = orc.Llama(cfg, ci, quantize=True, keep_f32=False)
    prompt = orc.prompt_ids(ci + 1, 37, cfg.vocab_size)
    ref_t, ref_l = om.generate_greedy(prompt, 20, mode=1, want_logits=True)
    for th in (0, 8):
        orc.set_threads(th)
        t, lg = om.generate_greedy_fast(prompt, 20, want_logits=True)
        assert (t == ref_t).all()
        assert np.array_equal(lg, ref_l)
    # a split over several calls, logits of several rows, cache contents
    c_ref = om.new_cache(60)
    ref_rows = [om.forward_with_cache(c_ref, int(tok), pos, mode=1)
                for pos, tok in enumerate(prompt[:30])]
    c = om.new_cache(60)
    got_a = om.forward_cache_seq(c, prompt[:11], 0, n_logits=3)
    got_b = om.forward_cache_seq(c, prompt[11:30], 11, n_logits=19)
    orc.set_threads(0)
    assert np.array_equal(got_a, np.stack(ref_rows[8:11]))
    assert np.array_equal(got_b, np.stack(ref_rows[11:30]))
    for layer in range(cfg.n_layers):
        assert c.seq_len(layer) == 30
        ka, va = c.layer(layer)
        kb, vb = c_ref.layer(layer)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    with pytest.raises(RuntimeError):
        om.forward_cache_seq(c, prompt[:31], 30)  # cache full
    om.close()


# ------------------------------------------------ the rest of the trait surface
def test_gelu_kat_and_erf_bound(orc):
    """cpu.rs:1494-1497 gelu_zero, published values of the tanh form, and the
    approximation bound against the exact erf GELU (a wrong constant in the
    tanh form breaks the bound)."""
    import math
    assert abs(orc.gelu([0.0])[0]) < 1e-7
    g = orc.gelu(np.array([1.0, -1.0, 2.0, -3.0], np.float32))
    assert np.allclose(g, [0.8411920, -0.1588080, 1.9545977, -0.0036373], atol=2e-7)
    xs = np.linspace(-6, 6, 2001).astype(np.float32)
    exact = np.array([0.5 * x * (1 + math.erf(x / math.sqrt(2))) for x in xs.astype(np.float64)])
    assert np.abs(orc.gelu(xs) - exact).max() < 6e-4
    assert (orc.gelu(np.array([20.0, -20.0], np.float32)) == np.array([20.0, -0.0], np.float32)).all()


def test_layernorm_kat_and_closed_form(orc):
    """cpu.rs:1585-1599 layernorm_inference_matches, and the closed form
    (x - mean) / sqrt(var + eps) * gamma + beta against numpy's mean / var."""
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)
    out, mu, rs = orc.layernorm(x, np.ones(3, np.float32), np.zeros(3, np.float32), 2, 3, 1e-5)
    want = np.array([-1.2247357, 0.0, 1.2247357] * 2, np.float32)
    assert np.abs(out - want).max() < 1e-6
    assert mu.tolist() == [2.0, 5.0]
    rng = np.random.default_rng(21)
    x = rng.normal(3, 2, (5, 77)).astype(np.float32)
    g = rng.normal(1, 0.3, 77).astype(np.float32)
    b = rng.normal(0, 0.3, 77).astype(np.float32)
    out, mu, rs = orc.layernorm(x, g, b, 5, 77, 1e-5)
    x64 = x.astype(np.float64)
    m = x64.mean(1, keepdims=True)
    r = 1 / np.sqrt(x64.var(1, keepdims=True) + np.float64(np.float32(1e-5)))
    assert np.abs(out.reshape(5, 77) - ((x64 - m) * r * g + b)).max() < 1e-5
    assert np.allclose(mu, m.ravel(), rtol=1e-7) and np.allclose(rs, r.ravel(), rtol=1e-7)


def test_sum_accumulates_in_f64(orc):
    """cpu.rs:500-503: an f64 sum rounded once (in f32 the 1 would be lost)."""
    assert orc.sum_(np.array([2.0**24, 1.0, -(2.0**24)], np.float32)) == 1.0
    assert orc.sum_(np.zeros(0, np.float32)) == 0.0
    x = np.random.default_rng(22).normal(0, 1, 10001).astype(np.float32)
    assert orc.sum_(x) == np.float32(x.astype(np.float64).sum())


def test_rope_trait_kat_and_rotation(orc):
    """cpu.rs:1538-1549 rope_basic (pos 1, head_dim 4: cos 1, sin 1), position
    0 is the identity, and each pair is the textbook rotation by
    pos / theta^(2i/hd); a trailing partial head and an odd last value are
    copied."""
    out = orc.rope(np.array([1, 0, 1, 0], np.float32), 1, 4, 1, 4, 10000.0)
    assert abs(out[0] - 0.5403) < 1e-3 and abs(out[1] - 0.8415) < 1e-3
    rng = np.random.default_rng(23)
    x = rng.normal(0, 1, 3 * 70).astype(np.float32)
    assert np.array_equal(orc.rope(x, 3, 70, 0, 16, 10000.0), x)
    pos, hd, th = 37, 16, 10000.0
    out = orc.rope(x, 3, 70, pos, hd, th).reshape(3, 70)
    xr = x.reshape(3, 70).astype(np.float64)
    for h in range(70 // hd):
        for i in range(hd // 2):
            ang = pos / th ** (2 * i / hd)
            z = (xr[:, h * hd + 2 * i] + 1j * xr[:, h * hd + 2 * i + 1]) * np.exp(1j * ang)
            assert np.abs(out[:, h * hd + 2 * i] - z.real).max() < 1e-5
            assert np.abs(out[:, h * hd + 2 * i + 1] - z.imag).max() < 1e-5
    assert np.array_equal(out[:, 64:], x.reshape(3, 70)[:, 64:])


def test_column_row_and_head_moves_match_numpy(orc):
    """gather_columns / scatter_columns (mod.rs:316-350), reshape_for_heads /
    reshape_from_heads (441-510) and split_qkv_reshape_heads (408-438, with
    cpu.rs:1601-1630 split_qkv_reshape_heads_matches_manual) against numpy
    slicing and transposes."""
    rng = np.random.default_rng(24)
    x = rng.normal(0, 1, (7, 13)).astype(np.float32)
    assert np.array_equal(orc.gather_columns(x, 7, 13, 4, 6), x[:, 4:10].ravel())
    src = rng.normal(0, 1, (7, 6)).astype(np.float32)
    want = x.copy()
    want[:, 4:10] += src
    assert np.array_equal(orc.scatter_columns(x, src, 7, 13, 4, 6), want.ravel())
    B, S, H, D = 2, 5, 3, 4
    flat = rng.normal(0, 1, (B * S, H * D)).astype(np.float32)
    heads = flat.reshape(B, S, H, D).transpose(0, 2, 1, 3).reshape(B * H, S, D)
    assert np.array_equal(orc.reshape_for_heads(flat, B, S, H, D), heads.ravel())
    assert np.array_equal(orc.reshape_from_heads(heads, B, S, H, D), flat.ravel())
    seq, nh, dh = 2, 2, 3
    qkv = np.arange(seq * 3 * nh * dh, dtype=np.float32)
    q, k, v = orc.split_qkv_reshape_heads(qkv, seq, nh, dh)
    rows = qkv.reshape(seq, 3, nh * dh)
    for got, part in ((q, 0), (k, 1), (v, 2)):
        assert np.array_equal(got, orc.reshape_for_heads(rows[:, part].copy(), 1, seq, nh, dh))


@pytest.mark.parametrize("ad,bd", [((4, 5), (4, 5)), ((4, 5), (1, 5)), ((4, 5), (5,)), ((1, 5), (4, 5)),
                                   ((4, 5), (4, 1)), ((4, 1), (4, 5)), ((2, 3, 4), (3, 1)),
                                   ((2, 1, 4), (1, 3, 1)), ((6,), (1,)), ((2, 1, 3, 1, 2, 1), (3, 4, 1, 5))])
def test_add_broadcast_matches_numpy(orc, ad, bd):
    """cpu.rs:94-188 add (every fast path and the generic broadcast) against
    numpy's broadcasting, bit-exact."""
    rng = np.random.default_rng(len(ad) * 10 + len(bd))
    a = rng.normal(0, 1, ad).astype(np.float32)
    b = rng.normal(0, 1, bd).astype(np.float32)
    want = a + b
    assert np.array_equal(orc.add_broadcast(a, ad, b, bd, want.shape), want.ravel())


def test_scaled_softmax_kat(orc):
    """cpu.rs:1569-1583 scaled_softmax_matches_separate: softmax of scale(x);
    with the same f32 products the two are bit-identical."""
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)
    assert np.array_equal(orc.scaled_softmax(x, 2, 3, 0.5), orc.softmax(orc.scale(x, 0.5), 2, 3))
    y = np.random.default_rng(25).normal(0, 4, (3, 50)).astype(np.float32)
    assert np.array_equal(orc.scaled_softmax(y, 3, 50, 0.125), orc.softmax(orc.scale(y, 0.125), 3, 50))
