"""GPU parity of the op-level C ABI against the CPU oracle (same inputs).
Integer/byte work is bit-exact; float ops have the tolerance stated per test."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


# ------------------------------------------------------------ quantize
@pytest.mark.parametrize("case", ["normal", "zeros", "kat", "halfway", "nan", "inf", "big"])
def test_quantize_symmetric_bit_exact(hip, orc, case):
    B = hip.HipBackend
    rng = np.random.default_rng(10)
    w = {
        "normal": rng.normal(0, 0.02, 100003).astype(F),
        "zeros": np.zeros(1000, F),
        "kat": np.array([1000.0, -1000.0, 0.0], F),
        "halfway": np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5], F),
        "nan": np.array([np.nan, 1.0, -0.5, 0.25], F),
        "inf": np.array([np.inf, 1.0, -3.0], F),
        "big": rng.normal(0, 0.02, 4096 * 4096).astype(F),
    }[case]
    print(f"[case] quantize {case} n={w.size}", flush=True)
    q_ref, s_ref = orc.quantize_symmetric(w)
    qd, s = B.quantize_symmetric(B.from_vec(w))
    q = qd.to_vec()
    assert (q == q_ref).all()
    assert (np.isinf(s) and np.isinf(s_ref)) or F(s) == s_ref
    if np.isfinite(s_ref):
        deq = B.dequantize(qd, s).to_vec()
        assert (deq == orc.dequantize(q_ref, s_ref)).all()


def test_quantize_block32_bit_exact(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(11)
    for k, n in [(100, 7), (4096, 96), (288, 864)]:
        w = rng.normal(0, 0.02, (k, n)).astype(F)
        q_ref, s_ref = orc.quantize_block32(w, k, n)
        qd, sd = B.quantize_block32(B.from_vec(w), k, n)
        assert (qd.to_vec() == q_ref).all()
        assert (sd.to_vec() == s_ref).all()


def test_i8_storage_round_trip(hip):
    B = hip.HipBackend
    q = np.random.default_rng(12).integers(-128, 128, 12345).astype(np.int8)
    assert (B.i8_to_vec(B.i8_from_vec(q)) == q).all()


# ------------------------------------------------------- int8 GEMV / GEMM
SHAPES = [
    (1, 4096, 4096),    # attention projection (config 2)
    (1, 4096, 11008),   # gate/up (config 3)
    (1, 11008, 4096),   # down (config 3)
    (4, 4096, 11008),
    (4, 11008, 4096),
    (16, 4096, 4096),
    (16, 4096, 11008),  # config 3 at batch 16
    (16, 11008, 4096),
    (1, 288, 864),      # tiny qkv
    (3, 100, 65),       # ragged
    (2, 16, 5),
    (5, 2000, 33),      # runtime-chunk path
    (1, 3088, 300),     # one row, 4 chunks, the last one 16 values wide
    (1, 3080, 300),     # one row, k % 16 != 0
    (1, 10256, 300),    # one row, 11 chunks, the last one 16 values wide
    (1, 14336, 300),    # config-5 down at one row (14 chunks)
]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_i8_f32(hip, orc, m, k, n):
    B = hip.HipBackend
    rng = np.random.default_rng(m * 7 + k + n)
    print(f"[case] matmul_i8_f32 m={m} k={k} n={n}", flush=True)
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    q, s = orc.quantize_symmetric(w)
    orc.set_threads(8)
    ref = orc.matmul_i8_f32(a, q, s, m, k, n)
    orc.set_threads(0)
    out = B.matmul_i8_f32(B.from_vec(a), B.i8_from_vec(q), s, m, k, n).to_vec().reshape(m, n)
    err = rel_err(out, ref)
    print(f"[err] rel {err:.3e}", flush=True)
    # f32 accumulation in a different order than the reference's sequential sum
    assert err < 2e-5


def test_matmul_i8_f32_bias_and_block32(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(13)
    m, k, n = 2, 4096, 1024
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    bias = rng.normal(0, 1, n).astype(F)
    q, s = orc.quantize_symmetric(w)
    ref = orc.matmul_i8_f32_bias(a, q, s, bias, m, k, n)
    out = B.matmul_i8_f32_bias(B.from_vec(a), B.i8_from_vec(q), s, B.from_vec(bias), m, k, n)
    assert rel_err(out.to_vec().reshape(m, n), ref) < 2e-5
    q32, s32 = orc.quantize_block32(w, k, n)
    ref = orc.matmul_i8_f32_b32(a, q32, s32, m, k, n)
    out = B.matmul_i8_f32_block32(B.from_vec(a), B.i8_from_vec(q32), B.from_vec(s32), m, k, n)
    assert rel_err(out.to_vec().reshape(m, n), ref) < 2e-5


@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (4, 4096, 11008), (16, 11008, 4096),
                                   (16, 4096, 11008), (1, 11008, 4096)])
def test_matmul_i8_f32_block32_shapes(hip, orc, m, k, n):
    """Block-32 scales at the config 2 / 3 shapes and batches."""
    B = hip.HipBackend
    rng = np.random.default_rng(m * 5 + k + 3 * n)
    print(f"[case] matmul_i8_f32_block32 m={m} k={k} n={n}", flush=True)
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    q32, s32 = orc.quantize_block32(w, k, n)
    orc.set_threads(8)
    ref = orc.matmul_i8_f32_b32(a, q32, s32, m, k, n)
    orc.set_threads(0)
    out = B.matmul_i8_f32_block32(B.from_vec(a), B.i8_from_vec(q32), B.from_vec(s32), m, k, n)
    err = rel_err(out.to_vec().reshape(m, n), ref)
    print(f"[err] rel {err:.3e}", flush=True)
    assert err < 2e-5


def test_matmul_i8_exact_integer(hip):
    B = hip.HipBackend
    rng = np.random.default_rng(14)
    k, n = 300, 77
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    out = B.matmul_i8_f32(B.from_vec(np.ones(k, F)), B.i8_from_vec(q), 1.0, 1, k, n).to_vec()
    assert (out == q.astype(np.int64).sum(0)).all()


# ------------------------------------------------ skinny MFMA route (2..16 rows)
# matmul_i8_f32 takes 3..16 activation rows with k % 8 == 0, k >= 256 and
# n >= 256 to the skinny MFMA kernel (three exact bf16 planes of x, q in bf16,
# k splits added in order); the shapes of test_matmul_i8_f32 at m = 4 and 16
# and the block-32 shapes above already run there.
@pytest.mark.parametrize("m,k,n", [(3, 1000, 300), (7, 4096, 4096), (13, 1032, 513), (16, 14336, 4096),
                                   (9, 11008, 300)])
def test_skinny_matmul_vs_oracle(hip, orc, m, k, n):
    """Ragged k (a partial last 64-wide block), ragged n (a partial column
    tile), every row count class, per-tensor with bias and block-32."""
    B = hip.HipBackend
    rng = np.random.default_rng(m * 11 + k + n)
    print(f"[case] skinny matmul m={m} k={k} n={n}", flush=True)
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    bias = rng.normal(0, 1, n).astype(F)
    q, s = orc.quantize_symmetric(w)
    q32, s32 = orc.quantize_block32(w, k, n)
    orc.set_threads(8)
    ref = orc.matmul_i8_f32_bias(a, q, s, bias, m, k, n)
    ref32 = orc.matmul_i8_f32_b32(a, q32, s32, m, k, n)
    orc.set_threads(0)
    out = B.matmul_i8_f32_bias(B.from_vec(a), B.i8_from_vec(q), s, B.from_vec(bias), m, k, n)
    out32 = B.matmul_i8_f32_block32(B.from_vec(a), B.i8_from_vec(q32), B.from_vec(s32), m, k, n)
    e, e32 = rel_err(out.to_vec().reshape(m, n), ref), rel_err(out32.to_vec().reshape(m, n), ref32)
    print(f"[err] per-tensor+bias {e:.3e} block-32 {e32:.3e}", flush=True)
    assert e < 2e-5 and e32 < 2e-5


def test_skinny_matmul_exact_integers(hip):
    """Exact results that pin the three activation planes, the k order inside
    an MFMA and the column mapping:
      - 24-bit integer activations (every plane carries bits) and one weight of
        +-1 per output column at a random k: each output is +-x exactly;
      - two such weights per column with 22-bit activations: exact sums;
      - 15-bit activations and full-range weights, two per column: exact;
      - block-32 with power-of-two scales and one weight per column: exact."""
    B = hip.HipBackend
    rng = np.random.default_rng(21)
    m, k, n = 5, 1024, 384

    def sparse_q(per_col, full_range):
        q = np.zeros((k, n), np.int8)
        for j in range(n):
            rows = rng.choice(k, per_col, replace=False)
            q[rows, j] = (rng.integers(-127, 128, per_col) if full_range
                          else rng.choice([-1, 1], per_col))
        return q

    def ints(bits):
        return (rng.integers(0, 2 ** bits, (m, k)) * rng.choice([-1, 1], (m, k))).astype(np.int64)

    for bits, per_col, full in ((23, 1, False), (22, 2, False), (15, 2, True)):
        x, q = ints(bits), sparse_q(per_col, full)
        want = x @ q.astype(np.int64)
        assert np.abs(want).max() < 2 ** 24
        out = B.matmul_i8_f32(B.from_vec(x.astype(F)), B.i8_from_vec(q), 1.0, m, k, n).to_vec()
        assert np.array_equal(out.reshape(m, n).astype(np.int64), want), (bits, per_col)
    x, q = ints(23), sparse_q(1, False)
    s32 = (2.0 ** rng.integers(-2, 3, (n, k // 32))).astype(F)
    w32 = q.astype(np.float64) * np.repeat(s32.T.astype(np.float64), 32, axis=0)
    want32 = x.astype(np.float64) @ w32
    out32 = B.matmul_i8_f32_block32(B.from_vec(x.astype(F)), B.i8_from_vec(q), B.from_vec(s32.ravel()),
                                    m, k, n).to_vec().reshape(m, n)
    assert np.array_equal(out32.astype(np.float64), want32)


def test_skinny_matmul_nonfinite(hip, orc):
    """Inf and NaN activations reach the outputs as the reference's f32 sums
    give them (Inf times a nonzero weight stays infinite, times 0 is NaN)."""
    B = hip.HipBackend
    rng = np.random.default_rng(22)
    m, k, n = 4, 512, 256
    a = rng.normal(0, 1, (m, k)).astype(F)
    a[0, 3] = np.inf
    a[1, 100] = -np.inf
    a[2, 7] = np.nan
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    q[3, :16] = 0
    ref = orc.matmul_i8_f32(a, q, 0.01, m, k, n)
    out = B.matmul_i8_f32(B.from_vec(a), B.i8_from_vec(q), 0.01, m, k, n).to_vec().reshape(m, n)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    assert np.array_equal(np.isinf(out), np.isinf(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(np.sign(out[np.isinf(out)]), np.sign(ref[np.isinf(ref)]))
    assert rel_err(out[fin], ref[fin]) < 2e-5


@pytest.mark.parametrize("m,k,n,b32", [(1, 4096, 512, False), (2, 4096, 512, False), (1, 11008, 256, False),
                                        (1, 300, 64, False), (1, 3600, 130, False), (1, 4096, 300, True),
                                        (1, 11008, 200, True)])
def test_gemv_matmul_nonfinite(hip, orc, m, k, n, b32):
    """The GEMV rows (m <= 2) with Inf and NaN activations, as the skinny test
    above: Inf times a nonzero weight stays infinite, times 0 is NaN."""
    B = hip.HipBackend
    rng = np.random.default_rng(31 + m + k)
    a = rng.normal(0, 1, (m, k)).astype(F)
    a[0, 3] = np.inf
    a[0, 900 % k] = np.nan if m == 1 and k == 11008 else a[0, 900 % k]
    if m > 1:
        a[1, 100] = -np.inf
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    q[3, :16] = 0
    if b32:
        s32 = rng.uniform(0.005, 0.02, (n, (k + 31) // 32)).astype(F)
        ref = orc.matmul_i8_f32_b32(a, q, s32, m, k, n)
        out = B.matmul_i8_f32_block32(B.from_vec(a), B.i8_from_vec(q), B.from_vec(s32), m, k, n).to_vec().reshape(m, n)
    else:
        ref = orc.matmul_i8_f32(a, q, 0.01, m, k, n)
        out = B.matmul_i8_f32(B.from_vec(a), B.i8_from_vec(q), 0.01, m, k, n).to_vec().reshape(m, n)
    print(f"[nf] m={m} k={k} b32={b32}: inf gpu {int(np.isinf(out).sum())} ref {int(np.isinf(ref).sum())}, "
          f"nan gpu {int(np.isnan(out).sum())} ref {int(np.isnan(ref).sum())}", flush=True)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    assert np.array_equal(np.isinf(out), np.isinf(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(np.sign(out[np.isinf(out)]), np.sign(ref[np.isinf(ref)]))
    if fin.any():
        assert rel_err(out[fin], ref[fin]) < 2e-5


def test_matmul_shape_errors(hip):
    B = hip.HipBackend
    with pytest.raises(hip.ScryHipError) as ei:
        B.matmul_i8_f32(B.from_vec(np.ones(10, F)), B.i8_from_vec(np.ones(30, np.int8)), 1.0, 1,
                        10, 4)
    assert ei.value.code == 1


# --------------------------------------------------------------- glue
def test_rmsnorm(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(15)
    x = rng.normal(0, 1, (3, 4096)).astype(F)
    w = rng.normal(1, 0.1, 4096).astype(F)
    ref = orc.rmsnorm(x, w, 3, 4096, 1e-5)
    out = B.rmsnorm(B.from_vec(x), B.from_vec(w), 3, 4096, 1e-5).to_vec()
    assert rel_err(out, ref) < 1e-6


def test_rope(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(16)
    seq, nh, hd, p0 = 4, 8, 128, 1000
    freqs = orc.compute_rope_freqs(hd, 10000.0).astype(F)
    x = rng.normal(size=(seq, nh, hd)).astype(F)
    ref = orc.rope_with_freqs_preloaded(x, seq, nh, hd, p0, freqs)
    out = B.rope_with_freqs_preloaded(B.from_vec(x), seq, nh, hd, p0, B.from_vec(freqs)).to_vec()
    assert np.abs(out - ref).max() < 1e-5
    sc = F(1.0 / np.sqrt(hd))
    ref2 = orc.scale(ref, sc)
    out2 = B.rope_with_freqs_scaled_preloaded(B.from_vec(x), seq, nh, hd, p0, B.from_vec(freqs),
                                              sc).to_vec()
    assert np.abs(out2 - ref2).max() < 1e-5


def test_softmax_swiglu_add_scale(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(17)
    x = rng.normal(0, 3, (32, 777)).astype(F)
    assert rel_err(B.softmax(B.from_vec(x), 32, 777).to_vec(), orc.softmax(x, 32, 777)) < 1e-6
    g = rng.normal(0, 2, 11008).astype(F)
    u = rng.normal(0, 2, 11008).astype(F)
    # silu in f64 with the device exp: rounds to the same f32 except at rare ties
    assert rel_err(B.swiglu(B.from_vec(g), B.from_vec(u)).to_vec(), orc.swiglu(g, u)) < 1e-6
    assert (B.add(B.from_vec(g), B.from_vec(u)).to_vec() == orc.add(g, u)).all()
    assert (B.scale(B.from_vec(g), 0.37).to_vec() == orc.scale(g, 0.37)).all()


def test_embedding_gather_scatter_exact(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(18)
    w = rng.normal(size=(50, 24)).astype(F)
    ids = [3, 49, 0, 3]
    assert (B.embedding(B.from_vec(w), ids, 50, 24).to_vec() == orc.embedding(w, ids, 50, 24)).all()
    with pytest.raises(hip.ScryHipError) as ei:
        B.embedding(B.from_vec(w), [50], 50, 24)
    assert ei.value.code == 5
    max_seq, L, nkv, nq, hd = 12, 7, 2, 6, 8
    cache = rng.normal(size=(max_seq, nkv * hd)).astype(F)
    out = B.gather_reshape_repeat_kv(B.from_vec(cache), max_seq, L, nkv, nq, hd).to_vec()
    assert (out == orc.gather_reshape_repeat_kv(cache, max_seq, L, nkv, nq, hd)).all()
    heads = rng.normal(size=(nkv, L, hd)).astype(F)
    assert (B.repeat_kv(B.from_vec(heads), nkv, nq, L, hd).to_vec()
            == orc.repeat_kv(heads, nkv, nq, L, hd)).all()
    dst = B.from_vec(np.zeros((max_seq, 16), F))
    row = rng.normal(size=16).astype(F)
    B.scatter_rows(dst, B.from_vec(row), max_seq, 16, 5, 1)
    d = dst.to_vec().reshape(max_seq, 16)
    assert (d[5] == row).all() and (np.delete(d, 5, 0) == 0).all()


def test_argmax_semantics(hip, orc):
    B = hip.HipBackend
    cases = [[1, 3, 3, 2], [5], [1, np.nan, 0.5], [3, np.nan, 1, 2], [2, np.nan],
             [np.nan, np.nan], [-np.inf, -np.inf]]
    for c in cases:
        assert B.argmax(B.from_vec(np.array(c, F))) == orc.argmax(c), c
    rng = np.random.default_rng(19)
    x = rng.normal(size=128256).astype(F)
    x[[5, 70000, 128255]] = x.max() + 1  # three-way tie: last index wins
    assert B.argmax(B.from_vec(x)) == 128255 == orc.argmax(x)


def test_f32_matmul_and_batched(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(20)
    for (m, k, n, ta, tb) in [(1, 64, 33, False, True), (1, 50, 64, False, False),
                              (7, 13, 9, True, False), (5, 8, 6, False, True)]:
        a = rng.normal(size=(k, m) if ta else (m, k)).astype(F)
        b = rng.normal(size=(n, k) if tb else (k, n)).astype(F)
        ref = orc.matmul_f32(a, b, m, k, n, ta, tb)
        out = B.matmul(B.from_vec(a), B.from_vec(b), m, k, n, ta, tb).to_vec().reshape(m, n)
        assert rel_err(out, ref) < 1e-5
    a = rng.normal(size=(4, 1, 16)).astype(F)
    b = rng.normal(size=(4, 10, 16)).astype(F)
    ref = orc.matmul_strided_batched(a, b, 4, 1, 16, 10, trans_b=True)
    out = B.matmul_strided_batched(B.from_vec(a), B.from_vec(b), 4, 1, 16, 10, False, True)
    assert rel_err(out.to_vec(), ref) < 1e-5
