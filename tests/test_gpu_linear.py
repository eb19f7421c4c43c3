"""The quantized Linear layer with bias (linear.rs:16-101; matmul_i8_f32_bias,
cpu.rs:553-570) on the GPU against the CPU oracle.

Callers it serves: GPT-2's projections (c_attn 768->2304, c_fc 768->3072,
c_proj 3072->768) and Whisper's MLP (fc1 d->4d, fc2 4d->d; base d=512, large
d=1280, scry-stt checkpoint/mod.rs:169-194), at decode row counts (1..16: the
dequant-fused GEMV with the bias in its store epilogue) and encoder / prompt
row counts (the MFMA GEMM, bias in its epilogue).

Bars: Linear::new's weights bit-exact with init::normal_vec on the same
fastrand state (and the state advanced by two calls per weight); the int8
weights and scale bit-exact; forward within 2e-5 relative (GEMV, f32
accumulation in another order) or 1e-4 (GEMM: bf16 hi/lo split, the prefill
bar) of the oracle; residual scaling exact where the factor is a power of two
and otherwise the f32 nearest to the f64 product.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32
WY0 = 0x2D358DCCAA6C78A5
M64 = (1 << 64) - 1
GEMV_TOL = 2e-5
GEMM_TOL = 1e-4


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def test_linear_new_matches_init_normal_vec(hip, orc):
    print("[case] Linear::new init on the fastrand stream", flush=True)
    rng = hip.Rng.with_seed(42)
    a = hip.Linear.new(768, 3072, rng)
    b = hip.Linear.new(3072, 768, rng)  # continues the stream
    n = 768 * 3072
    assert np.array_equal(a.weight.to_vec().view(np.uint32), orc.normal_vec(42, 0, n).view(np.uint32))
    assert np.array_equal(b.weight.to_vec().view(np.uint32), orc.normal_vec(42, 2 * n, n).view(np.uint32))
    assert rng.state == (42 + 4 * n * WY0) & M64
    assert not a.bias.to_vec().any() and a.bias.n == 3072
    a.free()
    b.free()


def test_residual_scaling(hip):
    print("[case] Linear::apply_residual_scaling", flush=True)
    w = np.random.default_rng(1).normal(0, 0.02, (64, 96)).astype(F)
    lin = hip.Linear.from_arrays(w, np.zeros(96, F))
    lin.apply_residual_scaling(2)  # 1/sqrt(4) = 0.5: exact
    assert np.array_equal(lin.weight.to_vec(), (w * F(0.5)).ravel())
    lin.apply_residual_scaling(8)  # 0.25
    assert np.array_equal(lin.weight.to_vec(), (w * F(0.125)).ravel())
    lin2 = hip.Linear.from_arrays(w, np.zeros(96, F))
    lin2.apply_residual_scaling(12)
    got = lin2.weight.to_vec().astype(np.float64)
    exact = w.ravel().astype(np.float64) * (1.0 / np.sqrt(24.0))
    # the f32 nearest to the f64 product: within half an ulp of it
    ulp = np.spacing(np.abs(got).astype(F)).astype(np.float64)
    assert (np.abs(got - exact) <= 0.5 * ulp).all()
    lin.free()
    lin2.free()


SHAPES = [  # (name, in, out)
    ("gpt2 c_attn", 768, 2304), ("gpt2 c_fc", 768, 3072), ("gpt2 c_proj", 3072, 768),
    ("whisper-base fc1", 512, 2048), ("whisper-base fc2", 2048, 512),
    ("whisper-large fc1", 1280, 5120), ("whisper-large fc2", 5120, 1280),
]


@pytest.mark.parametrize("name,k,n", SHAPES)
def test_quantized_forward(hip, orc, name, k, n):
    rng = np.random.default_rng(k * 7 + n)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    bias = rng.normal(0, 0.5, n).astype(F)
    lin = hip.Linear.from_arrays(w, bias)
    lin.quantize_weights()
    q, s = orc.quantize_symmetric(w)
    assert np.array_equal(lin.quant.weight_q.to_vec(), q.ravel()) and lin.quant.scale == s
    for seq in (1, 3, 16, 17, 150):
        print(f"[case] {name} {k}->{n} seq={seq}", flush=True)
        x = rng.normal(0, 1, (seq, k)).astype(F)
        xs = hip.HipBackend.from_vec(x)
        out = lin.forward(xs, seq).to_vec().reshape(seq, n)
        ref = orc.matmul_i8_f32_bias(x, q, s, bias, seq, k, n)
        err = rel_err(out, ref)
        print(f"[err] {err:.3e}", flush=True)
        assert err < (GEMV_TOL if seq <= 16 else GEMM_TOL), (name, seq)
        xs.free()
    lin.free()


def test_f32_forward_and_errors(hip, orc):
    print("[case] Linear forward without quantization; shape errors", flush=True)
    rng = np.random.default_rng(5)
    k, n, seq = 96, 40, 5
    w = rng.normal(0, 0.05, (k, n)).astype(F)
    bias = rng.normal(0, 1, n).astype(F)
    x = rng.normal(0, 1, (seq, k)).astype(F)
    lin = hip.Linear.from_arrays(w, bias)
    out = lin.forward(hip.HipBackend.from_vec(x), seq).to_vec().reshape(seq, n)
    ref = orc.matmul_f32(x, w, seq, k, n) + bias
    assert rel_err(out, ref) < GEMV_TOL
    # bf16 mode: bf16 product, the bias still added in f32 (ops::matmul_bias)
    hip.HipBackend.set_bf16_mode(True)
    try:
        ob = lin.forward(hip.HipBackend.from_vec(x), seq).to_vec().reshape(seq, n)
    finally:
        hip.HipBackend.set_bf16_mode(False)
    refb = orc.matmul_bf16(x, w, seq, k, n) + bias
    assert rel_err(ob, refb) < GEMV_TOL
    with pytest.raises(ValueError):
        lin.forward(hip.HipBackend.from_vec(x), seq + 1)
    with pytest.raises(ValueError):
        hip.Linear(lin.weight, hip.HipBackend.zeros(n + 1), k, n)
    lin.free()


@pytest.mark.parametrize("bf16", [False, True])
def test_matmul_bias_backend(hip, orc, bf16):
    """MathBackend::matmul_bias (mod.rs:62-86): the matmul, then the f32 bias
    row added to every output row; every transpose pairing, GEMV and GEMM row
    counts, f32 and bf16 mode."""
    rng = np.random.default_rng(11)
    k, n = 200, 72
    bias = rng.normal(0, 1, n).astype(F)
    bs = hip.HipBackend.from_vec(bias)
    hip.HipBackend.set_bf16_mode(bf16)
    try:
        for m in (1, 7, 150):
            for ta in (False, True):
                for tb in (False, True):
                    print(f"[case] matmul_bias bf16={bf16} m={m} ta={ta} tb={tb}", flush=True)
                    a = rng.normal(0, 1, (k, m) if ta else (m, k)).astype(F)
                    b = rng.normal(0, 0.1, (n, k) if tb else (k, n)).astype(F)
                    av, bv = hip.HipBackend.from_vec(a.ravel()), hip.HipBackend.from_vec(b.ravel())
                    got = hip.HipBackend.matmul_bias(av, bv, bs, m, k, n, ta, tb).to_vec()
                    mm = orc.matmul_bf16 if bf16 else orc.matmul_f32
                    ref = mm(a, b, m, k, n, ta, tb) + bias
                    # only the bf16 MFMA GEMM (untransposed A, > 16 rows)
                    # sums in another order than f32 / f64 accumulation
                    tol = GEMM_TOL if (bf16 and m > 16 and not ta) else GEMV_TOL
                    assert rel_err(got.reshape(m, n), ref) < tol, (m, ta, tb)
                    av.free()
                    bv.free()
        with pytest.raises(RuntimeError, match="bias holds"):
            hip.HipBackend.matmul_bias(hip.HipBackend.from_vec(np.ones(2 * k, F)),
                                       hip.HipBackend.from_vec(np.ones(k * (n + 1), F)),
                                       bs, 2, k, n + 1)
    finally:
        hip.HipBackend.set_bf16_mode(False)
    bs.free()
