"""GPU parity of the rest of the trait surface (backend/mod.rs) against the
oracle's restatement of the CPU backend: data movement and f32 arithmetic
bit-exact; f64 reductions and libm calls within the tolerance stated per
test (the device sums in a tree and uses the device libm)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32


def test_ones_and_concat_rows(hip):
    B = hip.HipBackend
    assert (B.ones(1001).to_vec() == 1.0).all()
    a = np.arange(12, dtype=F)
    b = -np.arange(6, dtype=F)
    out = B.concat_rows(B.from_vec(a), B.from_vec(b), 4, 2, 3).to_vec()
    assert np.array_equal(out, np.concatenate([a, b]))  # cpu.rs:526-539


@pytest.mark.parametrize("ad,bd", [((4, 5), (4, 5)), ((4, 5), (1, 5)), ((4, 5), (5,)), ((1, 5), (4, 5)),
                                   ((4, 5), (4, 1)), ((4, 1), (4, 5)), ((2, 3, 4), (3, 1)),
                                   ((2, 1, 4), (1, 3, 1)), ((6,), (1,)), ((2, 1, 3, 1, 2, 1), (3, 4, 1, 5)),
                                   ((1, 4096), (37, 4096))])
def test_add_broadcast(hip, orc, ad, bd):
    B = hip.HipBackend
    rng = np.random.default_rng(sum(ad) + 3 * sum(bd))
    a = rng.normal(0, 1, ad).astype(F)
    b = rng.normal(0, 1, bd).astype(F)
    od = np.broadcast_shapes(ad, bd)
    ref = orc.add_broadcast(a, ad, b, bd, od)
    out = B.add_shapes(B.from_vec(a), ad, B.from_vec(b), bd, od).to_vec()
    assert np.array_equal(out, ref)


def test_add_broadcast_errors(hip):
    B = hip.HipBackend
    a, b = B.from_vec(np.ones(6, F)), B.from_vec(np.ones(4, F))
    with pytest.raises(hip.ScryHipError) as ei:
        B.add_shapes(a, (2, 3), b, (4,), (2, 4))  # incompatible: the reference panics
    assert ei.value.code == 1
    with pytest.raises(hip.ScryHipError):
        B.add_shapes(a, (2, 3), B.from_vec(np.ones(3, F)), (3,), (3, 2))  # wrong output shape


def test_add_inplace_and_mul(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(31)
    a = rng.normal(0, 1, 5000).astype(F)
    b = rng.normal(0, 1, 5000).astype(F)
    d = B.from_vec(a)
    B.add_inplace(d, B.from_vec(b))
    assert np.array_equal(d.to_vec(), orc.add(a, b))
    assert np.array_equal(B.mul_elementwise(B.from_vec(a), B.from_vec(b)).to_vec(), orc.mul_elementwise(a, b))
    # zip semantics: the shorter operand sets the length
    assert np.array_equal(B.mul_elementwise(B.from_vec(a), B.from_vec(b[:77])).to_vec(),
                          orc.mul_elementwise(a[:77], b[:77]))


@pytest.mark.parametrize("rows,d", [(2, 3), (5, 77), (16, 4096), (3, 1)])
def test_layernorm(hip, orc, rows, d):
    """cpu.rs:416-475; f64 sums in a tree on the device: output within 2 f32
    ulps-scale of the oracle (1e-6 relative to the row scale), mean and rstd
    within 1e-6 relative."""
    B = hip.HipBackend
    rng = np.random.default_rng(rows * 100 + d)
    x = rng.normal(1.5, 3, (rows, d)).astype(F)
    g = rng.normal(1, 0.5, d).astype(F)
    bt = rng.normal(0, 0.5, d).astype(F)
    ref, mu_r, rs_r = orc.layernorm(x, g, bt, rows, d, 1e-5)
    o, mu, rs = B.layernorm(B.from_vec(x), B.from_vec(g), B.from_vec(bt), rows, d, 1e-5)
    assert np.abs(o.to_vec() - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())
    assert np.allclose(mu.to_vec(), mu_r, rtol=1e-6, atol=1e-7)
    assert np.allclose(rs.to_vec(), rs_r, rtol=1e-6)
    o2 = B.layernorm_inference(B.from_vec(x), B.from_vec(g), B.from_vec(bt), rows, d, 1e-5)
    assert np.array_equal(o2.to_vec(), o.to_vec())


def test_gelu(hip, orc):
    """cpu.rs:1110-1116 in f64 on the device (device tanh): each value equal to
    the oracle's or one f32 ulp away."""
    B = hip.HipBackend
    x = np.concatenate([np.linspace(-10, 10, 20001), [0.0, -0.0, 1e-30, -1e-30, 40.0, -40.0]]).astype(F)
    ref = orc.gelu(x)
    out = B.gelu(B.from_vec(x)).to_vec()
    ulp = np.abs(out.view(np.int32).astype(np.int64) - ref.view(np.int32))
    print(f"[err] gelu: {np.count_nonzero(ulp)} of {x.size} differ, max {ulp.max()} ulp", flush=True)
    assert ulp.max() <= 1
    assert abs(out[20001]) < 1e-7  # gelu_zero (cpu.rs:1494-1497)


@pytest.mark.parametrize("n", [0, 1, 3, 1000, 1 << 20])
def test_sum(hip, orc, n):
    """cpu.rs:500-503: f64 sum rounded to f32; the device's tree order differs
    from the sequential one by f64 rounding only."""
    B = hip.HipBackend
    x = np.random.default_rng(n).normal(0.3, 2, n).astype(F)
    ref = orc.sum_(x)
    got = B.sum(B.from_vec(x))
    assert abs(got - ref) <= max(abs(ref) * 2**-23, n * 2**-52 * float(np.abs(x).sum()))
    assert B.sum(B.from_vec(np.array([2.0**24, 1.0, -(2.0**24)], F))) == 1.0


@pytest.mark.parametrize("rows,last,pos,hd,theta", [(1, 4, 1, 4, 10000.0), (3, 70, 37, 16, 10000.0),
                                                    (5, 4096, 1999, 128, 500000.0), (2, 9, 3, 3, 100.0)])
def test_rope_trait(hip, orc, rows, last, pos, hd, theta):
    """cpu.rs:601-633: host (glibc) cos / sin table, f32 rotation -- bit-exact."""
    B = hip.HipBackend
    x = np.random.default_rng(rows + last).normal(0, 1, rows * last).astype(F)
    ref = orc.rope(x, rows, last, pos, hd, theta)
    out = B.rope(B.from_vec(x), rows, last, pos, hd, theta).to_vec()
    assert np.array_equal(out, ref)


def test_columns_rows_heads(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(33)
    x = rng.normal(0, 1, (7, 12288)).astype(F)
    # llama.rs:389-391: q / k / v slices of the fused qkv row
    for start, count in ((0, 4096), (4096, 4096), (8192, 4096), (5, 3)):
        assert np.array_equal(B.gather_columns(B.from_vec(x), 7, 12288, start, count).to_vec(),
                              orc.gather_columns(x, 7, 12288, start, count))
    src = rng.normal(0, 1, (7, 100)).astype(F)
    d = B.from_vec(x)
    B.scatter_columns(d, B.from_vec(src), 7, 12288, 300, 100)
    assert np.array_equal(d.to_vec(), orc.scatter_columns(x, src, 7, 12288, 300, 100))
    assert np.array_equal(B.gather_rows(B.from_vec(x), 7, 12288, 2, 3).to_vec(), x[2:5].ravel())
    with pytest.raises(hip.ScryHipError):
        B.gather_columns(B.from_vec(x), 7, 12288, 12280, 16)
    Bt, S, H, D = 2, 33, 8, 16
    flat = rng.normal(0, 1, (Bt * S, H * D)).astype(F)
    heads = B.reshape_for_heads(B.from_vec(flat), Bt, S, H, D).to_vec()
    assert np.array_equal(heads, orc.reshape_for_heads(flat, Bt, S, H, D))
    assert np.array_equal(B.reshape_from_heads(B.from_vec(heads), Bt, S, H, D).to_vec(), flat.ravel())
    one = rng.normal(0, 1, H * D).astype(F)  # batch 1, seq 1: a copy (mod.rs:449-451)
    assert np.array_equal(B.reshape_for_heads(B.from_vec(one), 1, 1, H, D).to_vec(), one)
    qkv = rng.normal(0, 1, (S, 3 * H * D)).astype(F)
    got = B.split_qkv_reshape_heads(B.from_vec(qkv), S, H, D)
    for g, r in zip(got, orc.split_qkv_reshape_heads(qkv, S, H, D)):
        assert np.array_equal(g.to_vec(), r)


def test_causal_masks_and_scaled_softmax(hip, orc):
    B = hip.HipBackend
    rng = np.random.default_rng(34)
    seq, nm = 19, 5
    sc = rng.normal(0, 3, nm * seq * seq).astype(F)
    ref = orc.causal_mask_scale(sc, nm, seq, 0.125, -np.inf)
    d = B.from_vec(sc)
    B.apply_batched_causal_mask_and_scale(d, nm, seq, 0.125, -np.inf)
    assert np.array_equal(d.to_vec(), ref)
    d1 = B.from_vec(sc[: seq * seq])
    B.apply_causal_mask_and_scale(d1, seq, 0.125, -1e9)
    assert np.array_equal(d1.to_vec(), orc.causal_mask_scale(sc[: seq * seq], 1, seq, 0.125, -1e9))
    x = rng.normal(0, 4, (6, 300)).astype(F)
    ref = orc.scaled_softmax(x, 6, 300, 0.0883883)
    out = B.scaled_softmax(B.from_vec(x), 0.0883883, 6, 300).to_vec()
    # device expf against glibc expf: within a few f32 ulps of each value
    assert np.abs(out - ref).max() <= 4e-7 * max(1.0, np.abs(ref).max())
