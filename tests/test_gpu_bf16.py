"""bf16 mode (the reference's `bf16` feature) on the GPU against the oracle:
init_gpu_bf16 / from_vec_with_bf16 (mod.rs:28-32, cuda.rs:55-59, 149-175,
230-254), matmul on bf16 operands with f32 accumulation (bf16_ops,
cuda.rs:1226-1290), the bf16 embedding (cuda.rs:480-503).

Bars: the device cast equals the reference's (oracle `orc_f32_to_bf16`) bit
for bit, seen through matmuls with an identity (GEMV and GEMM paths);
integer-valued operands give exact results on every path and transpose
combination; random operands stay within 2e-5 relative of the oracle's
exact-product f64 sum (f32 accumulation order); bf16-only storage widens
exactly in to_vec / embedding, and other ops refuse it.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32
TOL = 2e-5


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def widen(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.fixture
def bf16_mode(hip):
    B = hip.HipBackend
    B.set_bf16_mode(True)
    try:
        yield B
    finally:
        B.set_bf16_mode(False)


def test_cast_matches_reference_through_identity(bf16_mode, orc):
    B = bf16_mode
    print("[case] bf16 cast: x @ I, GEMV (1 row) and GEMM (40 rows)", flush=True)
    rng = np.random.default_rng(1)
    k = 256
    bits = rng.integers(0, 2**32, (40, k), dtype=np.uint64).astype(np.uint32)
    bits[:, :32] = (bits[:, :32] & 0xFFFF0000) | 0x8000  # exact ties
    x = bits.view(np.float32)
    x[~np.isfinite(x)] = 1.5  # identity products stay finite
    x[np.abs(x) > 1e30] = 2.5
    x[np.abs(x) < 1e-30] = 0.75  # no zeros (the sum of +0 terms drops a -0) or subnormals
    eye = np.eye(k, dtype=F)
    for m in (1, 40):
        y = B.matmul(B.from_vec(x[:m]), B.from_vec(eye), m, k, k).to_vec().reshape(m, k)
        want = widen(orc.f32_to_bf16(x[:m])).reshape(m, k)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), m


@pytest.mark.parametrize("m,k,n,ta,tb", [
    (1, 4096, 4096, False, False), (3, 768, 3072, False, True), (16, 1000, 300, False, False),
    (17, 4096, 1024, False, False), (200, 768, 2304, False, True), (8, 96, 40, True, False),
    (33, 64, 50, True, True), (1, 11008, 4096, False, True),
])
def test_matmul_bf16(bf16_mode, orc, m, k, n, ta, tb):
    B = bf16_mode
    print(f"[case] bf16 matmul m={m} k={k} n={n} ta={ta} tb={tb}", flush=True)
    rng = np.random.default_rng(m * 131 + k + n)
    a = rng.normal(0, 1, (m, k)).astype(F)
    w = rng.normal(0, 0.02, (k, n)).astype(F)
    A = np.ascontiguousarray(a.T) if ta else a
    W = np.ascontiguousarray(w.T) if tb else w
    # the weight as bf16-only storage (from_vec_with_bf16), the activation f32
    wb = B.from_vec_with_bf16(W, orc.f32_to_bf16(W))
    out = B.matmul(B.from_vec(A), wb, m, k, n, ta, tb).to_vec().reshape(m, n)
    ref = orc.matmul_bf16(A, W, m, k, n, ta, tb)
    err = rel_err(out, ref)
    print(f"[err] {err:.3e}", flush=True)
    assert err < TOL
    # both operands f32 (each rounded by the device cast): the same result
    out2 = B.matmul(B.from_vec(A), B.from_vec(W), m, k, n, ta, tb).to_vec().reshape(m, n)
    assert rel_err(out2, ref) < TOL
    # integer values: exact on this path
    ai = rng.integers(-8, 9, (m, k)).astype(F)
    wi = rng.integers(-8, 9, (k, n)).astype(F)
    Ai = np.ascontiguousarray(ai.T) if ta else ai
    Wi = np.ascontiguousarray(wi.T) if tb else wi
    oi = B.matmul(B.from_vec(Ai), B.from_vec(Wi), m, k, n, ta, tb).to_vec().reshape(m, n)
    assert np.array_equal(oi, ai @ wi)


def test_bf16_storage(bf16_mode, hip, orc):
    B = bf16_mode
    print("[case] bf16-only storage: to_vec, clone, embedding, refusals, stale caches", flush=True)
    rng = np.random.default_rng(2)
    vocab, dim = 300, 64
    emb = rng.normal(0, 1, (vocab, dim)).astype(F)
    h = orc.f32_to_bf16(emb)
    s = B.from_vec_with_bf16(emb, h)
    assert np.array_equal(s.to_vec().view(np.uint32), widen(h).view(np.uint32))
    c = B.clone_storage(s)
    assert np.array_equal(c.to_vec(), s.to_vec())
    ids = np.array([0, 299, 17, 17, 5], np.int64)
    e = B.embedding(s, ids, vocab, dim).to_vec().reshape(len(ids), dim)
    assert np.array_equal(e, widen(h).reshape(vocab, dim)[ids])
    with pytest.raises(hip.ScryHipError) as ei:
        B.softmax(s, vocab, dim)
    assert "bf16 data only" in str(ei.value)
    # outside bf16 mode from_vec_with_bf16 keeps the f32 data
    B.set_bf16_mode(False)
    f = B.from_vec_with_bf16(emb, h)
    assert np.array_equal(f.to_vec(), emb.ravel())
    B.set_bf16_mode(True)
    # scatter_rows writes in place: the next matmul sees the new rows
    k, n = 64, 32
    w = rng.integers(-4, 5, (k, n)).astype(F)
    ws = B.from_vec(w)
    x = np.ones((1, k), F)
    y0 = B.matmul(B.from_vec(x), ws, 1, k, n).to_vec()
    assert np.array_equal(y0, w.sum(0))
    B.scatter_rows(ws, B.from_vec(np.full((2, n), 3.0, F)), k, n, 10, 2)
    w[10:12] = 3.0
    y1 = B.matmul(B.from_vec(x), ws, 1, k, n).to_vec()
    assert np.array_equal(y1, w.sum(0))


# ------------------------------------------------- the bf16 model's decode step
# The bf16 model rounds every projection's activations to bf16, so a last-bit
# difference in an f32 value upstream (accumulation order) moves a rounded
# activation by one bf16 step whenever it sits at a rounding boundary, and
# such steps compound with depth and sequence length.  Measured on the oracle
# itself by switching its matmul from the f64 sum to an f32 sum in the same
# order: 2e-7..4e-5 relative on the logits at 1-2 layers of width <= 288 and a
# few positions ("shallow"), 2.3e-3..4.7e-3 at width 512-4096 or 6 layers x 40
# positions ("deep").  The gap between bf16 and f32 semantics (forward mode 3
# against mode 0) is 4e-3..1.3e-2 on the same cases, so the shallow bar below
# separates them by 10x either side; the deep bar catches gross errors (packing,
# chunking, epilogues at the large shapes) together with identical tokens, and
# every case also checks that each step's logits lie nearer the bf16 semantics
# than the f32 ones, on average under half as far.
SHALLOW_TOL = 5e-4
DEEP_TOL = 1e-2
TINY = dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
            n_kv_heads=6, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=True)


def _bf16_decode_vs_oracle(hip, orc, cfg, seed, prompt, steps, tol, init_on_device=False):
    """The GPU model in QUANT_BF16 (bf16 weights packed from the seeded f32
    init, activations cast to bf16 at each projection, f32 accumulation)
    against the oracle's forward mode 3 on the same seeded f32 weights
    (llama.rs:593-680 init, cuda.rs:1226-1290 matmul): logits within `tol`
    relative, identical greedy tokens, replays bit-identical."""
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), seed, quant_mode=hip.QUANT_BF16,
                                   init_on_device=init_on_device)
    try:
        kt, kl = hm.generate_greedy(prompt, steps, want_logits=True)
        kt2, kl2 = hm.generate_greedy(prompt, steps, want_logits=True)
        # the prompt through the batched prefill (the MFMA GEMM on the bf16 rows)
        pt, pl = hm.generate_greedy(prompt, steps, want_logits=True, prefill=True)
        with pytest.raises(hip.ScryHipError):
            hm.qtensor(orc.T_QKV, 0)  # the model holds no int8 weights
    finally:
        hm.free()
    orc.set_threads(16)
    om = orc.Llama(orc.LlamaConfig(**cfg), seed, quantize=False)
    try:
        ref_t, ref_l = om.generate_greedy(prompt, steps, mode=3, want_logits=True)
        f32_l = om.generate_greedy(prompt, steps, mode=0, want_logits=True)[1]
    finally:
        om.close()
        orc.set_threads(0)
    err = max(rel_err(kl[i], ref_l[i]) for i in range(steps))
    perr = max(rel_err(pl[i], ref_l[i]) for i in range(steps))
    gap = max(rel_err(f32_l[i], ref_l[i]) for i in range(steps))
    d3 = np.array([rel_err(kl[i], ref_l[i]) for i in range(steps)])
    d0 = np.array([rel_err(kl[i], f32_l[i]) for i in range(steps)])
    print(f"[err] bf16 decode {err:.3e}, with batched prefill {perr:.3e} (bar {tol:g}; f32 semantics "
          f"would be {gap:.3e} away); tokens {kt[:6].tolist()}", flush=True)
    print(f"[sep] mean over steps: to bf16 semantics {d3.mean():.3e} (max {d3.max():.3e}); to f32 "
          f"semantics {d0.mean():.3e} (min {d0.min():.3e}); steps nearer bf16 {(d3 < d0).mean():.2f}",
          flush=True)
    assert err < tol and perr < tol
    # the logits follow bf16 semantics rather than f32 ones: every step nearer
    # mode 3 than mode 0, and on average well under half as far (measured at
    # most 0.39 of the way on the deep cases, 2e-5 on the shallow ones)
    assert (d3 < d0).all()
    assert d3.mean() < 0.5 * d0.mean()
    assert (kt == ref_t).all() and (pt == ref_t).all()
    assert (kt2 == kt).all() and np.array_equal(kl2, kl)  # replays reproduce bit for bit


@pytest.mark.parametrize("layers", [1, 2])
def test_bf16_model_decode_shallow(hip, orc, layers):
    print(f"[case] bf16 model: tiny dims (tied head), {layers} layer(s), prompt 4, 4 greedy", flush=True)
    cfg = dict(TINY, n_layers=layers)
    _bf16_decode_vs_oracle(hip, orc, cfg, 0, orc.prompt_ids(1, 4, TINY["vocab_size"]), 4, SHALLOW_TOL)


def test_bf16_model_decode_shallow_gqa(hip, orc):
    print("[case] bf16 model: GQA nh=8 nkv=2 hd=4, prompt 100, 20 greedy", flush=True)
    cfg = dict(vocab_size=64, hidden_size=32, intermediate_size=256, n_layers=2, n_heads=8,
               n_kv_heads=2, max_seq_len=160, rope_theta=500000.0, tie_word_embeddings=False)
    _bf16_decode_vs_oracle(hip, orc, cfg, 7, orc.prompt_ids(3, 100, 64), 20, SHALLOW_TOL)


def test_bf16_model_decode_tiny_deep(hip, orc):
    print("[case] bf16 model: tiny, 6 layers, prompt 8, 32 greedy", flush=True)
    _bf16_decode_vs_oracle(hip, orc, TINY, 0, orc.prompt_ids(1, 8, TINY["vocab_size"]), 32, DEEP_TOL)


@pytest.mark.parametrize("nh,nkv,hd", [(4, 1, 128), (16, 4, 64)])
def test_bf16_model_decode_gqa_deep(hip, orc, nh, nkv, hd):
    print(f"[case] bf16 model: GQA nh={nh} nkv={nkv} hd={hd}, prompt 100, 20 greedy", flush=True)
    cfg = dict(vocab_size=64, hidden_size=nh * hd, intermediate_size=256, n_layers=2,
               n_heads=nh, n_kv_heads=nkv, max_seq_len=160, rope_theta=500000.0,
               tie_word_embeddings=False)
    _bf16_decode_vs_oracle(hip, orc, cfg, 7, orc.prompt_ids(3, 100, 64), 20, DEEP_TOL)


def test_bf16_model_decode_7b_dims(hip, orc):
    """Config-4 shapes with 2 layers (device init, as bench.py)."""
    print("[case] bf16 model: 7B dims, 2 layers, prompt 24, 8 greedy", flush=True)
    cfg = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, n_layers=2,
               n_heads=32, n_kv_heads=32, max_seq_len=2048, rope_theta=10000.0,
               tie_word_embeddings=False)
    _bf16_decode_vs_oracle(hip, orc, cfg, 0, orc.prompt_ids(1, 24, 32000), 8, DEEP_TOL,
                           init_on_device=True)


@pytest.mark.parametrize("layers,tol", [(1, SHALLOW_TOL), (6, DEEP_TOL)])
def test_bf16_model_forward_all_positions(hip, orc, layers, tol):
    """LlamaModel::forward (llama.rs:683-700) on the bf16 model: every
    position's logits through the batched GEMMs, against oracle forward mode 3."""
    print(f"[case] bf16 model forward, tiny dims, {layers} layer(s), 12 tokens", flush=True)
    cfg = dict(TINY, n_layers=layers)
    toks = orc.prompt_ids(5, 12, TINY["vocab_size"])
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 0, quant_mode=hip.QUANT_BF16)
    try:
        got = hm.forward(toks)
    finally:
        hm.free()
    om = orc.Llama(orc.LlamaConfig(**cfg), 0, quantize=False)
    try:
        ref = om.forward(toks, mode=3)
    finally:
        om.close()
    err = max(rel_err(got[i], ref[i]) for i in range(len(toks)))
    print(f"[err] bf16 forward {err:.3e} (bar {tol:g})", flush=True)
    assert err < tol
