"""Device sampling (sample_token, generate.rs:92-186, and generate's sampled
loop, generate.rs:51-89) against the CPU oracle's restatement.

The sampler reads the logits the GPU produced, so the token comparisons are
exact: for every step the oracle's sample_token on the GPU's own step logits,
with the same fastrand state, must give the same token and the same next
state.  The oracle sorts (value desc, index asc); the device uses radix
selects, f64 block sums and 2^62 fixed-point masses, so a token could only
differ when the draw r or the top-p mass lies within f64 rounding of a
boundary, which none of these seeded cases does (the test would show it).

Cases: random logits at vocabularies 1 .. 128256 under every filter
combination; ties cut by top-k and by top-p (kept in index order, the
oracle's rule); the uniform fallback (NaN, +inf, all -inf); top_k >= V and
tiny top_p; greedy below temperature 1e-8 (no rng draw); the sampled generate
loop (token by token and with prefill) and its rng bookkeeping; errors.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32
WY0 = 0x2D358DCCAA6C78A5
M64 = (1 << 64) - 1
LOGIT_TOL = 1e-3

CONFIGS = [  # (temperature, top_k, top_p)
    (1.0, 0, 1.0), (0.7, 40, 1.0), (0.8, 0, 0.9), (1.3, 50, 0.8), (0.5, 1, 1.0),
    (2.0, 0, 0.5), (100.0, 0, 0.95), (0.05, 0, 0.99), (1e-8, 0, 1.0), (0.9, 3, 0.3),
]


def device_draws(hip, logits, cfg, seed, n):
    B = hip.HipBackend
    s = B.from_vec(np.asarray(logits, F))
    rng = hip.Rng.with_seed(seed)
    sc = hip.SamplingConfig(temperature=cfg[0], top_k=cfg[1], top_p=cfg[2], max_tokens=1)
    toks = [B.sample_token(s, sc, rng) for _ in range(n)]
    s.free()
    return toks, rng.state


def oracle_draws(orc, logits, cfg, seed, n):
    st, toks = seed, []
    for _ in range(n):
        t, st = orc.sample_token(np.asarray(logits, F), cfg[0], cfg[1], cfg[2], st)
        toks.append(t)
    return toks, st


def check(hip, orc, logits, cfg, seed=7, n=6):
    gt, gs = device_draws(hip, logits, cfg, seed, n)
    ot, os_ = oracle_draws(orc, logits, cfg, seed, n)
    assert gt == ot, (cfg, gt, ot)
    assert gs == os_, cfg
    return gt


@pytest.mark.parametrize("V", [1, 2, 5, 1000, 32000, 128256])
def test_sample_token_random_logits(hip, orc, V):
    print(f"[case] sample_token random logits V={V}", flush=True)
    rng = np.random.default_rng(V)
    logits = (3.0 * rng.standard_normal(V)).astype(F)
    for i, cfg in enumerate(CONFIGS):
        check(hip, orc, logits, cfg, seed=1000 + i)
    # the rng state advances by one wyrand step per draw
    _, st = device_draws(hip, logits, (1.0, 0, 1.0), 5, 9)
    assert st == (5 + 9 * WY0) & M64


def test_sample_token_ties(hip, orc):
    print("[case] sample_token ties at the top-k and top-p cuts", flush=True)
    rng = np.random.default_rng(3)
    logits = rng.integers(-3, 4, 1000).astype(F)  # runs of equal values
    for cfg in [(1.0, 100, 1.0), (1.0, 1, 1.0), (0.6, 0, 0.3), (1.0, 0, 0.05), (0.8, 200, 0.45),
                (1.0, 0, 0.7)]:
        check(hip, orc, logits, cfg, seed=11, n=8)
    # equal logits everywhere: softmax 1/V, top-p keeps the first indices
    flat = np.full(1000, 0.25, F)
    toks = check(hip, orc, flat, (1.0, 0, 0.3337), seed=12, n=10)
    assert max(toks) < 334
    check(hip, orc, flat, (1.0, 10, 1.0), seed=13, n=4)
    # a tiny top-p keeps one entry: the first of the maxima
    t = check(hip, orc, np.array([1, 5, 5, 2], F), (1.0, 0, 1e-30), seed=14, n=4)
    assert t == [1, 1, 1, 1]


def test_sample_token_ties_large_kept_set(hip, orc):
    """More than 1024 entries survive top-k: the vocabulary-wide passes
    (selection levels, the tie search at the top-p cut, segment draw)."""
    print("[case] sample_token ties, kept set above 1024", flush=True)
    rng = np.random.default_rng(8)
    logits = rng.integers(-4, 5, 5000).astype(F)
    for cfg in [(1.0, 0, 0.3), (0.7, 3000, 0.6), (1.0, 0, 0.05), (1.5, 2000, 1.0), (1.0, 0, 0.97),
                (1.0, 0, 1e-30), (1.0, 4999, 0.5)]:
        check(hip, orc, logits, cfg, seed=31, n=6)
    flat = np.full(5000, -1.5, F)
    toks = check(hip, orc, flat, (1.0, 0, 0.41234), seed=32, n=8)
    assert max(toks) < 2062
    t = check(hip, orc, np.r_[np.zeros(3000, F), np.full(2000, 2.0, F)], (1.0, 0, 1e-30), seed=33, n=3)
    assert t == [3000] * 3
    wide = (rng.standard_normal(70000) * 40.0).astype(F)  # spans many binades
    for cfg in [(1.0, 0, 0.9), (3.0, 0, 0.999), (0.3, 5000, 0.8)]:
        check(hip, orc, wide, cfg, seed=34, n=4)
    nan = rng.standard_normal(5000).astype(F)
    nan[4321] = np.nan
    for cfg in [(1.0, 0, 1.0), (1.0, 0, 0.61)]:
        check(hip, orc, nan, cfg, seed=35, n=4)


def test_sample_token_degenerate(hip, orc):
    print("[case] sample_token uniform fallback, inf, top_k >= V", flush=True)
    rng = np.random.default_rng(4)
    base = rng.standard_normal(777).astype(F)
    nan = base.copy()
    nan[100] = np.nan
    pinf = base.copy()
    pinf[5] = np.inf
    ninf = np.full(300, -np.inf, F)
    half = base.copy()
    half[::2] = -np.inf
    for logits in (nan, pinf, ninf):  # softmax sum not > 0: uniform 1/V
        for cfg in [(1.0, 0, 1.0), (1.0, 0, 0.5), (0.7, 0, 0.25)]:
            check(hip, orc, logits, cfg, seed=21, n=5)
    for cfg in [(1.0, 776, 1.0), (1.0, 500, 0.9), (1.0, 0, 0.8)]:  # -inf entries: probability 0
        toks = check(hip, orc, half, cfg, seed=22, n=6)
        assert all(t % 2 == 1 for t in toks)
    for k in (777, 800):  # top_k >= V: no top-k filter
        a = check(hip, orc, base, (1.0, k, 1.0), seed=23)
        assert a == check(hip, orc, base, (1.0, 0, 1.0), seed=23)


def test_sample_token_greedy_below_1e8(hip, orc):
    print("[case] sample_token temperature < 1e-8", flush=True)
    x = np.random.default_rng(5).standard_normal(5000).astype(F)
    toks, st = device_draws(hip, x, (9e-9, 0, 0.5), 99, 3)
    assert toks == [orc.argmax(x)] * 3 and st == 99


SMALL = dict(vocab_size=2048, hidden_size=128, intermediate_size=256, n_layers=2, n_heads=4,
             n_kv_heads=2, max_seq_len=128, rope_theta=10000.0, tie_word_embeddings=True)


@pytest.fixture(scope="module")
def small(orc, hip):
    print("[case] small model init (h128 L2 V2048, seed 3)", flush=True)
    om = orc.Llama(orc.LlamaConfig(**SMALL), 3, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**SMALL), 3, 0)
    yield om, hm
    hm.free()
    om.close()


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


@pytest.mark.parametrize("cfg", [(1.0, 0, 1.0), (0.8, 40, 0.95), (1.2, 0, 0.9), (0.6, 5, 1.0)])
@pytest.mark.parametrize("prefill", [False, True])
def test_generate_sampled(small, orc, hip, cfg, prefill):
    om, hm = small
    T, k, p = cfg
    seed = 1234 + k
    print(f"[case] generate sampled T={T} top_k={k} top_p={p} prefill={prefill}", flush=True)
    prompt = orc.prompt_ids(5, 9, SMALL["vocab_size"])
    sc = hip.SamplingConfig(temperature=T, top_k=k, top_p=p, max_tokens=20)
    rng = hip.Rng.with_seed(seed)
    gt, gl = hm.generate(prompt, sc, rng, want_logits=True, prefill=prefill)
    assert len(gt) == 20
    # every token is sample_token of that step's logits, the rng state chained
    st = seed
    for i in range(len(gt)):
        t, st = orc.sample_token(gl[i], T, k, p, st)
        assert t == gt[i], i
    assert rng.state == st == (seed + 20 * WY0) & M64
    # and the whole loop agrees with the oracle's generate (same weights, seed)
    ot, ol = om.generate(prompt, 20, T, k, p, seed, mode=1, want_logits=True)
    err = max(rel_err(gl[i], ol[i]) for i in range(len(ot)))
    print(f"[err] sampled generate logits {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    assert (gt == ot).all()
    # through the module-level generate() too, continuing the same rng
    again = hip.generate(hm, prompt, sc, rng)
    assert rng.state == (seed + 40 * WY0) & M64 and len(again) == 20


def test_generate_edge_cases(small, orc, hip):
    om, hm = small
    print("[case] generate max_tokens 0 and 1, greedy temperature, errors", flush=True)
    prompt = orc.prompt_ids(6, 4, SMALL["vocab_size"])
    for mt in (0, 1):
        rng = hip.Rng.with_seed(77)
        t = hm.generate(prompt, hip.SamplingConfig(temperature=1.0, max_tokens=mt), rng)
        assert len(t) == 1 and rng.state == (77 + WY0) & M64
        assert (t == om.generate(prompt, mt, 1.0, 0, 1.0, 77, mode=1)).all()
    rng = hip.Rng.with_seed(5)
    g = hm.generate(prompt, hip.SamplingConfig(temperature=0.0, top_k=3, max_tokens=8), rng)
    assert (g == hm.generate_greedy(prompt, 8)).all() and rng.state == 5
    with pytest.raises(hip.ScryHipError):
        hm.generate(prompt, hip.SamplingConfig(temperature=1.0, top_k=-1, max_tokens=4), rng)
    with pytest.raises(hip.ScryHipError):
        hm.generate(prompt, hip.SamplingConfig(temperature=float("nan"), max_tokens=4), rng)
    with pytest.raises(ValueError):
        hip.generate(hm, prompt, hip.SamplingConfig(temperature=1.0, max_tokens=4))
