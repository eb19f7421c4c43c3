"""scry_hip_sample_token_noalloc (static scratch, no device allocation)
against scry_hip_sample_token: the same token and rng state on two calls in a
row, the second with a smaller vocabulary, for every filter combination and
the greedy path; and the error for a vocabulary above the scratch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONFIGS = [(0.0, 0, 1.0), (0.8, 40, 0.95), (0.8, 0, 0.95), (1.0, 0, 1.0), (0.7, 5, 1.0), (1.3, 0, 0.3)]


@pytest.mark.parametrize("t,k,p", CONFIGS)
def test_noalloc_matches_sample_token(hip, t, k, p):
    B = hip.HipBackend
    rng = np.random.default_rng(int(t * 10) + k)
    sizes = (128256, 32000)  # the second call's input is smaller
    for call_i, V in enumerate(sizes):
        logits = rng.normal(0, 3, V).astype(np.float32)
        logits[V // 3] = logits[V // 5]  # a tie
        lg = B.from_vec(logits)
        sc = hip.SamplingConfig(temperature=t, top_k=k, top_p=p, max_tokens=1)
        for seed in (1, 99):
            ra, rb = hip.Rng.with_seed(seed + call_i), hip.Rng.with_seed(seed + call_i)
            ta = B.sample_token(lg, sc, ra)
            tb = B.sample_token_noalloc(lg, sc, rb)
            print(f"[case] V={V} T={t} k={k} p={p} seed={seed}: {ta} {tb}", flush=True)
            assert ta == tb and ra.state == rb.state


def test_noalloc_refuses_vocabulary_above_scratch(hip):
    B = hip.HipBackend
    lg = B.from_vec(np.zeros(262145, np.float32))
    with pytest.raises(hip.ScryHipError) as ei:
        B.sample_token_noalloc(lg, hip.SamplingConfig(temperature=1.0), hip.Rng.with_seed(1))
    assert ei.value.code == 6
