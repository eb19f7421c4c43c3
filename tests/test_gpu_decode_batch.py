"""Batched greedy decode (scry_hip_llama_decode_batch): several sequences advance
one token per step together, each against its own KV cache.  The reference
decodes one sequence at a time (generate.rs:51-89 over llama.rs:744-763), so
every sequence is checked against the oracle's own greedy run of that
sequence, on the same seeded synthetic weights and token ids.

Bars: each step's logits within 1e-3 relative of the oracle's for that
sequence and position; greedy tokens identical; and against the GPU's
single-sequence decode step, identical tokens and logits within the same bar.
With per-tensor int8 weights the projections run on the int8 matrix cores:
each activation row's 512-value segment becomes 24-bit fixed point scaled to
the segment's largest value (one rounding, at most 2^-24 of that maximum per
value), the products with the weight bytes are summed exactly in i32, and
each split's partial is rounded once to f32.  Block-32 weights take three
exact bf16 planes of each value with f32 accumulation.
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


def run_batch(hm, prompts, steps, max_seq, chunks=None):
    """Prefill all but the last token of each prompt into its own cache, then
    decode the sequences together (in `chunks` calls when given)."""
    caches = [hm.new_llama_kv_cache(max_seq) for _ in prompts]
    for c, p in zip(caches, prompts):
        if len(p) > 1:
            hm.prefill([c], np.asarray(p[:-1])[None, :], want_logits=False)
    last = [int(p[-1]) for p in prompts]
    toks, lgs = [], []
    for n in (chunks or [steps]):
        t, lg = hm.decode_batch(caches, last, n, want_logits=True)
        toks.append(t)
        lgs.append(lg)
        last = [int(x) for x in t[:, -1]]
    for c, p in zip(caches, prompts):
        assert c.seq_len == len(p) - 1 + steps
    for c in caches:
        c.free()
    return np.concatenate(toks, axis=1), np.concatenate(lgs, axis=0)


def check_vs_oracle(om, prompts, toks, lgs, steps, mode=1):
    worst = 0.0
    for i, p in enumerate(prompts):
        ref_t, ref_l = om.generate_greedy(np.asarray(p, np.int64), steps, mode=mode, want_logits=True)
        assert len(ref_t) == steps
        e = max(rel_err(lgs[t, i], ref_l[t]) for t in range(steps))
        worst = max(worst, e)
        assert e < LOGIT_TOL, f"sequence {i}: {e:.3e}"
        assert (toks[i] == ref_t).all(), f"sequence {i}: tokens differ"
    return worst


def test_decode_batch_tiny_vs_oracle(orc, hip):
    """Four tiny-config sequences at different positions (1-, 9-, 21- and
    34-token prompts), 20 steps."""
    print("[case] decode_batch tiny 4 sequences", flush=True)
    orc.set_threads(8)
    om = orc.Llama(orc.LlamaConfig(**TINY), 0, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**TINY), 0)
    prompts = [orc.prompt_ids(s + 1, n, TINY["vocab_size"]) for s, n in enumerate([1, 9, 21, 34])]
    toks, lgs = run_batch(hm, prompts, 20, 64)
    e = check_vs_oracle(om, prompts, toks, lgs, 20)
    print(f"[err] decode_batch tiny vs oracle {e:.3e}", flush=True)
    hm.free()
    om.close()
    orc.set_threads(0)


@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 64), (4, 1, 128), (16, 4, 32), (6, 6, 48)])
def test_decode_batch_gqa_vs_oracle(orc, hip, nh, nkv, hd):
    """GQA geometries, three sequences, a small vocabulary (many distinct greedy
    tokens), 24 steps split over two calls."""
    print(f"[case] decode_batch nh={nh} nkv={nkv} hd={hd}", flush=True)
    cfg = dict(vocab_size=96, hidden_size=nh * hd, intermediate_size=320, n_layers=2, n_heads=nh,
               n_kv_heads=nkv, max_seq_len=160, rope_theta=500000.0, tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 3, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 3)
    prompts = [orc.prompt_ids(10 + s, n, 96) for s, n in enumerate([40, 7, 65])]
    toks, lgs = run_batch(hm, prompts, 24, 96, chunks=[10, 14])
    e = check_vs_oracle(om, prompts, toks, lgs, 24)
    print(f"[err] {e:.3e}; distinct tokens {len(np.unique(toks))}", flush=True)
    hm.free()
    om.close()


def test_decode_batch_block32_vs_oracle(orc, hip):
    """Block-32 scales: the skinny matrix-core kernel's per-block scaled path."""
    print("[case] decode_batch block-32", flush=True)
    cfg = dict(vocab_size=128, hidden_size=256, intermediate_size=384, n_layers=2, n_heads=4,
               n_kv_heads=2, max_seq_len=128, rope_theta=10000.0, tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 4, quantize=True, block32=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 4, hip.QUANT_BLOCK32)
    prompts = [orc.prompt_ids(20 + s, n, 128) for s, n in enumerate([12, 30])]
    toks, lgs = run_batch(hm, prompts, 16, 64)
    e = check_vs_oracle(om, prompts, toks, lgs, 16, mode=2)
    print(f"[err] block-32 {e:.3e}", flush=True)
    hm.free()
    om.close()


def test_decode_batch_sixteen_and_one(orc, hip):
    """The largest batch (16 sequences) and a batch of one."""
    print("[case] decode_batch 16 and 1 sequences", flush=True)
    cfg = dict(vocab_size=64, hidden_size=128, intermediate_size=256, n_layers=2, n_heads=4,
               n_kv_heads=2, max_seq_len=64, rope_theta=10000.0, tie_word_embeddings=False)
    om = orc.Llama(orc.LlamaConfig(**cfg), 6, quantize=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 6)
    prompts = [orc.prompt_ids(30 + s, 2 + (5 * s) % 17, 64) for s in range(16)]
    toks, lgs = run_batch(hm, prompts, 8, 32)
    check_vs_oracle(om, prompts, toks, lgs, 8)
    toks, lgs = run_batch(hm, prompts[5:6], 8, 32)
    check_vs_oracle(om, prompts[5:6], toks, lgs, 8)
    hm.free()
    om.close()


def test_decode_batch_llama3_dims_vs_single(hip):
    """Llama-3-8B layer shapes (h 4096, 32:8 GQA, FFN 14336, vocab 128256; 2
    layers): four sequences batched against the single-sequence decode step
    of each."""
    print("[case] decode_batch llama3-8b dims, 2 layers", flush=True)
    cfg = hip.LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, n_layers=2,
                          n_heads=32, n_kv_heads=8, max_seq_len=512, rope_theta=500000.0,
                          tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(cfg, 0, init_on_device=True)
    prompts = [hip.synth.prompt_ids(s + 1, n, 128256) for s, n in enumerate([200, 37, 129, 2])]
    toks, lgs = run_batch(hm, prompts, 12, 256)
    for i, p in enumerate(prompts):
        st, sl = hm.generate_greedy(p, 12, want_logits=True, prefill=True)
        e = max(rel_err(lgs[t, i], sl[t]) for t in range(12))
        print(f"[err] sequence {i} batched vs single {e:.3e}", flush=True)
        assert e < LOGIT_TOL
        assert (toks[i] == st).all()
    hm.free()


def test_decode_batch_errors(hip):
    cfg = hip.LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=128, n_layers=1,
                          n_heads=2, n_kv_heads=2, max_seq_len=32, rope_theta=10000.0,
                          tie_word_embeddings=False)
    hm = hip.LlamaModel.new_random(cfg, 1)
    a, b = hm.new_llama_kv_cache(16), hm.new_llama_kv_cache(16)
    hm.prefill([a], np.zeros((1, 10), np.int64), want_logits=False)
    with pytest.raises(hip.ScryHipError) as ei:  # 10 + 7 rows past the capacity of a
        hm.decode_batch([a, b], [1, 2], 7)
    assert "exceed" in str(ei.value)
    with pytest.raises(hip.ScryHipError):  # token id out of range
        hm.decode_batch([a, b], [1, 64], 2)
    with pytest.raises(hip.ScryHipError):  # the same cache twice
        hm.decode_batch([a, a], [1, 2], 2)
    many = [hm.new_llama_kv_cache(4) for _ in range(17)]
    with pytest.raises(hip.ScryHipError):  # more sequences than one step takes
        hm.decode_batch(many, [0] * 17, 1)
    assert a.seq_len == 10 and b.seq_len == 0  # failed calls leave the caches untouched
    t = hm.decode_batch([a, b], [1, 2], 6)  # exactly to a's capacity
    assert t.shape == (2, 6) and a.seq_len == 16 and b.seq_len == 6
    for x in many:
        x.free()
    a.free()
    b.free()
    hm.free()
    mb = hip.LlamaModel.new_random(cfg, 1, quant_mode=hip.QUANT_BF16)
    c = mb.new_llama_kv_cache(8)
    with pytest.raises(hip.ScryHipError) as ei:
        mb.decode_batch([c], [1], 1)
    assert "int8" in str(ei.value)
    c.free()
    mb.free()
