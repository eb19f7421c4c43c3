"""Parity at the full size of the headline configurations.

Config 4 (Llama-2-7B shape, 32 layers, 512-token prompt + 256 greedy tokens)
runs on the GPU exactly as bench.py runs it (device init of the same seeded
weights) and is checked against the CPU oracle on the GPU model's own int8
weights:
  - every step's logits within 1e-3 relative;
  - the oracle's greedy choice (argmax, generate.rs:167-173) equals the GPU's
    token at every step.
The oracle evaluates the cache path layer-major over the prompt plus the
GPU's tokens (orc_llama_forward_cache_seq, bit-identical to the token-by-token
path; tests/test_oracle.py).  Its logits at step t are what its own greedy run
computes at step t whenever the tokens before t agree.  Since every earlier
step's argmax also agrees, its own greedy run produces the same 256 tokens
(induction on t).

Config 5 (Llama-3-8B shape) is checked three ways:
  - at its dimensions with 2 layers against the oracle (batched prefill of 4
    sequences then greedy steps; the batched decode of 4 and of 8 sequences);
  - at full depth (32 layers) against the oracle on one sequence: a 64-token
    batched prefill and 8 greedy steps;
  - at full size (4 x 2048 prompts, 64 greedy steps) against the GPU's own
    token-by-token path.  The oracle would need ~6e13 multiply-adds for the
    4 x 2048 prompts.
"""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.slow]
LOGIT_TOL = 1e-3

LLAMA2_7B = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, n_layers=32,
                 n_heads=32, n_kv_heads=32, max_seq_len=2048, rope_theta=10000.0,
                 tie_word_embeddings=False)
LLAMA3_8B = dict(vocab_size=128256, hidden_size=4096, intermediate_size=14336, n_layers=32,
                 n_heads=32, n_kv_heads=8, max_seq_len=2048, rope_theta=500000.0,
                 tie_word_embeddings=False)
PROJ = ("T_QKV", "T_O", "T_GATE", "T_UP", "T_DOWN")


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def top2_margin(lg):
    t = np.partition(np.asarray(lg, np.float64), -2)[-2:]
    return float(t[1] - t[0])


def oracle_from_gpu(orc, hm, cfg, layers=None):
    """An oracle model holding exactly the GPU model's int8 weights, scales and
    f32 embedding table."""
    om = orc.Llama(orc.LlamaConfig(**cfg), None)
    for layer in range(cfg["n_layers"] if layers is None else layers):
        if layer % 8 == 0:
            print(f"[case] copying layer {layer} to the oracle", flush=True)
        for name in PROJ:
            tid = getattr(orc, name)
            q, s = hm.qtensor(tid, layer)
            om.set_qtensor(tid, layer, q, s)
    q, s = hm.qtensor(orc.T_LM_HEAD)
    om.set_qtensor(orc.T_LM_HEAD, 0, q, s)
    del q
    om.set_embed(hm.embed())
    return om


@pytest.fixture(scope="module")
def model7b(hip):
    print("[case] config 4 model: Llama-2-7B shape, seed 0, device init (as bench.py)", flush=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**LLAMA2_7B), seed=0, init_on_device=True)
    yield hm
    hm.free()


def test_config4_device_init_equals_host_init(hip, orc, model7b):
    """The bench's device init (k_normal_init) against the host init, which is
    bit-exact with the oracle's normal_vec (test_gpu_llama.py): every int8
    tensor, scale and the f32 embedding of the 7B model."""
    print("[case] config 4 host init (glibc, all host cores)", flush=True)
    hh = hip.LlamaModel.new_random(hip.LlamaConfig(**LLAMA2_7B), seed=0, init_on_device=False)
    diff = total = 0
    try:
        for layer in range(LLAMA2_7B["n_layers"]):
            for name in PROJ:
                tid = getattr(orc, name)
                qd, sd = model7b.qtensor(tid, layer)
                qh, sh = hh.qtensor(tid, layer)
                assert sd == sh, (layer, name, sd, sh)
                d = int(np.count_nonzero(qd != qh))
                if d:
                    assert np.abs(qd.astype(np.int16) - qh.astype(np.int16)).max() <= 1
                diff += d
                total += qd.size
        qd, sd = model7b.qtensor(orc.T_LM_HEAD)
        qh, sh = hh.qtensor(orc.T_LM_HEAD)
        assert sd == sh
        diff += int(np.count_nonzero(qd != qh))
        total += qd.size
        ed, eh = model7b.embed(), hh.embed()
        emb_diff = int(np.count_nonzero(ed != eh))
        emb_ulp = int(np.abs(ed.view(np.int32).astype(np.int64) - eh.view(np.int32)).max())
    finally:
        hh.free()
    print(f"[err] device vs host init: {diff} of {total} int8 weights differ; "
          f"{emb_diff} embedding values differ, by at most {emb_ulp} ulp", flush=True)
    # measured bit-exact on MI355X: the device log / cos / sqrt give glibc's
    # values on every one of the 6.6e9 samples of this model
    assert diff == 0
    assert emb_diff == 0


def test_config4_full_depth_vs_oracle(hip, orc, model7b):
    """32 layers, 512-token seeded prompt (seed 1), 256
    greedy tokens, token-by-token and with the batched prompt prefill."""
    cfg = LLAMA2_7B
    prompt = orc.prompt_ids(1, 512, cfg["vocab_size"])
    print("[case] config 4 GPU generate: 512 prompt + 256 greedy, token by token", flush=True)
    toks, lg = model7b.generate_greedy(prompt, 256, want_logits=True)
    print("[case] config 4 GPU generate with batched prefill", flush=True)
    toks_p, lg_p = model7b.generate_greedy(prompt, 256, want_logits=True, prefill=True)
    assert len(toks) == 256 and len(toks_p) == 256
    orc.set_threads(16)
    print("[case] config 4 oracle: GPU int8 weights, layer-major cache path over 767 rows",
          flush=True)
    om = oracle_from_gpu(orc, model7b, cfg)
    try:
        seq = np.concatenate([prompt, toks[:-1]])  # row i >= 511 gives step i - 511
        cache = om.new_cache(len(seq))
        ref = []
        for s0 in range(0, len(seq), 128):  # chunks: the same rows, bit-identical
            chunk = seq[s0:s0 + 128]
            nl = max(0, s0 + len(chunk) - 511) - max(0, s0 - 511)
            ref.append(om.forward_cache_seq(cache, chunk, s0, n_logits=nl))
            print(f"[case] oracle rows {s0}..{s0 + len(chunk) - 1} done", flush=True)
        ref = np.concatenate(ref)
        assert ref.shape == (256, cfg["vocab_size"])
        del cache
    finally:
        om.close()
        orc.set_threads(0)
    errs = np.array([rel_err(lg[i], ref[i]) for i in range(256)])
    errs_p = np.array([rel_err(lg_p[i], ref[i]) for i in range(256)])
    ref_toks = np.array([orc.argmax(ref[i]) for i in range(256)])
    margins = np.array([top2_margin(ref[i]) for i in range(256)])
    print(f"[err] config 4: max step rel err {errs.max():.3e} (prefill path {errs_p.max():.3e}); "
          f"{len(np.unique(toks))} distinct tokens; smallest top-1/top-2 margin "
          f"{margins.min():.4g}", flush=True)
    assert errs.max() < LOGIT_TOL
    assert (ref_toks == toks).all()
    assert (toks_p == toks).all()
    assert errs_p.max() < LOGIT_TOL


def test_config5_dims_two_layers_vs_oracle(hip, orc):
    """Config-5 tensor shapes (h4096, 32:8 GQA, ffn 14336, V 128256, theta 5e5)
    with 2 layers, against the oracle:
      - the batched prefill of 4 x 255 tokens (seeds 1-4), then 16 greedy
        steps per sequence, token by token;
      - the batched decode step (decode_batch, llama.rs:744-763 per row) of the
        same 4 sequences, and of 8 sequences (seeds 1-8).  From 5 rows on,
        every projection and the LM head run the 16-row int8-digit matrix-core
        kernel with 8 k-blocks per split; at 4 rows the 4-row kernel.
    Identical greedy tokens, logits within 1e-3 at every step."""
    cfg = dict(LLAMA3_8B, n_layers=2)
    NS = 16
    print("[case] config-5 dims, 2 layers: batched prefill 4 x 255 + 16 greedy; decode_batch 4 and 8",
          flush=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), seed=0, init_on_device=True)
    V = cfg["vocab_size"]
    prompts = np.stack([orc.prompt_ids(s + 1, 256, V) for s in range(8)])
    try:
        caches = [hm.new_llama_kv_cache(256 + NS) for _ in range(4)]
        last = hm.prefill(caches, prompts[:4, :255])
        gpu_lg, gpu_tok = [], []
        for s in range(4):
            tok, pos, lgs, ts = int(prompts[s, 255]), 255, [], []
            for _ in range(NS):
                lg, am = hm.forward_with_llama_cache(tok, pos, caches[s])
                lgs.append(lg)
                ts.append(am)
                tok, pos = am, pos + 1
            gpu_lg.append(np.stack(lgs))
            gpu_tok.append(np.array(ts))
            caches[s].free()
        batched = {}
        for n in (4, 8):
            print(f"[case] config-5 dims, 2 layers: decode_batch of {n} sequences", flush=True)
            cs = [hm.new_llama_kv_cache(256 + NS) for _ in range(n)]
            hm.prefill(cs, prompts[:n, :255], want_logits=False)
            batched[n] = hm.decode_batch(cs, prompts[:n, 255], NS, want_logits=True)
            for c in cs:
                c.free()
        orc.set_threads(16)
        om = oracle_from_gpu(orc, hm, cfg)
    finally:
        hm.free()
    try:
        for s in range(8):
            toks_s = gpu_tok[s] if s < 4 else batched[8][0][s]
            seq = np.concatenate([prompts[s], toks_s[:-1]])  # 271 rows
            cache = om.new_cache(len(seq))
            ref = om.forward_cache_seq(cache, seq, 0, n_logits=NS + 1)  # rows 254..270
            del cache
            ref_toks = np.array([orc.argmax(ref[i + 1]) for i in range(NS)])
            for n in (4, 8):
                if s >= n:
                    continue
                bt, bl = batched[n]
                e = max(rel_err(bl[i, s], ref[i + 1]) for i in range(NS))
                print(f"[err] config-5 dims seq {s}: decode_batch of {n}, max {e:.3e}", flush=True)
                assert e < LOGIT_TOL
                assert (bt[s] == ref_toks).all()
            if s >= 4:
                continue
            e_pre = rel_err(last[s], ref[0])
            errs = [rel_err(gpu_lg[s][i], ref[i + 1]) for i in range(NS)]
            print(f"[err] config-5 dims seq {s}: prefill last logits {e_pre:.3e}, "
                  f"decode max {max(errs):.3e}", flush=True)
            assert e_pre < LOGIT_TOL
            assert max(errs) < LOGIT_TOL
            assert (ref_toks == gpu_tok[s]).all()
    finally:
        om.close()
        orc.set_threads(0)


def test_config5_dims_block32_two_layers_vs_oracle(hip, orc):
    """Block-32 int8 weights (builder-defined: one scale per 32 values of a
    row) at the config-5 tensor shapes with 2 layers; both models from the same
    seeded host init.  Two 64-token prompts: the batched prefill of the first 63
    tokens, then 8 greedy steps per sequence token by token, and the batched
    decode step of both sequences (decode_batch: the bf16-plane skinny kernel
    with per-block scales), against the oracle's block-32 greedy run (forward
    mode 2).  Identical tokens, logits within 1e-3 at every step."""
    cfg = dict(LLAMA3_8B, n_layers=2)
    NS, NP = 8, 64
    print("[case] config-5 dims, 2 layers, block-32: host init (GPU and oracle)", flush=True)
    orc.set_threads(16)
    om = orc.Llama(orc.LlamaConfig(**cfg), 7, quantize=True, keep_f32=False, block32=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**cfg), 7, hip.QUANT_BLOCK32)
    V = cfg["vocab_size"]
    prompts = np.stack([orc.prompt_ids(s + 11, NP, V) for s in range(2)])
    try:
        print("[case] config-5 dims, block-32: prefill + token-by-token decode", flush=True)
        caches = [hm.new_llama_kv_cache(NP + NS) for _ in range(2)]
        hm.prefill(caches, prompts[:, :NP - 1], want_logits=False)
        gpu = []
        for s in range(2):
            tok, pos, lgs, ts = int(prompts[s, NP - 1]), NP - 1, [], []
            for _ in range(NS):
                lg, am = hm.forward_with_llama_cache(tok, pos, caches[s])
                lgs.append(lg)
                ts.append(am)
                tok, pos = am, pos + 1
            gpu.append((np.array(ts), np.stack(lgs)))
            caches[s].free()
        print("[case] config-5 dims, block-32: decode_batch of 2 sequences", flush=True)
        cs = [hm.new_llama_kv_cache(NP + NS) for _ in range(2)]
        hm.prefill(cs, prompts[:, :NP - 1], want_logits=False)
        bt, bl = hm.decode_batch(cs, prompts[:, NP - 1], NS, want_logits=True)
        for c in cs:
            c.free()
    finally:
        hm.free()
    try:
        for s in range(2):
            print(f"[case] config-5 dims, block-32: oracle greedy run of sequence {s}", flush=True)
            ref_t, ref_l = om.generate_greedy(prompts[s], NS, mode=2, want_logits=True)
            e = max(rel_err(gpu[s][1][i], ref_l[i]) for i in range(NS))
            eb = max(rel_err(bl[i, s], ref_l[i]) for i in range(NS))
            print(f"[err] config-5 dims block-32 seq {s}: decode {e:.3e}, decode_batch {eb:.3e}", flush=True)
            assert e < LOGIT_TOL and eb < LOGIT_TOL
            assert (gpu[s][0] == ref_t).all()
            assert (bt[s] == ref_t).all()
    finally:
        om.close()
        orc.set_threads(0)


@pytest.fixture(scope="module")
def model8b(hip):
    print("[case] config 5 model: Llama-3-8B shape, seed 0, device init (as bench.py)", flush=True)
    hm = hip.LlamaModel.new_random(hip.LlamaConfig(**LLAMA3_8B), seed=0, init_on_device=True)
    yield hm
    hm.free()


def test_config5_full_depth_one_sequence_vs_oracle(hip, orc, model8b):
    """BASELINE config 5 at full depth (32 layers, GQA 32:8, ffn 14336,
    V 128256; nn/llama.rs:683-700, 744-763) on one sequence: a 65-token seeded
    prompt (seed 1), its first 64 tokens through the batched prefill, then 8
    greedy steps (generate.rs:51-89) -- against the oracle on the GPU model's
    own int8 weights: identical tokens, logits within 1e-3 at every step."""
    cfg = LLAMA3_8B
    V = cfg["vocab_size"]
    prompt = orc.prompt_ids(1, 65, V)
    print("[case] config 5 full depth: 64-token batched prefill + 8 greedy", flush=True)
    toks, lg = model8b.generate_greedy(prompt, 8, want_logits=True, prefill=True)
    assert len(toks) == 8
    orc.set_threads(16)
    om = oracle_from_gpu(orc, model8b, cfg)
    try:
        seq = np.concatenate([prompt, toks[:-1]])  # 72 rows; row 64 + i gives step i
        cache = om.new_cache(len(seq))
        print("[case] config 5 oracle: layer-major cache path over 72 rows", flush=True)
        ref = om.forward_cache_seq(cache, seq, 0, n_logits=8)
        del cache
    finally:
        om.close()
        orc.set_threads(0)
    errs = np.array([rel_err(lg[i], ref[i]) for i in range(8)])
    ref_toks = np.array([orc.argmax(ref[i]) for i in range(8)])
    print(f"[err] config 5 full depth: max step rel err {errs.max():.3e}; tokens {toks.tolist()}; "
          f"smallest top-1/top-2 margin {min(top2_margin(ref[i]) for i in range(8)):.4g}", flush=True)
    assert errs.max() < LOGIT_TOL
    assert (ref_toks == toks).all()


def test_config5_full_batched_prefill_vs_token_by_token(hip, orc, model8b):
    """BASELINE config 5 at full size: 4 x 2048-token prompts (seeds 1-4), the
    first 2047 tokens of each through one batched prefill, then 64 greedy
    steps per sequence -- against the GPU's token-by-token cache path of each
    sequence (generate.rs:51-89): identical tokens, logits within 1e-3."""
    cfg = LLAMA3_8B
    print("[case] config 5 full: batched prefill 4 x 2047 + 64 greedy vs token by token",
          flush=True)
    hm = model8b
    V = cfg["vocab_size"]
    prompts = np.stack([orc.prompt_ids(s + 1, 2048, V) for s in range(4)])
    caches = []
    try:
        caches = [hm.new_llama_kv_cache(2048 + 64) for _ in range(4)]
        hm.prefill(caches, prompts[:, :2047], want_logits=False)
        for s in range(4):
            tok, pos, lgs, ts = int(prompts[s, 2047]), 2047, [], []
            for _ in range(64):
                lg, am = hm.forward_with_llama_cache(tok, pos, caches[s])
                lgs.append(lg)
                ts.append(am)
                tok, pos = am, pos + 1
            caches[s].free()
            print(f"[case] config 5 seq {s}: token-by-token generate", flush=True)
            ref_tok, ref_lg = hm.generate_greedy(prompts[s], 64, want_logits=True)
            err = max(rel_err(lgs[i], ref_lg[i]) for i in range(64))
            print(f"[err] config 5 seq {s}: max step rel err {err:.3e}; tokens "
                  f"{np.array(ts[:4]).tolist()}", flush=True)
            assert err < LOGIT_TOL
            assert (np.array(ts) == ref_tok).all()
    finally:
        for c in caches:
            c.free()
