"""HuggingFace safetensors checkpoints (LlamaModel::from_safetensors,
llama.rs:765-958) on the GPU against the CPU oracle.

The checkpoints are written here with the safetensors package (torch API):
BF16, F16 and F32 tensors over two shards, non-unit RMSNorm weights and a
non-default eps.  The oracle gets the same weights by the reference's route:
widened to f32 (BF16 as the upper half of an f32, F16 by IEEE decoding),
transposed to [in, out], q/k/v fused, quantize_symmetric per tensor, and the
loaded norms with config.rms_norm_eps.

Bars: int8 weights and scales bit-exact; the embedding table bit-exact
(including F16 subnormals, infinities and NaN payloads, checked against numpy's
independent half decoding); decode and batched-forward logits within 1e-3
relative, identical greedy tokens; error messages for a missing tensor, an
unsupported dtype, a wrong shape and an unreadable file.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")

LOGIT_TOL = 1e-3
BASE = dict(vocab_size=512, hidden_size=128, intermediate_size=256, n_layers=2, n_heads=4,
            n_kv_heads=2, max_seq_len=96, rope_theta=10000.0, rms_norm_eps=1e-6)


def rel_err(g, c):
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    return np.abs(g - c).max() / max(np.abs(c).max(), 1e-6)


def widened(t):
    """The f32 values the reference reads from a stored tensor (llama.rs:1070-1129)."""
    if t.dtype == torch.bfloat16:
        bits = t.view(torch.int16).numpy().astype(np.uint16).astype(np.uint32) << 16
        return bits.view(np.float32)
    if t.dtype == torch.float16:
        return t.numpy().astype(np.float32)  # numpy's half decoding, exact
    return t.numpy().astype(np.float32)


def make_checkpoint(tmp_path, cfg, seed, tied, dtypes):
    """Random HF-layout tensors; returns (paths, tensors by name)."""
    rng = np.random.default_rng(seed)
    h, ffn, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    hd = h // cfg["n_heads"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    shapes = {"model.embed_tokens.weight": (V, h), "model.norm.weight": (h,)}
    for i in range(cfg["n_layers"]):
        p = f"model.layers.{i}"
        shapes.update({
            f"{p}.self_attn.q_proj.weight": (qd, h), f"{p}.self_attn.k_proj.weight": (kvd, h),
            f"{p}.self_attn.v_proj.weight": (kvd, h), f"{p}.self_attn.o_proj.weight": (h, qd),
            f"{p}.mlp.gate_proj.weight": (ffn, h), f"{p}.mlp.up_proj.weight": (ffn, h),
            f"{p}.mlp.down_proj.weight": (h, ffn), f"{p}.input_layernorm.weight": (h,),
            f"{p}.post_attention_layernorm.weight": (h,)})
    if not tied:
        shapes["lm_head.weight"] = (V, h)
    tensors = {}
    for j, (name, shape) in enumerate(shapes.items()):
        if name.endswith("norm.weight"):
            a = (1.0 + 0.25 * rng.standard_normal(shape)).astype(np.float32)
        else:
            a = (0.05 * rng.standard_normal(shape)).astype(np.float32)
        tensors[name] = torch.from_numpy(a).to(dtypes[j % len(dtypes)]).contiguous()
    names = list(tensors)
    half = len(names) // 2
    paths = []
    for k, part in enumerate((names[:half], names[half:])):
        path = tmp_path / f"model-{k + 1:05d}-of-00002.safetensors"
        st_torch.save_file({n: tensors[n] for n in part}, str(path), metadata={"format": "pt"})
        paths.append(str(path))
    return paths, tensors


def oracle_model(orc, cfg, tensors, tied, block32=False):
    """The reference's from_safetensors + int8 layout step, on the oracle
    (block32: also the block-32 weights, for forward mode 2)."""
    c = dict(cfg, tie_word_embeddings=tied)
    om = orc.Llama(orc.LlamaConfig(**c), None)
    h, n_layers = cfg["hidden_size"], cfg["n_layers"]
    f = {n: widened(t) for n, t in tensors.items()}
    om.set_embed(f["model.embed_tokens.weight"])
    for i in range(n_layers):
        p = f"model.layers.{i}"
        qkv = np.concatenate([f[f"{p}.self_attn.{x}_proj.weight"].T for x in "qkv"], axis=1)
        for tid, w in ((orc.T_QKV, qkv), (orc.T_O, f[f"{p}.self_attn.o_proj.weight"].T),
                       (orc.T_GATE, f[f"{p}.mlp.gate_proj.weight"].T),
                       (orc.T_UP, f[f"{p}.mlp.up_proj.weight"].T),
                       (orc.T_DOWN, f[f"{p}.mlp.down_proj.weight"].T)):
            q, s = orc.quantize_symmetric(np.ascontiguousarray(w))
            om.set_qtensor(tid, i, q, s)
            if block32:
                q32, s32 = orc.quantize_block32(np.ascontiguousarray(w), w.shape[0], w.shape[1])
                om.set_qtensor_b32(tid, i, q32, s32)
        om.set_norm(0, i, f[f"{p}.input_layernorm.weight"], cfg["rms_norm_eps"])
        om.set_norm(1, i, f[f"{p}.post_attention_layernorm.weight"], cfg["rms_norm_eps"])
    om.set_norm(2, 0, f["model.norm.weight"], cfg["rms_norm_eps"])
    lm = f["model.embed_tokens.weight"] if tied else f["lm_head.weight"]
    q, s = orc.quantize_symmetric(lm)
    om.set_qtensor(orc.T_LM_HEAD, 0, q, s)
    if block32:  # the LM head is stored [V, h]: blocks of 32 along each row
        V, h = lm.shape
        nb = (h + 31) // 32
        q32 = np.empty((V, h), np.int8)
        s32 = np.empty((V, nb), np.float32)
        for j in range(V):
            for b in range(nb):
                q32[j, 32 * b:32 * b + 32], s32[j, b] = orc.quantize_symmetric(lm[j, 32 * b:32 * b + 32])
        om.set_qtensor_b32(orc.T_LM_HEAD, 0, q32, s32)
    return om


@pytest.mark.parametrize("tied", [False, True])
def test_loaded_model_matches_oracle(tmp_path, orc, hip, tied):
    print(f"[case] safetensors tiny Llama, tied={tied}", flush=True)
    dtypes = [torch.bfloat16, torch.float16, torch.float32]
    paths, tensors = make_checkpoint(tmp_path, BASE, 11, tied, dtypes)
    cfg = hip.LlamaConfig(**dict(BASE, tie_word_embeddings=tied))
    hm = hip.LlamaModel.from_safetensors(cfg, paths)
    om = oracle_model(orc, BASE, tensors, tied)
    # the layout step: int8 values and scales bit for bit
    for layer in range(BASE["n_layers"]):
        for tid in (orc.T_QKV, orc.T_O, orc.T_GATE, orc.T_UP, orc.T_DOWN):
            qg, sg = hm.qtensor(tid, layer)
            qo, so = om.qtensor(tid, layer)
            assert np.array_equal(qg, qo) and sg == so, (tid, layer)
    qg, sg = hm.qtensor(orc.T_LM_HEAD)
    qo, so = om.qtensor(orc.T_LM_HEAD)
    assert np.array_equal(qg, qo) and sg == so
    assert np.array_equal(hm.embed().view(np.uint32),
                          widened(tensors["model.embed_tokens.weight"]).ravel().view(np.uint32))
    # decode with the loaded norms and eps, against the oracle
    prompt = orc.prompt_ids(2, 12, BASE["vocab_size"])
    ref_t, ref_l = om.generate_greedy(prompt, 24, mode=1, want_logits=True)
    gt, gl = hm.generate_greedy(prompt, 24, want_logits=True)
    err = max(rel_err(gl[i], ref_l[i]) for i in range(len(ref_t)))
    print(f"[err] decode logits {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    assert (gt == ref_t).all()
    # batched forward (prefill kernels) with the same norms
    toks = orc.prompt_ids(3, 20, BASE["vocab_size"])
    fr = om.forward(toks, mode=1)
    fg = hm.forward(toks)
    ef = max(rel_err(fg[i], fr[i]) for i in range(len(toks)))
    print(f"[err] forward logits {ef:.3e}", flush=True)
    assert ef < LOGIT_TOL
    hm.free()
    om.close()


def test_loaded_block32_model_matches_oracle(tmp_path, orc, hip):
    """The loader with block-32 int8 weights (quant_mode 1): the oracle gets
    the same block-32 quantization of the widened weights (forward mode 2)."""
    print("[case] safetensors tiny Llama, block-32 int8", flush=True)
    paths, tensors = make_checkpoint(tmp_path, BASE, 13, False, [torch.bfloat16, torch.float32])
    cfg = hip.LlamaConfig(**dict(BASE, tie_word_embeddings=False))
    hm = hip.LlamaModel.from_safetensors(cfg, paths, hip.QUANT_BLOCK32)
    om = oracle_model(orc, BASE, tensors, False, block32=True)
    prompt = orc.prompt_ids(4, 10, BASE["vocab_size"])
    ref_t, ref_l = om.generate_greedy(prompt, 20, mode=2, want_logits=True)
    gt, gl = hm.generate_greedy(prompt, 20, want_logits=True)
    err = max(rel_err(gl[i], ref_l[i]) for i in range(len(ref_t)))
    print(f"[err] block-32 decode logits {err:.3e}", flush=True)
    assert err < LOGIT_TOL
    assert (gt == ref_t).all()
    hm.free()
    om.close()


def test_f16_special_values_widen_exactly(tmp_path, hip):
    """F16 zeros, subnormals, the extremes, infinities and NaNs with payloads
    widen to the f32 bits of IEEE half decoding (numpy's, independent)."""
    cfg = dict(BASE, n_layers=1)
    paths, tensors = make_checkpoint(tmp_path, cfg, 5, True, [torch.float16])
    emb = tensors["model.embed_tokens.weight"].clone()
    special = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03ff, 0x0200, 0x0400, 0x7bff, 0xfbff,
                        0x7c00, 0xfc00, 0x7e00, 0x7c01, 0xfd55, 0x3c00, 0x3555], np.uint16)
    flat = emb.view(torch.int16).view(-1)
    flat[: special.size] = torch.from_numpy(special.view(np.int16))
    tensors["model.embed_tokens.weight"] = emb
    st_torch.save_file({n: t for n, t in tensors.items()}, str(tmp_path / "one.safetensors"))
    hm = hip.LlamaModel.from_safetensors(hip.LlamaConfig(**dict(cfg, tie_word_embeddings=True)),
                                         [str(tmp_path / "one.safetensors")])
    got = hm.embed().view(np.uint32)
    want = emb.numpy().astype(np.float32).ravel().view(np.uint32)
    assert np.array_equal(got, want)
    hm.free()


def test_loader_errors(tmp_path, hip):
    cfg = dict(BASE, n_layers=1)
    paths, tensors = make_checkpoint(tmp_path, cfg, 7, False, [torch.float32])
    lcfg = hip.LlamaConfig(**dict(cfg, tie_word_embeddings=False))

    def expect(files, text):
        with pytest.raises(hip.ScryHipError) as ei:
            hip.LlamaModel.from_safetensors(lcfg, files)
        print(f"[err] {ei.value}", flush=True)
        assert text in str(ei.value)

    one = str(tmp_path / "x.safetensors")
    # a missing tensor (the reference's message, llama.rs:808-810)
    st_torch.save_file({n: t for n, t in tensors.items() if n != "lm_head.weight"}, one)
    expect([one], "tensor 'lm_head.weight' not found in any shard")
    # an unsupported dtype (llama.rs:801-804)
    bad = dict(tensors)
    bad["model.norm.weight"] = torch.ones(cfg["hidden_size"], dtype=torch.int32)
    st_torch.save_file(bad, one)
    expect([one], "unsupported dtype I32 for tensor 'model.norm.weight'")
    # a shape that does not match the config
    bad = dict(tensors)
    bad["model.layers.0.mlp.down_proj.weight"] = tensors["model.layers.0.mlp.up_proj.weight"].clone()
    st_torch.save_file(bad, one)
    expect([one], "tensor 'model.layers.0.mlp.down_proj.weight': shape [256, 128], expected [128, 256]")
    # an unreadable file, and a file that is not safetensors
    expect([str(tmp_path / "absent.safetensors")], "failed to read")
    (tmp_path / "junk.safetensors").write_bytes(b"\xff" * 64)
    expect([str(tmp_path / "junk.safetensors")], "header length")
    # the complete checkpoint still loads from the original shards
    hip.LlamaModel.from_safetensors(lcfg, paths).free()


def _with_norm_weights(tmp_path, cfg, tensors, edits):
    """The checkpoint with RMSNorm weight entries replaced: {(name, index): value}."""
    t = {n: v.clone() for n, v in tensors.items()}
    for (name, idx), val in edits.items():
        a = t[name].to(torch.float32)
        a[idx] = val
        t[name] = a.contiguous()
    path = tmp_path / "edited.safetensors"
    st_torch.save_file(t, str(path), metadata={"format": "pt"})
    return [str(path)], t


def test_forward_outlier_channels_vs_oracle(tmp_path, orc, hip):
    """Norm weights with outlier channels (x300, x-500), so one value of every
    normalised row dwarfs the rest.  The int8 prefill GEMMs hold each row as
    24-bit fixed point scaled to its largest value (absolute error 2^-24 of
    it), so this is their widest per-row range; the logits stay within the bar."""
    cfg = dict(BASE)
    _, tensors = make_checkpoint(tmp_path, cfg, 17, False, [torch.float32])
    edits = {}
    for i in range(cfg["n_layers"]):
        edits[(f"model.layers.{i}.input_layernorm.weight", 3 + i)] = 300.0
        edits[(f"model.layers.{i}.post_attention_layernorm.weight", 40 + i)] = -500.0
    edits[("model.norm.weight", 7)] = 400.0
    paths, t2 = _with_norm_weights(tmp_path, cfg, tensors, edits)
    print("[case] forward with outlier norm channels", flush=True)
    hm = hip.LlamaModel.from_safetensors(hip.LlamaConfig(**dict(cfg, tie_word_embeddings=False)), paths)
    om = oracle_model(orc, cfg, t2, False)
    toks = orc.prompt_ids(5, 40, cfg["vocab_size"])
    fr = om.forward(toks, mode=1)
    fg = hm.forward(toks)
    ef = max(rel_err(fg[i], fr[i]) for i in range(len(toks)))
    print(f"[err] forward logits {ef:.3e}", flush=True)
    assert ef < LOGIT_TOL
    hm.free()
    om.close()


def test_forward_nonfinite_norm_output(tmp_path, orc, hip):
    """An infinite RMSNorm weight makes one value of every normalised row
    infinite: the prefill GEMMs' digit rows carry a non-finite marker and
    give NaN, as the reference's sums of inf * q do; every logit is NaN on
    both sides."""
    cfg = dict(BASE, n_layers=1)
    _, tensors = make_checkpoint(tmp_path, cfg, 19, False, [torch.float32])
    paths, t2 = _with_norm_weights(tmp_path, cfg, tensors,
                                   {("model.layers.0.input_layernorm.weight", 5): float("inf")})
    print("[case] forward with an infinite norm weight", flush=True)
    hm = hip.LlamaModel.from_safetensors(hip.LlamaConfig(**dict(cfg, tie_word_embeddings=False)), paths)
    om = oracle_model(orc, cfg, t2, False)
    toks = orc.prompt_ids(6, 10, cfg["vocab_size"])
    fr = np.asarray(om.forward(toks, mode=1))
    fg = np.asarray(hm.forward(toks))
    print(f"[nan] oracle {np.isnan(fr).mean():.3f} gpu {np.isnan(fg).mean():.3f}", flush=True)
    assert np.isnan(fr).all() and np.isnan(fg).all()
    hm.free()
    om.close()


def test_decode_batch_nonfinite_norm_output(tmp_path, orc, hip):
    """The batched decode step with an infinite input RMSNorm weight in the
    first layer: q, k and v of every row hold infinities or NaN (the int8-digit
    projections give NaN for the row segment holding the infinity, the
    reference +-inf or NaN per column), the attention softmax makes both NaN
    (cpu.rs:336-366), and every logit of the first step is NaN on both sides
    (one-token prompts: no prefill)."""
    cfg = dict(BASE, n_layers=1)
    _, tensors = make_checkpoint(tmp_path, cfg, 23, False, [torch.float32])
    paths, t2 = _with_norm_weights(tmp_path, cfg, tensors,
                                   {("model.layers.0.input_layernorm.weight", 5): float("inf")})
    print("[case] decode_batch with an infinite norm weight", flush=True)
    hm = hip.LlamaModel.from_safetensors(hip.LlamaConfig(**dict(cfg, tie_word_embeddings=False)), paths)
    om = oracle_model(orc, cfg, t2, False)
    prompts = [orc.prompt_ids(7 + i, 1, cfg["vocab_size"]) for i in range(3)]
    caches = [hm.new_llama_kv_cache(16) for _ in prompts]
    _, lg = hm.decode_batch(caches, [int(p[0]) for p in prompts], 2, want_logits=True)
    for c in caches:
        c.free()
    for i, p in enumerate(prompts):
        _, rl = om.generate_greedy(np.asarray(p, np.int64), 2, mode=1, want_logits=True)
        print(f"[nan] sequence {i}: oracle {np.isnan(np.asarray(rl[0])).mean():.3f} "
              f"gpu {np.isnan(lg[0, i]).mean():.3f}", flush=True)
        assert np.isnan(np.asarray(rl[0])).all() and np.isnan(lg[0, i]).all()
    hm.free()
    om.close()


def _same_nonfinite(g, r):
    """Equal NaN positions and equal values elsewhere (infinities included)."""
    g, r = np.asarray(g), np.asarray(r)
    ng, nr = np.isnan(g), np.isnan(r)
    return np.array_equal(ng, nr) and np.array_equal(g[~ng], r[~nr])


def test_nonfinite_final_norm_logits(tmp_path, orc, hip):
    """An infinite final-norm weight: every LM-head column sums one infinite
    term, so the reference's logits are +inf, -inf or NaN per column (NaN where
    q = 0; cpu.rs:1128-1160).  The single-sequence GEMV, the batched decode's
    int8-digit LM head and the prefill GEMM of forward() give exactly that
    pattern, and the greedy tokens (generate.rs:167-173) agree."""
    cfg = dict(BASE, n_layers=1)
    V = cfg["vocab_size"]
    _, tensors = make_checkpoint(tmp_path, cfg, 29, False, [torch.float32])
    paths, t2 = _with_norm_weights(tmp_path, cfg, tensors, {("model.norm.weight", 9): float("inf")})
    print("[case] infinite final-norm weight: decode, decode_batch, forward", flush=True)
    hm = hip.LlamaModel.from_safetensors(hip.LlamaConfig(**dict(cfg, tie_word_embeddings=False)), paths)
    om = oracle_model(orc, cfg, t2, False)
    prompts = [orc.prompt_ids(31 + i, 1, V) for i in range(3)]
    caches = [hm.new_llama_kv_cache(16) for _ in prompts]
    bt, bl = hm.decode_batch(caches, [int(p[0]) for p in prompts], 3, want_logits=True)
    for c in caches:
        c.free()
    for i, p in enumerate(prompts):
        rt, rl = om.generate_greedy(np.asarray(p, np.int64), 3, mode=1, want_logits=True)
        st, sl = hm.generate_greedy(p, 3, want_logits=True)
        r0 = np.asarray(rl[0])
        print(f"[nan] sequence {i}: oracle +inf {np.isposinf(r0).mean():.3f} -inf {np.isneginf(r0).mean():.3f} "
              f"NaN {np.isnan(r0).mean():.3f}; tokens {list(rt)} gpu {list(st)} batched {list(bt[i])}", flush=True)
        assert np.isinf(r0).any()
        for t in range(3):
            assert _same_nonfinite(sl[t], rl[t]), (i, t)
            assert _same_nonfinite(bl[t, i], rl[t]), (i, t)
        assert (np.asarray(st) == np.asarray(rt)).all()
        assert (bt[i] == np.asarray(rt)).all()
    toks = orc.prompt_ids(37, 6, V)
    fr = np.asarray(om.forward(toks, mode=1))
    fg = np.asarray(hm.forward(toks))
    for i in range(len(toks)):
        assert _same_nonfinite(fg[i], fr[i]), i
    hm.free()
    om.close()
