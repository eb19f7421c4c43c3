#!/usr/bin/env python3
"""Headline benchmark: Llama-2-7B-shape int8 batch-1 greedy decode on one MI355X.

Workload: dim 4096, 32 layers, 32 heads, FFN 11008,
vocab 32000, RoPE theta 1e4, untied lm_head, random-init N(0, 0.02) weights
(fastrand seed 0) quantized per tensor to int8, batch 1, a 512-token seeded
prompt (seed 1) fed through the cache path, then greedy decode steps.

A "step" is one decode token (all 32 layers + lm_head + device argmax), one
replay of the captured decode-step graph.  W untimed warm-up steps run after the
prompt; the position is then rewound to the first decode position and exactly K
steps are timed with HIP events on the launch stream (device synchronised
before and after).  value = K / elapsed = decode tok/s on the one GPU.

Also reported:
  roofline      the dominant projection kernel (largest device time per token),
                timed with HIP events over launches that rotate through all 32
                layers' weights (so they stream from HBM, not the 256 MB MALL);
                achieved = algorithmic bytes per launch / average launch time;
                traffic = HBM bytes per launch from the committed rocprofv3
                FETCH_SIZE / WRITE_SIZE summary (profiles/)
  cpu_baseline  the oracle (C restatement of the reference CPU path) on the same
                int8 weights, reference-faithful single-threaded
                matmul_i8_f32_tiled, timed over a few decode steps on the host
  prefill       BASELINE config 5 (Llama-3-8B shape, 4 x 2048-token prompts):
                batched prefill of the first 2047 tokens of each prompt on the
                matrix cores, then 64 greedy decode steps per sequence

  bf16_decode   the same decode with the model in bf16 (the reference's bf16
                feature): tok/s and the per-projection GEMV rates
  gemv_micro    BASELINE configs 2 and 3: matmul_i8_f32 at 1, 4 and 16 rows,
                block-32 and per-tensor scales, 1000 launches over 32 weight
                copies: median / p10 / p90 per-launch device time

Profiling modes (no JSON line): --pmc-probe runs a 256 MiB device copy (the
counter calibration), each decode projection kernel over all layers and
decode attention at 640 cached rows;
--prefill-profile runs the config-5 batched prefill twice without decode;
--prefill-only runs the config-5 measurement alone; --gemv-only the
configs 2 / 3 micro-benchmark alone.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0  # dense
INT8_MFMA_PEAK_TOPS = 5000.0  # dense
# Matrix-core busy fraction of the config-5 prefill's projection GEMMs and
# attention, from the rocprofv3 counter run in
# profiles/prefill_llama3_8b_mfma_counters.md (SQ_VALU_MFMA_BUSY_CYCLES over
# GRBM_GUI_ACTIVE / 8 x 1024 SIMDs); counters cannot be read inside this
# process, so the line carries the profile's figures with their source.
PREFILL_MFMA_BUSY_PROFILE = {"qkv": 0.553, "o": 0.503, "gate_up": 0.584, "down": 0.583, "attention": 0.343,
                             "prefill": 0.502, "source": "profiles/prefill_llama3_8b_mfma_counters.md"}
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_projections_pmc_traffic.md")


def measured_traffic(kernel: str):
    """HBM bytes per launch of a decode projection kernel, from the committed
    rocprofv3 PMC summary (None when it has no figure for it)."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def prefill_config5(E, n_seq: int = 4, n_prompt: int = 2048, decode_steps: int = 64) -> dict:
    """BASELINE config 5 on the GPU: batched prefill, then greedy decode; and
    the same prefill with the model in bf16 (the reference's bf16 feature)."""
    import esolearn_amd.llama as EL
    cfg = E.LlamaConfig.llama3_8b()
    t0 = time.perf_counter()
    m = E.LlamaModel.new_random(cfg, seed=0)
    t_init = time.perf_counter() - t0
    prompts = [E.synth.prompt_ids(s + 1, n_prompt, cfg.vocab_size) for s in range(n_seq)]
    import numpy as np
    pm, dm, toks = m.bench_prefill(np.stack(prompts), decode_steps)
    # the same prefill, then the four sequences decoded together per step
    # (one skinny matrix-core pass per projection over the 4 rows)
    pm_b, dm_b, toks_b = m.bench_prefill(np.stack(prompts), decode_steps, batched=True)
    m.free()
    mb = E.LlamaModel.new_random(cfg, seed=0, quant_mode=EL.QUANT_BF16, init_on_device=True)
    pm_bf16, _, toks_bf16 = mb.bench_prefill(np.stack(prompts), 1)
    mb.free()
    # the builder-defined block-32 int8 weights (one scale per 32 values of a
    # row; the GEMMs take the split-bf16 matrix-core path)
    m32 = E.LlamaModel.new_random(cfg, seed=0, quant_mode=EL.QUANT_BLOCK32, init_on_device=True)
    pm_b32, _, toks_b32 = m32.bench_prefill(np.stack(prompts), 1)
    m32.free()
    h, ffn, L = cfg.hidden_size, cfg.intermediate_size, cfg.n_layers
    hd = h // cfg.n_heads
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    rows = n_seq * (n_prompt - 1)
    proj = 2.0 * rows * L * (h * (qd + 2 * kvd) + qd * h + 2 * h * ffn + ffn * h)
    s = n_prompt - 1
    attn = 4.0 * n_seq * L * cfg.n_heads * (s * (s + 1) / 2) * hd
    tf = proj / (pm / 1e3) / 1e12
    print(f"[bench] prefill {n_seq}x{s}: {pm:.1f} ms ({rows / pm * 1e3:.0f} tok/s, projections "
          f"{tf:.1f} TFLOP/s); decode {n_seq}x{decode_steps}: {dm:.1f} ms, batched {dm_b:.1f} ms "
          f"(tokens equal: {bool((toks_b == toks).all())}); init {t_init:.1f} s; "
          f"bf16 model prefill {pm_bf16:.1f} ms; block-32 model prefill {pm_b32:.1f} ms", file=sys.stderr, flush=True)
    return {
        "workload": "llama3-8b-shape int8: 4 x 2048-token prompts, batched prefill of the first "
                    "2047 tokens each (GEMMs on the int8 matrix cores: activations as per-row 24-bit "
                    "fixed point in three int8 digits, exact integer sums), then 64 greedy decode "
                    "steps per sequence (BASELINE config 5)",
        "prefill_ms": round(pm, 2),
        "prefill_tok_s": round(rows / (pm / 1e3), 1),
        "projection_tflop": round(proj / 1e12, 2),
        "attention_tflop_causal": round(attn / 1e12, 2),
        "projection_tflops": round(tf, 1),
        "mfma_peak_tflops_bf16": BF16_MFMA_PEAK_TFLOPS,
        "mfma_peak_tops_int8": INT8_MFMA_PEAK_TOPS,
        "mfma_frac_useful": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
        # three int8 MFMA operations per product (one per activation digit)
        "mfma_frac_issued_int8": round(3 * tf / INT8_MFMA_PEAK_TOPS, 4),
        "mfma_busy_counters": PREFILL_MFMA_BUSY_PROFILE,
        "decode_ms": round(dm, 2),
        "decode_tok_s": round(n_seq * decode_steps / (dm / 1e3), 1),
        "decode_batched": {
            "mode": f"{n_seq} sequences per step (skinny matrix-core projections, one attention launch over all caches)",
            "decode_ms": round(dm_b, 2),
            "decode_tok_s": round(n_seq * decode_steps / (dm_b / 1e3), 1),
            "prefill_ms": round(pm_b, 2),
            "tokens_equal_per_sequence_decode": bool((toks_b == toks).all()),
        },
        "greedy_tokens_head": [[int(t) for t in row[:4]] for row in toks],
        "bf16_model_prefill_ms": round(pm_bf16, 2),
        "bf16_model_prefill_tok_s": round(rows / (pm_bf16 / 1e3), 1),
        "bf16_model_first_tokens": [int(t) for t in toks_bf16[:, 0]],
        "block32_model_prefill_ms": round(pm_b32, 2),
        "block32_model_prefill_tok_s": round(rows / (pm_b32 / 1e3), 1),
        "block32_model_first_tokens": [int(t) for t in toks_b32[:, 0]],
    }


def pmc_probe(E) -> None:
    """The workload of the committed PMC summaries: calibration copy, the decode
    projections, and decode attention at 640 cached rows."""
    import esolearn_amd.llama as EL
    B = E.HipBackend
    src = B.zeros(64 * 1024 * 1024)  # 256 MiB
    B.synchronize()
    for _ in range(3):
        dst = B.clone_storage(src)
        B.synchronize()
        dst.free()
    src.free()
    m = E.LlamaModel.new_random(E.LlamaConfig.llama2_7b(), seed=0)
    for name, tid in (("qkv", EL.T_QKV), ("o", EL.T_O), ("gate_up", EL.T_GATE),
                      ("down", EL.T_DOWN), ("lm_head", EL.T_LM_HEAD)):
        us, b = m.time_projection(tid, 32)
        print(f"[probe] {name} {us:.2f} us {b:.0f} B", flush=True)
    us, b = m.time_attention(640, 32)
    print(f"[probe] attention (640 rows) {us:.2f} us {b:.0f} B", flush=True)
    m.free()


def prefill_profile(E) -> None:
    """The workload of the committed prefill counter summaries: config 5's
    batched prefill (4 x 2047 tokens), twice, without the decode steps."""
    import numpy as np
    cfg = E.LlamaConfig.llama3_8b()
    print("[profile] config-5 model, device init", flush=True)
    m = E.LlamaModel.new_random(cfg, seed=0, init_on_device=True)
    prompts = np.stack([E.synth.prompt_ids(s + 1, 2048, cfg.vocab_size) for s in range(4)])
    for p in range(2):
        caches = [m.new_llama_kv_cache(2048) for _ in range(4)]
        print(f"[profile] prefill pass {p}", flush=True)
        m.prefill(caches, prompts[:, :2047], want_logits=False)
        E.HipBackend.synchronize()
        for c in caches:
            c.free()
    m.free()
    print("[profile] done", flush=True)


SAMPLING_SWEEP = [(0.8, 40, 0.95), (0.8, 0, 0.95), (1.0, 0, 1.0), (0.7, 0, 0.5)]


def sampling_sweep(E, EL, model, prompt, warmup: int, steps: int) -> dict:
    """Decode with the device sampler after each LM head (generate.rs:92-186)
    against greedy decode, same session shape; device time of the steps."""
    ms, _ = model.bench_decode(prompt, warmup, steps)
    out = {"greedy_tok_s": round(steps / (ms / 1000.0), 2), "configs": []}
    for T, k, p in SAMPLING_SWEEP:
        sc = EL.SamplingConfig(temperature=T, top_k=k, top_p=p, max_tokens=steps)
        ms_s, _ = model.bench_decode_sampled(prompt, warmup, steps, sc, seed=42)
        out["configs"].append({"temperature": T, "top_k": k, "top_p": p,
                               "tok_s": round(steps / (ms_s / 1000.0), 2),
                               "extra_us_per_step": round((ms_s - ms) / steps * 1000.0, 2)})
        print(f"[bench] sampled T={T} k={k} p={p}: {out['configs'][-1]['tok_s']} tok/s, "
              f"+{out['configs'][-1]['extra_us_per_step']} us/step", file=sys.stderr, flush=True)
    return out


LINEAR_SHAPES = [("gpt2 c_attn", 768, 2304), ("gpt2 c_fc", 768, 3072), ("gpt2 c_proj", 3072, 768),
                 ("whisper-base fc1", 512, 2048), ("whisper-base fc2", 2048, 512),
                 ("whisper-large fc1", 1280, 5120), ("whisper-large fc2", 5120, 1280)]


def linear_sweep(E) -> list:
    """Quantized Linear::forward with bias (linear.rs:67-94) at one row: the
    dequant-fused GEMV, bias in its store epilogue.  Each shape rotates over
    about 1 GB of weight copies, so HBM (not the 256 MB Infinity Cache) serves
    the weights."""
    from esolearn_amd.linear import bench_linear_bias
    out = []
    for name, k, n in LINEAR_SHAPES:
        n_bufs = max(64, (1 << 30) // (k * n))
        us, b = bench_linear_bias(1, k, n, n_bufs=n_bufs, warmup=100, iters=2000)
        gbs = b / us / 1e3
        out.append({"layer": name, "in": k, "out": n, "rows": 1, "avg_us": round(us, 3),
                    "bytes": int(b), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        print(f"[bench] linear {name:18s} {k}x{n}: {us:7.2f} us {gbs:7.1f} GB/s", file=sys.stderr, flush=True)
    return out


BF16_SHAPES = [("q/k/v/o", 4096, 4096), ("gate/up", 4096, 11008), ("down", 11008, 4096),
               ("lm_head", 4096, 32000)]


def bf16_sweep(E) -> list:
    """bf16 mode (the reference's bf16 feature): matmul with bf16 weight rows at
    one activation row, Llama-2-7B projection shapes; about 1 GB of weight
    copies per shape."""
    import ctypes as C
    from esolearn_amd._lib import call
    out = []
    for name, k, n in BF16_SHAPES:
        n_bufs = max(4, (1 << 30) // (2 * k * n))
        us, b = C.c_double(), C.c_double()
        call("scry_hip_bench_gemv_bf16", 1, k, n, n_bufs, 50, 500, C.byref(us), C.byref(b))
        gbs = b.value / us.value / 1e3
        out.append({"proj": name, "in": k, "out": n, "rows": 1, "avg_us": round(us.value, 3),
                    "bytes": int(b.value), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        print(f"[bench] bf16 gemv {name:8s} {k}x{n}: {us.value:7.2f} us {gbs:7.1f} GB/s",
              file=sys.stderr, flush=True)
    return out


GEMV_CASES = [("config 2: attention projection", 4096, 4096, (1,)),
              ("config 3: gate/up", 4096, 11008, (1, 4, 16)),
              ("config 3: down", 11008, 4096, (1, 4, 16))]
FP32_VALU_PEAK_TFLOPS = 157.3


def gemv_micro(EL, iters: int = 1000, n_bufs: int = 32) -> list:
    """BASELINE configs 2 and 3: matmul_i8_f32 at batch 1, 4 and 16 with the
    reference's block (32-wide) scales and with per-tensor scales; iters timed
    launches over n_bufs distinct weight copies (more than the 256 MB Infinity
    Cache): the back-to-back average, and median and p10 / p90 of the
    per-launch device time of each group of 8 consecutive launches (an event
    between single launches would add its own gap to every sample).  Above one
    row the GEMV (up to 4 rows per weight pass), the skinny MFMA kernel (every
    weight byte once for up to 16 rows; matmul_i8_f32's route there) and, at 16
    rows, the prefill MFMA GEMM are timed."""
    import numpy as np
    out = []
    for name, k, n, ms in GEMV_CASES:
        for qm, qname in ((EL.QUANT_BLOCK32, "block-32"), (EL.QUANT_PER_TENSOR, "per-tensor")):
            for m in ms:
                for path in ((1, 3, 2) if m == 16 else (1, 3) if m > 1 else (0,)):
                    per, avg, b = EL.bench_qgemv_dist(m, k, n, qm, path, n_bufs, 50, iters, 8)
                    p10, med, p90 = (float(v) for v in np.percentile(per, [10, 50, 90]))
                    fl = 2.0 * m * k * n
                    e = {"case": name, "k": k, "n": n, "m": m, "scales": qname,
                         "kernel": {2: "mfma gemm", 3: "skinny mfma"}.get(path, "gemv"),
                         "iters": iters, "weight_buffers": n_bufs, "group": 8,
                         "median_us": round(med, 3), "p10_us": round(p10, 3), "p90_us": round(p90, 3),
                         "avg_us": round(avg, 3), "bytes": int(b),
                         "gbs_avg": round(b / avg / 1e3, 1), "hbm_frac_avg": round(b / avg / 1e3 / HBM_PEAK_GBS, 4),
                         "gbs_median": round(b / med / 1e3, 1), "hbm_frac_median": round(b / med / 1e3 / HBM_PEAK_GBS, 4),
                         "tflops_median": round(fl / med / 1e6, 2)}
                    out.append(e)
                    print(f"[bench] gemv {name:32s} m={m:2d} {qname:10s} {e['kernel']:11s} median {med:7.2f} us "
                          f"(p10 {p10:6.2f} p90 {p90:6.2f}) {e['gbs_median']:7.1f} GB/s {e['tflops_median']:6.2f} TFLOP/s",
                          file=sys.stderr, flush=True)
    return out


def step_profile(model, cfg, prompt, steps: int) -> dict:
    """Per-launch durations and gaps of the graph-replayed decode step
    (scry_hip_llama_profile_step: the step graph captured with per-workgroup
    s_memrealtime stamps, 100 MHz).  A launch's duration is its latest
    workgroup end minus its earliest workgroup start; its gap is its earliest
    start minus the previous launch's latest end.  Steps 2.. of the run
    (the first replay is excluded)."""
    import numpy as np

    st, en = model.profile_step(prompt, steps)
    st, en = st[1:], en[1:]
    L = cfg.n_layers
    kinds = ["qkv", "attention", "o", "gate_up", "down"]
    dur = en - st
    gap = np.zeros_like(st)
    gap[:, 1:] = st[:, 1:] - en[:, :-1]
    out = {"steps": int(st.shape[0]), "context": [len(prompt), len(prompt) + steps],
           "step_span_us": round(float(np.mean(en[:, -1])), 2),
           "sum_kernel_us": round(float(np.mean(dur.sum(axis=1))), 2),
           "sum_gap_us": round(float(np.mean(gap.sum(axis=1))), 2), "launches": {}}
    for j, k in enumerate(kinds):
        idx = [5 * l + j for l in range(L) if not (j == 0 and l == 0)]
        out["launches"][k] = {"count": len(idx), "mean_us": round(float(dur[:, idx].mean()), 2),
                              "mean_gap_before_us": round(float(gap[:, idx].mean()), 2),
                              "per_step_us": round(float(dur[:, idx].sum(axis=1).mean()), 1)}
    for name, i in (("qkv_layer0", 0), ("lm_head", 5 * L), ("finish", 5 * L + 1)):
        out["launches"][name] = {"count": 1, "mean_us": round(float(dur[:, i].mean()), 2),
                                 "mean_gap_before_us": round(float(gap[:, i].mean()), 2)}
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def weight_bytes(cfg) -> int:
    """int8 weight bytes + per-tensor scales read per decode token."""
    h, ffn, V, L = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.n_layers
    hd = h // cfg.n_heads
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    per_layer = h * (qd + 2 * kvd) + qd * h + 2 * h * ffn + ffn * h
    return L * per_layer + V * h + 4 * (5 * L + 1)


def bf16_decode(E, EL, cfg, prompt, warmup: int, steps: int, proj_iters: int) -> dict:
    """The same decode with the model in bf16 (the reference's bf16 feature:
    bf16 weights, activations cast to bf16 at each projection, f32
    accumulation), device init of the same seeded weights."""
    model = E.LlamaModel.new_random(cfg, seed=0, quant_mode=EL.QUANT_BF16, init_on_device=True)
    try:
        ms, toks = model.bench_decode(prompt, warmup, steps)
        proj = {}
        for name, tid in (("qkv", EL.T_QKV), ("o", EL.T_O), ("gate_up", EL.T_GATE),
                          ("down", EL.T_DOWN), ("lm_head", EL.T_LM_HEAD)):
            us, b = model.time_projection(tid, proj_iters)
            proj[name] = {"avg_us": round(us, 3), "bytes": int(b), "gbs": round(b / us / 1e3, 1),
                          "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
    finally:
        model.free()
    tok_s = steps / (ms / 1000.0)
    wb = 2 * (weight_bytes(cfg) - 4 * (5 * cfg.n_layers + 1))
    print(f"[bench] bf16 decode {tok_s:.1f} tok/s; gate_up {proj['gate_up']['gbs']} GB/s",
          file=sys.stderr, flush=True)
    return {"workload": "llama2-7b-shape bf16 batch-1 greedy decode, same prompt and steps",
            "tok_s": round(tok_s, 2), "ms_per_step": round(ms / steps, 4),
            "weight_bytes_per_token": wb,
            "decode_roofline_frac": round(tok_s * wb / (HBM_PEAK_GBS * 1e9), 4),
            "greedy_tokens_head": [int(t) for t in toks[:8]], "projections": proj}


def cpu_baseline(model, cfg, prompt, n_tok: int) -> dict:
    """Oracle decode on the GPU model's own int8 weights: reference-faithful
    single-threaded, and the bit-identical all-core mode beside it."""
    from oracle import oracle as O
    import esolearn_amd.llama as EL

    oc = O.LlamaConfig(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.n_layers,
                       cfg.n_heads, cfg.n_kv_heads, cfg.max_seq_len, cfg.rms_norm_eps,
                       cfg.rope_theta, cfg.tie_word_embeddings, cfg.rope_scaling)
    om = O.Llama(oc, None)
    for layer in range(cfg.n_layers):
        for tid in (EL.T_QKV, EL.T_O, EL.T_GATE, EL.T_UP, EL.T_DOWN):
            q, s = model.qtensor(tid, layer)
            om.set_qtensor(tid, layer, q, s)
    q, s = model.qtensor(EL.T_LM_HEAD)
    om.set_qtensor(EL.T_LM_HEAD, 0, q, s)
    del q
    om.set_embed(model.embed())
    # the bit-identical all-core mode: the same decode steps, one token at a
    # time through the layer-major cache path on every host core
    cores = min(16, os.cpu_count() or 1)
    O.set_threads(cores)
    cache = om.new_cache(n_tok + 1)
    t0 = time.perf_counter()
    for i in range(n_tok):
        om.forward_cache_seq(cache, [int(prompt[i])], i, n_logits=1)
    dt_all = time.perf_counter() - t0
    del cache
    O.set_threads(0)  # matmul_i8_f32_tiled exactly as written: one thread
    cache = om.new_cache(n_tok + 1)
    t0 = time.perf_counter()
    for i in range(n_tok):
        om.forward_with_cache(cache, int(prompt[i]), i, mode=1)
    dt = time.perf_counter() - t0
    om.close()
    model_name = cpu_model()
    return {
        "value": round(n_tok / dt, 5),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "cpu_model": model_name,
        "sample": (f"{n_tok} decode steps (positions 0..{n_tok - 1}) of the same "
                   "Llama-2-7B-shape int8 model on the host, oracle in reference-faithful "
                   "mode (single-threaded matmul_i8_f32_tiled, f64 products); "
                   f"{dt:.1f} s; host {model_name}, nproc {os.cpu_count()}"),
        "all_cores": {"value": round(n_tok / dt_all, 4), "unit": "tok/s", "cores": cores,
                      "mode": "bit-identical parallel oracle (layer-major cache path, SIMD across "
                              "output columns, the same per-element operation order)",
                      "seconds": round(dt_all, 2)},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps (K)")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode steps (W)")
    ap.add_argument("--prompt-len", type=int, default=512)
    ap.add_argument("--proj-iters", type=int, default=96)
    ap.add_argument("--cpu-tokens", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--host-init", action="store_true",
                    help="draw the random weights on the host (slow) instead of the GPU")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-5 prefill line")
    ap.add_argument("--pmc-probe", action="store_true", help="profiling workload only (see above)")
    ap.add_argument("--prefill-only", action="store_true", help="config-5 measurement only")
    ap.add_argument("--prefill-profile", action="store_true",
                    help="profiling workload only: config-5 prefill twice, no decode")
    ap.add_argument("--bf16-only", action="store_true",
                    help="bf16-mode GEMV (bf16 weights) at Llama-2-7B projection shapes only")
    ap.add_argument("--linear-only", action="store_true",
                    help="quantized Linear (bias GEMV) at GPT-2 / Whisper shapes only")
    ap.add_argument("--sampling-only", action="store_true",
                    help="greedy vs device-sampled decode over a few sampling configs only")
    ap.add_argument("--gemv-only", action="store_true",
                    help="the config 2 / 3 isolated GEMV micro-benchmark only")
    ap.add_argument("--no-gemv", action="store_true", help="skip the config 2 / 3 micro-benchmark")
    ap.add_argument("--no-bf16-decode", action="store_true", help="skip the bf16-model decode line")
    ap.add_argument("--step-profile", action="store_true",
                    help="per-launch durations and gaps of the graph-replayed decode step only")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on exactly one GPU (the int8 decode path has no "
              "multi-GPU mode: sequences would be sharded data-parallel). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import esolearn_amd as E
    import esolearn_amd.llama as EL

    E.init(0)
    if args.pmc_probe:
        pmc_probe(E)
        return 0
    if args.bf16_only:
        print(json.dumps({"bf16_gemv": bf16_sweep(E)}), flush=True)
        return 0
    if args.linear_only:
        print(json.dumps({"linear_bias_gemv": linear_sweep(E)}), flush=True)
        return 0
    if args.prefill_only:
        print(json.dumps(prefill_config5(E)), flush=True)
        return 0
    if args.prefill_profile:
        prefill_profile(E)
        return 0
    if args.gemv_only:
        print(json.dumps({"gemv_micro": gemv_micro(EL)}), flush=True)
        return 0
    info = E.HipBackend.device_info()
    cfg = E.LlamaConfig.llama2_7b()
    t0 = time.perf_counter()
    model = E.LlamaModel.new_random(cfg, seed=0, init_on_device=not args.host_init)
    t_init = time.perf_counter() - t0
    prompt = E.synth.prompt_ids(1, args.prompt_len, cfg.vocab_size)
    print(f"[bench] {info['name']} {info['arch']} CUs={info['cu_count']}; model init "
          f"{t_init:.1f} s", file=sys.stderr, flush=True)

    if args.sampling_only:
        print(json.dumps({"sampling": sampling_sweep(E, EL, model, prompt, args.warmup, args.steps),
                          "prompt_tokens": args.prompt_len, "steps": args.steps}), flush=True)
        model.free()
        return 0
    if args.step_profile:
        ms, _ = model.bench_decode(prompt, args.warmup, args.steps)
        prof = step_profile(model, cfg, prompt, args.steps)
        prof["bench_ms_per_step"] = round(ms / args.steps, 4)
        from esolearn_amd import _lib

        prof["graph_replay"] = bool(_lib.load().scry_hip_graph_replay())
        print(json.dumps({"step_profile": prof}), flush=True)
        model.free()
        return 0
    E.HipBackend.synchronize()
    t0 = time.perf_counter()
    ms, toks = model.bench_decode(prompt, args.warmup, args.steps)
    wall = time.perf_counter() - t0
    E.HipBackend.synchronize()
    tok_s = args.steps / (ms / 1000.0)
    print(f"[bench] decode {args.steps} steps in {ms:.2f} ms -> {tok_s:.1f} tok/s "
          f"(call wall {wall:.2f} s incl. prompt + warm-up)", file=sys.stderr, flush=True)

    # the same decode with the device sampler (top-k 40, top-p 0.95, T 0.8)
    # after each LM head instead of the argmax finish: its share of the step
    sc = EL.SamplingConfig(temperature=0.8, top_k=40, top_p=0.95, max_tokens=args.steps)
    ms_s, _ = model.bench_decode_sampled(prompt, args.warmup, args.steps, sc, seed=42)
    sampled = {"config": {"temperature": 0.8, "top_k": 40, "top_p": 0.95},
               "tok_s": round(args.steps / (ms_s / 1000.0), 2),
               "ms_per_step": round(ms_s / args.steps, 4),
               "extra_us_per_step_vs_greedy": round((ms_s - ms) / args.steps * 1000.0, 2)}
    print(f"[bench] sampled decode {sampled['tok_s']} tok/s "
          f"({sampled['extra_us_per_step_vs_greedy']} us/step over greedy)", file=sys.stderr, flush=True)

    # per-projection kernel timing (HIP events, rotating over layers)
    proj = {}
    per_token = {"qkv": cfg.n_layers, "o": cfg.n_layers, "gate_up": cfg.n_layers,
                 "down": cfg.n_layers, "lm_head": 1}
    for name, tid in (("qkv", EL.T_QKV), ("o", EL.T_O), ("gate_up", EL.T_GATE),
                      ("down", EL.T_DOWN), ("lm_head", EL.T_LM_HEAD)):
        us, b = model.time_projection(tid, args.proj_iters)
        proj[name] = {"avg_us": round(us, 3), "bytes": int(b), "gbs": round(b / us / 1e3, 1),
                      "us_per_token": round(us * per_token[name], 1)}
        print(f"[bench] {name:8s} {us:8.2f} us  {b / 1e6:8.2f} MB  {b / us / 1e3:7.1f} GB/s",
              file=sys.stderr, flush=True)
    # decode attention at the bench's mid-decode context (HIP events, rotating layers)
    ctx = args.prompt_len + args.steps // 2
    a_us, a_b = model.time_attention(ctx, args.proj_iters)
    attention = {"context": ctx, "avg_us": round(a_us, 3), "bytes": int(a_b),
                 "gbs": round(a_b / a_us / 1e3, 1), "us_per_token": round(a_us * cfg.n_layers, 1)}
    print(f"[bench] attention {a_us:8.2f} us  {a_b / 1e6:8.2f} MB  {a_b / a_us / 1e3:7.1f} GB/s "
          f"(context {ctx})", file=sys.stderr, flush=True)
    dom = max(proj, key=lambda k: proj[k]["us_per_token"])
    wb = weight_bytes(cfg)
    roofline = {
        "bound": "hbm",
        "achieved": proj[dom]["gbs"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(proj[dom]["gbs"] / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic(dom),
        "kernel": f"k_qgemv_sk ({dom} projection, decode epilogue)",
        "bytes_per_launch": proj[dom]["bytes"],
        "avg_launch_us": proj[dom]["avg_us"],
    }

    cpu = None
    if not args.no_cpu_baseline:
        print(f"[bench] cpu baseline: {args.cpu_tokens} tokens", file=sys.stderr, flush=True)
        cpu = cpu_baseline(model, cfg, prompt, args.cpu_tokens)
    model.free()
    bf16 = None if args.no_bf16_decode else bf16_decode(E, EL, cfg, prompt, args.warmup, args.steps,
                                                        args.proj_iters)
    gemv = None if args.no_gemv else gemv_micro(EL)
    pre = None if args.no_prefill else prefill_config5(E)

    line = {
        "metric": "decode tok/s, Llama-7B-shape int8 batch 1; quant-GEMV achieved HBM GB/s",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "llama2-7b-shape int8 batch-1 greedy decode (BASELINE config 4)",
            "dim": cfg.hidden_size, "layers": cfg.n_layers, "heads": cfg.n_heads,
            "ffn": cfg.intermediate_size, "vocab": cfg.vocab_size, "batch": 1,
            "prompt_tokens": args.prompt_len, "decode_tokens": args.steps,
            "context_end": args.prompt_len + args.steps, "weights": "int8 per-tensor (W8A32)",
            "parallelism": "single GPU",
        },
        "weight_bytes_per_token": wb,
        "decode_roofline_frac": round(tok_s * wb / (HBM_PEAK_GBS * 1e9), 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "projections": proj,
        "attention": attention,
        "greedy_tokens_head": [int(t) for t in toks[:8]],
        "sampled_decode": sampled,
        "bf16_decode": bf16,
        "gemv_micro": gemv,
        "prefill": pre,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
