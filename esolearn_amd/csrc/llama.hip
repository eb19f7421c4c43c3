// Llama model with int8 projections on the device (llama.rs), the
// device-resident KV cache (kv_cache.rs:70-145), the decode step
// (llama.rs:744-763) as one captured HIP graph, and greedy generation
// (generate.rs:51-98) as graph replays with the token loop on the device.
//
// Build-defined int8 composition (the reference LlamaModel has no int8 path):
// every projection matmul -- fused qkv, o, gate, up, down, lm_head -- becomes
// matmul_i8_f32 on quantize_symmetric weights (one scale per tensor; a tied
// lm_head gets its own int8 copy of embed_tokens; the f32 table stays for the
// embedding gather).
//
// Decode step, per layer (5 kernels):
//   qkv   : RMSNorm(x) -> int8 GEMV -> RoPE(Q)*1/sqrt(hd), RoPE(K), K/V row append
//           (layer 0 reads the embedding row of the current token directly)
//   attn  : split-L attention over the cache in place -> per-split partials,
//           merged by the last split of each KV group into the attention row
//   o     : int8 GEMV of the attention row + residual add into x
//   gateup: RMSNorm(x) -> fused gate/up int8 GEMV -> silu(g)*u
//   down  : int8 GEMV + residual add into x
// then lm_head: RMSNorm(x) -> int8 GEMV -> logits + per-workgroup argmax, and a
// one-workgroup finish kernel: ordered argmax -> next token, position advance.
// The current position and token live in device memory, so the same captured
// graph replays for every token.
#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.h"

using namespace scry;

struct scry_llama_s {
    scry_llama_config cfg{};
    int h = 0, V = 0, ffn = 0, nh = 0, nkv = 0, hd = 0, q_dim = 0, kv_dim = 0, qkv_dim = 0, L = 0;
    int quant_mode = 0;
    float *embed = nullptr;  // [V, h] f32
    float *norms = nullptr;  // [2L+1][h] RMSNorm weights (RMSNorm::new: ones)
    // RMSNorm eps: 1e-5 from RMSNorm::new (rmsnorm.rs:17-22), which ignores
    // config.rms_norm_eps; a loaded checkpoint uses the config's (llama.rs:880-914)
    float eps = 1e-5f;
    std::vector<float> freqs;  // [hd/2] f32 (llama.rs:618-622)
    struct Layer {
        Packed qkv, o, gu, down;
    };
    std::vector<Layer> layers;
    Packed lm;
    unsigned int *bits = nullptr;
    float *stage = nullptr;  // device f32 staging for one tensor
    size_t stage_n = 0;
    int live_caches = 0;
    // batched-prefill workspace (grown on demand): bf16 planes of the GEMM
    // inputs ([Mp][ld0] for k = h / q_dim, [Mp][ld1] for k = ffn; hi then
    // lo), the residual stream x [M][h], the qkv rows [M][qkv_dim], token ids
    struct Prefill {
        int Mp = 0, ld0 = 0, ld1 = 0;
        unsigned short *p0 = nullptr, *p1 = nullptr;
        float *x = nullptr, *qkv = nullptr, *last = nullptr, *xl = nullptr;
        int64_t *ids = nullptr;
        signed char *dg = nullptr;  // digit planes [3][Mp][ld] of the int8 GEMMs' inputs (ld = ld0 or ld1)
        int *de = nullptr;          // their row exponents [Mp]
    } pf;
    unsigned short *kvp = nullptr;  // the prefill attention's K / V planes (grown on demand)
    size_t kvp_n = 0;
    // batched-decode workspace (allocated on first use, PF_MAX_SEQS rows):
    // residual rows x, qkv rows, RoPE'd and scaled q, the attention rows xa,
    // SwiGLU rows act, logits; the residual rows' partial sums of squares ss
    // [rows][64] (the next RMSNorm's input); the skinny matmuls' split
    // partials; the LM head's argmax partials; per-sequence
    // attention partials and arrival counters; the device positions
    struct Batch {
        float *x = nullptr, *xa = nullptr, *act = nullptr, *logits = nullptr;
        double *ss = nullptr;
        float *ws = nullptr;
        size_t ws_bytes = 0;
        float *pv = nullptr;
        int *pi = nullptr, *pn = nullptr;
        float *ap_o = nullptr, *ap_ml = nullptr;
        unsigned *ctr = nullptr;
        int *pos = nullptr;
    } bd;
    const float *norm_in(int l) const { return norms + (size_t)(2 * l) * h; }
    const float *norm_post(int l) const { return norms + (size_t)(2 * l + 1) * h; }
    const float *norm_final() const { return norms + (size_t)(2 * L) * h; }
};

struct HostStage {
    DevState st;
    int64_t tok;
    int64_t amax;
};

struct scry_kv_cache_s {
    scry_llama m = nullptr;
    int max_seq = 0;
    int seq_len = 0;  // host mirror of LlamaLayerKvCache::seq_len
    float *kv = nullptr;  // [L][2][max_seq][kv_dim]
    float2 *rope_cs = nullptr;  // [max_seq][hd/2] (cos, sin), glibc values as cpu.rs:650-652
    DevState *state = nullptr;
    int64_t *tokens = nullptr;
    int tokens_len = 0;
    float *x = nullptr, *xq = nullptr, *act = nullptr, *logits = nullptr;
    // the residual row times the next RMSNorm weight, and the per-workgroup
    // sums of squares of the residual row (written by the residual GEMVs)
    float *xg = nullptr;
    float *ss = nullptr;
    // decode attention split partials and per-KV-group arrival counters (the
    // last split merges them), and the merged output row
    void *att_buf = nullptr;
    float *ap_o = nullptr, *ap_ml = nullptr;
    unsigned *att_ctr = nullptr;  // group g's at att_ctr[g * kCtrStride]
    float *xa = nullptr;
    float *lp_val = nullptr;
    int *lp_idx = nullptr, *lp_nan = nullptr;
    int64_t *amax = nullptr;
    // stochastic sampling (generate with temperature >= 1e-8): the config the
    // step graph was captured with, f64 scratch [V] and the wyrand state
    bool sampling = false;
    scry_sampling_config samp{};
    double *samp_ws = nullptr;
    unsigned long long *rng = nullptr;
    void *samp_prep = nullptr;  // zeroed; sample_uses_prep configurations
    int n_splits = 1, max_chunk = 16;
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    HostStage *hs = nullptr;  // pinned
    float *K(int l) const { return kv + (size_t)(2 * l) * max_seq * m->kv_dim; }
    float *Vc(int l) const { return kv + (size_t)(2 * l + 1) * max_seq * m->kv_dim; }
};

#define API_LOCK std::lock_guard<std::recursive_mutex> _api_lock(scry::api_mutex())

namespace {

int sync_stream() {
    SCRY_HIP(hipStreamSynchronize(ctx().stream));
    return SCRY_OK;
}

// Quantize a device f32 tensor into (a slice of) a Packed weight.
// src_nk: source stored [n,k]; (grp, stride, off): row interleave; second:
// the tensor is the up half of a fused gate/up pair.
int quant_into(scry_llama m, const float *dw, int k, int n, int src_nk, Packed &P, int grp,
               int stride, int off, bool second) {
    hipStream_t s = ctx().stream;
    if (m->quant_mode == SCRY_QUANT_BF16) {
        (void)second;
        SCRY_TRY(launch_pack_model_bf16(dw, k, n, src_nk, (unsigned short *)P.d, P.kp / 2, grp, stride, off, s));
        return sync_stream();
    }
    if (m->quant_mode == SCRY_QUANT_PER_TENSOR) {
        SCRY_TRY(launch_absmax(dw, (size_t)k * n, m->bits, s));
        unsigned int bits = 0;
        SCRY_HIP(hipMemcpyAsync(&bits, m->bits, sizeof bits, hipMemcpyDeviceToHost, s));
        SCRY_TRY(sync_stream());
        float absmax;
        std::memcpy(&absmax, &bits, sizeof absmax);
        const float scale = absmax == 0.0f ? 0.0f : absmax / 127.0f;  // quantize.rs:23
        if (second)
            P.scale2 = scale;
        else
            P.scale = scale;
        return launch_quant_pack(dw, k, n, src_nk, m->bits, P.d, P.kp, grp, stride, off, s);
    }
    // block-32: quantize per (output, 32-block), then pack bytes and scales
    const int nb = (k + 31) / 32;
    int8_t *q = nullptr;
    float *sc = nullptr;
    SCRY_TRY(dev_alloc((void **)&q, (size_t)k * n));
    int rc = dev_alloc((void **)&sc, sizeof(float) * (size_t)n * nb);
    if (!rc) rc = launch_quant_block32(dw, k, n, src_nk, q, sc, s);
    if (!rc) rc = launch_i8_pack(q, k, n, src_nk, P.d, P.kp, grp, stride, off, s);
    if (!rc) rc = launch_scales_pack(sc, n, nb, P.s32, grp, stride, off, s);
    if (!rc) rc = sync_stream();
    dev_free(q);
    dev_free(sc);
    return rc;
}

int alloc_packed(scry_llama m, Packed &P, int k, int n, int rows, int fused) {
    P.k = k;
    P.n = n;
    P.bf16 = m->quant_mode == SCRY_QUANT_BF16;
    P.kp = P.bf16 ? 2 * round_up(k, 8) : round_up(k, 16);
    P.scale = P.scale2 = 1.0f;
    P.rows = rows;
    P.fused = fused;
    SCRY_TRY(dev_alloc((void **)&P.d, P.bytes()));
    if (m->quant_mode == SCRY_QUANT_BLOCK32) {
        P.nb = (k + 31) / 32;
        SCRY_TRY(dev_alloc((void **)&P.s32, sizeof(float) * (size_t)rows * P.nb));
    }
    return SCRY_OK;
}

int upload_stage(scry_llama m, const float *host, size_t n) {
    if (n > m->stage_n) return set_error(SCRY_ERR_INVALID, "tensor larger than the staging buffer");
    SCRY_HIP(hipMemcpyAsync(m->stage, host, n * sizeof(float), hipMemcpyHostToDevice, ctx().stream));
    return sync_stream();
}

// Load one tensor (reference layout) into the model.
int load_tensor(scry_llama m, int id, int layer, const float *host) {
    const int h = m->h, V = m->V, ffn = m->ffn;
    if (id == SCRY_T_EMBED) {
        SCRY_HIP(hipMemcpyAsync(m->embed, host, sizeof(float) * (size_t)V * h, hipMemcpyHostToDevice,
                                ctx().stream));
        SCRY_TRY(sync_stream());
        if (m->cfg.tie_word_embeddings) return quant_into(m, m->embed, h, V, 1, m->lm, 1, 1, 0, false);
        return SCRY_OK;
    }
    if (id == SCRY_T_LM_HEAD) {
        if (m->cfg.tie_word_embeddings)
            return set_error(SCRY_ERR_INVALID, "lm_head is tied to embed_tokens");
        SCRY_TRY(upload_stage(m, host, (size_t)V * h));
        return quant_into(m, m->stage, h, V, 1, m->lm, 1, 1, 0, false);
    }
    if (layer < 0 || layer >= m->L) return set_error(SCRY_ERR_INVALID, "layer %d out of range", layer);
    auto &Ly = m->layers[layer];
    switch (id) {
        case SCRY_T_QKV:
            SCRY_TRY(upload_stage(m, host, (size_t)h * m->qkv_dim));
            return quant_into(m, m->stage, h, m->qkv_dim, 0, Ly.qkv, 1, 1, 0, false);
        case SCRY_T_O:
            SCRY_TRY(upload_stage(m, host, (size_t)m->q_dim * h));
            return quant_into(m, m->stage, m->q_dim, h, 0, Ly.o, 1, 1, 0, false);
        case SCRY_T_GATE:
            SCRY_TRY(upload_stage(m, host, (size_t)h * ffn));
            return quant_into(m, m->stage, h, ffn, 0, Ly.gu, 2, 4, 0, false);
        case SCRY_T_UP:
            SCRY_TRY(upload_stage(m, host, (size_t)h * ffn));
            return quant_into(m, m->stage, h, ffn, 0, Ly.gu, 2, 4, 2, true);
        case SCRY_T_DOWN:
            SCRY_TRY(upload_stage(m, host, (size_t)ffn * h));
            return quant_into(m, m->stage, ffn, h, 0, Ly.down, 1, 1, 0, false);
    }
    return set_error(SCRY_ERR_INVALID, "unknown tensor id %d", id);
}

void model_free(scry_llama m) {
    if (!m) return;
    for (auto &Ly : m->layers) {
        packed_free(Ly.qkv);
        packed_free(Ly.o);
        packed_free(Ly.gu);
        packed_free(Ly.down);
    }
    packed_free(m->lm);
    dev_free(m->embed);
    dev_free(m->norms);
    dev_free(m->bits);
    dev_free(m->stage);
    dev_free(m->pf.p0);
    dev_free(m->pf.p1);
    dev_free(m->pf.x);
    dev_free(m->pf.qkv);
    dev_free(m->pf.last);
    dev_free(m->pf.xl);
    dev_free(m->pf.ids);
    dev_free(m->pf.dg);
    dev_free(m->pf.de);
    dev_free(m->kvp);
    for (void *p : {(void *)m->bd.x, (void *)m->bd.xa, (void *)m->bd.act,
                    (void *)m->bd.logits, (void *)m->bd.ss, (void *)m->bd.ws, (void *)m->bd.pv, (void *)m->bd.pi, (void *)m->bd.pn, (void *)m->bd.ap_o, (void *)m->bd.ap_ml,
                    (void *)m->bd.ctr, (void *)m->bd.pos})
        dev_free(p);
    delete m;
}

int model_alloc(const scry_llama_config *cfg, int quant_mode, scry_llama *out) {
    if (!cfg || !out) return set_error(SCRY_ERR_INVALID, "null argument");
    if (quant_mode != SCRY_QUANT_PER_TENSOR && quant_mode != SCRY_QUANT_BLOCK32 && quant_mode != SCRY_QUANT_BF16)
        return set_error(SCRY_ERR_INVALID, "unknown quant mode %d", quant_mode);
    const int h = cfg->hidden_size, nh = cfg->n_heads, nkv = cfg->n_kv_heads;
    if (h <= 0 || nh <= 0 || nkv <= 0 || h % nh || nh % nkv || cfg->vocab_size <= 0 ||
        cfg->intermediate_size <= 0 || cfg->n_layers <= 0)
        return set_error(SCRY_ERR_INVALID, "invalid Llama config");
    const int hd = h / nh;
    if (hd % 4 || cfg->intermediate_size % 2)
        return set_error(SCRY_ERR_UNSUPPORTED, "head_dim must be a multiple of 4 and ffn even");
    if (h > 16384 || cfg->intermediate_size > 16384 || nh * hd > 16384)
        return set_error(SCRY_ERR_UNSUPPORTED, "GEMV k > 16384 not supported");
    auto *m = new (std::nothrow) scry_llama_s;
    if (!m) return set_error(SCRY_ERR_OOM, "host allocation failed");
    m->cfg = *cfg;
    m->quant_mode = quant_mode;
    m->h = h;
    m->V = cfg->vocab_size;
    m->ffn = cfg->intermediate_size;
    m->nh = nh;
    m->nkv = nkv;
    m->hd = hd;
    m->q_dim = nh * hd;
    m->kv_dim = nkv * hd;
    m->qkv_dim = m->q_dim + 2 * m->kv_dim;
    m->L = cfg->n_layers;
    // llama.rs:1035-1067 compute_rope_freqs (f64), stored as f32 (llama.rs:621)
    m->freqs.resize(hd / 2);
    const double th = (double)cfg->rope_theta;
    for (int i = 0; i < hd / 2; i++) {
        double f = 1.0 / std::pow(th, 2.0 * (double)i / (double)hd);
        if (cfg->has_rope_scaling) {
            const double old_ctx = (double)cfg->rs_original_max_pos;
            const double low_wl = old_ctx / cfg->rs_low_freq_factor;
            const double high_wl = old_ctx / cfg->rs_high_freq_factor;
            const double wl = 2.0 * M_PI / f;
            double sf;
            if (wl < high_wl)
                sf = 1.0;
            else if (wl > low_wl)
                sf = cfg->rs_factor;
            else {
                const double smooth = (old_ctx / wl - cfg->rs_low_freq_factor) /
                                      (cfg->rs_high_freq_factor - cfg->rs_low_freq_factor);
                sf = 1.0 / ((1.0 - smooth) / cfg->rs_factor + smooth);
            }
            f /= sf;
        }
        m->freqs[i] = (float)f;
    }
    int rc = dev_alloc((void **)&m->embed, sizeof(float) * (size_t)m->V * h);
    if (!rc) rc = dev_alloc((void **)&m->norms, sizeof(float) * (size_t)(2 * m->L + 1) * h);
    if (!rc) rc = launch_fill_f32(m->norms, (size_t)(2 * m->L + 1) * h, 1.0f, ctx().stream);
    if (!rc) rc = dev_alloc((void **)&m->bits, 16);
    const size_t sizes[] = {(size_t)m->V * h, (size_t)h * m->qkv_dim, (size_t)h * m->ffn,
                            (size_t)m->q_dim * h};
    for (size_t s : sizes) m->stage_n = std::max(m->stage_n, s);
    if (!rc) rc = dev_alloc((void **)&m->stage, sizeof(float) * m->stage_n);
    m->layers.resize(m->L);
    for (int l = 0; l < m->L && !rc; l++) {
        auto &Ly = m->layers[l];
        rc = alloc_packed(m, Ly.qkv, h, m->qkv_dim, m->qkv_dim, 0);
        if (!rc) rc = alloc_packed(m, Ly.o, m->q_dim, h, h, 0);
        if (!rc) rc = alloc_packed(m, Ly.gu, h, m->ffn, 2 * m->ffn, 1);
        if (!rc) rc = alloc_packed(m, Ly.down, m->ffn, h, h, 0);
    }
    if (!rc) rc = alloc_packed(m, m->lm, h, m->V, m->V, 0);
    if (rc) {
        model_free(m);
        return rc;
    }
    *out = m;
    return SCRY_OK;
}

// ---------------------------------------------------------------- sessions
void cache_free(scry_kv_cache c) {
    if (!c) return;
    if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    dev_free(c->kv);
    dev_free(c->rope_cs);
    dev_free(c->state);
    dev_free(c->tokens);
    dev_free(c->x);
    dev_free(c->xg);
    dev_free(c->ss);
    dev_free(c->xq);
    dev_free(c->act);
    dev_free(c->logits);
    dev_free(c->att_buf);
    dev_free(c->xa);
    dev_free(c->lp_val);
    dev_free(c->lp_idx);
    dev_free(c->lp_nan);
    dev_free(c->amax);
    dev_free(c->samp_ws);
    dev_free(c->rng);
    dev_free(c->samp_prep);
    if (c->hs) (void)hipHostFree(c->hs);
    if (c->m) c->m->live_caches--;
    delete c;
}

int cache_new(scry_llama m, int max_seq, scry_kv_cache *out) {
    if (max_seq <= 0) return set_error(SCRY_ERR_INVALID, "max_seq must be > 0");
    auto *c = new (std::nothrow) scry_kv_cache_s;
    if (!c) return set_error(SCRY_ERR_OOM, "host allocation failed");
    c->m = m;
    m->live_caches++;
    c->max_seq = max_seq;
    c->tokens_len = max_seq + 1;
    attn_pick_splits(m->nkv, max_seq, &c->n_splits, &c->max_chunk);
    hipStream_t s = ctx().stream;
    const size_t kvn = (size_t)m->L * 2 * max_seq * m->kv_dim;
    const int nparts = qgemv_blocks(EPI_LOGITS, m->lm, 1);
    const int n_ss = std::max(qgemv_blocks(EPI_RESID, m->layers[0].o, 1), qgemv_blocks(EPI_RESID, m->layers[0].down, 1));
    int rc = dev_alloc((void **)&c->kv, sizeof(float) * kvn);
    if (!rc) rc = launch_fill_f32(c->kv, kvn, 0.f, s);  // LlamaLayerKvCache::new zeros
    if (!rc) rc = dev_alloc((void **)&c->rope_cs, sizeof(float2) * (size_t)max_seq * (m->hd / 2));
    if (!rc) rc = dev_alloc((void **)&c->state, sizeof(DevState));
    if (!rc) rc = dev_alloc((void **)&c->tokens, sizeof(int64_t) * c->tokens_len);
    if (!rc) rc = dev_alloc((void **)&c->x, sizeof(float) * m->h);
    if (!rc) rc = dev_alloc((void **)&c->xg, sizeof(float) * m->h);
    if (!rc) rc = dev_alloc((void **)&c->ss, sizeof(float) * n_ss);
    if (!rc) rc = dev_alloc((void **)&c->xq, sizeof(float) * m->q_dim);
    if (!rc) rc = dev_alloc((void **)&c->act, sizeof(float) * m->ffn);
    if (!rc) rc = dev_alloc((void **)&c->logits, sizeof(float) * m->V);
    if (!rc) rc = dev_alloc((void **)&c->xa, sizeof(float) * m->q_dim);
    if (!rc) {
        auto al = [](size_t b) { return (b + 255) / 256 * 256; };
        const size_t b_o = al(sizeof(float) * (size_t)m->nh * c->n_splits * m->hd);
        const size_t b_ml = al(sizeof(float) * (size_t)m->nh * c->n_splits * 2);
        const size_t n_ctr = (size_t)m->nkv * kCtrStride;  // merge arrivals
        rc = dev_alloc(&c->att_buf, b_o + b_ml + al(sizeof(unsigned) * n_ctr));
        if (!rc) {
            char *base = (char *)c->att_buf;
            c->ap_o = (float *)base;
            c->ap_ml = (float *)(base + b_o);
            c->att_ctr = (unsigned *)(base + b_o + b_ml);
            rc = launch_fill_u32(c->att_ctr, n_ctr, 0u, s);
        }
    }
    if (!rc) rc = dev_alloc((void **)&c->lp_val, sizeof(float) * nparts);
    if (!rc) rc = dev_alloc((void **)&c->lp_idx, sizeof(int) * nparts);
    if (!rc) rc = dev_alloc((void **)&c->lp_nan, sizeof(int) * nparts);
    if (!rc) rc = dev_alloc((void **)&c->amax, sizeof(int64_t));
    if (!rc) {
        hipError_t e = hipHostMalloc((void **)&c->hs, sizeof(HostStage), hipHostMallocDefault);
        if (e != hipSuccess) rc = hip_fail(e, "hipHostMalloc", __FILE__, __LINE__);
    }
    if (!rc) {
        // RoPE table: cos/sin of f64(pos) * f64(freq_f32) rounded to f32, with
        // the host libm the reference uses (cpu.rs:648-652)
        const int hh = m->hd / 2;
        std::vector<float2> cs((size_t)max_seq * hh);
        for (int p = 0; p < max_seq; p++)
            for (int i = 0; i < hh; i++) {
                const double ang = (double)p * (double)m->freqs[i];
                cs[(size_t)p * hh + i] = make_float2((float)std::cos(ang), (float)std::sin(ang));
            }
        hipError_t e = hipMemcpyAsync(c->rope_cs, cs.data(), sizeof(float2) * cs.size(),
                                      hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "rope table upload", __FILE__, __LINE__);
    }
    if (rc) {
        cache_free(c);
        return rc;
    }
    *out = c;
    return SCRY_OK;
}

// Input of an RMSNorm'd GEMV that follows the residual GEMV on weights w: the
// row it left pre-multiplied by this norm's weight, and its partial sums of squares.
void pre_normed(scry_kv_cache c, const Packed &w, GemvArgs *g) {
    g->x = c->xg;
    g->ss_in = c->ss;
    g->n_ss = qgemv_blocks(EPI_RESID, w, 1);
}

// Residual GEMV outputs for the RMSNorm'd GEMV that follows it.
void next_norm(scry_kv_cache c, const float *g_next, GemvArgs *g) {
    g->xg_out = c->xg;
    g->g_next = g_next;
    g->ss_out = c->ss;
}

GemvArgs qkv_args(scry_kv_cache c, int l) {
    scry_llama m = c->m;
    GemvArgs g;
    g.w = &m->layers[l].qkv;
    g.ldx = m->h;
    g.embed = m->embed;
    g.tokens = c->tokens;
    g.state = c->state;
    g.eps = m->eps;
    if (l == 0) {
        g.x = nullptr;  // the embedding row, RMSNorm'd in the prologue
        g.norm_w = m->norm_in(0);
    } else {
        pre_normed(c, m->layers[l - 1].down, &g);
    }
    g.q_out = c->xq;
    g.k_cache = c->K(l);
    g.v_cache = c->Vc(l);
    g.rope_cs = c->rope_cs;
    g.q_dim = m->q_dim;
    g.kv_dim = m->kv_dim;
    g.head_dim = m->hd;
    g.q_scale = (float)(1.0 / std::sqrt((double)m->hd));  // llama.rs:394
    return g;
}

AttnArgs attn_args(scry_kv_cache c, int l) {
    scry_llama m = c->m;
    AttnArgs a;
    a.q = c->xq;
    a.k_cache = c->K(l);
    a.v_cache = c->Vc(l);
    a.part_o = c->ap_o;
    a.part_ml = c->ap_ml;
    a.merge_ctr = c->att_ctr;
    a.xa = c->xa;
    a.state = c->state;
    a.n_heads = m->nh;
    a.n_kv = m->nkv;
    a.head_dim = m->hd;
    a.n_splits = c->n_splits;
    a.max_chunk = c->max_chunk;
    return a;
}

GemvArgs o_args(scry_kv_cache c, int l) {
    scry_llama m = c->m;
    GemvArgs g;
    g.w = &m->layers[l].o;
    g.x = c->xa;  // the attention output row (merged by the attention kernel)
    g.ldx = m->q_dim;
    g.y = c->x;
    g.ldy = m->h;
    g.resid = l == 0 ? nullptr : c->x;  // layer 0: residual is the embedding row
    g.embed = m->embed;
    g.tokens = c->tokens;
    g.state = c->state;
    next_norm(c, m->norm_post(l), &g);
    return g;
}

GemvArgs gu_args(scry_kv_cache c, int l) {
    scry_llama m = c->m;
    GemvArgs g;
    g.w = &m->layers[l].gu;
    pre_normed(c, m->layers[l].o, &g);
    g.ldx = m->h;
    g.eps = m->eps;
    g.y = c->act;
    g.ldy = m->ffn;
    return g;
}

GemvArgs down_args(scry_kv_cache c, int l) {
    scry_llama m = c->m;
    GemvArgs g;
    g.w = &m->layers[l].down;
    g.x = c->act;
    g.ldx = m->ffn;
    g.y = c->x;
    g.ldy = m->h;
    g.resid = c->x;
    next_norm(c, l + 1 < m->L ? m->norm_in(l + 1) : m->norm_final(), &g);
    return g;
}

GemvArgs lm_args(scry_kv_cache c, int advance) {
    scry_llama m = c->m;
    GemvArgs g;
    g.w = &m->lm;
    pre_normed(c, m->layers[m->L - 1].down, &g);
    g.ldx = m->h;
    g.eps = m->eps;
    g.y = c->logits;
    g.ldy = m->V;
    g.state = c->state;
    g.part_val = c->lp_val;
    g.part_idx = c->lp_idx;
    g.part_nan = c->lp_nan;
    g.tokens_rw = c->tokens;
    g.argmax_out = c->amax;
    g.advance = advance;
    return g;
}

// The step's launches in order.  ts (step profile, may be null): launch i
// writes its workgroups' start / end stamps at ts + 2 * ts_slots * i.
int record_step(scry_kv_cache c, hipStream_t s, unsigned long long *ts = nullptr, size_t ts_slots = 0) {
    scry_llama m = c->m;
    int li = 0;
    auto slot = [&]() { return ts ? ts + 2 * ts_slots * (size_t)li++ : nullptr; };
    for (int l = 0; l < m->L; l++) {
        GemvArgs q = qkv_args(c, l);
        q.ts = slot();
        SCRY_TRY(launch_qgemv(EPI_QKV, q, s));
        AttnArgs at = attn_args(c, l);
        at.ts = slot();
        SCRY_TRY(launch_attn_decode(at, s));
        GemvArgs o = o_args(c, l);
        o.ts = slot();
        SCRY_TRY(launch_qgemv(EPI_RESID, o, s));
        GemvArgs gu = gu_args(c, l);
        gu.ts = slot();
        SCRY_TRY(launch_qgemv(EPI_SWIGLU, gu, s));
        GemvArgs dn = down_args(c, l);
        dn.ts = slot();
        SCRY_TRY(launch_qgemv(EPI_RESID, dn, s));
    }
    GemvArgs lg = lm_args(c, 1);
    lg.ts = slot();
    SCRY_TRY(launch_qgemv(EPI_LOGITS, lg, s));
    if (c->sampling)
        return launch_sample(c->logits, m->V, c->samp, c->samp_ws, c->rng, c->state, c->tokens, c->samp_prep, s);
    lg.ts = slot();
    return launch_logits_finish(lg, s);
}

}  // namespace

// Graph replay of the decode steps, unless SCRY_HIP_NO_GRAPH is set or a
// rocprofiler tool is attached to the process (rocprofv3 names its tool
// library in ROCP_TOOL_LIBRARIES).  Under rocprofv3 --kernel-trace the
// process faulted on the host inside the profiler's hipGraphLaunch
// interception (SIGSEGV below run_step -> hipGraphLaunch, in frames of the
// runtime and the tool), while the same graphs replay without a profiler in
// every test and bench run; so profiled runs take the same kernels as direct
// launches.
bool scry::graph_replay() {
    static const bool on = [] {
        if (std::getenv("SCRY_HIP_NO_GRAPH")) return false;
        const char *tool = std::getenv("ROCP_TOOL_LIBRARIES");
        return !(tool && *tool);
    }();
    return on;
}

namespace {

// One decode step: the captured graph when available, else direct launches
// (graph_replay()).
int run_step(scry_kv_cache c) {
    hipStream_t s = ctx().stream;
    if (!graph_replay()) return record_step(c, s);
    if (!c->gexec) {
        hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            int rc = record_step(c, s);
            hipGraph_t g = nullptr;
            e = hipStreamEndCapture(s, &g);
            if (rc) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            if (e == hipSuccess && g) {
                e = hipGraphInstantiate(&c->gexec, g, nullptr, nullptr, 0);
                if (e == hipSuccess) {
                    c->graph = g;
                } else {
                    (void)hipGetLastError();
                    (void)hipGraphDestroy(g);
                    c->gexec = nullptr;
                }
            } else {
                (void)hipGetLastError();
            }
        } else {
            (void)hipGetLastError();
        }
    }
    if (c->gexec) {
        SCRY_HIP(hipGraphLaunch(c->gexec, s));
        return SCRY_OK;
    }
    return record_step(c, s);
}

int set_state(scry_kv_cache c, int pos, int cache_len, int n_prompt) {
    c->hs->st.pos = pos;
    c->hs->st.cache_len = cache_len;
    c->hs->st.n_prompt = n_prompt;
    c->hs->st.max_tokens = c->tokens_len - 1;
    SCRY_HIP(hipMemcpyAsync(c->state, &c->hs->st, sizeof(DevState), hipMemcpyHostToDevice, ctx().stream));
    return sync_stream();
}

int check_ids(scry_llama m, const int64_t *ids, int n) {
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->V)
            return set_error(SCRY_ERR_RANGE, "token id %lld out of range (vocab %d)", (long long)ids[i], m->V);
    return SCRY_OK;
}

// ------------------------------------------------------------ batched prefill
// Workspace for M = n_seq * seq rows (planes zeroed when allocated: their
// padding rows and columns must read as zero).
int prefill_ws(scry_llama m, int M, int n_seq) {
    auto &P = m->pf;
    const int Mp = prefill_rows_pad(M);
    const int ld0 = prefill_k_pad(std::max(m->h, m->q_dim)), ld1 = prefill_k_pad(m->ffn);
    if (Mp <= P.Mp && P.ld0 == ld0 && P.ld1 == ld1) return SCRY_OK;
    dev_free(P.p0);
    dev_free(P.p1);
    dev_free(P.x);
    dev_free(P.qkv);
    dev_free(P.last);
    dev_free(P.xl);
    dev_free(P.ids);
    dev_free(P.dg);
    dev_free(P.de);
    P = scry_llama_s::Prefill{};
    const size_t n0 = 2 * (size_t)Mp * ld0, n1 = 2 * (size_t)Mp * ld1;
    SCRY_TRY(dev_alloc((void **)&P.p0, n0 * sizeof(unsigned short)));
    SCRY_TRY(dev_alloc((void **)&P.p1, n1 * sizeof(unsigned short)));
    SCRY_TRY(dev_alloc((void **)&P.x, (size_t)Mp * m->h * sizeof(float)));
    SCRY_TRY(dev_alloc((void **)&P.qkv, (size_t)Mp * m->qkv_dim * sizeof(float)));
    SCRY_TRY(dev_alloc((void **)&P.last, (size_t)PF_MAX_SEQS * m->V * sizeof(float)));
    SCRY_TRY(dev_alloc((void **)&P.xl, (size_t)PF_MAX_SEQS * m->h * sizeof(float)));
    SCRY_TRY(dev_alloc((void **)&P.ids, (size_t)Mp * sizeof(int64_t)));
    const size_t ldd = std::max(ld0, ld1);  // digit planes of the RMSNorm outputs (ld0) or the SwiGLU rows (ld1)
    SCRY_TRY(dev_alloc((void **)&P.dg, 3 * (size_t)Mp * ldd));
    SCRY_TRY(dev_alloc((void **)&P.de, (size_t)Mp * sizeof(int)));
    hipStream_t s = ctx().stream;
    SCRY_HIP(hipMemsetAsync(P.p0, 0, n0 * sizeof(unsigned short), s));
    SCRY_HIP(hipMemsetAsync(P.p1, 0, n1 * sizeof(unsigned short), s));
    SCRY_HIP(hipMemsetAsync(P.dg, 0, 3 * (size_t)Mp * ldd, s));
    SCRY_HIP(hipMemsetAsync(P.de, 0, (size_t)Mp * sizeof(int), s));
    P.Mp = Mp;
    P.ld0 = ld0;
    P.ld1 = ld1;
    (void)n_seq;
    return SCRY_OK;
}

// LlamaModel::forward (llama.rs:683-700) over n_seq sequences of seq tokens,
// each continuing its cache at cs[i]->seq_len: K/V rows are appended.  Every
// projection is one GEMM over all n_seq * seq rows.  all_logits (device,
// [M][V]) receives every position's logits; last_logits (device, [n_seq][V])
// each sequence's last position's.  Either may be null.  Queued on the
// stream; the caches' seq_len are advanced.
int prefill_core(scry_llama m, scry_kv_cache *cs, int n_seq, const int64_t *tokens, int seq, float *all_logits,
                 float *last_logits) {
    if (n_seq < 1 || n_seq > PF_MAX_SEQS || seq < 1)
        return set_error(SCRY_ERR_INVALID, "prefill: n_seq must be 1..%d and seq >= 1", PF_MAX_SEQS);
    if (m->hd > 128) return set_error(SCRY_ERR_UNSUPPORTED, "prefill: head_dim %d > 128", m->hd);
    PrefillSeqs t{};
    for (int i = 0; i < n_seq; i++) {
        scry_kv_cache c = cs[i];
        if (!c || c->m != m) return set_error(SCRY_ERR_INVALID, "prefill: cache %d does not belong to the model", i);
        for (int j = 0; j < i; j++)
            if (cs[j] == c) return set_error(SCRY_ERR_INVALID, "prefill: cache %d given twice", i);
        if (c->seq_len + seq > c->max_seq)
            return set_error(SCRY_ERR_RANGE, "prefill: %d + %d rows exceed the cache (%d)", c->seq_len, seq,
                             c->max_seq);
        t.k[i] = c->K(0);
        t.v[i] = c->Vc(0);
        t.ls[i] = (size_t)2 * c->max_seq * m->kv_dim;
        t.rope[i] = c->rope_cs;
        t.p0[i] = c->seq_len;
    }
    const int M = n_seq * seq;
    SCRY_TRY(check_ids(m, tokens, M));
    SCRY_TRY(prefill_ws(m, M, n_seq));
    // K / V planes for the bf16 matrix-core attention: rows [0, p0 + seq) of every sequence
    PrefillKVP kvp;
    if (attn_prefill_planes(m->hd)) {
        int rows = 0;
        for (int i = 0; i < n_seq; i++) rows = std::max(rows, t.p0[i] + seq);
        const size_t per = (size_t)n_seq * m->nkv * rows * m->hd;
        if (m->kvp_n < 4 * per) {
            SCRY_TRY(sync_stream());  // queued work may still read the old planes
            dev_free(m->kvp);
            m->kvp = nullptr;
            m->kvp_n = 0;
            SCRY_TRY(dev_alloc((void **)&m->kvp, sizeof(unsigned short) * 4 * per));
            m->kvp_n = 4 * per;
        }
        kvp.kh = m->kvp;
        kvp.kl = m->kvp + per;
        kvp.vh = m->kvp + 2 * per;
        kvp.vl = m->kvp + 3 * per;
        kvp.rows = rows;
    }
    auto &P = m->pf;
    hipStream_t s = ctx().stream;
    unsigned short *h0 = P.p0, *l0 = P.p0 + (size_t)P.Mp * P.ld0;
    unsigned short *h1 = P.p1, *l1 = P.p1 + (size_t)P.Mp * P.ld1;
    SCRY_HIP(hipMemcpyAsync(P.ids, tokens, sizeof(int64_t) * M, hipMemcpyHostToDevice, s));
    SCRY_TRY(launch_embedding(m->embed, P.ids, M, m->h, P.x, s));  // cpu.rs:485-498
    const float eps = m->eps;
    const size_t dstride = (size_t)P.Mp * P.ld0;
    // RMSNorm of the residual rows into the input of a GEMM over w: digit
    // planes for int8 per-tensor weights (the int8 matrix cores), bf16 planes
    // otherwise
    auto norm_for = [&](const float *nw, const Packed &w, PrefillGemm &g) -> int {
        g.lda = P.ld0;
        g.M = M;
        g.w = &w;
        if (gemm_takes_digits(w)) {
            g.ad = P.dg;
            g.ae = P.de;
            g.dstride = dstride;
            g.ahi = g.alo = nullptr;
            return launch_norm_digits(P.x, m->h, M, nw, m->h, eps, P.dg, dstride, P.de, P.ld0, s);
        }
        g.ahi = h0;
        g.alo = l0;
        return launch_norm_split(P.x, m->h, M, 1, 0, nw, m->h, eps, h0, l0, P.ld0, nullptr, 0, s);
    };
    for (int l = 0; l < m->L; l++) {
        const auto &Ly = m->layers[l];
        PrefillGemm g;
        SCRY_TRY(norm_for(m->norm_in(l), Ly.qkv, g));
        g.c = P.qkv;
        g.ldc = m->qkv_dim;
        SCRY_TRY(launch_gemm(PF_STORE, g, s));
        SCRY_TRY(launch_rope_kv(P.qkv, m->qkv_dim, M, seq, m->q_dim, m->kv_dim, m->hd, t, l, kvp, n_seq, s));
        PrefillAttn at;
        at.qkv = P.qkv;
        at.ldq = m->qkv_dim;
        at.seq = seq;
        at.hd = m->hd;
        at.nh = m->nh;
        at.nkv = m->nkv;
        at.kvd = m->kv_dim;
        at.scale = (float)(1.0 / std::sqrt((double)m->hd));  // llama.rs:225-234
        at.ldo = P.ld0;
        at.opad = prefill_k_pad(m->q_dim);
        PrefillGemm o;
        o.lda = P.ld0;
        o.M = M;
        o.w = &Ly.o;
        o.c = P.x;
        o.ldc = m->h;
        if (kvp.kh && gemm_takes_digits(Ly.o)) {
            // attention rows in f32 (in the planes' buffer), then their digit planes
            float *f0 = reinterpret_cast<float *>(P.p0);
            at.of = f0;
            SCRY_TRY(launch_attn_prefill(at, n_seq, t, l, kvp, s));
            SCRY_TRY(launch_norm_digits(f0, P.ld0, M, nullptr, m->q_dim, 0.f, P.dg, dstride, P.de, P.ld0, s));
            o.ad = P.dg;
            o.ae = P.de;
            o.dstride = dstride;
        } else {
            at.ohi = h0;
            at.olo = l0;
            SCRY_TRY(launch_attn_prefill(at, n_seq, t, l, kvp, s));
            o.ahi = h0;
            o.alo = l0;
        }
        SCRY_TRY(launch_gemm(PF_RESID, o, s));
        PrefillGemm u;
        SCRY_TRY(norm_for(m->norm_post(l), Ly.gu, u));
        PrefillGemm d;
        d.lda = P.ld1;
        d.M = M;
        d.w = &Ly.down;
        d.c = P.x;
        d.ldc = m->h;
        if (u.ad && gemm_takes_digits(Ly.down)) {
            // SwiGLU rows in f32 (in the planes' buffer), then their digit planes
            float *f1 = reinterpret_cast<float *>(P.p1);
            const size_t dstride1 = (size_t)P.Mp * P.ld1;
            u.of = f1;
            u.ldo = P.ld1;
            SCRY_TRY(launch_gemm(PF_SWIGLU, u, s));
            SCRY_TRY(launch_norm_digits(f1, P.ld1, M, nullptr, m->ffn, 0.f, P.dg, dstride1, P.de, P.ld1, s));
            d.ad = P.dg;
            d.ae = P.de;
            d.dstride = dstride1;
        } else {
            u.ohi = h1;
            u.olo = l1;
            u.ldo = P.ld1;
            u.opad = prefill_k_pad(m->ffn);
            SCRY_TRY(launch_gemm(PF_SWIGLU, u, s));
            d.ahi = h1;
            d.alo = l1;
        }
        SCRY_TRY(launch_gemm(PF_RESID, d, s));
    }
    if (all_logits) {
        PrefillGemm g;
        SCRY_TRY(norm_for(m->norm_final(), m->lm, g));
        g.c = all_logits;
        g.ldc = m->V;
        SCRY_TRY(launch_gemm(PF_STORE, g, s));
        SCRY_TRY(launch_logits_nonfinite(P.x, m->h, M, m->norm_final(), eps, m->lm, all_logits, m->V, s));
    }
    if (last_logits) {
        // the last row of each sequence: RMSNorm, then the LM-head GEMV
        SCRY_TRY(launch_norm_split(P.x, m->h, n_seq, seq, seq - 1, m->norm_final(), m->h, eps, nullptr, nullptr, 0,
                                   P.xl, m->h, s));
        GemvArgs g;
        g.w = &m->lm;
        g.x = P.xl;
        g.ldx = m->h;
        g.m = n_seq;
        g.y = last_logits;
        g.ldy = m->V;
        if (m->lm.bf16) {  // the bf16 GEMV takes one activation row per launch
            g.m = 1;
            for (int i = 0; i < n_seq; i++) {
                g.x = P.xl + (size_t)i * m->h;
                g.y = last_logits + (size_t)i * m->V;
                SCRY_TRY(launch_qgemv(EPI_STORE, g, s));
            }
        } else {
            SCRY_TRY(launch_qgemv(EPI_STORE, g, s));
        }
    }
    for (int i = 0; i < n_seq; i++) cs[i]->seq_len += seq;
    return SCRY_OK;
}

// Batched decode workspace, PF_MAX_SEQS rows (allocated on first use).
int batch_ws(scry_llama m) {
    auto &B = m->bd;
    if (B.pos) return SCRY_OK;
    const size_t R = PF_MAX_SEQS;
    const auto &L0 = m->layers[0];
    size_t ws = skinny_ws_bytes((int)R, m->h, m->lm.rows);
    for (const Packed *w : {&L0.qkv, &L0.o, &L0.gu, &L0.down}) ws = std::max(ws, skinny_ws_bytes((int)R, w->k, w->rows));
    const int lt = skinny_tiles(m->lm);
    const size_t nsp = 16;  // attention splits: attn_pick_splits picks at most 16
    int rc = dev_alloc((void **)&B.x, sizeof(float) * R * m->h);
    if (!rc) rc = dev_alloc((void **)&B.xa, sizeof(float) * R * m->q_dim);
    if (!rc) rc = dev_alloc((void **)&B.act, sizeof(float) * R * m->ffn);
    if (!rc) rc = dev_alloc((void **)&B.logits, sizeof(float) * R * m->V);
    if (!rc) rc = dev_alloc((void **)&B.ss, sizeof(double) * R * 64);
    if (!rc) rc = dev_alloc((void **)&B.ws, ws);
    if (!rc) rc = dev_alloc((void **)&B.pv, sizeof(float) * R * lt);
    if (!rc) rc = dev_alloc((void **)&B.pi, sizeof(int) * R * lt);
    if (!rc) rc = dev_alloc((void **)&B.pn, sizeof(int) * R * lt);
    if (!rc) rc = dev_alloc((void **)&B.ap_o, sizeof(float) * R * m->nh * nsp * m->hd);
    if (!rc) rc = dev_alloc((void **)&B.ap_ml, sizeof(float) * R * m->nh * nsp * 2);
    if (!rc) rc = dev_alloc((void **)&B.ctr, sizeof(unsigned) * R * m->nkv * kCtrStride);
    if (!rc) rc = launch_fill_u32(B.ctr, R * m->nkv * kCtrStride, 0u, ctx().stream);  // the last split of a group resets it
    if (!rc) rc = dev_alloc((void **)&B.pos, sizeof(int) * R);
    if (rc) {
        for (void *p : {(void *)B.x, (void *)B.xa, (void *)B.act, (void *)B.logits,
                        (void *)B.ss, (void *)B.ws, (void *)B.pv, (void *)B.pi, (void *)B.pn,
                        (void *)B.ap_o, (void *)B.ap_ml, (void *)B.ctr, (void *)B.pos})
            dev_free(p);
        B = scry_llama_s::Batch{};
        return rc;
    }
    B.ws_bytes = ws;
    return SCRY_OK;
}

// One batched decode step (the layer of record_step for n sequences): each
// projection is one fused skinny matmul over the n rows (the RMSNorms ride in
// them, from the residual rows' partial sums of squares, as in the
// single-sequence step); attention covers every sequence's cache in one
// launch and forms the queries and the new K / V rows from the qkv rows'
// split partials itself (QkvPro); the step ends with each sequence's next
// token and position advance.
int record_batch_step(scry_llama m, const DecodeSeqs &d, AttnSeqs c, int n_splits, int max_chunk, hipStream_t s) {
    auto &B = m->bd;
    const int n = d.n;
    const int n_ss = (m->h + 127) / 128;  // partial sums per residual row (128-column tiles)
    const float q_scale = (float)(1.0 / std::sqrt((double)m->hd));  // llama.rs:394
    auto mm = [&](const Packed &w, const float *x, int ldx, const float *norm_w, int epi, float *y, int ldy) {
        SkinnyFused f;
        f.w = &w;
        f.x = x;
        f.ldx = ldx;
        f.m = n;
        f.norm_w = norm_w;
        f.ss_in = B.ss;
        f.n_ss_in = n_ss;
        f.eps = m->eps;
        f.epi = epi;
        f.y = y;
        f.ldy = ldy;
        if (epi == SKE_RESID) f.ss_out = B.ss;
        f.pv = B.pv;
        f.pi = B.pi;
        f.pn = B.pn;
        return launch_skinny_fused(f, B.ws, B.ws_bytes, s);
    };
    AttnArgs at;
    at.part_o = B.ap_o;
    at.part_ml = B.ap_ml;
    at.merge_ctr = B.ctr;
    at.xa = B.xa;
    at.n_heads = m->nh;
    at.n_kv = m->nkv;
    at.head_dim = m->hd;
    at.n_splits = n_splits;
    at.max_chunk = max_chunk;
    QkvPro qp;
    qp.ss_in = B.ss;
    qp.n_ss_in = n_ss;
    qp.k = m->h;
    qp.eps = m->eps;
    qp.q_scale = q_scale;
    for (int i = 0; i < n; i++) qp.rope[i] = d.rope[i];
    SCRY_TRY(launch_bd_embed(m->embed, m->h, d, B.x, B.ss, s));
    for (int l = 0; l < m->L; l++) {
        const auto &Ly = m->layers[l];
        c.layer = l;
        {  // the qkv rows' split partials; the attention launch sums them (RoPE, K / V append)
            SkinnyFused f;
            f.w = &Ly.qkv;
            f.x = B.x;
            f.ldx = m->h;
            f.m = n;
            f.norm_w = m->norm_in(l);
            f.ss_in = B.ss;
            f.n_ss_in = n_ss;
            f.eps = m->eps;
            f.epi = SKE_NONE;
            SkinnyParts sp;
            SCRY_TRY(launch_skinny_fused(f, B.ws, B.ws_bytes, s, &sp));
            qp.part = B.ws;
            qp.n_split = sp.n_split;
            qp.n_pad = sp.n_pad;
            qp.scale = sp.scale;
        }
        SCRY_TRY(launch_attn_decode_seqs(at, c, s, &qp));
        SCRY_TRY(mm(Ly.o, B.xa, m->q_dim, nullptr, SKE_RESID, B.x, m->h));
        SCRY_TRY(mm(Ly.gu, B.x, m->h, m->norm_post(l), SKE_SWIGLU, B.act, m->ffn));
        SCRY_TRY(mm(Ly.down, B.act, m->ffn, nullptr, SKE_RESID, B.x, m->h));
    }
    SCRY_TRY(mm(m->lm, B.x, m->h, m->norm_final(), SKE_LOGITS, B.logits, m->V));
    return launch_bd_argmax(B.logits, m->V, B.pv, B.pi, B.pn, skinny_tiles(m->lm), d, s);
}

// `steps` greedy decode steps of n sequences at once: tokens[i] is the token
// at position cs[i]->seq_len (the last one fed), out_tokens [n][steps] the
// tokens that follow; logits (host, may be null) receives [steps][n][V].  The
// step is captured once per call and replayed (direct launches under
// SCRY_HIP_NO_GRAPH).  ev (may be null): events recorded around the replays.
int decode_batch_core(scry_llama m, scry_kv_cache *cs, int n, const int64_t *tokens, int steps,
                      int64_t *out_tokens, float *logits, hipEvent_t *ev) {
    if (n < 1 || n > PF_MAX_SEQS || steps < 1)
        return set_error(SCRY_ERR_INVALID, "decode_batch: n_seq must be 1..%d and steps >= 1", PF_MAX_SEQS);
    if (m->lm.bf16)
        return set_error(SCRY_ERR_UNSUPPORTED, "decode_batch: int8 models only (bf16 weights decode one sequence)");
    if (m->h % 8 || m->q_dim % 8 || m->ffn % 8 || m->h > 64 * 128)
        return set_error(SCRY_ERR_UNSUPPORTED, "decode_batch: hidden, q and ffn sizes must be multiples of 8 "
                         "(hidden at most 8192)");
    DecodeSeqs d{};
    AttnSeqs c{};
    int max_seq = 0;
    std::vector<int> pos0(n);
    for (int i = 0; i < n; i++) {
        scry_kv_cache k = cs[i];
        if (!k || k->m != m) return set_error(SCRY_ERR_INVALID, "decode_batch: cache %d does not belong to the model", i);
        for (int j = 0; j < i; j++)
            if (cs[j] == k) return set_error(SCRY_ERR_INVALID, "decode_batch: cache %d given twice", i);
        if (k->seq_len + steps > k->max_seq)
            return set_error(SCRY_ERR_RANGE, "decode_batch: %d + %d rows exceed the cache (%d)", k->seq_len, steps,
                             k->max_seq);
        d.tokens[i] = k->tokens;
        d.rope[i] = k->rope_cs;
        c.k[i] = k->K(0);
        c.v[i] = k->Vc(0);
        c.ls[i] = (size_t)2 * k->max_seq * m->kv_dim;
        pos0[i] = k->seq_len;
        max_seq = std::max(max_seq, k->max_seq);
    }
    SCRY_TRY(check_ids(m, tokens, n));
    SCRY_TRY(batch_ws(m));
    auto &B = m->bd;
    d.pos = B.pos;
    d.n = n;
    c.pos = B.pos;
    c.n = n;
    int ns = 1, max_chunk = 16;
    attn_pick_splits(m->nkv, max_seq, &ns, &max_chunk);
    // about 256 attention workgroups over all sequences: at the Llama-3-8B
    // shape with 4 sequences (8 KV groups) 8 splits measured 198.1 ms for
    // 4 x 64 tokens against 201.0 with 16, 205.4 with 12 and 205.2 with 4
    const int want = std::max(1, 256 / (m->nkv * n));
    if (ns > want) {
        ns = want;
        max_chunk = (max_seq + ns - 1) / ns;
    }
    hipStream_t s = ctx().stream;
    for (int i = 0; i < n; i++)
        SCRY_HIP(hipMemcpyAsync(cs[i]->tokens + pos0[i], tokens + i, sizeof(int64_t), hipMemcpyHostToDevice, s));
    SCRY_HIP(hipMemcpyAsync(B.pos, pos0.data(), sizeof(int) * n, hipMemcpyHostToDevice, s));
    SCRY_TRY(sync_stream());
    const bool no_graph = !graph_replay();
    hipGraph_t g = nullptr;
    hipGraphExec_t gx = nullptr;
    if (!no_graph) {
        SCRY_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        const int rc = record_batch_step(m, d, c, ns, max_chunk, s);
        const hipError_t e = hipStreamEndCapture(s, &g);
        if (rc || e != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            if (rc) return rc;
            return hip_fail(e, "decode_batch capture", __FILE__, __LINE__);
        }
        const hipError_t ei = hipGraphInstantiate(&gx, g, nullptr, nullptr, 0);
        if (ei != hipSuccess) {
            (void)hipGraphDestroy(g);
            return hip_fail(ei, "decode_batch instantiate", __FILE__, __LINE__);
        }
    }
    int rc = SCRY_OK;
    hipError_t e = hipSuccess;
    if (ev && (e = hipEventRecord(ev[0], s)) != hipSuccess) rc = hip_fail(e, "event", __FILE__, __LINE__);
    for (int t = 0; t < steps && !rc; t++) {
        if (gx) {
            if ((e = hipGraphLaunch(gx, s)) != hipSuccess) rc = hip_fail(e, "decode_batch replay", __FILE__, __LINE__);
        } else {
            rc = record_batch_step(m, d, c, ns, max_chunk, s);
        }
        if (!rc && logits) {
            e = hipMemcpyAsync(logits + (size_t)t * n * m->V, B.logits, sizeof(float) * (size_t)n * m->V,
                               hipMemcpyDeviceToHost, s);
            if (e != hipSuccess) rc = hip_fail(e, "logits readback", __FILE__, __LINE__);
            if (!rc) rc = sync_stream();
        }
    }
    if (!rc && ev && (e = hipEventRecord(ev[1], s)) != hipSuccess) rc = hip_fail(e, "event", __FILE__, __LINE__);
    if (!rc) rc = sync_stream();
    for (int i = 0; i < n && !rc; i++) {
        e = hipMemcpy(out_tokens + (size_t)i * steps, cs[i]->tokens + pos0[i] + 1, sizeof(int64_t) * steps,
                      hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_fail(e, "token readback", __FILE__, __LINE__);
    }
    if (gx) (void)hipGraphExecDestroy(gx);
    if (g) (void)hipGraphDestroy(g);
    if (rc) return rc;
    for (int i = 0; i < n; i++) cs[i]->seq_len += steps;
    return SCRY_OK;
}

// generate() (generate.rs:51-89): the prompt is fed token by token through
// the decode step (or, with prefill, all but its last token through one
// batched prefill), then tokens follow, greedy (samp == nullptr) or drawn by
// the device sampler with rng state seed; the token loop runs on the device.
int generate_impl(scry_llama m, const int64_t *prompt, int n_prompt, int max_tokens, int64_t *out_tokens,
                  int *n_out, float *step_logits, bool prefill, const scry_sampling_config *samp = nullptr,
                  uint64_t *rng_state = nullptr) {
    SCRY_REQUIRE_INIT();
    if (!m || !prompt || !out_tokens || !n_out) return set_error(SCRY_ERR_INVALID, "null argument");
    if (n_prompt <= 0) return set_error(SCRY_ERR_INVALID, "generate: prompt_tokens must not be empty");
    if (max_tokens < 0) return set_error(SCRY_ERR_INVALID, "generate: max_tokens < 0");
    SCRY_TRY(check_ids(m, prompt, n_prompt));
    const int nout = max_tokens > 0 ? max_tokens : 1;
    const int steps = n_prompt + nout - 1;
    scry_kv_cache c = nullptr;
    SCRY_TRY(cache_new(m, n_prompt + max_tokens, &c));  // generate.rs:62-63
    hipStream_t s = ctx().stream;
    int rc = SCRY_OK;
    hipError_t e = hipSuccess;
    if (samp) {
        c->sampling = true;
        c->samp = *samp;
        rc = dev_alloc((void **)&c->samp_ws, sizeof(double) * (size_t)m->V);
        if (!rc) rc = dev_alloc((void **)&c->rng, sizeof(unsigned long long));
        if (!rc && sample_uses_prep(*samp, m->V)) {
            const size_t pb = sample_prep_bytes(m->V);
            rc = dev_alloc(&c->samp_prep, pb);
            if (!rc) rc = launch_fill_u32((unsigned *)c->samp_prep, pb / 4, 0u, s);
        }
        if (!rc) {
            e = hipMemcpyAsync(c->rng, rng_state, sizeof *rng_state, hipMemcpyHostToDevice, s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (e != hipSuccess) rc = hip_fail(e, "rng upload", __FILE__, __LINE__);
        }
    }
    if (!rc) e = hipMemcpyAsync(c->tokens, prompt, sizeof(int64_t) * n_prompt, hipMemcpyHostToDevice, s);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "prompt upload", __FILE__, __LINE__);
    const int start = prefill ? n_prompt - 1 : 0;
    if (!rc && start > 0) rc = prefill_core(m, &c, 1, prompt, start, nullptr, nullptr);
    if (!rc) rc = set_state(c, start, start, n_prompt);
    for (int t = start; t < steps && !rc; t++) {
        rc = run_step(c);
        if (!rc && step_logits && t >= n_prompt - 1) {
            e = hipMemcpyAsync(step_logits + (size_t)(t - (n_prompt - 1)) * m->V, c->logits,
                               sizeof(float) * m->V, hipMemcpyDeviceToHost, s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (e != hipSuccess) rc = hip_fail(e, "logits readback", __FILE__, __LINE__);
        }
    }
    if (!rc) {
        e = hipMemcpyAsync(out_tokens, c->tokens + n_prompt, sizeof(int64_t) * nout, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess && samp) e = hipMemcpyAsync(rng_state, c->rng, sizeof *rng_state, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "token readback", __FILE__, __LINE__);
    }
    cache_free(c);
    if (rc) return rc;
    *n_out = nout;
    return SCRY_OK;
}

}  // namespace

extern "C" {

int scry_hip_llama_new_random(const scry_llama_config *cfg, uint64_t seed, int quant_mode,
                              int init_on_device, scry_llama *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    scry_llama m = nullptr;
    SCRY_TRY(model_alloc(cfg, quant_mode, &m));
    const int h = m->h, V = m->V, ffn = m->ffn, qd = m->q_dim, kvd = m->kv_dim, qkvd = m->qkv_dim;
    const int T = host_threads();
    const float stdv = 0.02f;  // llama.rs:598 (an f32, promoted in init.rs:8)
    hipStream_t s = ctx().stream;
    uint64_t calls = 0;
    int rc = SCRY_OK;
    std::vector<float> buf, fused;
    if (!init_on_device) buf.resize(m->stage_n);
    // Draw n samples of the next tensor into dst (device) as rows of `cols`
    // values at stride ld starting at column col0; host draws go through buf.
    auto draw = [&](float *dst, size_t n, int cols, int ld, int col0) -> int {
        int r = SCRY_OK;
        if (init_on_device) {
            r = launch_normal_init(dst, n, seed, calls, 0.0f, stdv, cols, ld, col0, s);
        } else {
            host_normal_vec(seed, calls, n, 0.0f, stdv, buf.data(), T);
            if (cols == ld) {
                hipError_t e = hipMemcpyAsync(dst, buf.data(), n * sizeof(float), hipMemcpyHostToDevice, s);
                if (e == hipSuccess) e = hipStreamSynchronize(s);
                if (e != hipSuccess) r = hip_fail(e, "weight upload", __FILE__, __LINE__);
            } else {
                const size_t rows = n / cols;
                hipError_t e = hipMemcpy2DAsync(dst + col0, sizeof(float) * ld, buf.data(),
                                                sizeof(float) * cols, sizeof(float) * cols, rows,
                                                hipMemcpyHostToDevice, s);
                if (e == hipSuccess) e = hipStreamSynchronize(s);
                if (e != hipSuccess) r = hip_fail(e, "weight upload", __FILE__, __LINE__);
            }
        }
        calls += 2 * (uint64_t)n;
        return r;
    };
    // llama.rs:602-605 embed_tokens first (a tied lm_head is quantized from it)
    rc = draw(m->embed, (size_t)V * h, h, h, 0);
    if (!rc && m->cfg.tie_word_embeddings) rc = quant_into(m, m->embed, h, V, 1, m->lm, 1, 1, 0, false);
    for (int l = 0; l < m->L && !rc; l++) {
        auto &Ly = m->layers[l];
        // llama.rs:613-616 q, k, v, fused column-wise (fuse_qkv_weights, llama.rs:1009-1029)
        rc = draw(m->stage, (size_t)h * qd, qd, qkvd, 0);
        if (!rc) rc = draw(m->stage, (size_t)h * kvd, kvd, qkvd, qd);
        if (!rc) rc = draw(m->stage, (size_t)h * kvd, kvd, qkvd, qd + kvd);
        if (!rc) rc = quant_into(m, m->stage, h, qkvd, 0, Ly.qkv, 1, 1, 0, false);
        // llama.rs:627-630 o_proj; 645-656 gate, up, down
        if (!rc) rc = draw(m->stage, (size_t)qd * h, h, h, 0);
        if (!rc) rc = quant_into(m, m->stage, qd, h, 0, Ly.o, 1, 1, 0, false);
        if (!rc) rc = draw(m->stage, (size_t)h * ffn, ffn, ffn, 0);
        if (!rc) rc = quant_into(m, m->stage, h, ffn, 0, Ly.gu, 2, 4, 0, false);
        if (!rc) rc = draw(m->stage, (size_t)h * ffn, ffn, ffn, 0);
        if (!rc) rc = quant_into(m, m->stage, h, ffn, 0, Ly.gu, 2, 4, 2, true);
        if (!rc) rc = draw(m->stage, (size_t)ffn * h, h, h, 0);
        if (!rc) rc = quant_into(m, m->stage, ffn, h, 0, Ly.down, 1, 1, 0, false);
    }
    // llama.rs:664-671 untied lm_head last
    if (!rc && !m->cfg.tie_word_embeddings) {
        rc = draw(m->stage, (size_t)V * h, h, h, 0);
        if (!rc) rc = quant_into(m, m->stage, h, V, 1, m->lm, 1, 1, 0, false);
    }
    if (!rc) rc = sync_stream();
    if (rc) {
        model_free(m);
        return rc;
    }
    *out = m;
    return SCRY_OK;
}

// LlamaModel::from_safetensors (llama.rs:765-958) with the int8 composition.
// Tensors are looked up by their HF names in the shards (the first shard
// holding a name wins), widened to f32 on the device and quantized with the
// same path as the random init.  HF stores projections as [out, in], the
// GEMV stream's row-per-output order, so they are packed from that layout
// directly (the reference transposes them to [in, out] on the host first,
// llama.rs:832-839; per-tensor absmax and per-element rounding give the same
// int8 values either way).  Unlike the reference, a tensor whose shape does
// not match the config is an error.
int scry_hip_llama_from_safetensors(const scry_llama_config *cfg, const char *const *paths, int n_paths,
                                    int quant_mode, scry_llama *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!out) return set_error(SCRY_ERR_INVALID, "null argument");
    scry_llama m = nullptr;
    SCRY_TRY(model_alloc(cfg, quant_mode, &m));
    StShards *sh = nullptr;
    int rc = st_open(paths, n_paths, &sh);
    hipStream_t s = ctx().stream;
    void *raw = nullptr;
    size_t raw_n = 0;
    const int h = m->h, V = m->V, ffn = m->ffn, qd = m->q_dim, kvd = m->kv_dim;
    // tensor `name` ([rows, cols], or [cols] when rows == 0) into dst as f32
    auto fetch = [&](const std::string &name, int rows, int cols, float *dst) -> int {
        const StTensor *t = st_find(sh, name.c_str());
        if (!t) return set_error(SCRY_ERR_INVALID, "tensor '%s' not found in any shard", name.c_str());
        if (t->dtype == ST_OTHER)
            return set_error(SCRY_ERR_UNSUPPORTED, "unsupported dtype %s for tensor '%s'", t->dtype_name.c_str(),
                             name.c_str());
        const bool ok = rows > 0 ? t->shape.size() == 2 && t->shape[0] == rows && t->shape[1] == cols
                                 : t->shape.size() == 1 && t->shape[0] == cols;
        if (!ok) {
            std::string sh_s;
            for (size_t i = 0; i < t->shape.size(); i++) sh_s += (i ? ", " : "") + std::to_string(t->shape[i]);
            return rows > 0 ? set_error(SCRY_ERR_INVALID, "tensor '%s': shape [%s], expected [%d, %d]", name.c_str(),
                                        sh_s.c_str(), rows, cols)
                            : set_error(SCRY_ERR_INVALID, "tensor '%s': shape [%s], expected [%d]", name.c_str(),
                                        sh_s.c_str(), cols);
        }
        if (t->bytes > raw_n) {  // the previous tensor's kernels are ordered before the free on the stream
            SCRY_TRY(sync_stream());
            dev_free(raw);
            raw = nullptr;
            raw_n = 0;
            SCRY_TRY(dev_alloc(&raw, t->bytes));
            raw_n = t->bytes;
        }
        SCRY_HIP(hipMemcpyAsync(raw, t->data, t->bytes, hipMemcpyHostToDevice, s));
        return launch_widen(raw, t->dtype, t->numel, dst, s);
    };
    // llama.rs:826-827 embed_tokens; a tied lm_head is quantized from it
    if (!rc) rc = fetch("model.embed_tokens.weight", V, h, m->embed);
    if (!rc && m->cfg.tie_word_embeddings) rc = quant_into(m, m->embed, h, V, 1, m->lm, 1, 1, 0, false);
    for (int l = 0; l < m->L && !rc; l++) {
        auto &Ly = m->layers[l];
        const std::string p = "model.layers." + std::to_string(l);
        // llama.rs:833-883: q, k, v fused along the outputs (fuse_qkv_weights) as rows of [qkv_dim][h]
        rc = fetch(p + ".self_attn.q_proj.weight", qd, h, m->stage);
        if (!rc) rc = fetch(p + ".self_attn.k_proj.weight", kvd, h, m->stage + (size_t)qd * h);
        if (!rc) rc = fetch(p + ".self_attn.v_proj.weight", kvd, h, m->stage + (size_t)(qd + kvd) * h);
        if (!rc) rc = quant_into(m, m->stage, h, m->qkv_dim, 1, Ly.qkv, 1, 1, 0, false);
        if (!rc) rc = fetch(p + ".self_attn.o_proj.weight", h, qd, m->stage);
        if (!rc) rc = quant_into(m, m->stage, qd, h, 1, Ly.o, 1, 1, 0, false);
        if (!rc) rc = fetch(p + ".mlp.gate_proj.weight", ffn, h, m->stage);
        if (!rc) rc = quant_into(m, m->stage, h, ffn, 1, Ly.gu, 2, 4, 0, false);
        if (!rc) rc = fetch(p + ".mlp.up_proj.weight", ffn, h, m->stage);
        if (!rc) rc = quant_into(m, m->stage, h, ffn, 1, Ly.gu, 2, 4, 2, true);
        if (!rc) rc = fetch(p + ".mlp.down_proj.weight", h, ffn, m->stage);
        if (!rc) rc = quant_into(m, m->stage, ffn, h, 1, Ly.down, 1, 1, 0, false);
        // llama.rs:880-881, 901-904, 912-915: the loaded norm weights
        if (!rc) rc = fetch(p + ".input_layernorm.weight", 0, h, m->norms + (size_t)(2 * l) * h);
        if (!rc) rc = fetch(p + ".post_attention_layernorm.weight", 0, h, m->norms + (size_t)(2 * l + 1) * h);
    }
    if (!rc) rc = fetch("model.norm.weight", 0, h, m->norms + (size_t)(2 * m->L) * h);  // llama.rs:936-940
    if (!rc && !m->cfg.tie_word_embeddings) {                                          // llama.rs:942-953
        rc = fetch("lm_head.weight", V, h, m->stage);
        if (!rc) rc = quant_into(m, m->stage, h, V, 1, m->lm, 1, 1, 0, false);
    }
    m->eps = cfg->rms_norm_eps;  // RMSNorm { eps: config.rms_norm_eps } (llama.rs:903, 914, 939)
    const int rs = sync_stream();
    if (!rc) rc = rs;
    dev_free(raw);
    st_close(sh);
    if (rc) {
        model_free(m);
        return rc;
    }
    *out = m;
    return SCRY_OK;
}

int scry_hip_llama_free(scry_llama m) {
    API_LOCK;
    if (!m) return SCRY_OK;
    if (m->live_caches > 0)
        return set_error(SCRY_ERR_INVALID, "free the model's %d KV cache(s) first", m->live_caches);
    if (ctx().init) (void)hipStreamSynchronize(ctx().stream);
    model_free(m);
    return SCRY_OK;
}

int scry_hip_llama_set_tensor(scry_llama m, int tensor_id, int layer, const float *host, size_t n) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !host) return set_error(SCRY_ERR_INVALID, "null argument");
    size_t need = 0;
    switch (tensor_id) {
        case SCRY_T_EMBED:
        case SCRY_T_LM_HEAD: need = (size_t)m->V * m->h; break;
        case SCRY_T_QKV: need = (size_t)m->h * m->qkv_dim; break;
        case SCRY_T_O: need = (size_t)m->q_dim * m->h; break;
        case SCRY_T_GATE:
        case SCRY_T_UP: need = (size_t)m->h * m->ffn; break;
        case SCRY_T_DOWN: need = (size_t)m->ffn * m->h; break;
        default: return set_error(SCRY_ERR_INVALID, "unknown tensor id %d", tensor_id);
    }
    if (n != need) return set_error(SCRY_ERR_INVALID, "tensor %d: %zu elements, expected %zu", tensor_id, n, need);
    SCRY_TRY(load_tensor(m, tensor_id, layer, host));
    return sync_stream();
}

int scry_hip_llama_get_qtensor(scry_llama m, int tensor_id, int layer, int8_t *host, size_t n,
                               float *scale) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !host) return set_error(SCRY_ERR_INVALID, "null argument");
    if (m->quant_mode == SCRY_QUANT_BF16)
        return set_error(SCRY_ERR_UNSUPPORTED, "get_qtensor: the model holds bf16 weights, not int8");
    const Packed *P = nullptr;
    int grp = 1, stride = 1, off = 0, nk = 0;
    float sc = 0.f;
    if (tensor_id == SCRY_T_LM_HEAD) {
        P = &m->lm;
        nk = 1;
        sc = P->scale;
    } else {
        if (layer < 0 || layer >= m->L) return set_error(SCRY_ERR_INVALID, "layer out of range");
        auto &Ly = m->layers[layer];
        switch (tensor_id) {
            case SCRY_T_QKV: P = &Ly.qkv; sc = P->scale; break;
            case SCRY_T_O: P = &Ly.o; sc = P->scale; break;
            case SCRY_T_GATE: P = &Ly.gu; grp = 2; stride = 4; off = 0; sc = P->scale; break;
            case SCRY_T_UP: P = &Ly.gu; grp = 2; stride = 4; off = 2; sc = P->scale2; break;
            case SCRY_T_DOWN: P = &Ly.down; sc = P->scale; break;
            default: return set_error(SCRY_ERR_INVALID, "tensor id %d has no int8 weights", tensor_id);
        }
    }
    if (n != (size_t)P->k * P->n) return set_error(SCRY_ERR_INVALID, "get_qtensor: expected %zu elements", (size_t)P->k * P->n);
    int8_t *d = nullptr;
    SCRY_TRY(dev_alloc((void **)&d, n));
    int rc = launch_unpack(P->d, P->kp, P->k, P->n, nk, grp, stride, off, d, ctx().stream);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(host, d, n, hipMemcpyDeviceToHost, ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "get_qtensor readback", __FILE__, __LINE__);
    }
    dev_free(d);
    if (scale) *scale = m->quant_mode == SCRY_QUANT_PER_TENSOR ? sc : 0.f;
    return rc;
}

int scry_hip_llama_get_embed(scry_llama m, float *host, size_t n) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !host || n != (size_t)m->V * m->h) return set_error(SCRY_ERR_INVALID, "get_embed: bad size");
    SCRY_HIP(hipMemcpyAsync(host, m->embed, n * sizeof(float), hipMemcpyDeviceToHost, ctx().stream));
    return sync_stream();
}

int scry_hip_llama_kv_cache_new(scry_llama m, int max_seq, scry_kv_cache *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !out) return set_error(SCRY_ERR_INVALID, "null argument");
    SCRY_TRY(cache_new(m, max_seq, out));
    return sync_stream();
}

int scry_hip_kv_cache_free(scry_kv_cache c) {
    API_LOCK;
    if (!c) return SCRY_OK;
    if (ctx().init) (void)hipStreamSynchronize(ctx().stream);
    cache_free(c);
    return SCRY_OK;
}

int scry_hip_kv_cache_seq_len(scry_kv_cache c, int *seq_len) {
    if (!c || !seq_len) return set_error(SCRY_ERR_INVALID, "null argument");
    *seq_len = c->seq_len;
    return SCRY_OK;
}

int scry_hip_kv_cache_layer_to_vec(scry_kv_cache c, int layer, float *k_host, float *v_host,
                                   size_t n) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!c || layer < 0 || layer >= c->m->L) return set_error(SCRY_ERR_INVALID, "bad layer");
    const size_t need = (size_t)c->max_seq * c->m->kv_dim;
    if (n != need) return set_error(SCRY_ERR_INVALID, "kv layer has %zu elements", need);
    if (k_host) SCRY_HIP(hipMemcpyAsync(k_host, c->K(layer), need * 4, hipMemcpyDeviceToHost, ctx().stream));
    if (v_host) SCRY_HIP(hipMemcpyAsync(v_host, c->Vc(layer), need * 4, hipMemcpyDeviceToHost, ctx().stream));
    return sync_stream();
}

int scry_hip_llama_forward_with_cache(scry_llama m, scry_kv_cache c, int64_t token, int pos,
                                      float *logits, int64_t *argmax_out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !c || c->m != m) return set_error(SCRY_ERR_INVALID, "cache does not belong to the model");
    SCRY_TRY(check_ids(m, &token, 1));
    if (c->seq_len >= c->max_seq)
        return set_error(SCRY_ERR_RANGE, "KV cache full (%d rows)", c->max_seq);
    if (pos < 0 || pos >= c->max_seq)
        return set_error(SCRY_ERR_RANGE, "position %d outside the cache's RoPE table (%d)", pos, c->max_seq);
    hipStream_t s = ctx().stream;
    c->hs->tok = token;
    SCRY_HIP(hipMemcpyAsync(c->tokens + pos, &c->hs->tok, sizeof(int64_t), hipMemcpyHostToDevice, s));
    SCRY_TRY(set_state(c, pos, c->seq_len, INT_MAX));
    SCRY_TRY(run_step(c));
    if (logits)
        SCRY_HIP(hipMemcpyAsync(logits, c->logits, sizeof(float) * m->V, hipMemcpyDeviceToHost, s));
    if (argmax_out) SCRY_HIP(hipMemcpyAsync(&c->hs->amax, c->amax, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    SCRY_TRY(sync_stream());
    if (argmax_out) *argmax_out = c->hs->amax;
    c->seq_len++;
    return SCRY_OK;
}

int scry_hip_llama_generate_greedy(scry_llama m, const int64_t *prompt, int n_prompt,
                                   int max_tokens, int64_t *out_tokens, int *n_out,
                                   float *step_logits) {
    API_LOCK;
    return generate_impl(m, prompt, n_prompt, max_tokens, out_tokens, n_out, step_logits, false);
}

int scry_hip_llama_generate_greedy_prefill(scry_llama m, const int64_t *prompt, int n_prompt, int max_tokens,
                                           int64_t *out_tokens, int *n_out, float *step_logits) {
    API_LOCK;
    return generate_impl(m, prompt, n_prompt, max_tokens, out_tokens, n_out, step_logits, true);
}

int scry_hip_llama_generate(scry_llama m, const int64_t *prompt, int n_prompt, const scry_sampling_config *cfg,
                            uint64_t *rng_state, int prefill, int64_t *out_tokens, int *n_out, float *step_logits) {
    API_LOCK;
    if (!cfg || !rng_state) return set_error(SCRY_ERR_INVALID, "null argument");
    if (cfg->temperature != cfg->temperature || cfg->top_p != cfg->top_p)
        return set_error(SCRY_ERR_INVALID, "generate: temperature and top_p must not be NaN");
    if (cfg->top_k < 0) return set_error(SCRY_ERR_INVALID, "generate: top_k < 0");
    // generate.rs:96-98: below 1e-8 every token is the argmax; no rng draws
    const bool greedy = cfg->temperature < 1e-8f;
    return generate_impl(m, prompt, n_prompt, cfg->max_tokens, out_tokens, n_out, step_logits, prefill != 0,
                         greedy ? nullptr : cfg, rng_state);
}

int scry_hip_llama_forward(scry_llama m, const int64_t *tokens, int seq, float *logits) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !tokens || !logits || seq <= 0) return set_error(SCRY_ERR_INVALID, "forward: bad arguments");
    SCRY_TRY(check_ids(m, tokens, seq));
    scry_kv_cache c = nullptr;
    SCRY_TRY(cache_new(m, seq, &c));
    float *dl = nullptr;
    int rc = dev_alloc((void **)&dl, sizeof(float) * (size_t)seq * m->V);
    if (!rc) rc = prefill_core(m, &c, 1, tokens, seq, dl, nullptr);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(logits, dl, sizeof(float) * (size_t)seq * m->V, hipMemcpyDeviceToHost,
                                      ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "logits readback", __FILE__, __LINE__);
    }
    dev_free(dl);
    cache_free(c);
    return rc;
}

int scry_hip_llama_prefill(scry_llama m, scry_kv_cache *caches, int n_seq, const int64_t *tokens, int seq,
                           float *last_logits) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !caches || !tokens) return set_error(SCRY_ERR_INVALID, "null argument");
    if (n_seq < 1 || n_seq > PF_MAX_SEQS || seq < 1)
        return set_error(SCRY_ERR_INVALID, "prefill: n_seq must be 1..%d and seq >= 1", PF_MAX_SEQS);
    SCRY_TRY(prefill_ws(m, n_seq * seq, n_seq));
    SCRY_TRY(prefill_core(m, caches, n_seq, tokens, seq, nullptr, last_logits ? m->pf.last : nullptr));
    if (last_logits)
        SCRY_HIP(hipMemcpyAsync(last_logits, m->pf.last, sizeof(float) * (size_t)n_seq * m->V,
                                hipMemcpyDeviceToHost, ctx().stream));
    return sync_stream();
}

int scry_hip_llama_decode_batch(scry_llama m, scry_kv_cache *caches, int n_seq, const int64_t *tokens, int steps,
                                int64_t *out_tokens, float *logits) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || !caches || !tokens || !out_tokens) return set_error(SCRY_ERR_INVALID, "null argument");
    return decode_batch_core(m, caches, n_seq, tokens, steps, out_tokens, logits, nullptr);
}

}  // extern "C"

namespace {

// Prefill then decode, timed (scry_hip_llama_bench_prefill / _batch): the
// decode steps run sequence after sequence through the single-sequence step,
// or (batched) all sequences per step through the batched step, whose time
// covers its graph replays (the capture, once per call, is outside).
int bench_prefill_impl(scry_llama m, const int64_t *prompts, int n_seq, int n_prompt, int decode_steps,
                       int batched, int64_t *out_tokens, double *prefill_ms, double *decode_ms) {
    if (!m || !prompts || !prefill_ms || !decode_ms || n_seq < 1 || n_seq > PF_MAX_SEQS || n_prompt < 2 ||
        decode_steps < 1)
        return set_error(SCRY_ERR_INVALID, "bench_prefill: bad arguments");
    SCRY_TRY(check_ids(m, prompts, n_seq * n_prompt));
    const int pre = n_prompt - 1;  // the last prompt token starts the decode loop, as in generate
    std::vector<scry_kv_cache> cs(n_seq, nullptr);
    std::vector<int64_t> toks((size_t)n_seq * pre);
    for (int i = 0; i < n_seq; i++)
        std::memcpy(&toks[(size_t)i * pre], prompts + (size_t)i * n_prompt, sizeof(int64_t) * pre);
    hipStream_t s = ctx().stream;
    hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr, e3 = nullptr;
    int rc = SCRY_OK;
    for (int i = 0; i < n_seq && !rc; i++) rc = cache_new(m, n_prompt + decode_steps, &cs[i]);
    hipError_t e = hipSuccess;
    if (!rc) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventCreate(&e2);
    if (e == hipSuccess) e = hipEventCreate(&e3);
    if (e != hipSuccess) rc = hip_fail(e, "event create", __FILE__, __LINE__);
    // untimed pass (kernel loading), then the caches restart empty
    if (!rc) rc = prefill_core(m, cs.data(), n_seq, toks.data(), pre, nullptr, nullptr);
    if (!rc) rc = sync_stream();
    for (int i = 0; i < n_seq && !rc; i++) cs[i]->seq_len = 0;
    if (!rc && (e = hipEventRecord(e0, s)) != hipSuccess) rc = hip_fail(e, "event", __FILE__, __LINE__);
    if (!rc) rc = prefill_core(m, cs.data(), n_seq, toks.data(), pre, nullptr, nullptr);
    if (!rc && (e = hipEventRecord(e1, s)) != hipSuccess) rc = hip_fail(e, "event", __FILE__, __LINE__);
    std::vector<int64_t> bt;
    if (batched && !rc) {
        std::vector<int64_t> last(n_seq);
        for (int i = 0; i < n_seq; i++) last[i] = prompts[(size_t)i * n_prompt + pre];
        bt.resize((size_t)n_seq * decode_steps);
        hipEvent_t ev[2] = {e3, e2};  // around the replays
        rc = decode_batch_core(m, cs.data(), n_seq, last.data(), decode_steps, bt.data(), nullptr, ev);
    }
    for (int i = 0; i < n_seq && !rc && !batched; i++) {
        scry_kv_cache c = cs[i];
        e = hipMemcpyAsync(c->tokens, prompts + (size_t)i * n_prompt, sizeof(int64_t) * n_prompt,
                           hipMemcpyHostToDevice, s);
        if (e != hipSuccess) rc = hip_fail(e, "prompt upload", __FILE__, __LINE__);
        if (!rc) rc = set_state(c, pre, pre, n_prompt);
        for (int t = 0; t < decode_steps && !rc; t++) rc = run_step(c);
    }
    if (!rc && !batched && (e = hipEventRecord(e2, s)) != hipSuccess) rc = hip_fail(e, "event", __FILE__, __LINE__);
    if (!rc) rc = sync_stream();
    float f1 = 0.f, f2 = 0.f;
    if (!rc && (e = hipEventElapsedTime(&f1, e0, e1)) == hipSuccess)
        e = hipEventElapsedTime(&f2, batched ? e3 : e1, e2);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "event time", __FILE__, __LINE__);
    if (!rc && out_tokens && batched) std::memcpy(out_tokens, bt.data(), sizeof(int64_t) * bt.size());
    for (int i = 0; i < n_seq && !rc && !batched; i++) {
        if (out_tokens) {
            e = hipMemcpy(out_tokens + (size_t)i * decode_steps, cs[i]->tokens + n_prompt,
                          sizeof(int64_t) * decode_steps, hipMemcpyDeviceToHost);
            if (e != hipSuccess) rc = hip_fail(e, "token readback", __FILE__, __LINE__);
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (e2) (void)hipEventDestroy(e2);
    if (e3) (void)hipEventDestroy(e3);
    for (auto c : cs) cache_free(c);
    if (rc) return rc;
    *prefill_ms = f1;
    *decode_ms = f2;
    return SCRY_OK;
}

}  // namespace

extern "C" {

int scry_hip_llama_bench_prefill(scry_llama m, const int64_t *prompts, int n_seq, int n_prompt, int decode_steps,
                                 int64_t *out_tokens, double *prefill_ms, double *decode_ms) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return bench_prefill_impl(m, prompts, n_seq, n_prompt, decode_steps, 0, out_tokens, prefill_ms, decode_ms);
}

int scry_hip_llama_bench_prefill_batch(scry_llama m, const int64_t *prompts, int n_seq, int n_prompt,
                                       int decode_steps, int64_t *out_tokens, double *prefill_ms,
                                       double *decode_ms) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return bench_prefill_impl(m, prompts, n_seq, n_prompt, decode_steps, 1, out_tokens, prefill_ms, decode_ms);
}

// ------------------------------------------------------------ measurement
}  // extern "C"

namespace {

int bench_decode_impl(scry_llama m, const int64_t *prompt, int n_prompt, int warmup, int steps,
                      const scry_sampling_config *samp, uint64_t seed, int64_t *out_tokens, double *ms) {
    SCRY_REQUIRE_INIT();
    if (!m || !prompt || n_prompt <= 0 || steps <= 0 || warmup < 0 || !ms)
        return set_error(SCRY_ERR_INVALID, "bench_decode: bad arguments");
    SCRY_TRY(check_ids(m, prompt, n_prompt));
    scry_kv_cache c = nullptr;
    SCRY_TRY(cache_new(m, n_prompt + std::max(warmup, steps) + 1, &c));
    hipStream_t s = ctx().stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = SCRY_OK;
    hipError_t e = hipSuccess;
    if (samp) {  // as generate_impl: the device sampler after each LM head
        c->sampling = true;
        c->samp = *samp;
        rc = dev_alloc((void **)&c->samp_ws, sizeof(double) * (size_t)m->V);
        if (!rc) rc = dev_alloc((void **)&c->rng, sizeof(unsigned long long));
        if (!rc && sample_uses_prep(*samp, m->V)) {
            const size_t pb = sample_prep_bytes(m->V);
            rc = dev_alloc(&c->samp_prep, pb);
            if (!rc) rc = launch_fill_u32((unsigned *)c->samp_prep, pb / 4, 0u, s);
        }
        if (!rc) e = hipMemcpyAsync(c->rng, &seed, sizeof seed, hipMemcpyHostToDevice, s);
        if (!rc && e != hipSuccess) rc = hip_fail(e, "rng upload", __FILE__, __LINE__);
    }
    if (!rc) e = hipMemcpyAsync(c->tokens, prompt, sizeof(int64_t) * n_prompt, hipMemcpyHostToDevice, s);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "prompt upload", __FILE__, __LINE__);
    if (!rc) rc = set_state(c, 0, 0, n_prompt);
    // the prompt through the cache path, as generate() does
    for (int t = 0; t < n_prompt && !rc; t++) rc = run_step(c);
    for (int t = 0; t < warmup && !rc; t++) rc = run_step(c);
    if (!rc) rc = sync_stream();
    // rewind to the first decode position; the cache rows and token written
    // there are the same ones the warm-up produced
    if (!rc) rc = set_state(c, n_prompt, n_prompt, n_prompt);
    if (!rc) {
        e = hipEventCreate(&e0);
        if (e == hipSuccess) e = hipEventCreate(&e1);
        if (e == hipSuccess) e = hipEventRecord(e0, s);
        if (e != hipSuccess) rc = hip_fail(e, "event setup", __FILE__, __LINE__);
    }
    for (int t = 0; t < steps && !rc; t++) rc = run_step(c);
    if (!rc) {
        e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float f = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&f, e0, e1);
        if (e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
        *ms = f;
    }
    if (!rc && out_tokens) {
        e = hipMemcpyAsync(out_tokens, c->tokens + n_prompt + 1, sizeof(int64_t) * steps,
                           hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "token readback", __FILE__, __LINE__);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    cache_free(c);
    return rc;
}

// Step profile: the prompt through the cache path, then `steps` replays of
// the decode step captured with per-workgroup start / end stamps (the same
// launches as the bench's graph; direct launches when graphs are off).  For
// each step and launch: the earliest workgroup start and the latest end, in
// us from the step's first start.
int profile_step_impl(scry_llama m, const int64_t *prompt, int n_prompt, int steps, int max_launches,
                      int *n_launches, double *start_us, double *end_us) {
    SCRY_REQUIRE_INIT();
    if (!m || !prompt || n_prompt <= 0 || steps <= 0 || !n_launches || !start_us || !end_us)
        return set_error(SCRY_ERR_INVALID, "profile_step: bad arguments");
    const int nl = 5 * m->L + 2;
    *n_launches = nl;
    if (max_launches < nl) return set_error(SCRY_ERR_INVALID, "profile_step: %d launches per step > %d", nl, max_launches);
    SCRY_TRY(check_ids(m, prompt, n_prompt));
    scry_kv_cache c = nullptr;
    SCRY_TRY(cache_new(m, n_prompt + steps + 1, &c));
    // stamp slots per launch: the largest grid of the step
    size_t slots = (size_t)qgemv_blocks(EPI_LOGITS, m->lm, 1);
    for (const auto &Ly : m->layers)
        for (const Packed *w : {&Ly.qkv, &Ly.o, &Ly.gu, &Ly.down})
            slots = std::max(slots, (size_t)qgemv_blocks(EPI_RESID, *w, 1));
    slots = std::max(slots, (size_t)8 * ((m->nkv + 7) / 8) * c->n_splits);
    slots = std::max(slots, (size_t)1);
    const size_t bytes = 2 * slots * nl * sizeof(unsigned long long);
    hipStream_t s = ctx().stream;
    unsigned long long *ts = nullptr;
    std::vector<unsigned long long> h;
    hipGraph_t g = nullptr;
    hipGraphExec_t gx = nullptr;
    hipError_t e = hipSuccess;
    int rc = dev_alloc((void **)&ts, bytes);
    if (!rc) {
        e = hipMemcpyAsync(c->tokens, prompt, sizeof(int64_t) * n_prompt, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) rc = hip_fail(e, "prompt upload", __FILE__, __LINE__);
    }
    if (!rc) rc = set_state(c, 0, 0, n_prompt);
    for (int t = 0; t < n_prompt && !rc; t++) rc = run_step(c);
    if (!rc && graph_replay()) {
        e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            rc = record_step(c, s, ts, slots);
            e = hipStreamEndCapture(s, &g);
            if (!rc && e == hipSuccess) e = hipGraphInstantiate(&gx, g, nullptr, nullptr, 0);
        }
        if (!rc && e != hipSuccess) rc = hip_fail(e, "profile graph capture", __FILE__, __LINE__);
    }
    if (!rc) {
        try {
            h.resize(bytes / sizeof(unsigned long long));
        } catch (...) {
            rc = set_error(SCRY_ERR_OOM, "profile_step: host buffer of %zu bytes", bytes);
        }
    }
    for (int t = 0; t < steps && !rc; t++) {
        e = hipMemsetAsync(ts, 0, bytes, s);  // outside the captured graph
        if (e == hipSuccess) e = gx ? hipGraphLaunch(gx, s) : hipSuccess;
        if (e != hipSuccess) {
            rc = hip_fail(e, "profile replay", __FILE__, __LINE__);
            break;
        }
        if (!gx) rc = record_step(c, s, ts, slots);
        if (!rc) e = hipMemcpyAsync(h.data(), ts, bytes, hipMemcpyDeviceToHost, s);
        if (!rc && e == hipSuccess) e = hipStreamSynchronize(s);
        if (!rc && e != hipSuccess) rc = hip_fail(e, "profile readback", __FILE__, __LINE__);
        if (rc) break;
        unsigned long long t0 = ~0ull;
        std::vector<unsigned long long> lo(nl, ~0ull), hi(nl, 0);
        for (int i = 0; i < nl; i++) {
            const unsigned long long *p = h.data() + 2 * slots * i;
            for (size_t b = 0; b < slots; b++) {
                if (p[2 * b]) lo[i] = std::min(lo[i], p[2 * b]);
                hi[i] = std::max(hi[i], p[2 * b + 1]);
            }
            t0 = std::min(t0, lo[i]);
        }
        for (int i = 0; i < nl; i++) {  // s_memrealtime: 100 MHz
            start_us[(size_t)t * max_launches + i] = lo[i] == ~0ull ? -1.0 : (double)(lo[i] - t0) * 0.01;
            end_us[(size_t)t * max_launches + i] = hi[i] == 0 ? -1.0 : (double)(hi[i] - t0) * 0.01;
        }
    }
    if (gx) (void)hipGraphExecDestroy(gx);
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamSynchronize(s);
    dev_free(ts);
    cache_free(c);
    return rc;
}

}  // namespace

extern "C" {

int scry_hip_graph_replay(void) { return graph_replay() ? 1 : 0; }

int scry_hip_llama_profile_step(scry_llama m, const int64_t *prompt, int n_prompt, int steps, int max_launches,
                                int *n_launches, double *start_us, double *end_us) {
    API_LOCK;
    return profile_step_impl(m, prompt, n_prompt, steps, max_launches, n_launches, start_us, end_us);
}

int scry_hip_llama_bench_decode(scry_llama m, const int64_t *prompt, int n_prompt, int warmup,
                                int steps, int64_t *out_tokens, double *ms) {
    API_LOCK;
    return bench_decode_impl(m, prompt, n_prompt, warmup, steps, nullptr, 0, out_tokens, ms);
}

int scry_hip_llama_bench_decode_sampled(scry_llama m, const int64_t *prompt, int n_prompt, int warmup, int steps,
                                        const scry_sampling_config *cfg, uint64_t seed, int64_t *out_tokens,
                                        double *ms) {
    API_LOCK;
    if (!cfg || !(cfg->temperature >= 1e-8f) || cfg->top_k < 0 || cfg->top_p != cfg->top_p)
        return set_error(SCRY_ERR_INVALID, "bench_decode_sampled: needs temperature >= 1e-8, top_k >= 0");
    return bench_decode_impl(m, prompt, n_prompt, warmup, steps, cfg, seed, out_tokens, ms);
}

int scry_hip_llama_time_projection(scry_llama m, int tensor_id, int layer, int iters,
                                   double *avg_us, double *bytes_per_launch) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    (void)layer;  // launches rotate over all layers so the weights stream from HBM
    if (!m || iters <= 0 || !avg_us) return set_error(SCRY_ERR_INVALID, "time_projection: bad arguments");
    scry_kv_cache c = nullptr;
    SCRY_TRY(cache_new(m, 16, &c));
    hipStream_t s = ctx().stream;
    int rc = launch_fill_f32(c->x, m->h, 1.0f, s);
    if (!rc) rc = launch_fill_f32(c->xa, m->q_dim, 0.5f, s);
    if (!rc) rc = launch_fill_f32(c->act, m->ffn, 0.25f, s);
    if (!rc) {
        c->hs->tok = 0;
        hipError_t e = hipMemcpyAsync(c->tokens, &c->hs->tok, sizeof(int64_t), hipMemcpyHostToDevice, s);
        if (e != hipSuccess) rc = hip_fail(e, "token upload", __FILE__, __LINE__);
    }
    if (!rc) rc = set_state(c, 0, 0, INT_MAX);
    double bytes = 0;
    auto launch = [&](int l) -> int {
        switch (tensor_id) {
            case SCRY_T_QKV: return launch_qgemv(EPI_QKV, qkv_args(c, l), s);
            case SCRY_T_O: return launch_qgemv(EPI_RESID, o_args(c, l), s);
            case SCRY_T_GATE: return launch_qgemv(EPI_SWIGLU, gu_args(c, l), s);
            case SCRY_T_DOWN: return launch_qgemv(EPI_RESID, down_args(c, l), s);
            case SCRY_T_LM_HEAD: return launch_qgemv(EPI_LOGITS, lm_args(c, 0), s);
        }
        return set_error(SCRY_ERR_INVALID, "time_projection: tensor id %d", tensor_id);
    };
    const Packed *P = nullptr;
    switch (tensor_id) {
        case SCRY_T_QKV: P = &m->layers[0].qkv; break;
        case SCRY_T_O: P = &m->layers[0].o; break;
        case SCRY_T_GATE: P = &m->layers[0].gu; break;
        case SCRY_T_DOWN: P = &m->layers[0].down; break;
        case SCRY_T_LM_HEAD: P = &m->lm; break;
        default: rc = set_error(SCRY_ERR_INVALID, "time_projection: tensor id %d", tensor_id);
    }
    if (P) {
        // algorithmic bytes: weights (int8 + scales, or bf16) + activation in + result out
        const double out_n = tensor_id == SCRY_T_GATE ? P->rows / 2.0 : (double)P->rows;
        const double scales = P->bf16 ? 0.0 : P->s32 ? 4.0 * P->rows * P->nb : (P->fused ? 8.0 : 4.0);
        bytes = (double)P->rows * P->k * (P->bf16 ? 2.0 : 1.0) + scales + 4.0 * P->k + 4.0 * out_n;
    }
    const int nl = tensor_id == SCRY_T_LM_HEAD ? 1 : m->L;
    // the RMSNorm'd GEMVs read the pre-scaled row and partial sums that the
    // residual GEMV before them leaves
    if (!rc && (tensor_id == SCRY_T_QKV || tensor_id == SCRY_T_LM_HEAD))
        rc = launch_qgemv(EPI_RESID, down_args(c, m->L - 1), s);
    if (!rc && tensor_id == SCRY_T_GATE) rc = launch_qgemv(EPI_RESID, o_args(c, 0), s);
    for (int i = 0; i < std::min(iters, 8) && !rc; i++) rc = launch(i % nl);  // warm-up
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) {
        hipError_t e = hipEventCreate(&e0);
        if (e == hipSuccess) e = hipEventCreate(&e1);
        if (e == hipSuccess) e = hipEventRecord(e0, s);
        if (e != hipSuccess) rc = hip_fail(e, "event setup", __FILE__, __LINE__);
    }
    for (int i = 0; i < iters && !rc; i++) rc = launch(i % nl);
    if (!rc) {
        hipError_t e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float f = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&f, e0, e1);
        if (e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
        *avg_us = 1000.0 * f / iters;
    }
    if (bytes_per_launch) *bytes_per_launch = bytes;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    cache_free(c);
    return rc;
}

int scry_hip_llama_time_attention(scry_llama m, int ctx_len, int iters, double *avg_us, double *bytes_per_launch) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!m || ctx_len <= 0 || ctx_len > m->cfg.max_seq_len || iters <= 0 || !avg_us)
        return set_error(SCRY_ERR_INVALID, "time_attention: bad arguments");
    scry_kv_cache c = nullptr;
    SCRY_TRY(cache_new(m, ctx_len, &c));
    hipStream_t s = ctx().stream;
    // every layer's cache holds ctx_len rows (the decode step's shape at that length)
    int rc = launch_fill_f32(c->kv, (size_t)m->L * 2 * ctx_len * m->kv_dim, 0.03125f, s);
    if (!rc) rc = launch_fill_f32(c->xq, m->q_dim, 0.0625f, s);
    auto launch = [&](int l) {
        AttnArgs a = attn_args(c, l);
        a.fixed_len = ctx_len;
        return launch_attn_decode(a, s);
    };
    for (int i = 0; i < std::min(iters, 8) && !rc; i++) rc = launch(i % m->L);  // warm-up
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) {
        hipError_t e = hipEventCreate(&e0);
        if (e == hipSuccess) e = hipEventCreate(&e1);
        if (e == hipSuccess) e = hipEventRecord(e0, s);
        if (e != hipSuccess) rc = hip_fail(e, "event setup", __FILE__, __LINE__);
    }
    for (int i = 0; i < iters && !rc; i++) rc = launch(i % m->L);  // rotating: K/V stream from HBM
    if (!rc) {
        hipError_t e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float f = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&f, e0, e1);
        if (e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
        *avg_us = 1000.0 * f / iters;
    }
    // algorithmic bytes: the K and V rows once, q in, the attention row out
    if (bytes_per_launch) *bytes_per_launch = 8.0 * ctx_len * m->kv_dim + 8.0 * m->q_dim;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    cache_free(c);
    return rc;
}

}  // extern "C"

namespace {

int bench_qgemv_impl(int m_rows, int k, int n, int quant_mode, int n_bufs, int warmup, int iters, bool with_bias,
                     double *avg_us, double *bytes_per_launch) {
    SCRY_REQUIRE_INIT();
    if (m_rows <= 0 || k <= 0 || n <= 0 || n_bufs <= 0 || iters <= 0 || !avg_us)
        return set_error(SCRY_ERR_INVALID, "bench_qgemv: bad arguments");
    hipStream_t s = ctx().stream;
    std::vector<Packed> W(n_bufs);
    float *x = nullptr, *y = nullptr, *bias = nullptr;
    int rc = dev_alloc((void **)&x, sizeof(float) * (size_t)m_rows * k);
    if (!rc) rc = dev_alloc((void **)&y, sizeof(float) * (size_t)m_rows * n);
    if (!rc) rc = launch_fill_f32(x, (size_t)m_rows * k, 0.5f, s);
    if (!rc && with_bias) rc = dev_alloc((void **)&bias, sizeof(float) * (size_t)n);
    if (!rc && with_bias) rc = launch_fill_f32(bias, (size_t)n, 0.25f, s);
    for (int b = 0; b < n_bufs && !rc; b++) {
        Packed &P = W[b];
        P.k = k;
        P.n = n;
        P.kp = round_up(k, 16);
        P.rows = n;
        P.scale = 1.0f / 127.0f;
        rc = dev_alloc((void **)&P.d, P.bytes());
        if (!rc) rc = launch_fill_u32((unsigned *)P.d, P.bytes() / 4, 0x8a7f9180u + b, s);
        if (!rc && quant_mode == SCRY_QUANT_BLOCK32) {
            P.nb = (k + 31) / 32;
            rc = dev_alloc((void **)&P.s32, sizeof(float) * (size_t)n * P.nb);
            if (!rc) rc = launch_fill_f32(P.s32, (size_t)n * P.nb, 1.0f / 127.0f, s);
        }
    }
    auto launch = [&](int i) {
        GemvArgs g;
        g.w = &W[i % n_bufs];
        g.x = x;
        g.ldx = k;
        g.m = m_rows;
        g.y = y;
        g.ldy = n;
        g.bias = bias;
        return launch_qgemv(EPI_STORE, g, s);
    };
    for (int i = 0; i < warmup && !rc; i++) rc = launch(i);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) {
        hipError_t e = hipEventCreate(&e0);
        if (e == hipSuccess) e = hipEventCreate(&e1);
        if (e == hipSuccess) e = hipEventRecord(e0, s);
        if (e != hipSuccess) rc = hip_fail(e, "event setup", __FILE__, __LINE__);
    }
    for (int i = 0; i < iters && !rc; i++) rc = launch(i);
    if (!rc) {
        hipError_t e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float f = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&f, e0, e1);
        if (e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
        *avg_us = 1000.0 * f / iters;
    }
    if (bytes_per_launch) {
        const double scales = quant_mode == SCRY_QUANT_BLOCK32 ? 4.0 * n * ((k + 31) / 32) : 4.0;
        *bytes_per_launch = (double)k * n + scales + 4.0 * m_rows * k + 4.0 * m_rows * n + (with_bias ? 4.0 * n : 0.0);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    for (auto &P : W) packed_free(P);
    dev_free(x);
    dev_free(y);
    dev_free(bias);
    return rc;
}

// Per-launch device times of matmul_i8_f32 at (m, k, n) over n_bufs weight
// copies.  path 0: the route matmul_i8_f32 takes (the skinny MFMA kernel where
// skinny_route admits the shape, else the GEMV up to GEMV_MAX_M activation
// rows, the MFMA GEMM above); 1: the GEMV; 2: the GEMM (its bf16 activation
// split included, as matmul_i8_f32 runs it); 3: the skinny MFMA kernel (its
// ordered split reduction included).
int bench_qgemv_dist_impl(int m, int k, int n, int quant_mode, int path, int n_bufs, int warmup, int iters,
                          int group, double *per_launch_us, double *avg_us, double *bytes_per_launch) {
    SCRY_REQUIRE_INIT();
    if (m <= 0 || k <= 0 || n <= 0 || n_bufs <= 0 || iters <= 0 || !avg_us || path < 0 || path > 3 ||
        group < 1 || iters % group ||
        (quant_mode != SCRY_QUANT_PER_TENSOR && quant_mode != SCRY_QUANT_BLOCK32))
        return set_error(SCRY_ERR_INVALID, "bench_qgemv_dist: bad arguments");
    const bool skinny = path == 3 || (path == 0 && skinny_route(m, k, n));
    const bool gemm = !skinny && (path == 2 || (path == 0 && m > GEMV_MAX_M));
    if (!gemm && !skinny && m > GEMV_MAX_M)
        return set_error(SCRY_ERR_INVALID, "bench_qgemv_dist: the GEMV takes <= %d rows", GEMV_MAX_M);
    if (skinny && (m > GEMV_MAX_M || k % 8 != 0))
        return set_error(SCRY_ERR_INVALID, "bench_qgemv_dist: the skinny kernel takes <= %d rows and k %% 8 == 0",
                         GEMV_MAX_M);
    hipStream_t s = ctx().stream;
    std::vector<Packed> W(n_bufs);
    float *x = nullptr, *y = nullptr;
    unsigned short *pl = nullptr;
    const int mp = prefill_rows_pad(m), ld = prefill_k_pad(k);
    int rc = dev_alloc((void **)&x, sizeof(float) * (size_t)m * k);
    if (!rc) rc = dev_alloc((void **)&y, sizeof(float) * (size_t)m * n);
    if (!rc) rc = launch_fill_f32(x, (size_t)m * k, 0.5f, s);
    // the GEMM's input as matmul_i8_f32 forms it: digit planes (per-tensor,
    // k <= 16384; the int8 matrix cores) or the bf16 hi / lo planes
    const bool digits = gemm && quant_mode == SCRY_QUANT_PER_TENSOR && k <= 16384;
    const size_t dstride = (size_t)mp * ld;
    if (!rc && gemm) rc = dev_alloc((void **)&pl, digits ? 3 * dstride + sizeof(int) * (size_t)mp
                                                         : sizeof(unsigned short) * 2 * dstride);
    if (!rc && gemm) rc = launch_fill_u32((unsigned *)pl, digits ? (3 * dstride) / 4 + mp : dstride, 0u, s);
    void *sws = nullptr;
    if (!rc && skinny) rc = ctx_workspace(skinny_ws_bytes(m, k, n), &sws);
    for (int b = 0; b < n_bufs && !rc; b++) {
        Packed &P = W[b];
        P.k = k;
        P.n = n;
        P.kp = round_up(k, 16);
        P.rows = n;
        P.scale = 1.0f / 127.0f;
        rc = dev_alloc((void **)&P.d, P.bytes());
        if (!rc) rc = launch_fill_u32((unsigned *)P.d, P.bytes() / 4, 0x8a7f9180u + b, s);
        if (!rc && quant_mode == SCRY_QUANT_BLOCK32) {
            P.nb = (k + 31) / 32;
            rc = dev_alloc((void **)&P.s32, sizeof(float) * (size_t)n * P.nb);
            if (!rc) rc = launch_fill_f32(P.s32, (size_t)n * P.nb, 1.0f / 127.0f, s);
        }
    }
    auto launch = [&](int i) {
        if (skinny) {
            SkinnyMM sm;
            sm.w = &W[i % n_bufs];
            sm.x = x;
            sm.ldx = k;
            sm.m = m;
            sm.y = y;
            sm.ldy = n;
            return launch_skinny(sm, (float *)sws, ctx().ws_bytes, s);
        }
        if (!gemm) {
            GemvArgs g;
            g.w = &W[i % n_bufs];
            g.x = x;
            g.ldx = k;
            g.m = m;
            g.y = y;
            g.ldy = n;
            return launch_qgemv(EPI_STORE, g, s);
        }
        PrefillGemm g;
        g.w = &W[i % n_bufs];
        g.lda = ld;
        g.M = m;
        g.c = y;
        g.ldc = n;
        if (digits) {
            signed char *dg = reinterpret_cast<signed char *>(pl);
            int *de = reinterpret_cast<int *>(dg + 3 * dstride);
            SCRY_TRY(launch_norm_digits(x, k, m, nullptr, k, 0.f, dg, dstride, de, ld, s));
            g.ad = dg;
            g.ae = de;
            g.dstride = dstride;
        } else {
            SCRY_TRY(launch_split(x, k, m, k, pl, pl + dstride, ld, s));
            g.ahi = pl;
            g.alo = pl + dstride;
        }
        return launch_gemm(PF_STORE, g, s);
    };
    for (int i = 0; i < warmup && !rc; i++) rc = launch(i);
    std::vector<hipEvent_t> ev;
    const int ng = iters / group;
    const int nev = per_launch_us ? ng + 1 : 0;
    for (int i = 0; i < nev + 2 && !rc; i++) {
        hipEvent_t e = nullptr;
        hipError_t he = hipEventCreate(&e);
        if (he != hipSuccess) rc = hip_fail(he, "event create", __FILE__, __LINE__);
        else ev.push_back(e);
    }
    // the average: back-to-back launches between two events
    if (!rc) {
        hipError_t e = hipEventRecord(ev[0], s);
        for (int i = 0; i < iters && !rc && e == hipSuccess; i++) rc = launch(i);
        if (!rc && e == hipSuccess) e = hipEventRecord(ev[1], s);
        if (!rc && e == hipSuccess) e = hipEventSynchronize(ev[1]);
        float f = 0.f;
        if (!rc && e == hipSuccess) e = hipEventElapsedTime(&f, ev[0], ev[1]);
        if (!rc && e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
        if (!rc) *avg_us = 1000.0 * f / iters;
    }
    // the distribution: an event after every `group` launches (per-launch
    // average of each group; an event between single launches adds its own
    // gap to every sample)
    if (!rc && per_launch_us) {
        hipError_t e = hipEventRecord(ev[2], s);
        for (int i = 0; i < iters && !rc && e == hipSuccess; i++) {
            rc = launch(i);
            if (!rc && (i + 1) % group == 0) e = hipEventRecord(ev[3 + i / group], s);
        }
        if (!rc && e == hipSuccess) e = hipEventSynchronize(ev[2 + ng]);
        for (int i = 0; i < ng && !rc && e == hipSuccess; i++) {
            float f = 0.f;
            e = hipEventElapsedTime(&f, ev[2 + i], ev[3 + i]);
            per_launch_us[i] = 1000.0 * f / group;
        }
        if (!rc && e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
    }
    if (bytes_per_launch) {
        const double scales = quant_mode == SCRY_QUANT_BLOCK32 ? 4.0 * n * ((k + 31) / 32) : 4.0;
        *bytes_per_launch = (double)k * n + scales + 4.0 * m * k + 4.0 * m * n;
    }
    for (auto e : ev) (void)hipEventDestroy(e);
    (void)hipStreamSynchronize(s);
    for (auto &P : W) packed_free(P);
    dev_free(x);
    dev_free(y);
    dev_free(pl);
    return rc;
}

}  // namespace

extern "C" {

int scry_hip_bench_qgemv(int m_rows, int k, int n, int quant_mode, int n_bufs, int warmup,
                         int iters, double *avg_us, double *bytes_per_launch) {
    API_LOCK;
    return bench_qgemv_impl(m_rows, k, n, quant_mode, n_bufs, warmup, iters, false, avg_us, bytes_per_launch);
}

int scry_hip_bench_qgemv_dist(int m, int k, int n, int quant_mode, int path, int n_bufs, int warmup, int iters,
                              int group, double *per_group_us, double *avg_us, double *bytes_per_launch) {
    API_LOCK;
    return bench_qgemv_dist_impl(m, k, n, quant_mode, path, n_bufs, warmup, iters, group, per_group_us, avg_us,
                                 bytes_per_launch);
}

int scry_hip_bench_gemv_bf16(int m_rows, int k, int n, int n_bufs, int warmup, int iters, double *avg_us,
                             double *bytes_per_launch) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (m_rows <= 0 || m_rows > GEMV_MAX_M || k <= 0 || n <= 0 || n_bufs <= 0 || iters <= 0 || !avg_us)
        return set_error(SCRY_ERR_INVALID, "bench_gemv_bf16: bad arguments");
    hipStream_t s = ctx().stream;
    const int kp = bf16_row_pad(k);
    std::vector<unsigned short *> W(n_bufs, nullptr);
    float *x = nullptr, *y = nullptr;
    int rc = dev_alloc((void **)&x, sizeof(float) * (size_t)m_rows * k);
    if (!rc) rc = dev_alloc((void **)&y, sizeof(float) * (size_t)m_rows * n);
    if (!rc) rc = launch_fill_f32(x, (size_t)m_rows * k, 0.5f, s);
    for (int b = 0; b < n_bufs && !rc; b++) {
        rc = dev_alloc((void **)&W[b], sizeof(unsigned short) * (size_t)n * kp);
        if (!rc) rc = launch_fill_u32((unsigned *)W[b], (size_t)n * kp / 2, 0x3c003c00u + b, s);  // finite bf16
    }
    auto launch = [&](int i) { return launch_gemv_bf16(W[i % n_bufs], kp, n, x, k, k, m_rows, y, n, nullptr, s); };
    for (int i = 0; i < warmup && !rc; i++) rc = launch(i);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) {
        hipError_t e = hipEventCreate(&e0);
        if (e == hipSuccess) e = hipEventCreate(&e1);
        if (e == hipSuccess) e = hipEventRecord(e0, s);
        if (e != hipSuccess) rc = hip_fail(e, "event setup", __FILE__, __LINE__);
    }
    for (int i = 0; i < iters && !rc; i++) rc = launch(i);
    if (!rc) {
        hipError_t e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float f = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&f, e0, e1);
        if (e != hipSuccess) rc = hip_fail(e, "event timing", __FILE__, __LINE__);
        *avg_us = 1000.0 * f / iters;
    }
    if (bytes_per_launch) *bytes_per_launch = 2.0 * k * n + 4.0 * m_rows * k + 4.0 * m_rows * n;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    for (auto *w : W) dev_free(w);
    dev_free(x);
    dev_free(y);
    return rc;
}

int scry_hip_bench_qgemv_bias(int m_rows, int k, int n, int n_bufs, int warmup, int iters, double *avg_us,
                              double *bytes_per_launch) {
    API_LOCK;
    return bench_qgemv_impl(m_rows, k, n, SCRY_QUANT_PER_TENSOR, n_bufs, warmup, iters, true, avg_us,
                            bytes_per_launch);
}

}  // extern "C"
