// Internal declarations shared by the scry_hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/scry_hip.h"

namespace scry {

struct Ctx {
    bool init = false;
    bool bf16 = false;  // bf16 mode (init_gpu_bf16, cuda.rs:55-59)
    int device = -1;
    hipStream_t stream = nullptr;
    int cu_count = 0;
    std::string name, arch;
    void *ws = nullptr;  // op workspace on the stream (grown on demand, kept)
    size_t ws_bytes = 0;
};

Ctx &ctx();
// The context's workspace, at least `bytes` large.  Work already queued on
// the stream may still use the old one, so growing it synchronises first.
int ctx_workspace(size_t bytes, void **p);
std::recursive_mutex &api_mutex();

int set_error(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *expr, const char *file, int line);
int dev_alloc(void **p, size_t bytes);
void dev_free(void *p);

#define SCRY_HIP(expr)                                                          \
    do {                                                                        \
        hipError_t _e = (expr);                                                 \
        if (_e != hipSuccess) return ::scry::hip_fail(_e, #expr, __FILE__, __LINE__); \
    } while (0)

#define SCRY_TRY(expr)                 \
    do {                               \
        int _rc = (expr);              \
        if (_rc != SCRY_OK) return _rc; \
    } while (0)

#define SCRY_REQUIRE_INIT()                                                          \
    do {                                                                             \
        if (!::scry::ctx().init) return ::scry::set_error(SCRY_ERR_NOT_INIT, "scry_hip_init not called"); \
    } while (0)

// ---------------------------------------------------------------- weights
// GEMV stream layout of an int8 weight W[k,n] (k = in, n = out):
// one row per output index, each row `kp` bytes (k rounded up to 16), byte =
// q XOR 0x80 (= q + 128 as an unsigned byte), padding bytes 0x80 (q = 0).
// A fused gate/up pair interleaves rows in groups of four:
// gate[2t], gate[2t+1], up[2t], up[2t+1].
// bf16 weights (a bf16-mode model) use the same rows of bf16 values (the
// reference's cast of the f32 weight), kp = 2 * (k rounded up to 8) bytes,
// padding 0.
struct Packed {
    uint8_t *d = nullptr;
    int k = 0;         // logical in-dimension
    int n = 0;         // logical out-dimension (per tensor)
    int kp = 0;        // row stride in bytes
    int rows = 0;      // packed rows (n, or 2n when fused)
    int fused = 0;     // 1 = gate/up interleave
    float scale = 0.f; // per-tensor scale (gate scale when fused)
    float scale2 = 0.f;// up scale when fused
    float *s32 = nullptr; // block-32 scales [rows][nb] (packed-row order) or nullptr
    int nb = 0;
    int bf16 = 0;         // 1: rows of bf16 values (no scales)
    size_t bytes() const { return (size_t)rows * kp; }
};

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

void packed_free(Packed &p);

// ---------------------------------------------------------------- kernels
// quant.hip
int launch_absmax(const float *w, size_t n, unsigned int *d_absmax_bits, hipStream_t s);
int launch_quantize_plain(const float *w, size_t n, const unsigned int *d_absmax_bits, int8_t *q,
                          float *d_scale, hipStream_t s);
// Quantize (per tensor, from the absmax bits) and pack a f32 tensor in one pass.
// src_nk = 1 when the source is stored [n,k] (embedding / lm_head).
// Row mapping for output j: row = (j / grp) * stride + off + (j % grp).
int launch_quant_pack(const float *w, int k, int n, int src_nk, const unsigned int *d_absmax_bits,
                      uint8_t *dst, int kp, int grp, int stride, int off, hipStream_t s);
int launch_i8_pack(const int8_t *q, int k, int n, int src_nk, uint8_t *dst, int kp, int grp,
                   int stride, int off, hipStream_t s);
int launch_unpack(const uint8_t *src, int kp, int k, int n, int dst_nk, int grp, int stride, int off,
                  int8_t *q, hipStream_t s);
int launch_quant_block32(const float *w, int k, int n, int src_nk, int8_t *q, float *scales,
                         hipStream_t s);
// scales [n][nb] (logical) -> packed-row order
int launch_scales_pack(const float *scales, int n, int nb, float *dst, int grp, int stride, int off,
                       hipStream_t s);
int launch_dequantize(const int8_t *q, size_t n, float scale, float *out, hipStream_t s);
int launch_normal_init(float *out, size_t n, uint64_t seed, uint64_t start_call, float mean,
                       float stdv, int cols, int ld, int col0, hipStream_t s);

// qgemv.hip
enum GemvEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3, EPI_LOGITS = 4 };

struct DevState {  // per decode session, device resident
    int pos;        // RoPE position of the token being processed
    int cache_len;  // rows already in the KV cache (the new row is written here)
    int n_prompt;   // prompt length (tokens beyond it are generated)
    int max_tokens; // capacity of the token array minus one
};

struct GemvArgs {
    const Packed *w = nullptr;
    // activation rows: x (m rows, stride ldx); x == nullptr reads the embedding
    // row of tokens[state->pos] instead (embedding fused into the prologue)
    const float *x = nullptr;
    int ldx = 0;
    int m = 1;
    const float *embed = nullptr;
    const int64_t *tokens = nullptr;
    DevState *state = nullptr;
    const float *norm_w = nullptr;  // RMSNorm weight -> fused RMSNorm prologue
    float eps = 1e-5f;
    // pre-scaled RMSNorm input: x holds x*g, and the residual GEMV that wrote
    // it left n_ss per-workgroup partial sums of x^2 (x itself, f32) in ss_in
    const float *ss_in = nullptr;
    int n_ss = 0;
    // outputs
    float *y = nullptr;
    int ldy = 0;
    const float *resid = nullptr;   // EPI_RESID source (may alias y); nullptr -> embed row
    const float *bias = nullptr;    // EPI_STORE optional bias
    // EPI_RESID, for the next RMSNorm'd GEMV: y*g_next and per-workgroup
    // sums of y^2 (qgemv_blocks entries)
    float *xg_out = nullptr;
    const float *g_next = nullptr;
    float *ss_out = nullptr;
    // EPI_QKV
    float *q_out = nullptr, *k_cache = nullptr, *v_cache = nullptr;
    const float2 *rope_cs = nullptr;  // [max_pos][head_dim/2] (cos, sin)
    int q_dim = 0, kv_dim = 0, head_dim = 0;
    float q_scale = 1.f;
    // EPI_LOGITS: per-workgroup argmax partials (reduced by launch_logits_finish,
    // which also records the token and advances the step state)
    float *part_val = nullptr;
    int *part_idx = nullptr, *part_nan = nullptr;
    int64_t *tokens_rw = nullptr;
    int64_t *argmax_out = nullptr;
    int advance = 0;
    unsigned long long *ts = nullptr;  // step profile: per-workgroup start / end stamps (null: off)
};

int launch_qgemv(int epi, const GemvArgs &a, hipStream_t s);
// Whether decode steps replay their captured graphs (llama.hip).
bool graph_replay();
// workgroups of one launch_qgemv launch (= EPI_LOGITS argmax partials, EPI_RESID
// sum-of-squares partials)
int qgemv_blocks(int epi, const Packed &w, int m);
// matmul_i8_f32 with more activation rows than this runs as the MFMA GEMM
constexpr int GEMV_MAX_M = 16;
// skinny.hip: matmul_i8_f32 for SKINNY_MIN_M..16 activation rows on the matrix
// cores (k splits into a workspace of partial sums, then an ordered reduction)
constexpr int SKINNY_MIN_M = 3;  // measured: the GEMV (two rows per weight pass) is faster at 2
struct SkinnyMM {
    const Packed *w = nullptr;  // int8 rows (not bf16): plain, or the fused gate/up pair with swiglu
    const float *x = nullptr;
    int ldx = 0, m = 0;
    const float *bias = nullptr;
    const float *resid = nullptr;  // y = resid + x W, resid rows at stride ldy (may alias y)
    int swiglu = 0;                // fused gate/up rows: y[r][j] = silu(gate_j) * up_j, j < w.n
    float *y = nullptr;
    int ldy = 0;
};
bool skinny_route(int m, int k, int n);
size_t skinny_ws_bytes(int m, int k, int n);  // n: packed weight rows (2 n for a fused pair)
// The fused form (the batched decode step's projections): the RMSNorm rides
// in the activation staging, and one workgroup per 128-column tile adds the
// k splits' partials in split order and applies the epilogue.
enum { SKE_NONE = 0, SKE_STORE = 1, SKE_RESID = 2, SKE_SWIGLU = 3, SKE_LOGITS = 4 };
struct DecodeSeqs;
struct AttnSeqs;
struct SkinnyFused {
    const Packed *w = nullptr;
    const float *x = nullptr;
    int ldx = 0, m = 0;
    // RMSNorm of x (rmsnorm.rs), applied as rstd * (W (x * g)); rstd from the
    // per-row partial sums of squares of x [m][n_ss_in] (f64, 1..64 of them)
    const float *norm_w = nullptr;
    const double *ss_in = nullptr;
    int n_ss_in = 0;
    float eps = 1e-5f;
    int epi = SKE_STORE;  // NONE (the split partials only), STORE, RESID (y += x W), SWIGLU (fused gate/up rows), LOGITS
    float *y = nullptr;
    int ldy = 0;
    double *ss_out = nullptr;  // RESID (may be null): [m][skinny_tiles(w)] partial sums of squares of y
    float *pv = nullptr;       // LOGITS: [m][skinny_tiles(w)] ordered argmax partials
    int *pi = nullptr, *pn = nullptr;
};
int skinny_tiles(const Packed &w);  // 128-row tiles of the packed rows
// SKE_NONE: the split partials of rows [m] in ws as part[n_split][16][n_pad];
// y[i][j] = scale * (sum over the splits of part[s][i][j], in split order)
// (times the row's RMSNorm scale under norm_w)
struct SkinnyParts {
    int n_split = 0, n_pad = 0;
    float scale = 1.f;
};
int launch_skinny_fused(const SkinnyFused &f, float *ws, size_t ws_bytes, hipStream_t s,
                        SkinnyParts *parts = nullptr);
int launch_skinny(const SkinnyMM &mm, float *ws, size_t ws_bytes, hipStream_t s);
int launch_logits_finish(const GemvArgs &a, hipStream_t s);
// sample_token on the device (sample.hip): logits [V] -> tokens[pos + 1] when
// the position draws a token, then the position advances.  ws: [V] f64
// scratch; rng: the wyrand state.
// prep: sample_prep_bytes(V) zeroed bytes when sample_uses_prep (top-k off and
// a large vocabulary: statistics and exp values over all CUs first)
bool sample_uses_prep(const scry_sampling_config &sc, int V);
size_t sample_prep_bytes(int V);
int launch_sample(const float *logits, int V, const scry_sampling_config &sc, double *ws,
                  unsigned long long *rng, DevState *st, int64_t *tokens, void *prep, hipStream_t s);

// noalloc.hip: with `device` current, look up the device address of the
// static scratch of scry_hip_sample_token_noalloc (once per device)
int noalloc_setup(int device);

// safetensors.hip: memory-mapped safetensors shards and the device dtype
// widening of the checkpoint loader
enum { ST_OTHER = 0, ST_F32 = 1, ST_BF16 = 2, ST_F16 = 3 };
struct StTensor {
    std::string name, dtype_name;
    int dtype = ST_OTHER;
    std::vector<int64_t> shape;
    size_t numel = 0, bytes = 0;
    const uint8_t *data = nullptr;  // inside the mapping
};
struct StShards;
int st_open(const char *const *paths, int n_paths, StShards **out);
void st_close(StShards *sh);
const StTensor *st_find(const StShards *sh, const char *name);  // nullptr if absent
int launch_widen(const void *src, int dtype, size_t n, float *dst, hipStream_t s);

// attn.hip
// Per-group hand-over counters sit kCtrStride words apart: each on its own
// 256-byte block, so the atomics and polls of different groups do not queue
// on one cache line.
constexpr int kCtrStride = 64;

struct AttnArgs {
    const float *q = nullptr;     // [n_heads*hd] pre-scaled
    const float *k_cache = nullptr, *v_cache = nullptr;  // [max_seq, n_kv*hd]
    // per (head, split) partials and per-KV-group arrival counters (zero
    // between launches)
    float *part_o = nullptr, *part_ml = nullptr;
    unsigned *merge_ctr = nullptr;  // group g's counter at merge_ctr[g * kCtrStride]
    float *xa = nullptr;          // merged output [n_heads*hd]
    const DevState *state = nullptr;
    int n_heads = 0, n_kv = 0, head_dim = 0, n_splits = 1, max_chunk = 0;
    int fixed_len = -1;  // >= 0: use this length instead of state->cache_len + 1
    unsigned long long *ts = nullptr;  // step profile: per-workgroup start / end stamps (null: off)
};
int launch_attn_decode(const AttnArgs &a, hipStream_t s);
int attn_pick_splits(int n_kv, int max_seq, int *n_splits, int *max_chunk);

// glue.hip
int launch_rmsnorm(const float *x, const float *w, int rows, int d, float eps, float *out,
                   hipStream_t s);
int launch_rope(const float *x, int seq, int n_heads, int hd, int start_pos, const float *freqs,
                int scaled, float scale, float *out, hipStream_t s);
int launch_scale(const float *x, size_t n, float s_, float *out, hipStream_t s);
int launch_softmax(const float *x, int rows, int cols, float *out, hipStream_t s);
int launch_swiglu(const float *g, const float *u, size_t n, float *out, hipStream_t s);
int launch_add(const float *a, const float *b, size_t n, float *out, hipStream_t s);
int launch_add_bias_rows(float *c, const float *bias, int rows, int n, hipStream_t s);
int launch_embedding(const float *w, const int64_t *ids, int n_ids, int dim, float *out,
                     hipStream_t s);
int launch_gather_repeat_kv(const float *cache, int cached_len, int n_kv, int n_q, int hd,
                            float *out, hipStream_t s);
int launch_repeat_kv(const float *x, int n_kv, int n_q, int seq, int d_head, float *out,
                     hipStream_t s);
int launch_matmul_f32(const float *a, const float *b, int batch, int m, int k, int n, int ta,
                      int tb, float *c, hipStream_t s);
int launch_argmax(const float *x, int64_t n, int64_t *out, hipStream_t s);
int launch_fill_f32(float *p, size_t n, float v, hipStream_t s);
int launch_fill_u32(unsigned int *p, size_t n, unsigned int v, hipStream_t s);
// Rows of int8 LM-head logits whose RMSNorm'd input holds a non-finite value:
// the reference's per-column +-inf / NaN in place of the prefill GEMM's NaN row.
int launch_logits_nonfinite(const float *x, int ldx, int rows, const float *norm_w, float eps, const Packed &w,
                            float *y, int ldy, hipStream_t s);

// ops.hip -- the rest of the trait surface
int launch_layernorm(const float *x, const float *g, const float *b, int rows, int d, float eps, float *out,
                     float *mean, float *rstd, hipStream_t s);
int launch_gelu(const float *x, size_t n, float *out, hipStream_t s);
int sum_partials(size_t n);  // f64 partials launch_sum needs
int launch_sum(const float *x, size_t n, double *part, float *out, hipStream_t s);
int launch_mul(const float *a, const float *b, size_t n, float *out, hipStream_t s);
int launch_rope_row(const float *x, size_t rows, int last_dim, int head_dim, const float2 *cs, float *out,
                    hipStream_t s);
int launch_gather_cols(const float *x, size_t rows, int total, int start, int count, float *out, hipStream_t s);
int launch_scatter_cols_add(float *dst, const float *src, size_t rows, int total, int start, int count,
                            hipStream_t s);
int launch_add_bcast(const float *a, const size_t *a_dims, int a_ndim, const float *b, const size_t *b_dims,
                     int b_ndim, const size_t *o_dims, int o_ndim, float *out, hipStream_t s);
int launch_add_inplace(float *d, const float *src, size_t n, hipStream_t s);
int launch_scaled_softmax(const float *x, int rows, int cols, float scale, float *out, hipStream_t s);
int launch_causal_mask(float *sc, size_t n_mat, int seq, float scale, float mask_value, hipStream_t s);
int launch_split_qkv(const float *qkv, int seq, int n_heads, int d_head, float *q, float *k, float *v,
                     hipStream_t s);
int launch_reshape_heads(const float *x, int batch, int seq, int n_heads, int d_head, int dir, float *out,
                         hipStream_t s);

// prefill.hip -- batched prefill (GEMMs on the matrix cores)
constexpr int PF_MAX_SEQS = 16;
struct PrefillSeqs {  // per sequence: its KV cache and first position
    float *k[PF_MAX_SEQS], *v[PF_MAX_SEQS];  // layer-0 K / V rows [max_seq][kv_dim]
    size_t ls[PF_MAX_SEQS];                  // floats from one layer's K (V) to the next
    const float2 *rope[PF_MAX_SEQS];         // (cos, sin) [max_seq][hd/2]
    int p0[PF_MAX_SEQS];
};
// Batched decode attention: one query row per sequence, each against its own
// cache (rows [0, pos[y]] of layer `layer`).  With it, the AttnArgs q, xa,
// part_o, part_ml and merge_ctr hold n consecutive per-sequence blocks
// ([q_dim], [q_dim], [n_heads][n_splits][hd], [n_heads][n_splits][2], [n_kv]);
// k_cache, v_cache, state and fixed_len are unused.
struct AttnSeqs {
    float *k[PF_MAX_SEQS], *v[PF_MAX_SEQS];        // layer-0 K / V rows of each cache
    size_t ls[PF_MAX_SEQS];                        // floats from one layer's K (V) to the next
    const int *pos;                                // device [n]: rows cached before this token
    int layer, n;
};
// The batched decode step's qkv epilogue, done by the attention launch: the
// qkv rows' split partials (SKE_NONE, row = the sequence) are summed in split
// order and scaled (scale, then the row's RMSNorm rstd from ss_in [n][n_ss_in]
// over k); each workgroup rotates its group's query heads (RoPE on adjacent
// pairs at the sequence's position, llama.rs:384-396) and multiplies them by
// q_scale, and the workgroup whose split holds the position rotates k and
// writes k and v into that row of the cache.  The arithmetic is the fused
// STORE epilogue's, so q, k and v are the same values.
struct QkvPro {
    const float *part = nullptr;
    int n_split = 0, n_pad = 0;
    float scale = 1.f;
    const double *ss_in = nullptr;
    int n_ss_in = 0, k = 0;
    float eps = 0.f, q_scale = 1.f;
    const float2 *rope[PF_MAX_SEQS] = {};
};
int launch_attn_decode_seqs(const AttnArgs &a, const AttnSeqs &b, hipStream_t s, const QkvPro *pro = nullptr);

// batch.hip -- glue of the batched decode step (n sequences, one token each)
struct DecodeSeqs {
    int64_t *tokens[PF_MAX_SEQS];     // each sequence's tokens: position p holds tokens[p]
    const float2 *rope[PF_MAX_SEQS];  // each cache's (cos, sin) [max_seq][hd/2]
    int *pos;                         // device [n]: the position being processed (= rows cached)
    int n;
};
// x [n][h] = the embedding rows of the current tokens; ss [n][ceil(h / 128)]
// their partial sums of squares (f64) for the first RMSNorm
int launch_bd_embed(const float *embed, int h, const DecodeSeqs &d, float *x, double *ss, hipStream_t s);
// ordered argmax of logits [n][V] per sequence (from the np per-row argmax
// partials of the LM head's fused skinny launch) -> tokens[pos + 1]; pos += 1
int launch_bd_argmax(const float *logits, int V, const float *pv, const int *pi, const int *pn, int np,
                     const DecodeSeqs &d, hipStream_t s);

// bf16 hi / lo planes of the K and V rows a prefill attends over, per
// (sequence, KV head): [n_seq][n_kv][rows][hd] each (hi = bf16(x), lo =
// bf16(x - hi)); null kh: the attention reads the f32 cache instead.
struct PrefillKVP {
    unsigned short *kh = nullptr, *kl = nullptr, *vh = nullptr, *vl = nullptr;
    int rows = 0;
};
struct PrefillGemm {
    const Packed *w = nullptr;
    const unsigned short *ahi = nullptr, *alo = nullptr;  // bf16 planes [Mp][lda], lda >= prefill_k_pad(k)
    int lda = 0, M = 0;
    float *c = nullptr;  // PF_STORE / PF_RESID output [M][ldc]
    int ldc = 0;
    const float *bias = nullptr;  // PF_STORE: + bias[n]
    unsigned short *ohi = nullptr, *olo = nullptr;  // GE_SWIGLU output planes
    int ldo = 0, opad = 0;
    // instead of ahi / alo (int8 per-tensor weights only): the activations as
    // 24-bit integers X 2^-E per row, in three balanced int8 digit planes
    // [3][Mp][lda] (plane stride dstride bytes) and the row exponents E [Mp]
    const signed char *ad = nullptr;
    const int *ae = nullptr;
    size_t dstride = 0;
    float *of = nullptr;  // GE_SWIGLU with digit planes: f32 output rows [M][ldo] instead of ohi / olo
};
struct PrefillAttn {
    const float *qkv = nullptr;  // rows [M][ldq], q part RoPE'd
    int ldq = 0, seq = 0, hd = 0, nh = 0, nkv = 0, kvd = 0;
    float scale = 1.f;
    unsigned short *ohi = nullptr, *olo = nullptr;  // o_proj input planes
    int ldo = 0, opad = 0;
    int nqb = 0, nseq = 0;  // set by the launcher: query blocks per sequence, sequences
    float *of = nullptr;    // instead of the planes: f32 rows [M][ldo] (the bf16 matrix-core kernel only)
};
enum { PF_STORE = 0, PF_RESID = 1, PF_SWIGLU = 2 };
int prefill_rows_pad(int M);  // GEMM input plane rows for M activation rows
int prefill_k_pad(int k);     // GEMM input plane columns (and zero padding) for k
int launch_norm_split(const float *x, int ldx, int rows, int rstep, int roff, const float *w, int k, float eps,
                      unsigned short *hi, unsigned short *lo, int ldp, float *outf, int ldf, hipStream_t s);
// RMSNorm (w non-null; the rows as they are for w null) into the digit
// planes of a PrefillGemm (rows r of [3][.][ldp] at plane stride dstride
// bytes; columns [k, prefill_k_pad(k)) zero) and the row exponents e[r]
int launch_norm_digits(const float *x, int ldx, int rows, const float *w, int k, float eps, signed char *dg,
                       size_t dstride, int *e, int ldp, hipStream_t s);
// true when a GEMM over w takes digit planes (int8 per-tensor weights)
bool gemm_takes_digits(const Packed &w);
int launch_split(const float *x, int ldx, int rows, int k, unsigned short *hi, unsigned short *lo, int ldp,
                 hipStream_t s);
int launch_gemm(int epi, const PrefillGemm &g, hipStream_t s);
// RoPE + K/V cache append; with kp.kh also the planes of the new K / V rows
// (and of the rows [0, p0) already in the caches)
int launch_rope_kv(float *qkv, int ldq, int M, int seq, int qd, int kvd, int hd, const PrefillSeqs &t, int l,
                   const PrefillKVP &kp, int n_seq, hipStream_t s);
bool attn_prefill_planes(int hd);  // head sizes the bf16 plane attention takes
int launch_attn_prefill(const PrefillAttn &a, int n_seq, const PrefillSeqs &t, int l, const PrefillKVP &kv,
                        hipStream_t s);

// bf16.hip -- bf16 mode: the reference's cast, widening, B-operand rows
// [n][kp] (kp = bf16_row_pad(k)), the GEMM activation plane, the bf16 GEMV
int bf16_row_pad(int k);
// a model's f32 weight as bf16 GEMV rows (row mapping as launch_quant_pack; kpe values per row)
int launch_pack_model_bf16(const float *w, int k, int n, int src_nk, unsigned short *dst, int kpe, int grp,
                           int stride, int off, hipStream_t s);
int launch_cast_bf16(const float *x, size_t n, unsigned short *y, hipStream_t s);
int launch_round_bf16(const float *x, size_t n, float *y, hipStream_t s);
int launch_widen_bf16(const unsigned short *x, size_t n, float *y, hipStream_t s);
int launch_embed_bf16(float *out, const unsigned short *w, const int64_t *ids, int n_ids, int dim, hipStream_t s);
int launch_pack_rows_bf16(const unsigned short *bs, const float *fs, int k, int n, int tb, unsigned short *pk,
                          int kp, hipStream_t s);
int launch_plane_bf16(const float *x, int ldx, int rows, int k, int kpad, unsigned short *hi, int ldp,
                      hipStream_t s);
int launch_gemv_bf16(const unsigned short *w, int kp, int n, const float *x, int ldx, int k, int m, float *y,
                     int ldy, const float *bias, hipStream_t s);
// prefill.hip: the MFMA GEMM over bf16 weight rows [N][kp] and one bf16 plane
int launch_gemm_bf16(const unsigned short *w, int kp, int N, int k, const unsigned short *ahi, int lda, int M,
                     float *c, int ldc, const float *bias, hipStream_t s);

// init.cpp -- host restatement of LlamaModel::new's random init (threaded)
void host_normal_vec(uint64_t seed, uint64_t start_call, size_t n, float mean, float stdv,
                     float *out, int threads);
int host_threads();

}  // namespace scry

struct scry_buf_s {
    float *d = nullptr;  // f32 data; null when the storage holds bf16 only (bf16 mode)
    size_t n = 0;
    // bf16 mode: the bf16 data of from_vec_with_bf16, or the f32 data rounded
    // once for a matmul (cleared when the f32 data is written in place)
    unsigned short *bf = nullptr;
    // bf16 rows [pk_n][pk_kp] of this storage as a matmul B operand for
    // logical (pk_k, pk_n, pk_tb), built on first use
    unsigned short *pk = nullptr;
    int pk_k = 0, pk_n = 0, pk_kp = 0, pk_tb = -1;
};

struct scry_i8buf_s {
    int8_t *d = nullptr;   // reference layout bytes
    size_t n = 0;
    scry::Packed packed;   // GEMV layout, built on first matmul for (k, n)
};
