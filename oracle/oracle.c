/*
 * CPU oracle (TEST INFRASTRUCTURE ONLY) -- plain-C restatement of scry-llm's
 * CPU path for the int8 Llama forward.  See oracle.h for the contract.
 *
 * Build: oracle/build.sh (gcc -O2 -ffp-contract=off -fno-fast-math -fopenmp).
 * Rust on x86_64-linux-gnu evaluates f32/f64 with SSE (no excess precision),
 * never contracts a*b+c into an FMA, and calls glibc libm for ln/cos/sin/
 * powf/exp/expf; this file does the same, so the arithmetic below is the
 * arithmetic of the cited reference lines.
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *   quantize_symmetric   reference KATs quantize.rs:46-83, round-half-away cases,
 *                        closed form, NaN/inf handling (pinned)
 *   quantize_block32     = quantize_symmetric on each block (pinned by A1)
 *   matmul_i8_f32        cpu.rs:1699-1756 tolerance tests, brute-force f64 dot,
 *                        exact-integer cases, tiled == parallel bit-identity (pinned)
 *   gemv / matmul f32    cpu.rs:1476-1481 identity, brute force, summation-order
 *                        cases that distinguish the 4-way unrolled order (pinned)
 *   rmsnorm              cpu.rs:1500-1511 closed form (pinned)
 *   rope                 cpu.rs:1538-1548 cos 1 / sin 1, textbook rotation (pinned)
 *   softmax, silu        cpu.rs:1483-1492, 1513-1522 (pinned)
 *   repeat_kv / gather   cpu.rs:1524-1536, 1662-1697 exact (pinned)
 *   argmax               generate.rs:167-173 Iterator::max_by semantics (pinned)
 *   rope freqs           closed form 1/theta^(2i/hd), Llama-3 scaling cases (pinned)
 *   Llama decode/forward tests/llama_smoke.rs invariants: cache == full forward
 *                        (1e-3), greedy determinism, GQA ratios (pinned as
 *                        invariants; no reference logits exist)
 *   loaded norms         llama.rs:880-914, 936-940 (set_norm): a final-norm
 *                        weight of 2 doubles every logit exactly (pinned)
 *   fastrand / Box-Muller parity UNPINNED: no reference test fixes any value
 *                        of the fastrand 2.3.0 stream.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;

void orc_set_threads(int n) { g_threads = n < 0 ? 0 : n; }
int orc_get_threads(void) { return g_threads; }

#define NT (g_threads > 0 ? g_threads : 1)
#define PAR_IF (g_threads > 1)

/* ------------------------------------------------------------------------
 * fastrand 2.3.0 (not vendored in the reference; pinned in Cargo.lock).
 * Published algorithm (wyrand): state += 0x2d358dccaa6c78a5;
 * t = (u128)state * (state ^ 0x8bb84b93962eacc9); out = lo(t) ^ hi(t).
 * Rng::with_seed(s) sets state = s.  f64() = from_bits(0x3FF0<<48 | u>>12) - 1.
 * Call sites: init.rs:3-4, llama.rs:593.  Parity unpinned.
 * ---------------------------------------------------------------------- */
#define WY0 0x2d358dccaa6c78a5ULL
#define WY1 0x8bb84b93962eacc9ULL

static inline uint64_t wy_mix(uint64_t s) {
    unsigned __int128 t = (unsigned __int128)s * (unsigned __int128)(s ^ WY1);
    return (uint64_t)t ^ (uint64_t)(t >> 64);
}

static inline double wy_f64(uint64_t u) {
    uint64_t bits = 0x3FF0000000000000ULL | (u >> 12);
    double d;
    memcpy(&d, &bits, sizeof d);
    return d - 1.0;
}

uint64_t orc_rng_u64_at(uint64_t seed, uint64_t call_index) {
    return wy_mix(seed + (call_index + 1) * WY0);
}

void orc_rng_fill_u64(uint64_t seed, uint64_t start_call, size_t n, uint64_t *out) {
    uint64_t s = seed + start_call * WY0;
    for (size_t i = 0; i < n; i++) {
        s += WY0;
        out[i] = wy_mix(s);
    }
}

void orc_rng_fill_f64(uint64_t seed, uint64_t start_call, size_t n, double *out) {
    uint64_t s = seed + start_call * WY0;
    for (size_t i = 0; i < n; i++) {
        s += WY0;
        out[i] = wy_f64(wy_mix(s));
    }
}

/* init.rs:2-9 normal_sample: Box-Muller on two consecutive f64 draws. */
static inline float normal_from(double u1, double u2, float mean, float stdv) {
    if (u1 < 1e-30) u1 = 1e-30;
    double z = sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
    return (float)((double)mean + (double)stdv * z);
}

/* init.rs:12-14 normal_vec, sequential state walk. */
void orc_normal_vec(uint64_t seed, uint64_t start_call, size_t n, float mean, float stdv,
                    float *out) {
    uint64_t s = seed + start_call * WY0;
    for (size_t i = 0; i < n; i++) {
        s += WY0;
        double u1 = wy_f64(wy_mix(s));
        s += WY0;
        double u2 = wy_f64(wy_mix(s));
        out[i] = normal_from(u1, u2, mean, stdv);
    }
}

/* Same values: wyrand's state is additive, so call c has state seed+(c+1)*WY0. */
void orc_normal_vec_par(uint64_t seed, uint64_t start_call, size_t n, float mean, float stdv,
                        float *out) {
    int64_t nn = (int64_t)n;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF)
    for (int64_t i = 0; i < nn; i++) {
        uint64_t c = start_call + 2 * (uint64_t)i;
        double u1 = wy_f64(wy_mix(seed + (c + 1) * WY0));
        double u2 = wy_f64(wy_mix(seed + (c + 2) * WY0));
        out[i] = normal_from(u1, u2, mean, stdv);
    }
}

/* ------------------------------------------------------------------------
 * quantize.rs:16-32 quantize_symmetric.  absmax folds with f32::max (NaN is
 * ignored, as fmaxf does); scale = absmax/127; inv = 1/scale; q = round(w*inv)
 * (half away from zero = roundf) clamped to [-127,127]; `as i8` maps NaN to 0.
 * ---------------------------------------------------------------------- */
static inline int8_t quant_one(float w, float inv) {
    float r = roundf(w * inv);
    if (isnan(r)) return 0;
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

void orc_quantize_symmetric(const float *w, size_t n, int8_t *q, float *scale) {
    float absmax = 0.0f;
    for (size_t i = 0; i < n; i++) absmax = fmaxf(absmax, fabsf(w[i]));
    if (absmax == 0.0f) {
        memset(q, 0, n);
        *scale = 0.0f;
        return;
    }
    float s = absmax / 127.0f;
    float inv = 1.0f / s;
    int64_t nn = (int64_t)n;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF && nn > (1 << 20))
    for (int64_t i = 0; i < nn; i++) q[i] = quant_one(w[i], inv);
    *scale = s;
}

/* quantize.rs:35-40 dequantize: f32::from(q) * scale */
void orc_dequantize(const int8_t *q, size_t n, float scale, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = (float)q[i] * scale;
}

/* Builder-defined block-32 extension (no reference counterpart): for each
 * output column j of W[k,n] and each k-block b, quantize_symmetric on
 * W[32b .. min(32b+32,k), j]; scales[j*nb + b]. */
void orc_quantize_block32(const float *w, int k, int n, int8_t *q, float *scales) {
    int nb = (k + 31) / 32;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF)
    for (int j = 0; j < n; j++) {
        float buf[32];
        int8_t qb[32];
        for (int b = 0; b < nb; b++) {
            int p0 = 32 * b, len = (k - p0) < 32 ? (k - p0) : 32;
            for (int t = 0; t < len; t++) buf[t] = w[(size_t)(p0 + t) * n + j];
            orc_quantize_symmetric(buf, (size_t)len, qb, &scales[(size_t)j * nb + b]);
            for (int t = 0; t < len; t++) q[(size_t)(p0 + t) * n + j] = qb[t];
        }
    }
}

/* ------------------------------------------------------------------------
 * cpu.rs:1128-1160 matmul_i8_f32_tiled, as written (single-threaded).
 * Per element: c += (f64(a) * (f64(q) * f64(scale))) as f32, p increasing.
 * ---------------------------------------------------------------------- */
void orc_matmul_i8_f32_tiled(const float *a, const int8_t *bq, float scale, int m, int k, int n,
                             float *c) {
    const int T = 32;
    double sd = (double)scale;
    memset(c, 0, sizeof(float) * (size_t)m * n);
    for (int it = 0; it < m; it += T) {
        int ie = it + T < m ? it + T : m;
        for (int pt = 0; pt < k; pt += T) {
            int pe = pt + T < k ? pt + T : k;
            for (int jt = 0; jt < n; jt += T) {
                int je = jt + T < n ? jt + T : n;
                for (int i = it; i < ie; i++) {
                    for (int p = pt; p < pe; p++) {
                        double av = (double)a[(size_t)i * k + p];
                        for (int j = jt; j < je; j++) {
                            double bv = (double)bq[(size_t)p * n + j] * sd;
                            c[(size_t)i * n + j] += (float)(av * bv);
                        }
                    }
                }
            }
        }
    }
}

/* Bit-identical column-parallel variant: the per-element operation sequence
 * (p increasing, same f64 product, same f32 add) is unchanged. */
void orc_matmul_i8_f32_par(const float *a, const int8_t *bq, float scale, int m, int k, int n,
                           float *c) {
    if (g_threads <= 0) {
        orc_matmul_i8_f32_tiled(a, bq, scale, m, k, n, c);
        return;
    }
    double sd = (double)scale;
    const int CH = 512;
    int nch = (n + CH - 1) / CH;
#pragma omp parallel for schedule(dynamic, 1) num_threads(NT) if (PAR_IF)
    for (int ch = 0; ch < nch; ch++) {
        int j0 = ch * CH, j1 = j0 + CH < n ? j0 + CH : n;
        for (int i = 0; i < m; i++) {
            float *cr = c + (size_t)i * n;
            for (int j = j0; j < j1; j++) cr[j] = 0.0f;
            for (int p = 0; p < k; p++) {
                double av = (double)a[(size_t)i * k + p];
                const int8_t *qr = bq + (size_t)p * n;
                for (int j = j0; j < j1; j++) cr[j] += (float)(av * ((double)qr[j] * sd));
            }
        }
    }
}

/* The same per-element formula over an int8 matrix stored [n,k] (the LM head,
 * which the reference multiplies with trans_b = true, llama.rs:761-762). */
void orc_matmul_i8_f32_tb(const float *a, const int8_t *bq_nk, float scale, int m, int k, int n,
                          float *c) {
    double sd = (double)scale;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF)
    for (int j = 0; j < n; j++) {
        const int8_t *qr = bq_nk + (size_t)j * k;
        for (int i = 0; i < m; i++) {
            const float *ar = a + (size_t)i * k;
            float acc = 0.0f;
            for (int p = 0; p < k; p++) acc += (float)((double)ar[p] * ((double)qr[p] * sd));
            c[(size_t)i * n + j] = acc;
        }
    }
}

/* Block-32 variant of the same formula (builder-defined). */
void orc_matmul_i8_f32_b32(const float *a, const int8_t *bq, const float *scales, int m, int k,
                           int n, float *c) {
    int nb = (k + 31) / 32;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF)
    for (int j = 0; j < n; j++) {
        for (int i = 0; i < m; i++) {
            float acc = 0.0f;
            for (int p = 0; p < k; p++) {
                double sd = (double)scales[(size_t)j * nb + p / 32];
                acc += (float)((double)a[(size_t)i * k + p] * ((double)bq[(size_t)p * n + j] * sd));
            }
            c[(size_t)i * n + j] = acc;
        }
    }
}

/* cpu.rs:553-570 matmul_i8_f32_bias: tiled result, then += bias[col] in f32. */
void orc_matmul_i8_f32_bias(const float *a, const int8_t *bq, float scale, const float *bias,
                            int m, int k, int n, float *c) {
    orc_matmul_i8_f32_par(a, bq, scale, m, k, n, c);
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) c[(size_t)i * n + j] += bias[j];
}

/* ------------------------------------------------------------------------
 * f32 GEMV family, cpu.rs:748-871.
 * ---------------------------------------------------------------------- */
/* cpu.rs:748-811 gemv_f32 (the rayon path at n >= 8192 splits columns only,
 * so the per-element arithmetic is the sequential path's). */
void orc_gemv_f32(const float *vec, const float *mat, int k, int n, float *out) {
    int k4 = k & ~3;
    const int CH = 4096;
    int nch = (n + CH - 1) / CH;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF && n >= 8192)
    for (int ch = 0; ch < nch; ch++) {
        int j0 = ch * CH, j1 = j0 + CH < n ? j0 + CH : n;
        for (int j = j0; j < j1; j++) out[j] = 0.0f;
        for (int p = 0; p < k4; p += 4) {
            float v0 = vec[p], v1 = vec[p + 1], v2 = vec[p + 2], v3 = vec[p + 3];
            const float *r0 = mat + (size_t)p * n, *r1 = r0 + n, *r2 = r1 + n, *r3 = r2 + n;
            for (int j = j0; j < j1; j++) out[j] += v0 * r0[j] + v1 * r1[j] + v2 * r2[j] + v3 * r3[j];
        }
        for (int p = k4; p < k; p++) {
            float v = vec[p];
            const float *r = mat + (size_t)p * n;
            for (int j = j0; j < j1; j++) out[j] += v * r[j];
        }
    }
}

/* cpu.rs:825-842 gemv_trans_b_into: 4 strided partials, ((a0+a1)+a2)+a3, tail. */
void orc_gemv_trans_b(const float *vec, const float *mat_t, int k, int n, float *out) {
    int k4 = k & ~3;
    for (int j = 0; j < n; j++) {
        const float *row = mat_t + (size_t)j * k;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (int p = 0; p < k4; p += 4) {
            a0 += vec[p] * row[p];
            a1 += vec[p + 1] * row[p + 1];
            a2 += vec[p + 2] * row[p + 2];
            a3 += vec[p + 3] * row[p + 3];
        }
        float acc = a0 + a1 + a2 + a3;
        for (int p = k4; p < k; p++) acc += vec[p] * row[p];
        out[j] = acc;
    }
}

/* cpu.rs:846-871 gemv_into */
void orc_gemv_into(const float *vec, const float *mat, int k, int n, float *out) {
    for (int j = 0; j < n; j++) out[j] = 0.0f;
    int k4 = k & ~3;
    for (int p = 0; p < k4; p += 4) {
        float v0 = vec[p], v1 = vec[p + 1], v2 = vec[p + 2], v3 = vec[p + 3];
        const float *r0 = mat + (size_t)p * n, *r1 = r0 + n, *r2 = r1 + n, *r3 = r2 + n;
        for (int j = 0; j < n; j++) out[j] += v0 * r0[j] + v1 * r1[j] + v2 * r2[j] + v3 * r3[j];
    }
    for (int p = k4; p < k; p++) {
        float v = vec[p];
        const float *r = mat + (size_t)p * n;
        for (int j = 0; j < n; j++) out[j] += v * r[j];
    }
}

/* cpu.rs:875-999 matmul_tiled_fallback (no blas/mkl/dnnl): f64 accumulation
 * per element, p increasing, rounded once to f32. */
static void matmul_fallback(const float *a, const float *b, int m, int k, int n, int ta, int tb,
                            float *c) {
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF && m >= 128)
    for (int i = 0; i < m; i++) {
        double *acc = (double *)calloc((size_t)n, sizeof(double));
        for (int p = 0; p < k; p++) {
            double av = ta ? (double)a[(size_t)p * m + i] : (double)a[(size_t)i * k + p];
            for (int j = 0; j < n; j++) {
                double bv = tb ? (double)b[(size_t)j * k + p] : (double)b[(size_t)p * n + j];
                acc[j] += av * bv;
            }
        }
        for (int j = 0; j < n; j++) c[(size_t)i * n + j] = (float)acc[j];
        free(acc);
    }
}

/* cpu.rs:924-961 matmul_tiled dispatch: m == 1 && !trans_a -> GEMV. */
void orc_matmul_f32(const float *a, const float *b, int m, int k, int n, int trans_a,
                    int trans_b, float *c) {
    if (m == 1 && !trans_a) {
        if (trans_b)
            orc_gemv_trans_b(a, b, k, n, c);
        else
            orc_gemv_f32(a, b, k, n, c);
        return;
    }
    matmul_fallback(a, b, m, k, n, trans_a, trans_b, c);
}

/* kernels.rs:629-633 float_to_bf16 (the bf16 feature's cast): round to
 * nearest even by adding 0x7fff + the lowest kept bit to the f32 bits, in
 * 32-bit unsigned arithmetic (a NaN whose payload lies in the low 16 bits
 * becomes inf; the all-ones negative NaN wraps to +0). */
uint16_t orc_f32_to_bf16(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

void orc_f32_to_bf16_vec(const float *x, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(x[i]);
}

static float bf16_val(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* bf16_ops::matmul_bf16 (cuda.rs:1226-1290): C = bf16(A) bf16(B) with f32
 * accumulation in cuBLAS (order unspecified).  The restatement rounds both
 * operands with the cast above and sums the (exact) products in f64, rounded
 * once: the value any f32 accumulation approximates. */
void orc_matmul_bf16(const float *a, const float *b, int m, int k, int n, int trans_a, int trans_b,
                     float *c) {
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            double acc = 0.0;
            for (int p = 0; p < k; p++) {
                const float av = trans_a ? a[(size_t)p * m + i] : a[(size_t)i * k + p];
                const float bv = trans_b ? b[(size_t)j * k + p] : b[(size_t)p * n + j];
                acc += (double)bf16_val(orc_f32_to_bf16(av)) * (double)bf16_val(orc_f32_to_bf16(bv));
            }
            c[(size_t)i * n + j] = (float)acc;
        }
}

/* orc_matmul_bf16 (trans_a = 0) on all cores, bit-identical: the same f64
 * sum of exact bf16 products in increasing p, per output element. */
void orc_matmul_bf16_par(const float *a, const float *b, int m, int k, int n, int trans_b, float *c) {
    double *ab = (double *)malloc(sizeof(double) * (size_t)m * k);
    for (size_t i = 0; i < (size_t)m * k; i++) ab[i] = (double)bf16_val(orc_f32_to_bf16(a[i]));
    if (trans_b) {
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF)
        for (int j = 0; j < n; j++) {
            const float *row = b + (size_t)j * k;
            for (int i = 0; i < m; i++) {
                const double *ar = ab + (size_t)i * k;
                double acc = 0.0;
                for (int p = 0; p < k; p++) acc += ar[p] * (double)bf16_val(orc_f32_to_bf16(row[p]));
                c[(size_t)i * n + j] = (float)acc;
            }
        }
    } else {
        const int CH = 256, nch = (n + CH - 1) / CH;
#pragma omp parallel for schedule(dynamic, 1) num_threads(NT) if (PAR_IF)
        for (int ch = 0; ch < nch; ch++) {
            const int j0 = ch * CH, j1 = j0 + CH < n ? j0 + CH : n;
            double *acc = (double *)malloc(sizeof(double) * CH);
            for (int i = 0; i < m; i++) {
                const double *ar = ab + (size_t)i * k;
                for (int j = j0; j < j1; j++) acc[j - j0] = 0.0;
                for (int p = 0; p < k; p++) {
                    const float *br = b + (size_t)p * n;
                    for (int j = j0; j < j1; j++) acc[j - j0] += ar[p] * (double)bf16_val(orc_f32_to_bf16(br[j]));
                }
                for (int j = j0; j < j1; j++) c[(size_t)i * n + j] = (float)acc[j - j0];
            }
            free(acc);
        }
    }
    free(ab);
}

/* cpu.rs:1321-1350 (+ fallback 1444-1468) matmul_strided_batched_impl */
void orc_matmul_strided_batched(const float *a, const float *b, int batch, int m, int k, int n,
                                int trans_a, int trans_b, float *c) {
    size_t as = (size_t)m * k, bs = (size_t)k * n, cs = (size_t)m * n;
    if (m == 1 && !trans_a) {
        for (int i = 0; i < batch; i++) {
            if (trans_b)
                orc_gemv_trans_b(a + (size_t)i * k, b + i * bs, k, n, c + (size_t)i * n);
            else
                orc_gemv_into(a + (size_t)i * k, b + i * bs, k, n, c + (size_t)i * n);
        }
        return;
    }
    for (int i = 0; i < batch; i++)
        matmul_fallback(a + i * as, b + i * bs, m, k, n, trans_a, trans_b, c + i * cs);
}

/* ------------------------------------------------------------------------
 * Glue ops.
 * ---------------------------------------------------------------------- */
/* cpu.rs:574-599 rmsnorm: f64 mean of squares, rstd = 1/sqrt(ms + eps) in f64,
 * out = f32(f64(x) * rstd * f64(w)). */
void orc_rmsnorm(const float *x, const float *w, int rows, int d, float eps, float *out) {
    for (int i = 0; i < rows; i++) {
        const float *r = x + (size_t)i * d;
        double ms = 0.0;
        for (int j = 0; j < d; j++) ms += (double)r[j] * (double)r[j];
        ms = ms / (double)d;
        double rstd = 1.0 / sqrt(ms + (double)eps);
        for (int j = 0; j < d; j++) out[(size_t)i * d + j] = (float)((double)r[j] * rstd * (double)w[j]);
    }
}

/* cpu.rs:635-664 rope_with_freqs_preloaded: angle = f64(pos) * f64(freq_f32);
 * cos/sin in f64 rounded to f32; interleaved pairs (2i, 2i+1) rotated in f32. */
void orc_rope_with_freqs_preloaded(const float *x, int seq, int n_heads, int head_dim,
                                   int start_pos, const float *freqs, float *out) {
    int total = n_heads * head_dim;
    int npairs = head_dim / 2;
    memcpy(out, x, sizeof(float) * (size_t)seq * total);
    for (int s = 0; s < seq; s++) {
        double pos = (double)(start_pos + s);
        for (int h = 0; h < n_heads; h++) {
            size_t hs = (size_t)s * total + (size_t)h * head_dim;
            for (int i = 0; i < npairs; i++) {
                double ang = pos * (double)freqs[i];
                float cv = (float)cos(ang), sv = (float)sin(ang);
                float x0 = x[hs + 2 * i], x1 = x[hs + 2 * i + 1];
                out[hs + 2 * i] = x0 * cv - x1 * sv;
                out[hs + 2 * i + 1] = x0 * sv + x1 * cv;
            }
        }
    }
}

/* cpu.rs:509-511 scale */
void orc_scale(const float *x, size_t n, float s, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = x[i] * s;
}

/* cpu.rs:336-366 softmax: f32 max (NaN-ignoring), e = expf(x - max) kept as
 * f32, f64 sum, out = f32(f64(e) / sum). */
void orc_softmax(const float *x, int rows, int cols, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *in = x + (size_t)r * cols;
        float *o = out + (size_t)r * cols;
        float mx = -INFINITY;
        for (int i = 0; i < cols; i++) mx = fmaxf(mx, in[i]);
        double sum = 0.0;
        for (int i = 0; i < cols; i++) {
            double e = (double)expf(in[i] - mx);
            o[i] = (float)e;
            sum += e;
        }
        for (int i = 0; i < cols; i++) o[i] = (float)((double)o[i] / sum);
    }
}

/* cpu.rs:1119-1122 silu_scalar (all in f64, rounded once) */
float orc_silu(float x) {
    double x64 = (double)x;
    return (float)(x64 / (1.0 + exp(-x64)));
}

/* cpu.rs:666-678 swiglu: silu(g) * u in f32 */
void orc_swiglu(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_silu(gate[i]) * up[i];
}

/* cpu.rs:104-113 add (same-shape path) */
void orc_add(const float *a, const float *b, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* cpu.rs:485-498 embedding: row gather; the reference panics on an id >= vocab,
 * here -1 is returned and nothing is written. */
int orc_embedding(const float *weight, const int64_t *idx, int n_idx, int vocab, int dim,
                  float *out) {
    for (int i = 0; i < n_idx; i++)
        if (idx[i] < 0 || idx[i] >= vocab) return -1;
    for (int i = 0; i < n_idx; i++)
        memcpy(out + (size_t)i * dim, weight + (size_t)idx[i] * dim, sizeof(float) * (size_t)dim);
    return 0;
}

/* cpu.rs:680-705 repeat_kv */
void orc_repeat_kv(const float *x, int n_kv, int n_q, int seq, int d_head, float *out) {
    int n_rep = n_q / n_kv;
    size_t hs = (size_t)seq * d_head;
    for (int kh = 0; kh < n_kv; kh++)
        for (int r = 0; r < n_rep; r++)
            memcpy(out + (size_t)(kh * n_rep + r) * hs, x + (size_t)kh * hs, sizeof(float) * hs);
}

/* cpu.rs:707-730 gather_reshape_repeat_kv: cache [max_seq, n_kv*hd] ->
 * [n_q, cached_len, hd], kv_head = q_head / (n_q / n_kv). */
void orc_gather_reshape_repeat_kv(const float *cache, int max_seq, int cached_len, int n_kv,
                                  int n_q, int head_dim, float *out) {
    (void)max_seq;
    int n_rep = n_q / n_kv;
    int kv_dim = n_kv * head_dim;
    for (int qh = 0; qh < n_q; qh++) {
        int kh = qh / n_rep;
        for (int s = 0; s < cached_len; s++)
            memcpy(out + ((size_t)qh * cached_len + s) * head_dim,
                   cache + (size_t)s * kv_dim + (size_t)kh * head_dim, sizeof(float) * head_dim);
    }
}

/* backend/mod.rs:368-381 scatter_rows default: overwrite rows */
void orc_scatter_rows(float *dst, const float *src, int total_rows, int cols, int row_start,
                      int row_count) {
    (void)total_rows;
    memcpy(dst + (size_t)row_start * cols, src, sizeof(float) * (size_t)row_count * cols);
}

/* backend/mod.rs:595-621 apply_batched_causal_mask_and_scale default body */
void orc_causal_mask_scale(float *scores, int n_mat, int seq, float scale, float mask_value) {
    for (int m = 0; m < n_mat; m++) {
        float *d = scores + (size_t)m * seq * seq;
        for (int s = 0; s < seq; s++)
            for (int t = 0; t < seq; t++) {
                if (t > s)
                    d[(size_t)s * seq + t] = mask_value;
                else
                    d[(size_t)s * seq + t] *= scale;
            }
    }
}

/* generate.rs:167-173 argmax: Iterator::max_by(partial_cmp, NaN -> Equal).
 * max_by keeps the running element only when it compares Greater, so the
 * last of equal maxima wins and an unordered pair hands over to the later
 * element.  Empty input -> 0. */
int64_t orc_argmax(const float *logits, int64_t n) {
    if (n <= 0) return 0;
    int64_t best = 0;
    for (int64_t i = 1; i < n; i++) {
        if (!(logits[best] > logits[i])) best = i;
    }
    return best;
}

/* generate.rs:92-165 sample_token, with the fastrand restatement above as
 * the rng (Rng::f64 once per sampled token, in weighted_sample).
 *
 * The reference sorts with sort_unstable_by (descending), whose order among
 * equal values is unspecified.  Top-k only reads the k-th value, so ties do
 * not matter there; top-p keeps the first cutoff entries of that order, so
 * when the cutoff falls inside a run of equal probabilities the reference's
 * choice of indices is unspecified.  This restatement breaks ties by the
 * smaller index (a sort by (value desc, index asc)). */
typedef struct {
    double v;
    int64_t i;
} orc_vi;

static int vi_desc(const void *a, const void *b) {
    const orc_vi *x = (const orc_vi *)a, *y = (const orc_vi *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : (x->i > y->i);
}

int64_t orc_sample_token(const float *logits, int64_t n, float temperature, int64_t top_k, float top_p,
                         uint64_t *rng_state) {
    if (temperature < 1e-8f) return orc_argmax(logits, n); /* generate.rs:96-98 */
    double *sc = (double *)malloc(sizeof(double) * (size_t)n);
    for (int64_t i = 0; i < n; i++) sc[i] = (double)logits[i] / (double)temperature;
    orc_vi *ix = (orc_vi *)malloc(sizeof(orc_vi) * (size_t)n);
    if (top_k > 0 && top_k < n) { /* generate.rs:108-118 */
        for (int64_t i = 0; i < n; i++) ix[i] = (orc_vi){sc[i], i};
        qsort(ix, (size_t)n, sizeof(orc_vi), vi_desc);
        const double thr = ix[top_k - 1].v;
        for (int64_t i = 0; i < n; i++)
            if (sc[i] < thr) sc[i] = -INFINITY;
    }
    /* generate.rs:120-131: softmax in f64, uniform when the sum is not > 0 */
    double mx = -INFINITY;
    for (int64_t i = 0; i < n; i++) mx = fmax(mx, sc[i]);
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) {
        sc[i] = exp(sc[i] - mx);
        sum += sc[i];
    }
    if (sum > 0.0) {
        for (int64_t i = 0; i < n; i++) sc[i] /= sum;
    } else {
        const double u = 1.0 / (double)n;
        for (int64_t i = 0; i < n; i++) sc[i] = u;
    }
    if (top_p < 1.0f && top_p > 0.0f) { /* generate.rs:134-160 */
        for (int64_t i = 0; i < n; i++) ix[i] = (orc_vi){sc[i], i};
        qsort(ix, (size_t)n, sizeof(orc_vi), vi_desc);
        double cum = 0.0;
        int64_t cut = n;
        for (int64_t j = 0; j < n; j++) {
            cum += ix[j].v;
            if (cum >= (double)top_p) {
                cut = j + 1;
                break;
            }
        }
        unsigned char *keep = (unsigned char *)calloc((size_t)n, 1);
        for (int64_t j = 0; j < cut; j++) keep[ix[j].i] = 1;
        for (int64_t i = 0; i < n; i++)
            if (!keep[i]) sc[i] = 0.0;
        free(keep);
        double sum2 = 0.0;
        for (int64_t i = 0; i < n; i++) sum2 += sc[i];
        if (sum2 > 0.0)
            for (int64_t i = 0; i < n; i++) sc[i] /= sum2;
    }
    /* generate.rs:175-186 weighted_sample */
    *rng_state += WY0;
    const double r = wy_f64(wy_mix(*rng_state));
    double cum = 0.0;
    int64_t tok = n - 1;
    for (int64_t i = 0; i < n; i++) {
        cum += sc[i];
        if (r < cum) {
            tok = i;
            break;
        }
    }
    free(sc);
    free(ix);
    return tok;
}

/* llama.rs:1035-1067 compute_rope_freqs (f64, optional Llama-3 scaling). */
void orc_compute_rope_freqs(int head_dim, float theta, int has_scaling, double factor,
                            double low_freq_factor, double high_freq_factor,
                            int64_t original_max_pos, double *out) {
    double th = (double)theta;
    int np = head_dim / 2;
    for (int i = 0; i < np; i++) out[i] = 1.0 / pow(th, 2.0 * (double)i / (double)head_dim);
    if (has_scaling) {
        double old_ctx = (double)original_max_pos;
        double low_wl = old_ctx / low_freq_factor;
        double high_wl = old_ctx / high_freq_factor;
        for (int i = 0; i < np; i++) {
            double wl = 2.0 * M_PI / out[i];
            double sf;
            if (wl < high_wl)
                sf = 1.0;
            else if (wl > low_wl)
                sf = factor;
            else {
                double smooth = (old_ctx / wl - low_freq_factor) / (high_freq_factor - low_freq_factor);
                sf = 1.0 / ((1.0 - smooth) / factor + smooth);
            }
            out[i] /= sf;
        }
    }
}

/* ------------------------------------------------------------------------
 * Llama model (llama.rs) with the build-defined int8 composition: every
 * projection matmul (fused qkv, o, gate, up, down, lm_head) becomes
 * matmul_i8_f32 on quantize_symmetric weights.
 * ---------------------------------------------------------------------- */
typedef struct {
    float *w;     /* f32 weights (NULL once freed) */
    int8_t *q;    /* per-tensor int8 */
    float s;
    int8_t *q32;  /* block-32 int8 */
    float *s32;   /* block-32 scales [n][ceil(k/32)] */
    int k, n;     /* logical [k, n] (lm head: stored [n, k]) */
    int tb;       /* stored transposed ([n,k]) */
} orc_proj;

struct orc_llama {
    orc_llama_config cfg;
    int hd, q_dim, kv_dim, qkv_dim;
    uint64_t rng_calls;
    float *embed;
    float *freqs;
    orc_proj *proj; /* n_layers * 5: qkv, o, gate, up, down */
    orc_proj lm;
    int lm_tied_f32; /* lm.w aliases embed */
    /* RMSNorm weights, (2 n_layers + 1) x h: input and post-attention per
     * layer, then the final norm.  RMSNorm::new (rmsnorm.rs:17-22) gives ones
     * and eps 1e-5; from_safetensors (llama.rs:880-914, 936-940) loads the
     * checkpoint's weights with config.rms_norm_eps. */
    float *norms;
    float norm_eps;
};

static void norms_init(orc_llama *m) {
    const size_t n = (size_t)(2 * m->cfg.n_layers + 1) * m->cfg.hidden_size;
    m->norms = (float *)malloc(sizeof(float) * n);
    for (size_t i = 0; i < n; i++) m->norms[i] = 1.0f;
    m->norm_eps = 1e-5f;
}

static const float *norm_w(const orc_llama *m, int which, int layer) {
    const int h = m->cfg.hidden_size;
    return m->norms + (which == 2 ? (size_t)(2 * m->cfg.n_layers) * h : (size_t)(2 * layer + which) * h);
}

struct orc_cache {
    int n_layers, max_seq, kv_dim;
    float **k, **v;
    int *len;
};

static float *gen(uint64_t seed, uint64_t *calls, size_t n) {
    float *w = (float *)malloc(sizeof(float) * n);
    orc_normal_vec_par(seed, *calls, n, 0.0f, 0.02f, w);
    *calls += 2 * (uint64_t)n;
    return w;
}

/* quantize a [k,n] (or [n,k] when tb) tensor per tensor and per block-32 */
static void proj_quantize(orc_proj *P, int block32) {
    size_t cnt = (size_t)P->k * P->n;
    P->q = (int8_t *)malloc(cnt);
    orc_quantize_symmetric(P->w, cnt, P->q, &P->s);
    if (block32) {
        int nb = (P->k + 31) / 32;
        P->q32 = (int8_t *)malloc(cnt);
        P->s32 = (float *)malloc(sizeof(float) * (size_t)P->n * nb);
        if (!P->tb) {
            orc_quantize_block32(P->w, P->k, P->n, P->q32, P->s32);
        } else {
            /* [n,k] storage: blocks run along each row */
            for (int j = 0; j < P->n; j++)
                for (int b = 0; b < nb; b++) {
                    int p0 = 32 * b, len = (P->k - p0) < 32 ? (P->k - p0) : 32;
                    orc_quantize_symmetric(P->w + (size_t)j * P->k + p0, (size_t)len,
                                           P->q32 + (size_t)j * P->k + p0,
                                           &P->s32[(size_t)j * nb + b]);
                }
        }
    }
}

orc_llama *orc_llama_new(const orc_llama_config *cfg, uint64_t seed, int quantize, int keep_f32,
                         int block32) {
    orc_llama *m = (orc_llama *)calloc(1, sizeof(orc_llama));
    m->cfg = *cfg;
    int h = cfg->hidden_size, V = cfg->vocab_size, ffn = cfg->intermediate_size;
    m->hd = h / cfg->n_heads;
    m->q_dim = cfg->n_heads * m->hd;
    m->kv_dim = cfg->n_kv_heads * m->hd;
    m->qkv_dim = m->q_dim + 2 * m->kv_dim;
    norms_init(m);
    uint64_t calls = 0;
    /* llama.rs:602-605 embed_tokens first */
    m->embed = gen(seed, &calls, (size_t)V * h);
    /* rope freqs (llama.rs:618-622), f64 -> f32 */
    int np = m->hd / 2;
    double *fd = (double *)malloc(sizeof(double) * np);
    orc_compute_rope_freqs(m->hd, cfg->rope_theta, cfg->has_rope_scaling, cfg->rs_factor,
                           cfg->rs_low_freq_factor, cfg->rs_high_freq_factor,
                           cfg->rs_original_max_pos, fd);
    m->freqs = (float *)malloc(sizeof(float) * np);
    for (int i = 0; i < np; i++) m->freqs[i] = (float)fd[i];
    free(fd);

    m->proj = (orc_proj *)calloc((size_t)cfg->n_layers * 5, sizeof(orc_proj));
    for (int l = 0; l < cfg->n_layers; l++) {
        orc_proj *P = m->proj + (size_t)l * 5;
        /* llama.rs:613-616 q, k, v then fuse_qkv_weights (1009-1029) */
        float *qw = gen(seed, &calls, (size_t)h * m->q_dim);
        float *kw = gen(seed, &calls, (size_t)h * m->kv_dim);
        float *vw = gen(seed, &calls, (size_t)h * m->kv_dim);
        float *qkv = (float *)malloc(sizeof(float) * (size_t)h * m->qkv_dim);
        for (int r = 0; r < h; r++) {
            float *dst = qkv + (size_t)r * m->qkv_dim;
            memcpy(dst, qw + (size_t)r * m->q_dim, sizeof(float) * m->q_dim);
            memcpy(dst + m->q_dim, kw + (size_t)r * m->kv_dim, sizeof(float) * m->kv_dim);
            memcpy(dst + m->q_dim + m->kv_dim, vw + (size_t)r * m->kv_dim,
                   sizeof(float) * m->kv_dim);
        }
        free(qw);
        free(kw);
        free(vw);
        P[0] = (orc_proj){qkv, NULL, 0, NULL, NULL, h, m->qkv_dim, 0};
        /* llama.rs:627-630 o_proj, then 645-656 gate, up, down */
        P[1] = (orc_proj){gen(seed, &calls, (size_t)m->q_dim * h), NULL, 0, NULL, NULL, m->q_dim, h, 0};
        P[2] = (orc_proj){gen(seed, &calls, (size_t)h * ffn), NULL, 0, NULL, NULL, h, ffn, 0};
        P[3] = (orc_proj){gen(seed, &calls, (size_t)h * ffn), NULL, 0, NULL, NULL, h, ffn, 0};
        P[4] = (orc_proj){gen(seed, &calls, (size_t)ffn * h), NULL, 0, NULL, NULL, ffn, h, 0};
        if (quantize)
            for (int t = 0; t < 5; t++) {
                proj_quantize(&P[t], block32);
                if (!keep_f32) {
                    free(P[t].w);
                    P[t].w = NULL;
                }
            }
    }
    /* llama.rs:664-671 untied lm_head last */
    if (cfg->tie_word_embeddings) {
        m->lm = (orc_proj){m->embed, NULL, 0, NULL, NULL, h, V, 1};
        m->lm_tied_f32 = 1;
    } else {
        m->lm = (orc_proj){gen(seed, &calls, (size_t)V * h), NULL, 0, NULL, NULL, h, V, 1};
    }
    if (quantize) {
        proj_quantize(&m->lm, block32);
        if (!keep_f32 && !m->lm_tied_f32) {
            free(m->lm.w);
            m->lm.w = NULL;
        }
    }
    m->rng_calls = calls;
    return m;
}

static void proj_free(orc_proj *P) {
    free(P->w);
    free(P->q);
    free(P->q32);
    free(P->s32);
}

void orc_llama_free(orc_llama *m) {
    if (!m) return;
    for (int i = 0; i < m->cfg.n_layers * 5; i++) proj_free(&m->proj[i]);
    free(m->proj);
    if (m->lm_tied_f32) m->lm.w = NULL;
    proj_free(&m->lm);
    free(m->embed);
    free(m->freqs);
    free(m->norms);
    free(m);
}

uint64_t orc_llama_rng_calls(const orc_llama *m) { return m->rng_calls; }

static const orc_proj *get_proj(const orc_llama *m, int id, int layer) {
    if (id == ORC_T_LM_HEAD) return &m->lm;
    if (id < ORC_T_QKV || id > ORC_T_DOWN || layer < 0 || layer >= m->cfg.n_layers) return NULL;
    return &m->proj[(size_t)layer * 5 + (id - ORC_T_QKV)];
}

size_t orc_llama_tensor(const orc_llama *m, int id, int layer, float *out) {
    if (id == ORC_T_EMBED) {
        size_t n = (size_t)m->cfg.vocab_size * m->cfg.hidden_size;
        if (out) memcpy(out, m->embed, sizeof(float) * n);
        return n;
    }
    if (id == ORC_T_ROPE_FREQS) {
        size_t n = (size_t)m->hd / 2;
        if (out) memcpy(out, m->freqs, sizeof(float) * n);
        return n;
    }
    const orc_proj *P = get_proj(m, id, layer);
    if (!P || !P->w) return 0;
    size_t n = (size_t)P->k * P->n;
    if (out) memcpy(out, P->w, sizeof(float) * n);
    return n;
}

size_t orc_llama_qtensor(const orc_llama *m, int id, int layer, int8_t *out, float *scale) {
    const orc_proj *P = get_proj(m, id, layer);
    if (!P || !P->q) return 0;
    size_t n = (size_t)P->k * P->n;
    if (out) memcpy(out, P->q, n);
    if (scale) *scale = P->s;
    return n;
}

size_t orc_llama_qscales_b32(const orc_llama *m, int id, int layer, float *out) {
    const orc_proj *P = get_proj(m, id, layer);
    if (!P || !P->s32) return 0;
    size_t n = (size_t)P->n * ((P->k + 31) / 32);
    if (out) memcpy(out, P->s32, sizeof(float) * n);
    return n;
}

/* one projection: rows x [k] -> rows x [n] */
static int run_proj(const orc_proj *P, const float *x, int rows, int mode, float *out) {
    if (mode == 0) {
        if (!P->w) return -1;
        orc_matmul_f32(x, P->w, rows, P->k, P->n, 0, P->tb, out);
        return 0;
    }
    if (mode == 3) {  /* the bf16 feature: bf16 operands, f32 result (cuda.rs:1226-1290) */
        if (!P->w) return -1;
        orc_matmul_bf16_par(x, P->w, rows, P->k, P->n, P->tb, out);
        return 0;
    }
    if (mode == 1) {
        if (!P->q) return -1;
        if (P->tb)
            orc_matmul_i8_f32_tb(x, P->q, P->s, rows, P->k, P->n, out);
        else
            orc_matmul_i8_f32_par(x, P->q, P->s, rows, P->k, P->n, out);
        return 0;
    }
    if (!P->q32) return -1;
    if (!P->tb) {
        orc_matmul_i8_f32_b32(x, P->q32, P->s32, rows, P->k, P->n, out);
    } else {
        int nb = (P->k + 31) / 32;
        for (int j = 0; j < P->n; j++)
            for (int i = 0; i < rows; i++) {
                float acc = 0.0f;
                for (int p = 0; p < P->k; p++) {
                    double sd = (double)P->s32[(size_t)j * nb + p / 32];
                    acc += (float)((double)x[(size_t)i * P->k + p] *
                                   ((double)P->q32[(size_t)j * P->k + p] * sd));
                }
                out[(size_t)i * P->n + j] = acc;
            }
    }
    return 0;
}


/* A model with the given int8 projections instead of a random init: the
 * projection buffers are allocated empty (orc_llama_set_* fill them).  Used to
 * time the CPU path on exactly the weights another implementation holds. */
orc_llama *orc_llama_new_empty(const orc_llama_config *cfg) {
    orc_llama *m = (orc_llama *)calloc(1, sizeof(orc_llama));
    m->cfg = *cfg;
    int h = cfg->hidden_size, V = cfg->vocab_size, ffn = cfg->intermediate_size;
    m->hd = h / cfg->n_heads;
    m->q_dim = cfg->n_heads * m->hd;
    m->kv_dim = cfg->n_kv_heads * m->hd;
    m->qkv_dim = m->q_dim + 2 * m->kv_dim;
    norms_init(m);
    m->embed = (float *)calloc((size_t)V * h, sizeof(float));
    int np = m->hd / 2;
    double *fd = (double *)malloc(sizeof(double) * np);
    orc_compute_rope_freqs(m->hd, cfg->rope_theta, cfg->has_rope_scaling, cfg->rs_factor,
                           cfg->rs_low_freq_factor, cfg->rs_high_freq_factor,
                           cfg->rs_original_max_pos, fd);
    m->freqs = (float *)malloc(sizeof(float) * np);
    for (int i = 0; i < np; i++) m->freqs[i] = (float)fd[i];
    free(fd);
    m->proj = (orc_proj *)calloc((size_t)cfg->n_layers * 5, sizeof(orc_proj));
    const int ks[5] = {h, m->q_dim, h, h, ffn}, ns[5] = {m->qkv_dim, h, ffn, ffn, h};
    for (int l = 0; l < cfg->n_layers; l++)
        for (int t = 0; t < 5; t++) {
            orc_proj *P = &m->proj[(size_t)l * 5 + t];
            P->k = ks[t];
            P->n = ns[t];
            P->q = (int8_t *)calloc((size_t)P->k * P->n, 1);
        }
    m->lm.k = h;
    m->lm.n = V;
    m->lm.tb = 1;
    m->lm.q = (int8_t *)calloc((size_t)V * h, 1);
    return m;
}

int orc_llama_set_qtensor(orc_llama *m, int id, int layer, const int8_t *q, float scale) {
    orc_proj *P = (orc_proj *)get_proj(m, id, layer);
    if (!P || !P->q) return -1;
    memcpy(P->q, q, (size_t)P->k * P->n);
    P->s = scale;
    return 0;
}

/* Block-32 int8 weights of a projection (forward mode 2): q32 in the
 * projection's storage layout ([k,n], or [n,k] for the LM head), scales
 * [n][ceil(k/32)]. */
int orc_llama_set_qtensor_b32(orc_llama *m, int id, int layer, const int8_t *q32, const float *s32) {
    orc_proj *P = (orc_proj *)get_proj(m, id, layer);
    if (!P) return -1;
    const size_t cnt = (size_t)P->k * P->n, ns = (size_t)P->n * ((P->k + 31) / 32);
    if (!P->q32) P->q32 = (int8_t *)malloc(cnt);
    if (!P->s32) P->s32 = (float *)malloc(sizeof(float) * ns);
    memcpy(P->q32, q32, cnt);
    memcpy(P->s32, s32, sizeof(float) * ns);
    return 0;
}

int orc_llama_set_embed(orc_llama *m, const float *w) {
    memcpy(m->embed, w, sizeof(float) * (size_t)m->cfg.vocab_size * m->cfg.hidden_size);
    return 0;
}

int orc_llama_set_norm(orc_llama *m, int which, int layer, const float *w, float eps) {
    if (which < 0 || which > 2 || (which < 2 && (layer < 0 || layer >= m->cfg.n_layers))) return -1;
    memcpy((float *)norm_w(m, which, layer), w, sizeof(float) * m->cfg.hidden_size);
    m->norm_eps = eps;
    return 0;
}

orc_cache *orc_cache_new(const orc_llama *m, int max_seq) {
    orc_cache *c = (orc_cache *)calloc(1, sizeof(orc_cache));
    c->n_layers = m->cfg.n_layers;
    c->max_seq = max_seq;
    c->kv_dim = m->kv_dim;
    c->k = (float **)calloc(c->n_layers, sizeof(float *));
    c->v = (float **)calloc(c->n_layers, sizeof(float *));
    c->len = (int *)calloc(c->n_layers, sizeof(int));
    for (int l = 0; l < c->n_layers; l++) {
        c->k[l] = (float *)calloc((size_t)max_seq * c->kv_dim, sizeof(float));
        c->v[l] = (float *)calloc((size_t)max_seq * c->kv_dim, sizeof(float));
    }
    return c;
}

void orc_cache_free(orc_cache *c) {
    if (!c) return;
    for (int l = 0; l < c->n_layers; l++) {
        free(c->k[l]);
        free(c->v[l]);
    }
    free(c->k);
    free(c->v);
    free(c->len);
    free(c);
}

int orc_cache_len(const orc_cache *c, int layer) { return c->len[layer]; }

void orc_cache_layer(const orc_cache *c, int layer, float *k_out, float *v_out) {
    size_t n = (size_t)c->max_seq * c->kv_dim;
    if (k_out) memcpy(k_out, c->k[layer], sizeof(float) * n);
    if (v_out) memcpy(v_out, c->v[layer], sizeof(float) * n);
}

#define ALLOC(n) ((float *)malloc(sizeof(float) * (size_t)(n)))

/* llama.rs:744-763 forward_with_llama_cache -> 556-569 layer ->
 * 371-468 attention -> 485-511 MLP, with projections per `mode`. */
int orc_llama_forward_with_cache(const orc_llama *m, orc_cache *c, int64_t token, int pos,
                                 int mode, float *logits) {
    const orc_llama_config *cf = &m->cfg;
    int h = cf->hidden_size, V = cf->vocab_size, ffn = cf->intermediate_size;
    int nh = cf->n_heads, nkv = cf->n_kv_heads, hd = m->hd;
    int qd = m->q_dim, kvd = m->kv_dim, qkvd = m->qkv_dim;
    (void)pos;
    float *x = ALLOC(h), *xn = ALLOC(h), *qkv = ALLOC(qkvd), *qr = ALLOC(qd), *qs = ALLOC(qd),
          *kr = ALLOC(kvd), *att = ALLOC(qd), *proj = ALLOC(h), *tmp = ALLOC(h), *g = ALLOC(ffn),
          *u = ALLOC(ffn), *act = ALLOC(ffn);
    float *K = NULL, *Vv = NULL, *sc = NULL, *pr = NULL;
    int rc = 0;
    if (orc_embedding(m->embed, &token, 1, V, h, x) != 0) {
        rc = -1;
        goto done;
    }
    for (int l = 0; l < cf->n_layers; l++) {
        const orc_proj *P = m->proj + (size_t)l * 5;
        if (c->len[l] >= c->max_seq) {
            rc = -2;
            goto done;
        }
        orc_rmsnorm(x, norm_w(m, 0, l), 1, h, m->norm_eps, xn);
        if ((rc = run_proj(&P[0], xn, 1, mode, qkv)) != 0) goto done;
        /* gather_columns (mod.rs:316-331) are slices of the fused row */
        orc_rope_with_freqs_preloaded(qkv, 1, nh, hd, pos, m->freqs, qr);
        orc_scale(qr, (size_t)qd, (float)(1.0 / sqrt((double)hd)), qs); /* mod.rs:219-230 */
        orc_rope_with_freqs_preloaded(qkv + qd, 1, nkv, hd, pos, m->freqs, kr);
        /* kv_cache.rs:99-118 append */
        orc_scatter_rows(c->k[l], kr, c->max_seq, kvd, c->len[l], 1);
        orc_scatter_rows(c->v[l], qkv + qd + kvd, c->max_seq, kvd, c->len[l], 1);
        c->len[l] += 1;
        int L = c->len[l];
        free(K);
        free(Vv);
        free(sc);
        free(pr);
        K = ALLOC((size_t)nh * L * hd);
        Vv = ALLOC((size_t)nh * L * hd);
        sc = ALLOC((size_t)nh * L);
        pr = ALLOC((size_t)nh * L);
        orc_gather_reshape_repeat_kv(c->k[l], c->max_seq, L, nkv, nh, hd, K);
        orc_gather_reshape_repeat_kv(c->v[l], c->max_seq, L, nkv, nh, hd, Vv);
        orc_matmul_strided_batched(qs, K, nh, 1, hd, L, 0, 1, sc);
        orc_softmax(sc, nh, L, pr);
        orc_matmul_strided_batched(pr, Vv, nh, 1, L, hd, 0, 0, att);
        if ((rc = run_proj(&P[1], att, 1, mode, proj)) != 0) goto done;
        orc_add(x, proj, (size_t)h, tmp);
        memcpy(x, tmp, sizeof(float) * h);
        orc_rmsnorm(x, norm_w(m, 1, l), 1, h, m->norm_eps, xn);
        if ((rc = run_proj(&P[2], xn, 1, mode, g)) != 0) goto done;
        if ((rc = run_proj(&P[3], xn, 1, mode, u)) != 0) goto done;
        orc_swiglu(g, u, (size_t)ffn, act);
        if ((rc = run_proj(&P[4], act, 1, mode, proj)) != 0) goto done;
        orc_add(x, proj, (size_t)h, tmp);
        memcpy(x, tmp, sizeof(float) * h);
    }
    orc_rmsnorm(x, norm_w(m, 2, 0), 1, h, m->norm_eps, xn);
    rc = run_proj(&m->lm, xn, 1, mode, logits);
done:
    free(x);
    free(xn);
    free(qkv);
    free(qr);
    free(qs);
    free(kr);
    free(att);
    free(proj);
    free(tmp);
    free(g);
    free(u);
    free(act);
    free(K);
    free(Vv);
    free(sc);
    free(pr);
    return rc;
}

/* llama.rs:683-700 forward -> 529-539 layer -> 162-266 attention (prefill). */
int orc_llama_forward(const orc_llama *m, const int64_t *tokens, int seq, int mode,
                      float *logits) {
    const orc_llama_config *cf = &m->cfg;
    int h = cf->hidden_size, V = cf->vocab_size, ffn = cf->intermediate_size;
    int nh = cf->n_heads, nkv = cf->n_kv_heads, hd = m->hd;
    int qd = m->q_dim, kvd = m->kv_dim, qkvd = m->qkv_dim;
    size_t S = (size_t)seq;
    float *x = ALLOC(S * h), *xn = ALLOC(S * h), *qkv = ALLOC(S * qkvd), *q = ALLOC(S * qd),
          *k = ALLOC(S * kvd), *v = ALLOC(S * kvd), *qr = ALLOC(S * qd), *kr = ALLOC(S * kvd),
          *qh = ALLOC(S * qd), *kh = ALLOC(S * kvd), *vh = ALLOC(S * kvd),
          *ke = ALLOC(S * qd), *ve = ALLOC(S * qd), *sc = ALLOC((size_t)nh * S * S),
          *pr = ALLOC((size_t)nh * S * S), *o = ALLOC(S * qd), *ho = ALLOC(S * qd),
          *proj = ALLOC(S * h), *g = ALLOC(S * ffn), *u = ALLOC(S * ffn), *act = ALLOC(S * ffn);
    int rc = orc_embedding(m->embed, tokens, seq, V, h, x);
    if (rc != 0) goto done;
    for (int l = 0; l < cf->n_layers; l++) {
        const orc_proj *P = m->proj + (size_t)l * 5;
        orc_rmsnorm(x, norm_w(m, 0, l), seq, h, m->norm_eps, xn);
        if ((rc = run_proj(&P[0], xn, seq, mode, qkv)) != 0) goto done;
        for (int s = 0; s < seq; s++) {
            memcpy(q + (size_t)s * qd, qkv + (size_t)s * qkvd, sizeof(float) * qd);
            memcpy(k + (size_t)s * kvd, qkv + (size_t)s * qkvd + qd, sizeof(float) * kvd);
            memcpy(v + (size_t)s * kvd, qkv + (size_t)s * qkvd + qd + kvd, sizeof(float) * kvd);
        }
        orc_rope_with_freqs_preloaded(q, seq, nh, hd, 0, m->freqs, qr);
        orc_rope_with_freqs_preloaded(k, seq, nkv, hd, 0, m->freqs, kr);
        /* reshape_for_heads (cpu.rs:215-240): [S, H*d] -> [H, S, d] */
        for (int hh = 0; hh < nh; hh++)
            for (int s = 0; s < seq; s++)
                memcpy(qh + ((size_t)hh * S + s) * hd, qr + (size_t)s * qd + (size_t)hh * hd,
                       sizeof(float) * hd);
        for (int hh = 0; hh < nkv; hh++)
            for (int s = 0; s < seq; s++) {
                memcpy(kh + ((size_t)hh * S + s) * hd, kr + (size_t)s * kvd + (size_t)hh * hd,
                       sizeof(float) * hd);
                memcpy(vh + ((size_t)hh * S + s) * hd, v + (size_t)s * kvd + (size_t)hh * hd,
                       sizeof(float) * hd);
            }
        orc_repeat_kv(kh, nkv, nh, seq, hd, ke);
        orc_repeat_kv(vh, nkv, nh, seq, hd, ve);
        orc_matmul_strided_batched(qh, ke, nh, seq, hd, seq, 0, 1, sc);
        orc_causal_mask_scale(sc, nh, seq, (float)(1.0 / sqrt((double)hd)), -INFINITY);
        orc_softmax(sc, nh * seq, seq, pr);
        orc_matmul_strided_batched(pr, ve, nh, seq, seq, hd, 0, 0, o);
        /* reshape_from_heads: [H, S, d] -> [S, H*d] */
        for (int hh = 0; hh < nh; hh++)
            for (int s = 0; s < seq; s++)
                memcpy(ho + (size_t)s * qd + (size_t)hh * hd, o + ((size_t)hh * S + s) * hd,
                       sizeof(float) * hd);
        if ((rc = run_proj(&P[1], ho, seq, mode, proj)) != 0) goto done;
        orc_add(x, proj, S * h, x);
        orc_rmsnorm(x, norm_w(m, 1, l), seq, h, m->norm_eps, xn);
        if ((rc = run_proj(&P[2], xn, seq, mode, g)) != 0) goto done;
        if ((rc = run_proj(&P[3], xn, seq, mode, u)) != 0) goto done;
        orc_swiglu(g, u, S * ffn, act);
        if ((rc = run_proj(&P[4], act, seq, mode, proj)) != 0) goto done;
        orc_add(x, proj, S * h, x);
    }
    orc_rmsnorm(x, norm_w(m, 2, 0), seq, h, m->norm_eps, xn);
    rc = run_proj(&m->lm, xn, seq, mode, logits);
done:
    free(x); free(xn); free(qkv); free(q); free(k); free(v); free(qr); free(kr);
    free(qh); free(kh); free(vh); free(ke); free(ve); free(sc); free(pr); free(o); free(ho);
    free(proj); free(g); free(u); free(act);
    return rc;
}

/* generate.rs:51-89 with temperature < 1e-8 (sample_token -> argmax).
 * Returns the number of tokens written: max(1, max_tokens), as the reference
 * pushes the prompt's sampled token before the generation loop. */
/* generate.rs:51-89 generate() with sample_token and Rng::with_seed(seed). */
int orc_generate(const orc_llama *m, const int64_t *prompt, int n_prompt, int max_tokens, float temperature,
                 int64_t top_k, float top_p, uint64_t seed, int mode, int64_t *out_tokens, float *step_logits) {
    if (n_prompt <= 0) return -1;
    int V = m->cfg.vocab_size;
    orc_cache *c = orc_cache_new(m, n_prompt + max_tokens);
    float *lg = ALLOC(V);
    uint64_t st = seed;
    int ng = 0, rc = 0;
    for (int pos = 0; pos < n_prompt; pos++) {
        if ((rc = orc_llama_forward_with_cache(m, c, prompt[pos], pos, mode, lg)) != 0) goto done;
        if (pos == n_prompt - 1) {
            if (step_logits) memcpy(step_logits + (size_t)ng * V, lg, sizeof(float) * V);
            out_tokens[ng++] = orc_sample_token(lg, V, temperature, top_k, top_p, &st);
        }
    }
    for (int i = 1; i < max_tokens; i++) {
        if ((rc = orc_llama_forward_with_cache(m, c, out_tokens[ng - 1], n_prompt + i - 1, mode, lg)) != 0) goto done;
        if (step_logits) memcpy(step_logits + (size_t)ng * V, lg, sizeof(float) * V);
        out_tokens[ng++] = orc_sample_token(lg, V, temperature, top_k, top_p, &st);
    }
    rc = ng;
done:
    free(lg);
    orc_cache_free(c);
    return rc;
}

int orc_generate_greedy(const orc_llama *m, const int64_t *prompt, int n_prompt, int max_tokens,
                        int mode, int64_t *out_tokens, float *step_logits) {
    if (n_prompt <= 0) return -1;
    int V = m->cfg.vocab_size;
    int max_seq = n_prompt + max_tokens;
    orc_cache *c = orc_cache_new(m, max_seq);
    float *lg = ALLOC(V);
    int ng = 0, rc = 0;
    for (int pos = 0; pos < n_prompt; pos++) {
        if ((rc = orc_llama_forward_with_cache(m, c, prompt[pos], pos, mode, lg)) != 0) goto done;
        if (pos == n_prompt - 1) {
            if (step_logits) memcpy(step_logits + (size_t)ng * V, lg, sizeof(float) * V);
            out_tokens[ng++] = orc_argmax(lg, V);
        }
    }
    for (int i = 1; i < max_tokens; i++) {
        int64_t last = out_tokens[ng - 1];
        int position = n_prompt + i - 1;
        if ((rc = orc_llama_forward_with_cache(m, c, last, position, mode, lg)) != 0) goto done;
        if (step_logits) memcpy(step_logits + (size_t)ng * V, lg, sizeof(float) * V);
        out_tokens[ng++] = orc_argmax(lg, V);
    }
    rc = ng;
done:
    free(lg);
    orc_cache_free(c);
    return rc;
}

/* ------------------------------------------------------------------------
 * Layer-major evaluation of the cache path, for parity runs at the
 * Llama-2-7B shape.  n tokens go through orc_llama_forward_with_cache one
 * after another (llama.rs:744-763) -- but computed layer by layer over all n
 * rows, so each int8 weight is read once per call instead of once per token.
 * Every element sees the same operations in the same order as in the
 * token-by-token function, so results are bit-identical (tested against it):
 *   - matmul_i8_f32 rows are independent; c[i][j] accumulates
 *     f32(f64(a) * (f64(q) * f64(scale))) in increasing p.  It is evaluated as
 *     f32((f64(a) * f64(scale)) * f64(q)): q*scale (8 x 24 bits) and a*scale
 *     (24 x 24 bits) are both exact in f64, so the single rounded f64 product
 *     is the same number;
 *   - row r's attention reads the cache rows 0 .. len+r, exactly those the
 *     token-by-token call sees, with gemv_trans_b / softmax / gemv_into
 *     arithmetic (cpu.rs:825-871, 336-366) on the cache rows in place;
 *   - rmsnorm, RoPE, scale, swiglu and add are per row.
 * Per-tensor int8 (forward mode 1) only.
 * ---------------------------------------------------------------------- */
#define MM_RB 8
#define MM_JW 256
#define MM_PD 24

__attribute__((target_clones("avx512f", "avx2", "default")))
static void mm_tile(const float *a, int k, int rows, const int8_t *q, int n, int j0, int jw,
                    double sd, float *c) {
    float acc[MM_RB][MM_JW];
    double qd[MM_JW];
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < jw; j++) acc[i][j] = 0.0f;
    for (int p = 0; p < k; p++) {
        const int8_t *qr = q + (size_t)p * n + j0;
        if (p + MM_PD < k)  /* rows are n bytes apart: no hardware prefetch */
            for (int j = 0; j < jw; j += 64) __builtin_prefetch(qr + (size_t)MM_PD * n + j);
        for (int j = 0; j < jw; j++) qd[j] = (double)qr[j];
        for (int i = 0; i < rows; i++) {
            const double asd = (double)a[(size_t)i * k + p] * sd;
            float *ar = acc[i];
            for (int j = 0; j < jw; j++) ar[j] += (float)(asd * qd[j]);
        }
    }
    for (int i = 0; i < rows; i++) memcpy(c + (size_t)i * n + j0, acc[i], sizeof(float) * (size_t)jw);
}

/* matmul_i8_f32 (cpu.rs:1128-1160 per-element order) of a [m,k] by q [k,n] */
static void mm_i8(const float *a, int m, int k, const int8_t *q, int n, float scale, float *c) {
    const double sd = (double)scale;
    const int nj = (n + MM_JW - 1) / MM_JW, ni = (m + MM_RB - 1) / MM_RB;
#pragma omp parallel for schedule(dynamic, 1) collapse(2) num_threads(NT) if (PAR_IF)
    for (int jc = 0; jc < nj; jc++)
        for (int ib = 0; ib < ni; ib++) {
            const int j0 = jc * MM_JW, jw = n - j0 < MM_JW ? n - j0 : MM_JW;
            const int i0 = ib * MM_RB, rows = m - i0 < MM_RB ? m - i0 : MM_RB;
            mm_tile(a + (size_t)i0 * k, k, rows, q, n, j0, jw, sd, c + (size_t)i0 * n);
        }
}

/* One query head against cache rows 0..L-1 (row stride kvd, head offset off):
 * gather_reshape_repeat_kv + gemv_trans_b (scores) + softmax + gemv_into,
 * with the cache read in place. */
static void attn_head(const float *qh, const float *K, const float *Vc, int kvd, int off, int L,
                      int hd, float *sc, float *pr, float *out) {
    const int k4 = hd & ~3;
    for (int j = 0; j < L; j++) {
        const float *row = K + (size_t)j * kvd + off;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (int p = 0; p < k4; p += 4) {
            a0 += qh[p] * row[p];
            a1 += qh[p + 1] * row[p + 1];
            a2 += qh[p + 2] * row[p + 2];
            a3 += qh[p + 3] * row[p + 3];
        }
        float acc = a0 + a1 + a2 + a3;
        for (int p = k4; p < hd; p++) acc += qh[p] * row[p];
        sc[j] = acc;
    }
    orc_softmax(sc, 1, L, pr);
    for (int j = 0; j < hd; j++) out[j] = 0.0f;
    const int L4 = L & ~3;
    for (int p = 0; p < L4; p += 4) {
        const float v0 = pr[p], v1 = pr[p + 1], v2 = pr[p + 2], v3 = pr[p + 3];
        const float *r0 = Vc + (size_t)p * kvd + off, *r1 = r0 + kvd, *r2 = r1 + kvd, *r3 = r2 + kvd;
        for (int j = 0; j < hd; j++) out[j] += v0 * r0[j] + v1 * r1[j] + v2 * r2[j] + v3 * r3[j];
    }
    for (int p = L4; p < L; p++) {
        const float v = pr[p];
        const float *r = Vc + (size_t)p * kvd + off;
        for (int j = 0; j < hd; j++) out[j] += v * r[j];
    }
}

/* the LM head [V,h] as q [h,V] (same values; the kernel above reads [k,n]) */
static int8_t *lm_transposed(const orc_llama *m) {
    const int h = m->cfg.hidden_size, V = m->cfg.vocab_size;
    int8_t *t = (int8_t *)malloc((size_t)h * V);
    if (!t) return NULL;
#pragma omp parallel for schedule(static) num_threads(NT) if (PAR_IF)
    for (int p = 0; p < h; p++)
        for (int j = 0; j < V; j++) t[(size_t)p * V + j] = m->lm.q[(size_t)j * h + p];
    return t;
}

static int fwd_seq(const orc_llama *m, orc_cache *c, const int8_t *lm_kn, const int64_t *tokens, int n,
                   int pos0, int n_logits, float *logits) {
    const orc_llama_config *cf = &m->cfg;
    const int h = cf->hidden_size, V = cf->vocab_size, ffn = cf->intermediate_size;
    const int nh = cf->n_heads, nkv = cf->n_kv_heads, hd = m->hd, nrep = nh / nkv;
    const int qd = m->q_dim, kvd = m->kv_dim, qkvd = m->qkv_dim;
    if (n <= 0 || n_logits < 0 || n_logits > n) return -4;
    for (int l = 0; l < cf->n_layers; l++) {
        for (int t = 0; t < 5; t++)
            if (!m->proj[(size_t)l * 5 + t].q) return -3;
        if (c->len[l] + n > c->max_seq) return -2;
    }
    if (n_logits && !m->lm.q) return -3;
    if (n_logits && m->lm.tb && !lm_kn) return -3;
    const size_t N = (size_t)n;
    float *x = ALLOC(N * h), *xn = ALLOC(N * h), *qkv = ALLOC(N * qkvd), *qs = ALLOC(N * qd),
          *att = ALLOC(N * qd), *proj = ALLOC(N * h), *g = ALLOC(N * ffn), *u = ALLOC(N * ffn),
          *act = ALLOC(N * ffn);
    const float qscale = (float)(1.0 / sqrt((double)hd));
    int rc = orc_embedding(m->embed, tokens, n, V, h, x);
    if (rc != 0) goto done;
    for (int l = 0; l < cf->n_layers; l++) {
        const orc_proj *P = m->proj + (size_t)l * 5;
        orc_rmsnorm(x, norm_w(m, 0, l), n, h, m->norm_eps, xn);
        mm_i8(xn, n, h, P[0].q, qkvd, P[0].s, qkv);
        const int base = c->len[l];
        float *Kc = c->k[l], *Vc = c->v[l];
#pragma omp parallel num_threads(NT) if (PAR_IF && n > 1)
        {
            float *qr = ALLOC(qd), *kr = ALLOC(kvd);
#pragma omp for schedule(static)
            for (int r = 0; r < n; r++) {
                const float *row = qkv + (size_t)r * qkvd;
                orc_rope_with_freqs_preloaded(row, 1, nh, hd, pos0 + r, m->freqs, qr);
                orc_scale(qr, (size_t)qd, qscale, qs + (size_t)r * qd);
                orc_rope_with_freqs_preloaded(row + qd, 1, nkv, hd, pos0 + r, m->freqs, kr);
                memcpy(Kc + (size_t)(base + r) * kvd, kr, sizeof(float) * kvd);
                memcpy(Vc + (size_t)(base + r) * kvd, row + qd + kvd, sizeof(float) * kvd);
            }
            free(qr);
            free(kr);
        }
        c->len[l] = base + n;
#pragma omp parallel num_threads(NT) if (PAR_IF)
        {
            float *sc = ALLOC(base + n), *pr = ALLOC(base + n);
#pragma omp for schedule(dynamic, 4) collapse(2)
            for (int r = 0; r < n; r++)
                for (int hh = 0; hh < nh; hh++)
                    attn_head(qs + (size_t)r * qd + (size_t)hh * hd, Kc, Vc, kvd, (hh / nrep) * hd,
                              base + r + 1, hd, sc, pr, att + (size_t)r * qd + (size_t)hh * hd);
            free(sc);
            free(pr);
        }
        mm_i8(att, n, qd, P[1].q, h, P[1].s, proj);
        orc_add(x, proj, N * h, x);
        orc_rmsnorm(x, norm_w(m, 1, l), n, h, m->norm_eps, xn);
        mm_i8(xn, n, h, P[2].q, ffn, P[2].s, g);
        mm_i8(xn, n, h, P[3].q, ffn, P[3].s, u);
        orc_swiglu(g, u, N * ffn, act);
        mm_i8(act, n, ffn, P[4].q, h, P[4].s, proj);
        orc_add(x, proj, N * h, x);
    }
    if (n_logits) {
        const int r0 = n - n_logits;
        orc_rmsnorm(x + (size_t)r0 * h, norm_w(m, 2, 0), n_logits, h, m->norm_eps, xn);
        mm_i8(xn, n_logits, h, m->lm.tb ? lm_kn : m->lm.q, V, m->lm.s, logits);
    }
done:
    free(x); free(xn); free(qkv); free(qs); free(att); free(proj); free(g); free(u); free(act);
    return rc;
}

int orc_llama_forward_cache_seq(const orc_llama *m, orc_cache *c, const int64_t *tokens, int n,
                                int pos0, int n_logits, float *logits) {
    int8_t *lm_kn = (n_logits > 0 && m->lm.tb && m->lm.q) ? lm_transposed(m) : NULL;
    int rc = fwd_seq(m, c, lm_kn, tokens, n, pos0, n_logits, logits);
    free(lm_kn);
    return rc;
}

/* orc_generate_greedy in mode 1, with the prompt run layer-major (one call)
 * and each generated token through the same layer-major code: the same
 * tokens and bit-identical step logits. */
int orc_generate_greedy_fast(const orc_llama *m, const int64_t *prompt, int n_prompt, int max_tokens,
                             int64_t *out_tokens, float *step_logits) {
    if (n_prompt <= 0) return -1;
    const int V = m->cfg.vocab_size;
    orc_cache *c = orc_cache_new(m, n_prompt + max_tokens);
    int8_t *lm_kn = (m->lm.tb && m->lm.q) ? lm_transposed(m) : NULL;
    float *lg = ALLOC(V);
    int ng = 0;
    int rc = fwd_seq(m, c, lm_kn, prompt, n_prompt, 0, 1, lg);
    if (rc != 0) goto done;
    if (step_logits) memcpy(step_logits, lg, sizeof(float) * V);
    out_tokens[ng++] = orc_argmax(lg, V);
    for (int i = 1; i < max_tokens; i++) {
        if ((rc = fwd_seq(m, c, lm_kn, &out_tokens[ng - 1], 1, n_prompt + i - 1, 1, lg)) != 0) goto done;
        if (step_logits) memcpy(step_logits + (size_t)ng * V, lg, sizeof(float) * V);
        out_tokens[ng++] = orc_argmax(lg, V);
    }
    rc = ng;
done:
    free(lg);
    free(lm_kn);
    orc_cache_free(c);
    return rc;
}

/* ------------------------------------------------------------------------
 * The rest of the trait surface (cpu.rs), for the device exports of the same
 * names.
 * ---------------------------------------------------------------------- */
/* cpu.rs:416-475 layernorm (layernorm_inference, 368-414, is the same output):
 * per row f64 mean (sequential sum / d), f64 variance of (x - mean),
 * rstd = 1 / sqrt(var + eps); out = f32((x - mean) * rstd * gamma + beta). */
void orc_layernorm(const float *x, const float *gamma, const float *beta, int rows, int d, float eps,
                   float *out, float *mean_out, float *rstd_out) {
    for (int i = 0; i < rows; i++) {
        const float *r = x + (size_t)i * d;
        double s = 0.0;
        for (int j = 0; j < d; j++) s += (double)r[j];
        const double mean = s / (double)d;
        double v = 0.0;
        for (int j = 0; j < d; j++) {
            const double df = (double)r[j] - mean;
            v += df * df;
        }
        const double var = v / (double)d;
        const double rstd = 1.0 / sqrt(var + (double)eps);
        if (mean_out) mean_out[i] = (float)mean;
        if (rstd_out) rstd_out[i] = (float)rstd;
        for (int j = 0; j < d; j++) {
            const double nrm = ((double)r[j] - mean) * rstd;
            out[(size_t)i * d + j] = (float)(nrm * (double)gamma[j] + (double)beta[j]);
        }
    }
}

/* cpu.rs:1110-1116 gelu_scalar (f64, tanh approximation) */
float orc_gelu(float x) {
    const double x64 = (double)x;
    const double c = sqrt(2.0 / M_PI);
    const double inner = c * (x64 + 0.044715 * x64 * x64 * x64);
    return (float)(0.5 * x64 * (1.0 + tanh(inner)));
}

void orc_gelu_vec(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_gelu(x[i]);
}

/* cpu.rs:500-503 sum: sequential f64, rounded once */
float orc_sum(const float *x, size_t n) {
    double s = 0.0;
    for (size_t i = 0; i < n; i++) s += (double)x[i];
    return (float)s;
}

/* cpu.rs:505-507 mul_elementwise */
void orc_mul(const float *a, const float *b, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = a[i] * b[i];
}

/* cpu.rs:601-633 rope: rows of last_dim, heads of head_dim, position pos;
 * freq_i = 1 / theta^(2i/head_dim) in f64, angle = pos * freq, cos / sin
 * rounded to f32, pairs (2i, 2i+1) rotated in f32; the rest copied. */
void orc_rope_rows(const float *x, size_t rows, int last_dim, int pos, int head_dim, float theta, float *out) {
    memcpy(out, x, sizeof(float) * rows * (size_t)last_dim);
    const double th = (double)theta;
    const int nh = last_dim / head_dim;
    for (size_t r = 0; r < rows; r++)
        for (int h = 0; h < nh; h++) {
            const size_t hs = r * (size_t)last_dim + (size_t)h * head_dim;
            for (int i = 0; i < head_dim / 2; i++) {
                const double freq = 1.0 / pow(th, 2.0 * (double)i / (double)head_dim);
                const double ang = (double)pos * freq;
                const float cv = (float)cos(ang), sv = (float)sin(ang);
                const float x0 = x[hs + 2 * i], x1 = x[hs + 2 * i + 1];
                out[hs + 2 * i] = x0 * cv - x1 * sv;
                out[hs + 2 * i + 1] = x0 * sv + x1 * cv;
            }
        }
}

/* mod.rs:316-331 gather_columns */
void orc_gather_columns(const float *x, int rows, int total, int start, int count, float *out) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < count; c++) out[(size_t)r * count + c] = x[(size_t)r * total + start + c];
}

/* mod.rs:334-350 scatter_columns (additive, in place) */
void orc_scatter_columns(float *dst, const float *src, int rows, int total, int start, int count) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < count; c++) dst[(size_t)r * total + start + c] += src[(size_t)r * count + c];
}

/* cpu.rs:94-188 add, generic broadcast form (tensor/shape.rs broadcast_strides):
 * every fast path of the CPU add computes the same a + b per output element. */
void orc_add_broadcast(const float *a, const size_t *ad, int an, const float *b, const size_t *bd, int bn,
                       const size_t *od, int on, float *out) {
    size_t os[6], as[6], bs[6], ast[6], bst[6], n = 1;
    for (int i = on - 1, acc = 1; i >= 0; i--) { os[i] = (size_t)acc; acc *= (int)od[i]; }
    { size_t acc = 1; for (int i = an - 1; i >= 0; i--) { as[i] = acc; acc *= ad[i]; } }
    { size_t acc = 1; for (int i = bn - 1; i >= 0; i--) { bs[i] = acc; acc *= bd[i]; } }
    for (int i = 0; i < on; i++) {
        const int ia = i - (on - an), ib = i - (on - bn);
        ast[i] = (ia < 0 || (ad[ia] == 1 && od[i] != 1)) ? 0 : as[ia];
        bst[i] = (ib < 0 || (bd[ib] == 1 && od[i] != 1)) ? 0 : bs[ib];
        n *= od[i];
    }
    for (size_t idx = 0; idx < n; idx++) {
        size_t rem = idx, ao = 0, bo = 0;
        for (int d = 0; d < on; d++) {
            const size_t c = rem / os[d];
            rem %= os[d];
            ao += c * ast[d];
            bo += c * bst[d];
        }
        out[idx] = a[ao] + b[bo];
    }
}

/* cpu.rs:300-334 scaled_softmax: f32 max of x*scale, e = expf(x*scale - max)
 * kept as f32, f64 sum, out = f32(f64(e) / sum) */
void orc_scaled_softmax(const float *x, int rows, int cols, float scale, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *in = x + (size_t)r * cols;
        float *o = out + (size_t)r * cols;
        float mx = -INFINITY;
        for (int i = 0; i < cols; i++) mx = fmaxf(mx, in[i] * scale);
        double sum = 0.0;
        for (int i = 0; i < cols; i++) {
            const double e = (double)expf(in[i] * scale - mx);
            o[i] = (float)e;
            sum += e;
        }
        for (int i = 0; i < cols; i++) o[i] = (float)((double)o[i] / sum);
    }
}

/* mod.rs:408-438 split_qkv_reshape_heads */
void orc_split_qkv_reshape_heads(const float *qkv, int seq, int n_heads, int d_head, float *q, float *k,
                                 float *v) {
    const int dm = n_heads * d_head;
    for (int s = 0; s < seq; s++)
        for (int h = 0; h < n_heads; h++)
            for (int d = 0; d < d_head; d++) {
                const size_t dst = ((size_t)h * seq + s) * d_head + d;
                const size_t src = (size_t)s * 3 * dm + (size_t)h * d_head + d;
                q[dst] = qkv[src];
                k[dst] = qkv[src + dm];
                v[dst] = qkv[src + 2 * dm];
            }
}

/* mod.rs:441-467 reshape_for_heads (dir 0) and 484-510 reshape_from_heads (dir 1) */
void orc_reshape_heads(const float *x, int batch, int seq, int n_heads, int d_head, int dir, float *out) {
    const int dm = n_heads * d_head;
    for (int b = 0; b < batch; b++)
        for (int h = 0; h < n_heads; h++)
            for (int s = 0; s < seq; s++)
                for (int d = 0; d < d_head; d++) {
                    const size_t heads = ((size_t)(b * n_heads + h) * seq + s) * d_head + d;
                    const size_t flat = (size_t)(b * seq + s) * dm + (size_t)h * d_head + d;
                    if (dir == 0)
                        out[heads] = x[flat];
                    else
                        out[flat] = x[heads];
                }
}
