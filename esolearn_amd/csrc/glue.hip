// Op-level glue kernels behind the MathBackend entry points (cpu.rs citations
// per kernel).  The decode step does not use these: its RMSNorm, RoPE, KV
// append, SwiGLU, residual add, embedding and argmax are fused into the GEMV
// and attention kernels.  These serve the per-op API (a Rust HipBackend's
// trait methods) and the parity tests.
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

inline unsigned grid1(size_t n, unsigned cap = 65536) {
    size_t g = (n + 255) / 256;
    return (unsigned)(g < 1 ? 1 : (g > cap ? cap : g));
}

#define GRID_STRIDE(i, n) \
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (size_t)gridDim.x * blockDim.x)

// cpu.rs:574-599: one workgroup per row, f64 sum of squares.
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x,
                                                 const float *__restrict__ w, int d, float eps,
                                                 float *__restrict__ out) {
    const float *r = x + (size_t)blockIdx.x * d;
    double ss = 0.0;
    for (int j = threadIdx.x; j < d; j += 256) ss += (double)r[j] * (double)r[j];
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    __shared__ double red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double rstd = 1.0 / sqrt(tot / (double)d + (double)eps);
    for (int j = threadIdx.x; j < d; j += 256)
        out[(size_t)blockIdx.x * d + j] = (float)((double)r[j] * rstd * (double)w[j]);
}

// cpu.rs:635-664 (+ mod.rs:219-230 scale): one thread per rotated pair.
__global__ void k_rope(const float *__restrict__ x, int seq, int n_heads, int hd, int start_pos,
                       const float *__restrict__ freqs, int scaled, float scale,
                       float *__restrict__ out) {
    const int np = hd / 2;
    const size_t total = (size_t)seq * n_heads * np;
    GRID_STRIDE(t, total) {
        const int i = (int)(t % np);
        const size_t hs = t / np;  // s * n_heads + h
        const int s = (int)(hs / n_heads);
        const size_t base = hs * hd + 2 * i;
        const double ang = (double)(start_pos + s) * (double)freqs[i];
        const float c = (float)cos(ang), sn = (float)sin(ang);
        const float x0 = x[base], x1 = x[base + 1];
        float r0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
        float r1 = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
        if (scaled) {
            r0 = __fmul_rn(r0, scale);
            r1 = __fmul_rn(r1, scale);
        }
        out[base] = r0;
        out[base + 1] = r1;
    }
}

__global__ void k_scale(const float *__restrict__ x, size_t n, float s, float *__restrict__ out) {
    GRID_STRIDE(i, n) out[i] = __fmul_rn(x[i], s);
}

// cpu.rs:336-366: f32 max (NaN ignored), e = expf(x - max) kept as f32,
// f64 sum, out = f32(f64(e) / sum).  One workgroup per row.
__global__ __launch_bounds__(256) void k_softmax(const float *__restrict__ x, int cols,
                                                 float *__restrict__ out) {
    const float *r = x + (size_t)blockIdx.x * cols;
    float *o = out + (size_t)blockIdx.x * cols;
    __shared__ float redf[4];
    __shared__ double redd[4];
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < cols; j += 256) mx = fmaxf(mx, r[j]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) redf[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
    double sum = 0.0;
    for (int j = threadIdx.x; j < cols; j += 256) {
        const float e = expf(__fsub_rn(r[j], mx));
        o[j] = e;
        sum += (double)e;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((threadIdx.x & 63) == 0) redd[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = redd[0] + redd[1] + redd[2] + redd[3];
    for (int j = threadIdx.x; j < cols; j += 256) o[j] = (float)((double)o[j] / sum);
}

// cpu.rs:666-678, 1119-1122
__global__ void k_swiglu(const float *__restrict__ g, const float *__restrict__ u, size_t n,
                         float *__restrict__ out) {
    GRID_STRIDE(i, n) {
        const double x = (double)g[i];
        out[i] = __fmul_rn((float)(x / (1.0 + exp(-x))), u[i]);
    }
}

__global__ void k_add(const float *__restrict__ a, const float *__restrict__ b, size_t n,
                      float *__restrict__ out) {
    GRID_STRIDE(i, n) out[i] = __fadd_rn(a[i], b[i]);
}

// mod.rs:76-83: the bias row added to every row of c [rows, n], in place
__global__ void k_add_bias_rows(float *__restrict__ c, const float *__restrict__ bias,
                                size_t total, int n) {
    GRID_STRIDE(i, total) c[i] = __fadd_rn(c[i], bias[i % n]);
}

// cpu.rs:485-498 (ids validated on the host)
__global__ void k_embedding(const float *__restrict__ w, const int64_t *__restrict__ ids,
                            int n_ids, int dim, float *__restrict__ out) {
    const size_t total = (size_t)n_ids * dim;
    GRID_STRIDE(t, total) {
        const size_t i = t / dim, d = t % dim;
        out[t] = w[(size_t)ids[i] * dim + d];
    }
}

// cpu.rs:707-730: [max_seq, n_kv*hd] -> [n_q, L, hd]
__global__ void k_gather_repeat_kv(const float *__restrict__ cache, int L, int n_kv, int n_q,
                                   int hd, float *__restrict__ out) {
    const int n_rep = n_q / n_kv;
    const size_t total = (size_t)n_q * L * hd;
    GRID_STRIDE(t, total) {
        const int d = (int)(t % hd);
        const size_t qs = t / hd;
        const int s = (int)(qs % L), qh = (int)(qs / L);
        out[t] = cache[(size_t)s * n_kv * hd + (size_t)(qh / n_rep) * hd + d];
    }
}

// cpu.rs:680-705
__global__ void k_repeat_kv(const float *__restrict__ x, int n_kv, int n_q, int seq, int d_head,
                            float *__restrict__ out) {
    const int n_rep = n_q / n_kv;
    const size_t hs = (size_t)seq * d_head;
    const size_t total = (size_t)n_q * hs;
    GRID_STRIDE(t, total) {
        const size_t qh = t / hs, w = t % hs;
        out[t] = x[(qh / n_rep) * hs + w];
    }
}

// Generic f32 (batched) matmul, one thread per output: f64 accumulation in
// increasing p (the reference's m > 1 fallback, cpu.rs:875-999; its m == 1
// GEMV sums in f32 -- the difference is within f32 rounding).
__global__ void k_matmul_f32(const float *__restrict__ a, const float *__restrict__ b, int batch,
                             int m, int k, int n, int ta, int tb, float *__restrict__ c) {
    const size_t total = (size_t)batch * m * n;
    GRID_STRIDE(t, total) {
        const int j = (int)(t % n);
        const size_t bi = t / n;
        const int i = (int)(bi % m);
        const size_t bt = bi / m;
        const float *A = a + bt * (size_t)m * k;
        const float *B = b + bt * (size_t)k * n;
        double acc = 0.0;
        for (int p = 0; p < k; p++) {
            const double av = ta ? (double)A[(size_t)p * m + i] : (double)A[(size_t)i * k + p];
            const double bv = tb ? (double)B[(size_t)j * k + p] : (double)B[(size_t)p * n + j];
            acc += av * bv;
        }
        c[t] = (float)acc;
    }
}

// Logits of the int8 LM head for rows whose normalised input holds an
// infinity or a NaN.  The prefill GEMMs mark such a row and give NaN for all
// of it, while the reference's sum of f64(a) (q s) over k (cpu.rs:1128-1160)
// is +-inf per column unless a NaN term or both infinities occur; only the
// terms of the non-finite inputs decide it.  One workgroup per row:
// RMSNorm's f64 scale (cpu.rs:574-599) and the normalised values
// f32(f64(x) rstd f64(g)); a row with none non-finite is left as it is;
// otherwise each 256-position chunk's non-finite values (at most 256) are
// gathered in LDS and every column's class is folded into its logit (the
// classes combine in any order).
__global__ __launch_bounds__(256) void k_logits_nonfinite(const float *__restrict__ x, int ldx,
                                                          const float *__restrict__ g, float eps, int k,
                                                          const uint8_t *__restrict__ W, int kp,
                                                          const float *__restrict__ s32, int nb, float scale,
                                                          int n, float *__restrict__ y, int ldy) {
    __shared__ double red[4];
    __shared__ int s_cnt;
    __shared__ int s_idx[256];
    __shared__ float s_val[256];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (size_t)row * ldx;
    float *yr = y + (size_t)row * ldy;
    double ss = 0.0;
    for (int p = tid; p < k; p += 256) ss += (double)xr[p] * (double)xr[p];
    ss = dev::block_sum_d(ss, red);
    const double rstd = 1.0 / sqrt(ss / (double)k + (double)eps);
    bool seen = false;  // uniform: a chunk with non-finite values was folded in
    for (int p0 = 0; p0 < k; p0 += 256) {
        const int p = p0 + tid;
        float t = 0.f;
        if (p < k) t = g ? (float)((double)xr[p] * rstd * (double)g[p]) : xr[p];
        __syncthreads();
        if (tid == 0) s_cnt = 0;
        __syncthreads();
        if (p < k && !isfinite(t)) {
            const int i = atomicAdd(&s_cnt, 1);
            s_idx[i] = p;
            s_val[i] = t;
        }
        __syncthreads();
        const int cnt = s_cnt;
        if (cnt == 0) continue;
        for (int j = tid; j < n; j += 256) {
            int cls = seen ? dev::nonfinite_class(yr[j]) : 0;
            const uint8_t *wr = W + (size_t)j * kp;
            for (int i = 0; i < cnt; i++) {
                const int q = s_idx[i];
                cls |= dev::nonfinite_term(s_val[i], wr[q], s32 ? s32[(size_t)j * nb + (q >> 5)] : scale);
            }
            yr[j] = dev::nonfinite_value(cls);
        }
        seen = true;
    }
}

__global__ void k_fill_f32(float *p, size_t n, float v) { GRID_STRIDE(i, n) p[i] = v; }
__global__ void k_fill_u32(unsigned int *p, size_t n, unsigned int v) { GRID_STRIDE(i, n) p[i] = v; }

}  // namespace

#define LAUNCH_CHECK() SCRY_HIP(hipGetLastError()); return SCRY_OK

int launch_rmsnorm(const float *x, const float *w, int rows, int d, float eps, float *out,
                   hipStream_t s) {
    if (rows <= 0) return SCRY_OK;
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), 0, s, x, w, d, eps, out);
    LAUNCH_CHECK();
}

int launch_rope(const float *x, int seq, int n_heads, int hd, int start_pos, const float *freqs,
                int scaled, float scale, float *out, hipStream_t s) {
    const size_t total = (size_t)seq * n_heads * (hd / 2);
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_rope, dim3(grid1(total)), dim3(256), 0, s, x, seq, n_heads, hd, start_pos,
                       freqs, scaled, scale, out);
    LAUNCH_CHECK();
}

int launch_scale(const float *x, size_t n, float sc, float *out, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_scale, dim3(grid1(n)), dim3(256), 0, s, x, n, sc, out);
    LAUNCH_CHECK();
}

int launch_softmax(const float *x, int rows, int cols, float *out, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return SCRY_OK;
    hipLaunchKernelGGL(k_softmax, dim3(rows), dim3(256), 0, s, x, cols, out);
    LAUNCH_CHECK();
}

int launch_swiglu(const float *g, const float *u, size_t n, float *out, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_swiglu, dim3(grid1(n)), dim3(256), 0, s, g, u, n, out);
    LAUNCH_CHECK();
}

int launch_add(const float *a, const float *b, size_t n, float *out, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_add, dim3(grid1(n)), dim3(256), 0, s, a, b, n, out);
    LAUNCH_CHECK();
}

int launch_add_bias_rows(float *c, const float *bias, int rows, int n, hipStream_t s) {
    const size_t total = (size_t)rows * n;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_add_bias_rows, dim3(grid1(total)), dim3(256), 0, s, c, bias, total, n);
    LAUNCH_CHECK();
}

int launch_embedding(const float *w, const int64_t *ids, int n_ids, int dim, float *out,
                     hipStream_t s) {
    const size_t total = (size_t)n_ids * dim;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_embedding, dim3(grid1(total)), dim3(256), 0, s, w, ids, n_ids, dim, out);
    LAUNCH_CHECK();
}

int launch_gather_repeat_kv(const float *cache, int cached_len, int n_kv, int n_q, int hd,
                            float *out, hipStream_t s) {
    const size_t total = (size_t)n_q * cached_len * hd;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_gather_repeat_kv, dim3(grid1(total)), dim3(256), 0, s, cache, cached_len,
                       n_kv, n_q, hd, out);
    LAUNCH_CHECK();
}

int launch_repeat_kv(const float *x, int n_kv, int n_q, int seq, int d_head, float *out,
                     hipStream_t s) {
    const size_t total = (size_t)n_q * seq * d_head;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_repeat_kv, dim3(grid1(total)), dim3(256), 0, s, x, n_kv, n_q, seq, d_head,
                       out);
    LAUNCH_CHECK();
}

int launch_matmul_f32(const float *a, const float *b, int batch, int m, int k, int n, int ta,
                      int tb, float *c, hipStream_t s) {
    const size_t total = (size_t)batch * m * n;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_matmul_f32, dim3(grid1(total)), dim3(256), 0, s, a, b, batch, m, k, n, ta,
                       tb, c);
    LAUNCH_CHECK();
}

int launch_logits_nonfinite(const float *x, int ldx, int rows, const float *norm_w, float eps, const Packed &w,
                            float *y, int ldy, hipStream_t s) {
    if (rows <= 0 || w.bf16) return SCRY_OK;  // bf16 rows: the GEMM's products already give +-inf
    hipLaunchKernelGGL(k_logits_nonfinite, dim3(rows), dim3(256), 0, s, x, ldx, norm_w, eps, w.k, w.d, w.kp, w.s32,
                       w.nb, w.scale, w.rows, y, ldy);
    LAUNCH_CHECK();
}

int launch_fill_f32(float *p, size_t n, float v, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_fill_f32, dim3(grid1(n)), dim3(256), 0, s, p, n, v);
    LAUNCH_CHECK();
}

int launch_fill_u32(unsigned int *p, size_t n, unsigned int v, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid1(n)), dim3(256), 0, s, p, n, v);
    LAUNCH_CHECK();
}

}  // namespace scry
