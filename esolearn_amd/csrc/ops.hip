// The rest of the MathBackend / DeviceBackend surface (backend/mod.rs:12-622):
// the required methods that have no default body (ones, layernorm, gelu, sum,
// mul_elementwise, concat_rows, rope, broadcasting add) and the defaulted ones
// whose default body is a host round trip (gather/scatter of columns and rows,
// add_inplace, scaled_softmax, the causal masks, the QKV split and the head
// reshapes).  Each kernel follows the CPU backend's arithmetic (cpu.rs,
// cited per kernel); f64 where the CPU uses f64, f32 otherwise, and no
// contraction of a*b+c into an FMA.
#include <cmath>
#include <vector>

#include "internal.h"

#pragma clang fp contract(off)

namespace scry {
namespace {

inline unsigned grid1(size_t n, unsigned cap = 65536) {
    size_t g = (n + 255) / 256;
    return (unsigned)(g < 1 ? 1 : (g > cap ? cap : g));
}

#define GRID_STRIDE(i, n) \
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (size_t)gridDim.x * blockDim.x)

// sum over a 256-thread workgroup (f64); every thread gets the total
__device__ double block_sum(double v, double *red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();  // red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// cpu.rs:416-475 (layernorm) and 368-414 (layernorm_inference): per row, f64
// mean, f64 variance of (x - mean), rstd = 1 / sqrt(var + eps),
// out = f32((x - mean) * rstd * gamma + beta); mean and rstd rounded to f32.
__global__ __launch_bounds__(256) void k_layernorm(const float *__restrict__ x, const float *__restrict__ g,
                                                   const float *__restrict__ b, int d, float eps,
                                                   float *__restrict__ out, float *__restrict__ mean_out,
                                                   float *__restrict__ rstd_out) {
    __shared__ double red[4];
    const float *r = x + (size_t)blockIdx.x * d;
    double s = 0.0;
    for (int j = threadIdx.x; j < d; j += 256) s += (double)r[j];
    const double mean = block_sum(s, red) / (double)d;
    double v = 0.0;
    for (int j = threadIdx.x; j < d; j += 256) {
        const double df = (double)r[j] - mean;
        v += df * df;
    }
    const double var = block_sum(v, red) / (double)d;
    const double rstd = 1.0 / sqrt(var + (double)eps);
    for (int j = threadIdx.x; j < d; j += 256) {
        const double nrm = ((double)r[j] - mean) * rstd;
        out[(size_t)blockIdx.x * d + j] = (float)(nrm * (double)g[j] + (double)b[j]);
    }
    if (threadIdx.x == 0 && mean_out) {
        mean_out[blockIdx.x] = (float)mean;
        rstd_out[blockIdx.x] = (float)rstd;
    }
}

// cpu.rs:1110-1116 gelu_scalar: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), f64
__global__ void k_gelu(const float *__restrict__ x, size_t n, double sqrt_2_over_pi, float *__restrict__ out) {
    GRID_STRIDE(i, n) {
        const double x64 = (double)x[i];
        const double inner = sqrt_2_over_pi * (x64 + 0.044715 * x64 * x64 * x64);
        out[i] = (float)(0.5 * x64 * (1.0 + tanh(inner)));
    }
}

// cpu.rs:500-503 sum: f64 partial sums per workgroup (then one workgroup adds
// the partials in order)
__global__ __launch_bounds__(256) void k_sum_partial(const float *__restrict__ x, size_t n, double *__restrict__ part) {
    __shared__ double red[4];
    double s = 0.0;
    GRID_STRIDE(i, n) s += (double)x[i];
    s = block_sum(s, red);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_sum_final(const double *__restrict__ part, int np, float *__restrict__ out) {
    __shared__ double red[4];
    double s = 0.0;
    for (int i = threadIdx.x; i < np; i += 256) s += part[i];
    s = block_sum(s, red);
    if (threadIdx.x == 0) *out = (float)s;
}

// cpu.rs:505-507 mul_elementwise (f32)
__global__ void k_mul(const float *__restrict__ a, const float *__restrict__ b, size_t n, float *__restrict__ out) {
    GRID_STRIDE(i, n) out[i] = a[i] * b[i];
}

// cpu.rs:601-633 rope: rows of last_dim values, heads of head_dim inside each
// row, pairs (2i, 2i+1) rotated in f32 by the (cos, sin) of pair i (computed
// on the host in f64 with glibc, rounded to f32, as the CPU does).  Values past
// the last whole head of a row are copied.
__global__ void k_rope_row(const float *__restrict__ x, size_t rows, int last_dim, int head_dim,
                           const float2 *__restrict__ cs, float *__restrict__ out) {
    const int np = head_dim / 2, nh = last_dim / head_dim;
    const size_t total = rows * (size_t)last_dim;
    GRID_STRIDE(t, total) {
        const int c = (int)(t % last_dim);
        const int h = c / head_dim, w = c % head_dim, i = w / 2;
        if (h >= nh || i >= np) {
            out[t] = x[t];
            continue;
        }
        const size_t b0 = t - (size_t)(w & 1);
        const float x0 = x[b0], x1 = x[b0 + 1];
        const float cv = cs[i].x, sv = cs[i].y;
        out[t] = (w & 1) ? (x0 * sv + x1 * cv) : (x0 * cv - x1 * sv);
    }
}

// mod.rs:316-331 gather_columns: out[r][c] = x[r][start + c]
__global__ void k_gather_cols(const float *__restrict__ x, size_t rows, int total, int start, int count,
                              float *__restrict__ out) {
    const size_t n = rows * (size_t)count;
    GRID_STRIDE(t, n) {
        const size_t r = t / count;
        out[t] = x[r * total + start + (t % count)];
    }
}

// mod.rs:334-350 scatter_columns (additive): dst[r][start + c] += src[r][c]
__global__ void k_scatter_cols_add(float *__restrict__ dst, const float *__restrict__ src, size_t rows, int total,
                                   int start, int count) {
    const size_t n = rows * (size_t)count;
    GRID_STRIDE(t, n) {
        const size_t r = t / count;
        float *p = dst + r * total + start + (t % count);
        *p = *p + src[t];
    }
}

// cpu.rs:94-188 add: out[idx] = a[a_off] + b[b_off] with broadcast strides
// (stride 0 on broadcast dimensions, Shape::broadcast_strides); the CPU's
// same-shape and row / column fast paths give the same values.
struct BcastArgs {
    int ndim;
    size_t out_stride[6], a_stride[6], b_stride[6];
};

__global__ void k_add_bcast(const float *__restrict__ a, const float *__restrict__ b, size_t n, BcastArgs s,
                            float *__restrict__ out) {
    GRID_STRIDE(idx, n) {
        size_t rem = idx, ao = 0, bo = 0;
        for (int d = 0; d < s.ndim; d++) {
            const size_t c = rem / s.out_stride[d];
            rem -= c * s.out_stride[d];
            ao += c * s.a_stride[d];
            bo += c * s.b_stride[d];
        }
        out[idx] = a[ao] + b[bo];
    }
}

// cpu.rs:88-92 add_inplace
__global__ void k_add_inplace(float *__restrict__ d, const float *__restrict__ s, size_t n) {
    GRID_STRIDE(i, n) d[i] = d[i] + s[i];
}

// cpu.rs:300-334 scaled_softmax: v = x * scale (f32), max of v, e = expf(v - max)
// kept as f32, f64 sum, out = f32(f64(e) / sum).  One workgroup per row.
__global__ __launch_bounds__(256) void k_scaled_softmax(const float *__restrict__ x, int cols, float scale,
                                                        float *__restrict__ out) {
    const float *r = x + (size_t)blockIdx.x * cols;
    float *o = out + (size_t)blockIdx.x * cols;
    __shared__ float redf[4];
    __shared__ double redd[4];
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < cols; j += 256) mx = fmaxf(mx, r[j] * scale);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) redf[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
    double sum = 0.0;
    for (int j = threadIdx.x; j < cols; j += 256) {
        const float e = expf(r[j] * scale - mx);
        o[j] = e;
        sum += (double)e;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((threadIdx.x & 63) == 0) redd[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = (redd[0] + redd[1]) + (redd[2] + redd[3]);
    for (int j = threadIdx.x; j < cols; j += 256) o[j] = (float)((double)o[j] / sum);
}

// mod.rs:384-401 / 595-621: t > s -> mask_value, else *= scale, on n_mat
// [seq, seq] matrices in place
__global__ void k_causal_mask(float *__restrict__ sc, size_t n_mat, int seq, float scale, float mask_value) {
    const size_t mat = (size_t)seq * seq, n = n_mat * mat;
    GRID_STRIDE(t, n) {
        const size_t w = t % mat;
        const int s = (int)(w / seq), c = (int)(w % seq);
        sc[t] = c > s ? mask_value : sc[t] * scale;
    }
}

// mod.rs:408-438 split_qkv_reshape_heads: [seq, 3 d_model] -> three
// [n_heads, seq, d_head]
__global__ void k_split_qkv(const float *__restrict__ qkv, int seq, int n_heads, int d_head,
                            float *__restrict__ q, float *__restrict__ k, float *__restrict__ v) {
    const int dm = n_heads * d_head;
    const size_t n = (size_t)seq * dm;
    GRID_STRIDE(t, n) {  // t = (h * seq + s) * d_head + d
        const int d = (int)(t % d_head);
        const size_t hs = t / d_head;
        const int s = (int)(hs % seq), h = (int)(hs / seq);
        const size_t row = (size_t)s * 3 * dm + (size_t)h * d_head + d;
        q[t] = qkv[row];
        k[t] = qkv[row + dm];
        v[t] = qkv[row + 2 * dm];
    }
}

// mod.rs:441-467 reshape_for_heads: [B*S, H*d] -> [B*H, S, d] (dir 0) and
// mod.rs:484-510 reshape_from_heads, its inverse (dir 1)
__global__ void k_reshape_heads(const float *__restrict__ x, int batch, int seq, int n_heads, int d_head, int dir,
                                float *__restrict__ out) {
    const size_t n = (size_t)batch * seq * n_heads * d_head;
    GRID_STRIDE(t, n) {  // t indexes the [B*H, S, d] layout
        const int d = (int)(t % d_head);
        const size_t r = t / d_head;
        const int s = (int)(r % seq);
        const size_t bh = r / seq;
        const int h = (int)(bh % n_heads);
        const size_t b = bh / n_heads;
        const size_t flat = ((b * seq + s) * n_heads + h) * d_head + d;  // [B*S, H*d] index
        if (dir == 0)
            out[t] = x[flat];
        else
            out[flat] = x[t];
    }
}

}  // namespace

#define LAUNCH_CHECK() SCRY_HIP(hipGetLastError()); return SCRY_OK

int launch_layernorm(const float *x, const float *g, const float *b, int rows, int d, float eps, float *out,
                     float *mean, float *rstd, hipStream_t s) {
    if (rows <= 0 || d <= 0) return SCRY_OK;
    hipLaunchKernelGGL(k_layernorm, dim3(rows), dim3(256), 0, s, x, g, b, d, eps, out, mean, rstd);
    LAUNCH_CHECK();
}

int launch_gelu(const float *x, size_t n, float *out, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    // (2.0 / PI).sqrt() in f64 (cpu.rs:1113)
    const double c = std::sqrt(2.0 / M_PI);
    hipLaunchKernelGGL(k_gelu, dim3(grid1(n)), dim3(256), 0, s, x, n, c, out);
    LAUNCH_CHECK();
}

int sum_partials(size_t n) { return (int)grid1(n, 1024); }

int launch_sum(const float *x, size_t n, double *part, float *out, hipStream_t s) {
    const int np = sum_partials(n);
    hipLaunchKernelGGL(k_sum_partial, dim3(np), dim3(256), 0, s, x, n, part);
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(256), 0, s, part, np, out);
    LAUNCH_CHECK();
}

int launch_mul(const float *a, const float *b, size_t n, float *out, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_mul, dim3(grid1(n)), dim3(256), 0, s, a, b, n, out);
    LAUNCH_CHECK();
}

int launch_rope_row(const float *x, size_t rows, int last_dim, int head_dim, const float2 *cs, float *out,
                    hipStream_t s) {
    const size_t n = rows * (size_t)last_dim;
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_rope_row, dim3(grid1(n)), dim3(256), 0, s, x, rows, last_dim, head_dim, cs, out);
    LAUNCH_CHECK();
}

int launch_gather_cols(const float *x, size_t rows, int total, int start, int count, float *out, hipStream_t s) {
    const size_t n = rows * (size_t)count;
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_gather_cols, dim3(grid1(n)), dim3(256), 0, s, x, rows, total, start, count, out);
    LAUNCH_CHECK();
}

int launch_scatter_cols_add(float *dst, const float *src, size_t rows, int total, int start, int count,
                            hipStream_t s) {
    const size_t n = rows * (size_t)count;
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_scatter_cols_add, dim3(grid1(n)), dim3(256), 0, s, dst, src, rows, total, start, count);
    LAUNCH_CHECK();
}

int launch_add_bcast(const float *a, const size_t *a_dims, int a_ndim, const float *b, const size_t *b_dims,
                     int b_ndim, const size_t *o_dims, int o_ndim, float *out, hipStream_t s) {
    BcastArgs ba{};
    ba.ndim = o_ndim;
    // Shape::strides / broadcast_strides (tensor/shape.rs)
    auto strides = [](const size_t *d, int nd, size_t *st) {
        size_t acc = 1;
        for (int i = nd - 1; i >= 0; i--) {
            st[i] = acc;
            acc *= d[i];
        }
    };
    size_t as[6], bs[6];
    strides(o_dims, o_ndim, ba.out_stride);
    strides(a_dims, a_ndim, as);
    strides(b_dims, b_ndim, bs);
    for (int i = 0; i < o_ndim; i++) {
        const int ia = i - (o_ndim - a_ndim), ib = i - (o_ndim - b_ndim);
        ba.a_stride[i] = ia < 0 || (a_dims[ia] == 1 && o_dims[i] != 1) ? 0 : as[ia];
        ba.b_stride[i] = ib < 0 || (b_dims[ib] == 1 && o_dims[i] != 1) ? 0 : bs[ib];
    }
    size_t n = 1;
    for (int i = 0; i < o_ndim; i++) n *= o_dims[i];
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_add_bcast, dim3(grid1(n)), dim3(256), 0, s, a, b, n, ba, out);
    LAUNCH_CHECK();
}

int launch_add_inplace(float *d, const float *src, size_t n, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_add_inplace, dim3(grid1(n)), dim3(256), 0, s, d, src, n);
    LAUNCH_CHECK();
}

int launch_scaled_softmax(const float *x, int rows, int cols, float scale, float *out, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return SCRY_OK;
    hipLaunchKernelGGL(k_scaled_softmax, dim3(rows), dim3(256), 0, s, x, cols, scale, out);
    LAUNCH_CHECK();
}

int launch_causal_mask(float *sc, size_t n_mat, int seq, float scale, float mask_value, hipStream_t s) {
    const size_t n = n_mat * (size_t)seq * seq;
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_causal_mask, dim3(grid1(n)), dim3(256), 0, s, sc, n_mat, seq, scale, mask_value);
    LAUNCH_CHECK();
}

int launch_split_qkv(const float *qkv, int seq, int n_heads, int d_head, float *q, float *k, float *v,
                     hipStream_t s) {
    const size_t n = (size_t)seq * n_heads * d_head;
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_split_qkv, dim3(grid1(n)), dim3(256), 0, s, qkv, seq, n_heads, d_head, q, k, v);
    LAUNCH_CHECK();
}

int launch_reshape_heads(const float *x, int batch, int seq, int n_heads, int d_head, int dir, float *out,
                         hipStream_t s) {
    const size_t n = (size_t)batch * seq * n_heads * d_head;
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_reshape_heads, dim3(grid1(n)), dim3(256), 0, s, x, batch, seq, n_heads, d_head, dir, out);
    LAUNCH_CHECK();
}

}  // namespace scry
