// Weight layout step on the device: quantize_symmetric (quantize.rs:16-32),
// the block-32 extension, and the repack into the GEMV stream layout.
//
// quantize_symmetric semantics kept bit-exact:
//   absmax = fold(0, f32::max(acc, |w|))  -- NaN ignored (fmaxf does the same)
//   scale  = absmax / 127 (f32, correctly rounded division)
//   inv    = 1 / scale
//   q      = clamp(round_half_away(w * inv), -127, 127), NaN -> 0 (Rust `as i8`)
// absmax is order independent, so a parallel max reduction gives the same value.
#include "internal.h"

namespace scry {

namespace {

__device__ __forceinline__ int8_t quant_one(float w, float inv) {
    float r = roundf(__fmul_rn(w, inv));
    if (isnan(r)) return 0;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int8_t)r;
}

__device__ __forceinline__ void scale_from_bits(unsigned int bits, float *scale, float *inv) {
    float absmax = __uint_as_float(bits);
    if (absmax == 0.0f) {
        *scale = 0.0f;
        *inv = 0.0f;
        return;
    }
    float s = absmax / 127.0f;
    *scale = s;
    *inv = 1.0f / s;
}

__global__ void k_absmax(const float *__restrict__ w, size_t n, unsigned int *out) {
    float m = 0.0f;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        m = fmaxf(m, fabsf(w[i]));
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    __shared__ float red[16];
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = red[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) t = fmaxf(t, red[i]);
        // non-negative, non-NaN floats order like their bit patterns
        atomicMax(out, __float_as_uint(t));
    }
}

__global__ void k_quantize_plain(const float *__restrict__ w, size_t n,
                                 const unsigned int *__restrict__ bits, int8_t *__restrict__ q,
                                 float *scale_out) {
    float s, inv;
    scale_from_bits(*bits, &s, &inv);
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i0 == 0 && scale_out) *scale_out = s;
    for (size_t i = i0; i < n; i += stride) q[i] = (s == 0.0f) ? (int8_t)0 : quant_one(w[i], inv);
}

__device__ __forceinline__ int map_row(int j, int grp, int stride, int off) {
    return (j / grp) * stride + off + (j % grp);
}

// [k,n] source -> packed rows: 64x64 tile transposed through LDS.
// MODE 0: f32 source quantized with the per-tensor scale; MODE 1: int8 source.
template <int MODE>
__global__ __launch_bounds__(256) void k_pack_kn(const void *__restrict__ src, int k, int n,
                                                 const unsigned int *__restrict__ bits,
                                                 uint8_t *__restrict__ dst, int kp, int grp,
                                                 int stride, int off) {
    __shared__ uint8_t tile[64][68];
    const int j0 = blockIdx.x * 64, p0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    float s = 0.f, inv = 0.f;
    if (MODE == 0) scale_from_bits(*bits, &s, &inv);
    for (int pp = ty; pp < 64; pp += 4) {
        int p = p0 + pp, j = j0 + tx;
        uint8_t b = 0x80;
        if (p < k && j < n) {
            int8_t q;
            if (MODE == 0) {
                float v = ((const float *)src)[(size_t)p * n + j];
                q = (s == 0.0f) ? (int8_t)0 : quant_one(v, inv);
            } else {
                q = ((const int8_t *)src)[(size_t)p * n + j];
            }
            b = (uint8_t)q ^ 0x80;
        }
        tile[pp][tx] = b;
    }
    __syncthreads();
    // each thread writes 4 consecutive k-bytes of one output row
    const int wx = threadIdx.x & 15, wy = threadIdx.x >> 4;
    for (int jj = wy; jj < 64; jj += 16) {
        int j = j0 + jj;
        int p = p0 + wx * 4;
        if (j >= n || p >= kp) continue;
        uint32_t v = (uint32_t)tile[wx * 4 + 0][jj] | ((uint32_t)tile[wx * 4 + 1][jj] << 8) |
                     ((uint32_t)tile[wx * 4 + 2][jj] << 16) | ((uint32_t)tile[wx * 4 + 3][jj] << 24);
        size_t r = (size_t)map_row(j, grp, stride, off);
        *(uint32_t *)(dst + r * kp + p) = v;  // kp % 16 == 0, p % 4 == 0
    }
}

// [n,k] source (rows are already output-major): 4 bytes per thread.
template <int MODE>
__global__ void k_pack_nk(const void *__restrict__ src, int k, int n,
                          const unsigned int *__restrict__ bits, uint8_t *__restrict__ dst, int kp,
                          int grp, int stride, int off) {
    float s = 0.f, inv = 0.f;
    if (MODE == 0) scale_from_bits(*bits, &s, &inv);
    const int words = kp / 4;
    size_t total = (size_t)n * words;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (size_t)gridDim.x * blockDim.x) {
        int j = (int)(t / words), p = (int)(t % words) * 4;
        uint32_t v = 0;
        for (int e = 0; e < 4; e++) {
            uint8_t b = 0x80;
            if (p + e < k) {
                int8_t q;
                if (MODE == 0) {
                    float x = ((const float *)src)[(size_t)j * k + p + e];
                    q = (s == 0.0f) ? (int8_t)0 : quant_one(x, inv);
                } else {
                    q = ((const int8_t *)src)[(size_t)j * k + p + e];
                }
                b = (uint8_t)q ^ 0x80;
            }
            v |= (uint32_t)b << (8 * e);
        }
        size_t r = (size_t)map_row(j, grp, stride, off);
        *(uint32_t *)(dst + r * kp + p) = v;
    }
}

__global__ void k_unpack(const uint8_t *__restrict__ src, int kp, int k, int n, int dst_nk, int grp,
                         int stride, int off, int8_t *__restrict__ q) {
    size_t total = (size_t)k * n;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (size_t)gridDim.x * blockDim.x) {
        int p, j;
        if (dst_nk) {
            j = (int)(t / k);
            p = (int)(t % k);
        } else {
            p = (int)(t / n);
            j = (int)(t % n);
        }
        size_t r = (size_t)map_row(j, grp, stride, off);
        q[t] = (int8_t)(src[r * kp + p] ^ 0x80);
    }
}

// block-32: one thread per (output j, k-block b); threads of a wave take
// consecutive j so [k,n] reads are coalesced.
__global__ void k_quant_block32(const float *__restrict__ w, int k, int n, int src_nk,
                                int8_t *__restrict__ q, float *__restrict__ scales) {
    const int nb = (k + 31) / 32;
    size_t total = (size_t)n * nb;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (size_t)gridDim.x * blockDim.x) {
        int b = (int)(t / n), j = (int)(t % n);
        int p0 = 32 * b, len = min(32, k - p0);
        float am = 0.f;
        for (int e = 0; e < len; e++) {
            size_t idx = src_nk ? (size_t)j * k + p0 + e : (size_t)(p0 + e) * n + j;
            am = fmaxf(am, fabsf(w[idx]));
        }
        float s = 0.f, inv = 0.f;
        if (am != 0.f) {
            s = am / 127.0f;
            inv = 1.0f / s;
        }
        for (int e = 0; e < len; e++) {
            size_t idx = src_nk ? (size_t)j * k + p0 + e : (size_t)(p0 + e) * n + j;
            q[idx] = (s == 0.f) ? (int8_t)0 : quant_one(w[idx], inv);
        }
        scales[(size_t)j * nb + b] = s;
    }
}

__global__ void k_scales_pack(const float *__restrict__ sc, int n, int nb, float *__restrict__ dst,
                              int grp, int stride, int off) {
    size_t total = (size_t)n * nb;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (size_t)gridDim.x * blockDim.x) {
        int j = (int)(t / nb), b = (int)(t % nb);
        dst[(size_t)map_row(j, grp, stride, off) * nb + b] = sc[t];
    }
}

__global__ void k_dequantize(const int8_t *__restrict__ q, size_t n, float scale,
                             float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __fmul_rn((float)q[i], scale);
}


// LlamaModel::new's N(mean, std) init (init.rs:2-9) on the device: sample i
// uses wyrand calls start+2i and start+2i+1 (the state is additive, so every
// sample is independent).  Box-Muller in f64 with the device libm; output i
// goes to out[(i / cols) * ld + col0 + i % cols] so fused layouts (qkv) can be
// written in place.
__global__ void k_normal_init(float *__restrict__ out, size_t n, uint64_t seed, uint64_t start,
                              float mean, float stdv, int cols, int ld, int col0) {
    const uint64_t W0 = 0x2d358dccaa6c78a5ULL, W1 = 0x8bb84b93962eacc9ULL;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t c = start + 2 * (uint64_t)i;
        double u[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint64_t s = seed + (c + 1 + t) * W0;
            const uint64_t y = s ^ W1;
            const uint64_t r = (s * y) ^ __umul64hi(s, y);
            u[t] = __longlong_as_double((long long)(0x3FF0000000000000ULL | (r >> 12))) - 1.0;
        }
        const double u1 = u[0] < 1e-30 ? 1e-30 : u[0];
        const double z = sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u[1]);
        const size_t row = i / (size_t)cols, col = i % (size_t)cols;
        out[row * (size_t)ld + col0 + col] = (float)((double)mean + (double)stdv * z);
    }
}

inline unsigned grid_for(size_t n, int per_block = 256, unsigned cap = 65536) {
    size_t g = (n + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

}  // namespace

int launch_absmax(const float *w, size_t n, unsigned int *d_absmax_bits, hipStream_t s) {
    SCRY_HIP(hipMemsetAsync(d_absmax_bits, 0, sizeof(unsigned int), s));
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_absmax, dim3(grid_for(n, 256 * 8, 4096)), dim3(256), 0, s, w, n,
                       d_absmax_bits);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_quantize_plain(const float *w, size_t n, const unsigned int *bits, int8_t *q,
                          float *d_scale, hipStream_t s) {
    hipLaunchKernelGGL(k_quantize_plain, dim3(grid_for(n)), dim3(256), 0, s, w, n, bits, q, d_scale);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_quant_pack(const float *w, int k, int n, int src_nk, const unsigned int *bits,
                      uint8_t *dst, int kp, int grp, int stride, int off, hipStream_t s) {
    if (src_nk) {
        hipLaunchKernelGGL(k_pack_nk<0>, dim3(grid_for((size_t)n * (kp / 4))), dim3(256), 0, s, w,
                           k, n, bits, dst, kp, grp, stride, off);
    } else {
        dim3 g((n + 63) / 64, (kp + 63) / 64);
        hipLaunchKernelGGL(k_pack_kn<0>, g, dim3(256), 0, s, w, k, n, bits, dst, kp, grp, stride,
                           off);
    }
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_i8_pack(const int8_t *q, int k, int n, int src_nk, uint8_t *dst, int kp, int grp,
                   int stride, int off, hipStream_t s) {
    if (src_nk) {
        hipLaunchKernelGGL(k_pack_nk<1>, dim3(grid_for((size_t)n * (kp / 4))), dim3(256), 0, s, q,
                           k, n, nullptr, dst, kp, grp, stride, off);
    } else {
        dim3 g((n + 63) / 64, (kp + 63) / 64);
        hipLaunchKernelGGL(k_pack_kn<1>, g, dim3(256), 0, s, q, k, n, nullptr, dst, kp, grp,
                           stride, off);
    }
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_unpack(const uint8_t *src, int kp, int k, int n, int dst_nk, int grp, int stride, int off,
                  int8_t *q, hipStream_t s) {
    hipLaunchKernelGGL(k_unpack, dim3(grid_for((size_t)k * n)), dim3(256), 0, s, src, kp, k, n,
                       dst_nk, grp, stride, off, q);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_quant_block32(const float *w, int k, int n, int src_nk, int8_t *q, float *scales,
                         hipStream_t s) {
    size_t total = (size_t)n * ((k + 31) / 32);
    hipLaunchKernelGGL(k_quant_block32, dim3(grid_for(total)), dim3(256), 0, s, w, k, n, src_nk, q,
                       scales);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_scales_pack(const float *scales, int n, int nb, float *dst, int grp, int stride, int off,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_scales_pack, dim3(grid_for((size_t)n * nb)), dim3(256), 0, s, scales, n,
                       nb, dst, grp, stride, off);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_normal_init(float *out, size_t n, uint64_t seed, uint64_t start_call, float mean,
                       float stdv, int cols, int ld, int col0, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_normal_init, dim3(grid_for(n, 256, 1u << 20)), dim3(256), 0, s, out, n,
                       seed, start_call, mean, stdv, cols, ld, col0);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_dequantize(const int8_t *q, size_t n, float scale, float *out, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_dequantize, dim3(grid_for(n)), dim3(256), 0, s, q, n, scale, out);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
