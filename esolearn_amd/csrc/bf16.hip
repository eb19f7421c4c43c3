// bf16 mode (the reference's `bf16` feature: init_gpu_bf16, cuda.rs:55-59;
// from_vec_with_bf16, mod.rs:28-32 / cuda.rs:149-175, 230-240; bf16_ops,
// cuda.rs:1201-1290; the bf16 kernels of kernels.rs:619-700).
//
// In bf16 mode a weight uploaded with from_vec_with_bf16 lives as bf16 only,
// and matmul rounds both operands to bf16 (products exact in f32) and
// accumulates in f32.  The kernels here:
//   - the reference's f32 -> bf16 cast (round to nearest even by adding
//     0x7fff + the lowest kept bit, 32-bit wrap-around included) and the
//     widening bf16 -> f32 (to_vec, embedding);
//   - the B operand of a matmul as bf16 rows [n][kp] (kp: k rounded up to 64,
//     zero padded), transposed through LDS tiles when B is stored [k][n];
//   - the activation plane of the MFMA GEMM (rows rounded to bf16, zero
//     padded);
//   - a GEMV for 1-16 activation rows over those bf16 rows: 16-byte weight
//     loads (8 bf16), 2 rows per wave, 2-4 k steps of 512 in flight, the
//     activations read from cache and rounded in the kernel.
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;
typedef unsigned short u16;

// kernels.rs:629-633 float_to_bf16
__device__ __forceinline__ u16 to_bf16(float x) {
    const unsigned b = __float_as_uint(x);
    return (u16)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float from_bf16(unsigned h) { return __uint_as_float(h << 16); }

// A model's f32 weight W[k, n] (or [n, k] when src_nk) as bf16 rows of the
// GEMV layout: output j -> packed row (j / grp) * stride + off + j % grp,
// kpe values per row (k, then zeros), each the reference's cast.  64 x 64
// tiles transpose through LDS so both the reads and the writes are coalesced.
__global__ __launch_bounds__(256) void k_pack_model_bf16(const float *__restrict__ w, int k, int n, int src_nk,
                                                         u16 *__restrict__ dst, int kpe, int grp, int stride,
                                                         int off) {
    __shared__ u16 tile[64][66];  // [p][j]
    const int j0 = blockIdx.x * 64, p0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        // src_nk: rows j, consecutive p; else rows p, consecutive j
        const int p = src_nk ? p0 + tx : p0 + i, j = src_nk ? j0 + i : j0 + tx;
        u16 v = 0;
        if (p < k && j < n) v = to_bf16(src_nk ? w[(size_t)j * k + p] : w[(size_t)p * n + j]);
        if (src_nk)
            tile[tx][i] = v;
        else
            tile[i][tx] = v;
    }
    __syncthreads();
    for (int jj = ty; jj < 64; jj += 4) {
        const int j = j0 + jj, p = p0 + tx;
        if (j >= n || p >= kpe) continue;
        const size_t row = (size_t)(j / grp) * stride + off + j % grp;
        dst[row * kpe + p] = tile[tx][jj];
    }
}

__global__ __launch_bounds__(256) void k_cast_bf16(const float *__restrict__ x, u16 *__restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) y[i] = to_bf16(x[i]);
}

// x -> the f32 value of its bf16 rounding
__global__ __launch_bounds__(256) void k_round_bf16(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        y[i] = from_bf16(to_bf16(x[i]));
}

__global__ __launch_bounds__(256) void k_widen_bf16(const u16 *__restrict__ x, float *__restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) y[i] = from_bf16(x[i]);
}

// kernels.rs:689-700 embedding_bf16_fwd
__global__ __launch_bounds__(256) void k_embed_bf16(float *__restrict__ out, const u16 *__restrict__ w,
                                                    const int64_t *__restrict__ ids, int n_ids, int dim) {
    const size_t total = (size_t)n_ids * dim;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t t = i / dim, d = i % dim;
        out[i] = from_bf16(w[(size_t)ids[t] * dim + d]);
    }
}

// B rows: pk[j][kk] = B(kk, j) as bf16 for kk < k, 0 for k <= kk < kp.
// tb = 0: B stored [k][n]; tb = 1: B stored [n][k].  Source bf16 (bs) or f32
// (fs, rounded).  32 x 32 tiles through LDS: grid (kp / 32, ceil(n / 32)).
__global__ __launch_bounds__(256) void k_pack_rows(const u16 *__restrict__ bs, const float *__restrict__ fs, int k,
                                                   int n, int tb, u16 *__restrict__ pk, int kp) {
    __shared__ u16 t[32][33];
    const int k0 = blockIdx.x * 32, j0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    auto src = [&](int kk, int j) -> u16 {
        if (kk >= k || j >= n) return 0;
        const size_t at = tb ? (size_t)j * k + kk : (size_t)kk * n + j;
        return bs ? bs[at] : to_bf16(fs[at]);
    };
    if (tb) {  // rows already along k: read and write along kk
        for (int r = ty; r < 32; r += 8) {
            const int j = j0 + r, kk = k0 + tx;
            if (j < n) pk[(size_t)j * kp + kk] = src(kk, j);
        }
        return;
    }
    for (int r = ty; r < 32; r += 8) t[r][tx] = src(k0 + r, j0 + tx);  // reads along j
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int j = j0 + r;
        if (j < n) pk[(size_t)j * kp + k0 + tx] = t[tx][r];  // writes along kk
    }
}

// GEMM activation plane: rows [rows][ldp] bf16, columns [k, kpad) zero
__global__ __launch_bounds__(256) void k_plane_bf16(const float *__restrict__ x, int ldx, int rows, int k, int kpad,
                                                    u16 *__restrict__ hi, int ldp) {
    const size_t total = (size_t)rows * kpad;
    for (size_t g = (size_t)blockIdx.x * 256 + threadIdx.x; g < total; g += (size_t)gridDim.x * 256) {
        const int r = (int)(g / kpad), j = (int)(g % kpad);
        hi[(size_t)r * ldp + j] = j < k ? to_bf16(x[(size_t)r * ldx + j]) : (u16)0;
    }
}

constexpr int GV_RW = 2, GV_NW = 4;  // rows per wave, waves

// y[m][n] = sum_k bf16(x[m][k]) * W[n][k] (+ bias[n]); W rows [n][kp] bf16.
// GV_U 512-wide k steps in flight (4 up to k = 8192, else 2: measured).
// Grid (ceil(n / 8), ceil(m / MT)).
template <int MT, int GV_U>
__global__ __launch_bounds__(64 * GV_NW) void k_gemv_bf16(const u16 *__restrict__ W, int kp, int n,
                                                          const float *__restrict__ x, int ldx, int k, int m,
                                                          float *__restrict__ y, int ldy,
                                                          const float *__restrict__ bias) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * GV_NW + wave) * GV_RW, m0 = blockIdx.y * MT;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(W, (size_t)n * kp * 2);
    unsigned woff[GV_RW];
#pragma unroll
    for (int r = 0; r < GV_RW; r++) woff[r] = (unsigned)((size_t)min(row0 + r, n - 1) * kp * 2) + (unsigned)(lane << 4);
    const bool vec = (ldx & 3) == 0;  // 16-byte activation loads
    float acc[MT][GV_RW];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int r = 0; r < GV_RW; r++) acc[mi][r] = 0.f;
    for (int k0 = 0; k0 < kp; k0 += 512 * GV_U) {
        u32x4 wv[GV_U][GV_RW];
#pragma unroll
        for (int u = 0; u < GV_U; u++) {
            const int kk = k0 + u * 512 + (lane << 3);
            // past the row: an offset beyond the buffer loads zeros
            const unsigned extra = kk < kp ? (unsigned)(k0 + u * 512) * 2 : 0x80000000u;
#pragma unroll
            for (int r = 0; r < GV_RW; r++) wv[u][r] = bload16(wr, woff[r] + extra);
        }
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            if (m0 + mi >= m) continue;  // the same for the whole workgroup
            const float *xr = x + (size_t)(m0 + mi) * ldx;
#pragma unroll
            for (int u = 0; u < GV_U; u++) {
                const int kk = k0 + u * 512 + (lane << 3);
                float xv[8];
                if (vec && kk + 8 <= k) {
                    const float4 a = *(const float4 *)(xr + kk), b = *(const float4 *)(xr + kk + 4);
                    xv[0] = a.x, xv[1] = a.y, xv[2] = a.z, xv[3] = a.w;
                    xv[4] = b.x, xv[5] = b.y, xv[6] = b.z, xv[7] = b.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) xv[e] = kk + e < k ? xr[kk + e] : 0.f;
                }
#pragma unroll
                for (int e = 0; e < 8; e++) xv[e] = from_bf16(to_bf16(xv[e]));
#pragma unroll
                for (int r = 0; r < GV_RW; r++) {
                    float s = acc[mi][r];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const unsigned wd = wv[u][r][q];
                        s = fmaf(xv[2 * q], __uint_as_float(wd << 16), s);
                        s = fmaf(xv[2 * q + 1], __uint_as_float(wd & 0xffff0000u), s);
                    }
                    acc[mi][r] = s;
                }
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
#pragma unroll
        for (int r = 0; r < GV_RW; r++) {
            const float s = wave_sum(acc[mi][r]);
            const int row = row0 + r;
            if (lane == r && m0 + mi < m && row < n) y[(size_t)(m0 + mi) * ldy + row] = bias ? s + bias[row] : s;
        }
    }
}

unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 8192); }

}  // namespace

int bf16_row_pad(int k) { return (k + 63) / 64 * 64; }

int launch_pack_model_bf16(const float *w, int k, int n, int src_nk, unsigned short *dst, int kpe, int grp,
                           int stride, int off, hipStream_t s) {
    dim3 g((n + 63) / 64, (kpe + 63) / 64);
    hipLaunchKernelGGL(k_pack_model_bf16, g, dim3(256), 0, s, w, k, n, src_nk, dst, kpe, grp, stride, off);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_cast_bf16(const float *x, size_t n, unsigned short *y, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_cast_bf16, dim3(grid_for(n)), dim3(256), 0, s, x, y, n);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_round_bf16(const float *x, size_t n, float *y, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_round_bf16, dim3(grid_for(n)), dim3(256), 0, s, x, y, n);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_widen_bf16(const unsigned short *x, size_t n, float *y, hipStream_t s) {
    if (n == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_widen_bf16, dim3(grid_for(n)), dim3(256), 0, s, x, y, n);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_embed_bf16(float *out, const unsigned short *w, const int64_t *ids, int n_ids, int dim, hipStream_t s) {
    const size_t total = (size_t)n_ids * dim;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_embed_bf16, dim3(grid_for(total)), dim3(256), 0, s, out, w, ids, n_ids, dim);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_pack_rows_bf16(const unsigned short *bs, const float *fs, int k, int n, int tb, unsigned short *pk,
                          int kp, hipStream_t s) {
    if (kp % 64 || kp < k || (!bs && !fs)) return set_error(SCRY_ERR_INVALID, "pack_rows_bf16: bad arguments");
    if (n <= 0 || k <= 0) return SCRY_OK;
    hipLaunchKernelGGL(k_pack_rows, dim3(kp / 32, (n + 31) / 32), dim3(256), 0, s, bs, fs, k, n, tb, pk, kp);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_plane_bf16(const float *x, int ldx, int rows, int k, int kpad, unsigned short *hi, int ldp,
                      hipStream_t s) {
    if (kpad > ldp || kpad < k) return set_error(SCRY_ERR_INVALID, "plane_bf16: bad stride");
    const size_t total = (size_t)rows * kpad;
    if (total == 0) return SCRY_OK;
    hipLaunchKernelGGL(k_plane_bf16, dim3(grid_for(total)), dim3(256), 0, s, x, ldx, rows, k, kpad, hi, ldp);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_gemv_bf16(const unsigned short *w, int kp, int n, const float *x, int ldx, int k, int m, float *y,
                     int ldy, const float *bias, hipStream_t s) {
    if (m <= 0 || n <= 0 || kp % 64 || kp < k || ldx < k) return set_error(SCRY_ERR_INVALID, "gemv_bf16: bad shape");
    if ((size_t)n * kp * 2 >= 0x7fffffffull) return set_error(SCRY_ERR_UNSUPPORTED, "gemv_bf16: weights above 2 GiB");
    const int rpb = GV_RW * GV_NW;
    const int mt = m >= 4 ? 4 : (m >= 2 ? 2 : 1);
    const dim3 grid((n + rpb - 1) / rpb, (m + mt - 1) / mt), blk(64 * GV_NW);
    const bool u4 = k <= 8192;
    if (mt == 4 && u4)
        hipLaunchKernelGGL((k_gemv_bf16<4, 4>), grid, blk, 0, s, w, kp, n, x, ldx, k, m, y, ldy, bias);
    else if (mt == 4)
        hipLaunchKernelGGL((k_gemv_bf16<4, 2>), grid, blk, 0, s, w, kp, n, x, ldx, k, m, y, ldy, bias);
    else if (mt == 2 && u4)
        hipLaunchKernelGGL((k_gemv_bf16<2, 4>), grid, blk, 0, s, w, kp, n, x, ldx, k, m, y, ldy, bias);
    else if (mt == 2)
        hipLaunchKernelGGL((k_gemv_bf16<2, 2>), grid, blk, 0, s, w, kp, n, x, ldx, k, m, y, ldy, bias);
    else if (u4)
        hipLaunchKernelGGL((k_gemv_bf16<1, 4>), grid, blk, 0, s, w, kp, n, x, ldx, k, m, y, ldy, bias);
    else
        hipLaunchKernelGGL((k_gemv_bf16<1, 2>), grid, blk, 0, s, w, kp, n, x, ldx, k, m, y, ldy, bias);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
