// Device-side helpers shared by the GEMV, attention and decode kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace scry {
namespace dev {

constexpr int TPB = 256;  // threads per workgroup (4 waves of 64)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 8 bf16 weights (little-endian pairs in w) times 8 activations: the bf16
// value is the upper half of its f32, so each product is exact in f32
__device__ __forceinline__ float dot8_bf16(u32x4 w, float4 x0, float4 x1, float acc) {
    acc = fmaf(x0.x, __uint_as_float(w.x << 16), acc);
    acc = fmaf(x0.y, __uint_as_float(w.x & 0xffff0000u), acc);
    acc = fmaf(x0.z, __uint_as_float(w.y << 16), acc);
    acc = fmaf(x0.w, __uint_as_float(w.y & 0xffff0000u), acc);
    acc = fmaf(x1.x, __uint_as_float(w.z << 16), acc);
    acc = fmaf(x1.y, __uint_as_float(w.z & 0xffff0000u), acc);
    acc = fmaf(x1.z, __uint_as_float(w.w << 16), acc);
    acc = fmaf(x1.w, __uint_as_float(w.w & 0xffff0000u), acc);
    return acc;
}

// The bf16 feature's cast (kernels.rs:629-633) as an f32 value: round to
// nearest even by adding 0x7fff plus the lowest kept bit to the f32 bits in
// 32-bit unsigned arithmetic, then drop the low half.
__device__ __forceinline__ float bf16_cast(float x) {
    const unsigned b = __float_as_uint(x);
    return __uint_as_float((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
}

__device__ __forceinline__ float dot16(u32x4 w, float4 x0, float4 x1, float4 x2, float4 x3,
                                       float acc) {
    acc = fmaf(x0.x, (float)(w.x & 0xffu), acc);
    acc = fmaf(x0.y, (float)((w.x >> 8) & 0xffu), acc);
    acc = fmaf(x0.z, (float)((w.x >> 16) & 0xffu), acc);
    acc = fmaf(x0.w, (float)(w.x >> 24), acc);
    acc = fmaf(x1.x, (float)(w.y & 0xffu), acc);
    acc = fmaf(x1.y, (float)((w.y >> 8) & 0xffu), acc);
    acc = fmaf(x1.z, (float)((w.y >> 16) & 0xffu), acc);
    acc = fmaf(x1.w, (float)(w.y >> 24), acc);
    acc = fmaf(x2.x, (float)(w.z & 0xffu), acc);
    acc = fmaf(x2.y, (float)((w.z >> 8) & 0xffu), acc);
    acc = fmaf(x2.z, (float)((w.z >> 16) & 0xffu), acc);
    acc = fmaf(x2.w, (float)(w.z >> 24), acc);
    acc = fmaf(x3.x, (float)(w.w & 0xffu), acc);
    acc = fmaf(x3.y, (float)((w.w >> 8) & 0xffu), acc);
    acc = fmaf(x3.z, (float)((w.w >> 16) & 0xffu), acc);
    acc = fmaf(x3.w, (float)(w.w >> 24), acc);
    return acc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// f64 wave sum over DPP row operations (no LDS permutes); the total is valid
// in lane 63 (returned to every lane by readlane)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(u & 0xffffffffu), CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(u >> 32), CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double wave_sum_d_dpp(double v) {
    v += dpp_d<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_d<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_d<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_d<0x140, 0xf>(v);  // row_mirror: every lane holds its row's sum
    v += dpp_d<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_d<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = __builtin_amdgcn_readlane((int)(u & 0xffffffffu), 63);
    const unsigned hi = __builtin_amdgcn_readlane((int)(u >> 32), 63);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// block-wide f64 sum (all 256 threads call it; result valid in every thread)
__device__ __forceinline__ double block_sum_d(double v, double *red) {
    v = wave_sum_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// Class of one term f64(a) * (f64(q) * f64(s)) of matmul_i8_f32
// (cpu.rs:1128-1160) with a non-finite activation a, from the stream byte
// b = q XOR 0x80: 1 = +inf, 2 = -inf, 4 = NaN (q s = 0 or a NaN).
__device__ __forceinline__ int nonfinite_term(float a, uint8_t b, float s) {
    const float t = a * ((float)(int)(signed char)(b ^ 0x80u) * s);
    return isnan(t) ? 4 : t > 0.f ? 1 : 2;
}
// The f32 sum of terms of these classes (finite terms cannot change it): NaN
// when a NaN term or both infinities occur, else the infinity.
__device__ __forceinline__ float nonfinite_value(int cls) {
    return (cls & 4) || cls == 3 ? __builtin_nanf("") : cls == 1 ? INFINITY : -INFINITY;
}
__device__ __forceinline__ int nonfinite_class(float v) { return isnan(v) ? 4 : v > 0.f ? 1 : 2; }

__device__ __forceinline__ float silu_f(float g) {
    double x = (double)g;  // cpu.rs:1119-1122: computed in f64, rounded once
    return (float)(x / (1.0 + exp(-x)));
}

// ---- ordered argmax (generate.rs:167-173: the last index among equal maxima)
struct ArgAcc {
    float v;
    int i;    // -1: empty
    int nan;  // largest NaN index seen, -1 if none
};

// Order-independent: the larger value, ties to the larger index (the last of
// equal maxima), the largest NaN index.  Accumulators over any partition of
// the indices combine in any order to the sequential scan's result.
__device__ __forceinline__ ArgAcc arg_combine(ArgAcc l, ArgAcc r) {
    ArgAcc o;
    if (l.i < 0)
        o = r;
    else if (r.i < 0)
        o = l;
    else
        o = (l.v > r.v || (l.v == r.v && l.i > r.i)) ? l : r;
    o.nan = max(l.nan, r.nan);
    return o;
}

// All 256 threads: reduction of per-thread accumulators over wave shuffles,
// then the four wave results through sh[0..3] (one barrier).  Result in every
// thread.
__device__ inline ArgAcc block_argmax(ArgAcc a, ArgAcc *sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        ArgAcc o;
        o.v = __shfl_down(a.v, off);
        o.i = __shfl_down(a.i, off);
        o.nan = __shfl_down(a.nan, off);
        if (lane + off < 64) a = arg_combine(a, o);
    }
    if (lane == 0) sh[wave] = a;
    __syncthreads();
    ArgAcc r = sh[0];
#pragma unroll
    for (int w = 1; w < TPB / 64; w++) r = arg_combine(r, sh[w]);
    __syncthreads();
    return r;
}

// sequential-semantics argmax over x[lo, hi) by the whole block
__device__ inline ArgAcc block_argmax_range(const float *x, int lo, int hi, ArgAcc *sh) {
    ArgAcc a{0.f, -1, -1};
    for (int i = lo + (int)threadIdx.x; i < hi; i += TPB) {  // coalesced; arg_combine is order-free
        float v = x[i];
        if (isnan(v)) {
            a.nan = i;
            continue;
        }
        if (a.i < 0 || !(a.v > v)) {
            a.v = v;
            a.i = i;
        }
    }
    return block_argmax(a, sh);
}

// Full generate.rs argmax semantics from a reduced accumulator over [0, n):
// with no NaN it is the last index of the maximum; with NaNs, max_by hands the
// running best to the element after the last NaN, so the answer is the argmax
// of the suffix after the last NaN (or that NaN if it is the last element).
__device__ inline int argmax_finish(ArgAcc r, const float *x, int n, ArgAcc *sh) {
    if (r.nan < 0) return r.i < 0 ? 0 : r.i;
    if (r.nan == n - 1) return r.nan;
    ArgAcc s = block_argmax_range(x, r.nan + 1, n, sh);
    return s.i;
}

// Step profile: workgroup b of a launch writes the 100 MHz constant clock to
// ts[2b] on entry and to ts[2b + 1] once all its waves are done (the host
// takes the earliest start and latest end of each launch).
__device__ __forceinline__ unsigned wg_linear_id() {
    return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
}
// Wave 0 stores (every lane the same value): a branch uniform in the wave,
// so the kernel's values derived from its arguments stay uniform.
__device__ __forceinline__ void wg_stamp_begin(unsigned long long *ts) {
    if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) == 0)
        ts[2 * wg_linear_id()] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void wg_stamp_end(unsigned long long *ts) {
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) == 0)
        ts[2 * wg_linear_id() + 1] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, size_t bytes) {
    const int n = bytes > 0x7fffffffu ? 0x7fffffff : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

// 16-byte buffer load; offsets at or past the resource size read as zero.
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}
__device__ __forceinline__ float4 bload16f(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}


// LDS float offset of the float4 holding x[p*1024 + 4t .. +3] in the permuted layout
__device__ __forceinline__ int xslot(int p, int t) { return (p << 10) | ((t & 3) << 8) | ((t >> 2) << 2); }

}  // namespace dev
}  // namespace scry
