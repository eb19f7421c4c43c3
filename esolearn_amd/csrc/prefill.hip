// Batched prefill for gfx950: LlamaModel::forward (llama.rs:683-700) with its
// attention (llama.rs:162-266), run over n_seq sequences of seq tokens at once
// so every projection is one GEMM on the matrix cores.  The K/V rows of the
// processed positions are appended to each sequence's KV cache, so decode can
// continue from them.
//
// GEMM numerics.  The reference accumulates f64(a) * f64(q * scale) into f32
// in k order (cpu.rs:1128-1160).  Two forms of the activations here:
//  - int8 per-tensor weights (every projection of an int8 model): each row of
//    activations as 24-bit fixed point, x = X 2^-E with E per row and
//    |x - X 2^-E| <= 2^-23 max|row|, X in three balanced int8 digits; the int8
//    matrix cores sum d q exactly in i32, and the epilogue forms the exact
//    integer dot product and rounds X.q 2^-E scale to f32 once
//    (k_norm_digits, k_gemm_digits);
//  - block-32 weights and bf16 weights: each f32 activation as two bf16
//    values hi = bf16(x), lo = bf16(x - hi) (|x - hi - lo| <= 2^-17 |x|), two
//    bf16 MFMAs per product accumulated in f32 (one for bf16 weights: the
//    reference's bf16 cast), scaled per output or per 32-wide k block.
// The differences from the reference are the activation rounding and the
// summation order, far inside the 1e-3 logit bar.
//
// Data layout.  GEMM inputs are [Mp][ld] planes (three int8 digit planes, or
// the bf16 hi and lo planes): Mp = rows rounded up to the M tile, ld = k
// rounded up to the k step (64); the columns past k are zero.  RMSNorm writes
// its planes directly; the attention and SwiGLU outputs, whose rows no single
// workgroup holds whole, go through f32 rows and a per-row pass into digit
// planes (bf16 planes directly for the other weight types).  Weights are the
// GEMV stream layout (one row of kp bytes per output, byte = q + 128), read
// as they are by the int8 matrix cores, converted to bf16 for the bf16 ones.
#include <cmath>

#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

typedef unsigned short u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define PF_LAUNCH_CHECK() SCRY_HIP(hipGetLastError()); return SCRY_OK

// hi = bf16(x), lo = bf16(x - hi) with the hardware round-to-nearest-even
// conversion: the bits of bf16_rn for every finite x (NaN stays NaN)
__device__ __forceinline__ void split_bf16(float x, u16 &hi, u16 &lo) {
    const __bf16 h = (__bf16)x;
    hi = __builtin_bit_cast(u16, h);
    lo = __builtin_bit_cast(u16, (__bf16)(x - (float)h));
}

// ------------------------------------------------------------------ RMSNorm
// cpu.rs:574-599 on the rows r*rstep + roff of x: rstd = 1/sqrt(mean(x^2)+eps)
// in f64, out = f32(x * rstd * w).  Writes the bf16 planes of row r (columns
// [k, ld) zeroed) and/or an f32 copy.
__global__ __launch_bounds__(256) void k_norm_split(const float *__restrict__ x, int ldx, int rstep, int roff,
                                                    const float *__restrict__ w, int k, float eps, u16 *hi,
                                                    u16 *lo, int ldp, int kpad, float *outf, int ldf) {
    __shared__ double red[4];
    const int r = blockIdx.x;
    const float *src = x + ((size_t)r * rstep + roff) * ldx;
    double ss = 0.0;
    for (int j = threadIdx.x; j < k; j += 256) ss += (double)src[j] * (double)src[j];
    const double rstd = 1.0 / sqrt(block_sum_d(ss, red) / (double)k + (double)eps);
    for (int j = threadIdx.x; j < kpad; j += 256) {
        const float v = j < k ? (float)((double)src[j] * rstd * (double)w[j]) : 0.f;
        if (hi) {
            u16 a, b;
            split_bf16(v, a, b);
            hi[(size_t)r * ldp + j] = a;
            lo[(size_t)r * ldp + j] = b;
        }
        if (outf && j < k) outf[(size_t)r * ldf + j] = v;
    }
}

// The same with 8 consecutive columns per thread and chunk, the row held in
// registers between the two passes, and 16-byte plane stores (k % 8 == 0,
// rows of x and w 16-byte aligned, planes only, NC = kpad / 2048 rounded up).
template <int NC>
__global__ __launch_bounds__(256) void k_norm_split8(const float *__restrict__ x, int ldx, int rstep, int roff,
                                                     const float *__restrict__ w, int k, float eps, u16 *hi,
                                                     u16 *lo, int ldp, int kpad) {
    __shared__ double red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    const float *src = x + ((size_t)r * rstep + roff) * ldx;
    float4 v[NC][2];
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int j = (c * 256 + t) * 8;
        v[c][0] = v[c][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < k) {
            v[c][0] = *(const float4 *)(src + j);
            v[c][1] = *(const float4 *)(src + j + 4);
        }
        const float e[8] = {v[c][0].x, v[c][0].y, v[c][0].z, v[c][0].w, v[c][1].x, v[c][1].y, v[c][1].z, v[c][1].w};
#pragma unroll
        for (int i = 0; i < 8; i++) ss += (double)e[i] * (double)e[i];
    }
    const double rstd = 1.0 / sqrt(block_sum_d(ss, red) / (double)k + (double)eps);
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int j = (c * 256 + t) * 8;
        if (j >= kpad) break;
        float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
        if (j < k) {
            w0 = *(const float4 *)(w + j);
            w1 = *(const float4 *)(w + j + 4);
        }
        const float e[8] = {v[c][0].x, v[c][0].y, v[c][0].z, v[c][0].w, v[c][1].x, v[c][1].y, v[c][1].z, v[c][1].w};
        const float g[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        unsigned ph[4], pl[4];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            u16 a0, b0, a1, b1;
            split_bf16(j + i < k ? (float)((double)e[i] * rstd * (double)g[i]) : 0.f, a0, b0);
            split_bf16(j + i + 1 < k ? (float)((double)e[i + 1] * rstd * (double)g[i + 1]) : 0.f, a1, b1);
            ph[i / 2] = (unsigned)a0 | ((unsigned)a1 << 16);
            pl[i / 2] = (unsigned)b0 | ((unsigned)b1 << 16);
        }
        *(u32x4 *)(hi + (size_t)r * ldp + j) = u32x4{ph[0], ph[1], ph[2], ph[3]};
        *(u32x4 *)(lo + (size_t)r * ldp + j) = u32x4{pl[0], pl[1], pl[2], pl[3]};
    }
}

// RMSNorm into digit planes (the input of the int8 GEMM, k_gemm_digits):
// the same normalised row y as k_norm_split, then per row an exponent E with
// max|y| 2^E <= 2^23 - 2^16 - 1, X = rint(y 2^E) (exact scaling in f64, one
// rounding: |y - X 2^-E| <= 2^-E-1 <= 2^-23 max|y|), and X = d0 + 2^8 d1 +
// 2^16 d2 in balanced digits (d0, d1 in [-128, 127]; the bound keeps d2 in
// [-127, 127]).  A row holding a NaN or an infinity gets E = DG_NONFINITE
// and the GEMM writes NaN for it, as the split planes do (lo = bf16(inf - inf)).
// Thread t holds columns 8 (c 256 + t) .. +7 of chunk c; VEC: 16-byte loads
// (k % 8 == 0, rows 16-byte aligned).  NORM false: the rows as they are (y = x;
// w and eps unused), for GEMM inputs that no single kernel holds whole rows of.
constexpr int DG_NONFINITE = 0x7fffffff;
constexpr double DG_XMAX = 8323071.0;  // 2^23 - 2^16 - 1

template <int NC, bool VEC, bool NORM>
__global__ __launch_bounds__(256) void k_norm_digits(const float *__restrict__ x, int ldx, const float *__restrict__ w,
                                                     int k, float eps, signed char *dg, size_t dstride, int *de,
                                                     int ldp, int kpad) {
    __shared__ double red[4];
    __shared__ float s_max[4];
    __shared__ int s_bad[4];
    const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const float *src = x + (size_t)r * ldx;
    float y[NC][8];
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int j = (c * 256 + t) * 8;
        if (VEC) {
            float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
            if (j < k) {
                v0 = *(const float4 *)(src + j);
                v1 = *(const float4 *)(src + j + 4);
            }
            y[c][0] = v0.x, y[c][1] = v0.y, y[c][2] = v0.z, y[c][3] = v0.w;
            y[c][4] = v1.x, y[c][5] = v1.y, y[c][6] = v1.z, y[c][7] = v1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) y[c][i] = j + i < k ? src[j + i] : 0.f;
        }
        if (NORM) {
#pragma unroll
            for (int i = 0; i < 8; i++) ss += (double)y[c][i] * (double)y[c][i];
        }
    }
    const double rstd = NORM ? 1.0 / sqrt(block_sum_d(ss, red) / (double)k + (double)eps) : 1.0;
    float amax = 0.f;
    int bad = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int j = (c * 256 + t) * 8;
        float g[8];
        if (NORM && VEC) {
            float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
            if (j < k) {
                w0 = *(const float4 *)(w + j);
                w1 = *(const float4 *)(w + j + 4);
            }
            g[0] = w0.x, g[1] = w0.y, g[2] = w0.z, g[3] = w0.w, g[4] = w1.x, g[5] = w1.y, g[6] = w1.z, g[7] = w1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) g[i] = NORM && j + i < k ? w[j + i] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float v = j + i >= k ? 0.f : NORM ? (float)((double)y[c][i] * rstd * (double)g[i]) : y[c][i];  // cpu.rs:574-599
            y[c][i] = v;
            amax = fmaxf(amax, fabsf(v));
            bad |= !isfinite(v);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off));
        bad |= __shfl_xor(bad, off);
    }
    if (lane == 0) s_max[wv] = amax, s_bad[wv] = bad;
    __syncthreads();
    amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    bad = s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3];
    int E = 0;
    if (bad) {
        E = DG_NONFINITE;
    } else if (amax > 0.f) {
        int ex;
        frexpf(amax, &ex);  // amax = m 2^ex, m in [0.5, 1)
        E = 23 - ex;
        if (ldexp((double)amax, E) > DG_XMAX) E--;
    }
    const int Es = bad ? 0 : E;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int j = (c * 256 + t) * 8;
        if (j >= kpad) break;
        unsigned b[3][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // y 2^E is exact in f32 (a power-of-two scaling to at most 2^23), rint then exact
            const int X = bad ? 0 : (int)rintf(ldexpf(y[c][i], Es));
            // balanced digits: d0 = sext8(X), d1 = sext8(X1), d2 = X2 with X1 = (X - d0) / 2^8, X2 = (X1 - d1) / 2^8
            const int X1 = (X - (int)(signed char)X) >> 8;
            const int X2 = (X1 - (int)(signed char)X1) >> 8;
            const int sh = 8 * (i & 3);
            b[0][i >> 2] |= (unsigned)(X & 255) << sh;
            b[1][i >> 2] |= (unsigned)(X1 & 255) << sh;
            b[2][i >> 2] |= (unsigned)(X2 & 255) << sh;
        }
#pragma unroll
        for (int pl = 0; pl < 3; pl++)
            *(uint2 *)(dg + pl * dstride + (size_t)r * ldp + j) = make_uint2(b[pl][0], b[pl][1]);
    }
    if (t == 0) de[r] = E;
}

// f32 rows -> bf16 planes (columns [k, kpad) zeroed)
__global__ void k_split(const float *__restrict__ x, int ldx, int rows, int k, int kpad, u16 *hi, u16 *lo, int ldp) {
    const size_t total = (size_t)rows * kpad;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(g / kpad), j = (int)(g % kpad);
        u16 a = 0, b = 0;
        if (j < k) split_bf16(x[(size_t)r * ldx + j], a, b);
        hi[(size_t)r * ldp + j] = a;
        lo[(size_t)r * ldp + j] = b;
    }
}

// ------------------------------------------------------------------ GEMM
// C[m][n] = sum_k (hi + lo)[m][k] * q[n][k], q the int8 weight of output n.
// Workgroup tile BM x BN, k step BK; 4 waves in 2 x 2, each 64 x 128 as 4 x 8
// tiles of v_mfma_f32_16x16x32_bf16.  Operand lane layouts of that
// instruction (16 x 32 A, 32 x 16 B, 16 x 16 D): lane l holds
// A[l % 16][8 (l / 16) + e] and B[8 (l / 16) + e][l % 16] for e = 0..7, and
// D[4 (l / 16) + r][l % 16] for r = 0..3.
// One LDS stage (the next k step is held in registers while the current one
// is consumed) keeps a workgroup at ~75 KB, so two fit on a CU: two waves per
// SIMD hide each other's LDS and barrier latency (measured: 45-48% of the
// bf16 issue rate, against 29-35% for a double-buffered stage at one wave
// per SIMD).
constexpr int BM = 128, BN = 256, BK = 64;
constexpr int LDT = BK + 8;  // LDS row stride in bf16 (144 B): 16-byte row reads hit distinct banks
constexpr int G_THREADS = 256;
constexpr size_t A_TILE = (size_t)BM * LDT, B_TILE = (size_t)BN * LDT;  // u16 elements
constexpr int AC = BM * BK / 8 / G_THREADS;   // 16-byte A chunks per thread and plane
// dynamic LDS: A hi, A lo, B + [BK/32][BN] block-32 scales
constexpr size_t GEMM_LDS = (2 * A_TILE + B_TILE) * sizeof(u16) + (BK / 32) * BN * sizeof(float);
static_assert(GEMM_LDS >= 2 * BM * (BN / 2 + 8) * sizeof(u16), "SwiGLU staging tile");

enum { GE_STORE = PF_STORE, GE_RESID = PF_RESID, GE_SWIGLU = PF_SWIGLU };

struct GemmP {
    const u16 *ahi, *alo;
    int lda;
    const uint8_t *w;
    int kp, N;
    const float *s32;  // block-32 scales [N][nb] (packed-row order) or null
    int nb;
    int M, nk;         // rows, k steps (k rounded up to 32, / 32)
    int n_mb, n_nb;    // tiles along M and N
    int n_super;       // super-tiles (4 M tiles x 8 N tiles)
    float scale, scale2;
    const float *bias;  // GE_STORE: + bias[n] (f32, after scaling)
    float *c;
    int ldc;
    u16 *ohi, *olo;
    int ldo, opad;     // SwiGLU planes: row stride, columns written (with zero pad)
    const signed char *ad;  // digit planes [3][.][lda] (k_gemm_digits), plane stride dstride bytes
    const int *ae;          // row exponents
    size_t dstride;
    float *of;              // SwiGLU output as f32 rows [M][ldo] instead of the planes (k_gemm_digits)
};

// Workgroup -> tile: workgroup b runs on XCD b % 8.  Tiles are grouped in
// super-tiles of 4 M tiles x 8 N tiles; an XCD works through whole
// super-tiles, so the workgroups it runs together share A rows and weight
// rows in its L2.
__device__ __forceinline__ bool gemm_tile(const GemmP &p, int &mb, int &nb) {
    const int b = blockIdx.x, xcd = b & 7, loc = b >> 3;
    const int sup = (loc >> 5) * 8 + xcd, in = loc & 31;
    if (sup >= p.n_super) return false;
    const int n_msup = (p.n_mb + 3) >> 2;
    mb = (sup % n_msup) * 4 + (in & 3);
    nb = (sup / n_msup) * 8 + (in >> 2);
    return mb < p.n_mb && nb < p.n_nb;
}

// 16 weight bytes (q + 128) -> 16 bf16 of q, as 8 words.  Flipping bit 7
// gives q's two's-complement byte; |q| <= 128 is exact in bf16
// (v_cvt_f32_i32 on the sign-extended byte, then v_cvt_pk_bf16_f32).
__device__ __forceinline__ void bytes_to_bf16(u32x4 v, u32x4 &o0, u32x4 &o1) {
    bf16x8 r0, r1;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r0[j] = (__bf16)(float)(int)(signed char)((v.x ^ 0x80808080u) >> (8 * j));
        r0[4 + j] = (__bf16)(float)(int)(signed char)((v.y ^ 0x80808080u) >> (8 * j));
        r1[j] = (__bf16)(float)(int)(signed char)((v.z ^ 0x80808080u) >> (8 * j));
        r1[4 + j] = (__bf16)(float)(int)(signed char)((v.w ^ 0x80808080u) >> (8 * j));
    }
    o0 = __builtin_bit_cast(u32x4, r0);
    o1 = __builtin_bit_cast(u32x4, r1);
}

// GEMM epilogue for a wave's TM x TN tiles of 16 x 16, D[4 (l / 16) + r][l % 16]
// of each tile at rows mw + 16 tm, columns nw + 16 tn; s_a / s_b scale the
// gate / up halves (s_a alone otherwise).
// lane value of the lane l ^ 2 / l ^ 1 (quad permutes, no LDS traffic)
__device__ __forceinline__ float quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
}
__device__ __forceinline__ int quad_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false); }

// GEMM epilogue for a wave's TM x TN tiles of 16 x 16, D[4 (l / 16) + r][l % 16]
// of each tile at rows mw + 16 tm, columns nw + 16 tn; s_a / s_b scale the
// gate / up halves (s_a alone otherwise).
template <int EPI, int TM, int TN>
__device__ __forceinline__ void gemm_store(const GemmP &p, const f32x4 (&acc)[TM][TN], int mw, int nw, int lane,
                                           float s_a, float s_b) {
    const int fr = lane & 15;
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int n = nw + tn * 16 + fr;
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
            if (EPI == GE_SWIGLU) {
                // fused gate/up rows of a group of 4: gate[2t], gate[2t+1],
                // up[2t], up[2t+1] in lanes 4q .. 4q+3.  Rows are taken in pairs
                // (r0, r1) so that every lane evaluates one SiLU: the gate lanes
                // form output row r0 (their gate, the up lane's r0 value), the up
                // lanes output row r1 (the gate lane's r1 value, their up); lanes
                // 4q and 4q+2 then store columns 2t, 2t+1 of their row as one
                // 32-bit word per plane
                const bool gate = (n & 2) == 0;
                const float sc = gate ? s_a : s_b;
#pragma unroll
                for (int rp = 0; rp < 2; rp++) {
                    const float v0 = acc[tm][tn][2 * rp] * sc, v1 = acc[tm][tn][2 * rp + 1] * sc;
                    const float recv = quad_xor2(gate ? v1 : v0);
                    const float gv = gate ? v0 : recv, uv = gate ? recv : v1;
                    u16 a, b;
                    split_bf16(silu_f(gv) * uv, a, b);  // cpu.rs:666-678
                    const unsigned hw = (unsigned)a | ((unsigned)quad_xor1((int)a) << 16);
                    const unsigned lw = (unsigned)b | ((unsigned)quad_xor1((int)b) << 16);
                    const int m = mw + tm * 16 + ((lane >> 4) << 2) + 2 * rp + (gate ? 0 : 1);
                    if ((n & 1) == 0 && m < p.M && n < p.N) {  // N is a multiple of 4
                        const size_t at = (size_t)m * p.ldo + ((n >> 2) << 1);
                        *(unsigned *)(p.ohi + at) = hw;
                        *(unsigned *)(p.olo + at) = lw;
                    }
                }
            }
        }
        if (EPI != GE_SWIGLU) {
            // this column's residual values (or bias) are all requested before the
            // first store: the compiler cannot tell the stores from later loads of
            // c apart, and would otherwise wait out one round trip per element
            const bool nok = n < p.N;
            const float bn = EPI == GE_STORE && p.bias && nok ? p.bias[n] : 0.f;  // cpu.rs:553-570
            float res[TM][4];
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = mw + tm * 16 + ((lane >> 4) << 2) + r;
                    res[tm][r] = EPI == GE_RESID && nok && m < p.M ? p.c[(size_t)m * p.ldc + n] : 0.f;
                }
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = mw + tm * 16 + ((lane >> 4) << 2) + r;
                    if (nok && m < p.M) {
                        const float v = acc[tm][tn][r] * s_a;
                        // cpu.rs:104-113 add
                        p.c[(size_t)m * p.ldc + n] = EPI == GE_RESID ? res[tm][r] + v : (EPI == GE_STORE && p.bias ? v + bn : v);
                    }
                }
        }
    }
}

// SwiGLU epilogue through LDS.  The MFMA layout leaves each lane one column
// of 4 rows, so direct plane stores are 4-byte pieces of 8 rows per
// instruction; instead each wave puts its outputs (one SiLU per lane and row
// pair, as in gemm_store) into an LDS tile [BM][BN / 2] per plane, and the
// workgroup then writes whole 256-byte plane rows with 16-byte stores.  The
// caller's LDS is free (no loads in flight, every wave past its last read);
// so (>= 2 BM (BN / 2 + 8) u16) holds the tile.  Rows past M are not written
// (they stay zero); columns past N / 2 neither.
// SiLU in f32 for outputs that become digit planes (each row to 2^-23 of
// its largest value) or split-bf16 planes (hi + lo hold x to 2^-17): the f32
// evaluation is within a few 2^-24 of the reference's f64 one
// (cpu.rs:1119-1122), so the planes agree with the f64 path's to their own
// bound, at a quarter of the cost.  Where the next GEMM reads
// one bf16 plane (the bf16 model: the reference's bf16 cast of the f32
// value), the f64 evaluation is kept, since one ulp of f32 can move a bf16
// rounding.
__device__ __forceinline__ float silu_split(float g) { return g / (1.f + expf(-g)); }

template <int TM, int TN, int NT, bool EXACT>
__device__ __forceinline__ void swiglu_store(const GemmP &p, const f32x4 (&acc)[TM][TN], u16 *so, int ml, int nl, int m0,
                                             int n0, int lane) {
    constexpr int OW = BN / 2, LDO = OW + 8;  // output columns per tile; LDS row stride (u16)
    constexpr int LDF = OW + 4;               // the same in f32 (p.of: f32 rows instead of planes)
    u16 *sh = so, *sl = so + BM * LDO;
    float *sf = reinterpret_cast<float *>(so);
    const int fr = lane & 15;
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int n = nl + tn * 16 + fr;  // tile column (n0 is a multiple of 4)
        const bool gate = (n & 2) == 0;
        const float sc = gate ? p.scale : p.scale2;
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
#pragma unroll
            for (int rp = 0; rp < 2; rp++) {
                const float v0 = acc[tm][tn][2 * rp] * sc, v1 = acc[tm][tn][2 * rp + 1] * sc;
                const float recv = quad_xor2(gate ? v1 : v0);
                const float gv = gate ? v0 : recv, uv = gate ? recv : v1;
                const float o = (EXACT ? silu_f(gv) : silu_split(gv)) * uv;  // cpu.rs:666-678
                const int r = ml + tm * 16 + ((lane >> 4) << 2) + 2 * rp + (gate ? 0 : 1);
                if (p.of) {
                    const float po = __int_as_float(quad_xor1(__float_as_int(o)));
                    if ((n & 1) == 0) *(float2 *)(sf + r * LDF + ((n >> 2) << 1)) = make_float2(o, po);
                } else {
                    u16 a, b;
                    split_bf16(o, a, b);
                    const unsigned hw = (unsigned)a | ((unsigned)quad_xor1((int)a) << 16);
                    const unsigned lw = (unsigned)b | ((unsigned)quad_xor1((int)b) << 16);
                    if ((n & 1) == 0) {
                        const int at = r * LDO + ((n >> 2) << 1);
                        *(unsigned *)(sh + at) = hw;
                        *(unsigned *)(sl + at) = lw;
                    }
                }
            }
        }
    }
    __syncthreads();
    const int oc0 = n0 >> 1, ocn = p.N >> 1;
    if (p.of) {  // f32 rows: 4 columns per 16-byte store
        constexpr int CPF = OW / 4;
        for (int idx = threadIdx.x; idx < BM * CPF; idx += NT) {
            const int r = idx / CPF, c = idx - r * CPF;
            const int m = m0 + r, col = oc0 + c * 4;
            if (m >= p.M || col >= ocn) continue;
            const float *src = sf + r * LDF + c * 4;
            float *dst = p.of + (size_t)m * p.ldo + col;
            if (col + 4 <= ocn) {
                *(float4 *)dst = *(const float4 *)src;
            } else {
                for (int e = 0; e < ocn - col; e++) dst[e] = src[e];
            }
        }
        return;
    }
    constexpr int CPR = OW / 8;  // 16-byte chunks per row
    for (int idx = threadIdx.x; idx < 2 * BM * CPR; idx += NT) {
        const int pl = idx / (BM * CPR), rem = idx - pl * (BM * CPR), r = rem / CPR, c = rem - r * CPR;
        const int m = m0 + r, col = oc0 + c * 8;
        if (m >= p.M || col >= ocn) continue;
        const u16 *src = (pl ? sl : sh) + r * LDO + c * 8;
        u16 *dst = (pl ? p.olo : p.ohi) + (size_t)m * p.ldo + col;
        if (col + 8 <= ocn) {
            *(u32x4 *)dst = *(const u32x4 *)src;
        } else {
            for (int e = 0; e < ocn - col; e++) dst[e] = src[e];
        }
    }
}

// zero the plane columns past the SwiGLU output (k padding of the next GEMM),
// rows [m0, m0 + BM); one wave of the last column tile
__device__ __forceinline__ void swiglu_pad(const GemmP &p, int m0, int lane) {
    const int c0 = p.N >> 1;
    for (int idx = lane; idx < BM * (p.opad - c0); idx += 64) {
        const int m = m0 + idx / (p.opad - c0), col = c0 + idx % (p.opad - c0);
        p.ohi[(size_t)m * p.ldo + col] = 0;
        p.olo[(size_t)m * p.ldo + col] = 0;
    }
}

// (block-32: the per-block scaling needs a second accumulator tile, so one
// workgroup per CU keeps it in registers)
// WBF: bf16 weight rows [N][kp] (2 bytes each, copied to LDS as they are) and
// a single bf16 activation plane (bf16 mode: both operands rounded to bf16,
// products exact, f32 accumulation); p.alo is not read.
template <int EPI, bool B32, bool WBF = false>
__global__ __launch_bounds__(G_THREADS, B32 ? 1 : 2) void k_gemm(GemmP p) {
    static_assert(!(WBF && B32), "bf16 weights carry no block scales");
    extern __shared__ float4 gsm[];
    u16 *sa = reinterpret_cast<u16 *>(gsm);
    u16 *sb = sa + 2 * A_TILE;
    float *s_sc = reinterpret_cast<float *>(sb + B_TILE);  // [BK/32][BN]
    int mb, nbk;
    if (!gemm_tile(p, mb, nbk)) return;
    const int m0 = mb * BM, n0 = nbk * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // global -> LDS assignment: A chunk c = tid + 256 i (row c / (BK/8), 8 bf16
    // at 8 (c % (BK/8))); B chunk c = tid + 256 i (row c / (BK/16), 16 bytes at
    // 16 (c % (BK/16)))
    constexpr int CPR = BK / 8, BPR = WBF ? BK / 8 : BK / 16;  // 16-byte chunks per row
    constexpr int BCW = BN * BPR / G_THREADS;                    // weight chunks per thread
    constexpr int NPL = WBF ? 1 : 2;                             // activation planes
    constexpr unsigned WB = WBF ? 2 : 1;                         // bytes per weight
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (size_t)p.N * p.kp * WB);
    const u16 *ga[2][AC];
    unsigned boff[BCW];
#pragma unroll
    for (int i = 0; i < AC; i++) {
        const int c = tid + 256 * i;
        ga[0][i] = p.ahi + (size_t)(m0 + c / CPR) * p.lda + (c % CPR) * 8;
        ga[1][i] = WBF ? ga[0][i] : p.alo + (size_t)(m0 + c / CPR) * p.lda + (c % CPR) * 8;
    }
#pragma unroll
    for (int i = 0; i < BCW; i++) {
        const int c = tid + 256 * i;
        const int n = n0 + c / BPR;
        boff[i] = n < p.N ? (unsigned)((size_t)n * p.kp * WB + (c % BPR) * 16) : 0x80000000u;
    }
    const bool s_ld = B32 && n0 + tid < p.N;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(p.s32, B32 ? (size_t)p.N * p.nb * sizeof(float) : 0);

    u32x4 ra[2][AC], rb[BCW];
    float rs[BK / 32];
    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int pl = 0; pl < NPL; pl++)
#pragma unroll
            for (int i = 0; i < AC; i++) ra[pl][i] = *(const u32x4 *)(ga[pl][i] + k0);
#pragma unroll
        for (int i = 0; i < BCW; i++) rb[i] = bload16(wr, boff[i] + (unsigned)k0 * WB);
        if (B32) {
#pragma unroll
            for (int j = 0; j < BK / 32; j++)  // blocks past the scales read as 0 (their A is 0)
                rs[j] = s_ld ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                             sr, (int)(((n0 + tid) * p.nb + kt * (BK / 32) + j) * 4), 0, 0))
                             : 0.f;
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int pl = 0; pl < NPL; pl++)
#pragma unroll
            for (int i = 0; i < AC; i++) {
                const int c = tid + 256 * i;
                *(u32x4 *)(sa + pl * A_TILE + (c / CPR) * LDT + (c % CPR) * 8) = ra[pl][i];
            }
#pragma unroll
        for (int i = 0; i < BCW; i++) {
            const int c = tid + 256 * i;
            if constexpr (WBF) {
                *(u32x4 *)(sb + (c / BPR) * LDT + (c % BPR) * 8) = rb[i];
            } else {
                u32x4 o0, o1;
                bytes_to_bf16(rb[i], o0, o1);
                u16 *d = sb + (c / BPR) * LDT + (c % BPR) * 16;
                *(u32x4 *)d = o0;
                *(u32x4 *)(d + 8) = o1;
            }
        }
        if (B32) {
#pragma unroll
            for (int j = 0; j < BK / 32; j++) s_sc[j * BN + tid] = rs[j];
        }
    };

    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    gload(0);
    lstore();
    __syncthreads();
    const int fr = lane & 15, fk = (lane >> 4) << 3;
    for (int kt = 0; kt < p.nk; kt++) {
        if (kt + 1 < p.nk) gload(kt + 1);  // in flight while this step is consumed
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            bf16x8 ah[4], al[4];
#pragma unroll
            for (int tm = 0; tm < 4; tm++) {
                const int r = wm * 64 + tm * 16 + fr;
                ah[tm] = *(const bf16x8 *)(sa + r * LDT + ks * 32 + fk);
                if (!WBF) al[tm] = *(const bf16x8 *)(sa + A_TILE + r * LDT + ks * 32 + fk);
            }
#pragma unroll
            for (int tn = 0; tn < 8; tn++) {
                const int cn = wn * 128 + tn * 16 + fr;
                const bf16x8 bv = *(const bf16x8 *)(sb + cn * LDT + ks * 32 + fk);
                if (B32) {
                    const float sc = s_sc[ks * BN + cn];
#pragma unroll
                    for (int tm = 0; tm < 4; tm++) {
                        f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
                        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bv, t, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bv, t, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[tm][tn][r] = fmaf(sc, t[r], acc[tm][tn][r]);
                    }
                } else {
#pragma unroll
                    for (int tm = 0; tm < 4; tm++) {
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bv, acc[tm][tn], 0, 0, 0);
                        if (!WBF)
                            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bv, acc[tm][tn], 0, 0, 0);
                    }
                }
            }
        }
        if (kt + 1 < p.nk) {
            __syncthreads();  // every wave is done with this step's LDS
            lstore();
        }
        __syncthreads();
    }

    // ---- epilogue: D[4 (l / 16) + r][l % 16] of each tile
    if (EPI == GE_SWIGLU && !B32) {  // (the last k step ended with a barrier: LDS is free)
        swiglu_store<4, 8, G_THREADS, WBF>(p, acc, sa, wm * 64, wn * 128, m0, n0, lane);
        if (wave == 0 && nbk == p.n_nb - 1) swiglu_pad(p, m0, lane);
    } else {
        gemm_store<EPI, 4, 8>(p, acc, m0 + wm * 64, n0 + wn * 128, lane, B32 ? 1.f : p.scale, B32 ? 1.f : p.scale2);
        if (EPI == GE_SWIGLU && wave == 0 && nbk == p.n_nb - 1) swiglu_pad(p, m0, lane);
    }
}

// ------------------------------------------------------------------ GEMM, direct-to-LDS ring
// The int8 per-tensor GEMM (every projection of an int8 model).  Same tile
// (128 x 256), numerics and epilogues as k_gemm; the staging differs:
//  - activations and weights go from memory straight into LDS (buffer loads
//    with the LDS destination: M0 = the 1 KB block, lane i writes its 16 bytes
//    at 16 i), through a ring of 3 k steps, so two steps are in flight while
//    one is consumed and no register holds staged data;
//  - the weights stay int8 in LDS (half the bytes of bf16) and each wave
//    converts the 16 bytes it reads (two MFMA k halves) after the read;
//  - one barrier per k step: a step's slot is refilled only after every wave
//    has passed the barrier that follows its last read.
// 8 waves (2 along M x 4 along N) of 64 x 64 outputs; 144 KB of LDS, one
// workgroup per CU.  Measured on the config-5 shapes against k_gemm (same box,
// same run): qkv 811 -> 728 us, gate/up 3129 -> 3045 us, down 1754 -> 1594 us,
// and a higher clock under the power limit.
//
// LDS step layout: hi plane [128 rows][128 B], lo plane likewise, weights
// [256 columns][64 B].  16-byte chunks are XOR-swizzled so the MFMA operand
// reads (16 rows of one chunk per 16 lanes) hit distinct banks: activation
// chunk c of row r sits at c ^ (r & 7), weight chunk c of column n at
// c ^ ((n >> 1) & 3).  MFMA k order within a step: lane group g of the
// 16x16x32 MFMA holds k = 16 g + 8 h + e for k half h, e < 8, which makes
// the weight operand of both halves one 16-byte read per lane.
namespace ring {
constexpr int WGM = 2, WGN = 4, TM = 4, TN = 4, NW = WGM * WGN, T = 64 * NW, S = 3;
static_assert(WGM * TM * 16 == BM && WGN * TN * 16 == BN && BK == 64, "ring tile");
// WBF: bf16 weight rows (128 B per column and step, read as they are) and
// one activation plane (the bf16 model); else int8 weights and hi, lo planes
template <bool WBF>
struct Lay {
    static constexpr int NPL = WBF ? 1 : 2, WB = WBF ? 2 : 1;  // activation planes; bytes per weight
    static constexpr int A_PL = BM * BK * 2, B_ST = BN * BK * WB, STAGE = NPL * A_PL + B_ST;
    static constexpr int JA = A_PL / 1024 / NW, JB = B_ST / 1024 / NW;  // 1 KB loads per wave and step
    static constexpr int L = NPL * JA + JB;
    static_assert((A_PL / 1024) % NW == 0 && (B_ST / 1024) % NW == 0, "ring units");
    static constexpr size_t LDS = (size_t)S * STAGE;
    static_assert(L * (S - 2) < 64, "vmcnt range");
    static_assert(LDS >= 2 * BM * (BN / 2 + 8) * sizeof(u16), "SwiGLU staging tile");
};
}  // namespace ring

// buffer descriptor words (base, stride 0, num_records, raw-buffer flags),
// wave-uniform
__device__ __forceinline__ u32x4 ring_desc(const void *base, size_t bytes) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const unsigned n = bytes > 0x7fffffffu ? 0x7fffffffu : (unsigned)bytes;
    u32x4 d = u32x4{(unsigned)b, (unsigned)(b >> 32) & 0xffffu, n, 0x00020000u};
#pragma unroll
    for (int i = 0; i < 4; i++) d[i] = __builtin_amdgcn_readfirstlane(d[i]);
    return d;
}

// 64 lanes x 16 bytes of buffer d at voff + soff -> LDS [lds, lds + 1024).
// The compiler does not see this load: callers wait with ring_wait before
// reading the LDS it fills (a vmcnt wait it cannot misplace), and M0 is
// restored.  Every lane's address stays inside the buffer's records or reads
// zero; no load is out of bounds for every lane (those can complete out of
// order and break partial vmcnt waits).
__device__ __forceinline__ void ring_load(u32x4 d, unsigned lds, unsigned voff, unsigned soff) {
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(d), "s"(soff)
        : "memory");
}
template <int N>
__device__ __forceinline__ void ring_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
// workgroup barrier without a memory fence (a fence would also wait for the
// ring's loads); LDS reads and writes of this wave complete first
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int EPI, bool WBF>
__global__ __launch_bounds__(ring::T, 1) void k_gemm_ring(GemmP p) {
    using namespace ring;
    using C = Lay<WBF>;
    constexpr int A_PL = C::A_PL, STAGE = C::STAGE, JA = C::JA, L = C::L, NPL = C::NPL, WB = C::WB;
    extern __shared__ float4 rsm[];
    unsigned char *sm = reinterpret_cast<unsigned char *>(rsm);
    int mb, nbk;
    if (!gemm_tile(p, mb, nbk)) return;
    const int m0 = mb * BM, n0 = nbk * BN;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const size_t a_bytes = (size_t)p.n_mb * BM * p.lda * 2;
    const u32x4 dh = ring_desc(p.ahi, a_bytes), dl = ring_desc(WBF ? p.ahi : p.alo, a_bytes);
    const u32x4 dw = ring_desc(p.w, (size_t)p.N * p.kp * WB);
    const unsigned sm0 = (unsigned)(uintptr_t)sm;  // LDS address (low half of the flat address)
    // load j of this wave fills 1 KB block u = j NW + wave: j < JA the hi plane
    // (8 rows of 128 B), j < 2 JA the lo plane, else the weights (int8: 16
    // columns of 64 B; bf16: 8 columns of 128 B)
    unsigned voff[L], loff[L];
#pragma unroll
    for (int j = 0; j < L; j++) {
        if (j < NPL * JA) {
            const int pl = j / JA, ua = (j % JA) * NW + wave;
            const int r = 8 * ua + (lane >> 3), c = (lane & 7) ^ (r & 7);
            voff[j] = (unsigned)((m0 + r) * p.lda * 2 + c * 16);
            loff[j] = (unsigned)(pl * A_PL + ua * 1024);
        } else if (WBF) {
            const int ub = (j - NPL * JA) * NW + wave;
            const int n = 8 * ub + (lane >> 3), c = (lane & 7) ^ (n & 7);
            const int row = min(n0 + n, p.N - 1);  // columns past N re-read row N - 1 (never stored)
            voff[j] = (unsigned)(row * p.kp * 2 + c * 16);
            loff[j] = (unsigned)(NPL * A_PL + ub * 1024);
        } else {
            const int ub = (j - NPL * JA) * NW + wave;
            const int n = 16 * ub + (lane >> 2), c = (lane & 3) ^ ((n >> 1) & 3);
            const int row = min(n0 + n, p.N - 1);  // columns past N re-read row N - 1 (never stored)
            voff[j] = (unsigned)(row * p.kp + c * 16);
            loff[j] = (unsigned)(NPL * A_PL + ub * 1024);
        }
    }
    // step kt into ring slot; steps past the last re-read the last (in bounds, never used)
    auto issue = [&](int kt, int slot) {
        const int ks = min(kt, p.nk - 1);
        const unsigned base = sm0 + (unsigned)(slot * STAGE);
#pragma unroll
        for (int j = 0; j < L; j++) {
            if (j < JA) ring_load(dh, base + loff[j], voff[j], (unsigned)(ks * BK * 2));
            else if (j < NPL * JA) ring_load(dl, base + loff[j], voff[j], (unsigned)(ks * BK * 2));
            else ring_load(dw, base + loff[j], voff[j], (unsigned)(ks * BK * WB));
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    ring_wait<0>();
#pragma unroll
    for (int s = 0; s < S - 1; s++) issue(s, s);
    const int fr = lane & 15, g = lane >> 4;
    int cur = 0;  // ring slot of step kt
    for (int kt = 0; kt < p.nk; kt++) {
        ring_wait<L * (S - 2)>();  // this wave's loads of step kt have landed
        ring_barrier();            // every wave's have; slot kt - 1 is free
        issue(kt + S - 1, cur == 0 ? S - 1 : cur - 1);
        const unsigned char *st = sm + cur * STAGE;
        cur = cur == S - 1 ? 0 : cur + 1;
        bf16x8 b0[TN], b1[TN];
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int n = wn * TN * 16 + tn * 16 + fr;
            if constexpr (WBF) {  // bf16 rows: chunk 2 g + h of the column's 128 bytes
                b0[tn] = *(const bf16x8 *)(st + A_PL + n * 128 + (((2 * g) ^ (fr & 7)) << 4));
                b1[tn] = *(const bf16x8 *)(st + A_PL + n * 128 + (((2 * g + 1) ^ (fr & 7)) << 4));
            } else {
                const u32x4 v = *(const u32x4 *)(st + 2 * A_PL + n * 64 + ((g ^ ((fr >> 1) & 3)) << 4));
                u32x4 o0, o1;
                bytes_to_bf16(v, o0, o1);
                b0[tn] = __builtin_bit_cast(bf16x8, o0);
                b1[tn] = __builtin_bit_cast(bf16x8, o1);
            }
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            bf16x8 ah[TM], al[TM];
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                const int off = (wm * TM * 16 + tm * 16 + fr) * 128 + (((2 * g + h) ^ (fr & 7)) << 4);
                ah[tm] = *(const bf16x8 *)(st + off);
                if (!WBF) al[tm] = *(const bf16x8 *)(st + A_PL + off);
            }
#pragma unroll
            for (int tn = 0; tn < TN; tn++)
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], h ? b1[tn] : b0[tn], acc[tm][tn], 0, 0, 0);
            if (!WBF) {
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
#pragma unroll
                    for (int tm = 0; tm < TM; tm++)
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], h ? b1[tn] : b0[tn], acc[tm][tn], 0, 0, 0);
            }
        }
    }
    ring_wait<0>();  // the re-read tail steps land before the workgroup's LDS is reused or released
    if (EPI == GE_SWIGLU) {
        __syncthreads();  // every wave's tail loads have landed
        swiglu_store<TM, TN, T, WBF>(p, acc, reinterpret_cast<u16 *>(sm), wm * TM * 16, wn * TN * 16, m0, n0, lane);
        if (wave == 0 && nbk == p.n_nb - 1) swiglu_pad(p, m0, lane);
    } else {
        gemm_store<EPI, TM, TN>(p, acc, m0 + wm * TM * 16, n0 + wn * TN * 16, lane, p.scale, p.scale2);
    }
}

// ------------------------------------------------------------------ GEMM on the int8 matrix cores
// Activations as digit planes (k_norm_digits): x = (d0 + 2^8 d1 + 2^16 d2)
// 2^-E per row, weights q (byte XOR 0x80).  Three v_mfma_i32_16x16x64_i8
// per 64-wide k step and tile (one per digit plane) accumulate exact integer
// sums in i32 (|d q| <= 2^14, k <= 131008); the epilogue forms
// S = A2 2^16 + A1 2^8 + A0 exactly in f64 and writes f32(S 2^-E scale)
// (one rounding) through the same store / SwiGLU epilogues.  Against the
// split-bf16 kernel: 3 int8 MFMAs at twice the bf16 rate instead of 4 bf16
// ones per 64 k, no weight conversion, 192 activation bytes per row and step
// instead of 256 (measured on the config-5 shapes in a stand-alone harness:
// qkv 715-820 -> 512 us, gate/up 3118-3189 -> 2288 us).
// Staging as k_gemm_ring: a 3-step direct-to-LDS ring; a step holds the three
// digit planes [128 rows][64 B] and the weights [256 columns][64 B], 16-byte
// chunk c of row r at c ^ ((r >> 1) & 3).  Lane group g of a 16x16x64 MFMA
// reads chunk g of its row / column for both operands, so every k pairs with
// itself.  8 waves of 64 x 64 outputs, 120 KB of LDS, one workgroup per CU.
namespace dring {
constexpr int WGM = 2, WGN = 4, TM = 4, TN = 4, NW = WGM * WGN, T = 64 * NW, S = 3;
static_assert(WGM * TM * 16 == BM && WGN * TN * 16 == BN && BK == 64, "digit ring tile");
constexpr int A_PL = BM * BK, B_ST = BN * BK, STAGE = 3 * A_PL + B_ST;
constexpr int A_UNITS = A_PL / 1024, B_UNITS = B_ST / 1024;  // 1 KB loads (16 rows of 64 B)
constexpr int JA = A_UNITS / NW, JB = B_UNITS / NW, L = 3 * JA + JB;
static_assert(A_UNITS % NW == 0 && B_UNITS % NW == 0, "digit ring units");
constexpr size_t LDS = (size_t)S * STAGE;
static_assert(L * (S - 2) < 64, "vmcnt range");
static_assert(LDS >= 2 * BM * (BN / 2 + 8) * sizeof(u16) && LDS >= BM * (BN / 2 + 4) * sizeof(float),
              "SwiGLU staging tile");
}  // namespace dring

template <int EPI>
__global__ __launch_bounds__(dring::T, 1) void k_gemm_digits(GemmP p) {
    using namespace dring;
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    extern __shared__ float4 dsm[];
    unsigned char *sm = reinterpret_cast<unsigned char *>(dsm);
    int mb, nbk;
    if (!gemm_tile(p, mb, nbk)) return;
    const int m0 = mb * BM, n0 = nbk * BN;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const u32x4 da = ring_desc(p.ad, 3 * p.dstride), dw = ring_desc(p.w, (size_t)p.N * p.kp);
    const unsigned sm0 = (unsigned)(uintptr_t)sm;  // LDS address (low half of the flat address)
    // load j of this wave fills 1 KB block u = j NW + wave: j < 3 JA digit
    // plane j / JA (16 rows of 64 B), else the weights (16 columns of 64 B)
    unsigned voff[L], loff[L];
#pragma unroll
    for (int j = 0; j < L; j++) {
        if (j < 3 * JA) {
            const int pl = j / JA, ua = (j % JA) * NW + wave;
            const int r = 16 * ua + (lane >> 2), c = (lane & 3) ^ ((r >> 1) & 3);
            voff[j] = (unsigned)(pl * p.dstride + (size_t)(m0 + r) * p.lda + c * 16);
            loff[j] = (unsigned)(pl * A_PL + ua * 1024);
        } else {
            const int ub = (j - 3 * JA) * NW + wave;
            const int n = 16 * ub + (lane >> 2), c = (lane & 3) ^ ((n >> 1) & 3);
            const int row = min(n0 + n, p.N - 1);  // columns past N re-read row N - 1 (never stored)
            voff[j] = (unsigned)(row * p.kp + c * 16);
            loff[j] = (unsigned)(3 * A_PL + ub * 1024);
        }
    }
    // step kt into ring slot; steps past the last re-read the last (in bounds, never used)
    auto issue = [&](int kt, int slot) {
        const unsigned ko = (unsigned)(min(kt, p.nk - 1) * BK);
        const unsigned base = sm0 + (unsigned)(slot * STAGE);
#pragma unroll
        for (int j = 0; j < L; j++) ring_load(j < 3 * JA ? da : dw, base + loff[j], voff[j], ko);
    };

    i32x4 acc[3][TM][TN];
#pragma unroll
    for (int d = 0; d < 3; d++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[d][i][j] = i32x4{0, 0, 0, 0};
    ring_wait<0>();
#pragma unroll
    for (int s = 0; s < S - 1; s++) issue(s, s);
    const int fr = lane & 15, g = lane >> 4;
    int cur = 0;  // ring slot of step kt
    for (int kt = 0; kt < p.nk; kt++) {
        ring_wait<L * (S - 2)>();  // this wave's loads of step kt have landed
        ring_barrier();            // every wave's have; slot kt - 1 is free
        issue(kt + S - 1, cur == 0 ? S - 1 : cur - 1);
        const unsigned char *st = sm + cur * STAGE;
        cur = cur == S - 1 ? 0 : cur + 1;
        i32x4 bq[TN];
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int n = wn * TN * 16 + tn * 16 + fr;
            const u32x4 v = *(const u32x4 *)(st + 3 * A_PL + n * 64 + ((g ^ ((fr >> 1) & 3)) << 4)) ^ 0x80808080u;
            bq[tn] = __builtin_bit_cast(i32x4, v);
        }
#pragma unroll
        for (int d = 0; d < 3; d++) {
            i32x4 a[TM];
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                const int r = wm * TM * 16 + tm * 16 + fr;
                a[tm] = *(const i32x4 *)(st + d * A_PL + r * 64 + ((g ^ ((fr >> 1) & 3)) << 4));
            }
#pragma unroll
            for (int tn = 0; tn < TN; tn++)
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
                    acc[d][tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[tm], bq[tn], acc[d][tm][tn], 0, 0, 0);
        }
    }
    ring_wait<0>();  // the re-read tail steps land before the workgroup's LDS is reused or released
    // S 2^-E scale, one rounding to f32; the store epilogues then run at unit scale
    int er[TM][4];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = m0 + wm * TM * 16 + tm * 16 + (g << 2) + r;
            er[tm][r] = m < p.M ? p.ae[m] : 0;
        }
    f32x4 v[TM][TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int n = n0 + wn * TN * 16 + tn * 16 + fr;
        const double sc = EPI == GE_SWIGLU && (n & 2) ? (double)p.scale2 : (double)p.scale;  // gate / up rows
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const double S = (double)acc[2][tm][tn][r] * 65536.0 + (double)acc[1][tm][tn][r] * 256.0 +
                                 (double)acc[0][tm][tn][r];
                const int E = er[tm][r];
                v[tm][tn][r] = E == DG_NONFINITE ? __builtin_nanf("") : (float)(S * ldexp(1.0, -E) * sc);
            }
    }
    GemmP q = p;
    q.scale = q.scale2 = 1.f;
    if (EPI == GE_SWIGLU) {
        __syncthreads();  // every wave's tail loads have landed
        swiglu_store<TM, TN, T, false>(q, v, reinterpret_cast<u16 *>(sm), wm * TM * 16, wn * TN * 16, m0, n0, lane);
        if (!p.of && wave == 0 && nbk == p.n_nb - 1) swiglu_pad(p, m0, lane);
    } else {
        gemm_store<EPI, TM, TN>(q, v, m0 + wm * TM * 16, n0 + wn * TN * 16, lane, 1.f, 1.f);
    }
}

// ------------------------------------------------------------------ RoPE + KV append
// Row m = s * seq + i is position p0[s] + i of sequence s.  q pairs are rotated
// in place (llama.rs:208-216 without a pre-scale: forward scales the scores),
// k pairs are rotated into the cache row, v is copied into the cache row
// (kv_cache.rs:99-118).  cpu.rs:655-658 in f32, no contraction.
__global__ void k_rope_kv(float *qkv, int ldq, int M, int seq, int qd, int kvd, int hd, PrefillSeqs t, int l,
                          PrefillKVP kp) {
    const int hh = hd >> 1, nkv = kvd / hd;
    const int per_row = (qd >> 1) + (kvd >> 1) + kvd;
    const size_t total = (size_t)M * per_row;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(g / per_row), e = (int)(g % per_row);
        const int s = m / seq, i = m - s * seq;
        const int pos = t.p0[s] + i;
        float *row = qkv + (size_t)m * ldq;
        float *kc = t.k[s] + (size_t)l * t.ls[s] + (size_t)pos * kvd;
        float *vc = t.v[s] + (size_t)l * t.ls[s] + (size_t)pos * kvd;
        if (e < (qd >> 1) + (kvd >> 1)) {
            const bool isq = e < (qd >> 1);
            const int j = isq ? 2 * e : 2 * (e - (qd >> 1));  // element index within q or k
            const float2 cs = t.rope[s][(size_t)pos * hh + ((j % hd) >> 1)];
            float *x = isq ? row + j : row + qd + j;
            const float x0 = x[0], x1 = x[1];
            const float r0 = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
            const float r1 = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
            if (isq) {
                x[0] = r0;
                x[1] = r1;
            } else {
                kc[j] = r0;
                kc[j + 1] = r1;
                if (kp.kh) {  // the attention's planes of this K row
                    const size_t at = ((size_t)(s * nkv + j / hd) * kp.rows + pos) * hd + j % hd;
                    u16 h0, l0, h1, l1;
                    split_bf16(r0, h0, l0);
                    split_bf16(r1, h1, l1);
                    *(unsigned *)(kp.kh + at) = (unsigned)h0 | ((unsigned)h1 << 16);
                    *(unsigned *)(kp.kl + at) = (unsigned)l0 | ((unsigned)l1 << 16);
                }
            }
        } else {
            const int j = e - (qd >> 1) - (kvd >> 1);
            const float v = row[qd + kvd + j];
            vc[j] = v;
            if (kp.kh) {
                const size_t at = ((size_t)(s * nkv + j / hd) * kp.rows + pos) * hd + j % hd;
                split_bf16(v, kp.vh[at], kp.vl[at]);
            }
        }
    }
}

// The same with 8 consecutive elements (four rotation pairs, or eight v
// values) per thread: float4 loads and stores, 16-byte plane stores
// (qd, kvd, hd multiples of 8; ldq, the caches and the tables 16-byte aligned).
__global__ void k_rope_kv8(float *qkv, int ldq, int M, int seq, int qd, int kvd, int hd, PrefillSeqs t, int l,
                           PrefillKVP kp) {
    const int hh = hd >> 1, nkv = kvd / hd;
    const int per_row = (qd + 2 * kvd) >> 3;
    const size_t total = (size_t)M * per_row;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(g / per_row), e8 = (int)(g % per_row) * 8;
        const int s = m / seq, i = m - s * seq;
        const int pos = t.p0[s] + i;
        float *row = qkv + (size_t)m * ldq;
        float *kc = t.k[s] + (size_t)l * t.ls[s] + (size_t)pos * kvd;
        float *vc = t.v[s] + (size_t)l * t.ls[s] + (size_t)pos * kvd;
        float o[8];
        int j;  // element index within q, k or v
        int part;  // 0 q, 1 k, 2 v
        if (e8 < qd) {
            part = 0;
            j = e8;
        } else if (e8 < qd + kvd) {
            part = 1;
            j = e8 - qd;
        } else {
            part = 2;
            j = e8 - qd - kvd;
        }
        const float4 a0 = *(const float4 *)(row + e8), a1 = *(const float4 *)(row + e8 + 4);
        const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        if (part < 2) {
            const float4 *cs4 = (const float4 *)(t.rope[s] + (size_t)pos * hh + ((j % hd) >> 1));
            const float4 c0 = cs4[0], c1 = cs4[1];
            const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};  // (cos, sin) x 4
#pragma unroll
            for (int p = 0; p < 4; p++) {  // cpu.rs:655-658 in f32, no contraction
                const float x0 = x[2 * p], x1 = x[2 * p + 1], c = cs[2 * p], sn = cs[2 * p + 1];
                o[2 * p] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
                o[2 * p + 1] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
            }
        } else {
#pragma unroll
            for (int q = 0; q < 8; q++) o[q] = x[q];
        }
        float *dst = part == 0 ? row + j : part == 1 ? kc + j : vc + j;
        *(float4 *)dst = make_float4(o[0], o[1], o[2], o[3]);
        *(float4 *)(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
        if (part > 0 && kp.kh) {  // the attention's planes of this K / V row
            const size_t at = ((size_t)(s * nkv + j / hd) * kp.rows + pos) * hd + j % hd;
            unsigned ph[4], pl[4];
#pragma unroll
            for (int q = 0; q < 8; q += 2) {
                u16 h0, l0, h1, l1;
                split_bf16(o[q], h0, l0);
                split_bf16(o[q + 1], h1, l1);
                ph[q / 2] = (unsigned)h0 | ((unsigned)h1 << 16);
                pl[q / 2] = (unsigned)l0 | ((unsigned)l1 << 16);
            }
            u16 *bh = part == 1 ? kp.kh : kp.vh, *bl = part == 1 ? kp.kl : kp.vl;
            *(u32x4 *)(bh + at) = u32x4{ph[0], ph[1], ph[2], ph[3]};
            *(u32x4 *)(bl + at) = u32x4{pl[0], pl[1], pl[2], pl[3]};
        }
    }
}

// The planes of the K / V rows [0, p0) that earlier calls left in the caches.
__global__ void k_kv_planes(PrefillSeqs t, int l, int n_seq, int kvd, int hd, PrefillKVP kp) {
    const int nkv = kvd / hd;
    for (int s = 0; s < n_seq; s++) {
        const size_t total = (size_t)t.p0[s] * kvd;
        const float *kc = t.k[s] + (size_t)l * t.ls[s], *vc = t.v[s] + (size_t)l * t.ls[s];
        for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
            const int row = (int)(g / kvd), c = (int)(g % kvd);
            const size_t at = ((size_t)(s * nkv + c / hd) * kp.rows + row) * hd + c % hd;
            split_bf16(kc[g], kp.kh[at], kp.kl[at]);
            split_bf16(vc[g], kp.vh[at], kp.vl[at]);
        }
    }
}

// ------------------------------------------------------------------ attention
// Causal attention of the processed rows over their cache (llama.rs:218-250:
// scores = q.k, x scale, mask keys after the query position, softmax, P.V),
// online over 32-key tiles.  Workgroup: 128 query rows of one (head, sequence);
// two threads per row, each holding half of head_dim (HT >= hd / 2 values).
// The output row goes straight into the bf16 planes of the o_proj input.
constexpr int AQ = 128, AK = 32;

template <int HT>
__global__ __launch_bounds__(256) void k_attn_prefill(PrefillAttn a, PrefillSeqs t, int l) {
    extern __shared__ float4 asm4[];
    float *sk = reinterpret_cast<float *>(asm4);  // [AK][hd]
    float *sv = sk + AK * a.hd;
    const int tid = threadIdx.x, row = tid >> 1, half = tid & 1;
    const int qb = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
    const int i = qb * AQ + row;
    const bool valid = i < a.seq;
    const int p0 = t.p0[s], pos = p0 + i;
    const int ht = a.hd >> 1, kvh = h / (a.nh / a.nkv);
    const size_t m = (size_t)s * a.seq + i;
    float q[HT], o[HT];
#pragma unroll
    for (int d = 0; d < HT; d++) {
        q[d] = (valid && d < ht) ? a.qkv[m * a.ldq + h * a.hd + half * ht + d] : 0.f;
        o[d] = 0.f;
    }
    float mx = -INFINITY, lsum = 0.f;
    const int kend = p0 + min(a.seq, (qb + 1) * AQ);  // keys [0, kend) cover this block
    const float *kc = t.k[s] + (size_t)l * t.ls[s] + (size_t)kvh * a.hd;
    const float *vc = t.v[s] + (size_t)l * t.ls[s] + (size_t)kvh * a.hd;
    for (int k0 = 0; k0 < kend; k0 += AK) {
        __syncthreads();
        for (int idx = tid; idx < AK * a.hd; idx += 256) {
            const int j = idx / a.hd, d = idx - j * a.hd;
            const bool in = k0 + j < kend;
            sk[idx] = in ? kc[(size_t)(k0 + j) * a.kvd + d] : 0.f;
            sv[idx] = in ? vc[(size_t)(k0 + j) * a.kvd + d] : 0.f;
        }
        __syncthreads();
        float sc[AK];
        float bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < AK; j++) {
            const float *kr = sk + j * a.hd + half * ht;
            float dt = 0.f;
#pragma unroll
            for (int d = 0; d < HT; d++)
                if (d < ht) dt = fmaf(q[d], kr[d], dt);
            dt += __shfl_xor(dt, 1);
            const float v = k0 + j <= pos ? dt * a.scale : -INFINITY;
            sc[j] = v;
            bm = fmaxf(bm, v);
        }
        const float mn = fmaxf(mx, bm);
        if (mn == -INFINITY) continue;  // every key so far masked (rows past seq)
        const float alpha = expf(mx - mn);
        lsum *= alpha;
#pragma unroll
        for (int d = 0; d < HT; d++) o[d] *= alpha;
#pragma unroll
        for (int j = 0; j < AK; j++) {
            const float pj = expf(sc[j] - mn);
            lsum += pj;
            const float *vr = sv + j * a.hd + half * ht;
#pragma unroll
            for (int d = 0; d < HT; d++)
                if (d < ht) o[d] = fmaf(pj, vr[d], o[d]);
        }
        mx = mn;
    }
    if (!valid) return;
    const float inv = 1.f / lsum;
    u16 *ph = a.ohi + m * a.ldo + h * a.hd + half * ht;
    u16 *pl = a.olo + m * a.ldo + h * a.hd + half * ht;
#pragma unroll
    for (int d = 0; d < HT; d++)
        if (d < ht) {
            u16 x0, x1;
            split_bf16(o[d] * inv, x0, x1);
            ph[d] = x0;
            pl[d] = x1;
        }
    if (h == a.nh - 1 && half == 1)  // zero the k padding of the o_proj input
        for (int c = a.nh * a.hd; c < a.opad; c++) {
            a.ohi[m * a.ldo + c] = 0;
            a.olo[m * a.ldo + c] = 0;
        }
}

// The same attention on the fp32 matrix cores (v_mfma_f32_16x16x4_f32: lane
// l holds A[l % 16][l / 16], B[l / 16][l % 16] and D[4 (l / 16) + r][l % 16]).
// Workgroup: MQ query rows of one (head, sequence), one wave per 16 rows; K/V
// tiles of MK keys in LDS.  Per wave and 16-key sub-tile:
//   S^T = K Q^T in HD/4 MFMAs; chunk c, position j holds head dim (HD/4) j + c,
//     so a lane's K and Q values are contiguous.  Lane l receives the scores
//     of query row l % 16 against keys 4 (l / 16) + r, r = 0..3;
//   online softmax per query row, reduced over the 4 lanes l % 16 + 16 g;
//   O^T += V^T P^T in HD/16 x 4 MFMAs; chunk r takes keys 4 j + r, so P^T is
//     the lane's own scores, and lane l accumulates query row l % 16 at head
//     dims 16 t + 4 (l / 16) + r.
// fp32 products and accumulation: the arithmetic of the VALU kernel above,
// in another summation order.
constexpr int MQW = 8, MQ = 16 * MQW, MK = 64;  // waves (16 query rows each) per workgroup; keys per tile

template <int HD>
__global__ __launch_bounds__(64 * MQW) void k_attn_mfma(PrefillAttn a, PrefillSeqs t, int l) {
    constexpr int NC = HD / 4, NT = HD / 16, LD = HD + 4;
    extern __shared__ float4 am4[];
    float *sk = reinterpret_cast<float *>(am4);  // [MK][LD]
    float *sv = sk + MK * LD;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int qb = (int)gridDim.x - 1 - (int)blockIdx.x;  // longest blocks first
    const int h = blockIdx.y, s = blockIdx.z;
    const int lr = lane & 15, lg = lane >> 4;
    const int i = qb * MQ + w * 16 + lr;
    const bool valid = i < a.seq;
    const int p0 = t.p0[s], pos = p0 + i;
    const int kvh = h / (a.nh / a.nkv);
    const size_t m = (size_t)s * a.seq + i;
    float q[NC];
    {
        const float *qr = a.qkv + m * a.ldq + h * HD + NC * lg;
#pragma unroll
        for (int c = 0; c < NC; c++) q[c] = valid ? qr[c] : 0.f;
    }
    f32x4 o[NT];
#pragma unroll
    for (int dt = 0; dt < NT; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrow = -INFINITY, lrow = 0.f;
    const int kend = p0 + min(a.seq, (qb + 1) * MQ);                 // keys of the workgroup
    const int wlast = p0 + min(a.seq, qb * MQ + w * 16 + 16) - 1;    // last key of this wave's rows
    const float *kc = t.k[s] + (size_t)l * t.ls[s] + (size_t)kvh * HD;
    const float *vc = t.v[s] + (size_t)l * t.ls[s] + (size_t)kvh * HD;
    for (int k0 = 0; k0 < kend; k0 += MK) {
        __syncthreads();
        for (int idx = tid; idx < MK * (HD / 4); idx += 64 * MQW) {
            const int j = idx / (HD / 4), c4 = idx - j * (HD / 4);
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (k0 + j < kend) {
                kv = *(const float4 *)(kc + (size_t)(k0 + j) * a.kvd + 4 * c4);
                vv = *(const float4 *)(vc + (size_t)(k0 + j) * a.kvd + 4 * c4);
            }
            *(float4 *)(sk + j * LD + 4 * c4) = kv;
            *(float4 *)(sv + j * LD + 4 * c4) = vv;
        }
        __syncthreads();
        for (int sb = 0; sb < MK; sb += 16) {
            const int kb = k0 + sb;
            if (kb > wlast) break;  // wave-uniform: masked for every row of the wave
            f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
            const float *kr = sk + (sb + lr) * LD + NC * lg;
#pragma unroll
            for (int c = 0; c < NC; c++) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[c], q[c], st, 0, 0, 0);
            float p[4];
            float tmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[r] = kb + 4 * lg + r <= pos ? st[r] * a.scale : -INFINITY;  // llama.rs:225-234
                tmax = fmaxf(tmax, p[r]);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float mn = fmaxf(mrow, tmax);  // finite: key 0 is visible to every row
            const float alpha = expf(mrow - mn);
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[r] = expf(p[r] - mn);
                ps += p[r];
            }
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            lrow = lrow * alpha + ps;
            mrow = mn;
#pragma unroll
            for (int dt = 0; dt < NT; dt++) o[dt] *= alpha;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float *vr = sv + (sb + 4 * lg + r) * LD + lr;
#pragma unroll
                for (int dt = 0; dt < NT; dt++)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[dt * 16], p[r], o[dt], 0, 0, 0);
            }
        }
    }
    if (!valid) return;
    const float inv = 1.f / lrow;
    u16 *ph = a.ohi + m * a.ldo + h * HD, *pl = a.olo + m * a.ldo + h * HD;
#pragma unroll
    for (int dt = 0; dt < NT; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int d = dt * 16 + 4 * lg + r;
            u16 x0, x1;
            split_bf16(o[dt][r] * inv, x0, x1);
            ph[d] = x0;
            pl[d] = x1;
        }
    if (h == a.nh - 1 && lg == 0)  // zero the k padding of the o_proj input
        for (int c = a.nh * HD; c < a.opad; c++) {
            a.ohi[m * a.ldo + c] = 0;
            a.olo[m * a.ldo + c] = 0;
        }
}

// The same attention on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16),
// every f32 operand x carried as hi = bf16(x), lo = bf16(x - hi) and each
// product as hi*hi + hi*lo + lo*hi (the lo*lo term is below 2^-16 of it):
// error ~2^-16 relative per product, where the fp32 matrix cores give 2^-24
// at one sixteenth of the rate.  K and V come as planes written once per row
// (k_rope_kv, k_kv_planes); q is split in registers.
// Workgroup: 16 query rows per wave, 8 waves, one (head, sequence); K / V
// tiles of 64 keys in LDS, K key-major [key][hd], V transposed [hd][key].
// Per wave and 32 keys:
//   S^T = K Q^T for two 16-key halves (A = K [16 keys][32 hd], B = Q^T):
//     lane l gets query l % 16 against keys 4 (l / 16) + r of each half;
//   online softmax per query over the 32 keys (4 lanes l % 16 + 16 g);
//   O^T += V^T P^T with the 32 keys as the MFMA's k: slot 8 g + e is key
//     4 g + e (e < 4) of the first half and 16 + 4 g + (e - 4) of the
//     second, which is exactly the P values lane (l % 16, g) holds.  The V
//     tile stores each 32-key chunk in that slot order, so a lane's 8 keys
//     are one 16-byte read (two 8-byte reads 32 bytes apart made 2-way bank
//     conflicts at the padded row stride).
constexpr int BQW = 8, BQ = 16 * BQW, BKT = 64;  // waves; query rows; keys per tile

// bf16 hi / lo words of two values with the hardware round-to-nearest-even
// conversion (the same bits as split_bf16 for finite inputs; NaN stays NaN)
__device__ __forceinline__ unsigned pack_hl(float a, float b, bool lo_plane) {
    const __bf16 ha = (__bf16)a, hb = (__bf16)b;
    if (!lo_plane) return (unsigned)__builtin_bit_cast(u16, ha) | ((unsigned)__builtin_bit_cast(u16, hb) << 16);
    const __bf16 la = (__bf16)(a - (float)ha), lb = (__bf16)(b - (float)hb);
    return (unsigned)__builtin_bit_cast(u16, la) | ((unsigned)__builtin_bit_cast(u16, lb) << 16);
}

template <int HD>
__global__ __launch_bounds__(64 * BQW) void k_attn_bf3(PrefillAttn a, PrefillSeqs t, PrefillKVP kv) {
    constexpr int NKB = HD / 32, NDT = HD / 16, KLD = HD + 8, VLD = BKT + 8;
    extern __shared__ float4 ab4[];
    u16 *sKh = reinterpret_cast<u16 *>(ab4);
    u16 *sKl = sKh + BKT * KLD, *sVh = sKl + BKT * KLD, *sVl = sVh + HD * VLD;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // 1-D grid, the longest query blocks of every (head, sequence) first; within
    // a block row, index g -> (sequence, KV head) g % (n_seq nkv), query head of
    // the group g / (n_seq nkv): the heads sharing K / V rows land on one XCD
    // (workgroup b runs on XCD b % 8)
    const int nhs = a.nh * a.nseq, nkvs = a.nkv * a.nseq;
    const int qb = a.nqb - 1 - (int)blockIdx.x / nhs, g = (int)blockIdx.x % nhs;
    const int kvg = g % nkvs, rep = g / nkvs;
    const int s = kvg / a.nkv, kvh = kvg % a.nkv, h = kvh * (a.nh / a.nkv) + rep;
    const int lr = lane & 15, lg = lane >> 4;
    const int i = qb * BQ + w * 16 + lr;
    const bool valid = i < a.seq;
    const int p0 = t.p0[s], pos = p0 + i;
    const size_t m = (size_t)s * a.seq + i;
    // Q^T fragments: lane (query lr, group lg) holds head dims 32 kb + 8 lg + e
    bf16x8 qh[NKB], ql[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) {
        float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
        if (valid) {
            const float *qr = a.qkv + m * a.ldq + h * HD + 32 * kb + 8 * lg;
            v0 = *(const float4 *)qr;
            v1 = *(const float4 *)(qr + 4);
        }
        u32x4 hv, lv;
        hv.x = pack_hl(v0.x, v0.y, false), lv.x = pack_hl(v0.x, v0.y, true);
        hv.y = pack_hl(v0.z, v0.w, false), lv.y = pack_hl(v0.z, v0.w, true);
        hv.z = pack_hl(v1.x, v1.y, false), lv.z = pack_hl(v1.x, v1.y, true);
        hv.w = pack_hl(v1.z, v1.w, false), lv.w = pack_hl(v1.z, v1.w, true);
        qh[kb] = __builtin_bit_cast(bf16x8, hv);
        ql[kb] = __builtin_bit_cast(bf16x8, lv);
    }
    f32x4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrow = -INFINITY, lrow = 0.f;
    const int kend = p0 + min(a.seq, (qb + 1) * BQ);               // keys of the workgroup
    const int wlast = p0 + min(a.seq, qb * BQ + w * 16 + 16) - 1;  // last key of this wave's rows
    const size_t pb = ((size_t)s * a.nkv + kvh) * kv.rows * HD;     // plane rows of (s, kvh)
    for (int k0 = 0; k0 < kend; k0 += BKT) {
        __syncthreads();
        // K planes: key j, 8 head dims per chunk
        for (int idx = tid; idx < 2 * BKT * (HD / 8); idx += 64 * BQW) {
            const int pl = idx / (BKT * (HD / 8)), r = idx - pl * (BKT * (HD / 8));
            const int j = r / (HD / 8), c = r - j * (HD / 8);
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (k0 + j < kend) v = *(const u32x4 *)((pl ? kv.kl : kv.kh) + pb + (size_t)(k0 + j) * HD + 8 * c);
            *(u32x4 *)((pl ? sKl : sKh) + j * KLD + 8 * c) = v;
        }
        // V planes transposed: keys 2 jp, 2 jp + 1 of 8 head dims -> 8 words [hd][key pair]
        for (int idx = tid; idx < 2 * (BKT / 2) * (HD / 8); idx += 64 * BQW) {
            const int pl = idx / ((BKT / 2) * (HD / 8)), r = idx - pl * ((BKT / 2) * (HD / 8));
            const int c = r / (BKT / 2), jp = r - c * (BKT / 2), j = 2 * jp;
            const u16 *src = (pl ? kv.vl : kv.vh) + pb;
            u32x4 v0 = u32x4{0u, 0u, 0u, 0u}, v1 = v0;
            if (k0 + j < kend) v0 = *(const u32x4 *)(src + (size_t)(k0 + j) * HD + 8 * c);
            if (k0 + j + 1 < kend) v1 = *(const u32x4 *)(src + (size_t)(k0 + j + 1) * HD + 8 * c);
            const int jj = j & 31;  // key 16 h + 4 g + e of its chunk -> slot 8 g + 4 h + e
            u16 *dst = (pl ? sVl : sVh) + (8 * c) * VLD + (j - jj) + 8 * ((jj >> 2) & 3) + 4 * (jj >> 4) + (jj & 3);
            const unsigned a0[4] = {v0.x, v0.y, v0.z, v0.w}, a1[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                *(unsigned *)(dst + (2 * e) * VLD) = (a0[e] & 0xffffu) | (a1[e] << 16);
                *(unsigned *)(dst + (2 * e + 1) * VLD) = (a0[e] >> 16) | (a1[e] & 0xffff0000u);
            }
        }
        __syncthreads();
        for (int c32 = 0; c32 < BKT; c32 += 32) {
            const int kb0 = k0 + c32;
            if (kb0 > wlast) break;  // wave-uniform: masked for every row of the wave
            float p[8];
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
                const int kr = (c32 + 16 * hf + lr) * KLD + 8 * lg;
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const bf16x8 kh = *(const bf16x8 *)(sKh + kr + 32 * kb);
                    const bf16x8 kl = *(const bf16x8 *)(sKl + kr + 32 * kb);
                    st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[kb], st, 0, 0, 0);
                    st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[kb], st, 0, 0, 0);
                    st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[kb], st, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; r++)
                    p[4 * hf + r] = kb0 + 16 * hf + 4 * lg + r <= pos ? st[r] * a.scale : -INFINITY;  // llama.rs:225-234
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int e = 0; e < 8; e++) tmax = fmaxf(tmax, p[e]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float mn = fmaxf(mrow, tmax);  // finite: key 0 is visible to every row
            // e^x as 2^(x log2 e) on the hardware exp: within ~1e-6 relative where
            // it matters, below the 2^-17 of the P planes it feeds; the row sum
            // is formed from the same values, so O / l stays consistent
            const float alpha = __builtin_amdgcn_exp2f((mrow - mn) * 1.44269504f);
            float ps = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                p[e] = __builtin_amdgcn_exp2f((p[e] - mn) * 1.44269504f);
                ps += p[e];
            }
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            lrow = lrow * alpha + ps;
            mrow = mn;
            u32x4 phv, plv;
            phv.x = pack_hl(p[0], p[1], false), plv.x = pack_hl(p[0], p[1], true);
            phv.y = pack_hl(p[2], p[3], false), plv.y = pack_hl(p[2], p[3], true);
            phv.z = pack_hl(p[4], p[5], false), plv.z = pack_hl(p[4], p[5], true);
            phv.w = pack_hl(p[6], p[7], false), plv.w = pack_hl(p[6], p[7], true);
            const bf16x8 ph = __builtin_bit_cast(bf16x8, phv), pl = __builtin_bit_cast(bf16x8, plv);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                o[dt] *= alpha;
                const int vr = (16 * dt + lr) * VLD + c32 + 8 * lg;
                const bf16x8 bvh = *(const bf16x8 *)(sVh + vr), bvl = *(const bf16x8 *)(sVl + vr);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bvh, ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bvh, pl, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bvl, ph, o[dt], 0, 0, 0);
            }
        }
    }
    if (!valid) return;
    const float inv = 1.f / lrow;
    if (a.of) {  // f32 rows (quantized for the o_proj GEMM afterwards)
        float *orow = a.of + m * a.ldo + h * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            *(float4 *)(orow + dt * 16 + 4 * lg) =
                make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
        return;
    }
    u16 *oh = a.ohi + m * a.ldo + h * HD, *ol = a.olo + m * a.ldo + h * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int d = dt * 16 + 4 * lg + r;
            u16 x0, x1;
            split_bf16(o[dt][r] * inv, x0, x1);
            oh[d] = x0;
            ol[d] = x1;
        }
    if (h == a.nh - 1 && lg == 0)  // zero the k padding of the o_proj input
        for (int c = a.nh * HD; c < a.opad; c++) {
            a.ohi[m * a.ldo + c] = 0;
            a.olo[m * a.ldo + c] = 0;
        }
}

template <int HD>
int attn_bf3_t(const PrefillAttn &a, int n_seq, const PrefillSeqs &t, const PrefillKVP &kv, hipStream_t s) {
    constexpr size_t lds = (2 * (size_t)BKT * (HD + 8) + 2 * (size_t)HD * (BKT + 8)) * sizeof(u16);
    static bool attr = false;
    if (!attr) {
        SCRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_bf3<HD>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    PrefillAttn ag = a;
    ag.nqb = (a.seq + BQ - 1) / BQ;
    ag.nseq = n_seq;
    hipLaunchKernelGGL(k_attn_bf3<HD>, dim3(ag.nqb * a.nh * n_seq), dim3(64 * BQW), lds, s, ag, t, kv);
    PF_LAUNCH_CHECK();
}

template <int HD>
int attn_mfma_t(const PrefillAttn &a, int n_seq, const PrefillSeqs &t, int l, hipStream_t s) {
    constexpr size_t lds = 2 * (size_t)MK * (HD + 4) * sizeof(float);
    static bool attr = false;
    if (!attr) {
        SCRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_mfma<HD>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    const dim3 grid((a.seq + MQ - 1) / MQ, a.nh, n_seq);
    hipLaunchKernelGGL(k_attn_mfma<HD>, grid, dim3(64 * MQW), lds, s, a, t, l);
    PF_LAUNCH_CHECK();
}

template <int EPI, bool B32, bool WBF = false>
int gemm_t(const GemmP &p, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        SCRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemm<EPI, B32, WBF>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)GEMM_LDS));
        attr = true;
    }
    const int grid = (p.n_super + 7) / 8 * 8 * 32;
    hipLaunchKernelGGL((k_gemm<EPI, B32, WBF>), dim3(grid), dim3(G_THREADS), GEMM_LDS, s, p);
    PF_LAUNCH_CHECK();
}

template <int EPI>
int gemm_digits_t(const GemmP &p, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        SCRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemm_digits<EPI>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)dring::LDS));
        attr = true;
    }
    const int grid = (p.n_super + 7) / 8 * 8 * 32;
    hipLaunchKernelGGL((k_gemm_digits<EPI>), dim3(grid), dim3(dring::T), dring::LDS, s, p);
    PF_LAUNCH_CHECK();
}

template <int EPI, bool WBF>
int gemm_ring_t(const GemmP &p, hipStream_t s) {
    constexpr size_t lds = ring::Lay<WBF>::LDS;
    static bool attr = false;
    if (!attr) {
        SCRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemm_ring<EPI, WBF>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    const int grid = (p.n_super + 7) / 8 * 8 * 32;
    hipLaunchKernelGGL((k_gemm_ring<EPI, WBF>), dim3(grid), dim3(ring::T), lds, s, p);
    PF_LAUNCH_CHECK();
}

}  // namespace

int prefill_rows_pad(int M) { return (M + BM - 1) / BM * BM; }
int prefill_k_pad(int k) { return (k + BK - 1) / BK * BK; }

int launch_norm_split(const float *x, int ldx, int rows, int rstep, int roff, const float *w, int k, float eps,
                      u16 *hi, u16 *lo, int ldp, float *outf, int ldf, hipStream_t s) {
    if (rows <= 0) return SCRY_OK;
    const int kpad = hi ? prefill_k_pad(k) : k;
    if (hi && kpad > ldp) return set_error(SCRY_ERR_INVALID, "norm_split: k %d exceeds plane stride %d", k, ldp);
    const bool al16 = ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0) && ((uintptr_t)hi % 16 == 0) &&
                      ((uintptr_t)lo % 16 == 0) && ldx % 4 == 0 && ldp % 8 == 0 && (rstep * ldx) % 4 == 0 &&
                      (roff * ldx) % 4 == 0;
    const int nc = (kpad + 2047) / 2048;
    if (hi && !outf && k % 8 == 0 && al16 && nc <= 8) {
        switch (nc) {
            case 1: hipLaunchKernelGGL(k_norm_split8<1>, dim3(rows), dim3(256), 0, s, x, ldx, rstep, roff, w, k, eps, hi, lo, ldp, kpad); break;
            case 2: hipLaunchKernelGGL(k_norm_split8<2>, dim3(rows), dim3(256), 0, s, x, ldx, rstep, roff, w, k, eps, hi, lo, ldp, kpad); break;
            case 3:
            case 4: hipLaunchKernelGGL(k_norm_split8<4>, dim3(rows), dim3(256), 0, s, x, ldx, rstep, roff, w, k, eps, hi, lo, ldp, kpad); break;
            default: hipLaunchKernelGGL(k_norm_split8<8>, dim3(rows), dim3(256), 0, s, x, ldx, rstep, roff, w, k, eps, hi, lo, ldp, kpad); break;
        }
        PF_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(k_norm_split, dim3(rows), dim3(256), 0, s, x, ldx, rstep, roff, w, k, eps, hi, lo, ldp,
                       kpad, outf, ldf);
    PF_LAUNCH_CHECK();
}

bool gemm_takes_digits(const Packed &w) {
    // int8 per-tensor weights; k bound: |sum of d q| <= 2^14 kpad stays in i32
    return !w.bf16 && !w.s32 && prefill_k_pad(w.k) <= 131008;
}

int launch_norm_digits(const float *x, int ldx, int rows, const float *w, int k, float eps, signed char *dg,
                       size_t dstride, int *e, int ldp, hipStream_t s) {
    if (rows <= 0) return SCRY_OK;
    const int kpad = prefill_k_pad(k);
    if (kpad > ldp || ldp % 16 || dstride % 16 || dstride < (size_t)rows * ldp || (uintptr_t)dg % 16)
        return set_error(SCRY_ERR_INVALID, "norm_digits: k %d, plane stride %d / %zu", k, ldp, dstride);
    const int nc = (kpad + 2047) / 2048;
    if (nc > 8) return set_error(SCRY_ERR_UNSUPPORTED, "norm_digits: k %d > 16384", k);
    const bool norm = w != nullptr;
    const bool vec = k % 8 == 0 && (uintptr_t)x % 16 == 0 && ldx % 4 == 0 && (uintptr_t)w % 16 == 0;
#define ND_LAUNCH(NC, V, N) \
    hipLaunchKernelGGL((k_norm_digits<NC, V, N>), dim3(rows), dim3(256), 0, s, x, ldx, w, k, eps, dg, dstride, e, ldp, kpad)
#define ND_NC(NC)                         \
    if (vec && norm) ND_LAUNCH(NC, true, true);   \
    else if (norm) ND_LAUNCH(NC, false, true);    \
    else if (vec) ND_LAUNCH(NC, true, false);     \
    else ND_LAUNCH(NC, false, false)
    switch (nc) {
        case 1: ND_NC(1); break;
        case 2: ND_NC(2); break;
        case 3:
        case 4: ND_NC(4); break;
        default: ND_NC(8); break;
    }
#undef ND_NC
#undef ND_LAUNCH
    PF_LAUNCH_CHECK();
}

int launch_split(const float *x, int ldx, int rows, int k, u16 *hi, u16 *lo, int ldp, hipStream_t s) {
    const int kpad = prefill_k_pad(k);
    if (kpad > ldp) return set_error(SCRY_ERR_INVALID, "split: k %d exceeds plane stride %d", k, ldp);
    const size_t total = (size_t)rows * kpad;
    if (total == 0) return SCRY_OK;
    const unsigned grid = (unsigned)std::min<size_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_split, dim3(grid), dim3(256), 0, s, x, ldx, rows, k, kpad, hi, lo, ldp);
    PF_LAUNCH_CHECK();
}

int launch_gemm(int epi, const PrefillGemm &g, hipStream_t s) {
    const Packed &w = *g.w;
    const int kp_el = w.bf16 ? w.kp / 2 : w.kp;  // row stride in weights
    if (w.kp % 16 || w.k > kp_el) return set_error(SCRY_ERR_INVALID, "gemm: bad packed layout");
    if (w.bf16 && w.s32) return set_error(SCRY_ERR_INVALID, "gemm: bf16 weights carry no block scales");
    if (w.bytes() >= 0x7fffffffull)  // buffer offsets are 32-bit
        return set_error(SCRY_ERR_UNSUPPORTED, "gemm: %zu weight bytes (limit 2 GiB per tensor)", w.bytes());
    const int kpad = prefill_k_pad(w.k);
    if (kpad > g.lda || g.lda % 8) return set_error(SCRY_ERR_INVALID, "gemm: plane stride %d < k %d", g.lda, w.k);
    if (epi == GE_SWIGLU && (w.fused != 1 || w.rows % 4 || (w.rows >> 1) > g.ldo || g.opad > g.ldo || g.ldo % 8 ||
                             ((uintptr_t)g.ohi | (uintptr_t)g.olo) % 16))
        return set_error(SCRY_ERR_INVALID, "gemm: swiglu needs the fused gate/up layout");
    if (w.s32 && w.nb * 32 < w.k) return set_error(SCRY_ERR_INVALID, "gemm: block-32 scales too short");
    if (g.of && (!g.ad || epi != GE_SWIGLU || (uintptr_t)g.of % 16 || g.ldo % 4))
        return set_error(SCRY_ERR_INVALID, "gemm: f32 SwiGLU rows need digit planes and 16-byte rows");
    if (g.ad) {  // digit planes: the int8 matrix cores
        if (!gemm_takes_digits(w) || !g.ae || g.lda % 16 || (uintptr_t)g.ad % 16 ||
            g.dstride < (size_t)prefill_rows_pad(g.M) * g.lda || 3 * g.dstride >= 0x7fffffffull)
            return set_error(SCRY_ERR_INVALID, "gemm: digit planes need int8 per-tensor weights and a %d-row stride",
                             prefill_rows_pad(g.M));
    }
    GemmP p{};
    p.ahi = g.ahi;
    p.alo = g.alo;
    p.ad = g.ad;
    p.ae = g.ae;
    p.dstride = g.dstride;
    p.of = g.of;
    p.lda = g.lda;
    p.w = w.d;
    p.kp = kp_el;
    p.N = w.rows;
    p.s32 = w.s32;
    p.nb = w.nb;
    p.M = g.M;
    p.nk = kpad / BK;
    p.n_mb = (g.M + BM - 1) / BM;
    p.n_nb = (w.rows + BN - 1) / BN;
    p.n_super = ((p.n_mb + 3) / 4) * ((p.n_nb + 7) / 8);
    p.scale = w.scale;
    p.scale2 = w.scale2;
    p.bias = g.bias;
    p.c = g.c;
    p.ldc = g.ldc;
    p.ohi = g.ohi;
    p.olo = g.olo;
    p.ldo = g.ldo;
    p.opad = g.opad;
    const bool b32 = w.s32 != nullptr;
    // the ring kernels address the planes through a buffer descriptor (32-bit
    // offsets); larger planes take the register-staged kernel
    const bool ring_ok = (size_t)p.n_mb * BM * p.lda * 2 < 0x7fffffffull;
    if (w.bf16) {  // the bf16 model: weight rows as they are, the hi plane = the reference's bf16 cast
        p.alo = nullptr;
        switch (epi) {
            case GE_STORE: return ring_ok ? gemm_ring_t<GE_STORE, true>(p, s) : gemm_t<GE_STORE, false, true>(p, s);
            case GE_RESID: return ring_ok ? gemm_ring_t<GE_RESID, true>(p, s) : gemm_t<GE_RESID, false, true>(p, s);
            case GE_SWIGLU: return ring_ok ? gemm_ring_t<GE_SWIGLU, true>(p, s) : gemm_t<GE_SWIGLU, false, true>(p, s);
        }
        return set_error(SCRY_ERR_INVALID, "gemm: unknown epilogue %d", epi);
    }
    if (p.ad) {
        switch (epi) {
            case GE_STORE: return gemm_digits_t<GE_STORE>(p, s);
            case GE_RESID: return gemm_digits_t<GE_RESID>(p, s);
            case GE_SWIGLU: return gemm_digits_t<GE_SWIGLU>(p, s);
        }
        return set_error(SCRY_ERR_INVALID, "gemm: unknown epilogue %d", epi);
    }
    if (b32) {
        switch (epi) {
            case GE_STORE: return gemm_t<GE_STORE, true>(p, s);
            case GE_RESID: return gemm_t<GE_RESID, true>(p, s);
            case GE_SWIGLU: return gemm_t<GE_SWIGLU, true>(p, s);
        }
        return set_error(SCRY_ERR_INVALID, "gemm: unknown epilogue %d", epi);
    }
    if (!ring_ok) {
        switch (epi) {
            case GE_STORE: return gemm_t<GE_STORE, false>(p, s);
            case GE_RESID: return gemm_t<GE_RESID, false>(p, s);
            case GE_SWIGLU: return gemm_t<GE_SWIGLU, false>(p, s);
        }
        return set_error(SCRY_ERR_INVALID, "gemm: unknown epilogue %d", epi);
    }
    switch (epi) {
        case GE_STORE: return gemm_ring_t<GE_STORE, false>(p, s);
        case GE_RESID: return gemm_ring_t<GE_RESID, false>(p, s);
        case GE_SWIGLU: return gemm_ring_t<GE_SWIGLU, false>(p, s);
    }
    return set_error(SCRY_ERR_INVALID, "gemm: unknown epilogue %d", epi);
}

int launch_gemm_bf16(const unsigned short *w, int kp, int N, int k, const unsigned short *ahi, int lda, int M,
                     float *c, int ldc, const float *bias, hipStream_t s) {
    const int kpad = prefill_k_pad(k);
    if (kp < kpad || kp % BK) return set_error(SCRY_ERR_INVALID, "gemm_bf16: weight rows of %d < k %d", kp, k);
    if (kpad > lda || lda % 8) return set_error(SCRY_ERR_INVALID, "gemm_bf16: plane stride %d < k %d", lda, k);
    if ((size_t)N * kp * 2 >= 0x7fffffffull)
        return set_error(SCRY_ERR_UNSUPPORTED, "gemm_bf16: weight bytes above 2 GiB");
    GemmP p{};
    p.ahi = ahi;
    p.alo = nullptr;
    p.lda = lda;
    p.w = reinterpret_cast<const uint8_t *>(w);
    p.kp = kp;
    p.N = N;
    p.M = M;
    p.nk = kpad / BK;
    p.n_mb = (M + BM - 1) / BM;
    p.n_nb = (N + BN - 1) / BN;
    p.n_super = ((p.n_mb + 3) / 4) * ((p.n_nb + 7) / 8);
    p.scale = 1.f;
    p.scale2 = 1.f;
    p.bias = bias;
    p.c = c;
    p.ldc = ldc;
    if ((size_t)p.n_mb * BM * p.lda * 2 < 0x7fffffffull) return gemm_ring_t<GE_STORE, true>(p, s);
    return gemm_t<GE_STORE, false, true>(p, s);
}

int launch_rope_kv(float *qkv, int ldq, int M, int seq, int qd, int kvd, int hd, const PrefillSeqs &t, int l,
                   const PrefillKVP &kp, int n_seq, hipStream_t s) {
    if (hd % 2 || qd % hd || kvd % hd) return set_error(SCRY_ERR_INVALID, "rope_kv: bad head dims");
    if (kp.kh) {
        int rmax = 0, any_old = 0;
        for (int i = 0; i < n_seq; i++) {
            rmax = std::max(rmax, t.p0[i] + seq);
            any_old |= t.p0[i] > 0;
        }
        if (rmax > kp.rows) return set_error(SCRY_ERR_INVALID, "rope_kv: %d plane rows < %d", kp.rows, rmax);
        if (any_old) {
            hipLaunchKernelGGL(k_kv_planes, dim3(1024), dim3(256), 0, s, t, l, n_seq, kvd, hd, kp);
            SCRY_HIP(hipGetLastError());
        }
    }
    bool v8 = hd % 8 == 0 && qd % 8 == 0 && kvd % 8 == 0 && ldq % 4 == 0 && (uintptr_t)qkv % 16 == 0 &&
              (!kp.kh || (uintptr_t)kp.kh % 16 == 0);
    for (int i = 0; i < n_seq && v8; i++)
        v8 = (uintptr_t)t.k[i] % 16 == 0 && (uintptr_t)t.v[i] % 16 == 0 && (uintptr_t)t.rope[i] % 16 == 0 &&
             t.ls[i] % 4 == 0;
    if (v8) {
        const size_t total8 = (size_t)M * ((qd + 2 * kvd) >> 3);
        if (total8 == 0) return SCRY_OK;
        const unsigned grid = (unsigned)std::min<size_t>((total8 + 255) / 256, 65536);
        hipLaunchKernelGGL(k_rope_kv8, dim3(grid), dim3(256), 0, s, qkv, ldq, M, seq, qd, kvd, hd, t, l, kp);
        PF_LAUNCH_CHECK();
    }
    const size_t total = (size_t)M * ((qd >> 1) + (kvd >> 1) + kvd);
    if (total == 0) return SCRY_OK;
    const unsigned grid = (unsigned)std::min<size_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_rope_kv, dim3(grid), dim3(256), 0, s, qkv, ldq, M, seq, qd, kvd, hd, t, l, kp);
    PF_LAUNCH_CHECK();
}

bool attn_prefill_planes(int hd) { return hd == 64 || hd == 128; }

int launch_attn_prefill(const PrefillAttn &a, int n_seq, const PrefillSeqs &t, int l, const PrefillKVP &kv,
                        hipStream_t s) {
    if (a.hd % 2 || a.hd > 128 || a.nkv <= 0 || a.nh % a.nkv)
        return set_error(SCRY_ERR_UNSUPPORTED, "attn_prefill: head_dim %d / heads %d,%d", a.hd, a.nh, a.nkv);
    if (a.of && (!kv.kh || !attn_prefill_planes(a.hd) || (uintptr_t)a.of % 16 || a.ldo % 4))
        return set_error(SCRY_ERR_INVALID, "attn_prefill: f32 output rows need the bf16 matrix-core kernel");
    if (kv.kh && attn_prefill_planes(a.hd)) {  // bf16 matrix cores on the K / V planes
        if (a.hd == 128) return attn_bf3_t<128>(a, n_seq, t, kv, s);
        return attn_bf3_t<64>(a, n_seq, t, kv, s);
    }
    switch (a.hd) {  // matrix-core kernel for the common head sizes
        case 32: return attn_mfma_t<32>(a, n_seq, t, l, s);
        case 48: return attn_mfma_t<48>(a, n_seq, t, l, s);
        case 64: return attn_mfma_t<64>(a, n_seq, t, l, s);
        case 128: return attn_mfma_t<128>(a, n_seq, t, l, s);
        default: break;
    }
    const dim3 grid((a.seq + AQ - 1) / AQ, a.nh, n_seq);
    const size_t lds = 2 * (size_t)AK * a.hd * sizeof(float);
    const int ht = a.hd / 2;
    if (ht <= 8)
        hipLaunchKernelGGL(k_attn_prefill<8>, grid, dim3(256), lds, s, a, t, l);
    else if (ht <= 16)
        hipLaunchKernelGGL(k_attn_prefill<16>, grid, dim3(256), lds, s, a, t, l);
    else if (ht <= 32)
        hipLaunchKernelGGL(k_attn_prefill<32>, grid, dim3(256), lds, s, a, t, l);
    else
        hipLaunchKernelGGL(k_attn_prefill<64>, grid, dim3(256), lds, s, a, t, l);
    PF_LAUNCH_CHECK();
}

}  // namespace scry
