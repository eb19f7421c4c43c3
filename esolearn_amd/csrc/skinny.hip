// matmul_i8_f32 for 3..16 activation rows on the matrix cores
// (ops::matmul_i8_f32 / _bias, quantize.rs block-32 variant; cpu.rs:1128-1160):
//   y[i][j] = scale * sum_p x[i][p] * q[j][p]  (+ bias[j])
// on the packed weight rows (bytes q + 128, the decode GEMV's layout).
//
// The GEMV takes at most 4 activation rows per weight pass and spends a VALU
// multiply-add per weight byte and row, so 16 rows cost four passes of VALU
// work.  Here one 16-row v_mfma_f32_16x16x32_bf16 tile consumes every weight
// byte once for all rows:
//   - activations: three bf16 planes per value, truncated so that
//     x = h + m + l exactly for finite x (8 + 8 + 8 significand bits); a
//     non-finite x goes whole into the first plane;
//   - weights: q = byte - 128 is an integer of at most 8 bits, exact in bf16;
//   - each product is exact in f32 and the matrix core accumulates in f32, so
//     the result carries f32 accumulation error only, like the GEMV.
// Block-32 scales: each MFMA covers exactly one 32-wide k block, its result is
// multiplied by that block's scale of the lane's output column.
//
// Work split: a workgroup (4 waves, 32 output columns each as two 16-column
// MFMA blocks) covers 128 columns over KS 64-wide k blocks; the k splits of a
// column tile write partial sums, which k_skinny_reduce adds in split order
// (deterministic), then applies the scale and the bias.
//
// Fused form (the batched decode step's projections): the k splits write
// their partials as above -- per-tensor weights through k_skinny_dg, on the
// int8 matrix cores with the activations as int8 digits (below) -- and
// k_skinny_epi (one workgroup per column tile)
// adds them in split order and applies the epilogue: store, residual add
// (plus per-row partial sums of squares of the result for the next RMSNorm),
// SwiGLU of the fused gate/up rows, or logits (plus per-row ordered argmax
// partials); or no epilogue (SKE_NONE: the batched decode step's qkv rows,
// whose partials the attention launch sums).  NORM: the activation is RMSNorm(x) applied as
// rstd * (W (x * g)) (rmsnorm.rs, cpu.rs:574-599): x * g is staged, and rstd
// (f64, from the producer's partial sums of squares) scales the sums.
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int SK_COLS = 128;  // output columns per workgroup
constexpr int SK_NT = 256;    // threads per workgroup
constexpr int SK_ROWS = 16;   // MFMA rows (activation rows, zero past m)

struct SkArgs {
    const float *x;
    int ldx, m, k;
    const uint8_t *w;
    int kp, n;
    const float *s32;  // block-32 scales [n][nb], or null
    int nb;
    float *part;  // [n_split][16][n_pad] partial sums
    int n_pad, n_split, kblocks;
    // fused form
    const float *g;       // NORM: RMSNorm weight [k]
    const double *ss_in;  // NORM: per-row partial sums of squares of x [m][n_ss_in]
    int n_ss_in;
    float eps;
    int tiles, n_out;
    float scale, scale2;
    float *y;  // output rows [m][ldy]; SKE_RESID: also the residual (in place)
    int ldy;
    double *ss_out;  // SKE_RESID: per-row partial sums of squares of y [m][tiles]
    float *pv;       // SKE_LOGITS: per-row ordered argmax partials [m][tiles]
    int *pi, *pn;
};


// x = h + m + l in truncated bf16 planes (bits of each plane's bf16)
__device__ __forceinline__ void split3(float x, unsigned &h, unsigned &mi, unsigned &lo) {
    const unsigned b = __float_as_uint(x);
    if ((b & 0x7f800000u) == 0x7f800000u) {
        h = b >> 16;
        mi = lo = 0;
        return;
    }
    const float r1 = x - __uint_as_float(b & 0xffff0000u);  // exact
    const unsigned b1 = __float_as_uint(r1);
    const float r2 = r1 - __uint_as_float(b1 & 0xffff0000u);  // exact, <= 8 significand bits
    h = b >> 16;
    mi = b1 >> 16;
    lo = __float_as_uint(r2) >> 16;
}

// bytes 4j..4j+3 of (d0, d1) hold q + 128: the bf16 values of q, in byte order.
// Flipping bit 7 gives q's two's-complement byte; |q| <= 128 is exact in bf16
// (v_cvt_f32_i32 on a sign-extended byte, then v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 q8_bf16(unsigned d0, unsigned d1) {
    const unsigned e0 = d0 ^ 0x80808080u, e1 = d1 ^ 0x80808080u;
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r[j] = (__bf16)(float)(int)(signed char)(e0 >> (8 * j));
        r[4 + j] = (__bf16)(float)(int)(signed char)(e1 >> (8 * j));
    }
    return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Lane layouts of v_mfma_f32_16x16x32_bf16 (16 x 32 A, 32 x 16 B, 16 x 16 D):
// lane l holds A[l % 16][8 (l / 16) + e], B[8 (l / 16) + e][l % 16] (e = 0..7)
// and D[4 (l / 16) + r][l % 16] (r = 0..3).  The k index inside an MFMA is a
// summation index only; the 64-wide block kb is laid out as
//   per-tensor: lane group g, half f -> k = 64 kb + 16 g + 8 f + e (one 16-byte
//               LDS read per lane and column block feeds both halves);
//   block-32:   lane group g, half f -> k = 64 kb + 32 f + 8 g + e (each half is
//               one 32-wide scale block).
// LDS: A planes as 16-byte fragments [kb][plane][half][lane group][row] (rows
// below MRT only: with at most 4 activation rows the other 12 MFMA rows are
// zero registers, a quarter of the LDS and so more workgroups per CU); per wave a
// [32 rows][144 B] weight tile for two 64-wide blocks (rows padded by 16 bytes
// so the 16-byte fragment reads of 16 rows hit distinct banks) and, for
// block-32, the wave's scales [32 columns][2 KS blocks].
//
// Weights come from HBM in whole 128-byte lines: load instruction j of segment
// s (128 bytes of k = two blocks) reads rows 8 (j % 4) .. +8 of the wave's 32,
// lane l taking bytes 16 (l % 8) of row l / 8.  Fragments in the MFMA layout
// (16 rows x 64 bytes per instruction) would split every line in two.
constexpr int SK_WROW = 144;                 // bytes per weight row in the LDS tile
constexpr int SK_WTILE = 32 * SK_WROW;       // bytes per wave
// MRT: activation rows kept in LDS (4: at most 4 rows; the MFMA's other A
// rows are zero registers; 16: all of them).
template <int KS, bool B32, bool NORM, int MRT>
__global__ __launch_bounds__(SK_NT) void k_skinny(SkArgs a) {
    static_assert(KS % 2 == 0, "weights come in 128-byte segments of two blocks");
    static_assert(MRT == 4 || MRT == 16, "4 or 16 activation rows");
    __shared__ u32x4 s_a[KS * 3 * 2 * 4 * MRT];
    __shared__ __attribute__((aligned(16))) unsigned char s_w[4 * SK_WTILE];
    __shared__ float s_sc[B32 ? 4 * 32 * 2 * KS : 1];
    const int split = blockIdx.x % a.n_split, tile = blockIdx.x / a.n_split;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kb0 = split * KS;
    const int nkb = min(KS, a.kblocks - kb0);
    const int k0 = kb0 * 64;

    // ---- 1. activation loads: unit u = (kb, row, q8) holds x[row][k0 + 64 kb + 8 q8 + 0..7];
    // eight consecutive threads read 256 contiguous bytes of one row
    constexpr int NU = KS * MRT * 8, UPT = (NU + SK_NT - 1) / SK_NT;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, ((size_t)(a.m - 1) * a.ldx + a.k) * 4);
    float4 xv[UPT][2];
    float4 gv[NORM ? UPT : 1][2];
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(NORM ? a.g : a.x, NORM ? (size_t)a.k * 4 : 0);
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + SK_NT * i, kb = u / (8 * MRT), row = (u >> 3) % MRT, q8 = u & 7;
        const int kk = k0 + kb * 64 + q8 * 8;
        const bool in = (NU % SK_NT == 0 || u < NU) && row < a.m && kb < nkb && kk < a.k;
        const unsigned off = in ? (unsigned)(row * a.ldx + kk) * 4 : 0x80000000u;
        xv[i][0] = bload16f(xr, off);
        xv[i][1] = bload16f(xr, off + 16);
        if constexpr (NORM) {
            const unsigned og = in ? (unsigned)kk * 4 : 0x80000000u;
            gv[i][0] = bload16f(gr, og);
            gv[i][1] = bload16f(gr, og + 16);
        }
    }

    // ---- 2. the wave's 32 weight rows over this split, all requested now
    const int cw = tile * SK_COLS + wave * 32;  // the wave's first column
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, (size_t)a.n * a.kp);
    constexpr int NSEG = KS / 2;
    u32x4 wv[NSEG][4];
#pragma unroll
    for (int sg = 0; sg < NSEG; sg++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = cw + 8 * j + (lane >> 3);
            const bool ok = 2 * sg < nkb && row < a.n;
            wv[sg][j] = bload16(wr, ok ? (unsigned)row * a.kp + k0 + 128 * sg + 16 * (lane & 7) : 0x80000000u);
        }
    float scv[B32 ? KS : 1];
    if constexpr (B32) {  // lane l: column cw + l / 2, blocks 2 kb0 + KS (l % 2) .. + KS
        const int c = cw + (lane >> 1), blk0 = 2 * kb0 + KS * (lane & 1);
#pragma unroll
        for (int i = 0; i < KS; i++)
            scv[i] = (c < a.n && blk0 + i < a.nb) ? a.s32[(size_t)c * a.nb + blk0 + i] : 0.f;
    }

    // ---- 3. stage the activation planes (and the scales)
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + SK_NT * i, kb = u / (8 * MRT), row = (u >> 3) % MRT, q8 = u & 7;
        if (NU % SK_NT != 0 && u >= NU) break;
        const int kk = k0 + kb * 64 + q8 * 8;
        float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                      xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
        if constexpr (NORM) {
            const float gg8[8] = {gv[i][0].x, gv[i][0].y, gv[i][0].z, gv[i][0].w,
                                  gv[i][1].x, gv[i][1].y, gv[i][1].z, gv[i][1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = __fmul_rn(v[e], gg8[e]);
        }
        unsigned pl[3][8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (kk + e >= a.k) v[e] = 0.f;  // past the row: the next row's values
            split3(v[e], pl[0][e], pl[1][e], pl[2][e]);
        }
        const int gg = B32 ? (q8 & 3) : (q8 >> 1), f = B32 ? (q8 >> 2) : (q8 & 1);
#pragma unroll
        for (int p = 0; p < 3; p++) {
            u32x4 q;
            q.x = pl[p][0] | (pl[p][1] << 16);
            q.y = pl[p][2] | (pl[p][3] << 16);
            q.z = pl[p][4] | (pl[p][5] << 16);
            q.w = pl[p][6] | (pl[p][7] << 16);
            s_a[(((kb * 3 + p) * 2 + f) * 4 + gg) * MRT + row] = q;
        }
    }
    float *scw = s_sc + wave * (32 * 2 * KS);  // [32 columns][2 KS blocks]
    if constexpr (B32) {
#pragma unroll
        for (int i = 0; i < KS; i++) scw[(lane >> 1) * 2 * KS + KS * (lane & 1) + i] = scv[i];
    }
    __syncthreads();

    // ---- 4. per 128-byte segment: weights through the wave's LDS tile, then
    // the matrix-core passes of its two blocks
    unsigned char *tw = s_w + wave * SK_WTILE;
    const int nn = lane & 15, g = lane >> 4;
    f32x4 acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sg = 0; sg < NSEG; sg++) {
        if (2 * sg >= nkb) break;  // uniform
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(u32x4 *)(tw + (8 * j + (lane >> 3)) * SK_WROW + 16 * (lane & 7)) = wv[sg][j];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int kb = 2 * sg + h;
            if (kb >= nkb) break;  // uniform
            bf16x8 av[3][2];
#pragma unroll
            for (int p = 0; p < 3; p++)
#pragma unroll
                for (int f = 0; f < 2; f++)
                    av[p][f] = (lane & 15) < MRT
                                   ? as_bf16x8(s_a[(((kb * 3 + p) * 2 + f) * 4 + (lane >> 4)) * MRT + (lane & 15)])
                                   : bf16x8{};
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                const unsigned char *wrow = tw + (16 * cb + nn) * SK_WROW + 64 * h;
                if constexpr (!B32) {
                    const u32x4 w = *(const u32x4 *)(wrow + 16 * g);
                    const bf16x8 b0 = q8_bf16(w.x, w.y), b1 = q8_bf16(w.z, w.w);
#pragma unroll
                    for (int p = 0; p < 3; p++) {
                        acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[p][0], b0, acc[cb], 0, 0, 0);
                        acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[p][1], b1, acc[cb], 0, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int f = 0; f < 2; f++) {
                        const uint2 w = *(const uint2 *)(wrow + 32 * f + 8 * g);
                        const bf16x8 bq = q8_bf16(w.x, w.y);
                        f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int p = 0; p < 3; p++) t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[p][f], bq, t, 0, 0, 0);
                        const float sc = scw[(16 * cb + nn) * 2 * KS + 2 * kb + f];
                        acc[cb].x = fmaf(t.x, sc, acc[cb].x);
                        acc[cb].y = fmaf(t.y, sc, acc[cb].y);
                        acc[cb].z = fmaf(t.z, sc, acc[cb].z);
                        acc[cb].w = fmaf(t.w, sc, acc[cb].w);
                    }
                }
            }
        }
    }
    int col[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++) col[cb] = cw + cb * 16 + nn;

    // ---- 5. this split's partial sums: lane holds rows 4 g + r of column col[cb]
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 4 * g + r;
            if (row < a.m) a.part[((size_t)split * SK_ROWS + row) * a.n_pad + col[cb]] = acc[cb][r];
        }
}

// The fused form with per-tensor int8 weights (the batched decode step's
// projections) on the int8 matrix cores.  The workgroup's activation segment
// (its KS 64-wide blocks of each row, x * g for the RMSNorm'd inputs) is
// carried as fixed point per row: E with max|v| 2^E <= 2^23 - 2^16 - 1 over
// the segment, X = rint(v 2^E) (a power-of-two scaling, one rounding:
// |v - X 2^-E| <= 2^-24 max|v|), and X = d0 + 2^8 d1 + 2^16 d2 in balanced
// int8 digits.  Three v_mfma_i32_16x16x64_i8 per 64-wide block and 16
// columns (one per digit plane) against the weight bytes as they are
// (q = byte XOR 0x80) give exact integer sums (|d q| <= 2^14, 512 values per
// segment); the split's partial is f32(S 2^-E) with S = A2 2^16 + A1 2^8 + A0
// formed exactly in f64.  A segment holding a NaN or an infinity gives NaN
// partials for its row (the prefill digit GEMM does the same).
// LDS: digit fragments [kb][plane][lane group][row] of 16 bytes (rows below
// MRT), the per-wave weight tile of k_skinny, per-(wave, row) maxima.
constexpr int SK_DG_NONFINITE = 0x7fffffff;
constexpr double SK_DG_XMAX = 8323071.0;  // 2^23 - 2^16 - 1

typedef int i32x4 __attribute__((ext_vector_type(4)));

// A row segment's exponent from its maximum magnitude m and whether it holds a
// NaN or an infinity
__device__ __forceinline__ int dg_exponent(float m, bool bad) {
    int E = 0;
    if (bad) {
        E = SK_DG_NONFINITE;
    } else if (m > 0.f) {
        int ex;
        frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1)
        E = 23 - ex;
        if (ldexp((double)m, E) > SK_DG_XMAX) E--;
    }
    return E;
}

// Eight values -> their bytes in the three digit planes (b[p][e / 4], byte e % 4)
__device__ __forceinline__ void dg_digits(const float (&v)[8], int E, unsigned (&b)[3][2]) {
    const int Es = E == SK_DG_NONFINITE ? 0 : E;
#pragma unroll
    for (int p = 0; p < 3; p++) b[p][0] = b[p][1] = 0u;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        // v 2^E is exact in f32 (a power-of-two scaling to at most 2^23), rint then exact
        const int X = E == SK_DG_NONFINITE ? 0 : (int)rintf(ldexpf(v[e], Es));
        const int X1 = (X - (int)(signed char)X) >> 8;
        const int X2 = (X1 - (int)(signed char)X1) >> 8;
        const int sh = 8 * (e & 3);
        b[0][e >> 2] |= (unsigned)(X & 255) << sh;
        b[1][e >> 2] |= (unsigned)(X1 & 255) << sh;
        b[2][e >> 2] |= (unsigned)(X2 & 255) << sh;
    }
}

// A split's partial of one row from the digit planes' integer sums
__device__ __forceinline__ float dg_partial(int a0, int a1, int a2, int E) {
    const double S = (double)a2 * 65536.0 + (double)a1 * 256.0 + (double)a0;
    return E == SK_DG_NONFINITE ? __builtin_nanf("") : (float)(S * ldexp(1.0, -E));
}

template <int KS, bool NORM, int MRT>
__global__ __launch_bounds__(SK_NT) void k_skinny_dg(SkArgs a) {
    static_assert(KS % 2 == 0, "weights come in 128-byte segments of two blocks");
    static_assert(MRT == 4 || MRT == 16, "4 or 16 activation rows");
    __shared__ u32x4 s_d[KS * 3 * 4 * MRT];
    __shared__ __attribute__((aligned(16))) unsigned char s_w[4 * SK_WTILE];
    __shared__ float s_wmax[4][MRT];
    __shared__ int s_wbad[4][MRT];
    __shared__ int s_e[MRT];
    const int split = blockIdx.x % a.n_split, tile = blockIdx.x / a.n_split;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kb0 = split * KS;
    const int nkb = min(KS, a.kblocks - kb0);
    const int k0 = kb0 * 64;

    // ---- 1. activation loads: unit u = (kb, row, q8) holds x[row][k0 + 64 kb + 8 q8 + 0..7];
    // every unit of a thread has the same row, (tid / 8) % MRT
    constexpr int NU = KS * MRT * 8, UPT = (NU + SK_NT - 1) / SK_NT;
    const int myrow = (tid >> 3) % MRT;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, ((size_t)(a.m - 1) * a.ldx + a.k) * 4);
    float4 xv[UPT][2];
    float4 gv[NORM ? UPT : 1][2];
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(NORM ? a.g : a.x, NORM ? (size_t)a.k * 4 : 0);
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + SK_NT * i, kb = u / (8 * MRT), q8 = u & 7;
        const int kk = k0 + kb * 64 + q8 * 8;
        const bool in = (NU % SK_NT == 0 || u < NU) && myrow < a.m && kb < nkb && kk < a.k;
        const unsigned off = in ? (unsigned)(myrow * a.ldx + kk) * 4 : 0x80000000u;
        xv[i][0] = bload16f(xr, off);
        xv[i][1] = bload16f(xr, off + 16);
        if constexpr (NORM) {
            const unsigned og = in ? (unsigned)kk * 4 : 0x80000000u;
            gv[i][0] = bload16f(gr, og);
            gv[i][1] = bload16f(gr, og + 16);
        }
    }

    // ---- 2. the wave's 32 weight rows over this split, all requested now
    const int cw = tile * SK_COLS + wave * 32;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, (size_t)a.n * a.kp);
    constexpr int NSEG = KS / 2;
    u32x4 wv[NSEG][4];
#pragma unroll
    for (int sg = 0; sg < NSEG; sg++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = cw + 8 * j + (lane >> 3);
            const bool ok = 2 * sg < nkb && row < a.n;
            wv[sg][j] = bload16(wr, ok ? (unsigned)row * a.kp + k0 + 128 * sg + 16 * (lane & 7) : 0x80000000u);
        }

    // ---- 3. the values, the segment maximum of each row, the digit planes
    float v[UPT][8];
    float amax = 0.f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + SK_NT * i, kb = u / (8 * MRT), q8 = u & 7;
        const int kk = k0 + kb * 64 + q8 * 8;
        const float xs[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                             xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float t = xs[e];
            if constexpr (NORM) {
                const float gg8[8] = {gv[i][0].x, gv[i][0].y, gv[i][0].z, gv[i][0].w,
                                      gv[i][1].x, gv[i][1].y, gv[i][1].z, gv[i][1].w};
                t = __fmul_rn(t, gg8[e]);
            }
            if (kk + e >= a.k || (NU % SK_NT != 0 && u >= NU)) t = 0.f;  // past the row / no unit
            v[i][e] = t;
            amax = fmaxf(amax, fabsf(t));
            bad |= !isfinite(t);
        }
    }
    // lanes of one row: MRT 4: lane bits 0-2 and 5 vary; MRT 16: bits 0-2
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off));
        bad |= __shfl_xor(bad, off);
    }
    if constexpr (MRT == 4) {
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        bad |= __shfl_xor(bad, 32);
    }
    if ((lane & 7) == 0 && (MRT == 16 || lane < 32)) {
        s_wmax[wave][myrow] = amax;
        s_wbad[wave][myrow] = bad;
    }
    __syncthreads();
    if (tid < MRT) {  // waves holding row tid: all four (MRT 4), or tid / 8 and tid / 8 + 2
        float m = 0.f;
        int b = 0;
#pragma unroll
        for (int w = 0; w < 4; w++)
            if (MRT == 4 || (w & 1) == (tid >> 3)) {
                m = fmaxf(m, s_wmax[w][tid]);
                b |= s_wbad[w][tid];
            }
        s_e[tid] = dg_exponent(m, b != 0);
    }
    __syncthreads();
    {
        const int E = s_e[myrow];
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + SK_NT * i, kb = u / (8 * MRT), q8 = u & 7;
            if (NU % SK_NT != 0 && u >= NU) break;
            unsigned b[3][2];
            dg_digits(v[i], E, b);
            // k = 64 kb + 16 g + 8 h + e: lane group g = q8 / 2, half h = q8 % 2
#pragma unroll
            for (int p = 0; p < 3; p++) {
                unsigned char *frag = reinterpret_cast<unsigned char *>(&s_d[((kb * 3 + p) * 4 + (q8 >> 1)) * MRT + myrow]);
                *reinterpret_cast<uint2 *>(frag + 8 * (q8 & 1)) = make_uint2(b[p][0], b[p][1]);
            }
        }
    }
    __syncthreads();

    // ---- 4. per 128-byte segment: weights through the wave's LDS tile, then
    // three int8 matrix-core passes (one per digit plane) per block and 16 columns
    unsigned char *tw = s_w + wave * SK_WTILE;
    const int nn = lane & 15, g = lane >> 4;
    i32x4 acc[3][2];
#pragma unroll
    for (int p = 0; p < 3; p++)
#pragma unroll
        for (int cb = 0; cb < 2; cb++) acc[p][cb] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int sg = 0; sg < NSEG; sg++) {
        if (2 * sg >= nkb) break;  // uniform
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(u32x4 *)(tw + (8 * j + (lane >> 3)) * SK_WROW + 16 * (lane & 7)) = wv[sg][j];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int kb = 2 * sg + h;
            if (kb >= nkb) break;  // uniform
            i32x4 ad[3];
#pragma unroll
            for (int p = 0; p < 3; p++)
                ad[p] = nn < MRT ? __builtin_bit_cast(i32x4, s_d[((kb * 3 + p) * 4 + g) * MRT + nn]) : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                const u32x4 w = *(const u32x4 *)(tw + (16 * cb + nn) * SK_WROW + 64 * h + 16 * g) ^ 0x80808080u;
                const i32x4 bq = __builtin_bit_cast(i32x4, w);
#pragma unroll
                for (int p = 0; p < 3; p++)
                    acc[p][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ad[p], bq, acc[p][cb], 0, 0, 0);
            }
        }
    }

    // ---- 5. this split's partial sums: lane holds rows 4 g + r of column cw + 16 cb + nn
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int row = 4 * g + r;
        if (row >= a.m) continue;
        const int E = s_e[row < MRT ? row : 0];
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
            a.part[((size_t)split * SK_ROWS + row) * a.n_pad + cw + 16 * cb + nn] =
                dg_partial(acc[0][cb][r], acc[1][cb][r], acc[2][cb][r], E);
    }
}

__device__ __forceinline__ ArgAcc wave_argmax(ArgAcc a) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        ArgAcc o;
        o.v = __shfl_xor(a.v, off);
        o.i = __shfl_xor(a.i, off);
        o.nan = __shfl_xor(a.nan, off);
        a = arg_combine(a, o);
    }
    return a;
}

__device__ __forceinline__ void arg_push(ArgAcc &p, float v, int i) {  // sequential scan order
    if (isnan(v)) {
        p.nan = i;
        return;
    }
    if (p.i < 0 || !(p.v > v)) {
        p.v = v;
        p.i = i;
    }
}

// One workgroup per column tile: wave w takes rows w, w + 4, ...; lane l the
// columns 2l, 2l + 1 of the tile, or (SwiGLU, lanes 0..31) the packed group
// 4l .. 4l + 3 = gate and up of outputs 2l, 2l + 1.  Every split's partials
// of a batch are requested before the first is used; the sums run in split
// order.
template <int EPI>
__global__ __launch_bounds__(SK_NT) void k_skinny_epi(SkArgs a) {
    const int tile = blockIdx.x;
    constexpr bool SW = EPI == SKE_SWIGLU;
    constexpr int NB = SW ? 16 : 32;  // splits per load batch
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool act = !SW || lane < 32;
    const int c = tile * SK_COLS + (SW ? 4 : 2) * (act ? lane : 0);
    const size_t st = (size_t)SK_ROWS * a.n_pad;
    for (int row = wave; row < a.m; row += SK_NT / 64) {
        const float *p = a.part + (size_t)row * a.n_pad + c;
        double ssq = 0.0;
        if (a.ss_in && lane < a.n_ss_in) ssq = a.ss_in[(size_t)row * a.n_ss_in + lane];
        // the residual values, requested with the partials (clamped in
        // bounds, unconditional): otherwise their load waits for the sums
        float r0 = 0.f, r1 = 0.f;
        if constexpr (EPI == SKE_RESID) {
            const float *yq = a.y + (size_t)row * a.ldy;
            r0 = yq[min(c, a.n_out - 1)];
            r1 = yq[min(c + 1, a.n_out - 1)];
        }
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
        for (int i0 = 0; i0 < a.n_split; i0 += NB) {
            float2 q0[NB], q1[SW ? NB : 1];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                if (i0 + j < a.n_split) {
                    q0[j] = *(const float2 *)(p + (size_t)(i0 + j) * st);
                    if constexpr (SW) q1[j] = *(const float2 *)(p + (size_t)(i0 + j) * st + 2);
                }
            }
#pragma unroll
            for (int j = 0; j < NB; j++) {
                if (i0 + j < a.n_split) {
                    s0 += q0[j].x;
                    s1 += q0[j].y;
                    if constexpr (SW) {
                        s2 += q1[j].x;
                        s3 += q1[j].y;
                    }
                }
            }
        }
        double rstd = 1.0;
        if (a.ss_in) {  // RMSNorm of the input row: f64 sum of the producer's partials
            const double v = wave_sum_d(ssq);
            rstd = 1.0 / sqrt(v / (double)a.k + (double)a.eps);
        }
        float *yr = a.y + (size_t)row * a.ldy;
        if constexpr (SW) {  // cpu.rs:666-678
            const int j = tile * (SK_COLS / 2) + 2 * lane;
            const float g0 = (float)((double)(s0 * a.scale) * rstd), g1 = (float)((double)(s1 * a.scale) * rstd);
            const float u0 = (float)((double)(s2 * a.scale2) * rstd), u1 = (float)((double)(s3 * a.scale2) * rstd);
            if (act && j < a.n_out) yr[j] = silu_f(g0) * u0;
            if (act && j + 1 < a.n_out) yr[j + 1] = silu_f(g1) * u1;
        } else {
            const int c1 = c + 1;
            const bool ok0 = c < a.n_out, ok1 = c1 < a.n_out;
            float v0 = (float)((double)(s0 * a.scale) * rstd), v1 = (float)((double)(s1 * a.scale) * rstd);
            if constexpr (EPI == SKE_RESID) {  // llama.rs:556-569: x + o, x + down
                v0 = r0 + v0;
                v1 = r1 + v1;
            }
            if (ok0) yr[c] = v0;
            if (ok1) yr[c1] = v1;
            if constexpr (EPI == SKE_RESID) {
                if (a.ss_out) {
                    double q = (ok0 ? (double)v0 * (double)v0 : 0.0) + (ok1 ? (double)v1 * (double)v1 : 0.0);
                    q = wave_sum_d(q);
                    if (lane == 0) a.ss_out[(size_t)row * a.tiles + tile] = q;
                }
            }
            if constexpr (EPI == SKE_LOGITS) {  // generate.rs:167-173, in index order
                // A row segment holding an infinity or a NaN makes the digit
                // kernel's partials NaN, while the reference's sum of
                // f64(a) (q s) over k (cpu.rs:1128-1160) is +-inf per column
                // unless a NaN term or both infinities occur.  Only the terms
                // of the non-finite normalised inputs decide it, so a NaN sum
                // (uniform over the row; never the case for finite rows)
                // classifies those terms, as the GEMV's logits epilogue does.
                const bool n0 = ok0 && isnan(v0), n1 = ok1 && isnan(v1);
                if (__builtin_amdgcn_ballot_w64(n0 || n1)) {
                    int cls0 = 0, cls1 = 0;
                    const float *xr = a.x + (size_t)row * a.ldx;
                    for (int p0 = 0; p0 < a.k; p0 += 64) {
                        const int p = p0 + lane;
                        float t = 0.f;
                        if (p < a.k) {  // rmsnorm (cpu.rs:574-599): f32(f64(x) rstd f64(w))
                            t = xr[p];
                            if (a.g) t = (float)((double)t * rstd * (double)a.g[p]);
                        }
                        unsigned long long mk = __builtin_amdgcn_ballot_w64(p < a.k && !isfinite(t));
                        while (mk) {
                            const int l = __builtin_ctzll(mk);
                            mk &= mk - 1;
                            const float tt = __shfl(t, l);
                            const int pp = p0 + l;
                            if (n0) cls0 |= nonfinite_term(tt, a.w[(size_t)c * a.kp + pp], a.s32 ? a.s32[(size_t)c * a.nb + (pp >> 5)] : a.scale);
                            if (n1) cls1 |= nonfinite_term(tt, a.w[(size_t)c1 * a.kp + pp], a.s32 ? a.s32[(size_t)c1 * a.nb + (pp >> 5)] : a.scale);
                        }
                    }
                    if (n0 && cls0) v0 = nonfinite_value(cls0);
                    if (n1 && cls1) v1 = nonfinite_value(cls1);
                    if (ok0) yr[c] = v0;
                    if (ok1) yr[c1] = v1;
                }
                ArgAcc pa{0.f, -1, -1};
                if (ok0) arg_push(pa, v0, c);
                if (ok1) arg_push(pa, v1, c1);
                pa = wave_argmax(pa);
                if (lane == 0) {
                    const size_t at = (size_t)row * a.tiles + tile;
                    a.pv[at] = pa.v;
                    a.pi[at] = pa.i;
                    a.pn[at] = pa.nan;
                }
            }
        }
    }
}

// y[row][col] = scale * (sum of the splits' partials, in split order) (+ bias[col]);
// RESID: y = resid[row][col] + that (resid rows at stride ldy, may alias y).
template <bool RESID>
__global__ __launch_bounds__(256) void k_skinny_reduce(const float *part, int n_split, int n_pad, int n,
                                                       float scale, const float *bias, const float *resid,
                                                       float *y, int ldy) {
    const int col = blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
    if (col >= n) return;
    const float bb = bias ? bias[col] : 0.f;  // requested with the partials
    const float rv = RESID ? resid[(size_t)row * ldy + col] : 0.f;
    const float *p = part + (size_t)row * n_pad + col;
    const size_t st = (size_t)SK_ROWS * n_pad;
    float s = 0.f;
#pragma unroll 8
    for (int i = 0; i < n_split; i++) s += p[i * st];
    float v = s * scale;
    if (bias) v = v + bb;
    if (RESID) v = rv + v;  // llama.rs:556-569: x + o, x + down
    y[(size_t)row * ldy + col] = v;
}

// Fused gate/up rows (gate[2t], gate[2t+1], up[2t], up[2t+1] in groups of four):
// y[row][j] = silu(sg * gate_j) * (su * up_j), j < n (cpu.rs:666-678).
__global__ __launch_bounds__(256) void k_skinny_reduce_swiglu(const float *part, int n_split, int n_pad, int n,
                                                              float sg, float su, float *y, int ldy) {
    const int j = blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
    if (j >= n) return;
    const int cg = (j >> 1) * 4 + (j & 1);
    const float *p = part + (size_t)row * n_pad + cg;
    const size_t st = (size_t)SK_ROWS * n_pad;
    float g = 0.f, u = 0.f;
#pragma unroll 8
    for (int i = 0; i < n_split; i++) {
        g += p[i * st];
        u += p[i * st + 2];
    }
    y[(size_t)row * ldy + j] = silu_f(g * sg) * (u * su);
}

struct SkPlan {
    int ks, kblocks, n_split, tiles, n_pad;
};

// min_wg: below this many workgroups at 8 k-blocks per split, splits take 4.
// The bf16-plane kernel was tuned at 512. The int8-digit kernel of the fused
// form at 256: its qkv and o launches (4 rows, Llama-3-8B shape) then run with
// 8 partials per column instead of 16, 4 x 64 batched decode 197.65 ->
// 195.7 ms.
SkPlan plan(int k, int n, size_t min_wg = 512) {
    SkPlan p;
    p.kblocks = (k + 63) / 64;
    p.tiles = (n + SK_COLS - 1) / SK_COLS;
    p.n_pad = p.tiles * SK_COLS;
    p.ks = 8;
    if ((size_t)p.tiles * ((p.kblocks + 7) / 8) < min_wg) p.ks = 4;  // enough workgroups to stream the weights
    p.n_split = (p.kblocks + p.ks - 1) / p.ks;
    return p;
}

template <int KS, bool B32, bool NORM = false>
int launch_ks(const SkArgs &a, int tiles, hipStream_t s) {
    if (a.m <= 4)
        hipLaunchKernelGGL((k_skinny<KS, B32, NORM, 4>), dim3(tiles * a.n_split), dim3(SK_NT), 0, s, a);
    else
        hipLaunchKernelGGL((k_skinny<KS, B32, NORM, 16>), dim3(tiles * a.n_split), dim3(SK_NT), 0, s, a);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

template <int KS, bool NORM>
int launch_dg(const SkArgs &a, hipStream_t s) {
    const dim3 grid(a.tiles * a.n_split);
    if (a.m <= 4)
        hipLaunchKernelGGL((k_skinny_dg<KS, NORM, 4>), grid, dim3(SK_NT), 0, s, a);
    else
        hipLaunchKernelGGL((k_skinny_dg<KS, NORM, 16>), grid, dim3(SK_NT), 0, s, a);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

template <bool NORM>
int launch_main(const SkArgs &a, int ks, bool b32, hipStream_t s) {
    if (!b32) return ks == 8 ? launch_dg<8, NORM>(a, s) : launch_dg<4, NORM>(a, s);
    if (ks == 8) return b32 ? launch_ks<8, true, NORM>(a, a.tiles, s) : launch_ks<8, false, NORM>(a, a.tiles, s);
    return b32 ? launch_ks<4, true, NORM>(a, a.tiles, s) : launch_ks<4, false, NORM>(a, a.tiles, s);
}

template <int EPI>
int launch_epi(const SkArgs &a, hipStream_t s) {
    hipLaunchKernelGGL((k_skinny_epi<EPI>), dim3(a.tiles), dim3(SK_NT), 0, s, a);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace

bool skinny_route(int m, int k, int n) {
    return m >= SKINNY_MIN_M && m <= SK_ROWS && k % 8 == 0 && k >= 256 && n >= 256;
}

size_t skinny_ws_bytes(int m, int k, int n) {
    (void)m;
    const SkPlan p = plan(k, n);
    return sizeof(float) * (size_t)p.n_split * SK_ROWS * p.n_pad;
}

int launch_skinny(const SkinnyMM &mm, float *ws, size_t ws_bytes, hipStream_t s) {
    const Packed &w = *mm.w;
    if (w.bf16 || (w.fused ? (!mm.swiglu || w.rows != 2 * w.n || w.rows % 4 != 0) : (mm.swiglu || w.rows != w.n)))
        return set_error(SCRY_ERR_UNSUPPORTED,
                         "skinny matmul: int8 weight rows only (the fused gate/up pair with the swiglu output)");
    if (mm.swiglu && (mm.bias || mm.resid))
        return set_error(SCRY_ERR_INVALID, "skinny matmul: swiglu output takes no bias or residual");
    if (mm.m < 1 || mm.m > SK_ROWS || mm.ldx < w.k || mm.ldy < w.n)
        return set_error(SCRY_ERR_INVALID, "skinny matmul: %d rows (1..%d), ldx %d, ldy %d", mm.m, SK_ROWS,
                         mm.ldx, mm.ldy);
    if (w.k % 8 != 0) return set_error(SCRY_ERR_UNSUPPORTED, "skinny matmul: k %% 8 != 0");
    if (w.kp < w.k || (size_t)w.rows * w.kp > 0x7fffffffu || (size_t)mm.m * mm.ldx * 4 > 0x7fffffffu)
        return set_error(SCRY_ERR_UNSUPPORTED, "skinny matmul: operands above the 2 GiB buffer range");
    const SkPlan p = plan(w.k, w.rows);
    if (ws_bytes < skinny_ws_bytes(mm.m, w.k, w.rows))
        return set_error(SCRY_ERR_INVALID, "skinny matmul: workspace too small");
    SkArgs a;
    a.x = mm.x;
    a.ldx = mm.ldx;
    a.m = mm.m;
    a.k = w.k;
    a.w = w.d;
    a.kp = w.kp;
    a.n = w.rows;
    a.s32 = w.s32;
    a.nb = w.nb;
    a.part = ws;
    a.n_pad = p.n_pad;
    a.n_split = p.n_split;
    a.kblocks = p.kblocks;
    const bool b32 = w.s32 != nullptr;
    const int rc = p.ks == 8 ? (b32 ? launch_ks<8, true>(a, p.tiles, s) : launch_ks<8, false>(a, p.tiles, s))
                             : (b32 ? launch_ks<4, true>(a, p.tiles, s) : launch_ks<4, false>(a, p.tiles, s));
    if (rc) return rc;
    const dim3 grid((w.n + 255) / 256, mm.m);
    if (mm.swiglu) {  // block-32 scales are applied per block by k_skinny
        hipLaunchKernelGGL(k_skinny_reduce_swiglu, grid, dim3(256), 0, s, ws, p.n_split, p.n_pad, w.n,
                           b32 ? 1.0f : w.scale, b32 ? 1.0f : w.scale2, mm.y, mm.ldy);
    } else if (mm.resid) {
        hipLaunchKernelGGL(k_skinny_reduce<true>, grid, dim3(256), 0, s, ws, p.n_split, p.n_pad, w.n,
                           b32 ? 1.0f : w.scale, mm.bias, mm.resid, mm.y, mm.ldy);
    } else {
        hipLaunchKernelGGL(k_skinny_reduce<false>, grid, dim3(256), 0, s, ws, p.n_split, p.n_pad, w.n,
                           b32 ? 1.0f : w.scale, mm.bias, mm.resid, mm.y, mm.ldy);
    }
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int skinny_tiles(const Packed &w) { return plan(w.k, w.rows).tiles; }

int launch_skinny_fused(const SkinnyFused &f, float *ws, size_t ws_bytes, hipStream_t s, SkinnyParts *parts) {
    const Packed &w = *f.w;
    const bool sw = f.epi == SKE_SWIGLU;
    if (f.epi < SKE_NONE || f.epi > SKE_LOGITS || (f.epi == SKE_NONE) != (parts != nullptr))
        return set_error(SCRY_ERR_INVALID, "skinny: epilogue %d", f.epi);
    if (w.bf16 || (w.fused ? (!sw || w.rows != 2 * w.n || w.rows % 4 != 0) : (sw || w.rows != w.n)))
        return set_error(SCRY_ERR_UNSUPPORTED,
                         "skinny matmul: int8 weight rows only (the fused gate/up pair with the swiglu output)");
    if (f.m < 1 || f.m > SK_ROWS || f.ldx < w.k || !f.x || (f.epi != SKE_NONE && (f.ldy < w.n || !f.y)))
        return set_error(SCRY_ERR_INVALID, "skinny matmul: %d rows (1..%d), ldx %d, ldy %d", f.m, SK_ROWS, f.ldx,
                         f.ldy);
    if (w.k % 8 != 0) return set_error(SCRY_ERR_UNSUPPORTED, "skinny matmul: k %% 8 != 0");
    if (w.kp < w.k || (size_t)w.rows * w.kp > 0x7fffffffu || (size_t)f.m * f.ldx * 4 > 0x7fffffffu)
        return set_error(SCRY_ERR_UNSUPPORTED, "skinny matmul: operands above the 2 GiB buffer range");
    if (f.norm_w && (!f.ss_in || f.n_ss_in < 1 || f.n_ss_in > 64))
        return set_error(SCRY_ERR_INVALID, "skinny matmul: RMSNorm input needs 1..64 partial sums per row");
    if (f.epi == SKE_LOGITS && (!f.pv || !f.pi || !f.pn))
        return set_error(SCRY_ERR_INVALID, "skinny matmul: logits epilogue needs argmax partials");
    // the workspace bound below holds: 256 gives no more splits than 512
    const SkPlan p = plan(w.k, w.rows, w.s32 ? 512 : 256);
    if (ws_bytes < skinny_ws_bytes(f.m, w.k, w.rows))
        return set_error(SCRY_ERR_INVALID, "skinny matmul: workspace too small");
    const bool b32 = w.s32 != nullptr;
    SkArgs a{};
    a.x = f.x;
    a.ldx = f.ldx;
    a.m = f.m;
    a.k = w.k;
    a.w = w.d;
    a.kp = w.kp;
    a.n = w.rows;
    a.s32 = w.s32;
    a.nb = w.nb;
    a.part = ws;
    a.n_pad = p.n_pad;
    a.n_split = p.n_split;
    a.kblocks = p.kblocks;
    a.g = f.norm_w;
    a.ss_in = f.norm_w ? f.ss_in : nullptr;
    a.n_ss_in = f.n_ss_in;
    a.eps = f.eps;
    a.tiles = p.tiles;
    a.n_out = w.n;
    a.scale = b32 ? 1.f : w.scale;  // block-32 scales are applied per block
    a.scale2 = b32 ? 1.f : (sw ? w.scale2 : w.scale);
    a.y = f.y;
    a.ldy = f.ldy;
    a.ss_out = f.ss_out;
    a.pv = f.pv;
    a.pi = f.pi;
    a.pn = f.pn;
    SCRY_TRY(f.norm_w ? launch_main<true>(a, p.ks, b32, s) : launch_main<false>(a, p.ks, b32, s));
    if (parts) {
        parts->n_split = p.n_split;
        parts->n_pad = p.n_pad;
        parts->scale = a.scale;
        return SCRY_OK;
    }
    switch (f.epi) {
        case SKE_STORE: return launch_epi<SKE_STORE>(a, s);
        case SKE_RESID: return launch_epi<SKE_RESID>(a, s);
        case SKE_SWIGLU: return launch_epi<SKE_SWIGLU>(a, s);
        default: return launch_epi<SKE_LOGITS>(a, s);
    }
}

}  // namespace scry
