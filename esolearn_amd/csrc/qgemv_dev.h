// W8A32 quantized GEMV / skinny GEMM for gfx950, with the decode-step fusions.
//
// Computes, for each activation row x and output j,
//   y[j] = scale * sum_p x[p] * q[p, j]            (matmul_i8_f32, cpu.rs:1128-1160)
// from the GEMV stream layout (one row of kp bytes per output j, byte = q + 128).
//
// Work split: a workgroup of NW waves owns NW * RWT consecutive output rows,
// each wave RWT rows over the whole k range.  Per 1024-wide k chunk a lane
// loads 16 consecutive weight bytes of each of its rows (one wave-wide
// buffer_load_dwordx4 reads 1 KiB contiguous) and four float4 activation
// fragments from LDS.  Each byte is converted with a single byte-select
// convert (v_cvt_f32_ubyte*) and FMA'd.
//
// Prologue (one barrier): the activation row is staged in LDS with a
// permutation that makes the float4 reads conflict-free; while staging, each
// quad of threads also writes the sum of the 16 values a consumer lane reads
// per chunk.  Those per-lane sums remove the +128 bias inside the final wave
// reduction (sum_p (q+128) x - 128 sum_p x) and are the block-32 group sums.
// The first PF chunks of every row are requested before the staging, so the
// weight stream is in flight during it.  Rows past the end load a valid row
// (and are never stored): a load that is out of range for every lane can
// complete out of order and release a partial vmcnt wait too early.
//
// RMSNorm (rmsnorm.rs, cpu.rs:574-599) is applied as y = rstd * (W (x*g)):
//   PRO_NORM   stages x*g and reduces sum(x^2) itself (the first layer, whose
//              activation is the embedding row);
//   PRO_NORMP  stages x*g written by the producing residual GEMV, with rstd
//              from that GEMV's per-workgroup sum(x^2) partials.
// Both sums of squares are reduced after the staging barrier, in a fixed order.
//
// bf16 weights (the reference's bf16 feature, cuda.rs:1206-1290) take the
// same path with a weight type WT = WT_BF16: rows of bf16 values (512 per
// 1 KiB chunk), and activations normalised (with the RMSNorm prologues) and
// rounded with the reference's bf16 cast while they are staged, since the
// reference's bf16 matmul rounds its activation operand.  Each product of two
// bf16 values is exact in f32; the accumulation is f32.
//
// Epilogues fused into the same pass (llama.rs:371-511):
//   EPI_STORE   y = acc (+ bias)                     -- matmul_i8_f32[_bias]
//   EPI_RESID   y = resid + acc; optionally x*g_next and sum(y^2) per workgroup
//               for the next RMSNorm'd GEMV          -- o_proj / down_proj + residual add
//   EPI_SWIGLU  h = silu(gate) * up on interleaved rows -- gate/up + swiglu
//   EPI_QKV     RoPE(Q)*1/sqrt(hd), RoPE(K), K/V appended to the cache row
//   EPI_LOGITS  logits + this workgroup's ordered argmax partial
// The row-combining epilogues exchange row values through LDS.
//
// This header holds the workgroup body (qgemv_block) and its argument block;
// qgemv.hip wraps the body in the k_qgemv kernel and holds the launchers.
#pragma once
#include "internal.h"
#include "kdev.h"

namespace scry {

// The fields the prologue needs come first: the kernel fetches them together.
struct KArgs {
    const uint8_t *W;
    const float *x;
    const float *ss_in;
    const float *norm_w;
    int k, kp, rows, nch;
    int ldx, m, n_ss;
    float eps;
    const float *s32;
    int nb;
    float scale, scale2;
    const float *embed;
    const int64_t *tokens;
    DevState *state;
    float *y;
    int ldy;
    const float *resid;
    const float *bias;
    float *xg_out;
    const float *g_next;
    float *ss_out;
    float *q_out, *k_cache, *v_cache;
    const float2 *rope_cs;
    int q_dim, kv_dim, head_dim;
    float q_scale;
    float *part_val;
    int *part_idx, *part_nan;
    unsigned long long *ts;  // step profile stamps (null: off)
};

// activation prologues
enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_NORMP = 2 };
// weight types
enum { WT_I8 = 0, WT_I8B32 = 1, WT_BF16 = 2 };

// Checks a decode GEMV's arguments and fills the kernel arguments, the weight
// type, the 1 KiB chunk count per row and the activation prologue
// (qgemv.hip).
int qgemv_kargs(int epi, const GemvArgs &g, KArgs *ka, int *wt, int *nch, int *pro);

namespace {

using namespace dev;
constexpr int SSW = 2;  // PRO_NORMP partial sums per thread (n_ss <= SSW * threads)

// Launch shape for a chunk count (0: runtime loop) and activation rows per
// pass.  Measured on the Llama-2-7B decode shapes (one launch of 4096 x 22016
// int8 weights: 4 rows per wave x 4 waves 17.7 us, 1 row per wave x 8 waves
// 15.0 us): single-row waves keep more loads in flight per CU and finish
// evenly.  The MT > 1 and runtime-k paths keep 4 rows per wave, which shares
// each LDS activation read between 4 rows.
struct Shape {
    int rwt, nw, pf;  // rows per wave, waves per workgroup, chunks in flight per row
};
constexpr Shape shape_for(int nch, int mt) {
    return mt > 1      ? Shape{4, 4, 4}
           : nch == 4  ? Shape{1, 8, 4}
           : nch == 11 ? Shape{1, 8, 11}  // down (k = 11008): every chunk in flight
           : nch == 14 ? Shape{1, 8, 7}
           : nch == 8  ? Shape{1, 8, 8}  // bf16 rows, k = 4096
           : nch == 22 ? Shape{1, 8, 8}  // bf16 rows, k = 11008
           : nch == 28 ? Shape{1, 8, 7}  // bf16 rows, k = 14336
           : nch == 0  ? Shape{1, 8, 4}  // any k, one row: 8 rows per workgroup
                       : Shape{4, 4, 4};
}

// activation values per 1 KiB weight chunk
constexpr int chunk_vals(int wt) { return wt == WT_BF16 ? 512 : 1024; }

// Activation row source for row mr (nullptr if mr >= m).  Only the
// self-contained RMSNorm prologue (the first layer) reads the embedding row of
// the current token when x is null; with one row per pass the grid has
// exactly m rows of workgroups.  Both keep argument-dependent branches (and
// their serialized argument fetches) off the common paths.
template <int PRO, int MT>
__device__ __forceinline__ const float *act_row(const KArgs &a, int mr) {
    if (MT > 1 && mr >= a.m) return nullptr;
    if (PRO == PRO_NORM && !a.x) return a.embed + (size_t)a.tokens[a.state->pos] * a.k;
    return a.x + (size_t)mr * a.ldx;
}

// Thread t loads the float4s f4 = p*NT + t (p < XP) of a k-vector.  A wave
// whose float4s all lie past k loads nothing (zeros).
template <int XP, int NT>
__device__ __forceinline__ void load_vec(const float *src, int k, int tot4, float4 (&v)[XP]) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src, src ? (size_t)k * 4 : 0);
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < XP; p++) {
        const int f4 = p * NT + tid;
        v[p] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (src && f4 < tot4 && (f4 & ~63) * 4 < k) v[p] = bload16f(r, (unsigned)f4 << 4);
    }
}

// One 1024-wide k chunk for RWT rows and MT activation rows.
template <int MT, int WT, int RWT>
__device__ __forceinline__ void chunk_fma(const u32x4 (&w)[RWT], int c, const float *xs, int kc,
                                          const float *xsum, __amdgpu_buffer_rsrc_t sr, int nb,
                                          const int (&wrow)[RWT], int lane, float (&acc)[MT][RWT],
                                          int kp) {
    constexpr bool B32 = WT == WT_I8B32;
    if constexpr (WT == WT_BF16) {
        // lane L holds bf16 values 8L .. 8L+7 of chunk c: x at c*512 + 4L (+256)
        if ((c << 10) + (lane << 4) >= kp) return;  // past the row (the next row's bytes)
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            const float *xb = xs + mi * kc + (c << 9) + (lane << 2);
            const float4 x0 = *(const float4 *)(xb);
            const float4 x1 = *(const float4 *)(xb + 256);
#pragma unroll
            for (int r = 0; r < RWT; r++) acc[mi][r] = dot8_bf16(w[r], x0, x1, acc[mi][r]);
        }
        return;
    }
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const float *xb = xs + mi * kc + (c << 10) + (lane << 2);
        const float4 x0 = *(const float4 *)(xb);
        const float4 x1 = *(const float4 *)(xb + 256);
        const float4 x2 = *(const float4 *)(xb + 512);
        const float4 x3 = *(const float4 *)(xb + 768);
        if (!B32) {
#pragma unroll
            for (int r = 0; r < RWT; r++) acc[mi][r] = dot16(w[r], x0, x1, x2, x3, acc[mi][r]);
        } else {
            // block-32: this lane's 16 bytes are half of k-block blk
            const float gs = xsum[mi * (kc >> 4) + (c << 6) + lane];
            const int blk = ((c << 10) + (lane << 4)) >> 5;
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                const float p = dot16(w[r], x0, x1, x2, x3, 0.f);
                const float sc = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(sr, (wrow[r] * nb + blk) * 4, 0, 0));
                acc[mi][r] = fmaf(sc, fmaf(-128.f, gs, p), acc[mi][r]);
            }
        }
    }
}

// One workgroup's rows: workgroup bx of the row blocks, by of the activation
// row groups (a kernel's blockIdx, or a fused kernel's own block mapping).
template <int EPI, int PRO, int WT, int MT, int NCH>
__device__ __forceinline__ void qgemv_block(const KArgs &a, const int bx, const int by) {
    constexpr Shape S = shape_for(NCH, MT);
    constexpr int RWT = S.rwt, NW = S.nw, PF = S.pf, RPW = RWT * NW, NT = 64 * NW;
    constexpr bool B32 = WT == WT_I8B32, WB = WT == WT_BF16;
    constexpr int CV = chunk_vals(WT);  // activation values per chunk
    constexpr int XP = ((NCH > 0 ? NCH : (WB ? 32 : 16)) * (CV / 4) + NT - 1) / NT;  // float4 per thread per row
    constexpr bool NORM = PRO != PRO_PLAIN;
    static_assert(!WB || MT == 1, "bf16 weights take one activation row per pass");
    static_assert(!NORM || MT == 1, "the RMSNorm prologues take one activation row");
    static_assert(EPI == EPI_STORE || MT == 1, "only the store epilogue takes several rows");
    static_assert(EPI == EPI_STORE || EPI == EPI_RESID || RPW % 4 == 0,
                  "the SwiGLU, QKV and logits epilogues combine rows in groups of 4");
    extern __shared__ float4 dyn4[];
    const int nch = NCH > 0 ? NCH : a.nch;
    const int kc = nch * CV;
    const int tot4 = kc >> 2;  // float4 slots of one staged activation row
    float *xs = reinterpret_cast<float *>(dyn4);  // [MT][kc] permuted activation rows
    float *xsum = xs + MT * kc;                    // [MT][nch][64] per-lane 16-value sums (int8)
    __shared__ double s_ss[NW];  // per-wave sums of squares for the RMSNorm
    __shared__ float s_rstd;
    __shared__ float s_val[MT * RPW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rb = bx * RPW, row0 = rb + wave * RWT;
    const int m0 = by * MT;

    // ---- 1. activation loads (and the RMSNorm inputs), then the first PF
    // chunks of every row: waiting for the activations leaves the weight
    // stream in flight
    float4 xr[XP];
    load_vec<XP, NT>(act_row<PRO, MT>(a, m0), a.k, tot4, xr);
    float4 gw[PRO == PRO_NORM ? XP : 1];
    if constexpr (PRO == PRO_NORM) load_vec<XP, NT>(a.norm_w, a.k, tot4, gw);
    // PRO_NORMP: this thread's share of the producer's partial sums
    // (unconditional clamped loads: no wait inside a branch)
    float ssv[PRO == PRO_NORMP ? SSW : 1];
    if constexpr (PRO == PRO_NORMP) {
#pragma unroll
        for (int j = 0; j < SSW; j++) ssv[j] = a.ss_in[min(tid + NT * j, a.n_ss - 1)];
    }

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.W, (size_t)a.rows * a.kp);
    int wrow[RWT];
    unsigned woff[RWT];
#pragma unroll
    for (int r = 0; r < RWT; r++) {
        wrow[r] = min(row0 + r, a.rows - 1);
        woff[r] = (unsigned)(wrow[r] * a.kp + (lane << 4));
    }
    u32x4 wb[PF][RWT];
#pragma unroll
    for (int d = 0; d < PF; d++)
        if (NCH > 0 || d < nch) {
#pragma unroll
            for (int r = 0; r < RWT; r++) wb[d][r] = bload16(wr, woff[r] + (d << 10));
        }
    // EPI_RESID: the residual and the next norm's weight of the row this lane
    // stores, requested now (they are used after the weight stream; the row
    // is read and written by this lane only)
    float pre_r[RWT], pre_g[RWT];
    if constexpr (EPI == EPI_RESID) {
        const float *R = a.resid ? a.resid : a.embed + (size_t)a.tokens[a.state->pos] * a.rows;
#pragma unroll
        for (int r = 0; r < RWT; r++) {
            pre_r[r] = pre_g[r] = 0.f;
            if (lane == r) {
                pre_r[r] = R[wrow[r]];
                if (a.xg_out) pre_g[r] = a.g_next[wrow[r]];
            }
        }
    }

    // ---- 2. stage the activation rows into LDS with the per-lane sums
    double ssp = 0.0;
    if constexpr (WB) {
        // bf16: the RMSNorm scale first (cpu.rs:574-599; f64 sum of squares,
        // reduced in a fixed order), then each value normalised and rounded
        // with the reference's cast as it is staged
        double rstd = 1.0;
        if constexpr (NORM) {
            if constexpr (PRO == PRO_NORM) {
#pragma unroll
                for (int p = 0; p < XP; p++) {
                    const float4 v = xr[p];
                    ssp += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < SSW; j++)
                    if (tid + NT * j < a.n_ss) ssp += ssv[j];
            }
            ssp = wave_sum_d_dpp(ssp);
            if (lane == 0) s_ss[wave] = ssp;
            __syncthreads();
            double t = 0.0;
#pragma unroll
            for (int w = 0; w < NW; w++) t += s_ss[w];
            rstd = 1.0 / sqrt(t / (double)a.k + (double)a.eps);
        }
#pragma unroll
        for (int p = 0; p < XP; p++) {
            const int f4 = p * NT + tid;
            if (f4 < tot4) {
                float4 v = xr[p];
                if constexpr (PRO == PRO_NORM) {  // f32(f64(x) * rstd * f64(w))
                    v.x = (float)((double)v.x * rstd * (double)gw[p].x);
                    v.y = (float)((double)v.y * rstd * (double)gw[p].y);
                    v.z = (float)((double)v.z * rstd * (double)gw[p].z);
                    v.w = (float)((double)v.w * rstd * (double)gw[p].w);
                } else if constexpr (PRO == PRO_NORMP) {  // the producer's x * w, times rstd
                    v.x = (float)((double)v.x * rstd);
                    v.y = (float)((double)v.y * rstd);
                    v.z = (float)((double)v.z * rstd);
                    v.w = (float)((double)v.w * rstd);
                }
                v.x = bf16_cast(v.x);
                v.y = bf16_cast(v.y);
                v.z = bf16_cast(v.z);
                v.w = bf16_cast(v.w);
                // value 512c + 8L + 4j + e (lane L's j-th float4 of chunk c)
                const int c = f4 >> 7, w = f4 & 127;
                *(float4 *)(xs + (c << 9) + ((w & 1) << 8) + ((w >> 1) << 2)) = v;
            }
        }
    } else {
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        if (mi > 0) load_vec<XP, NT>(act_row<PRO, MT>(a, m0 + mi), a.k, tot4, xr);
#pragma unroll
        for (int p = 0; p < XP; p++) {
            const int f4 = p * NT + tid;
            if (f4 < nch * 256) {  // whole waves: nch * 256 is a multiple of 64
                float4 v = xr[p];
                if constexpr (PRO == PRO_NORM) {
                    ssp += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
                    v.x *= gw[p].x;
                    v.y *= gw[p].y;
                    v.z *= gw[p].z;
                    v.w *= gw[p].w;
                }
                *(float4 *)(xs + mi * kc + xslot(f4 >> 8, f4 & 255)) = v;
                // consumer lane L of chunk c reads float4s c*256 + 4L .. 4L+3:
                // the quad of threads staging them sums its 16 values
                float s = (v.x + v.y) + (v.z + v.w);
                s += __shfl_xor(s, 1);
                s += __shfl_xor(s, 2);
                if ((tid & 3) == 0) xsum[mi * (kc >> 4) + ((f4 >> 8) << 6) + ((f4 & 255) >> 2)] = s;
            }
        }
    }
    if constexpr (NORM) {
        if constexpr (PRO == PRO_NORMP) {
#pragma unroll
            for (int j = 0; j < SSW; j++)
                if (tid + NT * j < a.n_ss) ssp += ssv[j];
        }
        ssp = wave_sum_d_dpp(ssp);
        if (lane == 0) s_ss[wave] = ssp;
    }
    }  // int8 staging
    __syncthreads();
    if (NORM && !WB && wave == 0) {
        // cpu.rs:574-599: rstd = 1/sqrt(mean(x^2) + eps) in f64 (waves in order)
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < NW; w++) t += s_ss[w];
        if (lane == 0) s_rstd = (float)(1.0 / sqrt(t / (double)a.k + (double)a.eps));
    }

    // ---- 3. stream the weights
    float acc[MT][RWT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int r = 0; r < RWT; r++) acc[mi][r] = 0.f;
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.s32, B32 ? (size_t)a.rows * a.nb * sizeof(float) : 0);

    if constexpr (NCH > 0) {
        // straight-line stream: chunk c computes from wb[c % PF], then refills it
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            chunk_fma<MT, WT, RWT>(wb[c % PF], c, xs, kc, xsum, sr, a.nb, wrow, lane, acc, a.kp);
            if (c + PF < NCH) {
#pragma unroll
                for (int r = 0; r < RWT; r++) wb[c % PF][r] = bload16(wr, woff[r] + ((c + PF) << 10));
            }
        }
    } else {
        for (int c0 = 0; c0 < nch; c0 += PF) {
#pragma unroll
            for (int d = 0; d < PF; d++) {
                const int c = c0 + d;
                if (c < nch) {
                    chunk_fma<MT, WT, RWT>(wb[d], c, xs, kc, xsum, sr, a.nb, wrow, lane, acc, a.kp);
                    if (c + PF < nch) {
#pragma unroll
                        for (int r = 0; r < RWT; r++) wb[d][r] = bload16(wr, woff[r] + ((c + PF) << 10));
                    }
                }
            }
        }
    }


    // ---- 4. remove the +128 bias inside the wave reduction, apply the scales
    float val[MT][RWT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        float sxl = 0.f;
        if (WT == WT_I8)
            for (int c = 0; c < nch; c++) sxl += xsum[mi * (kc >> 4) + (c << 6) + lane];
#pragma unroll
        for (int r = 0; r < RWT; r++) {
            const float s = wave_sum(WT == WT_I8 ? fmaf(-128.f, sxl, acc[mi][r]) : acc[mi][r]);
            // fused gate/up rows come as gate, gate, up, up
            const float sc = WT != WT_I8 ? 1.f : (EPI == EPI_SWIGLU && ((row0 + r) & 2)) ? a.scale2 : a.scale;
            val[mi][r] = sc * s;
        }
    }
    if constexpr (!WB && (EPI == EPI_STORE || EPI == EPI_LOGITS)) {
        // An activation row holding an infinity or a NaN: the +128 bias
        // removal made the sum NaN (inf - inf), while the reference's sum of
        // q x is +-inf unless a NaN term or both infinities occur.  Only the
        // terms of the non-finite values decide it, so a NaN sum (uniform in
        // the wave; never the case for finite rows) scans the row's staged
        // values and classifies those terms.  Done where the sums are final
        // (matmul_i8_f32, the logits); the decode step's other projections
        // feed an RMSNorm or a softmax, which make +-inf and NaN alike NaN.
        {
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
#pragma unroll
                for (int r = 0; r < RWT; r++) {
                    if (!isnan(val[mi][r])) continue;
                    const float sc = WT != WT_I8 ? 1.f : (EPI == EPI_SWIGLU && ((row0 + r) & 2)) ? a.scale2 : a.scale;
                    int cls = 0;  // +inf, -inf, NaN terms seen
#pragma unroll 1
                    for (int j = lane; j < a.k; j += 64) {
                        const float x = xs[mi * kc + xslot(j >> 10, (j >> 2) & 255) + (j & 3)];
                        if (!isfinite(x)) {
                            const int q = (int)(signed char)(a.W[(size_t)wrow[r] * a.kp + j] ^ 0x80);
                            const float ws = B32 ? a.s32[(size_t)wrow[r] * a.nb + (j >> 5)] : sc;
                            const float t = x * ((float)q * ws);
                            cls |= isnan(t) ? 4 : t > 0.f ? 1 : 2;
                        }
                    }
#pragma unroll
                    for (int off = 32; off > 0; off >>= 1) cls |= __shfl_xor(cls, off);
                    if (cls) val[mi][r] = (cls & 4) || cls == 3 ? __builtin_nanf("") : cls == 1 ? INFINITY : -INFINITY;
                }
            }
        }
    }

    // ---- 5. epilogues
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESID) {
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            const int mr = m0 + mi;
            // lane r stores row r (static indices: no private-array select)
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                const int row = row0 + r;
                if (lane == r && mr < a.m && row < a.rows) {
                    float v = val[mi][r];
                    if constexpr (EPI == EPI_STORE) {
                        if (a.bias) v = v + a.bias[row];
                    } else {
                        v = pre_r[r] + v;  // (EPI_RESID has one activation row: mr == 0)
                        if (a.xg_out) a.xg_out[row] = v * pre_g[r];
                        s_val[wave * RWT + r] = v;
                    }
                    a.y[(size_t)mr * a.ldy + row] = v;
                }
            }
        }
        if constexpr (EPI == EPI_RESID) {
            if (a.ss_out) {  // uniform: the next RMSNorm's sum of squares, in row order
                __syncthreads();
                if (tid == 0) {
                    double t = 0.0;
                    for (int i = 0; i < RPW && rb + i < a.rows; i++) t += (double)s_val[i] * s_val[i];
                    a.ss_out[bx] = (float)t;
                }
            }
        }
        return;
    } else {
#pragma unroll
        for (int r = 0; r < RWT; r++)
            if (lane == r) s_val[wave * RWT + r] = val[0][r];
        __syncthreads();
    }
    const float rs = (NORM && !WB) ? s_rstd : 1.f;  // bf16: normalised while staged
    if constexpr (EPI == EPI_SWIGLU) {
        // rows 4i..4i+3 = gate[2i], gate[2i+1], up[2i], up[2i+1]
        if (tid < RPW / 2 && rb + 2 * tid < a.rows) {
            const int q = (tid >> 1) * 4 + (tid & 1);
            a.y[(rb >> 1) + tid] = silu_f(s_val[q] * rs) * (s_val[q + 2] * rs);
        }
    } else if constexpr (EPI == EPI_QKV) {
        const int j = rb + 2 * tid;
        if (tid < RPW / 2 && j < a.rows) {
            const float x0 = s_val[2 * tid] * rs, x1 = s_val[2 * tid + 1] * rs;
            const int pos = a.state->pos, crow = a.state->cache_len;
            const int hh = a.head_dim >> 1;
            if (j < a.q_dim + a.kv_dim) {
                const bool isq = j < a.q_dim;
                const int jj = isq ? j : j - a.q_dim;
                const float2 cs = a.rope_cs[(size_t)pos * hh + ((jj % a.head_dim) >> 1)];
                // cpu.rs:655-658 in f32, no contraction
                const float r0 = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
                const float r1 = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
                if (isq) {
                    a.q_out[jj] = __fmul_rn(r0, a.q_scale);
                    a.q_out[jj + 1] = __fmul_rn(r1, a.q_scale);
                } else {
                    float *kr = a.k_cache + (size_t)crow * a.kv_dim;
                    kr[jj] = r0;
                    kr[jj + 1] = r1;
                }
            } else {
                const int jj = j - a.q_dim - a.kv_dim;
                float *vr = a.v_cache + (size_t)crow * a.kv_dim;
                vr[jj] = x0;
                vr[jj + 1] = x1;
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        // logits + this workgroup's ordered argmax partial (no fences: the
        // finish kernel that reduces the partials is the next launch)
        if (tid < RPW && rb + tid < a.rows) a.y[rb + tid] = s_val[tid] * rs;
        if (tid == 0) {
            ArgAcc p{0.f, -1, -1};
            for (int t = 0; t < RPW; t++) {
                const int row = rb + t;
                if (row >= a.rows) break;
                const float v = s_val[t] * rs;
                if (isnan(v)) {
                    p.nan = row;
                    continue;
                }
                if (p.i < 0 || !(p.v > v)) {
                    p.v = v;
                    p.i = row;
                }
            }
            a.part_val[bx] = p.v;
            a.part_idx[bx] = p.i;
            a.part_nan[bx] = p.nan;
        }
    }
}

// ---- split-k single-row GEMV (one activation row, NCH chunks of 1 KiB,
// k % 16 == 0; int8 per-tensor or block-32 weights, or bf16 rows).
//
// A workgroup of NCH / CPW * RG waves holds RG row groups of R rows; wave
// (g, cw) streams chunks cw + j NCH / CPW (j < CPW) of its group's rows.  For
// each of them lane L keeps the activation values under its 16 weight bytes
// (int8: x[1024 c + 16 L .. + 15]; bf16: x[512 c + 8 L .. + 7]) in registers,
// read straight from memory next to its weight requests (one 16-byte load per
// row and chunk), so each activation value is read once per workgroup, and
// the int8 stream needs no LDS stage and no barrier before it (the bf16
// RMSNorm scale is formed first: one barrier while the weights are in flight).  A lane's per-row partials are reduced over the wave by
// a transposed butterfly (R rows in log2(R) halving exchanges, then the rest
// of the wave inside 64 / R lane groups), and the chunk partials of a row meet
// in LDS at the single barrier; wave 0 sums them in chunk order and runs the
// epilogue with one row per lane.
template <int CTRL>
__device__ __forceinline__ float dpp_addf(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// a + b over lane pairs l, l ^ O: lanes with bit O clear keep a's pair sums,
// the others b's (O = 8 by DPP row_ror:8 within a 16-lane row, else ds_bpermute)
template <int O>
__device__ __forceinline__ float sk_pair(float a, float b, int lane) {
    const bool hi = (lane & O) != 0;
    const float keep = hi ? b : a, send = hi ? a : b;
    if constexpr (O == 8)
        return keep + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, send), 0x128, 0xF, 0xF, true));
    else
        return keep + __shfl_xor(send, O);
}

// Sum over the wave of each of R per-lane values: returns, in every lane, the
// total of value index sk_row(lane).  log2(R) halving exchanges, then the
// 64 / R lanes left holding parts of one value by DPP.
template <int R>
__device__ __forceinline__ float sk_reduce(const float (&v)[R], int lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8, "rows per wave: 1, 2, 4 or 8");
    float t;
    if constexpr (R == 8) {
        const float u0 = sk_pair<32>(v[0], v[4], lane), u1 = sk_pair<32>(v[1], v[5], lane);
        const float u2 = sk_pair<32>(v[2], v[6], lane), u3 = sk_pair<32>(v[3], v[7], lane);
        t = sk_pair<8>(sk_pair<16>(u0, u2, lane), sk_pair<16>(u1, u3, lane), lane);
    } else if constexpr (R == 4) {
        t = sk_pair<16>(sk_pair<32>(v[0], v[2], lane), sk_pair<32>(v[1], v[3], lane), lane);
    } else if constexpr (R == 2) {
        t = sk_pair<32>(v[0], v[1], lane);
    } else {
        t = v[0];
    }
    constexpr int G = 64 / R;
    if constexpr (G >= 2) t = dpp_addf<0xB1>(t);   // quad_perm [1,0,3,2]
    if constexpr (G >= 4) t = dpp_addf<0x4E>(t);   // quad_perm [2,3,0,1]
    if constexpr (G >= 8) t = dpp_addf<0x141>(t);  // row_half_mirror
    if constexpr (G >= 16) t = dpp_addf<0x140>(t); // row_mirror
    if constexpr (G >= 32) t += __shfl_xor(t, 16);
    if constexpr (G >= 64) t += __shfl_xor(t, 32);
    return t;
}
// the value index a lane holds after sk_reduce: lane bits 5, 4, 3 from the top
template <int R>
__device__ __forceinline__ int sk_row(int lane) {
    return R == 8 ? (((lane >> 5) & 1) << 2) | (((lane >> 4) & 1) << 1) | ((lane >> 3) & 1)
           : R == 4 ? (((lane >> 5) & 1) << 1) | ((lane >> 4) & 1)
           : R == 2 ? (lane >> 5) & 1
                    : 0;
}

template <int EPI, int PRO, int WT, int NCH, int RG, int R, int CPW>
__device__ __forceinline__ void qgemv_sk_block(const KArgs &a, const int bx) {
    constexpr int NWC = NCH / CPW, NW = NWC * RG, RPW = RG * R, NT = 64 * NW;
    static_assert(NCH % CPW == 0 && NW <= 16 && RPW <= 64, "split-k shape");
    constexpr bool NORM = PRO != PRO_PLAIN, WB = WT == WT_BF16, B32 = WT == WT_I8B32;
    constexpr int XF = WB ? 2 : 4;       // float4 of activations per lane and chunk
    constexpr int CV = WB ? 512 : 1024;  // activation values per chunk
    __shared__ float s_part[RPW][NWC];
    __shared__ double s_ss[NW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cw = wave % NWC, g = wave / NWC;  // chunks cw + j NWC of row group g
    const int rb = bx * RPW, row0 = rb + g * R;

    // ---- 1. this lane's activation values, the RMSNorm inputs, the weights
    const float *src = act_row<PRO, 1>(a, 0);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(src, (size_t)a.k * 4);
    float4 x[CPW][XF];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const unsigned xo = (unsigned)(((cw + j * NWC) * CV + lane * 4 * XF) * 4);
#pragma unroll
        for (int f = 0; f < XF; f++) x[j][f] = bload16f(xr, xo + 16 * f);  // past k: zeros
    }
    float4 gw[PRO == PRO_NORM ? CPW : 1][PRO == PRO_NORM ? XF : 1];
    if constexpr (PRO == PRO_NORM) {
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.norm_w, (size_t)a.k * 4);
#pragma unroll
        for (int j = 0; j < CPW; j++) {
            const unsigned xo = (unsigned)(((cw + j * NWC) * CV + lane * 4 * XF) * 4);
#pragma unroll
            for (int f = 0; f < XF; f++) gw[j][f] = bload16f(gr, xo + 16 * f);
        }
    }
    float ssv[PRO == PRO_NORMP ? SSW : 1];
    if constexpr (PRO == PRO_NORMP) {
#pragma unroll
        for (int j = 0; j < SSW; j++) ssv[j] = a.ss_in[min(tid + NT * j, a.n_ss - 1)];
    }
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.W, (size_t)a.rows * a.kp);
    u32x4 w[CPW][R];
#pragma unroll
    for (int j = 0; j < CPW; j++)
#pragma unroll
        for (int r = 0; r < R; r++)
            w[j][r] = bload16(wr, (unsigned)(min(row0 + r, a.rows - 1) * a.kp) + (unsigned)((cw + j * NWC) << 10) +
                                      (unsigned)(lane << 4));
    // block-32: the scale of the 32-value block this lane's 16 bytes are half of
    float bs[B32 ? CPW : 1][B32 ? R : 1];
    if constexpr (B32) {
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s32, (size_t)a.rows * a.nb * sizeof(float));
#pragma unroll
        for (int j = 0; j < CPW; j++)
#pragma unroll
            for (int r = 0; r < R; r++)
                bs[j][r] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(
                               sr, (min(row0 + r, a.rows - 1) * a.nb + (cw + j * NWC) * 32 + (lane >> 1)) * 4, 0, 0));
    }
    // EPI_RESID: the residual and the next norm's weight of the row lane t of
    // wave 0 finishes (clamped: unconditional loads)
    float pre_r = 0.f, pre_g = 0.f;
    if constexpr (EPI == EPI_RESID) {
        const int er = min(rb + min(lane, RPW - 1), a.rows - 1);
        const float *Rs = a.resid ? a.resid : a.embed + (size_t)a.tokens[a.state->pos] * a.rows;
        pre_r = Rs[er];
        if (a.xg_out) pre_g = a.g_next[er];
    }

    // ---- 2. the RMSNorm's sum of squares (its loads were issued first)
    if constexpr (NORM) {
        double ssp = 0.0;
        if constexpr (PRO == PRO_NORMP) {
#pragma unroll
            for (int j = 0; j < SSW; j++)
                if (tid + NT * j < a.n_ss) ssp += ssv[j];
        } else if (g == 0) {  // one row group covers the row once
#pragma unroll
            for (int j = 0; j < CPW; j++)
#pragma unroll
                for (int f = 0; f < XF; f++)
                    ssp += (double)x[j][f].x * x[j][f].x + (double)x[j][f].y * x[j][f].y +
                           (double)x[j][f].z * x[j][f].z + (double)x[j][f].w * x[j][f].w;
        }
        ssp = wave_sum_d_dpp(ssp);
        if (lane == 0) s_ss[wave] = ssp;
    }
    if constexpr (WB) {
        // bf16 (cpu.rs:574-599, cuda.rs:1206-1290): each activation value is
        // normalised, then rounded with the reference's cast, before the
        // products, so rstd is formed first (one barrier; the weights are in
        // flight): f32(f64(x) rstd f64(w)) for the embedding row, f32(f64(x g)
        // rstd) from the residual GEMV's row
        double rstd = 1.0;
        if constexpr (NORM) {
            __syncthreads();
            double t = 0.0;
#pragma unroll
            for (int ww = 0; ww < NW; ww++) t += s_ss[ww];
            rstd = 1.0 / sqrt(t / (double)a.k + (double)a.eps);
        }
#pragma unroll
        for (int j = 0; j < CPW; j++)
#pragma unroll
            for (int f = 0; f < XF; f++) {
                float4 v = x[j][f];
                if constexpr (PRO == PRO_NORM) {
                    v.x = (float)((double)v.x * rstd * (double)gw[j][f].x);
                    v.y = (float)((double)v.y * rstd * (double)gw[j][f].y);
                    v.z = (float)((double)v.z * rstd * (double)gw[j][f].z);
                    v.w = (float)((double)v.w * rstd * (double)gw[j][f].w);
                } else if constexpr (PRO == PRO_NORMP) {
                    v.x = (float)((double)v.x * rstd);
                    v.y = (float)((double)v.y * rstd);
                    v.z = (float)((double)v.z * rstd);
                    v.w = (float)((double)v.w * rstd);
                }
                x[j][f] = make_float4(bf16_cast(v.x), bf16_cast(v.y), bf16_cast(v.z), bf16_cast(v.w));
            }
    } else if constexpr (PRO == PRO_NORM) {
#pragma unroll
        for (int j = 0; j < CPW; j++)
#pragma unroll
            for (int f = 0; f < XF; f++) {
                x[j][f].x *= gw[j][f].x;
                x[j][f].y *= gw[j][f].y;
                x[j][f].z *= gw[j][f].z;
                x[j][f].w *= gw[j][f].w;
            }
    }

    // ---- 3. the stream: int8, sum_p (q + 128) x_p - 128 sum_p x_p per row
    // (block-32: per 16-value half block, scaled); bf16, the products of the
    // rounded values (lanes past the row's kp bytes read the next row's bytes
    // against zero activations: their weights are dropped, since bf16 bits
    // can be infinite)
    float xs[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        xs[j] = 0.f;
        if constexpr (!WB) {
#pragma unroll
            for (int f = 0; f < XF; f++) xs[j] += (x[j][f].x + x[j][f].y) + (x[j][f].z + x[j][f].w);
        }
    }
    float p[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < CPW; j++) {
            if constexpr (WB) {
                const bool in = ((cw + j * NWC) << 10) + (lane << 4) < a.kp;
                const u32x4 wv = in ? w[j][r] : u32x4{0u, 0u, 0u, 0u};
                acc = dot8_bf16(wv, x[j][0], x[j][1], acc);
            } else if constexpr (B32) {
                acc = fmaf(bs[j][r], fmaf(-128.f, xs[j], dot16(w[j][r], x[j][0], x[j][1], x[j][2], x[j][3], 0.f)), acc);
            } else {
                acc = dot16(w[j][r], x[j][0], x[j][1], x[j][2], x[j][3], acc);
            }
        }
        if constexpr (WT == WT_I8) {
            float xt = 0.f;
#pragma unroll
            for (int j = 0; j < CPW; j++) xt += xs[j];
            acc = fmaf(-128.f, xt, acc);
        }
        p[r] = acc;
    }
    const float tot = sk_reduce<R>(p, lane);
    if ((lane & (64 / R - 1)) == 0) s_part[g * R + sk_row<R>(lane)][cw] = tot;
    __syncthreads();
    if (wave != 0) return;

    // ---- 4. wave 0: row rb + lane, its chunks summed in order, scaled
    const int row = rb + lane;
    const bool live = lane < RPW && row < a.rows;
    float s = 0.f;
    if (lane < RPW) {
#pragma unroll
        for (int cc = 0; cc < NWC; cc++) s += s_part[lane][cc];
    }
    // int8 per tensor: the tensor scale (gate / up rows of the fused layout);
    // block-32 and bf16 products are already scaled
    const float sc = WT != WT_I8 ? 1.f : (EPI == EPI_SWIGLU && (row & 2)) ? a.scale2 : a.scale;
    float val = sc * s;
    float rs = 1.f;  // int8: the RMSNorm scale applied to the dot products
    if constexpr (NORM && !WB) {
        double t = 0.0;
#pragma unroll
        for (int ww = 0; ww < NW; ww++) t += s_ss[ww];
        rs = (float)(1.0 / sqrt(t / (double)a.k + (double)a.eps));
    }
    if constexpr (!WB && (EPI == EPI_STORE || EPI == EPI_LOGITS)) {
        // a non-finite activation: the reference's sum of q x from the
        // non-finite terms alone (see qgemv_block), one row at a time
        unsigned long long bad = __ballot(live && isnan(val));
        while (bad) {
            const int t = __builtin_ctzll(bad);
            bad &= bad - 1;
            int cls = 0;
            const size_t wrow_t = (size_t)(rb + t) * a.kp;
#pragma unroll 1
            for (int j = lane; j < a.k; j += 64) {
                float xv = src[j];
                if constexpr (PRO == PRO_NORM) xv *= a.norm_w[j];
                if (!isfinite(xv)) {
                    const int q = (int)(signed char)(a.W[wrow_t + j] ^ 0x80);
                    const float ws = B32 ? a.s32[(size_t)(rb + t) * a.nb + (j >> 5)] : a.scale;
                    const float tt = xv * ((float)q * ws);
                    cls |= isnan(tt) ? 4 : tt > 0.f ? 1 : 2;
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) cls |= __shfl_xor(cls, off);
            if (lane == t && cls) val = (cls & 4) || cls == 3 ? __builtin_nanf("") : cls == 1 ? INFINITY : -INFINITY;
        }
    }

    // ---- 5. epilogues (lane t: row rb + t)
    if constexpr (EPI == EPI_STORE) {
        if (live) a.y[row] = a.bias ? val + a.bias[row] : val;
    } else if constexpr (EPI == EPI_RESID) {
        const float v = pre_r + val;
        if (live) {
            if (a.xg_out) a.xg_out[row] = v * pre_g;
            a.y[row] = v;
        }
        if (a.ss_out) {  // the next RMSNorm's sum of squares over this workgroup's rows
            const double q = wave_sum_d_dpp(live ? (double)v * v : 0.0);
            if (lane == 0) a.ss_out[bx] = (float)q;
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        // rows 4i..4i+3 = gate[2i], gate[2i+1], up[2i], up[2i+1]
        const int qg = (lane >> 1) * 4 + (lane & 1);
        const float gv = __shfl(val, qg & 63), uv = __shfl(val, (qg + 2) & 63);
        if (lane < RPW / 2 && rb + 2 * lane < a.rows) a.y[(rb >> 1) + lane] = silu_f(gv * rs) * (uv * rs);
    } else if constexpr (EPI == EPI_QKV) {
        const float x0 = __shfl(val, (2 * lane) & 63) * rs, x1 = __shfl(val, (2 * lane + 1) & 63) * rs;
        const int j = rb + 2 * lane;
        if (lane < RPW / 2 && j < a.rows) {
            const int pos = a.state->pos, crow = a.state->cache_len;
            const int hh = a.head_dim >> 1;
            if (j < a.q_dim + a.kv_dim) {
                const bool isq = j < a.q_dim;
                const int jj = isq ? j : j - a.q_dim;
                const float2 cs = a.rope_cs[(size_t)pos * hh + ((jj % a.head_dim) >> 1)];
                // cpu.rs:655-658 in f32, no contraction
                const float r0 = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
                const float r1 = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
                if (isq) {
                    a.q_out[jj] = __fmul_rn(r0, a.q_scale);
                    a.q_out[jj + 1] = __fmul_rn(r1, a.q_scale);
                } else {
                    float *kr = a.k_cache + (size_t)crow * a.kv_dim;
                    kr[jj] = r0;
                    kr[jj + 1] = r1;
                }
            } else {
                const int jj = j - a.q_dim - a.kv_dim;
                float *vr = a.v_cache + (size_t)crow * a.kv_dim;
                vr[jj] = x0;
                vr[jj + 1] = x1;
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        const float v = val * rs;
        if (live) a.y[row] = v;
        // this workgroup's argmax partial: the order-free combine over its rows
        ArgAcc acc{0.f, -1, -1};
        if (live) {
            if (isnan(v)) acc.nan = row;
            else acc = ArgAcc{v, row, -1};
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            ArgAcc o;
            o.v = __shfl_xor(acc.v, off);
            o.i = __shfl_xor(acc.i, off);
            o.nan = __shfl_xor(acc.nan, off);
            acc = arg_combine(acc, o);
        }
        if (lane == 0) {
            a.part_val[bx] = acc.v;
            a.part_idx[bx] = acc.i;
            a.part_nan[bx] = acc.nan;
        }
    }
}

}  // namespace
}  // namespace scry
