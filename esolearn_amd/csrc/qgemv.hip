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
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

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
};

// activation prologues
enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_NORMP = 2 };
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
           : nch == 11 ? Shape{1, 8, 8}
           : nch == 14 ? Shape{1, 8, 7}
           : nch == 8  ? Shape{1, 8, 8}  // bf16 rows, k = 4096
           : nch == 22 ? Shape{1, 8, 8}  // bf16 rows, k = 11008
           : nch == 28 ? Shape{1, 8, 7}  // bf16 rows, k = 14336
           : nch == 0  ? Shape{1, 8, 4}  // any k, one row: 8 rows per workgroup
                       : Shape{4, 4, 4};
}

// weight types
enum { WT_I8 = 0, WT_I8B32 = 1, WT_BF16 = 2 };
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

template <int EPI, int PRO, int WT, int MT, int NCH>
__global__ __launch_bounds__(64 * shape_for(NCH, MT).nw) void k_qgemv(KArgs a) {
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
    const int rb = blockIdx.x * RPW, row0 = rb + wave * RWT;
    const int m0 = blockIdx.y * MT;

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
                    a.ss_out[blockIdx.x] = (float)t;
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
            a.part_val[blockIdx.x] = p.v;
            a.part_idx[blockIdx.x] = p.i;
            a.part_nan[blockIdx.x] = p.nan;
        }
    }
}

// Compile-time chunk count (straight-line stream) for the k on the Llama
// paths; 0 = runtime loop.  Several activation rows share a weight pass only
// in the store epilogue with k <= 4096.
struct Sel {
    int nch_t, mt;
};
Sel select_cfg(int epi, int nch, int m, int wt) {
    if (wt == WT_BF16) {  // one activation row per pass; the Llama k's compiled
        const int nt = (nch == 8 || nch == 22 || nch == 28) ? nch : 0;
        return {nt, 1};
    }
    int mt = 1;
    if (epi == EPI_STORE && nch <= 4) mt = m >= 4 ? 4 : (m >= 2 ? 2 : 1);
    int nt = 0;
    if (nch == 1 || nch == 4) nt = nch;
    if ((nch == 11 || nch == 14) && mt == 1 && (epi == EPI_STORE || epi == EPI_RESID)) nt = nch;
    return {nt, mt};
}

size_t lds_bytes(int epi, int nch, int mt, int pro, int wt) {
    const Shape S = shape_for(select_cfg(epi, nch, mt, wt).nch_t, mt);
    const size_t dyn = wt == WT_BF16 ? (size_t)nch * 512 * sizeof(float)
                                     : (size_t)mt * nch * 1024 * sizeof(float) * 17 / 16;
    (void)pro;
    const size_t stat = S.nw * sizeof(double) +
                        (size_t)mt * S.rwt * S.nw * sizeof(float);
    return dyn + stat;
}

constexpr size_t kLdsMax = 160 * 1024;  // gfx950 LDS per workgroup

template <int EPI, int PRO, int WT, int MT, int NCH>
int launch_t(const KArgs &ka, hipStream_t s) {
    constexpr Shape S = shape_for(NCH, MT);
    const size_t lds = WT == WT_BF16 ? (size_t)ka.nch * 512 * sizeof(float)
                                     : (size_t)MT * (ka.nch << 10) * sizeof(float) * 17 / 16;
    if (lds > 64 * 1024) {  // above the default dynamic LDS limit
        static bool attr = false;
        if (!attr) {
            const size_t stat = lds_bytes(EPI, ka.nch, MT, PRO, WT) - lds;
            SCRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_qgemv<EPI, PRO, WT, MT, NCH>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kLdsMax - stat)));
            attr = true;
        }
    }
    dim3 grid((ka.rows + S.rwt * S.nw - 1) / (S.rwt * S.nw), (ka.m + MT - 1) / MT);
    hipLaunchKernelGGL((k_qgemv<EPI, PRO, WT, MT, NCH>), grid, dim3(64 * S.nw), lds, s, ka);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

template <int EPI, int PRO, int WT, int MT>
int launch_nch(const KArgs &ka, int nch_t, hipStream_t s) {
    if constexpr (WT == WT_BF16) {
        switch (nch_t) {
            case 8: return launch_t<EPI, PRO, WT, MT, 8>(ka, s);
            case 22: return launch_t<EPI, PRO, WT, MT, 22>(ka, s);
            case 28: return launch_t<EPI, PRO, WT, MT, 28>(ka, s);
            default: return launch_t<EPI, PRO, WT, MT, 0>(ka, s);
        }
    } else {
        switch (nch_t) {
            case 1: return launch_t<EPI, PRO, WT, MT, 1>(ka, s);
            case 4: return launch_t<EPI, PRO, WT, MT, 4>(ka, s);
            default: break;
        }
        if constexpr (MT == 1 && (EPI == EPI_STORE || EPI == EPI_RESID)) {
            if (nch_t == 11) return launch_t<EPI, PRO, WT, MT, 11>(ka, s);
            if (nch_t == 14) return launch_t<EPI, PRO, WT, MT, 14>(ka, s);
        }
        return launch_t<EPI, PRO, WT, MT, 0>(ka, s);
    }
}

template <int EPI, int PRO, int WT>
int launch_mt(const KArgs &ka, Sel sel, hipStream_t s) {
    if constexpr (EPI == EPI_STORE && WT != WT_BF16) {
        if (sel.mt == 4) return launch_nch<EPI, PRO, WT, 4>(ka, sel.nch_t, s);
        if (sel.mt == 2) return launch_nch<EPI, PRO, WT, 2>(ka, sel.nch_t, s);
    }
    return launch_nch<EPI, PRO, WT, 1>(ka, sel.nch_t, s);
}

template <int EPI, int PRO>
int launch_wt(const KArgs &ka, int wt, Sel sel, hipStream_t s) {
    if (wt == WT_BF16) return launch_mt<EPI, PRO, WT_BF16>(ka, sel, s);
    if (wt == WT_I8B32) return launch_mt<EPI, PRO, WT_I8B32>(ka, sel, s);
    return launch_mt<EPI, PRO, WT_I8>(ka, sel, s);
}

template <int EPI>
int launch_e(const KArgs &ka, int pro, int wt, Sel sel, hipStream_t s) {
    // the decode epilogues QKV/SWIGLU/LOGITS always take a fused RMSNorm
    constexpr bool kNorm = (EPI == EPI_QKV || EPI == EPI_SWIGLU || EPI == EPI_LOGITS);
    if ((pro != PRO_PLAIN) != kNorm)
        return set_error(SCRY_ERR_INVALID, "qgemv: epilogue %d %s a fused RMSNorm", EPI,
                         kNorm ? "requires" : "does not take");
    if constexpr (kNorm) {
        if (pro == PRO_NORMP) return launch_wt<EPI, PRO_NORMP>(ka, wt, sel, s);
        return launch_wt<EPI, PRO_NORM>(ka, wt, sel, s);
    } else {
        return launch_wt<EPI, PRO_PLAIN>(ka, wt, sel, s);
    }
}

int weight_type(const Packed &w) { return w.bf16 ? WT_BF16 : (w.s32 ? WT_I8B32 : WT_I8); }
// 1 KiB weight chunks per row
int row_chunks(const Packed &w) { return (w.bf16 ? 2 * w.k + 1023 : w.k + 1023) / 1024; }

}  // namespace

int qgemv_blocks(int epi, const Packed &w, int m) {
    const Sel sel = select_cfg(epi, row_chunks(w), m, weight_type(w));
    const Shape S = shape_for(sel.nch_t, sel.mt);
    return (w.rows + S.rwt * S.nw - 1) / (S.rwt * S.nw);
}

int launch_qgemv(int epi, const GemvArgs &g, hipStream_t s) {
    const Packed &w = *g.w;
    if (w.kp % 16 != 0 || w.k > w.kp) return set_error(SCRY_ERR_INVALID, "qgemv: bad packed layout");
    if (w.bytes() >= 0x7fffffffull)  // buffer offsets are 32-bit
        return set_error(SCRY_ERR_UNSUPPORTED, "qgemv: %zu weight bytes (limit 2 GiB per tensor)", w.bytes());
    if (g.m < 1) return set_error(SCRY_ERR_INVALID, "qgemv: m must be >= 1");
    if (!g.x && !(g.norm_w && g.embed && g.tokens && g.state && g.m == 1))
        return set_error(SCRY_ERR_INVALID, "qgemv: no activation (only the fused RMSNorm reads the embedding row)");
    const int wt = weight_type(w);
    const int nch = row_chunks(w);
    const int pro = g.ss_in ? PRO_NORMP : g.norm_w ? PRO_NORM : PRO_PLAIN;
    const Sel sel = select_cfg(epi, nch, g.m, wt);
    if (nch > (wt == WT_BF16 ? 32 : 16) || lds_bytes(epi, nch, sel.mt, pro, wt) > kLdsMax)
        return set_error(SCRY_ERR_UNSUPPORTED, "qgemv: k=%d exceeds the LDS activation stage", w.k);
    if (wt == WT_BF16 && (g.m != 1 || w.kp != 2 * round_up(w.k, 8)))
        return set_error(SCRY_ERR_INVALID, "qgemv: bf16 rows take one activation row and a 16-byte row pad");
    if (epi == EPI_SWIGLU && (w.fused != 1 || w.rows % 4 != 0))
        return set_error(SCRY_ERR_INVALID, "qgemv: swiglu epilogue needs the fused gate/up layout");
    if ((epi == EPI_QKV || epi == EPI_LOGITS || epi == EPI_SWIGLU || epi == EPI_RESID) && g.m != 1)
        return set_error(SCRY_ERR_INVALID, "qgemv: decode epilogues take one activation row");
    if (epi == EPI_QKV && (w.rows % 2 != 0 || g.head_dim % 2 != 0 || g.q_dim % 2 != 0 || g.kv_dim % 2 != 0))
        return set_error(SCRY_ERR_INVALID, "qgemv: qkv epilogue needs even head, q and kv sizes");
    const int max_ss = SSW * 64 * shape_for(sel.nch_t, sel.mt).nw;
    if (g.ss_in && (g.n_ss < 1 || g.n_ss > max_ss || g.norm_w))
        return set_error(SCRY_ERR_INVALID,
                         "qgemv: pre-scaled RMSNorm input needs 1..%d partial sums and no norm weight", max_ss);
    if (epi == EPI_RESID && (!g.xg_out != !g.g_next || !g.xg_out != !g.ss_out))
        return set_error(SCRY_ERR_INVALID, "qgemv: residual RMSNorm outputs come together");
    KArgs ka{};
    ka.W = w.d;
    ka.k = w.k;
    ka.kp = w.kp;
    ka.rows = w.rows;
    ka.nch = nch;
    ka.s32 = w.s32;
    ka.nb = w.nb;
    ka.scale = w.scale;
    ka.scale2 = w.scale2;
    ka.x = g.x;
    ka.ldx = g.ldx;
    ka.m = g.m;
    ka.embed = g.embed;
    ka.tokens = g.tokens;
    ka.state = g.state;
    ka.norm_w = g.norm_w;
    ka.eps = g.eps;
    ka.ss_in = g.ss_in;
    ka.n_ss = g.n_ss;
    ka.y = g.y;
    ka.ldy = g.ldy;
    ka.resid = g.resid;
    ka.bias = g.bias;
    ka.xg_out = g.xg_out;
    ka.g_next = g.g_next;
    ka.ss_out = g.ss_out;
    ka.q_out = g.q_out;
    ka.k_cache = g.k_cache;
    ka.v_cache = g.v_cache;
    ka.rope_cs = g.rope_cs;
    ka.q_dim = g.q_dim;
    ka.kv_dim = g.kv_dim;
    ka.head_dim = g.head_dim;
    ka.q_scale = g.q_scale;
    ka.part_val = g.part_val;
    ka.part_idx = g.part_idx;
    ka.part_nan = g.part_nan;
    switch (epi) {
        case EPI_STORE: return launch_e<EPI_STORE>(ka, pro, wt, sel, s);
        case EPI_RESID: return launch_e<EPI_RESID>(ka, pro, wt, sel, s);
        case EPI_SWIGLU: return launch_e<EPI_SWIGLU>(ka, pro, wt, sel, s);
        case EPI_QKV: return launch_e<EPI_QKV>(ka, pro, wt, sel, s);
        case EPI_LOGITS: return launch_e<EPI_LOGITS>(ka, pro, wt, sel, s);
    }
    return set_error(SCRY_ERR_INVALID, "qgemv: unknown epilogue %d", epi);
}

// Ordered device argmax over one vector (generate.rs:167-173).
namespace {
__global__ __launch_bounds__(TPB) void k_argmax(const float *__restrict__ x, int n, int64_t *out) {
    __shared__ ArgAcc sh[TPB];
    ArgAcc r = block_argmax_range(x, 0, n, sh);
    int tok = argmax_finish(r, x, n, sh);
    if (threadIdx.x == 0) *out = (n <= 0) ? 0 : tok;
}
}  // namespace

// End of a decode step: reduce the LM head's per-workgroup argmax partials in
// index order (one workgroup), then record the token and advance the state.
namespace {
__global__ __launch_bounds__(TPB) void k_logits_finish(const float *__restrict__ logits, int V,
                                                       const float *__restrict__ pv,
                                                       const int *__restrict__ pi,
                                                       const int *__restrict__ pn, int np,
                                                       DevState *st, int64_t *tokens,
                                                       int64_t *argmax_out, int advance) {
    __shared__ ArgAcc sh[TPB];
    const int tid = threadIdx.x;
    // thread t combines partials t, t + TPB, ... (coalesced; arg_combine is
    // order-free), FP at a time with every load of a batch issued first
    constexpr int FP = 16;
    ArgAcc acc{0.f, -1, -1};
    for (int t0 = tid; t0 < np; t0 += FP * TPB) {
        ArgAcc q[FP];
#pragma unroll
        for (int j = 0; j < FP; j++) {
            const int t = min(t0 + j * TPB, np - 1);  // clamped: unconditional loads
            q[j] = ArgAcc{pv[t], pi[t], pn[t]};
        }
#pragma unroll
        for (int j = 0; j < FP; j++)
            if (t0 + j * TPB < np) acc = arg_combine(acc, q[j]);
    }
    const ArgAcc r = block_argmax(acc, sh);
    const int tok = argmax_finish(r, logits, V, sh);
    if (tid == 0) {
        const int p = st->pos;
        if (argmax_out) argmax_out[0] = tok;
        if (advance) {
            if (p + 1 <= st->max_tokens && p + 1 >= st->n_prompt) tokens[p + 1] = tok;
            st->pos = p + 1;
            st->cache_len = st->cache_len + 1;
        }
    }
}
}  // namespace

int launch_logits_finish(const GemvArgs &g, hipStream_t s) {
    const int np = qgemv_blocks(EPI_LOGITS, *g.w, 1);
    hipLaunchKernelGGL(k_logits_finish, dim3(1), dim3(TPB), 0, s, g.y, g.w->rows, g.part_val,
                       g.part_idx, g.part_nan, np, g.state, g.tokens_rw, g.argmax_out, g.advance);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_argmax(const float *x, int64_t n, int64_t *out, hipStream_t s) {
    if (n > 0x7fffffff) return set_error(SCRY_ERR_UNSUPPORTED, "argmax: n too large");
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(TPB), 0, s, x, (int)n, out);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
