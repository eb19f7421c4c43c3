// W8A32 quantized GEMV / skinny GEMM for gfx950, with the decode-step fusions.
//
// Computes, for each activation row x and output j,
//   y[j] = scale * sum_p x[p] * q[p, j]            (matmul_i8_f32, cpu.rs:1128-1160)
// from the GEMV stream layout (one row of kp bytes per output j, byte = q + 128).
//
// Work split: a 256-thread workgroup owns 16 output rows, each wave 4 rows
// over the whole k range.  Per 1024-wide k chunk a lane loads 16 consecutive
// weight bytes of each of its 4 rows (global_load_dwordx4; one wave-wide load
// reads 1 KiB contiguous) and four float4 activation fragments from LDS.
// The activation row is staged in LDS once per workgroup with a permutation
// that makes those float4 reads conflict-free.  Each byte is converted with a
// single byte-select convert (v_cvt_f32_ubyte*) and FMA'd; the +128 bias is
// removed once per row as 128 * sum(x).  The first PF chunks of weights are
// requested before the activation staging, so the weight stream starts while
// the (optional fused RMSNorm) prologue runs.
//
// Epilogues fused into the same pass (llama.rs:371-511):
//   EPI_STORE   y = acc (+ bias)                     -- matmul_i8_f32[_bias]
//   EPI_RESID   y = resid + acc                      -- o_proj / down_proj + residual add
//   EPI_SWIGLU  h = silu(gate) * up on interleaved rows -- gate/up + swiglu
//   EPI_QKV     RoPE(Q)*1/sqrt(hd), RoPE(K), K/V appended to the cache row
//   EPI_LOGITS  logits + device argmax (last-arriving workgroup) + step advance
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

constexpr int RW = 4;    // rows per wave (default; the residual GEMVs pick fewer)
constexpr int RPB = 16;  // rows per workgroup at RW
constexpr int PF4 = 4;   // chunks in flight per row (runtime-chunk path, k <= 4096)

struct KArgs {
    const uint8_t *W;
    int k, kp, rows, nch;
    const float *s32;
    int nb;
    float scale, scale2;
    const float *x;
    int ldx, m;
    const float *embed;
    const int64_t *tokens;
    DevState *state;
    const float *norm_w;
    float eps;
    float *y;
    int ldy;
    const float *resid;
    const float *bias;
    float *q_out, *k_cache, *v_cache;
    const float2 *rope_cs;
    int q_dim, kv_dim, head_dim;
    float q_scale;
    float *part_val;
    int *part_idx, *part_nan;
};

// activation prologues
enum { PRO_PLAIN = 0, PRO_NORM = 1 };

// Activation row source for row mr (nullptr if mr >= m).
__device__ __forceinline__ const float *act_row(const KArgs &a, int mr) {
    if (mr >= a.m) return nullptr;
    return a.x ? a.x + (size_t)mr * a.ldx : a.embed + (size_t)a.tokens[a.state->pos] * a.k;
}

// Thread t loads x[p*1024 + 4t .. +3] for p < XP (zero past k).
template <int XP>
__device__ __forceinline__ void load_x(const float *src, int k, float4 (&xr)[XP]) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src, src ? (size_t)k * 4 : 0);
#pragma unroll
    for (int p = 0; p < XP; p++) xr[p] = bload16f(r, (unsigned)((p << 12) + (threadIdx.x << 4)));
}


// One 1024-wide k chunk for RWT rows and MT activation rows.
template <int MT, bool B32, int RWT>
__device__ __forceinline__ void chunk_fma(const u32x4 (&w)[RWT], int c, const float *xs, int kc,
                                          const float *xg, __amdgpu_buffer_rsrc_t sr, int nb,
                                          int row0, int lane, float (&acc)[MT][RWT]) {
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
            const float gs = xg[mi * (kc >> 4) + (c << 6) + lane];
            const int blk = ((c << 10) + (lane << 4)) >> 5;
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                const float p = dot16(w[r], x0, x1, x2, x3, 0.f);
                const float sc = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(sr, ((row0 + r) * nb + blk) * 4, 0, 0));
                acc[mi][r] = fmaf(sc, fmaf(-128.f, gs, p), acc[mi][r]);
            }
        }
    }
}

// RWT rows per wave (4 * RWT per workgroup), PFT chunks in flight per row.
template <int EPI, int PRO, bool B32, int MT, int NCH, int RWT = RW, int PFT = PF4>
__global__ __launch_bounds__(TPB) void k_qgemv(KArgs a) {
    static_assert(RWT == RW || EPI == EPI_RESID || EPI == EPI_STORE,
                  "the SwiGLU, QKV and logits epilogues work on 4-row groups");
    constexpr bool NORM = PRO == PRO_NORM;
    constexpr int XP = NCH > 0 ? NCH : 16;
    constexpr int PF = PFT;
    extern __shared__ float4 dyn4[];
    float *xs = reinterpret_cast<float *>(dyn4);
    const int kc = (NCH > 0 ? NCH : a.nch) << 10;
    float *xg = xs + MT * kc;  // B32: per-16 group sums
    __shared__ double red_d[4];
    __shared__ float sx_sh[MT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * (4 * RWT) + wave * RWT;
    const int m0 = blockIdx.y * MT;

    // ---- 1. activation loads first, then the first PF weight chunks: waiting
    // for the activations then leaves the weight stream in flight.
    float4 xr[XP];
    load_x<XP>(act_row(a, m0), a.k, xr);
    float4 nw[NORM ? XP : 1];
    if (NORM) load_x<XP>(a.norm_w, a.k, reinterpret_cast<float4(&)[XP]>(nw));

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.W, (size_t)a.rows * a.kp);
    unsigned woff[RWT];
#pragma unroll
    for (int r = 0; r < RWT; r++)  // rows past the end read zeros (never stored)
        woff[r] = (row0 + r) < a.rows ? (unsigned)((row0 + r) * a.kp + (lane << 4)) : 0x80000000u;
    u32x4 wb[PF][RWT];
#pragma unroll
    for (int d = 0; d < PF; d++)
#pragma unroll
        for (int r = 0; r < RWT; r++) wb[d][r] = bload16(wr, woff[r] + (d << 10));

    // ---- 2. stage the activation rows (optionally RMSNorm'd) into LDS
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        if (mi > 0) load_x<XP>(act_row(a, m0 + mi), a.k, xr);
        float *xrow = xs + mi * kc;
        double acc2 = 0.0;
#pragma unroll
        for (int p = 0; p < XP; p++) {
            const float4 v = xr[p];
            if (NORM)
                acc2 += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
            else
                acc2 += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
        }
        double tot = block_sum_d(acc2, red_d);
        if (NORM) {
            // cpu.rs:574-599: rstd = 1/sqrt(mean(x^2) + eps) in f64; out = f32(x*rstd*w)
            const double rstd = 1.0 / sqrt(tot / (double)a.k + (double)a.eps);
            double sx = 0.0;
#pragma unroll
            for (int p = 0; p < XP; p++) {
                const float4 w4 = nw[NORM ? p : 0];
                float4 v = xr[p];
                v.x = (float)((double)v.x * rstd * (double)w4.x);
                v.y = (float)((double)v.y * rstd * (double)w4.y);
                v.z = (float)((double)v.z * rstd * (double)w4.z);
                v.w = (float)((double)v.w * rstd * (double)w4.w);
                xr[p] = v;
                sx += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
            }
            tot = block_sum_d(sx, red_d);
        }
#pragma unroll
        for (int p = 0; p < XP; p++)
            if (NCH > 0 || p < a.nch) *(float4 *)(xrow + xslot(p, tid)) = xr[p];
        if (tid == 0) sx_sh[mi] = (float)tot;
    }
    __syncthreads();
    if (B32) {
        const int ng = kc >> 4;
        for (int t = tid; t < MT * ng; t += TPB) {
            const int mi = t / ng, g = t % ng;
            const int c = g >> 6, L = g & 63;
            const float *xq = xs + mi * kc + (c << 10) + (L << 2);
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int e = 0; e < 4; e++) s += xq[(q << 8) + e];
            xg[t] = s;
        }
        __syncthreads();
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
            chunk_fma<MT, B32, RWT>(wb[c % PF], c, xs, kc, xg, sr, a.nb, row0, lane, acc);
            if (c + PF < NCH) {
#pragma unroll
                for (int r = 0; r < RWT; r++) wb[c % PF][r] = bload16(wr, woff[r] + ((c + PF) << 10));
            }
        }
    } else {
        for (int c0 = 0; c0 < a.nch; c0 += PF) {
#pragma unroll
            for (int d = 0; d < PF; d++) {
                const int c = c0 + d;
                if (c < a.nch) {
                    chunk_fma<MT, B32, RWT>(wb[d], c, xs, kc, xg, sr, a.nb, row0, lane, acc);
                    if (c + PF < a.nch) {
#pragma unroll
                        for (int r = 0; r < RWT; r++) wb[d][r] = bload16(wr, woff[r] + ((c + PF) << 10));
                    }
                }
            }
        }
    }

    // ---- 4. reduce over the wave, remove the +128 bias, apply the scale
    float val[MT][RWT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const float corr = 128.f * sx_sh[mi];
#pragma unroll
        for (int r = 0; r < RWT; r++) {
            const float s = wave_sum(acc[mi][r]);
            if (B32) {
                val[mi][r] = s;
            } else {
                const float sc = (EPI == EPI_SWIGLU && r >= 2) ? a.scale2 : a.scale;
                val[mi][r] = sc * (s - corr);
            }
        }
    }

    // ---- 5. epilogues
    if (EPI == EPI_STORE || EPI == EPI_RESID) {
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            const int mr = m0 + mi;
            // lane r stores row r (static indices: no private-array select)
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                const int row = row0 + r;
                if (lane == r && mr < a.m && row < a.rows) {
                    float v = val[mi][r];
                    if (EPI == EPI_STORE) {
                        if (a.bias) v = v + a.bias[row];
                        a.y[(size_t)mr * a.ldy + row] = v;
                    } else {
                        const float *R = a.resid ? a.resid + (size_t)mr * a.ldy
                                                 : a.embed + (size_t)a.tokens[a.state->pos] * a.rows;
                        a.y[(size_t)mr * a.ldy + row] = R[row] + v;
                    }
                }
            }
        }
    } else if (EPI == EPI_SWIGLU) {
        // wave rows = gate[2t], gate[2t+1], up[2t], up[2t+1]
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            const int mr = m0 + mi;
            if (lane < 2 && mr < a.m && row0 < a.rows) {
                const float g = lane ? val[mi][1] : val[mi][0];
                const float u = lane ? val[mi][3] : val[mi][2];
                const int t = (row0 >> 1) + lane;  // (row0/4)*2 + lane
                a.y[(size_t)mr * a.ldy + t] = silu_f(g) * u;
            }
        }
    } else if (EPI == EPI_QKV) {
        if (lane < 2) {
            const int j = row0 + 2 * lane;
            if (j < a.rows) {
                const float x0 = lane ? val[0][2] : val[0][0];
                const float x1 = lane ? val[0][3] : val[0][1];
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
        }
    } else if (EPI == EPI_LOGITS) {
        // logits + this workgroup's ordered argmax partial (no fences: the
        // finish kernel that reduces the partials is the next launch)
        __shared__ float s_v[RPB];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (lane == r) {
                if (row0 + r < a.rows) a.y[row0 + r] = val[0][r];
                s_v[wave * RW + r] = val[0][r];
            }
        }
        __syncthreads();
        if (tid == 0) {
            ArgAcc p{0.f, -1, -1};
            for (int t = 0; t < RPB; t++) {
                const int row = blockIdx.x * RPB + t;
                if (row >= a.rows) break;
                const float v = s_v[t];
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

template <int EPI, int PRO, bool B32, int MT, int NCH, int RWT = RW, int PFT = PF4>
int launch_t(const KArgs &ka, hipStream_t s) {
    const int kc = ka.nch << 10;
    size_t lds = (size_t)MT * kc * sizeof(float) + (B32 ? (size_t)MT * (kc >> 4) * sizeof(float) : 0);
    dim3 grid((ka.rows + 4 * RWT - 1) / (4 * RWT), (ka.m + MT - 1) / MT);
    hipLaunchKernelGGL((k_qgemv<EPI, PRO, B32, MT, NCH, RWT, PFT>), grid, dim3(TPB), lds, s, ka);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

// NCH = compile-time chunk count (straight-line stream) for the k on the
// Llama path; 0 = runtime loop for any other k <= 16384.
// The residual GEMVs of the decode step (o_proj, down_proj: 4096 outputs)
// have few rows per launch: fewer rows per wave put more waves on each CU,
// and for long rows every chunk is requested at once (measured on the 7B
// shapes: o 5.6 -> 5.3 us with 2 rows per wave, down 12.9 -> 10.5 us with one
// row per wave and all 11 chunks in flight).
template <int EPI, int PRO, bool B32, int MT>
int launch_nch(const KArgs &ka, hipStream_t s) {
    constexpr bool resid1 = EPI == EPI_RESID && MT == 1;
    switch (ka.nch) {
        case 1: return launch_t<EPI, PRO, B32, MT, 1>(ka, s);
        case 4:
            if constexpr (resid1) return launch_t<EPI, PRO, B32, MT, 4, 2, 4>(ka, s);
            return launch_t<EPI, PRO, B32, MT, 4>(ka, s);
        case 11:
            if constexpr (resid1) return launch_t<EPI, PRO, B32, MT, 11, 1, 11>(ka, s);
            if (MT == 1) return launch_t<EPI, PRO, B32, MT, 11>(ka, s);
            break;
        case 14:
            if constexpr (resid1) return launch_t<EPI, PRO, B32, MT, 14, 1, 14>(ka, s);
            if (MT == 1) return launch_t<EPI, PRO, B32, MT, 14>(ka, s);
            break;
        default: break;
    }
    return launch_t<EPI, PRO, B32, MT, 0>(ka, s);
}

template <int EPI, int PRO, bool B32>
int launch_mt(const KArgs &ka, hipStream_t s) {
    // skinny GEMM: MT activation rows share one weight pass (k <= 4096 keeps
    // MT * k floats within the 64 KiB LDS stage)
    if constexpr (EPI == EPI_STORE) {
        if (ka.m >= 4 && ka.nch <= 4) return launch_nch<EPI, PRO, B32, 4>(ka, s);
        if (ka.m >= 2 && ka.nch <= 4) return launch_nch<EPI, PRO, B32, 2>(ka, s);
    }
    return launch_nch<EPI, PRO, B32, 1>(ka, s);
}

template <int EPI>
int launch_e(const KArgs &ka, bool norm, bool b32, hipStream_t s) {
    // decode epilogues QKV/SWIGLU/LOGITS always take the fused RMSNorm
    constexpr bool kNorm = (EPI == EPI_QKV || EPI == EPI_SWIGLU || EPI == EPI_LOGITS);
    if (norm != kNorm)
        return set_error(SCRY_ERR_INVALID, "qgemv: epilogue %d %s a fused RMSNorm", EPI,
                         kNorm ? "requires" : "does not take");
    if constexpr (kNorm) {
        return b32 ? launch_mt<EPI, PRO_NORM, true>(ka, s) : launch_mt<EPI, PRO_NORM, false>(ka, s);
    } else {
        return b32 ? launch_mt<EPI, PRO_PLAIN, true>(ka, s) : launch_mt<EPI, PRO_PLAIN, false>(ka, s);
    }
}

}  // namespace

int launch_qgemv(int epi, const GemvArgs &g, hipStream_t s) {
    const Packed &w = *g.w;
    if (w.kp % 16 != 0 || w.k > w.kp) return set_error(SCRY_ERR_INVALID, "qgemv: bad packed layout");
    if (w.bytes() >= 0x7fffffffull)  // buffer offsets are 32-bit
        return set_error(SCRY_ERR_UNSUPPORTED, "qgemv: %zu weight bytes (limit 2 GiB per tensor)", w.bytes());
    const int nch = (w.k + 1023) / 1024;
    if (nch > 16 || (size_t)nch * 1024 * sizeof(float) * (w.s32 ? 17 : 16) / 16 > 64 * 1024)
        return set_error(SCRY_ERR_UNSUPPORTED, "qgemv: k=%d exceeds the LDS activation stage", w.k);
    if (epi == EPI_SWIGLU && (w.fused != 1 || w.rows % 4 != 0))
        return set_error(SCRY_ERR_INVALID, "qgemv: swiglu epilogue needs the fused gate/up layout");
    if ((epi == EPI_QKV || epi == EPI_LOGITS) && g.m != 1)
        return set_error(SCRY_ERR_INVALID, "qgemv: decode epilogues take one activation row");
    if (g.m < 1) return set_error(SCRY_ERR_INVALID, "qgemv: m must be >= 1");
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
    ka.y = g.y;
    ka.ldy = g.ldy;
    ka.resid = g.resid;
    ka.bias = g.bias;
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
    const bool norm = g.norm_w != nullptr;
    const bool b32 = w.s32 != nullptr;
    switch (epi) {
        case EPI_STORE: return launch_e<EPI_STORE>(ka, norm, b32, s);
        case EPI_RESID: return launch_e<EPI_RESID>(ka, norm, b32, s);
        case EPI_SWIGLU: return launch_e<EPI_SWIGLU>(ka, norm, b32, s);
        case EPI_QKV: return launch_e<EPI_QKV>(ka, norm, b32, s);
        case EPI_LOGITS: return launch_e<EPI_LOGITS>(ka, norm, b32, s);
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
    const int per = (np + TPB - 1) / TPB;
    ArgAcc acc{0.f, -1, -1};
    for (int t = tid * per; t < min(np, tid * per + per); t++) acc = arg_combine(acc, ArgAcc{pv[t], pi[t], pn[t]});
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
    const int np = (g.w->rows + RPB - 1) / RPB;
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
