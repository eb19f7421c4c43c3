// Decode attention over the device KV cache (one query token, GQA), replacing
// the reference's per-token sequence (llama.rs:411-455):
//   gather_reshape_repeat_kv (cpu.rs:707-730) x2, strided-batched Q.K^T
//   (gemv_trans_b, cpu.rs:825-842), softmax (cpu.rs:336-366), strided-batched
//   P.V (gemv_into, cpu.rs:846-871).
// Q arrives pre-scaled by 1/sqrt(hd) and RoPE'd (fused into the QKV GEMV).
//
// The cache is read in place ([max_seq, n_kv*hd] rows, no repeat_kv copy):
// one workgroup handles KV head g and position split s for all n_rep query
// heads of the group, so each K/V row is read once per group.  Splits write
// (max, sum, unnormalised output); the last split of a group to finish merges
// the group's splits (log-sum-exp rescaling, in split order) into the
// attention output row.
//
// The exchange stays inside one XCD's L2: workgroups are dispatched to the
// XCDs round-robin by linear block id, and the 1-D grid gives every split of
// group g the same block id mod 8, so all of them (their partial stores, the
// group's arrival counter, and the last arrival's L1-bypassing loads) meet in
// the same L2.  A split's stores are complete in L2 before its counter
// increment.  The split count is fixed per cache, so the launch shape does
// not depend on the current length and the kernel can live in a replayed
// graph; the length comes from the device state.
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

// device-scope load: misses the CU's L1 and reads the L2 the other splits
// stored to (a vector load: scalar loads would go through the scalar cache)
__device__ __forceinline__ float cload(const float *p) {
    return __builtin_bit_cast(float, __hip_atomic_load((const unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

constexpr int MAX_SPLITS = 16;  // attn_pick_splits never picks more

// v + v of the lane the DPP control names (within a row of 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of G lanes, every lane of a group left with it.
// DPP: lane pairs and quads by quad permutes, then the other half of each
// 8-lane and 16-lane block by the half-row and row mirrors (each half is
// uniform by then), ds_bpermute only across rows: a fifth of the LDS-pipe
// shuffles, for more DPP wait states on the dependent chain.  Measured: with
// four query heads per KV head (4 x 64 batched decode) 203.4 -> 200.8 ms;
// with one (Llama-2-7B decode) 574.4 -> 571.3 tok/s, so that shape keeps the
// butterfly of ds_bpermute shuffles.
template <int G, bool DPP>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (DPP) {
        if constexpr (G >= 2) v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
        if constexpr (G >= 4) v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
        if constexpr (G >= 8) v = dpp_add<0x141>(v);  // row_half_mirror
        if constexpr (G >= 16) v = dpp_add<0x140>(v); // row_mirror
#pragma unroll
        for (int off = 16; off < G; off <<= 1) v += __shfl_xor(v, off);
    } else {
#pragma unroll
        for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    }
    return v;
}

// G = lanes per cached position (each lane holds 4 of the hd values);
// NR = max query heads per KV head handled by one workgroup; NW = waves.
//
// Each wave walks its positions U*P at a time: the K and V rows of a step are
// requested together (one memory round trip per step), the scores are reduced
// over the G lanes of a position, and an online softmax keeps (max, sum, out)
// per lane group.  The NW*P lane groups of the workgroup are merged through
// LDS into one partial per (query head, split); with a single split that is
// the attention row itself.
// PRO: a callable run by every thread after the position range is known and
// before the queries are read; it returns the LDS queries [nrep][hd] or null
// (a.q).  PRE: the first step's K / V rows are requested before it, unless the
// new position (written by the prologue of the split holding it) is among
// them.
template <int G, int NR, int NW, bool PRE, class PRO>
__device__ __forceinline__ void attn_body(const AttnArgs &a, const int blk, PRO &&pro) {
    constexpr int NT = 64 * NW;
    constexpr int P = 64 / G;  // positions per load instruction
    // load instructions per step: 12 keeps the most K/V rows in flight; with
    // four or more query heads per KV head the score and output registers of
    // 12 steps leave 2 waves per SIMD (190 VGPRs), 6 leave 4 (124 VGPRs)
    constexpr int U = NR >= 4 ? 6 : 12;
    constexpr int PI = P * U;  // positions per wave step
    constexpr int SLOTS = NW * P;
    extern __shared__ float sm[];
    float *s_o = sm;                    // [SLOTS][NR][hd]
    __shared__ float s_m[SLOTS][NR], s_l[SLOTS][NR];
    // block b: group (b % 8) + 8 * ((b / 8) / n_splits), split (b / 8) % n_splits
    const int bi = blk >> 3;
    const int g = (blk & 7) + 8 * (bi / a.n_splits), split = bi % a.n_splits;
    if (g >= a.n_kv) return;  // padding of the last row of 8 groups
    const int nrep = a.n_heads / a.n_kv, hd = a.head_dim, kv_dim = a.n_kv * hd;
    const int L = a.fixed_len >= 0 ? a.fixed_len : a.state->cache_len + 1;
    const int chunk = (L + a.n_splits - 1) / a.n_splits;
    const int t0 = min(L, split * chunk), t1 = min(L, t0 + chunk);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / G, gl = lane % G;
    const bool dact = gl * 4 < hd;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.k_cache, (size_t)t1 * kv_dim * 4);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.v_cache, (size_t)t1 * kv_dim * 4);
    const unsigned col = (unsigned)(g * hd + gl * 4) * 4;

    auto load = [&](float4(&kv)[U], float4(&vv)[U], int tb) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = tb + u * P + sub;
            const unsigned off = (t < t1 && dact) ? (unsigned)t * kv_dim * 4 + col : 0x80000000u;
            kv[u] = bload16f(kr, off);
            vv[u] = bload16f(vr, off);
        }
    };
    const int tb0 = t0 + wave * PI;
    float4 kv0[U], vv0[U];
    bool pre = false;
    if constexpr (PRE) {
        const bool holder = t1 == L && t0 < t1;
        pre = tb0 < t1 && (!holder || t1 - 1 >= t0 + NW * PI);
        if (pre) load(kv0, vv0, tb0);
    }
    const float *q_lds = pro();

    float4 qf[NR];
    float m[NR], l[NR];
    float4 o[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        qf[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nrep && dact)
            qf[r] = q_lds ? *(const float4 *)(q_lds + r * hd + gl * 4)
                          : *(const float4 *)(a.q + (size_t)(g * nrep + r) * hd + gl * 4);
        m[r] = -INFINITY;
        l[r] = 0.f;
        o[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    auto step = [&](const float4(&kv)[U], const float4(&vv)[U], int tb) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if (r >= nrep) break;
            float sc[U];
            float mx = m[r];
            bool any = false;
#pragma unroll
            for (int u = 0; u < U; u++) {
                float d = qf[r].x * kv[u].x + qf[r].y * kv[u].y + qf[r].z * kv[u].z + qf[r].w * kv[u].w;
                d = group_sum<G, (NR >= 4)>(d);
                const bool in = tb + u * P + sub < t1;
                any |= in;
                sc[u] = in ? d : -INFINITY;
                mx = fmaxf(mx, sc[u]);
            }
            // no position of this lane group in the step; a step of NaN scores
            // only is not skipped: with mx = -inf its sum becomes NaN (the
            // reference's softmax of a NaN score is NaN, cpu.rs:336-366)
            if (!any) continue;
            // the running softmax's exponentials by v_exp_f32 (2^(x log2 e)):
            // relative error about |x| 2^-24 plus an ulp against expf, 1e-6 where
            // a weight e^x (x <= 0 against the running maximum) is above 2^-20
            // and so can move the sums; expf took 3% of the attention time
            const float f = __expf(m[r] - mx);
            l[r] *= f;
            o[r].x *= f;
            o[r].y *= f;
            o[r].z *= f;
            o[r].w *= f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float p = __expf(sc[u] - mx);
                l[r] += p;
                o[r].x += p * vv[u].x;
                o[r].y += p * vv[u].y;
                o[r].z += p * vv[u].z;
                o[r].w += p * vv[u].w;
            }
            m[r] = mx;
        }
    };
    int tbs = tb0;
    if (pre) {
        step(kv0, vv0, tb0);
        tbs += NW * PI;
    }
    for (int tb = tbs; tb < t1; tb += NW * PI) {
        float4 kv[U], vv[U];
        load(kv, vv, tb);
        step(kv, vv, tb);
    }
    const int slot = wave * P + sub;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        if (r >= nrep) break;
        if (gl == 0) {
            s_m[slot][r] = m[r];
            s_l[slot][r] = l[r];
        }
        if (dact) *(float4 *)(s_o + ((size_t)slot * NR + r) * hd + gl * 4) = o[r];
    }
    __syncthreads();
    const bool single = a.n_splits == 1;
    for (int idx = tid; idx < nrep * hd; idx += NT) {
        const int r = idx / hd, d = idx % hd;
        // a lane group that saw only NaN scores has max -inf and a NaN sum
        float M = -INFINITY;
        bool poison = false;
#pragma unroll
        for (int q = 0; q < SLOTS; q++) {
            M = fmaxf(M, s_m[q][r]);
            poison |= isnan(s_l[q][r]);
        }
        float lsum = 0.f, osum = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int q = 0; q < SLOTS; q++) {
                if (s_m[q][r] == -INFINITY) continue;
                const float f = expf(s_m[q][r] - M);
                lsum += s_l[q][r] * f;
                osum += s_o[((size_t)q * NR + r) * hd + d] * f;
            }
        }
        if (poison) lsum = osum = __builtin_nanf("");
        if (single) {  // the whole sequence: softmax-normalised row
            a.xa[(size_t)(g * nrep + r) * hd + d] = M == -INFINITY && !poison ? 0.f : osum / lsum;
            continue;
        }
        const size_t ph = (size_t)(g * nrep + r) * a.n_splits + split;
        a.part_o[ph * hd + d] = osum;
        if (d == 0) {
            a.part_ml[ph * 2 + 0] = M;
            a.part_ml[ph * 2 + 1] = lsum;
        }
    }
    if (single) return;
    // count this split in once its partial stores are complete
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(a.merge_ctr + (size_t)g * kCtrStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(a.n_splits - 1);
    __syncthreads();
    if (!s_last) return;
    // last split of group g: x[h*hd + d] = sum_s O_s[d] e^(M_s - M) / sum_s L_s e^(M_s - M),
    // every load issued before the first use (one memory round trip)
    const int ns = a.n_splits;
    for (int idx = tid; idx < nrep * hd; idx += NT) {
        const int r = idx / hd, d = idx % hd, h = g * nrep + r;
        const float *ml = a.part_ml + (size_t)h * ns * 2;
        const float *po = a.part_o + (size_t)h * ns * hd + d;
        float mq[MAX_SPLITS], lq[MAX_SPLITS], oq[MAX_SPLITS];
#pragma unroll
        for (int q = 0; q < MAX_SPLITS; q++) {
            mq[q] = q < ns ? cload(ml + 2 * q) : -INFINITY;
            lq[q] = q < ns ? cload(ml + 2 * q + 1) : 0.f;
            oq[q] = q < ns ? cload(po + (size_t)q * hd) : 0.f;
        }
        float M = -INFINITY;
        bool poison = false;
#pragma unroll
        for (int q = 0; q < MAX_SPLITS; q++) {
            M = fmaxf(M, mq[q]);
            poison |= isnan(lq[q]);
        }
        float Ls = 0.f, v = 0.f;
#pragma unroll
        for (int q = 0; q < MAX_SPLITS; q++) {
            if (q < ns && mq[q] != -INFINITY) {
                const float e = expf(mq[q] - M);
                Ls += lq[q] * e;
                v += oq[q] * e;
            }
        }
        a.xa[(size_t)h * hd + d] = poison ? __builtin_nanf("") : M == -INFINITY ? 0.f : v / Ls;
    }
    if (tid == 0) a.merge_ctr[(size_t)g * kCtrStride] = 0;  // ready for the next launch on the stream
}

template <int G, int NR, int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_decode(AttnArgs a) {
    if (a.ts) wg_stamp_begin(a.ts);
    attn_body<G, NR, NW, false>(a, blockIdx.x, [] { return (const float *)nullptr; });
    if (a.ts) wg_stamp_end(a.ts);
}

// The qkv epilogue of the batched decode step for sequence y and the
// workgroup's KV group (QkvPro): its query heads into s_q [nrep][hd], and, in
// the split holding the new position, that position's K / V row into the
// cache.  One element per thread and pass; a RoPE pair is two neighbouring
// lanes.  The sums, scaling and rotation are the fused STORE epilogue's.
constexpr int QP_MAX_SPLIT = 16;  // qkv partials per column (launch_attn_decode_seqs checks)

template <int NW>
__device__ __forceinline__ void qkv_prologue(const AttnArgs &a, const AttnSeqs &b, const QkvPro &qp, int y, int blk,
                                             float *s_q) {
    constexpr int NT = 64 * NW;
    __shared__ double s_rstd;
    const int bi = blk >> 3;
    const int g = (blk & 7) + 8 * (bi / a.n_splits), split = bi % a.n_splits;
    if (g >= a.n_kv) return;  // padding of the last row of 8 groups (attn_body returns too)
    const int tid = threadIdx.x, nrep = a.n_heads / a.n_kv, hd = a.head_dim;
    const int qd = a.n_heads * hd, kvd = a.n_kv * hd;
    const int pos = b.pos[y], L = pos + 1, chunk = (L + a.n_splits - 1) / a.n_splits;
    const int t0 = min(L, split * chunk), t1 = min(L, t0 + chunk);
    const bool holder = t0 <= pos && pos < t1;
    const float *pr = qp.part + (size_t)y * qp.n_pad;
    const size_t st = (size_t)16 * qp.n_pad;  // one split's 16 rows
    const float2 *rope = qp.rope[y] + (size_t)pos * (hd >> 1);
    // items: the group's query values (nq), then in the holder k and v (2 hd);
    // item i's column and RoPE dimension
    const int nq = nrep * hd, ni = nq + (holder ? 2 * hd : 0);
    auto col = [&](int i) {
        return i < nq ? g * nrep * hd + i : i < nq + hd ? qd + g * hd + (i - nq) : qd + kvd + g * hd + (i - nq - hd);
    };
    // every load of a pass is issued before the first use (one memory round trip)
    float pv[QP_MAX_SPLIT];
    float2 cs;
    auto load = [&](int i) {
        const int ii = min(i, ni - 1), c = col(ii);
#pragma unroll
        for (int sp = 0; sp < QP_MAX_SPLIT; sp++) pv[sp] = sp < qp.n_split ? pr[sp * st + c] : 0.f;
        cs = rope[((ii < nq ? ii : ii - nq) % hd) >> 1];
    };
    // finish item i: the split sum in split order, the scales, the rotation of
    // the pair (c, c + 1) held by lanes 2j, 2j + 1 (llama.rs:384-396)
    auto finish = [&](int i, double rstd) {
        float sum = 0.f;
#pragma unroll
        for (int sp = 0; sp < QP_MAX_SPLIT; sp++)
            if (sp < qp.n_split) sum += pv[sp];
        const bool in = i < ni;
        const float v = in ? (float)((double)(sum * qp.scale) * rstd) : 0.f;
        const float w = __shfl_xor(v, 1);
        const float r = (i & 1) ? __fadd_rn(__fmul_rn(w, cs.y), __fmul_rn(v, cs.x))
                                : __fsub_rn(__fmul_rn(v, cs.x), __fmul_rn(w, cs.y));
        if (!in) return;
        if (i < nq) {
            s_q[i] = __fmul_rn(r, qp.q_scale);
        } else {
            const size_t at = (size_t)b.layer * b.ls[y] + (size_t)pos * kvd + (size_t)g * hd;
            if (i < nq + hd) b.k[y][at + (i - nq)] = r;
            else b.v[y][at + (i - nq - hd)] = v;
        }
    };
    load(tid);
    if (tid < 64) {  // RMSNorm scale of row y (rmsnorm.rs, cpu.rs:574-599), f64
        const double q = tid < qp.n_ss_in ? qp.ss_in[(size_t)y * qp.n_ss_in + tid] : 0.0;
        const double v = wave_sum_d(q);
        if (tid == 0) s_rstd = 1.0 / sqrt(v / (double)qp.k + (double)qp.eps);
    }
    __syncthreads();
    const double rstd = s_rstd;
    finish(tid, rstd);
    for (int i = tid + NT; i - tid < ni; i += NT) {  // more items than threads (uniform trip count)
        load(i);
        finish(i, rstd);
    }
    if (holder) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the new row is in memory before the workgroup reads it
    __syncthreads();
}

// Several sequences, one per blockIdx.y, each with its own cache, length and
// partial buffers (the rows of a batched decode step).  The linear block id is
// blockIdx.x + gridDim.x * blockIdx.y with gridDim.x a multiple of 8, so the
// XCD of a workgroup is still blockIdx.x % 8 and the exchange stays in one L2.
// QP: the queries and the new K / V rows come from the qkv partials (QkvPro).
template <int G, int NR, int NW, bool QP>
__global__ __launch_bounds__(64 * NW) void k_attn_decode_seqs(AttnArgs a, AttnSeqs b, QkvPro qp) {
    const int y = blockIdx.y;
    const int qd = a.n_heads * a.head_dim;
    AttnArgs s = a;
    s.q = a.q + (size_t)y * qd;
    s.k_cache = b.k[y] + (size_t)b.layer * b.ls[y];
    s.v_cache = b.v[y] + (size_t)b.layer * b.ls[y];
    s.part_o = a.part_o + (size_t)y * a.n_heads * a.n_splits * a.head_dim;
    s.part_ml = a.part_ml + (size_t)y * a.n_heads * a.n_splits * 2;
    s.merge_ctr = a.merge_ctr + (size_t)y * a.n_kv * kCtrStride;
    s.xa = a.xa + (size_t)y * qd;
    s.fixed_len = b.pos[y] + 1;
    if constexpr (QP) {
        __shared__ float s_q[NR * 256];  // head_dim <= 256
        attn_body<G, NR, NW, true>(s, blockIdx.x, [&] {
            qkv_prologue<NW>(a, b, qp, y, blockIdx.x, s_q);
            return (const float *)s_q;
        });
    } else {
        attn_body<G, NR, NW, false>(s, blockIdx.x, [] { return (const float *)nullptr; });
    }
}

template <int G, int NR, int NW>
void launch_k(const AttnArgs &a, const AttnSeqs *b, const QkvPro *qp, dim3 grid, size_t lds, hipStream_t s) {
    if (b) {
        grid.y = b->n;
        if (qp)
            hipLaunchKernelGGL((k_attn_decode_seqs<G, NR, NW, true>), grid, dim3(64 * NW), lds, s, a, *b, *qp);
        else
            hipLaunchKernelGGL((k_attn_decode_seqs<G, NR, NW, false>), grid, dim3(64 * NW), lds, s, a, *b, QkvPro{});
    } else {
        hipLaunchKernelGGL((k_attn_decode<G, NR, NW>), grid, dim3(64 * NW), lds, s, a);
    }
}

template <int G, int NW>
int launch_gw(const AttnArgs &a, const AttnSeqs *b, const QkvPro *qp, int nrep, hipStream_t s) {
    const int P = 64 / G;
    auto lds = [&](int nr) { return (size_t)NW * P * nr * a.head_dim * 4; };
    dim3 grid(8 * ((a.n_kv + 7) / 8) * a.n_splits);
    if (nrep <= 1) {
        launch_k<G, 1, NW>(a, b, qp, grid, lds(1), s);
    } else if (nrep <= 2) {
        launch_k<G, 2, NW>(a, b, qp, grid, lds(2), s);
    } else if (nrep <= 4) {
        launch_k<G, 4, NW>(a, b, qp, grid, lds(4), s);
    } else if (nrep <= 8) {
        launch_k<G, 8, NW>(a, b, qp, grid, lds(8), s);
    } else {
        return set_error(SCRY_ERR_UNSUPPORTED, "attention: n_heads/n_kv = %d > 8", nrep);
    }
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

// 16 waves when one workgroup covers a whole KV group's sequence (more loads
// in flight per CU). Split sequences: 4 waves for one or two query heads per
// KV head; 8 for more, which carry 6 loads per step instead of 12. Measured
// at the Llama-3-8B shape, 4 sequences of ~2100 rows: batched decode
// 212.0 -> 203.5 ms, one sequence at a time 571.7 -> 531.5 ms; 8 waves at one
// head per KV head (Llama-2-7B) were 0.2% slower.
template <int G>
int launch_g(const AttnArgs &a, const AttnSeqs *b, const QkvPro *qp, int nrep, hipStream_t s) {
    if (a.n_splits == 1) return launch_gw<G, 16>(a, b, qp, nrep, s);
    return nrep >= 3 ? launch_gw<G, 8>(a, b, qp, nrep, s) : launch_gw<G, 4>(a, b, qp, nrep, s);
}

}  // namespace

int attn_pick_splits(int n_kv, int max_seq, int *n_splits, int *max_chunk) {
    // ~512 workgroups per launch (two per CU: measured at the 7B shape, 32 KV
    // groups, against 256: 9.83 against 10.08 us at 768 cached rows, 13.95
    // against 14.3 us at 1536, decode +0.6%; against 384: 14.0 against 15.3 us
    // at 1536, decode 568.4 against 564.5 tok/s), at most 16 splits (the last
    // split merges n_splits partials per query head), >= 16 rows per split
    int ns = (512 + n_kv - 1) / n_kv;
    if (ns > 16) ns = 16;
    const int cap = (max_seq + 15) / 16;
    if (ns > cap) ns = cap;
    if (ns < 1) ns = 1;
    *n_splits = ns;
    *max_chunk = (max_seq + ns - 1) / ns;
    return SCRY_OK;
}

namespace {
int launch_attn(const AttnArgs &a, const AttnSeqs *b, const QkvPro *qp, hipStream_t s) {
    if (!a.xa || (a.n_splits > 1 && (!a.merge_ctr || !a.part_o || !a.part_ml)))
        return set_error(SCRY_ERR_INVALID, "attention: missing output / partial / merge buffers");
    if (a.n_splits < 1 || a.n_splits > MAX_SPLITS)
        return set_error(SCRY_ERR_INVALID, "attention: %d splits (1..%d)", a.n_splits, MAX_SPLITS);
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0)
        return set_error(SCRY_ERR_INVALID, "attention: n_heads %% n_kv != 0");
    if (a.head_dim % 4 != 0 || a.head_dim > 256)
        return set_error(SCRY_ERR_UNSUPPORTED, "attention: head_dim %d (need %%4 == 0, <= 256)",
                         a.head_dim);
    const int nrep = a.n_heads / a.n_kv;
    const int lanes = a.head_dim / 4;
    if (lanes <= 1) return launch_g<1>(a, b, qp, nrep, s);
    if (lanes <= 2) return launch_g<2>(a, b, qp, nrep, s);
    if (lanes <= 4) return launch_g<4>(a, b, qp, nrep, s);
    if (lanes <= 8) return launch_g<8>(a, b, qp, nrep, s);
    if (lanes <= 16) return launch_g<16>(a, b, qp, nrep, s);
    if (lanes <= 32) return launch_g<32>(a, b, qp, nrep, s);
    return launch_g<64>(a, b, qp, nrep, s);
}
}  // namespace

int launch_attn_decode(const AttnArgs &a, hipStream_t s) { return launch_attn(a, nullptr, nullptr, s); }

int launch_attn_decode_seqs(const AttnArgs &a, const AttnSeqs &b, hipStream_t s, const QkvPro *pro) {
    if (b.n < 1 || b.n > PF_MAX_SEQS || !b.pos || (!pro && !a.q))
        return set_error(SCRY_ERR_INVALID, "attention: %d sequences (1..%d) with positions and queries", b.n,
                         PF_MAX_SEQS);
    if (pro) {
        bool ok = pro->part && pro->n_split >= 1 && pro->n_split <= QP_MAX_SPLIT && pro->ss_in && pro->n_ss_in >= 1 &&
                  pro->n_ss_in <= 64 &&
                  pro->k >= 1 && a.head_dim % 2 == 0 && a.head_dim <= 256 &&
                  pro->n_pad >= (a.n_heads + 2 * a.n_kv) * a.head_dim;
        for (int i = 0; ok && i < b.n; i++) ok = pro->rope[i] != nullptr;
        if (!ok) return set_error(SCRY_ERR_INVALID, "attention: qkv partials, norm partials and RoPE tables");
    }
    return launch_attn(a, &b, pro, s);
}

}  // namespace scry
