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
template <int G, int NR, int NW>
__device__ __forceinline__ void attn_body(const AttnArgs &a, const int blk) {
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

    float4 qf[NR];
    float m[NR], l[NR];
    float4 o[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        qf[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nrep && dact) qf[r] = *(const float4 *)(a.q + (size_t)(g * nrep + r) * hd + gl * 4);
        m[r] = -INFINITY;
        l[r] = 0.f;
        o[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int tb = t0 + wave * PI; tb < t1; tb += NW * PI) {
        float4 kv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = tb + u * P + sub;
            const unsigned off = (t < t1 && dact) ? (unsigned)t * kv_dim * 4 + col : 0x80000000u;
            kv[u] = bload16f(kr, off);
            vv[u] = bload16f(vr, off);
        }
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
            const float f = expf(m[r] - mx);
            l[r] *= f;
            o[r].x *= f;
            o[r].y *= f;
            o[r].z *= f;
            o[r].w *= f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float p = expf(sc[u] - mx);
                l[r] += p;
                o[r].x += p * vv[u].x;
                o[r].y += p * vv[u].y;
                o[r].z += p * vv[u].z;
                o[r].w += p * vv[u].w;
            }
            m[r] = mx;
        }
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
    attn_body<G, NR, NW>(a, blockIdx.x);
    if (a.ts) wg_stamp_end(a.ts);
}

// Several sequences, one per blockIdx.y, each with its own cache, length and
// partial buffers (the rows of a batched decode step).  The linear block id is
// blockIdx.x + gridDim.x * blockIdx.y with gridDim.x a multiple of 8, so the
// XCD of a workgroup is still blockIdx.x % 8 and the exchange stays in one L2.
template <int G, int NR, int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_decode_seqs(AttnArgs a, AttnSeqs b) {
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
    attn_body<G, NR, NW>(s, blockIdx.x);
}

template <int G, int NR, int NW>
void launch_k(const AttnArgs &a, const AttnSeqs *b, dim3 grid, size_t lds, hipStream_t s) {
    if (b) {
        grid.y = b->n;
        hipLaunchKernelGGL((k_attn_decode_seqs<G, NR, NW>), grid, dim3(64 * NW), lds, s, a, *b);
    } else {
        hipLaunchKernelGGL((k_attn_decode<G, NR, NW>), grid, dim3(64 * NW), lds, s, a);
    }
}

template <int G, int NW>
int launch_gw(const AttnArgs &a, const AttnSeqs *b, int nrep, hipStream_t s) {
    const int P = 64 / G;
    auto lds = [&](int nr) { return (size_t)NW * P * nr * a.head_dim * 4; };
    dim3 grid(8 * ((a.n_kv + 7) / 8) * a.n_splits);
    if (nrep <= 1) {
        launch_k<G, 1, NW>(a, b, grid, lds(1), s);
    } else if (nrep <= 2) {
        launch_k<G, 2, NW>(a, b, grid, lds(2), s);
    } else if (nrep <= 4) {
        launch_k<G, 4, NW>(a, b, grid, lds(4), s);
    } else if (nrep <= 8) {
        launch_k<G, 8, NW>(a, b, grid, lds(8), s);
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
int launch_g(const AttnArgs &a, const AttnSeqs *b, int nrep, hipStream_t s) {
    if (a.n_splits == 1) return launch_gw<G, 16>(a, b, nrep, s);
    return nrep >= 3 ? launch_gw<G, 8>(a, b, nrep, s) : launch_gw<G, 4>(a, b, nrep, s);
}

}  // namespace

int attn_pick_splits(int n_kv, int max_seq, int *n_splits, int *max_chunk) {
    // ~512 workgroups per launch (two per CU: measured at the 7B shape, 32 KV
    // groups, against 256: 9.83 against 10.08 us at 768 cached rows, 13.95
    // against 14.3 us at 1536, decode +0.6%), at most 16 splits (the last
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
int launch_attn(const AttnArgs &a, const AttnSeqs *b, hipStream_t s) {
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
    if (lanes <= 1) return launch_g<1>(a, b, nrep, s);
    if (lanes <= 2) return launch_g<2>(a, b, nrep, s);
    if (lanes <= 4) return launch_g<4>(a, b, nrep, s);
    if (lanes <= 8) return launch_g<8>(a, b, nrep, s);
    if (lanes <= 16) return launch_g<16>(a, b, nrep, s);
    if (lanes <= 32) return launch_g<32>(a, b, nrep, s);
    return launch_g<64>(a, b, nrep, s);
}
}  // namespace

int launch_attn_decode(const AttnArgs &a, hipStream_t s) { return launch_attn(a, nullptr, s); }

int launch_attn_decode_seqs(const AttnArgs &a, const AttnSeqs &b, hipStream_t s) {
    if (b.n < 1 || b.n > PF_MAX_SEQS || !b.pos || !a.q)
        return set_error(SCRY_ERR_INVALID, "attention: %d sequences (1..%d) with positions and queries", b.n,
                         PF_MAX_SEQS);
    return launch_attn(a, &b, s);
}

}  // namespace scry
