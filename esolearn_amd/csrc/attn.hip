// Decode attention over the device KV cache (one query token, GQA), replacing
// the reference's per-token sequence (llama.rs:411-455):
//   gather_reshape_repeat_kv (cpu.rs:707-730) x2, strided-batched Q.K^T
//   (gemv_trans_b, cpu.rs:825-842), softmax (cpu.rs:336-366), strided-batched
//   P.V (gemv_into, cpu.rs:846-871).
// Q arrives pre-scaled by 1/sqrt(hd) and RoPE'd (fused into the QKV GEMV).
//
// The cache is read in place ([max_seq, n_kv*hd] rows, no repeat_kv copy):
// workgroup (g, s) handles KV head g and position split s for all n_rep query
// heads of the group, so each K/V row is read once per group.  Splits write
// (max, sum, unnormalised output); the last workgroup to finish for a group
// (atomic counter, reset by that workgroup) merges them with the usual
// log-sum-exp rescaling.  The split count is fixed per cache, so the launch
// shape does not depend on the current length and the kernel can live in a
// replayed graph; the length comes from the device state.
#include "internal.h"

namespace scry {
namespace {

constexpr int TPB = 256;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, size_t bytes) {
    const int n = bytes > 0x7fffffffu ? 0x7fffffff : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}
__device__ __forceinline__ float4 bload16f(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// G = lanes per cached position (each lane holds 4 of the hd values);
// NR = max query heads per KV head handled by one workgroup.
template <int G, int NR>
__global__ __launch_bounds__(TPB) void k_attn_decode(AttnArgs a) {
    constexpr int P = 64 / G;  // positions per wave step
    extern __shared__ float sm[];
    const int g = blockIdx.x, split = blockIdx.y;
    const int nrep = a.n_heads / a.n_kv, hd = a.head_dim, kv_dim = a.n_kv * hd;
    const int L = a.fixed_len >= 0 ? a.fixed_len : a.state->cache_len + 1;
    const int chunk = (L + a.n_splits - 1) / a.n_splits;
    const int t0 = min(L, split * chunk), t1 = min(L, t0 + chunk);
    const int n = t1 - t0;
    const int mc = a.max_chunk;
    float *sc = sm;                  // [NR][mc] scores, then probabilities
    float *red = sm + NR * mc;       // [4*P][NR][hd] partial outputs
    __shared__ float s_m[NR], s_l[NR];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / G, gl = lane % G;
    const bool dact = gl * 4 < hd;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.k_cache, (size_t)(t1) * kv_dim * 4);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.v_cache, (size_t)(t1) * kv_dim * 4);
    const unsigned col = (unsigned)(g * hd + gl * 4) * 4;

    // ---- scores s[r][t] = q_r . K[t]
    float4 qf[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        qf[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nrep && dact) qf[r] = *(const float4 *)(a.q + (size_t)(g * nrep + r) * hd + gl * 4);
    }
    for (int tb = t0 + wave * P; tb < t1; tb += 4 * P) {
        const int t = tb + sub;
        const bool ok = t < t1 && dact;
        const float4 kv = bload16f(kr, ok ? (unsigned)t * kv_dim * 4 + col : 0x80000000u);
#pragma unroll
        for (int r = 0; r < NR; r++) {
            float s = qf[r].x * kv.x + qf[r].y * kv.y + qf[r].z * kv.z + qf[r].w * kv.w;
            s = group_sum<G>(s);
            if (gl == 0 && t < t1 && r < nrep) sc[r * mc + (t - t0)] = s;
        }
    }
    __syncthreads();

    // ---- per-head max and sum of exp over this split
    for (int r = wave; r < nrep; r += 4) {
        float mx = -INFINITY;
        for (int i = lane; i < n; i += 64) mx = fmaxf(mx, sc[r * mc + i]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        float l = 0.f;
        for (int i = lane; i < n; i += 64) {
            const float p = expf(sc[r * mc + i] - mx);
            sc[r * mc + i] = p;
            l += p;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            s_m[r] = mx;
            s_l[r] = l;
        }
    }
    __syncthreads();

    // ---- o[r] = sum_t p[r][t] V[t]
    float4 o[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) o[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int tb = t0 + wave * P; tb < t1; tb += 4 * P) {
        const int t = tb + sub;
        const bool ok = t < t1 && dact;
        const float4 v = bload16f(vr, ok ? (unsigned)t * kv_dim * 4 + col : 0x80000000u);
        if (t < t1) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                if (r < nrep) {
                    const float p = sc[r * mc + (t - t0)];
                    o[r].x += p * v.x;
                    o[r].y += p * v.y;
                    o[r].z += p * v.z;
                    o[r].w += p * v.w;
                }
            }
        }
    }
    if (dact) {
        const int slot = wave * P + sub;
#pragma unroll
        for (int r = 0; r < NR; r++)
            if (r < nrep) *(float4 *)(red + ((size_t)slot * NR + r) * hd + gl * 4) = o[r];
    }
    __syncthreads();
    for (int idx = tid; idx < nrep * hd; idx += TPB) {
        const int r = idx / hd, d = idx % hd;
        float s = 0.f;
        for (int slot = 0; slot < 4 * P; slot++) s += red[((size_t)slot * NR + r) * hd + d];
        const size_t ph = (size_t)(g * nrep + r) * a.n_splits + split;
        a.part_o[ph * hd + d] = s;
        if (d == 0) {
            a.part_ml[ph * 2 + 0] = s_m[r];
            a.part_ml[ph * 2 + 1] = s_l[r];
        }
    }

    // ---- last workgroup of group g merges the splits
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const unsigned prev = atomicAdd(a.counter + g, 1u);
        s_last = (prev == (unsigned)a.n_splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int idx = tid; idx < nrep * hd; idx += TPB) {
        const int r = idx / hd, d = idx % hd;
        const size_t h0 = (size_t)(g * nrep + r) * a.n_splits;
        float M = -INFINITY;
        for (int s = 0; s < a.n_splits; s++) M = fmaxf(M, a.part_ml[(h0 + s) * 2]);
        float lsum = 0.f, osum = 0.f;
        for (int s = 0; s < a.n_splits; s++) {
            const float ms = a.part_ml[(h0 + s) * 2];
            if (ms == -INFINITY) continue;  // empty split
            const float f = expf(ms - M);
            lsum += a.part_ml[(h0 + s) * 2 + 1] * f;
            osum += a.part_o[(h0 + s) * hd + d] * f;
        }
        a.out[(size_t)(g * nrep + r) * hd + d] = osum / lsum;
    }
    if (tid == 0) a.counter[g] = 0u;
}

template <int G>
int launch_g(const AttnArgs &a, int nrep, hipStream_t s) {
    const int P = 64 / G;
    auto lds = [&](int nr) { return (size_t)nr * a.max_chunk * 4 + (size_t)4 * P * nr * a.head_dim * 4; };
    dim3 grid(a.n_kv, a.n_splits);
    if (nrep <= 1) {
        hipLaunchKernelGGL((k_attn_decode<G, 1>), grid, dim3(TPB), lds(1), s, a);
    } else if (nrep <= 2) {
        hipLaunchKernelGGL((k_attn_decode<G, 2>), grid, dim3(TPB), lds(2), s, a);
    } else if (nrep <= 4) {
        hipLaunchKernelGGL((k_attn_decode<G, 4>), grid, dim3(TPB), lds(4), s, a);
    } else if (nrep <= 8) {
        hipLaunchKernelGGL((k_attn_decode<G, 8>), grid, dim3(TPB), lds(8), s, a);
    } else {
        return set_error(SCRY_ERR_UNSUPPORTED, "attention: n_heads/n_kv = %d > 8", nrep);
    }
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace

int attn_pick_splits(int n_kv, int max_seq, int *n_splits, int *max_chunk) {
    // ~512 workgroups per launch, at least 16 positions per split
    int ns = (512 + n_kv - 1) / n_kv;
    const int cap = (max_seq + 15) / 16;
    if (ns > cap) ns = cap;
    if (ns < 1) ns = 1;
    *n_splits = ns;
    *max_chunk = ((max_seq + ns - 1) / ns + 3) & ~3;  // keeps the LDS reduction area 16-byte aligned
    return SCRY_OK;
}

int launch_attn_decode(const AttnArgs &a, hipStream_t s) {
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0)
        return set_error(SCRY_ERR_INVALID, "attention: n_heads %% n_kv != 0");
    if (a.head_dim % 4 != 0 || a.head_dim > 256)
        return set_error(SCRY_ERR_UNSUPPORTED, "attention: head_dim %d (need %%4 == 0, <= 256)",
                         a.head_dim);
    const int nrep = a.n_heads / a.n_kv;
    const int lanes = a.head_dim / 4;
    if (lanes <= 1) return launch_g<1>(a, nrep, s);
    if (lanes <= 2) return launch_g<2>(a, nrep, s);
    if (lanes <= 4) return launch_g<4>(a, nrep, s);
    if (lanes <= 8) return launch_g<8>(a, nrep, s);
    if (lanes <= 16) return launch_g<16>(a, nrep, s);
    if (lanes <= 32) return launch_g<32>(a, nrep, s);
    return launch_g<64>(a, nrep, s);
}

}  // namespace scry
