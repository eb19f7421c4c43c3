// Glue of the batched decode step: n sequences, one token each, through the
// same layer as the single-sequence step (llama.rs:744-763, 556-569), with
// each projection as one fused skinny matmul over the n rows (skinny.hip:
// RMSNorm, split reduction and epilogue in the launch) and the attention of
// every sequence against its own cache in one launch (attn.hip).
// The reference runs each sequence's decode separately; the per-sequence
// arithmetic here is that step's:
//   embedding row of the current token            (cpu.rs:485-498)
//   RoPE of q and k from the cache's cos/sin table, q times 1/sqrt(hd) in a
//   separate rounding, K / V rows appended at the position (llama.rs:371-410,
//   cpu.rs:655-658, kv_cache.rs:99-118)
//   next token = ordered argmax of the logits     (generate.rs:167-173)
// Positions and tokens live in device memory, so a captured step replays.
#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

// x[y][i] = embed[tokens_y[pos_y]][i], and per 128 columns the f64 sum of
// squares (the first RMSNorm's partials, ss [n][n_ss])
__global__ __launch_bounds__(128) void k_bd_embed(const float *__restrict__ embed, int h, DecodeSeqs d,
                                                  float *__restrict__ x, double *__restrict__ ss, int n_ss) {
    __shared__ double sh[2];
    const int y = blockIdx.y, i = blockIdx.x * 128 + threadIdx.x;
    const int64_t tok = d.tokens[y][d.pos[y]];
    float v = 0.f;
    if (i < h) {
        v = embed[(size_t)tok * h + i];
        x[(size_t)y * h + i] = v;
    }
    const double q = wave_sum_d((double)v * (double)v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = q;
    __syncthreads();
    if (threadIdx.x == 0) ss[(size_t)y * n_ss + blockIdx.x] = sh[0] + sh[1];
}

// One workgroup per sequence: the ordered argmax of its logits row (from the
// LM head's per-tile partials, combined in any order) becomes the token at
// pos + 1, and the position advances.
__global__ __launch_bounds__(TPB) void k_bd_argmax(const float *__restrict__ logits, int V,
                                                   const float *__restrict__ pv, const int *__restrict__ pi,
                                                   const int *__restrict__ pn, int np, DecodeSeqs d) {
    __shared__ ArgAcc sh[TPB];
    const int y = blockIdx.x;
    const float *x = logits + (size_t)y * V;
    const size_t b = (size_t)y * np;
    constexpr int FP = 8;
    ArgAcc acc{0.f, -1, -1};
    for (int t0 = threadIdx.x; t0 < np; t0 += FP * TPB) {
        ArgAcc q[FP];
#pragma unroll
        for (int j = 0; j < FP; j++) {
            const int t = min(t0 + j * TPB, np - 1);  // clamped: unconditional loads
            q[j] = ArgAcc{pv[b + t], pi[b + t], pn[b + t]};
        }
#pragma unroll
        for (int j = 0; j < FP; j++)
            if (t0 + j * TPB < np) acc = arg_combine(acc, q[j]);
    }
    const ArgAcc r = block_argmax(acc, sh);
    const int tok = argmax_finish(r, x, V, sh);
    if (threadIdx.x == 0) {
        const int p = d.pos[y];
        d.tokens[y][p + 1] = tok;
        d.pos[y] = p + 1;
    }
}

}  // namespace

int launch_bd_embed(const float *embed, int h, const DecodeSeqs &d, float *x, double *ss, hipStream_t s) {
    if (d.n < 1 || d.n > PF_MAX_SEQS) return set_error(SCRY_ERR_INVALID, "batched decode: %d sequences", d.n);
    const int n_ss = (h + 127) / 128;
    hipLaunchKernelGGL(k_bd_embed, dim3(n_ss, d.n), dim3(128), 0, s, embed, h, d, x, ss, n_ss);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

int launch_bd_argmax(const float *logits, int V, const float *pv, const int *pi, const int *pn, int np,
                     const DecodeSeqs &d, hipStream_t s) {
    if (d.n < 1 || d.n > PF_MAX_SEQS || V < 1 || np < 1)
        return set_error(SCRY_ERR_INVALID, "batched decode: %d sequences, vocab %d", d.n, V);
    hipLaunchKernelGGL(k_bd_argmax, dim3(d.n), dim3(TPB), 0, s, logits, V, pv, pi, pn, np, d);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
