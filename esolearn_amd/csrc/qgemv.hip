// W8A32 quantized GEMV / skinny GEMM for gfx950: the kernel over the
// workgroup body in qgemv_dev.h, its launchers, and the end-of-step argmax.
#include "qgemv_dev.h"

namespace scry {
namespace {

using namespace dev;

template <int EPI, int PRO, int WT, int MT, int NCH>
__global__ __launch_bounds__(64 * shape_for(NCH, MT).nw) void k_qgemv(KArgs a) {
    if (a.ts) wg_stamp_begin(a.ts);
    qgemv_block<EPI, PRO, WT, MT, NCH>(a, blockIdx.x, blockIdx.y);
    if (a.ts) wg_stamp_end(a.ts);
}

// The split-k body for one activation row with k % 16 == 0 (every lane's
// activation values wholly inside or past k) at the Llama chunk counts:
// int8 per-tensor and block-32 rows of 4 chunks (k <= 4096; two row groups of
// 4 waves), 11 and 14 (the down projections; one row group of 11 or 14
// waves); bf16 rows of 8 chunks (k = 4096; 8 waves).  Rows per wave, measured
// on the Llama-2-7B step (stamped graph replays): 8 at k <= 4096 (4: decode
// 553.5 against 576.5 tok/s; 16: 567.6-573.9 against 577.1), 4 for the down
// projections (down 9.68 against 9.96-10.0 us at 8, 10.7 at 16, 12.4 at 2).
// gate/up takes one row group (4 waves, 2752 workgroups): 572.3 against
// 569.6 tok/s, event-timed gate/up 16.75 against 16.9 us.  The bf16
// down rows (22 and 28 chunks) stay on the LDS-staged body: as 11 waves of
// two chunks the bf16 model decoded 369-370 against 377-378 tok/s (4 rows
// per wave; 364 with 8).  Wave 0 finishes last, after the barrier.
constexpr int sk_cpw(int wt, int nch) { return wt == WT_BF16 && nch > 8 ? 2 : 1; }  // chunks per wave (2: measured only)
constexpr int sk_r(int epi, int wt, int nch) { return nch == 4 || nch == 8 ? 8 : 4; }  // rows per wave
constexpr int sk_groups(int epi, int wt, int nch) { return nch == 4 && epi != EPI_SWIGLU ? 2 : 1; }  // row groups per workgroup
constexpr int sk_waves(int epi, int wt, int nch) { return nch / sk_cpw(wt, nch) * sk_groups(epi, wt, nch); }
bool use_sk(int nch, int m, int wt, int k) {
    if (m != 1 || k % 16 != 0) return false;
    return wt == WT_BF16 ? nch == 8 : (nch == 4 || nch == 11 || nch == 14);
}
int sk_rows(int epi, int wt, int nch) { return sk_groups(epi, wt, nch) * sk_r(epi, wt, nch); }  // rows per workgroup

template <int EPI, int PRO, int WT, int NCH>
__global__ __launch_bounds__(64 * sk_waves(EPI, WT, NCH)) void k_qgemv_sk(KArgs a) {
    if (a.ts) wg_stamp_begin(a.ts);
    qgemv_sk_block<EPI, PRO, WT, NCH, sk_groups(EPI, WT, NCH), sk_r(EPI, WT, NCH), sk_cpw(WT, NCH)>(a, blockIdx.x);
    if (a.ts && __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) == 0)
        a.ts[2 * wg_linear_id() + 1] = __builtin_amdgcn_s_memrealtime();
}

template <int EPI, int PRO, int WT, int NCH>
int launch_sk_t(const KArgs &ka, hipStream_t s) {
    constexpr int RPW = sk_groups(EPI, WT, NCH) * sk_r(EPI, WT, NCH);
    hipLaunchKernelGGL((k_qgemv_sk<EPI, PRO, WT, NCH>), dim3((ka.rows + RPW - 1) / RPW),
                       dim3(64 * sk_waves(EPI, WT, NCH)), 0, s, ka);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

template <int EPI, int PRO>
int launch_sk(const KArgs &ka, int wt, hipStream_t s) {
    if (wt == WT_BF16) {
        if (ka.nch == 8) return launch_sk_t<EPI, PRO, WT_BF16, 8>(ka, s);
    } else if (wt == WT_I8B32) {
        if (ka.nch == 4) return launch_sk_t<EPI, PRO, WT_I8B32, 4>(ka, s);
        if (ka.nch == 11) return launch_sk_t<EPI, PRO, WT_I8B32, 11>(ka, s);
        if (ka.nch == 14) return launch_sk_t<EPI, PRO, WT_I8B32, 14>(ka, s);
    } else {
        if (ka.nch == 4) return launch_sk_t<EPI, PRO, WT_I8, 4>(ka, s);
        if (ka.nch == 11) return launch_sk_t<EPI, PRO, WT_I8, 11>(ka, s);
        if (ka.nch == 14) return launch_sk_t<EPI, PRO, WT_I8, 14>(ka, s);
    }
    return set_error(SCRY_ERR_INVALID, "qgemv: no split-k shape for %d chunks", ka.nch);
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
    if (use_sk(ka.nch, ka.m, wt, ka.k)) return launch_sk<EPI, PRO>(ka, wt, s);
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
    const int wt = weight_type(w), nch = row_chunks(w);
    if (use_sk(nch, m, wt, w.k)) return (w.rows + sk_rows(epi, wt, nch) - 1) / sk_rows(epi, wt, nch);
    const Sel sel = select_cfg(epi, row_chunks(w), m, weight_type(w));
    const Shape S = shape_for(sel.nch_t, sel.mt);
    return (w.rows + S.rwt * S.nw - 1) / (S.rwt * S.nw);
}

int qgemv_kargs(int epi, const GemvArgs &g, KArgs *out, int *wt_out, int *nch_out, int *pro_out) {
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
    const int max_ss = SSW * 64 * (use_sk(nch, g.m, wt, w.k) ? sk_waves(epi, wt, nch) : shape_for(sel.nch_t, sel.mt).nw);
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
    ka.ts = g.ts;
    *out = ka;
    *wt_out = wt;
    *nch_out = nch;
    *pro_out = pro;
    return SCRY_OK;
}

int launch_qgemv(int epi, const GemvArgs &g, hipStream_t s) {
    KArgs ka;
    int wt = 0, nch = 0, pro = 0;
    SCRY_TRY(qgemv_kargs(epi, g, &ka, &wt, &nch, &pro));
    const Sel sel = select_cfg(epi, nch, g.m, wt);
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
                                                       int64_t *argmax_out, int advance,
                                                       unsigned long long *ts) {
    if (ts) wg_stamp_begin(ts);
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
    if (ts) wg_stamp_end(ts);
}
}  // namespace

int launch_logits_finish(const GemvArgs &g, hipStream_t s) {
    const int np = qgemv_blocks(EPI_LOGITS, *g.w, 1);
    hipLaunchKernelGGL(k_logits_finish, dim3(1), dim3(TPB), 0, s, g.y, g.w->rows, g.part_val,
                       g.part_idx, g.part_nan, np, g.state, g.tokens_rw, g.argmax_out, g.advance, g.ts);
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
