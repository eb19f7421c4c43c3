// Persistent decode step for gfx950: one launch runs a whole token -- every
// layer's qkv / attention / o / gate-up / down stages and the LM head with the
// greedy argmax (llama.rs:744-763 per token, generate.rs:51-98 per step).
//
// Launch shape: one 512-thread workgroup per CU (the dynamic LDS request is
// sized so two cannot share a CU, so all workgroups are resident together).
// Waves are specialised:
//   waves 0-3  compute: stream weight items (4 rows x 1 KiB of one GEMV) through
//              a register ring RING items deep that runs ahead across stage
//              boundaries, FMA them against the activation chunk in LDS and
//              write one reduced partial per (item, row) to LDS.  They issue
//              only loads, so their in-flight prefetch never has to drain.
//   wave 4     control: between stages it finishes this workgroup's rows
//              (chunk partials -> bias removal -> scale -> fused epilogue),
//              publishes them with device-coherent stores, signals, waits for
//              every other workgroup, and stages the next stage's input vector
//              (with the fused RMSNorm) into LDS.
//   waves 4-7  attention: split-L attention over the cache for one
//              (query head, split) unit per workgroup; the last split of a
//              head to finish merges the head.
// Stage boundaries are a counter protocol without cache-wide fences: outputs
// are written with sc1 (device-coherent) stores, the control wave waits for
// them (vmcnt(0)) and adds 1 to one of 16 sub-counters of the stage; readers
// poll the sub-counters with device-scope atomic loads and read the outputs
// with sc1 loads.  Each (layer, stage) has its own output buffer, written once
// per launch.  Counters are never reset: after launch e every sub-counter of
// every stage holds (e+1) x (its number of workgroups).  Every wait is
// bounded; on timeout the kernel raises an abort flag and every workgroup
// leaves at its next barrier, so a grid that is not co-resident ends instead
// of hanging (the host reports the abort).
//
// Numerics follow the per-kernel path (qgemv.hip / attn.hip): RMSNorm in f64,
// int8 bytes stored as q+128 with the bias removed once per row as 128*sum(x),
// per-tensor scale, RoPE/SwiGLU/attention as there.  Row sums are taken per
// 1024-wide chunk and added in chunk order, so results are deterministic.
#include <cmath>

#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

using namespace dev;

constexpr int NCW = 4;               // compute waves
constexpr int NXW = 4;               // attention waves (the first is the control wave)
constexpr int RING = 8;              // weight items in flight per compute wave
// loads issued after a slot's four: 4 * (RING - 1)
#define RING_WAIT "s_waitcnt vmcnt(28)"
static_assert(4 * (RING - 1) == 28, "RING_WAIT must match RING");
constexpr int NSUB = 16;             // sub-counters per stage
constexpr int AU = 8;                // attention position loads in flight per lane group
constexpr unsigned OOB = 0x80000000u;  // buffer offset past every resource: reads 0
constexpr int SLOTS_MAX = 256;       // attention lane groups per workgroup (NXW * 64 / G)

enum { ST_QKV = 0, ST_ATTN = 1, ST_O = 2, ST_GU = 3, ST_DOWN = 4 };

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// device-coherent accesses (sc1): used for every value another workgroup
// produced in the same launch
__device__ __forceinline__ float4 cload16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16));
}
__device__ __forceinline__ float cloadf(const float *p) {
    return __builtin_bit_cast(float, __hip_atomic_load((unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ int cloadi(const int *p) {
    return __hip_atomic_load((int *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstoref(float *p, float v) {
    __hip_atomic_store((unsigned *)p, __builtin_bit_cast(unsigned, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstorei(int *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until this wave's stores are complete (vector memory counter to zero);
// also a compiler barrier for memory operations
__device__ __forceinline__ void drain_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float *ws_layer(const DecArgs &a, int l) { return a.ws + (size_t)l * a.ws_stride; }

// The per-layer table is read through the constant address space: the kernel
// stores to global memory, so generic loads of it would not become scalar
// loads (and a vector load here would make the compute waves wait for their
// whole weight prefetch).
typedef const __attribute__((address_space(4))) DecLayer *CLayers;
__device__ __forceinline__ CLayers lay(const DecArgs &a, int l) { return (CLayers)(uintptr_t)a.layers + l; }

struct GDesc {
    const uint8_t *W;
    int k, kp, rows, nch;
};

// GEMV stage g (g = 5l + type, g = 5L: LM head)
__device__ __forceinline__ GDesc gdesc(const DecArgs &a, int g) {
    GDesc d;
    if (g >= 5 * a.L) {
        d.W = a.w_lm;
        d.k = a.h;
        d.kp = a.kp_h;
        d.rows = a.V;
    } else {
        // scalar selects (a switch here becomes a private-memory lookup table)
        const int t = g % 5;
        const bool o = t == ST_O, gu = t == ST_GU, dn = t == ST_DOWN;
        d.W = lay(a, g / 5)->w[o ? 1 : gu ? 2 : dn ? 3 : 0];
        d.k = o ? a.qd : dn ? a.ffn : a.h;
        d.kp = o ? a.kp_q : dn ? a.kp_f : a.kp_h;
        d.rows = (o || dn) ? a.h : gu ? 2 * a.ffn : a.qkv_rows;
    }
    d.nch = (d.k + 1023) >> 10;
    return d;
}

// This workgroup's row groups (4 rows each): [rg0, rg0 + nrg)
__device__ __forceinline__ void rg_range(int rows, int &rg0, int &nrg) {
    const unsigned n_rg = (unsigned)(rows + 3) >> 2, b = blockIdx.x, nw = gridDim.x;
    rg0 = (int)(n_rg * b / nw);
    nrg = (int)(n_rg * (b + 1) / nw) - rg0;
}

// ------------------------------------------------------------ compute waves
// Load cursor over this wave's items of all GEMV stages of the token: item f
// of a stage is (row group f / nch, chunk f % nch) of the workgroup's list;
// wave w takes f = w, w + 4, ...
struct LCur {
    int g, f, rgl, c, nit, nch, kp, rg0;
    u32x4 desc;  // buffer descriptor of the stage's weights (scalar registers)
};

// Buffer descriptor words (as __builtin_amdgcn_make_buffer_rsrc builds them):
// base, stride 0, num_records, raw-buffer flags.
__device__ __forceinline__ u32x4 make_desc(const void *base, size_t bytes) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const unsigned n = bytes > 0x7fffffffu ? 0x7fffffffu : (unsigned)bytes;
    return u32x4{(unsigned)b, (unsigned)(b >> 32) & 0xffffu, n, 0x00020000u};
}

// Weight loads of the compute waves are issued from inline assembly and waited
// for explicitly (RING_WAIT below): the compiler's wait-count analysis cannot
// follow a ring that spans the stage-transition control flow and would wait
// for the whole ring before every item.  `dep` orders the load after the
// computation that last read the destination registers.
__device__ __forceinline__ u32x4 ring_load(u32x4 desc, unsigned off, float dep) {
    // the descriptor is wave-uniform; say so (folds away when already scalar)
    desc.x = __builtin_amdgcn_readfirstlane(desc.x);
    desc.y = __builtin_amdgcn_readfirstlane(desc.y);
    desc.z = __builtin_amdgcn_readfirstlane(desc.z);
    desc.w = __builtin_amdgcn_readfirstlane(desc.w);
    u32x4 v;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen nt" : "=v"(v) : "v"(off), "s"(desc), "v"(dep) : "memory");
    return v;
}

__device__ __forceinline__ void lcur_seek(LCur &q, const DecArgs &a, int g, int w) {
    const int last = 5 * a.L;
    for (; g <= last; g++) {
        if (g < last && g % 5 == ST_ATTN) continue;
        const GDesc d = gdesc(a, g);
        int rg0, nrg;
        rg_range(d.rows, rg0, nrg);
        const int nit = nrg * d.nch;
        if (w < nit) {
            q.g = g;
            q.f = w;
            q.rgl = w / d.nch;
            q.c = w - q.rgl * d.nch;
            q.nit = nit;
            q.nch = d.nch;
            q.kp = d.kp;
            q.rg0 = rg0;
            q.desc = make_desc(d.W, (size_t)d.rows * d.kp);
            return;
        }
    }
    // exhausted: a null descriptor (num_records 0), so the placeholder loads
    // the ring keeps issuing read zeros without touching memory -- also for a
    // wave that never had an item
    q.g = last + 1;
    q.desc = u32x4{0u, 0u, 0u, 0x00020000u};
}

__device__ __forceinline__ void lcur_next(LCur &q, const DecArgs &a, int w) {
    q.f += NCW;
    if (q.f >= q.nit) {
        lcur_seek(q, a, q.g + 1, w);
        return;
    }
    q.c += NCW;
    while (q.c >= q.nch) {
        q.c -= q.nch;
        q.rgl++;
    }
}

// One item: 4 rows x 16 bytes per lane against x[c*1024 + 16 lane ..], reduced
// over the wave to one partial per row; lanes 0/16/32/48 store rows 0-3.
__device__ __forceinline__ float item_fma(const u32x4 (&wv)[4], const float *xs, float *part, int c, int f,
                                          int lane) {
    const float *xb = xs + (c << 10) + (lane << 2);
    const float4 x0 = *(const float4 *)(xb);
    const float4 x1 = *(const float4 *)(xb + 256);
    const float4 x2 = *(const float4 *)(xb + 512);
    const float4 x3 = *(const float4 *)(xb + 768);
    const float a0 = dot16(wv[0], x0, x1, x2, x3, 0.f);
    const float a1 = dot16(wv[1], x0, x1, x2, x3, 0.f);
    const float a2 = dot16(wv[2], x0, x1, x2, x3, 0.f);
    const float a3 = dot16(wv[3], x0, x1, x2, x3, 0.f);
    // reduce-scatter: lanes keep rows {0,1} / {2,3} by bit 5, then one row by bit 4
    const bool h32 = (lane & 32) != 0, h16 = (lane & 16) != 0;
    float k0 = h32 ? a2 : a0, k1 = h32 ? a3 : a1;
    const float s0 = h32 ? a0 : a2, s1 = h32 ? a1 : a3;
    k0 += __shfl_xor(s0, 32);
    k1 += __shfl_xor(s1, 32);
    float k = h16 ? k1 : k0;
    const float s = h16 ? k0 : k1;
    k += __shfl_xor(s, 16);
    k += __shfl_xor(k, 8);
    k += __shfl_xor(k, 4);
    k += __shfl_xor(k, 2);
    k += __shfl_xor(k, 1);
    if ((lane & 15) == 0) part[(f << 2) + (lane >> 4)] = k;
    return k;
}

// ------------------------------------------------------------ control wave
struct Shared {
    int abort, pos, crow, tok, n_prompt, max_tokens;
    float sx;
};

// Counter-based grid barrier wait for stage g (control wave).
__device__ __forceinline__ bool poll_stage(const DecArgs &a, int g, int lane) {
    const int nwg = gridDim.x;
    unsigned *c = a.ctr + (size_t)g * NSUB;
    const unsigned tgt = lane < NSUB ? (a.epoch + 1u) * (unsigned)((nwg - lane + NSUB - 1) / NSUB) : 0u;
    for (unsigned it = 0;; it++) {
        const unsigned v = lane < NSUB ? __hip_atomic_load(c + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        const bool ok = (int)(v - tgt) >= 0;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (it >= a.spin_limit) {
            if (lane == 0) cstorei(a.abort_flag, 1);
            return false;
        }
        if ((it & 31) == 31 && uni(cloadi(a.abort_flag))) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    asm volatile("" ::: "memory");
    return true;
}

__device__ __forceinline__ void signal_stage(const DecArgs &a, int g, int lane) {
    drain_stores();
    if (lane == 0)
        __hip_atomic_fetch_add(a.ctr + (size_t)g * NSUB + (blockIdx.x & (NSUB - 1)), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// Stage k floats of src (optionally RMSNorm'd with weight nw) into the LDS
// activation layout: x[p*1024 + 4t .. +3] at xslot(p, t), zero past k; sum of
// the staged values -> sh.sx (one wave, t = lane + 64 q).
__device__ __forceinline__ void stage_x(const float *src, int k, const float *nw, float eps, float *xs, Shared &sh, int lane) {
    const int nch = (k + 1023) >> 10;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (size_t)k * 4);
    auto off = [&](int p, int q) -> unsigned {
        return p < nch ? (unsigned)(((p << 10) + ((lane + (q << 6)) << 2)) << 2) : OOB;
    };
    double sx = 0.0;
    if (nw != nullptr && nch <= 4) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(nw, (size_t)k * 4);
        float4 v[16], wv[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = cload16(r, off(j >> 2, j & 3));
#pragma unroll
        for (int j = 0; j < 16; j++) wv[j] = bload16f(rw, off(j >> 2, j & 3));
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++)
            ss += (double)v[j].x * v[j].x + (double)v[j].y * v[j].y + (double)v[j].z * v[j].z +
                  (double)v[j].w * v[j].w;
        ss = wave_sum_d(ss);
        // cpu.rs:574-599: rstd = 1/sqrt(mean(x^2) + eps) in f64; out = f32(x*rstd*w)
        const double rstd = 1.0 / sqrt(ss / (double)k + (double)eps);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            float4 o;
            o.x = (float)((double)v[j].x * rstd * (double)wv[j].x);
            o.y = (float)((double)v[j].y * rstd * (double)wv[j].y);
            o.z = (float)((double)v[j].z * rstd * (double)wv[j].z);
            o.w = (float)((double)v[j].w * rstd * (double)wv[j].w);
            sx += (double)o.x + (double)o.y + (double)o.z + (double)o.w;
            const int p = j >> 2;
            if (p < nch) *(float4 *)(xs + xslot(p, lane + ((j & 3) << 6))) = o;
        }
    } else if (nw != nullptr) {
        // k > 4096: sum of squares first, then a second (cache-resident) pass
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(nw, (size_t)k * 4);
        double ss = 0.0;
        for (int p0 = 0; p0 < nch; p0 += 4) {
            float4 v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = cload16(r, off(p0 + (j >> 2), j & 3));
#pragma unroll
            for (int j = 0; j < 16; j++)
                ss += (double)v[j].x * v[j].x + (double)v[j].y * v[j].y + (double)v[j].z * v[j].z +
                      (double)v[j].w * v[j].w;
        }
        ss = wave_sum_d(ss);
        const double rstd = 1.0 / sqrt(ss / (double)k + (double)eps);
        for (int p0 = 0; p0 < nch; p0 += 4) {
            float4 v[16], wv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = cload16(r, off(p0 + (j >> 2), j & 3));
#pragma unroll
            for (int j = 0; j < 16; j++) wv[j] = bload16f(rw, off(p0 + (j >> 2), j & 3));
#pragma unroll
            for (int j = 0; j < 16; j++) {
                float4 o;
                o.x = (float)((double)v[j].x * rstd * (double)wv[j].x);
                o.y = (float)((double)v[j].y * rstd * (double)wv[j].y);
                o.z = (float)((double)v[j].z * rstd * (double)wv[j].z);
                o.w = (float)((double)v[j].w * rstd * (double)wv[j].w);
                sx += (double)o.x + (double)o.y + (double)o.z + (double)o.w;
                const int p = p0 + (j >> 2);
                if (p < nch) *(float4 *)(xs + xslot(p, lane + ((j & 3) << 6))) = o;
            }
        }
    } else {
        for (int p0 = 0; p0 < nch; p0 += 8) {
            float4 v[32];
#pragma unroll
            for (int j = 0; j < 32; j++) v[j] = cload16(r, off(p0 + (j >> 2), j & 3));
#pragma unroll
            for (int j = 0; j < 32; j++) {
                sx += (double)v[j].x + (double)v[j].y + (double)v[j].z + (double)v[j].w;
                const int p = p0 + (j >> 2);
                if (p < nch) *(float4 *)(xs + xslot(p, lane + ((j & 3) << 6))) = v[j];
            }
        }
    }
    sx = wave_sum_d(sx);
    if (lane == 0) sh.sx = (float)sx;
}

// Input of GEMV stage s (s = 5L: LM head) staged into LDS.
__device__ __forceinline__ void stage_input(const DecArgs &a, int s, float *xs, Shared &sh, int lane) {
    const int last = 5 * a.L;
    const int l = s >= last ? a.L : s / 5;
    const int t = s >= last ? -1 : s % 5;
    const float *src;
    const float *nw = nullptr;
    int k = a.h;
    if (t == ST_QKV) {
        src = l == 0 ? a.embed + (size_t)uni(sh.tok) * a.h : ws_layer(a, l - 1) + a.o_xd;
        nw = lay(a, l)->norm_in;
    } else if (t == ST_O) {
        src = ws_layer(a, l) + a.o_xa;
        k = a.qd;
    } else if (t == ST_GU) {
        src = ws_layer(a, l) + a.o_xo;
        nw = lay(a, l)->norm_post;
    } else if (t == ST_DOWN) {
        src = ws_layer(a, l) + a.o_xg;
        k = a.ffn;
    } else {
        src = ws_layer(a, a.L - 1) + a.o_xd;
        nw = a.norm_final;
    }
    stage_x(src, k, nw, a.eps, xs, sh, lane);
}

// Row i of this workgroup's block: chunk partials in order, bias, scale.
__device__ __forceinline__ float row_val(const float *part, int i, int nch, float sc, float corr) {
    const int rgl = i >> 2, r = i & 3;
    float s = 0.f;
    for (int c = 0; c < nch; c++) s += part[(((rgl * nch) + c) << 2) + r];
    return sc * (s - corr);
}

__device__ __forceinline__ ArgAcc wave_argmax(ArgAcc acc, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        ArgAcc o;
        o.v = __shfl_down(acc.v, off);
        o.i = __shfl_down(acc.i, off);
        o.nan = __shfl_down(acc.nan, off);
        if ((lane & (2 * off - 1)) == 0) acc = arg_combine(acc, o);
    }
    acc.v = __shfl(acc.v, 0);
    acc.i = __shfl(acc.i, 0);
    acc.nan = __shfl(acc.nan, 0);
    return acc;
}

__device__ __forceinline__ void acc_value(ArgAcc &p, float v, int row) {
    if (isnan(v)) {
        p.nan = row;
        return;
    }
    if (p.i < 0 || !(p.v > v)) {
        p.v = v;
        p.i = row;
    }
}

// Fused epilogue of GEMV stage g for this workgroup's rows (control wave).
__device__ __forceinline__ void epilogue(const DecArgs &a, int g, const float *part, Shared &sh, int lane) {
    const GDesc d = gdesc(a, g);
    int rg0, nrg;
    rg_range(d.rows, rg0, nrg);
    const int R0 = rg0 * 4;
    const int nr = min(d.rows, (rg0 + nrg) * 4) - R0;
    if (nr <= 0 && g < 5 * a.L) return;
    const float corr = 128.f * sh.sx;
    const int nch = d.nch;
    if (g >= 5 * a.L) {  // LM head: logits + ordered argmax partial of this workgroup
        ArgAcc p{0.f, -1, -1};
        const int per = (max(nr, 0) + 63) >> 6;
        const int i0 = lane * per, i1 = min(nr, i0 + per);
        for (int i = i0; i < i1; i++) {
            const float v = row_val(part, i, nch, a.s_lm, corr);
            cstoref(a.logits + R0 + i, v);
            acc_value(p, v, R0 + i);
        }
        p = wave_argmax(p, lane);
        if (lane == 0) {
            cstoref(a.lm_pv + blockIdx.x, p.v);
            cstorei(a.lm_pi + blockIdx.x, p.i);
            cstorei(a.lm_pn + blockIdx.x, p.nan);
        }
        return;
    }
    const int l = g / 5;
    const CLayers Ly = lay(a, l);
    float *W = ws_layer(a, l);
    switch (g % 5) {
        case ST_QKV: {
            const int pos = uni(sh.pos), crow = uni(sh.crow), hh = a.hd >> 1;
            float *kr = Ly->k_cache + (size_t)crow * a.kvd;
            float *vr = Ly->v_cache + (size_t)crow * a.kvd;
            for (int pidx = lane; pidx < (nr >> 1); pidx += 64) {
                const int j = R0 + 2 * pidx;
                const float x0 = row_val(part, 2 * pidx, nch, Ly->scale[0], corr);
                const float x1 = row_val(part, 2 * pidx + 1, nch, Ly->scale[0], corr);
                if (j < a.qd + a.kvd) {
                    const bool isq = j < a.qd;
                    const int jj = isq ? j : j - a.qd;
                    const float2 cs = a.rope_cs[(size_t)pos * hh + ((jj % a.hd) >> 1)];
                    // cpu.rs:655-658 in f32, no contraction
                    const float r0 = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
                    const float r1 = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
                    if (isq) {
                        cstoref(W + a.o_xq + jj, __fmul_rn(r0, a.q_scale));
                        cstoref(W + a.o_xq + jj + 1, __fmul_rn(r1, a.q_scale));
                    } else {
                        cstoref(kr + jj, r0);
                        cstoref(kr + jj + 1, r1);
                    }
                } else {
                    const int jj = j - a.qd - a.kvd;
                    cstoref(vr + jj, x0);
                    cstoref(vr + jj + 1, x1);
                }
            }
            break;
        }
        case ST_O: {
            const float *res = l == 0 ? a.embed + (size_t)uni(sh.tok) * a.h : ws_layer(a, l - 1) + a.o_xd;
            for (int i = lane; i < nr; i += 64) {
                const int j = R0 + i;
                cstoref(W + a.o_xo + j, cloadf(res + j) + row_val(part, i, nch, Ly->scale[1], corr));
            }
            break;
        }
        case ST_GU: {
            // rows of a group: gate[2t], gate[2t+1], up[2t], up[2t+1]
            for (int q = lane; q < nrg; q += 64) {
                const float g0 = row_val(part, 4 * q, nch, Ly->scale[2], corr);
                const float g1 = row_val(part, 4 * q + 1, nch, Ly->scale[2], corr);
                const float u0 = row_val(part, 4 * q + 2, nch, Ly->scale[3], corr);
                const float u1 = row_val(part, 4 * q + 3, nch, Ly->scale[3], corr);
                const int t = 2 * (rg0 + q);
                cstoref(W + a.o_xg + t, silu_f(g0) * u0);
                cstoref(W + a.o_xg + t + 1, silu_f(g1) * u1);
            }
            break;
        }
        case ST_DOWN: {
            const float *res = W + a.o_xo;
            for (int i = lane; i < nr; i += 64) {
                const int j = R0 + i;
                cstoref(W + a.o_xd + j, cloadf(res + j) + row_val(part, i, nch, Ly->scale[4], corr));
            }
            break;
        }
        default: break;
    }
}

// ------------------------------------------------------------ attention
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Unit (query head hq, split sp) over cache positions [t0, t1) of layer l by
// the attention waves (aw = 0..3); per-lane-group online softmax state -> LDS.
template <int G>
__device__ __forceinline__ void attn_part(const DecArgs &a, int l, int unit, int aw, int crow, float *s_ao, float *s_am,
                          float *s_al, int lane) {
    constexpr int P = 64 / G;
    constexpr int PI = P * AU;
    const int sub = lane / G, gl = lane % G;
    const int ns = a.ns, hq = unit / ns, sp = unit - hq * ns;
    const int kh = hq / (a.n_heads / a.n_kv), hd = a.hd, kvd = a.kvd;
    const int Lc = crow + 1, chunk = (Lc + ns - 1) / ns;
    const int t0 = min(Lc, sp * chunk), t1 = min(Lc, t0 + chunk);
    const bool dact = gl * 4 < hd;
    const CLayers Ly = lay(a, l);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(Ly->k_cache, (size_t)t1 * kvd * 4);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(Ly->v_cache, (size_t)t1 * kvd * 4);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(ws_layer(a, l) + a.o_xq, (size_t)a.qd * 4);
    const unsigned col = (unsigned)(kh * hd + gl * 4) * 4;
    const float4 qf = cload16(qr, dact ? (unsigned)(hq * hd + gl * 4) * 4 : OOB);
    float m = -INFINITY, ls = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int tb = t0 + aw * PI; tb < t1; tb += NXW * PI) {
        float4 kv[AU], vv[AU];
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int t = tb + u * P + sub;
            const unsigned off = (t < t1 && dact) ? (unsigned)t * kvd * 4 + col : OOB;
            kv[u] = cload16(kr, off);
            vv[u] = cload16(vr, off);
        }
        float sc[AU];
        float mx = m;
#pragma unroll
        for (int u = 0; u < AU; u++) {
            float d = qf.x * kv[u].x + qf.y * kv[u].y + qf.z * kv[u].z + qf.w * kv[u].w;
            d = group_sum<G>(d);
            sc[u] = (tb + u * P + sub < t1) ? d : -INFINITY;
            mx = fmaxf(mx, sc[u]);
        }
        if (mx == -INFINITY) continue;  // no position for this lane group yet
        const float f = expf(m - mx);
        ls *= f;
        o.x *= f;
        o.y *= f;
        o.z *= f;
        o.w *= f;
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const float p = expf(sc[u] - mx);
            ls += p;
            o.x += p * vv[u].x;
            o.y += p * vv[u].y;
            o.z += p * vv[u].z;
            o.w += p * vv[u].w;
        }
        m = mx;
    }
    const int slot = aw * P + sub;
    if (gl == 0) {
        s_am[slot] = m;
        s_al[slot] = ls;
    }
    if (dact) *(float4 *)(s_ao + (size_t)slot * hd + gl * 4) = o;
}

// Control wave after the attention waves: merge the lane-group slots into the
// unit's partial (M, L, O), publish it, and if this was the head's last split,
// merge the head's splits into the attention output row.
__device__ __forceinline__ void attn_publish(const DecArgs &a, int l, int unit, int nslots, const float *s_ao,
                             const float *s_am, const float *s_al, int lane) {
    const int ns = a.ns, hq = unit / ns, sp = unit - hq * ns, hd = a.hd;
    float *W = ws_layer(a, l);
    float *apo = W + a.o_apo, *apm = W + a.o_apm;
    float M = -INFINITY;
    for (int q = 0; q < nslots; q++) M = fmaxf(M, s_am[q]);
    float lsum = 0.f;
    if (M != -INFINITY)
        for (int q = 0; q < nslots; q++)
            if (s_am[q] != -INFINITY) lsum += s_al[q] * expf(s_am[q] - M);
    const size_t ph = (size_t)hq * ns + sp;
    for (int d = lane; d < hd; d += 64) {
        float osum = 0.f;
        if (M != -INFINITY)
            for (int q = 0; q < nslots; q++)
                if (s_am[q] != -INFINITY) osum += s_ao[(size_t)q * hd + d] * expf(s_am[q] - M);
        cstoref(apo + ph * hd + d, osum);
    }
    if (lane == 0) {
        cstoref(apm + ph * 2, M);
        cstoref(apm + ph * 2 + 1, lsum);
    }
    drain_stores();
    unsigned old = 0;
    unsigned *hc = a.ctr + (size_t)(5 * a.L + 1) * NSUB + (size_t)l * a.n_heads + hq;
    if (lane == 0) old = __hip_atomic_fetch_add(hc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (unsigned)uni((int)old);
    if (old + 1u != (a.epoch + 1u) * (unsigned)ns) return;
    asm volatile("" ::: "memory");
    // last split of head hq: x[hq*hd + d] = sum_s O_s[d] e^(M_s - M) / sum_s L_s e^(M_s - M)
    float Mh = -INFINITY;
    for (int s = 0; s < ns; s++) Mh = fmaxf(Mh, cloadf(apm + ((size_t)hq * ns + s) * 2));
    float Ls = 0.f;
    for (int s = 0; s < ns; s++) {
        const float ms = cloadf(apm + ((size_t)hq * ns + s) * 2);
        if (ms != -INFINITY) Ls += cloadf(apm + ((size_t)hq * ns + s) * 2 + 1) * expf(ms - Mh);
    }
    for (int d = lane; d < hd; d += 64) {
        float v = 0.f;
        for (int s = 0; s < ns; s++) {
            const float ms = cloadf(apm + ((size_t)hq * ns + s) * 2);
            const float w = ms == -INFINITY ? 0.f : expf(ms - Mh) / Ls;
            v += w * cloadf(apo + ((size_t)hq * ns + s) * hd + d);
        }
        cstoref(W + a.o_xa + hq * hd + d, v);
    }
}

// Workgroup 0 after the LM head: ordered argmax over the workgroup partials
// (generate.rs:167-173), next token, position advance.
__device__ __forceinline__ void finish(const DecArgs &a, Shared &sh, int lane) {
    const int nwg = gridDim.x, V = a.V;
    const int per = (nwg + 63) >> 6;
    ArgAcc acc{0.f, -1, -1};
    for (int t = lane * per; t < min(nwg, lane * per + per); t++)
        acc = arg_combine(acc, ArgAcc{cloadf(a.lm_pv + t), cloadi(a.lm_pi + t), cloadi(a.lm_pn + t)});
    acc = wave_argmax(acc, lane);
    int tok;
    if (acc.nan < 0) {
        tok = acc.i < 0 ? 0 : acc.i;
    } else if (acc.nan == V - 1) {
        tok = acc.nan;
    } else {
        // max_by hands the running best to the element after the last NaN:
        // the answer is the argmax of the suffix after it
        const int lo = acc.nan + 1, n = V - lo, per2 = (n + 63) >> 6;
        ArgAcc s{0.f, -1, -1};
        for (int i = lo + lane * per2; i < min(V, lo + lane * per2 + per2); i++) acc_value(s, cloadf(a.logits + i), i);
        s = wave_argmax(s, lane);
        tok = s.i;
    }
    if (lane == 0) {
        const int p = sh.pos;
        if (a.argmax_out) a.argmax_out[0] = tok;
        if (a.advance) {
            if (p + 1 <= sh.max_tokens && p + 1 >= sh.n_prompt) a.tokens[p + 1] = tok;
            a.state->pos = p + 1;
            a.state->cache_len = sh.crow + 1;
        }
    }
}

// ------------------------------------------------------------ the kernel
template <int G>
__global__ __launch_bounds__(DEC_THREADS) void k_decode(DecArgs a) {
    extern __shared__ float4 dyn4[];
    float *xs = reinterpret_cast<float *>(dyn4);
    float *part = xs + (size_t)a.nch_max * 1024;
    float *s_ao = part + (size_t)a.part_cap * 4;
    float *s_am = s_ao + 1024;
    float *s_al = s_am + SLOTS_MAX;
    __shared__ Shared sh;

    const int lane = threadIdx.x & 63;
    const int wave = uni(threadIdx.x >> 6);
    const int last = 5 * a.L;

    if (wave < NCW) {
        // ---------------- compute waves
        const int w = wave;
        const unsigned lane16 = (unsigned)lane << 4;
        LCur lq;
        lcur_seek(lq, a, 0, w);
        u32x4 wr[RING][4];
        int tg[RING], tf[RING], tc[RING];
        float dep = 0.f;
#define SCRY_ISSUE(r)                                                                         \
    {                                                                                         \
        const bool v_ = lq.g <= last;                                                         \
        const unsigned b_ = (unsigned)((lq.rg0 + lq.rgl) * 4 * lq.kp + (lq.c << 10)) + lane16; \
        _Pragma("unroll") for (int q_ = 0; q_ < 4; q_++)                                      \
            wr[r][q_] = ring_load(lq.desc, v_ ? b_ + (unsigned)(q_ * lq.kp) : OOB, dep);       \
        tg[r] = v_ ? lq.g : -1;                                                               \
        tf[r] = lq.f;                                                                         \
        tc[r] = lq.c;                                                                         \
        if (v_) lcur_next(lq, a, w);                                                          \
    }
#pragma unroll
        for (int r = 0; r < RING; r++) SCRY_ISSUE(r)
        __syncthreads();  // B0: launch state read
        if (uni(sh.abort)) return;
        __syncthreads();  // B2(0)
        if (uni(sh.abort)) return;
        int cur = 0;
        for (;;) {
#pragma unroll
            for (int r = 0; r < RING; r++) {
                const int g = tg[r];
                if (g < 0) goto drain;
                if (g != cur) {
                    __syncthreads();  // B1(cur)
                    for (cur++; cur < g; cur++) {
                        __syncthreads();  // B2(cur)
                        if (uni(sh.abort)) return;
                        __syncthreads();  // B1(cur)
                    }
                    __syncthreads();  // B2(g)
                    if (uni(sh.abort)) return;
                }
                asm volatile(RING_WAIT : "+v"(wr[r][0]), "+v"(wr[r][1]), "+v"(wr[r][2]), "+v"(wr[r][3])::"memory");
                dep = item_fma(wr[r], xs, part, tc[r], tf[r], lane);
                SCRY_ISSUE(r)
            }
        }
#undef SCRY_ISSUE
    drain:
        __syncthreads();  // B1(cur)
        for (cur++; cur <= last; cur++) {
            __syncthreads();  // B2(cur)
            if (uni(sh.abort)) return;
            __syncthreads();  // B1(cur)
        }
        return;
    }

    // ---------------- attention / control waves
    const int aw = wave - NCW;
    const bool ctl = aw == 0;
    const int units = a.n_heads * a.ns;
    const int nslots = NXW * (64 / G);
    if (ctl) {
        const int ab = cloadi(a.abort_flag);
        const int pos = a.state->pos;
        const int tok = (int)a.tokens[pos];
        if (lane == 0) {
            sh.abort = ab;
            sh.pos = pos;
            sh.crow = a.state->cache_len;
            sh.tok = tok;
            sh.n_prompt = a.state->n_prompt;
            sh.max_tokens = a.state->max_tokens;
        }
    }
    __syncthreads();  // B0
    if (uni(sh.abort)) return;
    const int crow = uni(sh.crow);
    if (ctl) stage_input(a, 0, xs, sh, lane);
    __syncthreads();  // B2(0)
    if (uni(sh.abort)) return;
    for (int g = 0; g <= last; g++) {
        const int t = g < last ? g % 5 : -1;
        const int l = g / 5;
        if (t == ST_ATTN && (int)blockIdx.x < units) attn_part<G>(a, l, blockIdx.x, aw, crow, s_ao, s_am, s_al, lane);
        __syncthreads();  // B1(g)
        if (ctl) {
            if (t == ST_ATTN) {
                if ((int)blockIdx.x < units) attn_publish(a, l, blockIdx.x, nslots, s_ao, s_am, s_al, lane);
            } else {
                epilogue(a, g, part, sh, lane);
            }
            signal_stage(a, g, lane);
            if (g == last) {
                if (blockIdx.x == 0 && poll_stage(a, g, lane)) finish(a, sh, lane);
                return;
            }
            if (poll_stage(a, g, lane)) {
                if (t != ST_QKV) stage_input(a, g + 1, xs, sh, lane);
            } else if (lane == 0) {
                sh.abort = 1;
            }
        }
        if (g == last) return;
        __syncthreads();  // B2(g+1)
        if (uni(sh.abort)) return;
    }
}

template <int G>
const void *kfn() {
    return reinterpret_cast<const void *>(&k_decode<G>);
}

int pick_g(int hd) {
    const int lanes = (hd + 3) / 4;
    if (lanes <= 8) return 8;
    if (lanes <= 16) return 16;
    if (lanes <= 32) return 32;
    if (lanes <= 64) return 64;
    return 0;
}

const void *kernel_for(int hd) {
    switch (pick_g(hd)) {
        case 8: return kfn<8>();
        case 16: return kfn<16>();
        case 32: return kfn<32>();
        case 64: return kfn<64>();
    }
    return nullptr;
}

}  // namespace

size_t decode_lds_bytes(int nch_max, int part_cap) {
    return sizeof(float) * ((size_t)nch_max * 1024 + (size_t)part_cap * 4 + 1024 + 2 * SLOTS_MAX);
}

int decode_prepare(int hd, size_t lds, int n_wg) {
    const void *f = kernel_for(hd);
    if (!f) return set_error(SCRY_ERR_UNSUPPORTED, "decode: head_dim %d > 256", hd);
    SCRY_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int nb = 0;
    SCRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, DEC_THREADS, lds));
    if (nb < 1 || n_wg > ctx().cu_count * nb)
        return set_error(SCRY_ERR_UNSUPPORTED, "decode: %d workgroups cannot be co-resident (%d per CU)", n_wg, nb);
    return SCRY_OK;
}

int launch_decode(const DecArgs &a, int n_wg, size_t lds, hipStream_t s) {
    switch (pick_g(a.hd)) {
        case 8: hipLaunchKernelGGL((k_decode<8>), dim3(n_wg), dim3(DEC_THREADS), lds, s, a); break;
        case 16: hipLaunchKernelGGL((k_decode<16>), dim3(n_wg), dim3(DEC_THREADS), lds, s, a); break;
        case 32: hipLaunchKernelGGL((k_decode<32>), dim3(n_wg), dim3(DEC_THREADS), lds, s, a); break;
        case 64: hipLaunchKernelGGL((k_decode<64>), dim3(n_wg), dim3(DEC_THREADS), lds, s, a); break;
        default: return set_error(SCRY_ERR_UNSUPPORTED, "decode: head_dim %d", a.hd);
    }
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
