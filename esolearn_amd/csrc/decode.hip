// Persistent decode step for gfx950: one launch runs a whole token -- every
// layer's qkv / attention / o / gate-up / down stages and the LM head with the
// greedy argmax (llama.rs:744-763 per token, generate.rs:51-98 per step).
//
// Launch shape: one 512-thread workgroup per CU (the LDS request and register
// count keep two from sharing a CU, so all workgroups are resident together).
// Waves are specialised:
//   waves 0-3  compute: stream weight items (4 rows x 1 KiB of one GEMV) into
//              a per-wave LDS ring RING items deep (buffer loads that write
//              LDS directly), FMA them against the activation chunk in LDS and
//              write one reduced partial per (item, row) to LDS.  They issue
//              only loads.
//   waves 4-7  aux: stage each stage's input vector into LDS (with the fused
//              RMSNorm), and run split-L attention for one (query head, split)
//              unit per workgroup.  Wave 4, the control wave, also finishes
//              this workgroup's rows of every GEMV (chunk partials -> bias
//              removal -> scale -> fused epilogue), publishes them and merges
//              attention splits.
// A CU's vector memory requests are served in order, so anything on the
// critical path of a stage boundary (epilogue stores, input loads) waits
// behind all weight loads the CU already has in flight.  Hence:
//   - the ring runs at full depth inside a stage but only LOOKAHEAD items per
//     compute wave into the next stage, so at a boundary the queue is short;
//   - completion is signalled per (stage, XCD) with device-scope atomic adds
//     after the outputs are written (s_waitcnt vmcnt(0) orders them), and
//     polled with scalar loads (glc), which do not queue behind vector loads;
//   - residual rows and RoPE factors are kept in LDS instead of re-read.
// Outputs live in uncached device memory, use device-coherent (sc1) stores and
// are read with sc1 loads; each
// (layer, stage) buffer is written once per launch; counters are never reset
// (after launch t each holds t x its number of contributors).  Every wait is
// bounded: on timeout the kernel raises an abort flag and every workgroup
// leaves at its next barrier (the host reports it).
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
constexpr int RING = 4;              // weight items in flight per compute wave (LDS slots)
constexpr int SLOT_BYTES = 4096;     // one item: 4 rows x 1 KiB
// loads issued after a slot's four: 4 * (RING - 1)
#define RING_WAIT "s_waitcnt vmcnt(12)"
static_assert(4 * (RING - 1) == 12, "RING_WAIT must match RING");
constexpr int AU = 8;                // attention position loads in flight per lane group
constexpr unsigned OOB = 0x80000000u;  // buffer offset past every resource: reads 0
constexpr int SLOTS_MAX = 256;       // attention lane groups per workgroup (NXW * 64 / G)
constexpr int MAXNS = 16;            // attention splits per head
constexpr int MAXCH = 16;            // 1024-wide chunks of a staged input (k <= 16384)
constexpr int LOOKAHEAD = 2;         // items a compute wave loads ahead into the next stage
constexpr int NXCD = 8;              // XCDs: workgroup b runs on XCD b % 8

enum { ST_QKV = 0, ST_ATTN = 1, ST_O = 2, ST_GU = 3, ST_DOWN = 4 };

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// device-coherent (sc1) accesses
__device__ __forceinline__ float4 cload16f(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16));
}
__device__ __forceinline__ float cloadf(const float *p) {
    return __uint_as_float(__hip_atomic_load((unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void cstoref(float *p, float v) {
    __hip_atomic_store((unsigned *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstoreu(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int cloadi(const int *p) {
    return __hip_atomic_load((int *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstorei(int *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float *wsl(const DecArgs &a, int l) { return a.ws + (size_t)l * a.ws_stride; }

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
    int g, f, rgl, c, nit, nch, kp, rg0, rows;
    u32x4 desc;  // buffer descriptor of the stage's weights (scalar registers)
};

// Buffer descriptor words (as __builtin_amdgcn_make_buffer_rsrc builds them):
// base, stride 0, num_records, raw-buffer flags.
__device__ __forceinline__ u32x4 make_desc(const void *base, size_t bytes) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const unsigned n = bytes > 0x7fffffffu ? 0x7fffffffu : (unsigned)bytes;
    return u32x4{(unsigned)b, (unsigned)(b >> 32) & 0xffffu, n, 0x00020000u};
}

// Weight items stream straight into LDS: buffer loads with the LDS-direct
// destination (M0 = row base in LDS, lane i writes bytes 16i..16i+15), RING
// slots per compute wave.  The compute waves' memory traffic is all inline
// assembly with explicit waits: the loads into the ring, the LDS reads of a
// slot and of the activation chunk (one block that first waits for the slot's
// loads, vmcnt(RING_WAIT), and ends with lgkmcnt(0), so every result register
// is valid when the block ends), the partial-sum writes and the barriers.
// The compiler therefore never holds in-flight data in registers (it could
// copy such a register before the data arrives) and inserts no waits of its
// own (it would wait for every outstanding load before any LDS access).  M0 is
// saved and restored around each load.
// A partial wait (vmcnt(N) > 0) relies on loads completing in issue order.  A
// load that is out of bounds for every lane can complete ahead of older loads
// on this hardware, so placeholder slots re-read offset 0 of a valid buffer
// instead, and no instruction in this kernel is issued entirely out of bounds
// where a partial wait could follow it.
__device__ __forceinline__ unsigned lds_addr(const void *p) { return (unsigned)(uintptr_t)p; }

__device__ __forceinline__ void ring_load(u32x4 desc, unsigned lds, unsigned off) {
    // descriptor and LDS address are wave-uniform (folds away when scalar)
    desc.x = __builtin_amdgcn_readfirstlane(desc.x);
    desc.y = __builtin_amdgcn_readfirstlane(desc.y);
    desc.z = __builtin_amdgcn_readfirstlane(desc.z);
    desc.w = __builtin_amdgcn_readfirstlane(desc.w);
    lds = __builtin_amdgcn_readfirstlane(lds);
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(off), "s"(desc)
        : "memory");
}

// Workgroup barrier for the compute waves (LDS writes complete first; no
// memory fence, which would also wait for the ring's loads).
__device__ __forceinline__ void cw_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ int cw_read_flag(unsigned addr) {
    int v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return __builtin_amdgcn_readfirstlane(v);
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
            q.rows = d.rows;
            q.desc = make_desc(d.W, (size_t)d.rows * d.kp);
            return;
        }
    }
    // exhausted: the ring keeps issuing placeholder loads, which must be real
    // in-bounds reads (see ring_load), so keep a valid descriptor -- also for a
    // wave that never had an item
    q.g = last + 1;
    q.desc = make_desc(a.w_lm, (size_t)a.V * a.kp_h);
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
// slot: LDS address of this lane's 16 bytes of row 0; xb: LDS address of the
// lane's first activation float4 in chunk c.
__device__ __forceinline__ void item_fma(unsigned slot, unsigned xb, unsigned part_row0, int lane) {
    u32x4 w0, w1, w2, w3;
    float4 x0, x1, x2, x3;
    asm volatile(
        RING_WAIT "\n\t"
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8 offset:1024\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\t"
        "ds_read_b128 %3, %8 offset:3072\n\t"
        "ds_read_b128 %4, %9\n\t"
        "ds_read_b128 %5, %9 offset:1024\n\t"
        "ds_read_b128 %6, %9 offset:2048\n\t"
        "ds_read_b128 %7, %9 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3), "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
        : "v"(slot), "v"(xb)
        : "memory");
    const float a0 = dot16(w0, x0, x1, x2, x3, 0.f);
    const float a1 = dot16(w1, x0, x1, x2, x3, 0.f);
    const float a2 = dot16(w2, x0, x1, x2, x3, 0.f);
    const float a3 = dot16(w3, x0, x1, x2, x3, 0.f);
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
    if ((lane & 15) == 0) asm volatile("ds_write_b32 %0, %1" ::"v"(part_row0 + ((lane >> 4) << 2)), "v"(k) : "memory");
}

// ------------------------------------------------------------ completion
typedef unsigned u32x8 __attribute__((ext_vector_type(8)));

struct Shared {
    int abort, pos, crow, tok, n_prompt, max_tokens;
    double red[NXW];      // staging pass-1 partial sums (sum of squares)
    double red2[2][NXW];  // sums of the staged inputs, by stage parity
};

// One bounded wait step: false (abort flag raised) after spin_limit steps, or
// when another workgroup has raised it.
__device__ __forceinline__ bool spin_step(const DecArgs &a, unsigned &it, int lane) {
    if (++it >= a.spin_limit) {
        if (lane == 0) cstorei(a.abort_flag, 1);
        return false;
    }
    if ((it & 15) == 0 && uni(cloadi(a.abort_flag))) return false;
    __builtin_amdgcn_s_sleep(1);
    return true;
}

__device__ __forceinline__ unsigned *stage_ctr(const DecArgs &a, int g) { return a.ctr + (size_t)g * NXCD; }
__device__ __forceinline__ unsigned *head_ctr(const DecArgs &a, int l, int hq) {
    return a.ctr + (size_t)(5 * a.L + 1) * NXCD + (size_t)l * a.n_heads + hq;
}

// Publish: wait until this wave's stores are complete, then count this
// workgroup in.  Everything exchanged between workgroups lives in uncached
// device memory (the host allocates it so), where a completed store is in
// memory: no L2 write-back is needed (a release fence here writes back the
// whole L2 of the XCD and costs tens of microseconds per stage).
__device__ __forceinline__ void publish(unsigned *c, int lane) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Scalar (glc) read of 8 consecutive counters: served outside the CU's vector
// memory queue, coherent across XCDs.
__device__ __forceinline__ u32x8 sload8(const unsigned *c) {
    u32x8 v;
    asm volatile("s_load_dwordx8 %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(c) : "memory");
    return v;
}
__device__ __forceinline__ unsigned sload1(const unsigned *c) {
    unsigned v;
    asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(c) : "memory");
    return v;
}

// Wait until every workgroup has published stage g of this launch.
__device__ __forceinline__ bool wait_stage(const DecArgs &a, int g, int lane) {
    const unsigned *c = stage_ctr(a, g);
    const unsigned nwg = gridDim.x, t = a.tag;
    unsigned it = 0;
    for (;;) {
        const u32x8 v = sload8(c);
        bool ok = true;
#pragma unroll
        for (int x = 0; x < NXCD; x++) ok = ok && (int)(v[x] - t * ((nwg - x + NXCD - 1) / NXCD)) >= 0;
        if (ok) return true;
        if (!spin_step(a, it, lane)) return false;
    }
}

// Wait until all ns splits of head hq (layer l) have published their partials.
__device__ __forceinline__ bool wait_head(const DecArgs &a, int l, int hq, int lane) {
    const unsigned *c = head_ctr(a, l, hq);
    const unsigned want = a.tag * (unsigned)a.ns;
    unsigned it = 0;
    for (;;) {
        if ((int)(sload1(c) - want) >= 0) return true;
        if (!spin_step(a, it, lane)) return false;
    }
}

// ------------------------------------------------------------ input staging
struct Src {
    const float *p;
    const float *nw;  // RMSNorm weight or nullptr
    int k;
    int prod;         // stage whose completion makes p valid (-1: model data)
};

// Input of GEMV stage s (s = 5L: LM head).
__device__ __forceinline__ Src stage_src(const DecArgs &a, int s, const Shared &sh) {
    const int last = 5 * a.L;
    Src r{nullptr, nullptr, a.h, -1};
    if (s >= last) {
        r.p = wsl(a, a.L - 1) + a.o_xd;
        r.nw = a.norm_final;
        r.prod = last - 1;
        return r;
    }
    const int l = s / 5, t = s % 5;
    if (t == ST_QKV) {
        if (l == 0) {
            r.p = a.embed + (size_t)uni(sh.tok) * a.h;
        } else {
            r.p = wsl(a, l - 1) + a.o_xd;
            r.prod = s - 1;
        }
        r.nw = lay(a, l)->norm_in;
    } else if (t == ST_O) {
        r.p = wsl(a, l) + a.o_xa;
        r.k = a.qd;
        r.prod = s - 1;
    } else if (t == ST_GU) {
        r.p = wsl(a, l) + a.o_xo;
        r.nw = lay(a, l)->norm_post;
        r.prod = s - 1;
    } else {
        r.p = wsl(a, l) + a.o_xg;
        r.k = a.ffn;
        r.prod = s - 1;
    }
    return r;
}

// Pass 1 (aux wave aw): element groups t = aw*64 + lane of every 1024-chunk,
// x[p*1024 + 4t .. +3], into the LDS layout, raw, once the producing stage is
// complete.  Partial sum of squares (normed input) to sh.red, or the partial
// sum to sh.red2.  RMSNorm weights of the group come back in w4 (normed inputs
// have k <= 4096).
__device__ __forceinline__ bool stage_pass1(const DecArgs &a, int s, float *xs, Shared &sh, int aw, int lane,
                                            float4 (&w4)[4]) {
    const Src src = stage_src(a, s, sh);
    const int nch = (src.k + 1023) >> 10;
    const int t = aw * 64 + lane;
    if (src.nw) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(src.nw, (size_t)src.k * 4);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            w4[p] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p < nch) w4[p] = bload16f(rw, (unsigned)(((p << 10) + 4 * t) * 4));
        }
    }
    bool ok = true;
    if (src.prod >= 0) ok = wait_stage(a, src.prod, lane);
    asm volatile("" ::: "memory");
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src.p, (size_t)src.k * 4);
    float4 v[MAXCH];
#pragma unroll
    for (int p = 0; p < MAXCH; p++) {
        v[p] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p < nch) v[p] = cload16f(r, (unsigned)(((p << 10) + 4 * t) * 4));
    }
    double acc = 0.0;
#pragma unroll
    for (int p = 0; p < MAXCH; p++) {
        if (p >= nch) continue;
        *(float4 *)(xs + xslot(p, t)) = v[p];
        if (src.nw)
            acc += (double)v[p].x * v[p].x + (double)v[p].y * v[p].y + (double)v[p].z * v[p].z +
                   (double)v[p].w * v[p].w;
        else
            acc += (double)v[p].x + (double)v[p].y + (double)v[p].z + (double)v[p].w;
    }
    acc = wave_sum_d(acc);
    if (lane == 0) {
        if (src.nw)
            sh.red[aw] = acc;
        else
            sh.red2[s & 1][aw] = acc;
    }
    return ok;
}

// Pass 2 (normed inputs, after every wave's pass 1): keep the raw row in xres
// (the next residual add reads it), RMSNorm the wave's groups in place;
// partial sum of the normed values to sh.red2.
__device__ __forceinline__ void stage_pass2(const DecArgs &a, int s, float *xs, float *xres, Shared &sh, int aw,
                                            int lane, const float4 (&w4)[4]) {
    const int k = a.h, nch = (k + 1023) >> 10, t = aw * 64 + lane;
    const double ss = sh.red[0] + sh.red[1] + sh.red[2] + sh.red[3];
    // cpu.rs:574-599: rstd = 1/sqrt(mean(x^2) + eps) in f64; out = f32(x*rstd*w)
    const double rstd = 1.0 / sqrt(ss / (double)k + (double)a.eps);
    double acc = 0.0;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        if (p >= nch) continue;
        float4 *px = (float4 *)(xs + xslot(p, t));
        const float4 v = *px;
        if ((p << 10) + 4 * t < k) *(float4 *)(xres + (p << 10) + 4 * t) = v;  // k % 4 == 0
        float4 o;
        o.x = (float)((double)v.x * rstd * (double)w4[p].x);
        o.y = (float)((double)v.y * rstd * (double)w4[p].y);
        o.z = (float)((double)v.z * rstd * (double)w4[p].z);
        o.w = (float)((double)v.w * rstd * (double)w4[p].w);
        *px = o;
        acc += (double)o.x + (double)o.y + (double)o.z + (double)o.w;
    }
    acc = wave_sum_d(acc);
    if (lane == 0) sh.red2[s & 1][aw] = acc;
}

__device__ __forceinline__ bool stage_normed(const DecArgs &a, int s) {
    if (s >= 5 * a.L) return true;
    const int t = s % 5;
    return t == ST_QKV || t == ST_GU;
}

// ------------------------------------------------------------ epilogues
// Row i of this workgroup's block: chunk partials in order, bias, scale.
__device__ __forceinline__ float row_val(const float *part, int i, int nch, float sc, float corr) {
    const int rgl = i >> 2, r = i & 3;
    float s = 0.f;
    for (int c = 0; c < nch; c++) s += part[(((rgl * nch) + c) << 2) + r];
    return sc * (s - corr);
}

// ordered argmax state: the whole range (v, i, nan) and the range after its
// last NaN (sv, si); generate.rs:167-173 picks the suffix maximum when a NaN
// is present (max_by hands the running best to the element after it)
struct LmAcc {
    float v;
    int i, nan;
    float sv;
    int si;
};

__device__ __forceinline__ void vi_pick(float &v, int &i, float v2, int i2) {  // (v, i) precedes (v2, i2)
    if (i2 < 0) return;
    if (i < 0 || !(v > v2)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ LmAcc lm_combine(LmAcc l, LmAcc r) {  // l precedes r
    LmAcc o = l;
    vi_pick(o.v, o.i, r.v, r.i);
    o.nan = max(l.nan, r.nan);
    if (r.nan >= 0) {
        o.sv = r.sv;
        o.si = r.si;
    } else {
        vi_pick(o.sv, o.si, r.v, r.i);
    }
    return o;
}

__device__ __forceinline__ void lm_take(LmAcc &p, float v, int row) {
    if (isnan(v)) {
        p.nan = row;
        p.si = -1;
        return;
    }
    vi_pick(p.v, p.i, v, row);
    vi_pick(p.sv, p.si, v, row);
}

__device__ __forceinline__ LmAcc lm_wave(LmAcc acc, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        LmAcc o;
        o.v = __shfl_down(acc.v, off);
        o.i = __shfl_down(acc.i, off);
        o.nan = __shfl_down(acc.nan, off);
        o.sv = __shfl_down(acc.sv, off);
        o.si = __shfl_down(acc.si, off);
        if ((lane & (2 * off - 1)) == 0) acc = lm_combine(acc, o);
    }
    acc.v = __shfl(acc.v, 0);
    acc.i = __shfl(acc.i, 0);
    acc.nan = __shfl(acc.nan, 0);
    acc.sv = __shfl(acc.sv, 0);
    acc.si = __shfl(acc.si, 0);
    return acc;
}

// Fused epilogue of GEMV stage g for this workgroup's rows (control wave),
// then publish.  xres holds the raw input of the last normed stage (x for o,
// the o output for down); s_cs the RoPE (cos, sin) of this workgroup's qkv
// pairs at the current position.
__device__ __forceinline__ void epilogue(const DecArgs &a, int g, const float *part, const float *xres,
                                         const float2 *s_cs, const Shared &sh, int lane) {
    const GDesc d = gdesc(a, g);
    int rg0, nrg;
    rg_range(d.rows, rg0, nrg);
    const int R0 = rg0 * 4;
    const int nr = max(0, min(d.rows, (rg0 + nrg) * 4) - R0);
    const double *r2 = sh.red2[g & 1];
    const float sx = (float)(r2[0] + r2[1] + r2[2] + r2[3]);
    const float corr = 128.f * sx;
    const int nch = d.nch;
    if (g >= 5 * a.L) {  // LM head: logits + this workgroup's ordered argmax partial
        LmAcc p{0.f, -1, -1, 0.f, -1};
        const int per = (nr + 63) >> 6;
        const int i0 = lane * per, i1 = min(nr, i0 + per);
        for (int i = i0; i < i1; i++) {
            const float v = row_val(part, i, nch, a.s_lm, corr);
            a.logits[R0 + i] = v;
            lm_take(p, v, R0 + i);
        }
        p = lm_wave(p, lane);
        if (lane < 5) {
            const unsigned w = lane == 0 ? __float_as_uint(p.v) : lane == 1 ? (unsigned)p.i : lane == 2 ? (unsigned)p.nan
                             : lane == 3 ? __float_as_uint(p.sv) : (unsigned)p.si;
            cstoreu(a.lm_part + (size_t)blockIdx.x * 8 + lane, w);
        }
        publish(stage_ctr(a, g) + (blockIdx.x & (NXCD - 1)), lane);
        return;
    }
    const int l = g / 5;
    const CLayers Ly = lay(a, l);
    float *W = wsl(a, l);
    switch (g % 5) {
        case ST_QKV: {
            const int crow = uni(sh.crow);
            float *kr = Ly->k_cache + (size_t)crow * a.kvd;
            float *vr = Ly->v_cache + (size_t)crow * a.kvd;
            for (int pidx = lane; pidx < (nr >> 1); pidx += 64) {
                const int j = R0 + 2 * pidx;
                const float x0 = row_val(part, 2 * pidx, nch, Ly->scale[0], corr);
                const float x1 = row_val(part, 2 * pidx + 1, nch, Ly->scale[0], corr);
                if (j < a.qd + a.kvd) {
                    const bool isq = j < a.qd;
                    const int jj = isq ? j : j - a.qd;
                    const float2 cs = s_cs[pidx];
                    // cpu.rs:655-658 in f32, no contraction
                    const float r0 = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
                    const float r1 = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
                    if (isq) {
                        cstoref(W + a.o_xq + jj, __fmul_rn(r0, a.q_scale));
                        cstoref(W + a.o_xq + jj + 1, __fmul_rn(r1, a.q_scale));
                    } else {
                        kr[jj] = r0;  // cache row: read by later launches
                        kr[jj + 1] = r1;
                        cstoref(W + a.o_xk + jj, r0);
                        cstoref(W + a.o_xk + jj + 1, r1);
                    }
                } else {
                    const int jj = j - a.qd - a.kvd;
                    vr[jj] = x0;
                    vr[jj + 1] = x1;
                    cstoref(W + a.o_xv + jj, x0);
                    cstoref(W + a.o_xv + jj + 1, x1);
                }
            }
            break;
        }
        case ST_O: {
            for (int i = lane; i < nr; i += 64) {
                const int j = R0 + i;
                cstoref(W + a.o_xo + j, xres[j] + row_val(part, i, nch, Ly->scale[1], corr));
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
            for (int i = lane; i < nr; i += 64) {
                const int j = R0 + i;
                cstoref(W + a.o_xd + j, xres[j] + row_val(part, i, nch, Ly->scale[4], corr));
            }
            break;
        }
        default: break;
    }
    publish(stage_ctr(a, g) + (blockIdx.x & (NXCD - 1)), lane);
}

// ------------------------------------------------------------ attention
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Unit (query head hq, split sp) by the aux waves (aw = 0..3) once the qkv
// stage is complete: positions [t0, t1) of layer l; cached rows come from the
// KV cache, the current row (position crow, in one split) from the copy the
// qkv stage published.  Per-lane-group online softmax state -> LDS slots.
template <int G>
__device__ __forceinline__ bool attn_part(const DecArgs &a, int l, int unit, int aw, int crow, float *s_ao,
                                          float *s_am, float *s_al, int lane) {
    constexpr int P = 64 / G;
    constexpr int PI = P * AU;
    const int sub = lane / G, gl = lane % G;
    const int ns = a.ns, hq = unit / ns, sp = unit - hq * ns;
    const int kh = hq / (a.n_heads / a.n_kv), hd = a.hd, kvd = a.kvd;
    const int Lc = crow + 1, chunk = (Lc + ns - 1) / ns;
    const int t0 = min(Lc, sp * chunk), t1 = min(Lc, t0 + chunk);
    const bool has_new = t0 <= crow && crow < t1;
    const int tc = has_new ? crow : t1;  // cached rows [t0, tc)
    const bool dact = gl * 4 < hd;
    const CLayers Ly = lay(a, l);
    const float *W = wsl(a, l);
    // cached rows do not depend on this launch: start them before the wait
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(Ly->k_cache, (size_t)tc * kvd * 4);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(Ly->v_cache, (size_t)tc * kvd * 4);
    const unsigned col = (unsigned)(kh * hd + gl * 4) * 4;
    const bool ok = wait_stage(a, 5 * l + ST_QKV, lane);
    asm volatile("" ::: "memory");
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(W, a.ws_stride * 4);
    const float4 qf = cload16f(rw, dact ? (unsigned)(a.o_xq + hq * hd + gl * 4) * 4 : OOB);
    float4 kn = make_float4(0.f, 0.f, 0.f, 0.f), vn = kn;
    if (has_new) {
        kn = cload16f(rw, dact ? (unsigned)(a.o_xk + kh * hd + gl * 4) * 4 : OOB);
        vn = cload16f(rw, dact ? (unsigned)(a.o_xv + kh * hd + gl * 4) * 4 : OOB);
    }
    float m = -INFINITY, ls = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int tb = t0 + aw * PI; tb < tc; tb += NXW * PI) {
        float4 kv[AU], vv[AU];
#pragma unroll
        for (int u = 0; u < AU; u++) {
            const int t = tb + u * P + sub;
            const unsigned offc = (t < tc && dact) ? (unsigned)t * kvd * 4 + col : OOB;
            kv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            vv[u] = kv[u];
            if (tb + u * P < tc) {  // some lane group in bounds
                kv[u] = bload16f(kr, offc);
                vv[u] = bload16f(vr, offc);
            }
        }
        float sc[AU];
        float mx = m;
#pragma unroll
        for (int u = 0; u < AU; u++) {
            float d = qf.x * kv[u].x + qf.y * kv[u].y + qf.z * kv[u].z + qf.w * kv[u].w;
            d = group_sum<G>(d);
            sc[u] = (tb + u * P + sub < tc) ? d : -INFINITY;
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
    if (has_new && aw == 0) {  // position crow, by lane group 0 of this wave
        const float d = group_sum<G>(qf.x * kn.x + qf.y * kn.y + qf.z * kn.z + qf.w * kn.w);
        if (sub == 0) {
            const float mx = fmaxf(m, d);
            const float f = expf(m - mx), p = expf(d - mx);
            ls = ls * f + p;
            o.x = o.x * f + p * vn.x;
            o.y = o.y * f + p * vn.y;
            o.z = o.z * f + p * vn.z;
            o.w = o.w * f + p * vn.w;
            m = mx;
        }
    }
    const int slot = aw * P + sub;
    if (gl == 0) {
        s_am[slot] = m;
        s_al[slot] = ls;
    }
    if (dact) *(float4 *)(s_ao + (size_t)slot * hd + gl * 4) = o;
    return ok;
}

// Control wave after the attention waves: merge the lane-group slots into the
// unit's partial (M, L, O) and publish it; the workgroup of the head's last
// split then merges the head's splits into the attention output row.  Every
// workgroup publishes the attention stage when its part is done.
__device__ __forceinline__ bool attn_publish(const DecArgs &a, int l, int unit, bool has_unit, int nslots,
                                             const float *s_ao, const float *s_am, const float *s_al, int lane) {
    unsigned *sc = stage_ctr(a, 5 * l + ST_ATTN) + (blockIdx.x & (NXCD - 1));
    if (!has_unit) {
        publish(sc, lane);
        return true;
    }
    const int ns = a.ns, hq = unit / ns, sp = unit - hq * ns, hd = a.hd;
    float *W = wsl(a, l);
    float M = -INFINITY;
    for (int q = 0; q < nslots; q++) M = fmaxf(M, s_am[q]);
    float lsum = 0.f;
    if (M != -INFINITY)
        for (int q = 0; q < nslots; q++)
            if (s_am[q] != -INFINITY) lsum += s_al[q] * expf(s_am[q] - M);
    for (int d = lane; d < hd; d += 64) {
        float osum = 0.f;
        if (M != -INFINITY)
            for (int q = 0; q < nslots; q++)
                if (s_am[q] != -INFINITY) osum += s_ao[(size_t)q * hd + d] * expf(s_am[q] - M);
        cstoref(W + a.o_apo + (size_t)hq * a.apo_hs + (size_t)sp * hd + d, osum);
    }
    if (lane == 0) {
        cstoref(W + a.o_apm + (size_t)hq * 64 + 2 * sp, M);
        cstoref(W + a.o_apm + (size_t)hq * 64 + 2 * sp + 1, lsum);
    }
    publish(head_ctr(a, l, hq), lane);
    if (sp != ns - 1) {
        publish(sc, lane);
        return true;
    }
    // x[hq*hd + d] = sum_s O_s[d] e^(M_s - M) / sum_s L_s e^(M_s - M)
    if (!wait_head(a, l, hq, lane)) return false;
    asm volatile("" ::: "memory");
    const float *apm = W + a.o_apm + (size_t)hq * 64;
    const float Ms = lane < ns ? cloadf(apm + 2 * lane) : -INFINITY;
    const float Ls = lane < ns ? cloadf(apm + 2 * lane + 1) : 0.f;
    float Mh = -INFINITY;
    for (int s = 0; s < ns; s++) Mh = fmaxf(Mh, __shfl(Ms, s));
    float Lt = 0.f;
    for (int s = 0; s < ns; s++) {
        const float ms = __shfl(Ms, s);
        if (ms != -INFINITY) Lt += __shfl(Ls, s) * expf(ms - Mh);
    }
    const float ws = Ms == -INFINITY ? 0.f : expf(Ms - Mh) / Lt;  // lane s: weight of split s
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(W, a.ws_stride * 4);
    for (int d0 = 4 * lane; d0 - 4 * lane < hd; d0 += 256) {
        float4 bo[MAXNS];
#pragma unroll
        for (int s = 0; s < MAXNS; s++) {
            bo[s] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (s < ns)
                bo[s] = cload16f(rw, d0 < hd ? (unsigned)(a.o_apo + (size_t)hq * a.apo_hs + (size_t)s * hd + d0) * 4 : OOB);
        }
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < MAXNS; s++) {
            const float w = __shfl(ws, s);
            if (s < ns) {
                v.x += w * bo[s].x;
                v.y += w * bo[s].y;
                v.z += w * bo[s].z;
                v.w += w * bo[s].w;
            }
        }
        if (d0 < hd) {
            float *xa = W + a.o_xa + hq * hd + d0;
            cstoref(xa, v.x);
            cstoref(xa + 1, v.y);
            cstoref(xa + 2, v.z);
            cstoref(xa + 3, v.w);
        }
    }
    publish(sc, lane);
    return true;
}

// Workgroup 0 after the LM head: ordered argmax over the workgroup partials,
// next token, position advance.
__device__ __forceinline__ bool finish(const DecArgs &a, const Shared &sh, int lane) {
    if (!wait_stage(a, 5 * a.L, lane)) return false;
    asm volatile("" ::: "memory");
    const int nwg = gridDim.x, V = a.V;
    const int per = (nwg + 63) >> 6;  // <= 4
    LmAcc acc{0.f, -1, -1, 0.f, -1};
    for (int q = 0; q < per; q++) {
        const int w = lane * per + q;
        if (w >= nwg) break;
        const unsigned *pp = a.lm_part + (size_t)w * 8;
        const LmAcc p{__uint_as_float(__hip_atomic_load((unsigned *)pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                      cloadi((const int *)pp + 1), cloadi((const int *)pp + 2),
                      __uint_as_float(__hip_atomic_load((unsigned *)pp + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                      cloadi((const int *)pp + 4)};
        acc = lm_combine(acc, p);
    }
    acc = lm_wave(acc, lane);
    int tok;
    if (acc.nan < 0)
        tok = acc.i < 0 ? 0 : acc.i;
    else if (acc.nan == V - 1)
        tok = acc.nan;
    else
        tok = acc.si;
    if (lane == 0) {
        const int p = sh.pos;
        if (a.argmax_out) a.argmax_out[0] = tok;
        if (a.advance) {
            if (p + 1 <= sh.max_tokens && p + 1 >= sh.n_prompt) a.tokens[p + 1] = tok;
            a.state->pos = p + 1;
            a.state->cache_len = sh.crow + 1;
        }
    }
    return true;
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
    float *xres = s_al + SLOTS_MAX;                              // [h] raw residual row
    float2 *s_cs = reinterpret_cast<float2 *>(xres + a.h);      // [qkv pairs of this workgroup]
    __shared__ Shared sh;

    const int lane = threadIdx.x & 63;
    const int wave = uni(threadIdx.x >> 6);
    const int last = 5 * a.L;

    // Barrier sequence, identical in every wave:
    //   B0 (launch state)  S1i  B2(0)  then per stage g: B1(g) [S1(g) B2(g+1)]
    // B2(g): the input of stage g is in LDS; B1(g): stage g's work is done;
    // S1(g): every aux wave has loaded its share of stage g+1's input.
    // The abort flag is checked after B0, every S1 and every B2.
    if (wave < NCW) {
        // ---------------- compute waves
        // The compiler lays the aux path out first and joins both paths here;
        // a wait it can see (vmcnt(0): nothing of this wave is in flight yet)
        // clears the aux path's pending loads from its wait-count model, which
        // would otherwise make it drain the weight ring inside the loop below.
        __builtin_amdgcn_s_waitcnt(0x0f70);
        const int w = wave;
        const unsigned lane16 = (unsigned)lane << 4;
        const unsigned ring = lds_addr(s_cs + a.qkv_pairs) + (unsigned)(w * RING * SLOT_BYTES);
        const unsigned xs_l = lds_addr(xs) + lane16, part_l = lds_addr(part), abort_l = lds_addr(&sh.abort);
        LCur lq;
        lcur_seek(lq, a, 0, w);
        int tg[RING], tf[RING], tc[RING];
        int cur = 0;    // stage being computed
        int ahead = 0;  // ring items of stages after cur
        // Slot tags: stage of the item, -1 stream end, -2 placeholder (the
        // load cursor waits at the lookahead limit)
#define SCRY_ISSUE(R)                                                                        \
    {                                                                                        \
        const bool v_ = lq.g <= last && (lq.g == cur || ahead < LOOKAHEAD);                  \
        const unsigned b_ = (unsigned)((lq.rg0 + lq.rgl) * 4 * lq.kp + (lq.c << 10)) + lane16; \
        _Pragma("unroll") for (int q_ = 0; q_ < 4; q_++) {                                   \
            /* rows past the tensor end and placeholders read offset 0 (never used) */      \
            const bool rv_ = v_ && (lq.rg0 + lq.rgl) * 4 + q_ < lq.rows;                     \
            ring_load(lq.desc, ring + (R) * SLOT_BYTES + (q_ << 10), rv_ ? b_ + (unsigned)(q_ * lq.kp) : 0u); \
        }                                                                                    \
        tg[R] = v_ ? lq.g : (lq.g <= last ? -2 : -1);                                        \
        tf[R] = lq.f;                                                                        \
        tc[R] = lq.c;                                                                        \
        if (v_) {                                                                            \
            if (lq.g != cur) ahead++;                                                        \
            lcur_next(lq, a, w);                                                             \
        }                                                                                    \
    }
        // one ring step on slot R (the oldest in flight)
#define SCRY_STEP(R)                                                                         \
    {                                                                                        \
        const int g = tg[R];                                                                 \
        if (g == -1) goto drain;                                                             \
        if (g >= 0) {                                                                        \
            if (g != cur) {                                                                  \
                /* cur < g <= last */                                                        \
                cw_barrier(); /* B1(cur) */                                                  \
                cw_barrier(); /* S1(cur) */                                                  \
                if (cw_read_flag(abort_l)) return;                                           \
                for (cur++; cur < g; cur++) {                                                \
                    cw_barrier(); /* B2(cur) */                                              \
                    if (cw_read_flag(abort_l)) return;                                       \
                    cw_barrier(); /* B1(cur) */                                              \
                    cw_barrier(); /* S1(cur) */                                              \
                    if (cw_read_flag(abort_l)) return;                                       \
                }                                                                            \
                cw_barrier(); /* B2(g) */                                                    \
                if (cw_read_flag(abort_l)) return;                                           \
                ahead = (tg[0] > cur) + (tg[1] > cur) + (tg[2] > cur) + (tg[3] > cur);       \
            }                                                                                \
            item_fma(ring + (R) * SLOT_BYTES + lane16, xs_l + ((unsigned)tc[R] << 12),       \
                     part_l + ((unsigned)tf[R] << 4), lane);                                 \
        }                                                                                    \
        SCRY_ISSUE(R)                                                                        \
    }
        SCRY_ISSUE(0)
        SCRY_ISSUE(1)
        SCRY_ISSUE(2)
        SCRY_ISSUE(3)
        cw_barrier();  // B0
        if (cw_read_flag(abort_l)) return;
        cw_barrier();  // S1i
        if (cw_read_flag(abort_l)) return;
        cw_barrier();  // B2(0)
        if (cw_read_flag(abort_l)) return;
        for (;;) {
            SCRY_STEP(0)
            SCRY_STEP(1)
            SCRY_STEP(2)
            SCRY_STEP(3)
        }
#undef SCRY_STEP
#undef SCRY_ISSUE
    drain:
        for (;;) {
            cw_barrier();  // B1(cur)
            if (cur == last) return;
            cw_barrier();  // S1(cur)
            if (cw_read_flag(abort_l)) return;
            cur++;
            cw_barrier();  // B2(cur)
            if (cw_read_flag(abort_l)) return;
        }
    }

    // ---------------- aux waves (wave NCW: control)
    const int aw = wave - NCW;
    const bool ctl = aw == 0;
    const int units = a.n_heads * a.ns;
    const int nslots = NXW * (64 / G);
    const bool has_unit = (int)blockIdx.x < units;
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
        // RoPE (cos, sin) of this workgroup's qkv row pairs at this position
        int rg0, nrg;
        rg_range(a.qkv_rows, rg0, nrg);
        const int npairs = max(0, min(a.qkv_rows, (rg0 + nrg) * 4) - rg0 * 4) >> 1;
        const int hh = a.hd >> 1;
        for (int pidx = lane; pidx < npairs; pidx += 64) {
            const int j = rg0 * 4 + 2 * pidx;
            const int jj = j < a.qd ? j : j - a.qd;
            s_cs[pidx] = j < a.qd + a.kvd ? a.rope_cs[(size_t)pos * hh + ((jj % a.hd) >> 1)] : make_float2(0.f, 0.f);
        }
    }
    __syncthreads();  // B0
    if (uni(sh.abort)) return;
    const int crow = uni(sh.crow);
    float4 w4[4];
    if (!stage_pass1(a, 0, xs, sh, aw, lane, w4) && lane == 0) sh.abort = 1;
    __syncthreads();  // S1i
    if (uni(sh.abort)) return;
    stage_pass2(a, 0, xs, xres, sh, aw, lane, w4);
    __syncthreads();  // B2(0)
    if (uni(sh.abort)) return;
    for (int g = 0; g <= last; g++) {
        const int t = g < last ? g % 5 : -1;
        const int l = g / 5;
        if (t == ST_ATTN && has_unit && !attn_part<G>(a, l, blockIdx.x, aw, crow, s_ao, s_am, s_al, lane) &&
            lane == 0)
            sh.abort = 1;
        __syncthreads();  // B1(g)
        if (g == last) {
            if (ctl) {
                epilogue(a, g, part, xres, s_cs, sh, lane);
                if (blockIdx.x == 0) finish(a, sh, lane);
            }
            return;
        }
        if (ctl) {
            if (t == ST_ATTN) {
                if (!attn_publish(a, l, blockIdx.x, has_unit, nslots, s_ao, s_am, s_al, lane) && lane == 0)
                    sh.abort = 1;
            } else {
                epilogue(a, g, part, xres, s_cs, sh, lane);
            }
        }
        const int s = g + 1;
        const bool gemv_next = s == last || s % 5 != ST_ATTN;
        if (gemv_next && !stage_pass1(a, s, xs, sh, aw, lane, w4) && lane == 0) sh.abort = 1;
        __syncthreads();  // S1(g)
        if (uni(sh.abort)) return;
        if (gemv_next && stage_normed(a, s)) stage_pass2(a, s, xs, xres, sh, aw, lane, w4);
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

size_t decode_lds_bytes(int nch_max, int part_cap, int h, int qkv_pairs) {
    return sizeof(float) * ((size_t)nch_max * 1024 + (size_t)part_cap * 4 + 1024 + 2 * SLOTS_MAX + h) +
           sizeof(float2) * (size_t)qkv_pairs + (size_t)NCW * RING * SLOT_BYTES;
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
