// generate.rs:92-186 sample_token on the device, so a stochastic decode loop
// stays in the captured step graph (no logits download per token).
//
// One workgroup of 1024 threads after the LM head.  Every pass over the
// vocabulary is coalesced (thread t reads entries t, t + 1024, ...), so entry
// i lies in the 64-entry segment i / 64 that one wave covers in one step.
//
//  0. one pass: the NaN-ignoring maximum, the smallest finite key, the count
//     of finite logits, and whether a NaN or +inf is present (then the f64
//     softmax sum is NaN and the reference falls back to uniform 1/V).
//  1. top-k (0 < k < V): the k-th largest logit by a selection over the
//     order-preserving 32-bit key of the f32 logits: 11-bit digits of
//     (key - smallest key), at most three levels, histograms in LDS.
//     Dividing by a positive temperature keeps the order, so "scaled <
//     threshold" (generate.rs:108-118) is "key < the k-th key"; equal values
//     at the threshold stay, as in the reference.
//  2. softmax in f64 (generate.rs:120-131): e = exp(f64(x)/f64(T) - max).
//  3. top-p (generate.rs:134-160): probabilities follow the logit order, so
//     the cut of the descending order is the same selection with 2^62
//     fixed-point masses (integer sums: the same in every run).  Entry i is
//     kept when the mass before it in (value desc, index asc) order is below
//     top_p, or it comes first; equal values at the cut are kept in index order
//     (the reference's unstable sort leaves their order unspecified).  The
//     kept mass renormalises.
//  4. weighted_sample (generate.rs:175-186): r = Rng::f64() (fastrand,
//     wyrand, state on the device); the first index whose cumulative
//     probability exceeds r: sums per 64-entry segment, a scan over the
//     segments, then the one segment that crosses r.
// When at most 256 entries lie at or above the first selection level's bin
// holding the k-th key (or there are that few finite logits), they are
// gathered into LDS after that level and steps 1-4 finish there by pairwise
// counting.  Else, when at most 1024 entries survive top-k, they are gathered
// in index order into LDS and steps 2-4 run there, one entry per thread.
// The f64 sums run in a fixed order other than the reference's sequential
// one, so probabilities agree within f64 rounding; a draw can differ only if r
// or the top-p mass lies within that rounding of a boundary.
#include <climits>

#include "internal.h"
#include "kdev.h"

namespace scry {
namespace {

constexpr int SN = 1024;  // threads
constexpr int SW = SN / 64;
constexpr int NB = 2048;      // bins per selection level (11-bit digits)
constexpr int LCAP = SN;      // kept entries finished in LDS
constexpr int MAXSEG = 4096;  // 64-entry segments
constexpr int MAXV = MAXSEG * 64;
constexpr double FX = 4611686018427387904.0;  // 2^62

__device__ __forceinline__ unsigned okey(float x) {  // ascending with x
    const unsigned b = __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// fastrand 2.3.0 Rng (wyrand) and Rng::f64
__device__ __forceinline__ double wy_next_f64(unsigned long long *st) {
    const unsigned long long s = *st + 0x2d358dccaa6c78a5ull;
    *st = s;
    const unsigned long long b = s ^ 0x8bb84b93962eacc9ull;
    const unsigned long long u = (s * b) ^ __umul64hi(s, b);
    return __longlong_as_double((long long)(0x3FF0000000000000ull | (u >> 12))) - 1.0;
}

struct SampleArgs {
    const float *logits;
    int V;
    float temperature;
    int top_k;
    float top_p;
    double *ws;               // [V] exp values (large kept sets)
    unsigned long long *rng;  // fastrand state
    DevState *st;
    int64_t *tokens;
    // top-k off and V > LCAP: the statistics, exp values (ws) and 64-entry
    // segment sums come from the two vocabulary-wide kernels below
    unsigned *prep;  // [PREP_WORDS], cleared by k_sample for the next step
    double *segsum;  // [ceil(V / 64)]
};

// prep words: the largest finite key, ~(smallest finite key), finite count,
// NaN/+inf flag, ~(smallest key with e > 0) (atomic max of the complement:
// all start at 0)
enum { PR_MAXKEY = 0, PR_NKMIN = 1, PR_NFIN = 2, PR_BAD = 3, PR_NKMINP = 4, PREP_WORDS = 8 };

__device__ __forceinline__ float key_f32(unsigned key) {  // inverse of okey
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// the draw condition of k_sample (generate.rs:67-83), read before it advances
__device__ __forceinline__ bool draws(const DevState *st) {
    const int p = st->pos;
    return p + 1 >= st->n_prompt && p + 1 <= st->max_tokens;
}

// Vocabulary-wide statistics for k_sample, over all CUs.
__global__ __launch_bounds__(256) void k_prep_stats(const float *__restrict__ lg, int V, const DevState *st,
                                                    unsigned *prep) {
    if (!draws(st)) return;
    unsigned kmax = 0, kmin = ~0u, nfin = 0, bad = 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < V; i += gridDim.x * 256) {
        const float x = lg[i];
        bad |= !(x < INFINITY);
        if (x > -INFINITY && x < INFINITY) {
            const unsigned k = okey(x);
            kmax = max(kmax, k);
            kmin = min(kmin, k);
            nfin++;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        kmax = max(kmax, (unsigned)__shfl_xor((int)kmax, off));
        kmin = min(kmin, (unsigned)__shfl_xor((int)kmin, off));
        nfin += (unsigned)__shfl_xor((int)nfin, off);
        bad |= (unsigned)__shfl_xor((int)bad, off);
    }
    // one set of atomics per workgroup (they meet on four words in L2)
    __shared__ unsigned r[4][4];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        r[0][wave] = kmax;
        r[1][wave] = kmin;
        r[2][wave] = nfin;
        r[3][wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) {
            kmax = max(kmax, r[0][w]);
            kmin = min(kmin, r[1][w]);
            nfin += r[2][w];
            bad |= r[3][w];
        }
        atomicMax(prep + PR_MAXKEY, kmax);
        atomicMax(prep + PR_NKMIN, ~kmin);
        atomicAdd(prep + PR_NFIN, nfin);
        if (bad) atomicOr(prep + PR_BAD, 1u);
    }
}

// e = exp(f64(x)/f64(T) - max) for every entry (top-k off: every finite
// logit is kept; -inf gives 0) into ws, one wave per 64-entry segment with
// its sum, and the smallest key with e > 0.
__global__ __launch_bounds__(256) void k_prep_exp(const float *__restrict__ lg, int V, float temperature,
                                                  const DevState *st, unsigned *prep, double *__restrict__ ws,
                                                  double *__restrict__ segsum) {
    if (!draws(st)) return;
    if (prep[PR_BAD] || prep[PR_NFIN] == 0) return;  // k_sample takes the uniform path
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, s = blockIdx.x * 4 + wave;
    const int nseg = (V + 63) >> 6;
    const double T = (double)temperature;
    const double mxs = (double)key_f32(prep[PR_MAXKEY]) / T;
    const int i = s * 64 + lane;  // (segments past the end: x = -inf, nothing stored)
    const float x = i < V ? lg[i] : -INFINITY;
    const double e = x != -INFINITY ? exp((double)x / T - mxs) : 0.0;
    if (i < V) ws[i] = e;
    const double t = dev::wave_sum_d_dpp(e);
    unsigned km = e > 0.0 ? okey(x) : ~0u;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) km = min(km, (unsigned)__shfl_xor((int)km, off));
    __shared__ unsigned r[4];
    if (lane == 0) {
        if (s < nseg) segsum[s] = t;
        r[wave] = km;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        km = min(min(r[0], r[1]), min(r[2], r[3]));
        if (km != ~0u) atomicMax(prep + PR_NKMINP, ~km);  // one per workgroup
    }
}

struct Shared {
    unsigned hcnt[NB];
    union {
        unsigned long long hw[NB];
        struct {
            int idx[LCAP];
            unsigned key[LCAP];
            float x[LCAP];
        } L;  // gathered kept entries, index order
    } a;
    union {
        double segq[MAXSEG];
        unsigned segc[MAXSEG];
        unsigned long long w[LCAP];
    } b;
    double rd[SW];
    unsigned long long ru[SW];
    unsigned rk[SW], rn[SW], rb[SW];
    float rf[SW];
    int i0, i1, draw;
    unsigned u0;
    unsigned long long q0;
    double r;
};

template <class T>
__device__ __forceinline__ T wscan_incl(T v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const T o = __shfl_up(v, off);
        if (lane >= off) v += o;
    }
    return v;
}

// exclusive prefix over the block in thread order; *tot: the block total
// (the same value in every thread)
template <class T>
__device__ __forceinline__ T block_exscan(T v, T *red, T *tot) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const T inc = wscan_incl(v);
    T exc = __shfl_up(inc, 1);
    if (lane == 0) exc = T(0);
    if (lane == 63) red[wave] = inc;
    __syncthreads();
    T base = T(0), t = T(0);
    for (int w = 0; w < SW; w++) {
        if (w == wave) base = t;
        t += red[w];
    }
    __syncthreads();
    *tot = t;
    return base + exc;
}

__device__ __forceinline__ double block_sum(double v, double *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < SW; w++) t += red[w];
    __syncthreads();
    return t;
}

__device__ __forceinline__ unsigned block_min_u(unsigned v, unsigned *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = min(v, (unsigned)__shfl_xor((int)v, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned t = red[0];
    for (int w = 1; w < SW; w++) t = min(t, red[w]);
    __syncthreads();
    return t;
}

// Logits (and the f64 exp values) visited in passes: thread t takes entries
// t, t + SN, ... (step j covers entries j*SN .. j*SN + SN-1, 16 segments of
// 64).  Each pass loads B steps before using them, so B loads per thread are
// in flight (one workgroup cannot hide the latency otherwise).
constexpr int B = 16;

struct Src {
    const float *lg;
    const double *ws;
    int V, nj;  // nj = ceil(V / SN) steps
};

// f(i, x, e, ok) for every step, all lanes of a wave together (f may vote);
// ok = i < V; x = logits[i] (-inf past V); e = ws[i] when NE, else 0.
template <bool NE, class F>
__device__ __forceinline__ void each(const Src &s, F f) {
    const int tid = threadIdx.x;
    for (int j0 = 0; j0 < s.nj; j0 += B) {
        float xv[B];
        double ev[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int i = (j0 + u) * SN + tid;
            const bool ok = i < s.V;
            xv[u] = ok ? s.lg[i] : -INFINITY;
            ev[u] = (NE && ok) ? s.ws[i] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < B; u++)
            if (j0 + u < s.nj) {
                const int i = (j0 + u) * SN + tid;
                f(i, xv[u], ev[u], i < s.V);
            }
    }
}

// entry i read directly (one wave's segment)
template <bool NE>
__device__ __forceinline__ void load_one(const Src &s, int i, float &x, double &e) {
    const bool ok = i < s.V;
    x = ok ? s.lg[i] : -INFINITY;
    e = (NE && ok) ? s.ws[i] : 0.0;
}

struct Sel {
    bool small;              // stopped early: cnt_ge entries have key >= lo
    unsigned lo, cnt_ge;
    bool reached;            // the weights reach the target
    unsigned key;            // the key at the cut
    unsigned long long acc;  // weight of the keys above it
    unsigned nt;             // entries with that key
    unsigned long long wt;   // their weight
};

// The key K of the candidates where the weight summed from the largest key
// down reaches T: sum(w, key > K) < T <= sum(w, key >= K).  UNIT: every
// weight is 1 (counts, no exp values read).  cw(x, e, key, w) says whether
// the entry is a candidate.
// With stop > 0 (UNIT only) it returns after the first level when the entries
// at or above the chosen bin number at most stop.
template <bool UNIT, class CW>
__device__ __forceinline__ Sel select_top(const Src &src, unsigned kmin, unsigned kmax,
                          unsigned long long T, CW cw, Shared &S, unsigned stop = 0) {
    const int tid = threadIdx.x;
    const unsigned span = kmax - kmin;
    // digits at bits 22.., 11..21, 0..10: each level's NB bins cover exactly
    // the bin chosen one level up
    const int bits = span ? 32 - __clz((int)span) : 0;
    int shift = bits > 22 ? 22 : (bits > 11 ? 11 : 0);
    unsigned klo = kmin;
    unsigned long long acc = 0;
    Sel out{false, 0, 0, false, kmin, 0, 0, 0};
    for (;;) {  // at most three levels
        for (int b = tid; b < NB; b += SN) {
            S.hcnt[b] = 0;
            if (!UNIT) S.a.hw[b] = 0;
        }
        if (tid == 0) S.i0 = -1;
        __syncthreads();
        each<!UNIT>(src, [&](int, float x, double e, bool ok) {
            unsigned key;
            unsigned long long w;
            if (ok && cw(x, e, key, w) && key >= klo) {
                const unsigned d = (key - klo) >> shift;
                if (d < (unsigned)NB) {
                    atomicAdd(&S.hcnt[d], 1u);
                    if (!UNIT && w) atomicAdd(&S.a.hw[d], w);
                }
            }
        });
        __syncthreads();
        // descending order: thread t holds bins NB-1-2t and NB-2-2t
        const int b0 = NB - 1 - 2 * tid, b1 = b0 - 1;
        const unsigned long long v0 = UNIT ? S.hcnt[b0] : S.a.hw[b0];
        const unsigned long long v1 = UNIT ? S.hcnt[b1] : S.a.hw[b1];
        unsigned long long tot;
        const unsigned long long c0 = acc + block_exscan<unsigned long long>(v0 + v1, S.ru, &tot);
        const unsigned long long c1 = c0 + v0, c2 = c1 + v1;
        if (c0 < T && T <= c1) {
            S.i0 = b0;
            S.q0 = c0;
        } else if (c1 < T && T <= c2) {
            S.i0 = b1;
            S.q0 = c1;
        }
        __syncthreads();
        const int bs = S.i0;
        if (bs < 0) break;  // the total is below T
        acc = S.q0;
        if (UNIT && stop && acc + S.hcnt[bs] <= stop) {
            out.small = true;
            out.lo = klo + ((unsigned)bs << shift);
            out.cnt_ge = (unsigned)acc + S.hcnt[bs];
            break;
        }
        if (shift == 0) {
            out.reached = true;
            out.key = klo + (unsigned)bs;
            out.acc = acc;
            out.nt = S.hcnt[bs];
            out.wt = UNIT ? (unsigned long long)S.hcnt[bs] : S.a.hw[bs];
            break;
        }
        klo += (unsigned)bs << shift;
        shift -= 11;
        __syncthreads();  // the bins are read above before the next level clears them
    }
    __syncthreads();
    return out;
}

// per-segment counts of flagged entries into S.b.segc, then each replaced by
// the count before it (index order); returns the total
template <bool NE, class F>
__device__ __forceinline__ unsigned seg_count_exscan(const Src &src, F flag, Shared &S) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int nseg = (src.V + 63) >> 6;
    each<NE>(src, [&](int i, float x, double e, bool ok) {
        const unsigned long long m = __ballot(ok && flag(i, x, e));
        const int s = i >> 6;
        if (lane == 0 && s < nseg) S.b.segc[s] = (unsigned)__popcll(m);
    });
    __syncthreads();
    const int spt = (nseg + SN - 1) / SN, s0 = tid * spt;
    unsigned loc = 0;
    for (int u = 0; u < spt && s0 + u < nseg; u++) loc += S.b.segc[s0 + u];
    unsigned tot;
    unsigned cnt = block_exscan<unsigned>(loc, S.rn, &tot);
    for (int u = 0; u < spt && s0 + u < nseg; u++) {
        const unsigned c = S.b.segc[s0 + u];
        S.b.segc[s0 + u] = cnt;
        cnt += c;
    }
    __syncthreads();
    return tot;
}

// index of the m-th (1-based) flagged entry in index order (m <= the count)
template <bool NE, class F>
__device__ __forceinline__ int find_mth(const Src &src, F flag, unsigned m, Shared &S) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nseg = (src.V + 63) >> 6;
    if (tid == 0) S.i0 = -1;
    const unsigned tot = seg_count_exscan<NE>(src, flag, S);
    const int spt = (nseg + SN - 1) / SN, s0 = tid * spt;
    for (int u = 0; u < spt && s0 + u < nseg; u++) {
        const int s = s0 + u;
        const unsigned before = S.b.segc[s];
        const unsigned after = s + 1 < nseg ? S.b.segc[s + 1] : tot;
        if (before < m && m <= after) {
            S.i0 = s;
            S.u0 = m - before;
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int s = S.i0;
        int idx = src.V;
        if (s >= 0) {
            const int i = s * 64 + lane;
            float x;
            double e;
            load_one<NE>(src, i, x, e);
            unsigned long long mk = __ballot(i < src.V && flag(i, x, e));
            for (unsigned k = 1; k < S.u0; k++) mk &= mk - 1;
            idx = s * 64 + __ffsll((unsigned long long)mk) - 1;
        }
        if (lane == 0) S.i1 = idx;
    }
    __syncthreads();
    return S.i1;
}

// The walk of weighted_sample over per-segment sums already in S.b.segq
// (S.i0 = INT_MAX, synchronised): a scan over segments finds the first whose
// cumulative sum exceeds r, then one wave scans that segment's values val(i)
// (0 past V).  The segment sums may be summed in another order than that
// scan: when r lies within that rounding of the segment's end, its last entry
// with a value > 0.
template <class VAL>
__device__ __forceinline__ int draw_walk(int V, double r, VAL val, Shared &S) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nseg = (V + 63) >> 6;
    const int spt = (nseg + SN - 1) / SN, s0 = tid * spt;
    double loc = 0.0;
    for (int u = 0; u < spt && s0 + u < nseg; u++) loc += S.b.segq[s0 + u];
    double tot;
    double cum = block_exscan<double>(loc, S.rd, &tot);
    bool found = false;
    for (int u = 0; u < spt && s0 + u < nseg; u++) {
        const double prev = cum;
        cum = prev + S.b.segq[s0 + u];
        S.b.segq[s0 + u] = prev;  // now the sum before the segment
        if (!found && r < cum) {
            found = true;
            atomicMin(&S.i0, s0 + u);
        }
    }
    __syncthreads();
    const int sx = S.i0;
    if (sx == INT_MAX) return V - 1;  // r beyond the total (generate.rs:185)
    if (wave == 0) {
        const int i = sx * 64 + lane;
        const double q = i < V ? val(i) : 0.0;
        const double c = S.b.segq[sx] + wscan_incl(q);
        const unsigned long long mk = __ballot(r < c);
        const unsigned long long nz = __ballot(q > 0.0);
        if (lane == 0)
            S.i1 = mk ? sx * 64 + __ffsll((unsigned long long)mk) - 1
                      : (nz ? sx * 64 + 63 - __clzll((long long)nz) : V - 1);
    }
    __syncthreads();
    return S.i1;
}

// weighted_sample over prob(i, x, e): per-segment sums (one wave per
// segment), then the walk (prob must give the same value for an entry in
// every call)
template <bool NE, class P>
__device__ __forceinline__ int draw_segments(const Src &src, P prob, Shared &S) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int V = src.V, nseg = (V + 63) >> 6;
    each<NE>(src, [&](int i, float x, double e, bool ok) {
        const double tot = dev::wave_sum_d_dpp(ok ? prob(i, x, e) : 0.0);
        const int s = i >> 6;
        if (lane == 0 && s < nseg) S.b.segq[s] = tot;
    });
    if (tid == 0) S.i0 = INT_MAX;
    __syncthreads();
    return draw_walk(V, S.r, [&](int i) {
        float x;
        double e;
        load_one<NE>(src, i, x, e);
        return prob(i, x, e);
    }, S);
}

// At most LCAP kept entries (finite, key >= kk): gathered in index order,
// then softmax, top-p and the draw with one entry per thread.
__device__ __forceinline__ int finish_small(const SampleArgs &a, const Src &src, Shared &S, unsigned kk,
                            double mxs, bool topp, unsigned long long Tp) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int V = a.V;
    const double T = (double)a.temperature;
    auto kept = [&](int, float x, double) { return x != -INFINITY && okey(x) >= kk; };
    const int c = min((int)seg_count_exscan<false>(src, kept, S), LCAP);
    each<false>(src, [&](int i, float x, double, bool ok) {
        const bool f = ok && kept(i, x, 0.0);
        const unsigned long long m = __ballot(f);
        const int pos = f ? (int)S.b.segc[i >> 6] + __popcll(m & ((1ull << lane) - 1)) : LCAP;
        if (pos < LCAP) {  // pos < c <= LCAP (the selection's count)
            S.a.L.idx[pos] = i;
            S.a.L.key[pos] = okey(x);
            S.a.L.x[pos] = x;
        }
    });
    __syncthreads();
    const bool mine = tid < c;
    const unsigned kj = mine ? S.a.L.key[tid] : 0u;
    const double e = mine ? exp((double)S.a.L.x[tid] / T - mxs) : 0.0;
    const double sum = block_sum(e, S.rd);
    const double p = e / sum;
    double q = p;
    if (topp) {
        const unsigned long long w = mine ? (unsigned long long)(p * FX + 0.5) : 0ull;
        S.b.w[tid] = w;
        __syncthreads();
        bool keep = false;
        if (mine) {
            unsigned long long above = 0;
            unsigned gt = 0, rk = 0;
            for (int l = 0; l < c; l++) {
                const unsigned kl = S.a.L.key[l];
                if (kl > kj) {
                    above += S.b.w[l];
                    gt++;
                } else if (kl == kj && l < tid) {
                    rk++;
                }
            }
            keep = (gt == 0 && rk == 0) || above + (unsigned long long)rk * w < Tp;
        }
        const double sum2 = block_sum(keep ? p : 0.0, S.rd);
        q = keep ? (sum2 > 0.0 ? p / sum2 : p) : 0.0;
    }
    double tot;
    const double cum = block_exscan<double>(q, S.rd, &tot) + q;
    if (tid == 0) S.i0 = INT_MAX;
    __syncthreads();
    if (mine && S.r < cum) atomicMin(&S.i0, tid);
    __syncthreads();
    const int j = S.i0;
    return j == INT_MAX ? V - 1 : S.a.L.idx[j];
}

// At most GCAP entries have a finite key >= lo, and the kept set (the k
// largest with ties, k >= the count meaning all) is among them: they are
// gathered into LDS in any order, and every quantity that needs an order is
// counted pairwise: the top-k cut (fewer than k larger values), the rank among
// equal values (by index), the mass before an entry in (value desc, index asc)
// order, and the cumulative probability up to an index.
constexpr int GCAP = SN / 4;

__device__ __forceinline__ int finish_gather(const SampleArgs &a, const Src &src, Shared &S, unsigned lo,
                                             unsigned k, double mxs, bool topp, unsigned long long Tp) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int V = a.V;
    const double T = (double)a.temperature;
    if (tid == 0) S.i0 = 0;
    __syncthreads();
    each<false>(src, [&](int i, float x, double, bool ok) {
        const bool f = ok && x != -INFINITY && okey(x) >= lo;
        const unsigned long long m = __ballot(f);
        if (m) {
            const int first = __ffsll((unsigned long long)m) - 1;
            int base = 0;
            if (lane == first) base = atomicAdd(&S.i0, __popcll(m));
            base = __shfl(base, first);
            const int pos = base + __popcll(m & ((1ull << lane) - 1));
            if (f && pos < GCAP) {
                S.a.L.idx[pos] = i;
                S.a.L.key[pos] = okey(x);
                S.a.L.x[pos] = x;
            }
        }
    });
    __syncthreads();
    // four lanes per entry (GCAP * 4 == SN), each taking every fourth partner
    const int c = min(S.i0, GCAP);
    const int j = tid >> 2, part = tid & 3;
    const bool mine = j < c;
    const unsigned kj = mine ? S.a.L.key[j] : 0u;
    const int ij = mine ? S.a.L.idx[j] : INT_MAX;
    unsigned gt = 0, rk = 0;
    if (mine)
#pragma unroll 4
        for (int l = part; l < c; l += 4) {
            const unsigned kl = S.a.L.key[l];
            gt += kl > kj;
            rk += kl == kj && S.a.L.idx[l] < ij;
        }
    gt += (unsigned)__shfl_xor((int)gt, 1);
    gt += (unsigned)__shfl_xor((int)gt, 2);
    rk += (unsigned)__shfl_xor((int)rk, 1);
    rk += (unsigned)__shfl_xor((int)rk, 2);
    const bool kept = mine && gt < k;  // value >= the k-th largest value
    const double e = kept ? exp((double)S.a.L.x[j] / T - mxs) : 0.0;
    const double sum = block_sum(part == 0 ? e : 0.0, S.rd);
    const double p = e / sum;
    double q = p;
    if (topp) {
        const unsigned long long w = kept ? (unsigned long long)(p * FX + 0.5) : 0ull;
        if (part == 0) S.b.w[j] = w;
        __syncthreads();
        unsigned long long above = 0;
        if (kept)
#pragma unroll 4
            for (int l = part; l < c; l += 4)
                if (S.a.L.key[l] > kj) above += S.b.w[l];
        above += __shfl_xor(above, 1);
        above += __shfl_xor(above, 2);
        const bool keep = kept && ((gt == 0 && rk == 0) || above + (unsigned long long)rk * w < Tp);
        const double sum2 = block_sum(part == 0 && keep ? p : 0.0, S.rd);
        q = keep ? (sum2 > 0.0 ? p / sum2 : p) : 0.0;
    }
    if (part == 0) S.b.segq[j] = q;  // (w is no longer read: the block sum above synchronised)
    if (tid == 0) S.i1 = INT_MAX;
    __syncthreads();
    double cum = 0.0;
    if (mine)
#pragma unroll 4
        for (int l = part; l < c; l += 4)
            if (S.a.L.idx[l] <= ij) cum += S.b.segq[l];
    cum += __shfl_xor(cum, 1);
    cum += __shfl_xor(cum, 2);
    if (mine && part == 0 && S.r < cum) atomicMin(&S.i1, ij);
    __syncthreads();
    const int tok = S.i1;
    return tok == INT_MAX ? V - 1 : tok;
}

__device__ __forceinline__ int sample_body(const SampleArgs &a, Shared &S) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int V = a.V, nseg = (V + 63) >> 6;
    const float *lg = a.logits;
    const double T = (double)a.temperature;
    const Src src{lg, a.ws, V, (V + SN - 1) / SN};
    // ---- 0. max, smallest finite key, finite count, NaN / +inf
    float mx = -INFINITY;
    unsigned kmin = ~0u, nfin = 0, bad = 0;
    if (a.prep) {  // from k_prep_stats
        const unsigned km = a.prep[PR_MAXKEY];
        mx = km ? key_f32(km) : -INFINITY;
        kmin = ~a.prep[PR_NKMIN];
        nfin = a.prep[PR_NFIN];
        bad = a.prep[PR_BAD];
        if (tid == 0) S.r = wy_next_f64(a.rng);  // generate.rs:176
        __syncthreads();
    } else {
    float fmin = INFINITY;
    each<false>(src, [&](int, float x, double, bool ok) {
        // past V, x is -inf; NaN and +inf fail x < inf; fmaxf ignores NaN
        bad |= !(x < INFINITY);
        mx = fmaxf(mx, x);
        const bool fin = x > -INFINITY && x < INFINITY;
        fmin = fminf(fmin, fin ? x : INFINITY);
        nfin += fin;
    });
    // (fminf does not order -0 below +0: a zero minimum takes the key of -0,
    // which is at or below every finite key; kmin only starts key ranges)
    kmin = fmin < INFINITY ? okey(fmin == 0.0f ? -0.0f : fmin) : ~0u;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        kmin = min(kmin, (unsigned)__shfl_xor((int)kmin, off));
        nfin += (unsigned)__shfl_xor((int)nfin, off);
        bad |= (unsigned)__shfl_xor((int)bad, off);
    }
    if (lane == 0) {
        S.rf[wave] = mx;
        S.rk[wave] = kmin;
        S.rn[wave] = nfin;
        S.rb[wave] = bad;
    }
    if (tid == 0) S.r = wy_next_f64(a.rng);  // generate.rs:176
    __syncthreads();
    for (int w = 0; w < SW; w++) {
        mx = fmaxf(mx, S.rf[w]);
        kmin = min(kmin, S.rk[w]);
        bad |= S.rb[w];
    }
    nfin = 0;
    for (int w = 0; w < SW; w++) nfin += S.rn[w];
    __syncthreads();
    }
    const bool topp = a.top_p < 1.0f && a.top_p > 0.0f;
    const unsigned long long Tp = topp ? (unsigned long long)((double)a.top_p * FX + 0.5) : 0ull;
    if (bad || nfin == 0) {
        // the softmax sum is NaN (NaN, +inf, or every logit -inf): 1/V each
        const double uni = 1.0 / (double)V;
        int m = V;
        double sum2 = 1.0;
        if (topp) {
            if (tid == 0) {  // the first m indices, m from the sequential cumsum
                double cum = 0.0;
                int mm = V;
                for (int j = 0; j < V; j++) {
                    cum += uni;
                    if (cum >= (double)a.top_p) {
                        mm = j + 1;
                        break;
                    }
                }
                S.i1 = mm;
            }
            __syncthreads();
            m = S.i1;
            double part = 0.0;
            for (int i = tid; i < m; i += SN) part += uni;
            sum2 = block_sum(part, S.rd);
        }
        return draw_segments<false>(
            src,
            [&](int i, float, double) { return !topp ? uni : (i < m ? (sum2 > 0.0 ? uni / sum2 : uni) : 0.0); },
            S);
    }
    const double mxs = (double)mx / T;
    const unsigned kmax = okey(mx);
    // ---- 1. top-k: kept = finite with key >= kk
    unsigned kk = kmin, nkept = nfin;
    const int k = a.top_k;
    if (k > 0 && k < V && nfin > (unsigned)k) {
        const Sel s = select_top<true>(
            src, kmin, kmax, (unsigned long long)k,
            [&](float x, double, unsigned &key, unsigned long long &w) {
                key = okey(x);
                w = 1;
                return x != -INFINITY;
            },
            S, GCAP);
        if (s.small) return finish_gather(a, src, S, s.lo, (unsigned)k, mxs, topp, Tp);
        kk = s.key;
        nkept = (unsigned)(s.acc + s.nt);
    } else if (nfin <= (unsigned)GCAP) {
        return finish_gather(a, src, S, kmin, ~0u, mxs, topp, Tp);
    }
    if (nkept <= (unsigned)LCAP) return finish_small(a, src, S, kk, mxs, topp, Tp);
    // ---- 2. softmax over the kept entries
    double part = 0.0;
    unsigned kminp = ~0u;
    if (a.prep) {  // exp values and segment sums from k_prep_exp
        for (int sg = tid; sg < nseg; sg += SN) part += a.segsum[sg];
        kminp = ~a.prep[PR_NKMINP];
    } else {
        each<false>(src, [&](int i, float x, double, bool ok) {
            if (!ok) return;
            const unsigned key = okey(x);
            const double e = (x != -INFINITY && key >= kk) ? exp((double)x / T - mxs) : 0.0;
            a.ws[i] = e;
            part += e;
            if (e > 0.0) kminp = min(kminp, key);
        });
    }
    const double sum = block_sum(part, S.rd);
    if (!a.prep) kminp = block_min_u(kminp, S.rk);
    if (a.prep && !(a.top_p < 1.0f && a.top_p > 0.0f)) {
        // no top-p: r < sum(p up to i) is r * sum < sum(e up to i), up to rounding
        for (int sg = tid; sg < nseg; sg += SN) S.b.segq[sg] = a.segsum[sg];
        if (tid == 0) S.i0 = INT_MAX;
        __syncthreads();
        return draw_walk(V, S.r * sum, [&](int i) { return a.ws[i]; }, S);
    }
    // p = e * (1 / sum) in the vocabulary-wide passes (within an ulp of e / sum)
    const double isum = 1.0 / sum, wsc = FX / sum;
    // ---- 3. top-p: entries above the cut key kp, and ties up to index cut
    bool pfilter = false;
    unsigned kp = 0;
    int cut = V;
    if (topp) {
        unsigned m = 1, nt = 0;
        pfilter = true;
        if (Tp == 0) {  // top_p rounds to 0 in 2^-62 units: the first maximum only
            kp = kmax;
            nt = 2;  // forces the tie search below
        } else {
            const Sel s = select_top<false>(
                src, kminp, kmax, Tp,
                [&](float x, double e, unsigned &key, unsigned long long &w) {
                    key = okey(x);
                    w = (unsigned long long)(e * wsc + 0.5);
                    return e > 0.0;
                },
                S);
            if (!s.reached) {
                pfilter = false;  // the kept mass never reaches top_p: keep all
            } else {
                kp = s.key;
                nt = s.nt;
                // equal logits have equal masses: ceil((Tp - acc) / one), 1 .. nt
                const unsigned long long one = s.wt / nt;
                m = nt;
                if (s.acc >= Tp) {
                    m = 1;
                } else if (one > 0) {
                    const unsigned long long need = (Tp - s.acc + one - 1) / one;
                    m = (unsigned)(need < nt ? need : nt);
                }
            }
        }
        if (pfilter && m < nt)
            cut = find_mth<true>(
                src, [&](int, float x, double e) { return e > 0.0 && okey(x) == kp; }, m, S);
    }
    auto keptp = [&](int i, float x) {
        const unsigned key = okey(x);
        return !pfilter || key > kp || (key == kp && i <= cut);
    };
    double sum2 = 1.0;
    if (topp) {
        double p2 = 0.0;
        each<true>(src, [&](int i, float x, double e, bool ok) {
            if (ok && keptp(i, x)) p2 += e * isum;
        });
        sum2 = block_sum(p2, S.rd);
    }
    const double isum2 = sum2 > 0.0 ? 1.0 / sum2 : 1.0;
    // ---- 4. weighted_sample
    return draw_segments<true>(
        src,
        [&](int i, float x, double e) {
            const double p = e * isum;
            if (!topp) return p;
            return keptp(i, x) ? p * isum2 : 0.0;
        },
        S);
}

__global__ __launch_bounds__(SN) void k_sample(SampleArgs a) {
    __shared__ Shared S;
    const int tid = threadIdx.x;
    // generate.rs:67-83: a token is drawn after the last prompt position and
    // at every later step; the prompt positions consume no random numbers.
    // The state is read once, before any thread can advance it.
    if (tid == 0) {
        const int p = a.st->pos;
        S.i1 = p;
        S.draw = p + 1 >= a.st->n_prompt && p + 1 <= a.st->max_tokens;
    }
    __syncthreads();
    const int p = S.i1;
    const bool draw = S.draw != 0;
    __syncthreads();
    int tok = 0;
    if (draw) tok = sample_body(a, S);
    if (tid == 0) {
        if (draw) a.tokens[p + 1] = tok;
        a.st->pos = p + 1;
        a.st->cache_len = a.st->cache_len + 1;
        if (a.prep)  // (every thread read it before the body's barriers)
            for (int w = 0; w < PREP_WORDS; w++) a.prep[w] = 0u;
    }
}

}  // namespace

bool sample_uses_prep(const scry_sampling_config &sc, int V) {
    return (sc.top_k <= 0 || sc.top_k >= V) && V > LCAP;
}

size_t sample_prep_bytes(int V) { return sizeof(unsigned) * PREP_WORDS + sizeof(double) * ((V + 63) / 64); }

int launch_sample(const float *logits, int V, const scry_sampling_config &sc, double *ws,
                  unsigned long long *rng, DevState *st, int64_t *tokens, void *prep, hipStream_t s) {
    if (!logits || V <= 0 || !ws || !rng || !st || !tokens)
        return set_error(SCRY_ERR_INVALID, "sample: missing buffers");
    if (V > MAXV) return set_error(SCRY_ERR_UNSUPPORTED, "sample: vocabulary %d above %d", V, MAXV);
    if (!(sc.temperature >= 1e-8f)) return set_error(SCRY_ERR_INVALID, "sample: temperature < 1e-8 is greedy");
    const bool use = sample_uses_prep(sc, V);
    if (use && !prep) return set_error(SCRY_ERR_INVALID, "sample: missing the prep buffer");
    unsigned *pw = use ? (unsigned *)prep : nullptr;
    double *seg = use ? (double *)((unsigned *)prep + PREP_WORDS) : nullptr;
    SampleArgs a{logits, V, sc.temperature, sc.top_k, sc.top_p, ws, rng, st, tokens, pw, seg};
    if (use) {
        const int nseg = (V + 63) / 64;
        hipLaunchKernelGGL(k_prep_stats, dim3(std::min(64, (V + 1023) / 1024)), dim3(256), 0, s, logits, V,
                           (const DevState *)st, pw);
        hipLaunchKernelGGL(k_prep_exp, dim3((nseg + 3) / 4), dim3(256), 0, s, logits, V, sc.temperature,
                           (const DevState *)st, pw, ws, seg);
    }
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(SN), 0, s, a);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
