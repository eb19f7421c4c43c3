// Host restatement of LlamaModel::new's random init (llama.rs:593-680,
// init.rs:2-14) with fastrand 2.3.0's wyrand stream (not vendored in the
// reference; Cargo.lock pins 2.3.0).  wyrand's state is additive
// (call c sees state seed + (c+1)*0x2d358dccaa6c78a5), so sample j of a
// tensor can be computed independently and the init runs on all host cores
// with results identical to the sequential stream.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "internal.h"

namespace scry {
namespace {

constexpr uint64_t WY0 = 0x2d358dccaa6c78a5ULL;
constexpr uint64_t WY1 = 0x8bb84b93962eacc9ULL;

inline uint64_t wy_mix(uint64_t s) {
    unsigned __int128 t = (unsigned __int128)s * (unsigned __int128)(s ^ WY1);
    return (uint64_t)t ^ (uint64_t)(t >> 64);
}

// fastrand Rng::f64: 52 random mantissa bits in [1, 2), minus 1
inline double wy_f64(uint64_t u) {
    uint64_t bits = 0x3FF0000000000000ULL | (u >> 12);
    double d;
    std::memcpy(&d, &bits, sizeof d);
    return d - 1.0;
}

// init.rs:2-9 normal_sample (Box-Muller, f64, rounded once to f32)
inline float normal_at(uint64_t seed, uint64_t call, float mean, float stdv) {
    double u1 = wy_f64(wy_mix(seed + (call + 1) * WY0));
    double u2 = wy_f64(wy_mix(seed + (call + 2) * WY0));
    if (u1 < 1e-30) u1 = 1e-30;
    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2);
    return (float)((double)mean + (double)stdv * z);
}

}  // namespace

int host_threads() {
    unsigned n = std::thread::hardware_concurrency();
    if (n == 0) n = 1;
    if (n > 16) n = 16;  // the GPU box grants 16 host cores per GPU
    return (int)n;
}

void host_normal_vec(uint64_t seed, uint64_t start_call, size_t n, float mean, float stdv,
                     float *out, int threads) {
    if (threads <= 1 || n < (1u << 16)) {
        for (size_t i = 0; i < n; i++) out[i] = normal_at(seed, start_call + 2 * i, mean, stdv);
        return;
    }
    std::vector<std::thread> pool;
    const size_t per = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        const size_t b = t * per, e = std::min(n, b + per);
        if (b >= e) break;
        pool.emplace_back([=] {
            for (size_t i = b; i < e; i++) out[i] = normal_at(seed, start_call + 2 * i, mean, stdv);
        });
    }
    for (auto &th : pool) th.join();
}

}  // namespace scry
