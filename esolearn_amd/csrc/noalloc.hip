// sample_token without any device allocation, for callers that must not call
// hipMalloc (between replays of a captured graph, tight serving loops).  It
// waits for the stream and reads the token and the rng state back on the
// host, so it cannot itself be captured: call it outside stream capture.
//
// scry_hip_sample_token allocates its scratch on every call: the step state
// and token slots, the wyrand state, an f64 workspace of V entries and, for
// large vocabularies without top-k, the all-CU statistics block.  This variant
// keeps all of it in one file-scope device array, `scratch`, sized for the
// sampler's largest vocabulary (262144 entries: about 2 MiB, held by each GPU
// the library runs on until the process ends).  The host reaches the array
// only through its device address, looked up once per device with
// hipGetSymbolAddress at scry_hip_init; the array's name is never used on the
// host side.  Every call on a device shares that device's array and leaves
// the last call's contents in it: each call rewrites the state it reads and
// clears the statistics block, and calls that overlap on one GPU race (the
// library serialises its own calls, and each call waits for its result).
#include "internal.h"

namespace scry {
namespace {

constexpr int NA_MAX_V = 262144;  // the sampler's vocabulary limit
constexpr size_t NA_HDR = 64;     // DevState, two token slots, the wyrand state
constexpr size_t NA_PREP = 32 + sizeof(double) * (NA_MAX_V / 64);  // sample_prep_bytes(NA_MAX_V)
constexpr size_t NA_BYTES = NA_HDR + sizeof(double) * NA_MAX_V + NA_PREP;
constexpr int NA_MAX_DEVICES = 64;

char *g_scratch[NA_MAX_DEVICES];  // device address of `scratch` per device

}  // namespace

static __device__ __align__(256) unsigned char scratch[NA_BYTES];

// With the device current: record the device address of this device's copy
// of the scratch array (once per device).
int noalloc_setup(int device) {
    if (device < 0 || device >= NA_MAX_DEVICES)
        return set_error(SCRY_ERR_UNSUPPORTED, "device %d above the %d the static scratch tracks", device,
                         NA_MAX_DEVICES);
    if (g_scratch[device]) return SCRY_OK;
    void *p = nullptr;
    SCRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(SCRY_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch array");
    g_scratch[device] = static_cast<char *>(p);
    return SCRY_OK;
}

}  // namespace scry

using namespace scry;

extern "C" int scry_hip_sample_token_noalloc(scry_buf logits, const scry_sampling_config *cfg,
                                             uint64_t *rng_state, int64_t *out) {
    std::lock_guard<std::recursive_mutex> lock(api_mutex());
    if (!ctx().init) return set_error(SCRY_ERR_NOT_INIT, "scry_hip_init not called");
    if (!logits || !logits->d) return set_error(SCRY_ERR_INVALID, "sample_token_noalloc: null storage");
    if (!cfg || !rng_state || !out) return set_error(SCRY_ERR_INVALID, "sample_token_noalloc: null argument");
    if (cfg->temperature != cfg->temperature || cfg->top_p != cfg->top_p || cfg->top_k < 0)
        return set_error(SCRY_ERR_INVALID, "sample_token_noalloc: NaN temperature / top_p or negative top_k");
    const size_t V = logits->n;
    if (V == 0 || V > (size_t)NA_MAX_V)
        return set_error(SCRY_ERR_UNSUPPORTED, "sample_token_noalloc: vocabulary %zu outside 1..%d (the static scratch)",
                         V, NA_MAX_V);
    SCRY_TRY(noalloc_setup(ctx().device));
    char *blk = g_scratch[ctx().device];
    hipStream_t s = ctx().stream;
    DevState *st = (DevState *)blk;
    int64_t *toks = (int64_t *)(blk + 16);
    unsigned long long *rng = (unsigned long long *)(blk + 32);
    double *ws = (double *)(blk + NA_HDR);
    void *pw = blk + NA_HDR + sizeof(double) * NA_MAX_V;
    struct {
        DevState st;
        int64_t toks[2];
        uint64_t rng;
    } h{{0, 0, 1, 1}, {0, 0}, *rng_state};  // position 0 of a 1-token prompt: one draw
    static_assert(sizeof(DevState) == 16, "DevState layout");
    static_assert(sizeof(h) <= NA_HDR, "scratch header");
    if (cfg->temperature < 1e-8f) {  // generate.rs:96-98: argmax, no draw
        SCRY_TRY(launch_argmax(logits->d, (int64_t)V, toks + 1, s));
        SCRY_HIP(hipMemcpyAsync(&h.toks[1], toks + 1, sizeof(int64_t), hipMemcpyDeviceToHost, s));
        SCRY_HIP(hipStreamSynchronize(s));
        *out = h.toks[1];
        return SCRY_OK;
    }
    const bool prep = sample_uses_prep(*cfg, (int)V);
    if (prep && sample_prep_bytes((int)V) > NA_PREP)
        return set_error(SCRY_ERR_UNSUPPORTED, "sample_token_noalloc: statistics block above the static scratch");
    SCRY_HIP(hipMemcpyAsync(blk, &h, sizeof h, hipMemcpyHostToDevice, s));
    if (prep) SCRY_TRY(launch_fill_u32((unsigned *)pw, sample_prep_bytes((int)V) / 4, 0u, s));  // starts at zero
    SCRY_TRY(launch_sample(logits->d, (int)V, *cfg, ws, rng, st, toks, prep ? pw : nullptr, s));
    SCRY_HIP(hipMemcpyAsync(&h, blk, sizeof h, hipMemcpyDeviceToHost, s));
    SCRY_HIP(hipStreamSynchronize(s));
    *out = h.toks[1];
    *rng_state = h.rng;
    return SCRY_OK;
}
