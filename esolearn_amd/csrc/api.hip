// Runtime (device, stream, errors) and the op-level C ABI: DeviceBackend
// storage and the MathBackend methods on the int8 Llama path.  The reference
// trait methods are static and panic on failure (backend/mod.rs:12-622); here
// every entry point returns a status code instead.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "internal.h"

namespace scry {

Ctx &ctx() {
    static Ctx c;
    return c;
}

std::recursive_mutex &api_mutex() {
    static std::recursive_mutex m;
    return m;
}

static thread_local std::string g_err;

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *expr, const char *file, int line) {
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? SCRY_ERR_OOM
                                                                                  : SCRY_ERR_HIP;
    (void)hipGetLastError();
    return set_error(code, "%s failed: %s (%s:%d)", expr, hipGetErrorString(e), file, line);
}

int dev_alloc(void **p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return set_error(SCRY_ERR_OOM, "hipMalloc(%zu bytes) failed: %s", bytes, hipGetErrorString(e));
    }
    return SCRY_OK;
}

int ctx_workspace(size_t bytes, void **p) {
    Ctx &c = ctx();
    if (c.ws_bytes < bytes) {
        SCRY_HIP(hipStreamSynchronize(c.stream));
        dev_free(c.ws);
        c.ws = nullptr;
        c.ws_bytes = 0;
        const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
        SCRY_TRY(dev_alloc(&c.ws, want));
        c.ws_bytes = want;
    }
    *p = c.ws;
    return SCRY_OK;
}

void dev_free(void *p) {
    if (p) (void)hipFree(p);
}

void packed_free(Packed &p) {
    dev_free(p.d);
    dev_free(p.s32);
    p = Packed{};
}

}  // namespace scry

using namespace scry;

#define API_LOCK std::lock_guard<std::recursive_mutex> _api_lock(scry::api_mutex())

namespace {

int new_buf(size_t n, scry_buf *out) {
    if (!out) return set_error(SCRY_ERR_INVALID, "null output handle");
    auto *b = new (std::nothrow) scry_buf_s;
    if (!b) return set_error(SCRY_ERR_OOM, "host allocation failed");
    int rc = dev_alloc((void **)&b->d, n * sizeof(float));
    if (rc) {
        delete b;
        return rc;
    }
    b->n = n;
    *out = b;
    return SCRY_OK;
}

void del_buf(scry_buf b) {
    if (!b) return;
    dev_free(b->d);
    dev_free(b->bf);
    dev_free(b->pk);
    delete b;
}

// the f32 data changed in place: drop the bf16 copies made from it
void bf16_stale(scry_buf b) {
    if (!b->d) return;
    dev_free(b->bf);
    dev_free(b->pk);
    b->bf = nullptr;
    b->pk = nullptr;
    b->pk_tb = -1;
}

int sync() {
    SCRY_HIP(hipStreamSynchronize(ctx().stream));
    return SCRY_OK;
}

#define CHECK_BUF(b, what)                                                                          \
    do {                                                                                            \
        if ((b) && !(b)->d && (b)->bf)                                                              \
            return set_error(SCRY_ERR_INVALID, "%s: the storage holds bf16 data only (bf16 mode)", what); \
        if (!(b) || !(b)->d) return set_error(SCRY_ERR_INVALID, "%s: null storage", what);          \
    } while (0)
// f32 or bf16-only storage
#define CHECK_ANY(b, what)                                                                          \
    do {                                                                                            \
        if (!(b) || (!(b)->d && !(b)->bf)) return set_error(SCRY_ERR_INVALID, "%s: null storage", what); \
    } while (0)

// bf16 rows [n][kp] of b as the B operand of a bf16-mode matmul (logical
// [k, n]; tb: stored [n][k]), built once per (k, n, tb)
int bf16_rows(scry_buf b, int k, int n, int tb, const unsigned short **rows, int *kp) {
    if (!(b->pk && b->pk_k == k && b->pk_n == n && b->pk_tb == tb)) {
        dev_free(b->pk);
        b->pk = nullptr;
        b->pk_tb = -1;
        const int p = bf16_row_pad(k);
        SCRY_TRY(dev_alloc((void **)&b->pk, sizeof(unsigned short) * (size_t)n * p));
        SCRY_TRY(launch_pack_rows_bf16(b->d ? nullptr : b->bf, b->d, k, n, tb, b->pk, p, ctx().stream));
        b->pk_k = k;
        b->pk_n = n;
        b->pk_kp = p;
        b->pk_tb = tb;
    }
    *rows = b->pk;
    *kp = b->pk_kp;
    return SCRY_OK;
}

// An f32 view of a (the f32 data, or its bf16 data widened into *tmp)
int f32_of(scry_buf a, float **tmp, const float **x) {
    if (a->d) {
        *x = a->d;
        return SCRY_OK;
    }
    SCRY_TRY(dev_alloc((void **)tmp, sizeof(float) * (a->n ? a->n : 1)));
    SCRY_TRY(launch_widen_bf16(a->bf, a->n, *tmp, ctx().stream));
    *x = *tmp;
    return SCRY_OK;
}

// bf16_ops::matmul_bf16 (cuda.rs:1226-1290): C = bf16(A) bf16(B), f32
// accumulation.  Untransposed A: the bf16 GEMV (1-16 rows) or the MFMA GEMM
// over B's bf16 rows; transposed A: the f32 kernel on bf16-rounded copies
// (the same exact products).
int matmul_bf16(scry_buf a, scry_buf b, int m, int k, int n, int ta, int tb, scry_buf *out) {
    hipStream_t s = ctx().stream;
    SCRY_TRY(new_buf((size_t)m * n, out));
    float *tmp = nullptr, *tb_f = nullptr;
    unsigned short *plane = nullptr;
    const float *x = nullptr;
    int rc = SCRY_OK;
    if (!ta) {
        const unsigned short *rows = nullptr;
        int kp = 0;
        rc = bf16_rows(b, k, n, tb, &rows, &kp);
        if (!rc) rc = f32_of(a, &tmp, &x);
        if (!rc && m <= GEMV_MAX_M) {
            rc = launch_gemv_bf16(rows, kp, n, x, k, k, m, (*out)->d, n, nullptr, s);
        } else if (!rc) {
            const int mp = prefill_rows_pad(m), lda = prefill_k_pad(k);
            rc = dev_alloc((void **)&plane, sizeof(unsigned short) * (size_t)mp * lda);
            if (!rc) rc = launch_fill_u32((unsigned *)plane, (size_t)mp * lda / 2, 0u, s);
            if (!rc) rc = launch_plane_bf16(x, k, m, k, lda, plane, lda, s);
            if (!rc) rc = launch_gemm_bf16(rows, kp, n, k, plane, lda, m, (*out)->d, n, nullptr, s);
        }
    } else {
        // both operands as the f32 values of their bf16 roundings
        float *ra = nullptr;
        rc = f32_of(a, &tmp, &x);
        if (!rc) rc = dev_alloc((void **)&ra, sizeof(float) * (size_t)m * k);
        if (!rc) rc = launch_round_bf16(x, (size_t)m * k, ra, s);
        const float *xb = nullptr;
        float *tmpb = nullptr;
        if (!rc) rc = f32_of(b, &tmpb, &xb);
        if (!rc) rc = dev_alloc((void **)&tb_f, sizeof(float) * (size_t)k * n);
        if (!rc) rc = launch_round_bf16(xb, (size_t)k * n, tb_f, s);
        if (!rc) rc = launch_matmul_f32(ra, tb_f, 1, m, k, n, ta, tb, (*out)->d, s);
        if (!rc) rc = sync();
        dev_free(ra);
        dev_free(tmpb);
    }
    if (!rc) rc = sync();  // temporaries are freed below
    dev_free(tmp);
    dev_free(tb_f);
    dev_free(plane);
    if (rc) {
        del_buf(*out);
        *out = nullptr;
    }
    return rc;
}

// Ensure the GEMV layout of an I8Storage for logical [k, n].
int ensure_packed(scry_i8buf q, int k, int n) {
    Packed &p = q->packed;
    if (p.d && p.k == k && p.n == n) return SCRY_OK;
    packed_free(p);
    p.k = k;
    p.n = n;
    p.kp = round_up(k, 16);
    p.rows = n;
    SCRY_TRY(dev_alloc((void **)&p.d, p.bytes()));
    return launch_i8_pack(q->d, k, n, 0, p.d, p.kp, 1, 1, 0, ctx().stream);
}

int check_mkn(size_t a_len, size_t b_len, int m, int k, int n) {
    if (m <= 0 || k <= 0 || n <= 0) return set_error(SCRY_ERR_INVALID, "matmul: m, k, n must be > 0");
    if (a_len != (size_t)m * k) return set_error(SCRY_ERR_INVALID, "matmul: A has %zu elements, m*k = %zu", a_len, (size_t)m * k);
    if (b_len != (size_t)k * n) return set_error(SCRY_ERR_INVALID, "matmul: B has %zu elements, k*n = %zu", b_len, (size_t)k * n);
    return SCRY_OK;
}

int qmatmul(scry_buf a, scry_i8buf bq, float scale, const float *scales32, const float *bias, int m,
            int k, int n, scry_buf *out) {
    CHECK_BUF(a, "matmul_i8_f32");
    if (!bq || !bq->d) return set_error(SCRY_ERR_INVALID, "matmul_i8_f32: null int8 storage");
    SCRY_TRY(check_mkn(a->n, bq->n, m, k, n));
    SCRY_TRY(ensure_packed(bq, k, n));
    scry_buf o = nullptr;
    SCRY_TRY(new_buf((size_t)m * n, &o));
    Packed w = bq->packed;
    w.scale = scale;
    w.s32 = const_cast<float *>(scales32);
    w.nb = (k + 31) / 32;
    int rc;
    if (skinny_route(m, k, n)) {
        void *ws = nullptr;
        rc = ctx_workspace(skinny_ws_bytes(m, k, n), &ws);
        SkinnyMM sm;
        sm.w = &w;
        sm.x = a->d;
        sm.ldx = k;
        sm.m = m;
        sm.bias = bias;
        sm.y = o->d;
        sm.ldy = n;
        if (!rc) rc = launch_skinny(sm, (float *)ws, ctx().ws_bytes, ctx().stream);
    } else if (m <= GEMV_MAX_M) {
        GemvArgs g;
        g.w = &w;
        g.x = a->d;
        g.ldx = k;
        g.m = m;
        g.y = o->d;
        g.ldy = n;
        g.bias = bias;
        rc = launch_qgemv(EPI_STORE, g, ctx().stream);
    } else if (gemm_takes_digits(w) && k <= 16384) {
        // prefill shapes, int8 per-tensor: the rows as digit planes (per-row
        // 24-bit fixed point), then the GEMM on the int8 matrix cores
        const int mp = prefill_rows_pad(m), ld = prefill_k_pad(k);
        const size_t dstride = (size_t)mp * ld;
        signed char *dg = nullptr;
        rc = dev_alloc((void **)&dg, 3 * dstride + sizeof(int) * (size_t)mp);
        int *de = reinterpret_cast<int *>(dg + 3 * dstride);
        if (!rc) rc = launch_fill_u32((unsigned *)dg, (3 * dstride) / 4 + mp, 0u, ctx().stream);
        if (!rc) rc = launch_norm_digits(a->d, k, m, nullptr, k, 0.f, dg, dstride, de, ld, ctx().stream);
        PrefillGemm g;
        g.w = &w;
        g.ad = dg;
        g.ae = de;
        g.dstride = dstride;
        g.lda = ld;
        g.M = m;
        g.c = o->d;
        g.ldc = n;
        g.bias = bias;
        if (!rc) rc = launch_gemm(PF_STORE, g, ctx().stream);
        if (!rc) rc = sync();  // the planes are freed below
        dev_free(dg);
    } else {
        // prefill shapes: the activations as bf16 planes, then the MFMA GEMM
        const int mp = prefill_rows_pad(m), ld = prefill_k_pad(k);
        unsigned short *pl = nullptr;
        rc = dev_alloc((void **)&pl, sizeof(unsigned short) * 2 * (size_t)mp * ld);
        if (!rc) rc = launch_fill_u32((unsigned *)pl, (size_t)mp * ld, 0u, ctx().stream);  // 2 planes of u16
        if (!rc) rc = launch_split(a->d, k, m, k, pl, pl + (size_t)mp * ld, ld, ctx().stream);
        PrefillGemm g;
        g.w = &w;
        g.ahi = pl;
        g.alo = pl + (size_t)mp * ld;
        g.lda = ld;
        g.M = m;
        g.c = o->d;
        g.ldc = n;
        g.bias = bias;
        if (!rc) rc = launch_gemm(PF_STORE, g, ctx().stream);
        if (!rc) rc = sync();  // the planes are freed below
        dev_free(pl);
    }
    if (rc) {
        del_buf(o);
        return rc;
    }
    *out = o;
    return SCRY_OK;
}

}  // namespace

extern "C" {

// ------------------------------------------------------------------ runtime
int scry_hip_init(int device) {
    API_LOCK;
    Ctx &c = ctx();
    if (c.init) {
        if (c.device == device) return SCRY_OK;
        return set_error(SCRY_ERR_INVALID, "already initialised on device %d", c.device);
    }
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        (void)hipGetLastError();
        return set_error(SCRY_ERR_NOT_INIT, "no HIP device available (%s)",
                         e == hipSuccess ? "count 0" : hipGetErrorString(e));
    }
    if (device < 0 || device >= n) return set_error(SCRY_ERR_INVALID, "device %d of %d", device, n);
    SCRY_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    SCRY_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(SCRY_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only",
                         device, prop.gcnArchName);
    // Decode attention hands its split partials over inside one XCD's L2: it
    // relies on the whole MI355X (8 XCDs of 32 CUs, one partition), whose
    // dispatcher gives workgroup b to XCD b % 8.  A partitioned device (fewer
    // CUs per agent) may map blocks to XCDs otherwise, which would read stale
    // partials instead of faulting, so it is refused.
    if (prop.multiProcessorCount != 256)
        return set_error(SCRY_ERR_UNSUPPORTED,
                         "device %d has %d CUs; the decode attention exchange needs the 256-CU, 8-XCD "
                         "MI355X in one partition",
                         device, prop.multiProcessorCount);
    SCRY_TRY(noalloc_setup(device));  // the device address of the static sampler scratch
    SCRY_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    c.bf16 = false;
    c.device = device;
    c.cu_count = prop.multiProcessorCount;
    c.name = prop.name;
    c.arch = prop.gcnArchName;
    c.init = true;
    return SCRY_OK;
}

int scry_hip_shutdown(void) {
    API_LOCK;
    Ctx &c = ctx();
    if (!c.init) return SCRY_OK;
    (void)hipStreamSynchronize(c.stream);
    dev_free(c.ws);
    (void)hipStreamDestroy(c.stream);
    c = Ctx{};
    return SCRY_OK;
}

const char *scry_hip_last_error(void) { return g_err.c_str(); }

int scry_hip_synchronize(void) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return sync();
}

int scry_hip_device_count(int *count) {
    if (!count) return set_error(SCRY_ERR_INVALID, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        n = 0;
    }
    *count = n;
    return SCRY_OK;
}

int scry_hip_device_info(char *name, size_t name_len, int *cu_count, char *arch, size_t arch_len) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    Ctx &c = ctx();
    if (name && name_len) std::snprintf(name, name_len, "%s", c.name.c_str());
    if (arch && arch_len) std::snprintf(arch, arch_len, "%s", c.arch.c_str());
    if (cu_count) *cu_count = c.cu_count;
    return SCRY_OK;
}

// ------------------------------------------------------------ f32 storage
int scry_hip_zeros(size_t n, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    SCRY_TRY(new_buf(n, out));
    return launch_fill_f32((*out)->d, n, 0.f, ctx().stream);
}

int scry_hip_from_vec(const float *host, size_t n, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!host && n) return set_error(SCRY_ERR_INVALID, "from_vec: null host pointer");
    SCRY_TRY(new_buf(n, out));
    if (n) {
        SCRY_HIP(hipMemcpyAsync((*out)->d, host, n * sizeof(float), hipMemcpyHostToDevice, ctx().stream));
        SCRY_TRY(sync());
    }
    return SCRY_OK;
}

int scry_hip_to_vec(scry_buf b, float *host, size_t n) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_ANY(b, "to_vec");
    if (n != b->n) return set_error(SCRY_ERR_INVALID, "to_vec: storage has %zu elements, asked %zu", b->n, n);
    if (!n) return SCRY_OK;
    if (!b->d) {  // cuda.rs:244-254: bf16-only storage widens to f32
        float *t = nullptr;
        SCRY_TRY(dev_alloc((void **)&t, n * sizeof(float)));
        int rc = launch_widen_bf16(b->bf, n, t, ctx().stream);
        hipError_t e = hipSuccess;
        if (!rc) e = hipMemcpyAsync(host, t, n * sizeof(float), hipMemcpyDeviceToHost, ctx().stream);
        if (!rc && e != hipSuccess) rc = hip_fail(e, "to_vec copy", __FILE__, __LINE__);
        if (!rc) rc = sync();
        dev_free(t);
        return rc;
    }
    SCRY_HIP(hipMemcpyAsync(host, b->d, n * sizeof(float), hipMemcpyDeviceToHost, ctx().stream));
    return sync();
}

int scry_hip_init_bf16(int device) {
    API_LOCK;
    SCRY_TRY(scry_hip_init(device));
    ctx().bf16 = true;
    return SCRY_OK;
}

int scry_hip_set_bf16_mode(int on) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    ctx().bf16 = on != 0;
    return SCRY_OK;
}

int scry_hip_bf16_mode(int *on) {
    if (!on) return set_error(SCRY_ERR_INVALID, "bf16_mode: null argument");
    *on = ctx().bf16 ? 1 : 0;
    return SCRY_OK;
}

int scry_hip_from_vec_with_bf16(const float *host, const uint16_t *bf16, size_t n, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!ctx().bf16) return scry_hip_from_vec(host, n, out);  // mod.rs:28-32 default
    if (!out || (!bf16 && n)) return set_error(SCRY_ERR_INVALID, "from_vec_with_bf16: null argument");
    auto *b = new (std::nothrow) scry_buf_s;
    if (!b) return set_error(SCRY_ERR_OOM, "host allocation failed");
    b->n = n;
    int rc = dev_alloc((void **)&b->bf, sizeof(uint16_t) * (n ? n : 1));
    if (!rc && n) {
        hipError_t e = hipMemcpyAsync(b->bf, bf16, sizeof(uint16_t) * n, hipMemcpyHostToDevice, ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "from_vec_with_bf16 upload", __FILE__, __LINE__);
        if (!rc) rc = sync();
    }
    if (rc) {
        del_buf(b);
        return rc;
    }
    *out = b;
    return SCRY_OK;
}

int scry_hip_clone_storage(scry_buf src, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_ANY(src, "clone_storage");
    if (!src->d) {  // bf16 only
        if (!out) return set_error(SCRY_ERR_INVALID, "null output handle");
        auto *b = new (std::nothrow) scry_buf_s;
        if (!b) return set_error(SCRY_ERR_OOM, "host allocation failed");
        b->n = src->n;
        int rc = dev_alloc((void **)&b->bf, sizeof(uint16_t) * (src->n ? src->n : 1));
        if (!rc && src->n) {
            hipError_t e = hipMemcpyAsync(b->bf, src->bf, sizeof(uint16_t) * src->n, hipMemcpyDeviceToDevice,
                                          ctx().stream);
            if (e != hipSuccess) rc = hip_fail(e, "clone_storage", __FILE__, __LINE__);
        }
        if (rc) {
            del_buf(b);
            return rc;
        }
        *out = b;
        return SCRY_OK;
    }
    SCRY_TRY(new_buf(src->n, out));
    if (src->n)
        SCRY_HIP(hipMemcpyAsync((*out)->d, src->d, src->n * sizeof(float), hipMemcpyDeviceToDevice,
                                ctx().stream));
    return SCRY_OK;
}

int scry_hip_buf_len(scry_buf b, size_t *n) {
    if (!b || !n) return set_error(SCRY_ERR_INVALID, "buf_len: null argument");
    *n = b->n;
    return SCRY_OK;
}

int scry_hip_free(scry_buf b) {
    API_LOCK;
    if (b && ctx().init) (void)hipStreamSynchronize(ctx().stream);
    del_buf(b);
    return SCRY_OK;
}

// ----------------------------------------------------------- int8 storage
int scry_hip_i8_from_vec(const int8_t *host, size_t n, scry_i8buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!out || (!host && n)) return set_error(SCRY_ERR_INVALID, "i8_from_vec: null argument");
    auto *q = new (std::nothrow) scry_i8buf_s;
    if (!q) return set_error(SCRY_ERR_OOM, "host allocation failed");
    int rc = dev_alloc((void **)&q->d, n);
    if (rc) {
        delete q;
        return rc;
    }
    q->n = n;
    if (n) {
        hipError_t e = hipMemcpyAsync(q->d, host, n, hipMemcpyHostToDevice, ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) {
            dev_free(q->d);
            delete q;
            return hip_fail(e, "i8_from_vec copy", __FILE__, __LINE__);
        }
    }
    *out = q;
    return SCRY_OK;
}

int scry_hip_i8_to_vec(scry_i8buf b, int8_t *host, size_t n) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!b || !b->d) return set_error(SCRY_ERR_INVALID, "i8_to_vec: null storage");
    if (n != b->n) return set_error(SCRY_ERR_INVALID, "i8_to_vec: storage has %zu elements, asked %zu", b->n, n);
    if (n) SCRY_HIP(hipMemcpyAsync(host, b->d, n, hipMemcpyDeviceToHost, ctx().stream));
    return sync();
}

int scry_hip_i8_len(scry_i8buf b, size_t *n) {
    if (!b || !n) return set_error(SCRY_ERR_INVALID, "i8_len: null argument");
    *n = b->n;
    return SCRY_OK;
}

int scry_hip_i8_free(scry_i8buf b) {
    API_LOCK;
    if (!b) return SCRY_OK;
    if (ctx().init) (void)hipStreamSynchronize(ctx().stream);
    packed_free(b->packed);
    dev_free(b->d);
    delete b;
    return SCRY_OK;
}

// --------------------------------------------------------------- quantize
int scry_hip_quantize_symmetric(scry_buf w, scry_i8buf *q_out, float *scale_out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(w, "quantize_symmetric");
    if (!q_out || !scale_out) return set_error(SCRY_ERR_INVALID, "quantize_symmetric: null output");
    auto *q = new (std::nothrow) scry_i8buf_s;
    if (!q) return set_error(SCRY_ERR_OOM, "host allocation failed");
    unsigned int *bits = nullptr;
    float *dscale = nullptr;
    int rc = dev_alloc((void **)&q->d, w->n);
    if (!rc) rc = dev_alloc((void **)&bits, 16);
    if (!rc) rc = dev_alloc((void **)&dscale, 16);
    if (!rc) rc = launch_absmax(w->d, w->n, bits, ctx().stream);
    if (!rc) rc = launch_quantize_plain(w->d, w->n, bits, q->d, dscale, ctx().stream);
    float s = 0.f;
    if (!rc && w->n) {
        hipError_t e = hipMemcpyAsync(&s, dscale, sizeof(float), hipMemcpyDeviceToHost, ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "quantize scale readback", __FILE__, __LINE__);
    }
    dev_free(bits);
    dev_free(dscale);
    if (rc) {
        dev_free(q->d);
        delete q;
        return rc;
    }
    q->n = w->n;
    *q_out = q;
    *scale_out = s;
    return SCRY_OK;
}

int scry_hip_dequantize(scry_i8buf q, float scale, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!q || !q->d) return set_error(SCRY_ERR_INVALID, "dequantize: null storage");
    SCRY_TRY(new_buf(q->n, out));
    return launch_dequantize(q->d, q->n, scale, (*out)->d, ctx().stream);
}

int scry_hip_quantize_block32(scry_buf w, int k, int n, scry_i8buf *q_out, scry_buf *scales_out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(w, "quantize_block32");
    if (k <= 0 || n <= 0 || w->n != (size_t)k * n)
        return set_error(SCRY_ERR_INVALID, "quantize_block32: storage has %zu elements, k*n = %zu", w->n,
                         (size_t)k * n);
    auto *q = new (std::nothrow) scry_i8buf_s;
    if (!q) return set_error(SCRY_ERR_OOM, "host allocation failed");
    scry_buf sc = nullptr;
    int rc = dev_alloc((void **)&q->d, w->n);
    if (!rc) rc = new_buf((size_t)n * ((k + 31) / 32), &sc);
    if (!rc) rc = launch_quant_block32(w->d, k, n, 0, q->d, sc->d, ctx().stream);
    if (rc) {
        dev_free(q->d);
        delete q;
        del_buf(sc);
        return rc;
    }
    q->n = w->n;
    *q_out = q;
    *scales_out = sc;
    return SCRY_OK;
}

// ------------------------------------------------------------- int8 matmul
int scry_hip_matmul_i8_f32(scry_buf a, scry_i8buf b_q, float scale, int m, int k, int n,
                           scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return qmatmul(a, b_q, scale, nullptr, nullptr, m, k, n, out);
}

int scry_hip_matmul_i8_f32_bias(scry_buf a, scry_i8buf b_q, float scale, scry_buf bias, int m,
                                int k, int n, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(bias, "matmul_i8_f32_bias");
    if (bias->n < (size_t)n) return set_error(SCRY_ERR_INVALID, "matmul_i8_f32_bias: bias shorter than n");
    return qmatmul(a, b_q, scale, nullptr, bias->d, m, k, n, out);
}

int scry_hip_matmul_i8_f32_block32(scry_buf a, scry_i8buf b_q, scry_buf scales, int m, int k,
                                   int n, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(scales, "matmul_i8_f32_block32");
    if (scales->n != (size_t)n * ((k + 31) / 32))
        return set_error(SCRY_ERR_INVALID, "matmul_i8_f32_block32: need n*ceil(k/32) scales");
    return qmatmul(a, b_q, 0.f, scales->d, nullptr, m, k, n, out);
}

// --------------------------------------------------------------- f32 glue
int scry_hip_matmul(scry_buf a, scry_buf b, int m, int k, int n, int trans_a, int trans_b,
                    scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (ctx().bf16) {  // cuda.rs:274-277
        CHECK_ANY(a, "matmul");
        CHECK_ANY(b, "matmul");
        SCRY_TRY(check_mkn(a->n, b->n, m, k, n));
        return matmul_bf16(a, b, m, k, n, trans_a, trans_b, out);
    }
    CHECK_BUF(a, "matmul");
    CHECK_BUF(b, "matmul");
    SCRY_TRY(check_mkn(a->n, b->n, m, k, n));
    SCRY_TRY(new_buf((size_t)m * n, out));
    return launch_matmul_f32(a->d, b->d, 1, m, k, n, trans_a, trans_b, (*out)->d, ctx().stream);
}

// MathBackend::matmul_bias (mod.rs:62-86; the CUDA backend keeps the default):
// the matmul above (bf16 operands in bf16 mode), then the f32 bias row added
// to every output row on the device.  A bf16-only bias is widened first, as
// the default's to_vec does.
int scry_hip_matmul_bias(scry_buf a, scry_buf b, scry_buf bias, int m, int k, int n, int trans_a,
                         int trans_b, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_ANY(bias, "matmul_bias");
    if (n > 0 && bias->n < (size_t)n)
        return set_error(SCRY_ERR_INVALID, "matmul_bias: bias holds %zu values, needs %d",
                         bias->n, n);
    SCRY_TRY(scry_hip_matmul(a, b, m, k, n, trans_a, trans_b, out));
    float *tmp = nullptr;
    const float *bv = nullptr;
    int rc = f32_of(bias, &tmp, &bv);
    if (!rc) rc = launch_add_bias_rows((*out)->d, bv, m, n, ctx().stream);
    if (tmp && !rc) rc = sync();  // the widened copy is freed below
    dev_free(tmp);
    if (rc) {
        del_buf(*out);
        *out = nullptr;
    }
    return rc;
}

int scry_hip_matmul_strided_batched(scry_buf a, scry_buf b, int batch, int m, int k, int n,
                                    int trans_a, int trans_b, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(a, "matmul_strided_batched");
    CHECK_BUF(b, "matmul_strided_batched");
    if (batch <= 0 || m <= 0 || k <= 0 || n <= 0)
        return set_error(SCRY_ERR_INVALID, "matmul_strided_batched: sizes must be > 0");
    if (a->n < (size_t)batch * m * k || b->n < (size_t)batch * k * n)
        return set_error(SCRY_ERR_INVALID, "matmul_strided_batched: operand too short");
    SCRY_TRY(new_buf((size_t)batch * m * n, out));
    return launch_matmul_f32(a->d, b->d, batch, m, k, n, trans_a, trans_b, (*out)->d, ctx().stream);
}

int scry_hip_rmsnorm(scry_buf x, scry_buf w, int rows, int d, float eps, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "rmsnorm");
    CHECK_BUF(w, "rmsnorm");
    if (rows <= 0 || d <= 0 || x->n != (size_t)rows * d || w->n < (size_t)d)
        return set_error(SCRY_ERR_INVALID, "rmsnorm: shape mismatch");
    SCRY_TRY(new_buf(x->n, out));
    return launch_rmsnorm(x->d, w->d, rows, d, eps, (*out)->d, ctx().stream);
}

static int rope_common(scry_buf x, int seq, int n_heads, int head_dim, int start_pos, scry_buf freqs,
                       int scaled, float scale, scry_buf *out) {
    CHECK_BUF(x, "rope");
    CHECK_BUF(freqs, "rope");
    if (seq <= 0 || n_heads <= 0 || head_dim <= 0 || head_dim % 2 ||
        x->n != (size_t)seq * n_heads * head_dim || freqs->n != (size_t)head_dim / 2)
        return set_error(SCRY_ERR_INVALID, "rope: shape mismatch");
    SCRY_TRY(new_buf(x->n, out));
    return launch_rope(x->d, seq, n_heads, head_dim, start_pos, freqs->d, scaled, scale, (*out)->d,
                       ctx().stream);
}

int scry_hip_rope_with_freqs_preloaded(scry_buf x, int seq, int n_heads, int head_dim,
                                       int start_pos, scry_buf freqs, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return rope_common(x, seq, n_heads, head_dim, start_pos, freqs, 0, 1.f, out);
}

int scry_hip_rope_with_freqs_scaled_preloaded(scry_buf x, int seq, int n_heads, int head_dim,
                                              int start_pos, scry_buf freqs, float scale,
                                              scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return rope_common(x, seq, n_heads, head_dim, start_pos, freqs, 1, scale, out);
}

int scry_hip_scale(scry_buf x, float s, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "scale");
    SCRY_TRY(new_buf(x->n, out));
    return launch_scale(x->d, x->n, s, (*out)->d, ctx().stream);
}

int scry_hip_softmax(scry_buf x, int rows, int cols, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "softmax");
    if (rows <= 0 || cols <= 0 || x->n != (size_t)rows * cols)
        return set_error(SCRY_ERR_INVALID, "softmax: shape mismatch");
    SCRY_TRY(new_buf(x->n, out));
    return launch_softmax(x->d, rows, cols, (*out)->d, ctx().stream);
}

int scry_hip_swiglu(scry_buf gate, scry_buf up, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(gate, "swiglu");
    CHECK_BUF(up, "swiglu");
    if (gate->n != up->n) return set_error(SCRY_ERR_INVALID, "swiglu: length mismatch");
    SCRY_TRY(new_buf(gate->n, out));
    return launch_swiglu(gate->d, up->d, gate->n, (*out)->d, ctx().stream);
}

int scry_hip_add(scry_buf a, scry_buf b, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(a, "add");
    CHECK_BUF(b, "add");
    if (a->n != b->n) return set_error(SCRY_ERR_INVALID, "add: length mismatch (same-shape add only)");
    SCRY_TRY(new_buf(a->n, out));
    return launch_add(a->d, b->d, a->n, (*out)->d, ctx().stream);
}

int scry_hip_embedding(scry_buf weight, const int64_t *ids, int n_ids, int vocab, int dim,
                       scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_ANY(weight, "embedding");
    if (n_ids < 0 || vocab <= 0 || dim <= 0 || weight->n != (size_t)vocab * dim || (n_ids && !ids))
        return set_error(SCRY_ERR_INVALID, "embedding: shape mismatch");
    for (int i = 0; i < n_ids; i++)
        if (ids[i] < 0 || ids[i] >= vocab)
            return set_error(SCRY_ERR_RANGE, "embedding index out of range: %lld >= vocab %d",
                             (long long)ids[i], vocab);
    int64_t *d_ids = nullptr;
    SCRY_TRY(dev_alloc((void **)&d_ids, sizeof(int64_t) * (size_t)(n_ids ? n_ids : 1)));
    int rc = new_buf((size_t)n_ids * dim, out);
    if (!rc && n_ids) {
        hipError_t e = hipMemcpyAsync(d_ids, ids, sizeof(int64_t) * n_ids, hipMemcpyHostToDevice,
                                      ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "embedding ids upload", __FILE__, __LINE__);
        if (!rc)
            rc = weight->d ? launch_embedding(weight->d, d_ids, n_ids, dim, (*out)->d, ctx().stream)
                           : launch_embed_bf16((*out)->d, weight->bf, d_ids, n_ids, dim, ctx().stream);  // cuda.rs:480-503
        if (!rc) rc = sync();
    }
    dev_free(d_ids);
    return rc;
}

int scry_hip_gather_reshape_repeat_kv(scry_buf cache, int max_seq, int cached_len, int n_kv,
                                      int n_q, int head_dim, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(cache, "gather_reshape_repeat_kv");
    if (n_kv <= 0 || n_q % n_kv || cached_len < 0 || cached_len > max_seq ||
        cache->n < (size_t)max_seq * n_kv * head_dim)
        return set_error(SCRY_ERR_INVALID, "gather_reshape_repeat_kv: shape mismatch");
    SCRY_TRY(new_buf((size_t)n_q * cached_len * head_dim, out));
    return launch_gather_repeat_kv(cache->d, cached_len, n_kv, n_q, head_dim, (*out)->d, ctx().stream);
}

int scry_hip_repeat_kv(scry_buf x, int n_kv, int n_q, int seq, int d_head, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "repeat_kv");
    if (n_kv <= 0 || n_q % n_kv || x->n != (size_t)n_kv * seq * d_head)
        return set_error(SCRY_ERR_INVALID, "repeat_kv: shape mismatch");
    SCRY_TRY(new_buf((size_t)n_q * seq * d_head, out));
    return launch_repeat_kv(x->d, n_kv, n_q, seq, d_head, (*out)->d, ctx().stream);
}

int scry_hip_scatter_rows(scry_buf dst, scry_buf src, int total_rows, int cols, int row_start,
                          int row_count) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(dst, "scatter_rows");
    CHECK_BUF(src, "scatter_rows");
    if (row_start < 0 || row_count < 0 || row_start + row_count > total_rows ||
        dst->n < (size_t)total_rows * cols || src->n < (size_t)row_count * cols)
        return set_error(SCRY_ERR_RANGE, "scatter_rows: rows [%d, %d) outside %d", row_start,
                         row_start + row_count, total_rows);
    if (row_count && cols)
        SCRY_HIP(hipMemcpyAsync(dst->d + (size_t)row_start * cols, src->d,
                                sizeof(float) * (size_t)row_count * cols, hipMemcpyDeviceToDevice,
                                ctx().stream));
    bf16_stale(dst);  // (the reference's bf16 shadow would keep the old rows)
    return SCRY_OK;
}

int scry_hip_argmax(scry_buf logits, int64_t *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(logits, "argmax");
    if (!out) return set_error(SCRY_ERR_INVALID, "argmax: null output");
    int64_t *d = nullptr;
    SCRY_TRY(dev_alloc((void **)&d, sizeof(int64_t)));
    int rc = launch_argmax(logits->d, (int64_t)logits->n, d, ctx().stream);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(out, d, sizeof(int64_t), hipMemcpyDeviceToHost, ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "argmax readback", __FILE__, __LINE__);
    }
    dev_free(d);
    return rc;
}

int scry_hip_normal_vec(uint64_t *rng_state, size_t n, float mean, float stdv, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!rng_state || !out) return set_error(SCRY_ERR_INVALID, "normal_vec: null argument");
    // init.rs:3-14: two Rng::f64 per sample (Box-Muller), glibc libm on the
    // host as the reference; the wyrand state is additive, so sample i of a
    // draw from state s uses the calls 2i+1 and 2i+2 after s
    std::vector<float> h(n);
    host_normal_vec(*rng_state, 0, n, mean, stdv, h.data(), host_threads());
    SCRY_TRY(new_buf(n, out));
    if (n) {
        hipError_t e = hipMemcpyAsync((*out)->d, h.data(), sizeof(float) * n, hipMemcpyHostToDevice, ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) {
            del_buf(*out);
            *out = nullptr;
            return hip_fail(e, "normal_vec upload", __FILE__, __LINE__);
        }
    }
    *rng_state += 2ull * n * 0x2d358dccaa6c78a5ull;
    return SCRY_OK;
}

int scry_hip_sample_token(scry_buf logits, const scry_sampling_config *cfg, uint64_t *rng_state, int64_t *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(logits, "sample_token");
    if (!cfg || !rng_state || !out) return set_error(SCRY_ERR_INVALID, "sample_token: null argument");
    if (cfg->temperature != cfg->temperature || cfg->top_p != cfg->top_p || cfg->top_k < 0)
        return set_error(SCRY_ERR_INVALID, "sample_token: NaN temperature / top_p or negative top_k");
    if (logits->n > 0x7fffffff) return set_error(SCRY_ERR_UNSUPPORTED, "sample_token: vocabulary too large");
    if (cfg->temperature < 1e-8f) return scry_hip_argmax(logits, out);  // generate.rs:96-98
    hipStream_t s = ctx().stream;
    // one block: DevState, tokens[2], the rng state, f64 scratch [n]
    const size_t V = logits->n;
    const bool prep = sample_uses_prep(*cfg, (int)V);
    const size_t pb = prep ? sample_prep_bytes((int)V) : 0;
    char *blk = nullptr;
    SCRY_TRY(dev_alloc((void **)&blk, 64 + sizeof(double) * V + pb));
    DevState *st = (DevState *)blk;
    int64_t *toks = (int64_t *)(blk + 16);
    unsigned long long *rng = (unsigned long long *)(blk + 32);
    double *ws = (double *)(blk + 64);
    void *pw = prep ? (void *)(blk + 64 + sizeof(double) * V) : nullptr;
    struct {
        DevState st;
        int64_t toks[2];
        uint64_t rng;
    } h{{0, 0, 1, 1}, {0, 0}, *rng_state};  // position 0 of a 1-token prompt: one draw
    static_assert(sizeof(DevState) == 16, "DevState layout");
    hipError_t e = hipMemcpyAsync(blk, &h, sizeof h, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? SCRY_OK : hip_fail(e, "sample_token upload", __FILE__, __LINE__);
    if (!rc && prep) rc = launch_fill_u32((unsigned *)pw, pb / 4, 0u, s);
    if (!rc) rc = launch_sample(logits->d, (int)V, *cfg, ws, rng, st, toks, pw, s);
    if (!rc) {
        e = hipMemcpyAsync(&h, blk, sizeof h, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "sample_token readback", __FILE__, __LINE__);
    }
    dev_free(blk);
    if (rc) return rc;
    *out = h.toks[1];
    *rng_state = h.rng;
    return SCRY_OK;
}

// ------------------------------------------- the rest of the trait surface
int scry_hip_ones(size_t n, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    SCRY_TRY(new_buf(n, out));
    return launch_fill_f32((*out)->d, n, 1.f, ctx().stream);
}

int scry_hip_add_broadcast(scry_buf a, const size_t *a_dims, int a_ndim, scry_buf b, const size_t *b_dims,
                           int b_ndim, const size_t *out_dims, int out_ndim, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(a, "add");
    CHECK_BUF(b, "add");
    if (a_ndim < 1 || b_ndim < 1 || out_ndim < 1 || a_ndim > 6 || b_ndim > 6 || out_ndim > 6 || !a_dims ||
        !b_dims || !out_dims)
        return set_error(SCRY_ERR_INVALID, "add: 1 to 6 dimensions per shape (Shape MAX_DIMS)");
    // Shape::broadcast (tensor/shape.rs): the output shape must be the broadcast of a and b
    const int nd = a_ndim > b_ndim ? a_ndim : b_ndim;
    if (out_ndim != nd) return set_error(SCRY_ERR_INVALID, "add: output shape is not the broadcast shape");
    size_t na = 1, nb = 1;
    for (int i = 0; i < a_ndim; i++) na *= a_dims[i];
    for (int i = 0; i < b_ndim; i++) nb *= b_dims[i];
    for (int i = 0; i < nd; i++) {
        const size_t da = i < a_ndim ? a_dims[a_ndim - 1 - i] : 1, db = i < b_ndim ? b_dims[b_ndim - 1 - i] : 1;
        const size_t want = da == db ? da : (da == 1 ? db : (db == 1 ? da : (size_t)-1));
        if (want == (size_t)-1) return set_error(SCRY_ERR_INVALID, "add: broadcast failed (incompatible shapes)");
        if (out_dims[nd - 1 - i] != want)
            return set_error(SCRY_ERR_INVALID, "add: output shape is not the broadcast shape");
    }
    if (a->n < na || b->n < nb) return set_error(SCRY_ERR_INVALID, "add: storage shorter than its shape");
    size_t no = 1;
    for (int i = 0; i < nd; i++) no *= out_dims[i];
    SCRY_TRY(new_buf(no, out));
    return launch_add_bcast(a->d, a_dims, a_ndim, b->d, b_dims, b_ndim, out_dims, out_ndim, (*out)->d,
                            ctx().stream);
}

int scry_hip_add_inplace(scry_buf dst, scry_buf src) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(dst, "add_inplace");
    CHECK_BUF(src, "add_inplace");
    SCRY_TRY(launch_add_inplace(dst->d, src->d, dst->n < src->n ? dst->n : src->n, ctx().stream));  // zip
    bf16_stale(dst);
    return SCRY_OK;
}

int scry_hip_scaled_softmax(scry_buf x, float scale, int rows, int cols, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "scaled_softmax");
    if (rows <= 0 || cols <= 0 || x->n != (size_t)rows * cols)
        return set_error(SCRY_ERR_INVALID, "scaled_softmax: shape mismatch");
    SCRY_TRY(new_buf(x->n, out));
    return launch_scaled_softmax(x->d, rows, cols, scale, (*out)->d, ctx().stream);
}

static int layernorm_common(scry_buf x, scry_buf gamma, scry_buf beta, int rows, int d, float eps, scry_buf *out,
                            scry_buf *mean, scry_buf *rstd) {
    CHECK_BUF(x, "layernorm");
    CHECK_BUF(gamma, "layernorm");
    CHECK_BUF(beta, "layernorm");
    if (rows <= 0 || d <= 0 || x->n != (size_t)rows * d || gamma->n < (size_t)d || beta->n < (size_t)d)
        return set_error(SCRY_ERR_INVALID, "layernorm: shape mismatch");
    scry_buf o = nullptr, mu = nullptr, rs = nullptr;
    int rc = new_buf(x->n, &o);
    if (!rc && mean) rc = new_buf((size_t)rows, &mu);
    if (!rc && mean) rc = new_buf((size_t)rows, &rs);
    if (!rc)
        rc = launch_layernorm(x->d, gamma->d, beta->d, rows, d, eps, o->d, mu ? mu->d : nullptr,
                              rs ? rs->d : nullptr, ctx().stream);
    if (rc) {
        del_buf(o);
        del_buf(mu);
        del_buf(rs);
        return rc;
    }
    *out = o;
    if (mean) {
        *mean = mu;
        *rstd = rs;
    }
    return SCRY_OK;
}

int scry_hip_layernorm(scry_buf x, scry_buf gamma, scry_buf beta, int rows, int d, float eps, scry_buf *out,
                       scry_buf *mean, scry_buf *rstd) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!out || !mean || !rstd) return set_error(SCRY_ERR_INVALID, "layernorm: null output handle");
    return layernorm_common(x, gamma, beta, rows, d, eps, out, mean, rstd);
}

int scry_hip_layernorm_inference(scry_buf x, scry_buf gamma, scry_buf beta, int rows, int d, float eps,
                                 scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    if (!out) return set_error(SCRY_ERR_INVALID, "layernorm_inference: null output handle");
    return layernorm_common(x, gamma, beta, rows, d, eps, out, nullptr, nullptr);
}

int scry_hip_gelu(scry_buf x, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "gelu");
    SCRY_TRY(new_buf(x->n, out));
    return launch_gelu(x->d, x->n, (*out)->d, ctx().stream);
}

int scry_hip_sum(scry_buf x, float *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "sum");
    if (!out) return set_error(SCRY_ERR_INVALID, "sum: null output");
    char *blk = nullptr;
    SCRY_TRY(dev_alloc((void **)&blk, 16 + sizeof(double) * (size_t)sum_partials(x->n)));
    float *d_out = (float *)blk;
    int rc = launch_sum(x->d, x->n, (double *)(blk + 16), d_out, ctx().stream);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(out, d_out, sizeof(float), hipMemcpyDeviceToHost, ctx().stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) rc = hip_fail(e, "sum readback", __FILE__, __LINE__);
    }
    dev_free(blk);
    return rc;
}

int scry_hip_mul_elementwise(scry_buf a, scry_buf b, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(a, "mul_elementwise");
    CHECK_BUF(b, "mul_elementwise");
    const size_t n = a->n < b->n ? a->n : b->n;  // zip
    SCRY_TRY(new_buf(n, out));
    return launch_mul(a->d, b->d, n, (*out)->d, ctx().stream);
}

int scry_hip_concat_rows(scry_buf a, scry_buf b, int a_rows, int b_rows, int cols, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(a, "concat_rows");
    CHECK_BUF(b, "concat_rows");
    if (a_rows < 0 || b_rows < 0 || cols < 0) return set_error(SCRY_ERR_INVALID, "concat_rows: negative shape");
    // cpu.rs:526-539: the whole of a, then the whole of b
    SCRY_TRY(new_buf(a->n + b->n, out));
    if (a->n)
        SCRY_HIP(hipMemcpyAsync((*out)->d, a->d, sizeof(float) * a->n, hipMemcpyDeviceToDevice, ctx().stream));
    if (b->n)
        SCRY_HIP(hipMemcpyAsync((*out)->d + a->n, b->d, sizeof(float) * b->n, hipMemcpyDeviceToDevice,
                                ctx().stream));
    return SCRY_OK;
}

int scry_hip_rope(scry_buf x, size_t rows, int last_dim, int pos, int head_dim, float theta, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "rope");
    if (last_dim <= 0 || head_dim <= 0 || pos < 0 || x->n != rows * (size_t)last_dim)
        return set_error(SCRY_ERR_INVALID, "rope: shape mismatch");
    // cpu.rs:612-624: freq = 1 / theta^(2i / head_dim), angle = pos * freq,
    // cos / sin in f64 (glibc, as the reference) rounded to f32
    const int np = head_dim / 2;
    std::vector<float2> cs((size_t)(np > 0 ? np : 1));
    const double th = (double)theta;
    for (int i = 0; i < np; i++) {
        const double freq = 1.0 / std::pow(th, 2.0 * (double)i / (double)head_dim);
        const double ang = (double)pos * freq;
        cs[i] = make_float2((float)std::cos(ang), (float)std::sin(ang));
    }
    float2 *d_cs = nullptr;
    SCRY_TRY(dev_alloc((void **)&d_cs, sizeof(float2) * cs.size()));
    int rc = new_buf(x->n, out);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(d_cs, cs.data(), sizeof(float2) * cs.size(), hipMemcpyHostToDevice,
                                      ctx().stream);
        rc = e == hipSuccess ? SCRY_OK : hip_fail(e, "rope table upload", __FILE__, __LINE__);
        if (!rc) rc = launch_rope_row(x->d, rows, last_dim, head_dim, d_cs, (*out)->d, ctx().stream);
        if (!rc) rc = sync();  // the table is freed below
    }
    dev_free(d_cs);
    return rc;
}

int scry_hip_gather_columns(scry_buf x, int rows, int total_cols, int col_start, int col_count, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "gather_columns");
    if (rows < 0 || col_start < 0 || col_count < 0 || col_start + col_count > total_cols ||
        x->n < (size_t)rows * total_cols)
        return set_error(SCRY_ERR_RANGE, "gather_columns: columns [%d, %d) outside %d", col_start,
                         col_start + col_count, total_cols);
    SCRY_TRY(new_buf((size_t)rows * col_count, out));
    return launch_gather_cols(x->d, (size_t)rows, total_cols, col_start, col_count, (*out)->d, ctx().stream);
}

int scry_hip_scatter_columns(scry_buf dst, scry_buf src, int rows, int total_cols, int col_start, int col_count) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(dst, "scatter_columns");
    CHECK_BUF(src, "scatter_columns");
    if (rows < 0 || col_start < 0 || col_count < 0 || col_start + col_count > total_cols ||
        dst->n < (size_t)rows * total_cols || src->n < (size_t)rows * col_count)
        return set_error(SCRY_ERR_RANGE, "scatter_columns: columns [%d, %d) outside %d", col_start,
                         col_start + col_count, total_cols);
    SCRY_TRY(launch_scatter_cols_add(dst->d, src->d, (size_t)rows, total_cols, col_start, col_count, ctx().stream));
    bf16_stale(dst);
    return SCRY_OK;
}

int scry_hip_gather_rows(scry_buf x, int total_rows, int cols, int row_start, int row_count, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(x, "gather_rows");
    if (cols < 0 || row_start < 0 || row_count < 0 || x->n < (size_t)(row_start + row_count) * cols)
        return set_error(SCRY_ERR_RANGE, "gather_rows: rows [%d, %d) outside the storage", row_start,
                         row_start + row_count);
    (void)total_rows;  // mod.rs:360 ignores it as well
    const size_t n = (size_t)row_count * cols;
    SCRY_TRY(new_buf(n, out));
    if (n)
        SCRY_HIP(hipMemcpyAsync((*out)->d, x->d + (size_t)row_start * cols, sizeof(float) * n,
                                hipMemcpyDeviceToDevice, ctx().stream));
    return SCRY_OK;
}

int scry_hip_apply_causal_mask_and_scale(scry_buf scores, int seq, float scale, float mask_value) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(scores, "apply_causal_mask_and_scale");
    if (seq < 0 || scores->n < (size_t)seq * seq)
        return set_error(SCRY_ERR_INVALID, "apply_causal_mask_and_scale: shape mismatch");
    SCRY_TRY(launch_causal_mask(scores->d, seq ? 1 : 0, seq, scale, mask_value, ctx().stream));
    bf16_stale(scores);
    return SCRY_OK;
}

int scry_hip_apply_batched_causal_mask_and_scale(scry_buf scores, int num_matrices, int seq, float scale,
                                                 float mask_value) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(scores, "apply_batched_causal_mask_and_scale");
    if (seq <= 0 || num_matrices < 0) return set_error(SCRY_ERR_INVALID, "apply_batched_causal_mask_and_scale: shape");
    // mod.rs:602-606: every whole [seq, seq] matrix of the storage (num_matrices unused)
    SCRY_TRY(launch_causal_mask(scores->d, scores->n / ((size_t)seq * seq), seq, scale, mask_value, ctx().stream));
    bf16_stale(scores);
    return SCRY_OK;
}

int scry_hip_split_qkv_reshape_heads(scry_buf qkv, int seq, int n_heads, int d_head, scry_buf *q, scry_buf *k,
                                     scry_buf *v) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    CHECK_BUF(qkv, "split_qkv_reshape_heads");
    if (!q || !k || !v) return set_error(SCRY_ERR_INVALID, "split_qkv_reshape_heads: null output handle");
    const size_t hl = (size_t)seq * n_heads * d_head;
    if (seq < 0 || n_heads < 0 || d_head < 0 || qkv->n < 3 * hl)
        return set_error(SCRY_ERR_INVALID, "split_qkv_reshape_heads: shape mismatch");
    scry_buf bq = nullptr, bk = nullptr, bv = nullptr;
    int rc = new_buf(hl, &bq);
    if (!rc) rc = new_buf(hl, &bk);
    if (!rc) rc = new_buf(hl, &bv);
    if (!rc) rc = launch_split_qkv(qkv->d, seq, n_heads, d_head, bq->d, bk->d, bv->d, ctx().stream);
    if (rc) {
        del_buf(bq);
        del_buf(bk);
        del_buf(bv);
        return rc;
    }
    *q = bq;
    *k = bk;
    *v = bv;
    return SCRY_OK;
}

static int reshape_heads(scry_buf x, int batch, int seq, int n_heads, int d_head, int dir, scry_buf *out) {
    CHECK_BUF(x, "reshape_heads");
    const size_t n = (size_t)batch * seq * n_heads * d_head;
    if (batch < 0 || seq < 0 || n_heads < 0 || d_head < 0 || x->n < n)
        return set_error(SCRY_ERR_INVALID, "reshape_heads: shape mismatch");
    if (batch == 1 && seq == 1) return scry_hip_clone_storage(x, out);  // mod.rs:449-451, 492-494
    SCRY_TRY(new_buf(n, out));
    return launch_reshape_heads(x->d, batch, seq, n_heads, d_head, dir, (*out)->d, ctx().stream);
}

int scry_hip_reshape_for_heads(scry_buf x, int batch, int seq, int n_heads, int d_head, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return reshape_heads(x, batch, seq, n_heads, d_head, 0, out);
}

int scry_hip_reshape_from_heads(scry_buf x, int batch, int seq, int n_heads, int d_head, scry_buf *out) {
    API_LOCK;
    SCRY_REQUIRE_INIT();
    return reshape_heads(x, batch, seq, n_heads, d_head, 1, out);
}

}  // extern "C"
