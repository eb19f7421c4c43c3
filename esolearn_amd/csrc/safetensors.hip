// safetensors shards for the checkpoint loader (LlamaModel::from_safetensors,
// llama.rs:765-958, which reads them with the safetensors crate).
//
// File format: an 8-byte little-endian header length N, N bytes of JSON
//   {"__metadata__": {...}, "<name>": {"dtype": "BF16", "shape": [r, c],
//    "data_offsets": [begin, end]}, ...}
// then the data section; offsets are relative to its start (8 + N).
//
// The shards are memory-mapped read-only.  A tensor's raw bytes go to the
// device as stored and k_widen turns them into f32 there, with the
// reference's conversions (llama.rs:1070-1129): F32 as is, BF16 as the upper
// 16 bits of an f32, F16 by IEEE half decoding (subnormals normalised, Inf and
// NaN keep their payload bits).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "internal.h"

namespace scry {

struct StFile {
    std::string path;
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0, data0 = 0;
    std::vector<StTensor> tensors;
};

struct StShards {
    std::vector<StFile> files;
};

namespace {

// ---- a JSON reader for the header: objects, arrays, strings, integers, and
// any other value skipped
struct Json {
    const char *p, *e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < e && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool str(std::string &out) {
        ws();
        if (p >= e || *p != '"') return ok = false;
        p++;
        out.clear();
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) return ok = false;
                switch (*p) {
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u':  // names here are ASCII; keep the escape verbatim
                        out += "\\u";
                        break;
                    default: out += *p;
                }
                p++;
            } else {
                out += *p++;
            }
        }
        if (p >= e) return ok = false;
        p++;
        return true;
    }
    bool integer(int64_t &v) {
        ws();
        const char *s = p;
        if (p < e && *p == '-') p++;
        if (p >= e || *p < '0' || *p > '9') return ok = false;
        v = 0;
        bool neg = *s == '-';
        while (p < e && *p >= '0' && *p <= '9') {
            if (v > (INT64_MAX - 9) / 10) return ok = false;
            v = v * 10 + (*p++ - '0');
        }
        if (neg) v = -v;
        return true;
    }
    bool skip() {  // any value
        ws();
        if (p >= e) return ok = false;
        if (*p == '"') {
            std::string t;
            return str(t);
        }
        if (*p == '{' || *p == '[') {
            const char open = *p, close = open == '{' ? '}' : ']';
            p++;
            if (eat(close)) return true;
            do {
                if (open == '{') {
                    std::string k;
                    if (!str(k) || !eat(':')) return ok = false;
                }
                if (!skip()) return false;
            } while (eat(','));
            return eat(close) || (ok = false);
        }
        while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n') p++;  // number / literal
        return true;
    }
    bool int_array(std::vector<int64_t> &v) {
        v.clear();
        if (!eat('[')) return ok = false;
        if (eat(']')) return true;
        do {
            int64_t x;
            if (!integer(x)) return false;
            v.push_back(x);
        } while (eat(','));
        return eat(']') || (ok = false);
    }
};

int dtype_of(const std::string &s, int *bytes) {
    if (s == "F32") return *bytes = 4, ST_F32;
    if (s == "BF16") return *bytes = 2, ST_BF16;
    if (s == "F16") return *bytes = 2, ST_F16;
    *bytes = 0;
    return ST_OTHER;
}

int parse_header(StFile &f) {
    if (f.size < 8) return set_error(SCRY_ERR_INVALID, "safetensors: %s is too short", f.path.c_str());
    uint64_t n = 0;
    std::memcpy(&n, f.map, 8);  // little-endian (x86 host)
    if (n > f.size - 8 || n > (100u << 20))
        return set_error(SCRY_ERR_INVALID, "safetensors: %s header length %llu is invalid", f.path.c_str(),
                         (unsigned long long)n);
    f.data0 = 8 + (size_t)n;
    const size_t data_bytes = f.size - f.data0;
    Json j{(const char *)f.map + 8, (const char *)f.map + 8 + n};
    if (!j.eat('{')) return set_error(SCRY_ERR_INVALID, "safetensors: %s header is not a JSON object", f.path.c_str());
    if (!j.eat('}')) {
        do {
            std::string name;
            if (!j.str(name) || !j.eat(':')) break;
            if (name == "__metadata__") {
                if (!j.skip()) break;
                continue;
            }
            StTensor t;
            t.name = name;
            std::string dt;
            std::vector<int64_t> off;
            bool have_dt = false, have_shape = false, have_off = false;
            if (!j.eat('{')) break;
            if (!j.eat('}')) {
                do {
                    std::string key;
                    if (!j.str(key) || !j.eat(':')) break;
                    if (key == "dtype") {
                        have_dt = j.str(dt);
                    } else if (key == "shape") {
                        have_shape = j.int_array(t.shape);
                    } else if (key == "data_offsets") {
                        have_off = j.int_array(off);
                    } else if (!j.skip()) {
                        break;
                    }
                } while (j.ok && j.eat(','));
                if (j.ok && !j.eat('}')) j.ok = false;
            }
            if (!j.ok) break;
            if (!have_dt || !have_shape || !have_off || off.size() != 2)
                return set_error(SCRY_ERR_INVALID, "safetensors: %s: entry '%s' lacks dtype, shape or data_offsets",
                                 f.path.c_str(), name.c_str());
            int eb = 0;
            t.dtype = dtype_of(dt, &eb);
            t.dtype_name = dt;
            int64_t numel = 1;
            for (int64_t d : t.shape) {
                if (d < 0 || (d > 0 && numel > INT64_MAX / d))
                    return set_error(SCRY_ERR_INVALID, "safetensors: %s: bad shape of '%s'", f.path.c_str(), name.c_str());
                numel *= d;
            }
            t.numel = (size_t)numel;
            if (off[0] < 0 || off[1] < off[0] || (size_t)off[1] > data_bytes)
                return set_error(SCRY_ERR_INVALID, "safetensors: %s: data_offsets of '%s' out of the file",
                                 f.path.c_str(), name.c_str());
            t.bytes = (size_t)(off[1] - off[0]);
            if (eb && t.bytes != t.numel * (size_t)eb)
                return set_error(SCRY_ERR_INVALID, "safetensors: %s: '%s' holds %zu bytes for %zu %s elements",
                                 f.path.c_str(), name.c_str(), t.bytes, t.numel, dt.c_str());
            t.data = f.map + f.data0 + off[0];
            f.tensors.push_back(std::move(t));
        } while (j.ok && j.eat(','));
        if (j.ok && !j.eat('}')) j.ok = false;
    }
    if (!j.ok) return set_error(SCRY_ERR_INVALID, "safetensors: %s: malformed header", f.path.c_str());
    return SCRY_OK;
}

// F32 / BF16 / F16 words -> f32 (llama.rs:1070-1129)
__device__ __forceinline__ float f16_bits_to_f32(unsigned h) {
    const unsigned sign = (h >> 15) << 31, ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (ex == 0) {
        // zero or subnormal: man * 2^-24 is exact in f32
        return __uint_as_float(sign | __float_as_uint((float)man * 0x1p-24f));
    }
    if (ex == 31) return __uint_as_float(sign | 0x7f800000u | (man << 13));  // Inf / NaN, payload kept
    return __uint_as_float(sign | ((ex + 112u) << 23) | (man << 13));
}

__global__ __launch_bounds__(256) void k_widen(const void *__restrict__ src, int dtype, size_t n,
                                               float *__restrict__ dst) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        if (dtype == ST_F32) {
            dst[i] = ((const float *)src)[i];
        } else {
            const unsigned w = ((const unsigned short *)src)[i];
            dst[i] = dtype == ST_BF16 ? __uint_as_float(w << 16) : f16_bits_to_f32(w);
        }
    }
}

}  // namespace

int st_open(const char *const *paths, int n_paths, StShards **out) {
    if (!paths || n_paths <= 0 || !out) return set_error(SCRY_ERR_INVALID, "safetensors: no shard paths");
    auto *sh = new (std::nothrow) StShards;
    if (!sh) return set_error(SCRY_ERR_OOM, "host allocation failed");
    sh->files.resize(n_paths);
    int rc = SCRY_OK;
    for (int i = 0; i < n_paths && !rc; i++) {
        StFile &f = sh->files[i];
        f.path = paths[i] ? paths[i] : "";
        f.fd = open(f.path.c_str(), O_RDONLY);
        struct stat st;
        if (f.fd < 0 || fstat(f.fd, &st) != 0) {
            rc = set_error(SCRY_ERR_INVALID, "failed to read %s: %s", f.path.c_str(), std::strerror(errno));
            break;
        }
        f.size = (size_t)st.st_size;
        void *m = f.size ? mmap(nullptr, f.size, PROT_READ, MAP_PRIVATE, f.fd, 0) : MAP_FAILED;
        if (m == MAP_FAILED) {
            rc = set_error(SCRY_ERR_INVALID, "failed to map %s", f.path.c_str());
            break;
        }
        f.map = (const uint8_t *)m;
        rc = parse_header(f);
    }
    if (rc) {
        st_close(sh);
        return rc;
    }
    *out = sh;
    return SCRY_OK;
}

void st_close(StShards *sh) {
    if (!sh) return;
    for (auto &f : sh->files) {
        if (f.map) munmap((void *)f.map, f.size);
        if (f.fd >= 0) close(f.fd);
    }
    delete sh;
}

const StTensor *st_find(const StShards *sh, const char *name) {
    for (const auto &f : sh->files)  // llama.rs:794-811: the first shard holding it
        for (const auto &t : f.tensors)
            if (t.name == name) return &t;
    return nullptr;
}

int launch_widen(const void *src, int dtype, size_t n, float *dst, hipStream_t s) {
    if (dtype != ST_F32 && dtype != ST_BF16 && dtype != ST_F16)
        return set_error(SCRY_ERR_INVALID, "widen: dtype %d", dtype);
    if (n == 0) return SCRY_OK;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(k_widen, dim3((unsigned)blocks), dim3(256), 0, s, src, dtype, n, dst);
    SCRY_HIP(hipGetLastError());
    return SCRY_OK;
}

}  // namespace scry
