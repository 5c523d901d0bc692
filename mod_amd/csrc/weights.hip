// int8 on-disk weights: a safetensors reader for the int8 linear path.
//
// Replaces the reference loader (plugins/cpu/c_src/safetensors_loader.c:
// open_safetensors :40-120, load_tensor_data :147-243, close_safetensors
// :245-265, bound at core/engine/backend.py:120-126, used by load_safetensors
// backend.py:812-835) and extends it to the dtypes an int8 checkpoint holds:
// I8 weights, F32 per-channel scales, and BF16 / F16 / F32 fp weights to be
// quantized. The reference finds a tensor by searching the header text for
// "<name>" and then the next "data_offsets" (a name that is a suffix of
// another, or a field order other than its own, reads the wrong tensor), and
// picks F32 or F16 from the byte count (BF16 data is read as F16). Here the
// header is parsed as JSON into a table of (dtype, shape, offsets), every
// entry is checked against the file size and against its dtype x shape, and
// conversions follow the stored dtype.
//
// File layout (safetensors): u64 little-endian header length N, N bytes of
// JSON {"name": {"dtype": "I8", "shape": [..], "data_offsets": [b, e]}, ...,
// "__metadata__": {..}}, then the data; offsets are relative to byte 8 + N.
// The file is mapped read-only: the header is parsed and host reads copy from
// the mapping; device loads read the file with pread into pinned staging
// buffers (below) and convert on the GPU.
#include "pio_common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace pio {

// Stored element types (the safetensors dtype strings), as reported by
// pio_safetensors_info.
enum {
    ST_F64 = 0, ST_F32 = 1, ST_F16 = 2, ST_BF16 = 3, ST_I64 = 4, ST_I32 = 5,
    ST_I16 = 6, ST_I8 = 7, ST_U8 = 8, ST_BOOL = 9, ST_U16 = 10, ST_U32 = 11, ST_U64 = 12,
};

static int st_dtype_of(const std::string& s) {
    static const char* names[] = {"F64", "F32", "F16", "BF16", "I64", "I32", "I16",
                                  "I8",  "U8",  "BOOL", "U16", "U32", "U64"};
    for (int i = 0; i < (int)(sizeof(names) / sizeof(names[0])); i++)
        if (s == names[i]) return i;
    return -1;
}
static int st_size(int dt) {
    switch (dt) {
    case ST_F64: case ST_I64: case ST_U64: return 8;
    case ST_F32: case ST_I32: case ST_U32: return 4;
    case ST_F16: case ST_BF16: case ST_I16: case ST_U16: return 2;
    default: return 1;
    }
}

struct StEntry {
    int dtype = -1;
    std::vector<int64_t> shape;
    int64_t begin = 0, end = 0;
};

struct StFile {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    size_t data0 = 0;   // 8 + header length
    std::vector<std::string> names;   // in header order
    std::unordered_map<std::string, StEntry> t;
    ~StFile() {
        if (map) munmap((void*)map, size);
        if (fd >= 0) close(fd);
    }
};

// ------------------------------------------------------------- JSON subset
// Objects, arrays, strings (with escapes; \u escapes below 0x80 decoded, others
// kept as '?'), numbers (integers are what the entries need), true/false/null.
struct Json {
    const char* p;
    const char* e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < e && *p == c) { p++; return true; }
        return false;
    }
    bool str(std::string& out) {
        ws();
        if (p >= e || *p != '"') return ok = false;
        p++;
        out.clear();
        while (p < e && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= e) return ok = false;
                const char x = *p++;
                switch (x) {
                case 'n': c = '\n'; break;
                case 't': c = '\t'; break;
                case 'r': c = '\r'; break;
                case 'b': c = '\b'; break;
                case 'f': c = '\f'; break;
                case 'u': {
                    if (e - p < 4) return ok = false;
                    unsigned v = 0;
                    for (int i = 0; i < 4; i++) {
                        const char h = p[i];
                        const int d = h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                    : h >= 'A' && h <= 'F' ? h - 'A' + 10 : -1;
                        if (d < 0) return ok = false;
                        v = v * 16 + (unsigned)d;
                    }
                    p += 4;
                    c = v < 0x80 ? (char)v : '?';
                    break;
                }
                default: c = x;   // \" \\ \/
                }
            }
            out.push_back(c);
        }
        if (p >= e) return ok = false;
        p++;
        return true;
    }
    bool integer(int64_t& v) {
        ws();
        const char* s = p;
        bool neg = false;
        if (p < e && *p == '-') { neg = true; p++; }
        if (p >= e || *p < '0' || *p > '9') return ok = false;
        uint64_t x = 0;
        while (p < e && *p >= '0' && *p <= '9') {
            if (x > (uint64_t)INT64_MAX / 10) return ok = false;
            x = x * 10 + (uint64_t)(*p++ - '0');
        }
        if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) { p = s; return ok = false; }
        if (x > (uint64_t)INT64_MAX) return ok = false;
        v = neg ? -(int64_t)x : (int64_t)x;
        return true;
    }
    bool skip(int depth = 0) {
        if (depth > 64) return ok = false;
        ws();
        if (p >= e) return ok = false;
        const char c = *p;
        if (c == '"') { std::string s; return str(s); }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            p++;
            if (eat(close)) return true;
            do {
                if (c == '{') {
                    std::string k;
                    if (!str(k) || !eat(':')) return ok = false;
                }
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return eat(close) ? true : (ok = false);
        }
        // number or literal
        const char* s = p;
        while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n' && *p != '\r' &&
               *p != '\t')
            p++;
        return p > s ? true : (ok = false);
    }
    bool int_array(std::vector<int64_t>& out) {
        out.clear();
        if (!eat('[')) return ok = false;
        if (eat(']')) return true;
        do {
            int64_t v;
            if (!integer(v)) return false;
            out.push_back(v);
        } while (eat(','));
        return eat(']') ? true : (ok = false);
    }
};

static int parse_entry(Json& j, StEntry& en, const std::string& name) {
    if (!j.eat('{')) return set_error(PIO_ERR_INVALID, "safetensors: entry '%s' is not an object", name.c_str());
    bool have_dt = false, have_off = false, have_shape = false;
    if (!j.eat('}')) {
        do {
            std::string k;
            if (!j.str(k) || !j.eat(':')) return set_error(PIO_ERR_INVALID, "safetensors: bad entry '%s'", name.c_str());
            if (k == "dtype") {
                std::string d;
                if (!j.str(d)) return set_error(PIO_ERR_INVALID, "safetensors: bad dtype of '%s'", name.c_str());
                en.dtype = st_dtype_of(d);
                if (en.dtype < 0)
                    return set_error(PIO_ERR_UNSUPPORTED, "safetensors: '%s' has unknown dtype %s", name.c_str(), d.c_str());
                have_dt = true;
            } else if (k == "shape") {
                if (!j.int_array(en.shape)) return set_error(PIO_ERR_INVALID, "safetensors: bad shape of '%s'", name.c_str());
                have_shape = true;
            } else if (k == "data_offsets") {
                std::vector<int64_t> o;
                if (!j.int_array(o) || o.size() != 2)
                    return set_error(PIO_ERR_INVALID, "safetensors: bad data_offsets of '%s'", name.c_str());
                en.begin = o[0];
                en.end = o[1];
                have_off = true;
            } else if (!j.skip()) {
                return set_error(PIO_ERR_INVALID, "safetensors: bad field '%s' of '%s'", k.c_str(), name.c_str());
            }
        } while (j.eat(','));
        if (!j.eat('}')) return set_error(PIO_ERR_INVALID, "safetensors: unterminated entry '%s'", name.c_str());
    }
    if (!have_dt || !have_off || !have_shape)
        return set_error(PIO_ERR_INVALID, "safetensors: entry '%s' lacks dtype, shape or data_offsets", name.c_str());
    return PIO_OK;
}

static int st_open(const char* path, StFile*& out) {
    out = nullptr;
    PIO_REQUIRE(path, "open_safetensors: null path");
    StFile* f = new StFile();
    auto fail = [&](int rc) { delete f; return rc; };
    f->fd = open(path, O_RDONLY);
    if (f->fd < 0) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: cannot open %s", path));
    struct stat sb;
    if (fstat(f->fd, &sb) != 0 || sb.st_size < 8)
        return fail(set_error(PIO_ERR_INVALID, "open_safetensors: %s is too short", path));
    f->size = (size_t)sb.st_size;
    void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: cannot map %s", path));
    f->map = (const uint8_t*)m;
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | f->map[i];
    if (n > f->size - 8) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: header length %llu exceeds the file",
                                               (unsigned long long)n));
    f->data0 = 8 + (size_t)n;
    const size_t data_bytes = f->size - f->data0;
    Json j{(const char*)f->map + 8, (const char*)f->map + 8 + n};
    if (!j.eat('{')) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: header is not a JSON object"));
    if (!j.eat('}')) {
        do {
            std::string name;
            if (!j.str(name) || !j.eat(':')) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: bad header key"));
            if (name == "__metadata__") {
                if (!j.skip()) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: bad __metadata__"));
                continue;
            }
            StEntry en;
            const int rc = parse_entry(j, en, name);
            if (rc != PIO_OK) return fail(rc);
            int64_t count = 1;
            for (int64_t d : en.shape) {
                if (d < 0 || (d > 0 && count > INT64_MAX / d))
                    return fail(set_error(PIO_ERR_INVALID, "safetensors: bad shape of '%s'", name.c_str()));
                count *= d;
            }
            if (en.begin < 0 || en.end < en.begin || (uint64_t)en.end > data_bytes)
                return fail(set_error(PIO_ERR_INVALID, "safetensors: '%s' offsets [%lld, %lld) outside the %zu data bytes",
                                      name.c_str(), (long long)en.begin, (long long)en.end, data_bytes));
            if (count > INT64_MAX / 8 || en.end - en.begin != count * st_size(en.dtype))
                return fail(set_error(PIO_ERR_INVALID, "safetensors: '%s' holds %lld bytes, its dtype and shape need %lld",
                                      name.c_str(), (long long)(en.end - en.begin), (long long)(count * st_size(en.dtype))));
            if (f->t.count(name)) return fail(set_error(PIO_ERR_INVALID, "safetensors: '%s' appears twice", name.c_str()));
            f->names.push_back(name);
            f->t.emplace(name, en);
        } while (j.eat(','));
        if (!j.eat('}')) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: unterminated header"));
    }
    if (!j.ok) return fail(set_error(PIO_ERR_INVALID, "open_safetensors: malformed header"));
    out = f;
    return PIO_OK;
}

static int st_find(void* ctx, const char* name, const StEntry*& en) {
    en = nullptr;
    PIO_REQUIRE(ctx && name, "safetensors: null context or name");
    StFile* f = (StFile*)ctx;
    auto it = f->t.find(name);
    PIO_REQUIRE(it != f->t.end(), "safetensors: no tensor '%s'", name);
    en = &it->second;
    return PIO_OK;
}

static int64_t st_count(const StEntry& en) {
    int64_t c = 1;
    for (int64_t d : en.shape) c *= d;
    return c;
}

// bf16 / f16 -> f32, exact.
static inline float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline float f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            u = s;
        } else {   // subnormal: normalize
            // m * 2^-24 with the leading one at bit p: exponent p - 24.
            int ee = 0;
            uint32_t mm = m;
            while (!(mm & 1024)) { mm <<= 1; ee--; }
            u = s | (uint32_t)(127 - 15 + 1 + ee) << 23 | (mm & 1023) << 13;
        }
    } else {
        u = s | (e - 15 + 127) << 23 | m << 13;
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// Element i of a stored tensor as f32 (float and integer dtypes except 64-bit).
static int st_to_f32(const StEntry& en, const uint8_t* src, float* dst, int64_t n) {
    switch (en.dtype) {
    case ST_F32: memcpy(dst, src, (size_t)n * 4); return PIO_OK;
    case ST_F16:
        for (int64_t i = 0; i < n; i++) { uint16_t h; memcpy(&h, src + 2 * i, 2); dst[i] = f16_to_f32(h); }
        return PIO_OK;
    case ST_BF16:
        for (int64_t i = 0; i < n; i++) { uint16_t h; memcpy(&h, src + 2 * i, 2); dst[i] = bf16_to_f32(h); }
        return PIO_OK;
    case ST_I8:
        for (int64_t i = 0; i < n; i++) dst[i] = (float)(int8_t)src[i];
        return PIO_OK;
    case ST_U8: case ST_BOOL:
        for (int64_t i = 0; i < n; i++) dst[i] = (float)src[i];
        return PIO_OK;
    case ST_I32:
        for (int64_t i = 0; i < n; i++) { int32_t v; memcpy(&v, src + 4 * i, 4); dst[i] = (float)v; }
        return PIO_OK;
    case ST_I16:
        for (int64_t i = 0; i < n; i++) { int16_t v; memcpy(&v, src + 2 * i, 2); dst[i] = (float)v; }
        return PIO_OK;
    default:
        return set_error(PIO_ERR_UNSUPPORTED, "safetensors: no f32 conversion for this dtype");
    }
}

}  // namespace pio

using namespace pio;

PIO_EXPORT void* open_safetensors(const char* filepath) {
    StFile* f = nullptr;
    return st_open(filepath, f) == PIO_OK ? (void*)f : nullptr;
}

PIO_EXPORT void close_safetensors(void* ctx) { delete (StFile*)ctx; }

// Reference convention: 1 on success, 0 on failure; `size` is the element
// count of `buffer` and must equal the stored tensor's.
PIO_EXPORT int load_tensor_data(void* ctx, const char* name, float* buffer, int size) {
    const StEntry* en;
    if (st_find(ctx, name, en) != PIO_OK || !buffer) return 0;
    if (st_count(*en) != (int64_t)size) {
        set_error(PIO_ERR_INVALID, "load_tensor_data: '%s' has %lld elements, buffer %d", name,
                  (long long)st_count(*en), size);
        return 0;
    }
    const StFile* f = (const StFile*)ctx;
    return st_to_f32(*en, f->map + f->data0 + en->begin, buffer, size) == PIO_OK ? 1 : 0;
}

PIO_EXPORT int pio_safetensors_count(void* ctx) { return ctx ? (int)((StFile*)ctx)->names.size() : 0; }

PIO_EXPORT const char* pio_safetensors_name(void* ctx, int i) {
    if (!ctx || i < 0 || i >= (int)((StFile*)ctx)->names.size()) return nullptr;
    return ((StFile*)ctx)->names[i].c_str();
}

PIO_EXPORT int pio_safetensors_info(void* ctx, const char* name, int* dtype, int64_t* shape, int max_dims,
                                    int* ndim, int64_t* nbytes) {
    const StEntry* en;
    PIO_TRY(st_find(ctx, name, en));
    if (dtype) *dtype = en->dtype;
    if (ndim) *ndim = (int)en->shape.size();
    if (nbytes) *nbytes = en->end - en->begin;
    if (shape)
        for (int i = 0; i < (int)en->shape.size() && i < max_dims; i++) shape[i] = en->shape[i];
    return PIO_OK;
}

// Raw stored bytes into host memory (nbytes must equal the stored size).
PIO_EXPORT int pio_safetensors_read(void* ctx, const char* name, void* dst, int64_t nbytes) {
    const StEntry* en;
    PIO_TRY(st_find(ctx, name, en));
    PIO_REQUIRE(dst, "pio_safetensors_read: null destination");
    PIO_REQUIRE(nbytes == en->end - en->begin, "pio_safetensors_read: '%s' holds %lld bytes, asked %lld", name,
                (long long)(en->end - en->begin), (long long)nbytes);
    const StFile* f = (const StFile*)ctx;
    memcpy(dst, f->map + f->data0 + en->begin, (size_t)nbytes);
    return PIO_OK;
}

// ------------------------------------------------------------ device loads
// Host -> device path: the stored bytes are read with pread (page cache ->
// pinned memory, no page faults on the mapping) by a small pool of threads
// into one of two pinned staging buffers while the other buffer's DMA runs,
// so the copy rate approaches the PCIe link's rather than one core's memcpy.
// (Measured on the config-2 checkpoint: 16 MiB chunks with one DMA each beat
// 4 MiB chunks and per-thread slice DMAs, whose per-copy overheads cost more
// than the overlap they add.) The pool and the staging buffers are
// process-wide, created on first use and kept until exit (NSTAGE x
// STAGE_BYTES of pinned host memory); device loads from any context
// serialize on them.
namespace {

constexpr size_t STAGE_BYTES = 16u << 20;
constexpr int NSTAGE = 2;
constexpr size_t POOL_MIN_BYTES = 2u << 20;   // below this one thread reads

bool pread_full(int fd, uint8_t* dst, size_t n, off_t off) {
    while (n) {
        const ssize_t r = pread(fd, dst, n, off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        dst += r;
        n -= (size_t)r;
        off += r;
    }
    return true;
}

class ReadPool {
  public:
    explicit ReadPool(int nthreads) : T(nthreads) {
        for (int i = 0; i < T; i++) th.emplace_back([this, i] { worker(i); });
    }
    // Reads n bytes at `off` of `fd` into dst, split over the pool's threads.
    bool read(int fd_, uint8_t* dst_, size_t n_, off_t off_) {
        if (n_ < POOL_MIN_BYTES || T == 1) return pread_full(fd_, dst_, n_, off_);
        std::unique_lock<std::mutex> lk(m);
        fd = fd_; dst = dst_; n = n_; off = off_;
        pending = T;
        failed = false;
        gen++;
        cv.notify_all();
        done.wait(lk, [&] { return pending == 0; });
        return !failed;
    }

  private:
    void worker(int id) {
        unsigned seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lk(m);
            cv.wait(lk, [&] { return gen != seen; });
            seen = gen;
            const size_t per = (n + T - 1) / T, b = std::min(n, per * id), e = std::min(n, b + per);
            const int fd_ = fd;
            uint8_t* dst_ = dst;
            const off_t off_ = off;
            lk.unlock();
            const bool ok = e <= b || pread_full(fd_, dst_ + b, e - b, off_ + (off_t)b);
            lk.lock();
            if (!ok) failed = true;
            if (--pending == 0) done.notify_one();
        }
    }
    int T;
    std::vector<std::thread> th;
    std::mutex m;
    std::condition_variable cv, done;
    unsigned gen = 0;
    int pending = 0;
    bool failed = false;
    int fd = -1;
    uint8_t* dst = nullptr;
    size_t n = 0;
    off_t off = 0;
};

struct Stager {
    std::mutex mu;
    ReadPool* pool = nullptr;
    void* stage[NSTAGE] = {};
};
Stager g_stager;

// Copies file bytes [off, off+n) of `f` to device address dst on stream st;
// returns once they have landed. Caller holds g_stager.mu.
int stage_to_device(const StFile* f, size_t off, size_t n, void* dst, hipStream_t st) {
    Stager& S = g_stager;
    if (!S.pool) {
        const unsigned hc = std::thread::hardware_concurrency();
        S.pool = new ReadPool((int)std::max(1u, std::min(8u, hc ? hc : 1u)));   // lives until exit
    }
    for (int b = 0; b < NSTAGE; b++)
        if (!S.stage[b] && hipHostMalloc(&S.stage[b], STAGE_BYTES, hipHostMallocDefault) != hipSuccess) {
            S.stage[b] = nullptr;
            return set_error(PIO_ERR_OOM, "safetensors: pinned staging allocation failed");
        }
    hipEvent_t ev[NSTAGE] = {};
    int rc = PIO_OK;
    for (int b = 0; b < NSTAGE && rc == PIO_OK; b++)
        if (hipEventCreateWithFlags(&ev[b], hipEventDisableTiming) != hipSuccess)
            rc = set_error(PIO_ERR_HIP, "safetensors: event creation failed");
    const size_t file_off = f->data0 + off;
    for (size_t done = 0, i = 0; rc == PIO_OK && done < n; done += STAGE_BYTES, i++) {
        const int b = (int)(i % NSTAGE);
        const size_t len = std::min(STAGE_BYTES, n - done);
        if (i >= (size_t)NSTAGE && hipEventSynchronize(ev[b]) != hipSuccess) {
            rc = set_error(PIO_ERR_HIP, "safetensors: staging wait failed");
            break;
        }
        if (!S.pool->read(f->fd, (uint8_t*)S.stage[b], len, (off_t)(file_off + done))) {
            rc = set_error(PIO_ERR_INVALID, "safetensors: read of %zu bytes at %zu failed", len, file_off + done);
            break;
        }
        if (hipMemcpyAsync((char*)dst + done, S.stage[b], len, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipEventRecord(ev[b], st) != hipSuccess)
            rc = set_error(PIO_ERR_HIP, "safetensors: host-to-device copy failed");
    }
    // Drain before the staging buffers can be reused, also after an error.
    if (hipStreamSynchronize(st) != hipSuccess && rc == PIO_OK) rc = set_error(PIO_ERR_HIP, "stream sync failed");
    for (int b = 0; b < NSTAGE; b++)
        if (ev[b]) (void)hipEventDestroy(ev[b]);
    return rc;
}

// Stored element -> f32, one element per thread (grid-stride).
template <int DT>
__global__ void widen_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v;
        if constexpr (DT == ST_BF16) {
            v = __uint_as_float((uint32_t)((const uint16_t*)src)[i] << 16);
        } else if constexpr (DT == ST_F16) {
            v = (float)((const _Float16*)src)[i];
        } else if constexpr (DT == ST_I8) {
            v = (float)((const int8_t*)src)[i];
        } else if constexpr (DT == ST_U8 || DT == ST_BOOL) {
            v = (float)src[i];
        } else if constexpr (DT == ST_I16) {
            v = (float)((const int16_t*)src)[i];
        } else {   // ST_I32
            v = (float)((const int32_t*)src)[i];
        }
        dst[i] = v;
    }
}

int launch_widen(int dt, const void* src, float* dst, int64_t n, hipStream_t st) {
    if (n == 0) return PIO_OK;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
    const uint8_t* s = (const uint8_t*)src;
    switch (dt) {
    case ST_BF16: widen_kernel<ST_BF16><<<blocks, 256, 0, st>>>(s, dst, n); break;
    case ST_F16: widen_kernel<ST_F16><<<blocks, 256, 0, st>>>(s, dst, n); break;
    case ST_I8: widen_kernel<ST_I8><<<blocks, 256, 0, st>>>(s, dst, n); break;
    case ST_U8: case ST_BOOL: widen_kernel<ST_U8><<<blocks, 256, 0, st>>>(s, dst, n); break;
    case ST_I16: widen_kernel<ST_I16><<<blocks, 256, 0, st>>>(s, dst, n); break;
    case ST_I32: widen_kernel<ST_I32><<<blocks, 256, 0, st>>>(s, dst, n); break;
    default: return set_error(PIO_ERR_UNSUPPORTED, "safetensors: no f32 conversion for this dtype");
    }
    PIO_LAUNCHED();
    return PIO_OK;
}

}  // namespace

// Raw stored bytes into device memory; returns when the data has landed.
PIO_EXPORT int pio_safetensors_to_device(void* ctx, const char* name, void* dst, int64_t nbytes, void* stream) {
    const StEntry* en;
    PIO_TRY(st_find(ctx, name, en));
    PIO_REQUIRE(dst, "pio_safetensors_to_device: null destination");
    PIO_REQUIRE(nbytes == en->end - en->begin, "pio_safetensors_to_device: '%s' holds %lld bytes, asked %lld", name,
                (long long)(en->end - en->begin), (long long)nbytes);
    if (nbytes == 0) return PIO_OK;
    std::lock_guard<std::mutex> lk(g_stager.mu);
    return stage_to_device((const StFile*)ctx, (size_t)en->begin, (size_t)nbytes, dst, pick_stream(stream));
}

// `name` converted to fp32 into device memory (count elements): F32 is
// copied, the other dtypes land raw in a device scratch buffer and are
// widened there by a kernel. Returns when done.
PIO_EXPORT int pio_safetensors_to_device_f32(void* ctx, const char* name, float* dst, int64_t count, void* stream) {
    const StEntry* en;
    PIO_TRY(st_find(ctx, name, en));
    PIO_REQUIRE(dst, "pio_safetensors_to_device_f32: null destination");
    PIO_REQUIRE(count == st_count(*en), "pio_safetensors_to_device_f32: '%s' has %lld elements, asked %lld", name,
                (long long)st_count(*en), (long long)count);
    const int64_t nbytes = en->end - en->begin;
    if (en->dtype == ST_F32) return pio_safetensors_to_device(ctx, name, dst, nbytes, stream);
    switch (en->dtype) {
    case ST_BF16: case ST_F16: case ST_I8: case ST_U8: case ST_BOOL: case ST_I16: case ST_I32: break;
    default: return set_error(PIO_ERR_UNSUPPORTED, "pio_safetensors_to_device_f32: '%s' has no f32 conversion", name);
    }
    if (count == 0) return PIO_OK;
    hipStream_t st = pick_stream(stream);
    Scratch raw;
    PIO_TRY(raw.get((size_t)nbytes, st));
    {
        std::lock_guard<std::mutex> lk(g_stager.mu);
        PIO_TRY(stage_to_device((const StFile*)ctx, (size_t)en->begin, (size_t)nbytes, raw.ptr, st));
    }
    PIO_TRY(launch_widen(en->dtype, raw.ptr, dst, count, st));
    PIO_HIP(hipStreamSynchronize(st));   // the scratch returns to the cache after this
    return PIO_OK;
}

// Into a device Tensor: int8 tensors (create_tensor_typed PIO_I8) take I8 / U8
// data as raw bytes; fp16 tensors take F16 raw; fp32 tensors take any dtype
// with an fp32 conversion (done on the GPU). The element counts must match.
PIO_EXPORT int tensor_load_safetensors_status(void* ctx, const char* name, Tensor* out) {
    const StEntry* en;
    PIO_TRY(st_find(ctx, name, en));
    PIO_TRY(check_device_tensor(out, "tensor_load_safetensors out"));
    const int64_t n = st_count(*en);
    PIO_REQUIRE(n == (int64_t)out->size, "tensor_load_safetensors: '%s' has %lld elements, out %d", name,
                (long long)n, out->size);
    const int odt = tensor_dtype_of(out);
    if ((odt == PIO_I8 && (en->dtype == ST_I8 || en->dtype == ST_U8)) || (odt == PIO_F16 && en->dtype == ST_F16))
        return pio_safetensors_to_device(ctx, name, out->data, en->end - en->begin, nullptr);
    PIO_REQUIRE(odt == PIO_F32, "tensor_load_safetensors: cannot load dtype %d into a tensor of type %d", en->dtype, odt);
    return pio_safetensors_to_device_f32(ctx, name, out->data, n, nullptr);
}
PIO_EXPORT void tensor_load_safetensors(void* ctx, const char* name, Tensor* out) {
    tensor_load_safetensors_status(ctx, name, out);
}
