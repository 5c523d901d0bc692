// Runtime half of libtensor_ops_rocm.so: error channel, streams, graphs, the
// HBM allocator and the reference's required Tensor* exports.
//
// Allocator. The reference CPU backend owns one bump arena (tensor_ops.c:69-133)
// and falls back to aligned malloc; its Python layer allocates every op output
// (backend.py:463), so a decode step creates and frees hundreds of tensors. On a
// GPU each hipMalloc/hipFree is a driver call (hipFree also synchronizes), so
// here device memory goes through a caching allocator: sizes are rounded (256 B
// granules up to 1 MiB, 2 MiB granules above), freed blocks go to an exact-size
// free list and are reused by the next request of that size. init_memory_pool()
// adds the reference's arena on top: while it has room, device tensors are
// bump-allocated from it and freeing them is a no-op (tensor_ops.c:135-162).
// A block remembers the stream it was allocated for and, once freed, is handed
// out again only for that stream: a block freed right after its last kernel
// was enqueued is then safe to reuse, because the next owner's work queues
// behind that kernel. (Blocks move between streams only through
// tensor_empty_cache / an out-of-memory retry, whose hipFree synchronizes.)
// Streams are known to the cache by a generation id, not by their handle: a
// destroyed stream's id is retired (its cached blocks are released after the
// stream drains), so a later stream that receives the same handle value starts
// with an empty cache.
//
// Graph capture. A block freed while its stream is capturing (an op's
// workspace, freed once its kernels are recorded) is still used by every
// replay of the graph being built, so it is not cached: it is parked under the
// capture's id, where only later ops of the same capture on the same stream
// may take it again (the graph orders them after the op that freed it; this
// also keeps a capture of many ops from calling hipMalloc, which some capture
// modes forbid). end_capture hands the parked blocks to the graph it
// instantiates and returns them to the cache only when that graph is replaced
// (their stream then orders any new owner after the old replays). Blocks of
// captures made by other means (the caller's own hipStreamBeginCapture,
// torch.cuda.graph) stay parked for the life of the process, since the library
// cannot see when such a graph dies; tensor_pool_graph_bytes() reports them.
#include "pio_common.hpp"

#include <mutex>
#include <tuple>
#include <map>
#include <unordered_map>
#include <vector>
#include <string.h>
#include <stdio.h>
#include <stdlib.h>

namespace pio {

// ---------------------------------------------------------------- errors ---
static thread_local char t_err[1024];

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof(t_err), fmt, ap);
    va_end(ap);
    if (getenv("PIO_VERBOSE")) fprintf(stderr, "[tensor_ops_rocm] %s\n", t_err);
    return code;
}
void clear_error() { t_err[0] = 0; }

// --------------------------------------------------------------- streams ---
static std::mutex g_mu;
static hipStream_t g_user_stream = nullptr;
static std::map<int, hipStream_t> g_dev_stream;

hipStream_t current_stream() {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_user_stream) return g_user_stream;
    int dev = 0;
    (void)hipGetDevice(&dev);
    auto it = g_dev_stream.find(dev);
    if (it != g_dev_stream.end()) return it->second;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    g_dev_stream[dev] = s;
    return s;
}

// ------------------------------------------------------------- allocator ---
struct Arena {
    char* base = nullptr;
    size_t size = 0;
    size_t used = 0;
};

struct Alloc {
    std::mutex mu;
    struct Live {
        size_t bytes;        // rounded
        int dev;
        hipStream_t stream;  // the stream whose order protects reuse
        uint64_t sid;        // that stream's generation id
    };
    std::unordered_map<void*, Live> live;
    std::unordered_map<void*, int> arena_live;                // ptr -> device
    // (device, rounded bytes, stream id) -> cached blocks
    std::map<std::tuple<int, size_t, uint64_t>, std::vector<void*>> free_lists;
    std::map<int, Arena> arenas;
    std::unordered_map<hipStream_t, uint64_t> stream_ids;     // live streams -> generation id
    uint64_t next_sid = 1;
    // blocks freed during a capture, by capture id; and those the library's
    // own captured graph (begin_capture / end_capture) holds
    std::map<unsigned long long, std::vector<std::pair<void*, Live>>> parked;
    std::vector<std::pair<void*, Live>> graph_held;
    size_t reserved = 0, in_use = 0, cached = 0, peak = 0, n_malloc = 0, held = 0;
};
static Alloc& A() {
    static Alloc* a = new Alloc();   // never destroyed: frees after exit are no-ops
    return *a;
}

static size_t round_bytes(size_t b) {
    if (b == 0) b = 1;
    const size_t small = 256, big = size_t(2) << 20;
    return b <= (size_t(1) << 20) ? (b + small - 1) / small * small : (b + big - 1) / big * big;
}

static uint64_t stream_id_locked(Alloc& a, hipStream_t s) {
    auto it = a.stream_ids.find(s);
    if (it != a.stream_ids.end()) return it->second;
    const uint64_t id = a.next_sid++;
    a.stream_ids[s] = id;
    return id;
}

static void cache_block_locked(Alloc& a, void* p, const Alloc::Live& l) {
    a.cached += l.bytes;
    a.free_lists[std::make_tuple(l.dev, l.bytes, l.sid)].push_back(p);
}

static void empty_cache_locked(Alloc& a) {
    for (auto& kv : a.free_lists) {
        for (void* p : kv.second) {
            int cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(std::get<0>(kv.first));
            (void)hipFree(p);
            (void)hipSetDevice(cur);
            a.reserved -= std::get<1>(kv.first);
            a.cached -= std::get<1>(kv.first);
        }
    }
    a.free_lists.clear();
}

int device_alloc(void** out, size_t bytes, hipStream_t stream) {
    *out = nullptr;
    int dev = 0;
    PIO_HIP(hipGetDevice(&dev));
    if (!stream) stream = current_stream();
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    size_t r = round_bytes(bytes);
    auto ait = a.arenas.find(dev);
    if (ait != a.arenas.end() && ait->second.base) {
        Arena& ar = ait->second;
        size_t off = (ar.used + 255) / 256 * 256;
        if (off + r <= ar.size) {
            *out = ar.base + off;
            ar.used = off + r;
            a.arena_live[*out] = dev;
            return PIO_OK;
        }
    }
    const uint64_t sid = stream_id_locked(a, stream);
    // While the stream captures, first reuse a block an earlier op of the same
    // capture freed: the graph orders that op's kernels before this one's.
    const unsigned long long cid = capture_id(stream);
    if (cid) {
        auto pit = a.parked.find(cid);
        if (pit != a.parked.end()) {
            auto& v = pit->second;
            for (size_t i = 0; i < v.size(); i++) {
                if (v[i].second.bytes != r || v[i].second.sid != sid || v[i].second.dev != dev) continue;
                *out = v[i].first;
                v.erase(v.begin() + (std::ptrdiff_t)i);
                a.held -= r;
                a.live[*out] = {r, dev, stream, sid};
                a.in_use += r;
                if (a.in_use > a.peak) a.peak = a.in_use;
                return PIO_OK;
            }
        }
    }
    auto fit = a.free_lists.find(std::make_tuple(dev, r, sid));
    if (fit != a.free_lists.end() && !fit->second.empty()) {
        *out = fit->second.back();
        fit->second.pop_back();
        a.cached -= r;
    } else {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, r);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            empty_cache_locked(a);
            e = hipMalloc(&p, r);
        }
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return set_error(PIO_ERR_OOM, "hipMalloc(%zu) failed on device %d: %s", r, dev,
                             hipGetErrorString(e));
        }
        a.reserved += r;
        a.n_malloc++;
        *out = p;
    }
    a.live[*out] = {r, dev, stream, sid};
    a.in_use += r;
    if (a.in_use > a.peak) a.peak = a.in_use;
    return PIO_OK;
}

void device_free(void* p) {
    if (!p) return;
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    if (a.arena_live.erase(p)) return;   // pool memory: reclaimed by reset_memory_pool
    auto it = a.live.find(p);
    if (it == a.live.end()) return;
    const Alloc::Live l = it->second;
    a.live.erase(it);
    a.in_use -= l.bytes;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (a.stream_ids.count(l.stream) && a.stream_ids[l.stream] == l.sid &&
        hipStreamGetCaptureInfo(l.stream, &cs, &cid) == hipSuccess &&
        cs == hipStreamCaptureStatusActive) {
        // recorded into a graph that is still being built: keep it out of reach
        // (a capture the runtime invalidated records nothing more, and no
        // graph will run what it recorded)
        a.parked[cid].emplace_back(p, l);
        a.held += l.bytes;
        return;
    }
    (void)hipGetLastError();
    cache_block_locked(a, p, l);
}

unsigned long long capture_id(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (hipStreamGetCaptureInfo(s, &cs, &cid) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return cs == hipStreamCaptureStatusNone ? 0 : cid;
}

// end_capture's hand-over: the blocks parked under capture `cid` now belong to
// the library's graph; the ones the replaced graph held return to the cache.
// When the capture failed (`captured` false) no graph will ever run the
// recorded kernels, so the blocks parked under it return to the cache too.
static void graph_replaced(unsigned long long cid, bool captured) {
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    for (auto& pl : a.graph_held) {
        a.held -= pl.second.bytes;
        cache_block_locked(a, pl.first, pl.second);
    }
    a.graph_held.clear();
    auto it = cid ? a.parked.find(cid) : a.parked.end();
    if (it != a.parked.end()) {
        if (captured) {
            a.graph_held = std::move(it->second);
        } else {
            for (auto& pl : it->second) {
                a.held -= pl.second.bytes;
                cache_block_locked(a, pl.first, pl.second);
            }
        }
        a.parked.erase(it);
    }
}

// Before a stream is destroyed: drain it, release the blocks cached for it and
// retire its id (blocks still live keep the old id and are only reclaimed by
// tensor_empty_cache or an out-of-memory retry once freed).
void release_stream(hipStream_t s) {
    if (!s) return;
    if (hipStreamSynchronize(s) != hipSuccess) (void)hipGetLastError();
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    auto it = a.stream_ids.find(s);
    if (it == a.stream_ids.end()) return;
    const uint64_t sid = it->second;
    a.stream_ids.erase(it);
    int cur = 0;
    (void)hipGetDevice(&cur);
    for (auto f = a.free_lists.begin(); f != a.free_lists.end();) {
        if (std::get<2>(f->first) != sid) {
            ++f;
            continue;
        }
        (void)hipSetDevice(std::get<0>(f->first));
        for (void* p : f->second) {
            (void)hipFree(p);
            a.reserved -= std::get<1>(f->first);
            a.cached -= std::get<1>(f->first);
        }
        f = a.free_lists.erase(f);
    }
    (void)hipSetDevice(cur);
}

// ------------------------------------------------------ tensor metadata ---
struct Meta {
    int dtype;
    size_t bytes;
    bool pinned;   // host tensor in hipHostMalloc memory (create_tensor_pinned)
};
static std::mutex g_meta_mu;
static std::unordered_map<const Tensor*, Meta> g_meta;

int tensor_dtype_of(const Tensor* t) {
    std::lock_guard<std::mutex> lk(g_meta_mu);
    auto it = g_meta.find(t);
    return it == g_meta.end() ? PIO_F32 : it->second.dtype;
}
static bool tensor_pinned_of(const Tensor* t) {
    std::lock_guard<std::mutex> lk(g_meta_mu);
    auto it = g_meta.find(t);
    return it != g_meta.end() && it->second.pinned;
}
static size_t tensor_bytes_of(const Tensor* t) {
    std::lock_guard<std::mutex> lk(g_meta_mu);
    auto it = g_meta.find(t);
    return it == g_meta.end() ? (size_t)t->size * 4 : it->second.bytes;
}

int check_device_tensor(const Tensor* t, const char* what) {
    if (!t) return set_error(PIO_ERR_INVALID, "%s: null tensor", what);
    if (!t->data && t->size > 0) return set_error(PIO_ERR_INVALID, "%s: null data", what);
    if (t->device_id < 0)
        return set_error(PIO_ERR_INVALID, "%s: tensor is on the host (device_id=%d)", what,
                         t->device_id);
    if (t->ndim < 1 || !t->shape) return set_error(PIO_ERR_INVALID, "%s: ndim < 1", what);
    return PIO_OK;
}

// --------------------------------------------------------- small kernels ---
template <typename T>
__global__ void fill_kernel(T* p, int64_t n, T v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}
__global__ void binary_kernel(const float* a, const float* b, float* o, int64_t n, int op) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        o[i] = op == 0 ? a[i] + b[i] : a[i] * b[i];
}

static int grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    if (g < 1) g = 1;
    if (g > 8192) g = 8192;
    return (int)g;
}

}  // namespace pio

using namespace pio;

// ======================================================== exported C ABI ===

PIO_EXPORT const char* tensor_last_error(void) { return t_err; }
PIO_EXPORT void tensor_clear_error(void) { clear_error(); }

PIO_EXPORT const char* pio_version(void) {
    return "libtensor_ops_rocm 0.1 (gfx950, int8 quantized-linear path)";
}

static Tensor* make_tensor(const int* shape, int ndim, int device_id, int dtype, bool pinned = false) {
    if (ndim < 0 || (ndim > 0 && !shape)) {
        set_error(PIO_ERR_INVALID, "create_tensor: bad ndim %d", ndim);
        return nullptr;
    }
    size_t eb = dtype_bytes(dtype);
    if (!eb) {
        set_error(PIO_ERR_INVALID, "create_tensor: bad dtype %d", dtype);
        return nullptr;
    }
    int64_t n = 1;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] < 0) {
            set_error(PIO_ERR_INVALID, "create_tensor: negative dim");
            return nullptr;
        }
        n *= shape[i];
    }
    if (n > INT32_MAX) {
        set_error(PIO_ERR_INVALID, "create_tensor: %lld elements exceed the int size field",
                  (long long)n);
        return nullptr;
    }
    Tensor* t = (Tensor*)calloc(1, sizeof(Tensor));
    if (!t) return nullptr;
    t->ndim = ndim;
    t->shape = (int*)malloc(sizeof(int) * (ndim > 0 ? ndim : 1));
    if (!t->shape) {
        free(t);
        return nullptr;
    }
    for (int i = 0; i < ndim; i++) t->shape[i] = shape[i];
    t->size = (int)n;
    t->device_id = device_id;
    size_t bytes = (size_t)n * eb;
    if (device_id >= 0) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (cur != device_id && hipSetDevice(device_id) != hipSuccess) {
            set_error(PIO_ERR_INVALID, "create_tensor: no device %d", device_id);
            free(t->shape);
            free(t);
            return nullptr;
        }
        void* p = nullptr;
        if (device_alloc(&p, bytes) != PIO_OK) {
            free(t->shape);
            free(t);
            return nullptr;
        }
        t->data = (float*)p;
    } else if (pinned) {
        void* p = nullptr;
        if (hipHostMalloc(&p, bytes ? bytes : 64, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            set_error(PIO_ERR_OOM, "create_tensor_pinned: hipHostMalloc of %zu bytes failed", bytes);
            free(t->shape);
            free(t);
            return nullptr;
        }
        t->data = (float*)p;
    } else {
        size_t hb = (bytes + 63) / 64 * 64;
        t->data = (float*)aligned_alloc(64, hb ? hb : 64);
        if (!t->data) {
            set_error(PIO_ERR_OOM, "create_tensor: host alloc of %zu bytes failed", bytes);
            free(t->shape);
            free(t);
            return nullptr;
        }
    }
    {
        std::lock_guard<std::mutex> lk(g_meta_mu);
        g_meta[t] = Meta{dtype, bytes, pinned && device_id < 0};
    }
    return t;
}

PIO_EXPORT Tensor* create_tensor(int* shape, int ndim, int device_id) {
    return make_tensor(shape, ndim, device_id, PIO_F32);
}
PIO_EXPORT Tensor* create_tensor_typed(int* shape, int ndim, int device_id, int dtype) {
    return make_tensor(shape, ndim, device_id, dtype);
}
PIO_EXPORT Tensor* create_tensor_pinned(int* shape, int ndim, int dtype) {
    return make_tensor(shape, ndim, -1, dtype, true);
}
PIO_EXPORT int tensor_dtype(Tensor* t) { return tensor_dtype_of(t); }

PIO_EXPORT void free_tensor(Tensor* t) {
    if (!t) return;
    bool ours = false, pinned = false;
    {
        std::lock_guard<std::mutex> lk(g_meta_mu);
        auto it = g_meta.find(t);
        if (it != g_meta.end()) {
            ours = true;
            pinned = it->second.pinned;
            g_meta.erase(it);
        }
    }
    if (ours && t->data) {
        if (t->device_id >= 0) device_free(t->data);
        else if (pinned) (void)hipHostFree(t->data);
        else free(t->data);
    }
    if (ours) {
        free(t->shape);
        free(t);
    }
}

static int fill_impl(Tensor* t, float v) {
    if (!t) return set_error(PIO_ERR_INVALID, "tensor_fill: null tensor");
    int dt = tensor_dtype_of(t);
    int64_t n = t->size;
    if (t->device_id < 0) {
        for (int64_t i = 0; i < n; i++) {
            if (dt == PIO_F32) t->data[i] = v;
            else return set_error(PIO_ERR_UNSUPPORTED, "tensor_fill: host fill needs fp32");
        }
        return PIO_OK;
    }
    if (n == 0) return PIO_OK;
    hipStream_t s = current_stream();
    switch (dt) {
    case PIO_F32: fill_kernel<float><<<grid_for(n), 256, 0, s>>>(t->data, n, v); break;
    case PIO_F16:
        fill_kernel<_Float16><<<grid_for(n), 256, 0, s>>>((_Float16*)t->data, n, (_Float16)v);
        break;
    case PIO_I8: {
        float c = v > 127.f ? 127.f : (v < -128.f ? -128.f : v);
        fill_kernel<int8_t><<<grid_for(n), 256, 0, s>>>((int8_t*)t->data, n, (int8_t)(int)c);
        break;
    }
    case PIO_I32:
        fill_kernel<int32_t><<<grid_for(n), 256, 0, s>>>((int32_t*)t->data, n, (int32_t)v);
        break;
    default: return set_error(PIO_ERR_INVALID, "tensor_fill: bad dtype");
    }
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_fill(Tensor* t, float value) { fill_impl(t, value); }

static int binary_impl(Tensor* a, Tensor* b, Tensor* o, int op) {
    const char* nm = op == 0 ? "tensor_add" : "tensor_mul";
    PIO_REQUIRE(a && b && o, "%s: null tensor", nm);
    PIO_REQUIRE(a->size >= o->size && b->size >= o->size, "%s: operands smaller than out", nm);
    if (o->device_id < 0) {
        PIO_REQUIRE(a->device_id < 0 && b->device_id < 0, "%s: device mismatch", nm);
        for (int i = 0; i < o->size; i++)
            o->data[i] = op == 0 ? a->data[i] + b->data[i] : a->data[i] * b->data[i];
        return PIO_OK;
    }
    PIO_REQUIRE(a->device_id == o->device_id && b->device_id == o->device_id,
                "%s: device mismatch", nm);
    if (o->size == 0) return PIO_OK;
    binary_kernel<<<grid_for(o->size), 256, 0, current_stream()>>>(a->data, b->data, o->data,
                                                                    o->size, op);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_add(Tensor* a, Tensor* b, Tensor* out) { binary_impl(a, b, out, 0); }
PIO_EXPORT void tensor_mul(Tensor* a, Tensor* b, Tensor* out) { binary_impl(a, b, out, 1); }

static int copy_bytes(Tensor* t, void* host, size_t nbytes, bool h2d) {
    PIO_REQUIRE(t && (host || nbytes == 0), "tensor copy: null argument");
    size_t cap = tensor_bytes_of(t);
    PIO_REQUIRE(nbytes <= cap, "tensor copy: %zu bytes exceed the tensor's %zu", nbytes, cap);
    if (nbytes == 0) return PIO_OK;
    if (t->device_id < 0) {
        if (h2d) memcpy(t->data, host, nbytes);
        else memcpy(host, t->data, nbytes);
        return PIO_OK;
    }
    hipStream_t s = current_stream();
    if (h2d) PIO_HIP(hipMemcpyAsync(t->data, host, nbytes, hipMemcpyHostToDevice, s));
    else PIO_HIP(hipMemcpyAsync(host, t->data, nbytes, hipMemcpyDeviceToHost, s));
    PIO_HIP(hipStreamSynchronize(s));
    return PIO_OK;
}

PIO_EXPORT void tensor_load_data(Tensor* t, float* buffer, int size) {
    copy_bytes(t, buffer, size > 0 ? (size_t)size * 4 : 0, true);
}
PIO_EXPORT void tensor_get_data(Tensor* t, float* buffer, int size) {
    copy_bytes(t, buffer, size > 0 ? (size_t)size * 4 : 0, false);
}
PIO_EXPORT int tensor_load_bytes_status(Tensor* t, const void* src, size_t nbytes) {
    return copy_bytes(t, (void*)src, nbytes, true);
}
PIO_EXPORT int tensor_get_bytes_status(Tensor* t, void* dst, size_t nbytes) {
    return copy_bytes(t, dst, nbytes, false);
}
PIO_EXPORT void tensor_load_bytes(Tensor* t, const void* src, size_t nbytes) {
    tensor_load_bytes_status(t, src, nbytes);
}
PIO_EXPORT void tensor_get_bytes(Tensor* t, void* dst, size_t nbytes) {
    tensor_get_bytes_status(t, dst, nbytes);
}

// ------------------------------------------------------------ pool / stats ---
PIO_EXPORT void init_memory_pool(size_t size_bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error(PIO_ERR_HIP, "init_memory_pool: no device");
        return;
    }
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    Arena& ar = a.arenas[dev];
    if (ar.base) return;   // already initialised (tensor_ops.c:75)
    void* p = nullptr;
    if (hipMalloc(&p, size_bytes) != hipSuccess) {
        (void)hipGetLastError();
        set_error(PIO_ERR_OOM, "init_memory_pool: hipMalloc(%zu) failed", size_bytes);
        return;
    }
    ar.base = (char*)p;
    ar.size = size_bytes;
    ar.used = 0;
}

PIO_EXPORT void reset_memory_pool(void) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    auto it = a.arenas.find(dev);
    if (it == a.arenas.end()) return;
    it->second.used = 0;
    for (auto i = a.arena_live.begin(); i != a.arena_live.end();)
        i = i->second == dev ? a.arena_live.erase(i) : std::next(i);
}

PIO_EXPORT void tensor_pool_stats(size_t* s) {
    if (!s) return;
    int dev = 0;
    (void)hipGetDevice(&dev);
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    s[0] = a.reserved;
    s[1] = a.in_use;
    s[2] = a.cached;
    s[3] = a.peak;
    s[4] = a.n_malloc;
    auto it = a.arenas.find(dev);
    s[5] = it == a.arenas.end() ? 0 : it->second.size;
    s[6] = it == a.arenas.end() ? 0 : it->second.used;
}

PIO_EXPORT size_t tensor_pool_graph_bytes(void) {
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    return a.held;
}

PIO_EXPORT void tensor_empty_cache(void) {
    Alloc& a = A();
    std::lock_guard<std::mutex> lk(a.mu);
    empty_cache_locked(a);
}

PIO_EXPORT void* allocate_pinned_memory(size_t size) {
    void* p = nullptr;
    if (hipHostMalloc(&p, size ? size : 1, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        set_error(PIO_ERR_OOM, "allocate_pinned_memory(%zu) failed", size);
        return nullptr;
    }
    return p;
}
PIO_EXPORT void free_pinned_memory(void* ptr) {
    if (ptr) (void)hipHostFree(ptr);
}

// ---------------------------------------------------------------- streams ---
PIO_EXPORT void* create_stream(void) {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        set_error(PIO_ERR_HIP, "create_stream failed");
        return nullptr;
    }
    return (void*)s;
}
PIO_EXPORT void destroy_stream(void* s) {
    if (!s) return;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (g_user_stream == (hipStream_t)s) g_user_stream = nullptr;
    }
    release_stream((hipStream_t)s);
    if (hipStreamDestroy((hipStream_t)s) != hipSuccess) (void)hipGetLastError();
}
PIO_EXPORT void stream_synchronize(void* s) {
    // a failure here (e.g. a synchronize while the stream captures) must not
    // stay behind as the runtime's last error for the next launch check
    if (hipStreamSynchronize(s ? (hipStream_t)s : current_stream()) != hipSuccess) (void)hipGetLastError();
}
PIO_EXPORT void set_current_stream(void* s) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_user_stream = (hipStream_t)s;
}
PIO_EXPORT void* get_current_stream(void) { return (void*)current_stream(); }

// Copies src's bytes into dst (same byte size; host or device on either side)
// on `stream` (NULL: the current stream) without waiting. Host memory must stay
// untouched until the copy is done: record an event after it, or synchronize.
// With a pinned host tensor (create_tensor_pinned) the copy is a DMA that
// overlaps kernels on other streams; pageable host memory makes it synchronous.
PIO_EXPORT int tensor_copy_async(Tensor* dst, Tensor* src, void* stream) {
    PIO_REQUIRE(dst && src, "tensor_copy_async: null tensor");
    const size_t nb = tensor_bytes_of(src);
    PIO_REQUIRE(tensor_bytes_of(dst) == nb, "tensor_copy_async: %zu bytes into a tensor of %zu",
                nb, tensor_bytes_of(dst));
    PIO_REQUIRE(tensor_dtype_of(dst) == tensor_dtype_of(src), "tensor_copy_async: dtype mismatch");
    if (nb == 0) return PIO_OK;
    PIO_REQUIRE(dst->data && src->data, "tensor_copy_async: null data");
    const hipStream_t s = pick_stream(stream);
    const bool hd = dst->device_id >= 0, hs = src->device_id >= 0;
    const hipMemcpyKind kind = hs ? (hd ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost)
                                  : (hd ? hipMemcpyHostToDevice : hipMemcpyHostToHost);
    PIO_HIP(hipMemcpyAsync(dst->data, src->data, nb, kind, s));
    return PIO_OK;
}
PIO_EXPORT int tensor_is_pinned(Tensor* t) { return t && tensor_pinned_of(t) ? 1 : 0; }

// ----------------------------------------------------------------- events ---
// Ordering between streams (a transfer stream and a compute stream): record
// on one, wait on another. Events are created without timing.
PIO_EXPORT void* create_event(void) {
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        set_error(PIO_ERR_HIP, "create_event failed");
        return nullptr;
    }
    return (void*)e;
}
PIO_EXPORT void destroy_event(void* e) {
    if (e) (void)hipEventDestroy((hipEvent_t)e);
}
PIO_EXPORT int record_event(void* e, void* stream) {
    PIO_REQUIRE(e, "record_event: null event");
    PIO_HIP(hipEventRecord((hipEvent_t)e, pick_stream(stream)));
    return PIO_OK;
}
PIO_EXPORT int stream_wait_event(void* stream, void* e) {
    PIO_REQUIRE(e, "stream_wait_event: null event");
    PIO_HIP(hipStreamWaitEvent(pick_stream(stream), (hipEvent_t)e, 0));
    return PIO_OK;
}
PIO_EXPORT int event_synchronize(void* e) {
    PIO_REQUIRE(e, "event_synchronize: null event");
    PIO_HIP(hipEventSynchronize((hipEvent_t)e));
    return PIO_OK;
}
PIO_EXPORT int event_query(void* e) {
    PIO_REQUIRE(e, "event_query: null event");
    const hipError_t r = hipEventQuery((hipEvent_t)e);
    if (r == hipSuccess) return 1;
    if (r == hipErrorNotReady) {
        (void)hipGetLastError();
        return 0;
    }
    return set_error(PIO_ERR_HIP, "event_query: %s", hipGetErrorString(r));
}
PIO_EXPORT void device_synchronize(void) { (void)hipDeviceSynchronize(); }

// ----------------------------------------------------------------- graphs ---
// One captured graph per process, matching the reference wrapper's
// begin_capture/end_capture/replay_graph (backend.py:801-810).
static hipGraph_t g_graph = nullptr;
static hipGraphExec_t g_graph_exec = nullptr;
static hipStream_t g_capture_stream = nullptr;
// id of the capture begin_capture started: taken at the start, since a capture
// the runtime has invalidated may no longer report it
static unsigned long long g_capture_cid = 0;

PIO_EXPORT void begin_capture(void) {
    g_capture_stream = current_stream();
    g_capture_cid = 0;
    if (hipStreamBeginCapture(g_capture_stream, hipStreamCaptureModeRelaxed) != hipSuccess)
        set_error(PIO_ERR_HIP, "begin_capture failed");
    else
        g_capture_cid = capture_id(g_capture_stream);
}
PIO_EXPORT void end_capture(void) {
    if (!g_capture_stream) return;
    const unsigned long long cid = g_capture_cid;
    g_capture_cid = 0;
    if (g_graph_exec) {
        (void)hipGraphExecDestroy(g_graph_exec);
        g_graph_exec = nullptr;
    }
    if (g_graph) {
        (void)hipGraphDestroy(g_graph);
        g_graph = nullptr;
    }
    if (hipStreamEndCapture(g_capture_stream, &g_graph) != hipSuccess) {
        (void)hipGetLastError();
        set_error(PIO_ERR_HIP, "end_capture failed");
        g_graph = nullptr;
        graph_replaced(cid, false);
        return;
    }
    graph_replaced(cid, true);
    if (hipGraphInstantiate(&g_graph_exec, g_graph, nullptr, nullptr, 0) != hipSuccess)
        set_error(PIO_ERR_HIP, "hipGraphInstantiate failed");
}
PIO_EXPORT void replay_graph(void) {
    if (!g_graph_exec) {
        set_error(PIO_ERR_INVALID, "replay_graph: nothing captured");
        return;
    }
    if (hipGraphLaunch(g_graph_exec, g_capture_stream) != hipSuccess)
        set_error(PIO_ERR_HIP, "hipGraphLaunch failed");
}
