// Internal helpers shared by the HIP translation units of libtensor_ops_rocm.so.
// gfx950 only: wave64, int8 MFMA, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>
#include <stdarg.h>

#include <atomic>

#include "tensor_rocm.h"

#define PIO_EXPORT extern "C" __attribute__((visibility("default")))

namespace pio {

// ---- error channel -------------------------------------------------------
// Records a printf-style message for tensor_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Wraps a HIP call; on failure records the HIP error string and returns.
#define PIO_HIP(call)                                                                      \
    do {                                                                                   \
        hipError_t _e = (call);                                                            \
        if (_e != hipSuccess)                                                              \
            return ::pio::set_error(PIO_ERR_HIP, "%s failed: %s (%s:%d)", #call,           \
                                    hipGetErrorString(_e), __FILE__, __LINE__);            \
    } while (0)

#define PIO_REQUIRE(cond, ...)                                                             \
    do {                                                                                   \
        if (!(cond)) return ::pio::set_error(PIO_ERR_INVALID, __VA_ARGS__);                \
    } while (0)

// Propagates a non-OK status.
#define PIO_TRY(...)                                                                       \
    do {                                                                                   \
        int _s = (__VA_ARGS__);                                                            \
        if (_s != PIO_OK) return _s;                                                       \
    } while (0)

// Checks the launch status of the kernel just issued.
#define PIO_LAUNCHED() PIO_HIP(hipGetLastError())

// Raises KERNEL's dynamic-LDS limit above the 64 KB default to what a launch
// asks for, per device and only when it grows (one entry per kernel: the
// template argument is the kernel itself, not its type). The limit is the
// dynamic bytes, so a kernel with static LDS cannot ask for the whole 160 KB.
template <auto KERNEL>
inline int allow_lds(size_t bytes) {
    static std::atomic<uint32_t> set_to[64];
    if (bytes <= 65536) return PIO_OK;
    int dev = 0;
    PIO_HIP(hipGetDevice(&dev));
    std::atomic<uint32_t>& cur = set_to[dev & 63];
    if (cur.load(std::memory_order_acquire) >= bytes) return PIO_OK;
    PIO_HIP(hipFuncSetAttribute((const void*)KERNEL, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    uint32_t seen = cur.load(std::memory_order_relaxed);
    while (seen < bytes && !cur.compare_exchange_weak(seen, (uint32_t)bytes, std::memory_order_release)) {
    }
    return PIO_OK;
}

// ---- streams -------------------------------------------------------------
// The stream raw entry points run on when given NULL: the one set by
// set_current_stream(), else the library's own in-order stream for the
// current device (created on first use, default priority).
hipStream_t current_stream();
inline hipStream_t pick_stream(void* s) { return s ? (hipStream_t)s : current_stream(); }

// ---- dtypes --------------------------------------------------------------
inline size_t dtype_bytes(int dt) {
    switch (dt) {
    case PIO_F32: return 4;
    case PIO_F16: return 2;
    case PIO_I8: return 1;
    case PIO_I32: return 4;
    default: return 0;
    }
}

// ---- device allocation (caching allocator, runtime.hip) -------------------
// On the current device. A freed block is cached and handed out again only
// to a request for the same stream (`stream`, NULL = the current stream), so
// stream order makes the reuse safe: the new owner's work is queued behind
// the old owner's last kernel.
int device_alloc(void** p, size_t bytes, hipStream_t stream = nullptr);
// Back to the cache (a no-op for pool memory). A block whose stream is
// capturing is parked with the capture instead: the graph keeps using it.
void device_free(void* p);
// Drains `s`, releases the blocks cached for it and retires its cache id; call
// before destroying a stream the library created.
void release_stream(hipStream_t s);
// Id of the capture `s` is recording (0 when it is not capturing).
unsigned long long capture_id(hipStream_t s);

// Scoped device scratch from the caching allocator, for work queued on `st`;
// freed when the scope ends, possibly while that work is still running.
struct Scratch {
    void* ptr = nullptr;
    ~Scratch() { if (ptr) device_free(ptr); }
    int get(size_t bytes, hipStream_t st) { return bytes ? device_alloc(&ptr, bytes, st) : PIO_OK; }
};

// ---- Tensor metadata -------------------------------------------------------
// Element type the tensor was created with (PIO_F32 for create_tensor and for
// tensors this library did not create).
int tensor_dtype_of(const Tensor* t);
inline int64_t numel(const Tensor* t) { return t ? (int64_t)t->size : 0; }
inline int last_dim(const Tensor* t) { return t->shape[t->ndim - 1]; }

// Validates a device tensor argument.
int check_device_tensor(const Tensor* t, const char* what);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---- device helpers --------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---- wave reductions on the VALU (DPP and readlane), without the LDS queue
// that __shfl's ds_bpermute uses.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rlane(float x, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), i));
}
enum : int {
    DPP_XOR1 = 0xB1,       // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,       // quad_perm [2,3,0,1]
    DPP_ROR8 = 0x128,      // row_ror:8 (lane i <- lane i^8 within a 16-lane row)
    DPP_MIRROR = 0x140,    // row_mirror (i <- 15-i)
    DPP_HMIRROR = 0x141,   // row_half_mirror (i <- 7-i within 8)
};
// Sum over each group of 8 consecutive lanes, in every lane of the group.
__device__ __forceinline__ float sum8(float x) {
    x += dpp<DPP_XOR1>(x);
    x += dpp<DPP_XOR2>(x);
    return x + dpp<DPP_HMIRROR>(x);
}
// Sum over all 64 lanes (same value, bit for bit, in every lane).
__device__ __forceinline__ float wsum(float x) {
    x = sum8(x);
    x += dpp<DPP_MIRROR>(x);
    return (rlane(x, 0) + rlane(x, 16)) + (rlane(x, 32) + rlane(x, 48));
}
__device__ __forceinline__ float wmax(float x) {
    x = fmaxf(x, dpp<DPP_XOR1>(x));
    x = fmaxf(x, dpp<DPP_XOR2>(x));
    x = fmaxf(x, dpp<DPP_HMIRROR>(x));
    x = fmaxf(x, dpp<DPP_MIRROR>(x));
    return fmaxf(fmaxf(rlane(x, 0), rlane(x, 16)), fmaxf(rlane(x, 32), rlane(x, 48)));
}

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<_Float16>(_Float16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
// v_cvt_f16_f32 under the default round-to-nearest-even mode.
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

template <typename XT>
__device__ __forceinline__ void load8(const XT* p, float (&v)[8]);
template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
    float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <>
__device__ __forceinline__ void load8<_Float16>(const _Float16* p, float (&v)[8]) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 h = *(const h8*)p;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)h[i];
}

// The same 8 elements as raw bits, widened later: a load whose conversion
// follows at once inside a (guarded or unrolled) branch waits for that load
// before the next one issues; loading every group's raw bits first keeps all
// the loads in flight together.
template <typename XT>
struct Raw8 {
    uint4 u[sizeof(XT) / 2];
};
template <typename XT>
__device__ __forceinline__ Raw8<XT> raw8_load(const XT* p) {
    Raw8<XT> r;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(XT) / 2); i++) r.u[i] = ((const uint4*)p)[i];
    return r;
}
template <typename XT>
__device__ __forceinline__ void raw8_widen(const Raw8<XT>& r, float (&v)[8]) {
    if constexpr (sizeof(XT) == 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = __uint_as_float(((const uint32_t*)&r.u[0])[i]);
            v[4 + i] = __uint_as_float(((const uint32_t*)&r.u[1])[i]);
        }
    } else {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 h = __builtin_bit_cast(h8, r.u[0]);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)h[i];
    }
}

// Per-token quantizer step: clamp(rint(x / s), -127, 127), IEEE division,
// round-half-even.
__device__ __forceinline__ int8_t quant1(float x, float s) {
    float r = __builtin_rintf(x / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return (int8_t)(int)r;
}


// e^x by a fixed sequence of IEEE fp32 operations (Cody-Waite reduction by
// ln2 in two parts, degree-7 Taylor polynomial in Horner form with explicit
// fmaf, scaling by ldexp), so that the host oracle's identical C function
// gives the same bits: within 2 ulp of e^x, exact 1 at 0, +inf above the
// overflow bound, +0 below -103.98, NaN propagated. The MoE SwiGLU uses it
// where a last-ulp difference of expf between libm and the device library
// could move a requantized byte.
__device__ __forceinline__ float exp_det(float x) {
    if (!(x < 88.72283935546875f)) return x != x ? x : __builtin_inff();
    if (x < -103.97208f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.428606765330187045e-06f, r);
    float p = 1.98412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333377e-3f);
    p = __builtin_fmaf(p, r, 4.16666679e-2f);
    p = __builtin_fmaf(p, r, 1.66666672e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

}  // namespace pio
