// Per-token symmetric int8 activation quantizer (the path's a7 op; the
// reference has no quantizer, so the definition is this library's):
//   amax[m] = max_k |x[m,k]|            (fp32; fmaxf, so NaNs are skipped)
//   s[m]    = amax[m] / 127.0f           (IEEE division), s = 1 when amax == 0
//   q[m,k]  = clamp(rint(x[m,k] / s[m]), -127, 127)   rint = round-half-even
// Division is the correctly rounded one (hipcc's default for fp32 '/', which
// emits the v_div_scale/v_div_fmas/v_div_fixup sequence), not a reciprocal
// multiply, so the host C restatement reproduces every byte.
//
// One wavefront per token row, 4 rows per 256-thread block. A row is read
// twice (amax pass, quantize pass); the second read hits L2 (a 12288-wide fp16
// row is 24 KB). HBM traffic is one read of x plus the int8 and scale writes.
#include "pio_common.hpp"

namespace pio {

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

__device__ __forceinline__ int8_t quant1(float x, float s) {
    float r = __builtin_rintf(x / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return (int8_t)(int)r;
}

// VEC: K % 8 == 0 and 16-byte aligned rows -> 8 elements per lane per step.
template <typename XT, bool VEC>
__global__ __launch_bounds__(256) void quant_per_token_kernel(const XT* __restrict__ x,
                                                              int8_t* __restrict__ q,
                                                              float* __restrict__ s, int M,
                                                              int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const XT* xr = x + (int64_t)row * K;
    int8_t* qr = q + (int64_t)row * K;

    float amax = 0.f;
    if (VEC) {
        for (int k = lane * 8; k < K; k += 512) {
            float v[8];
            load8<XT>(xr + k, v);
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
        }
    } else {
        for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(to_f32<XT>(xr[k])));
    }
    amax = wave_max(amax);
    const float sc = amax == 0.f ? 1.f : amax / 127.0f;
    if (lane == 0) s[row] = sc;

    if (VEC) {
        for (int k = lane * 8; k < K; k += 512) {
            float v[8];
            load8<XT>(xr + k, v);
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) lo |= (uint32_t)(uint8_t)quant1(v[i], sc) << (8 * i);
#pragma unroll
            for (int i = 0; i < 4; i++) hi |= (uint32_t)(uint8_t)quant1(v[4 + i], sc) << (8 * i);
            *(uint2*)(qr + k) = make_uint2(lo, hi);
        }
    } else {
        for (int k = lane; k < K; k += 64) qr[k] = quant1(to_f32<XT>(xr[k]), sc);
    }
}

int quantize_per_token(const void* x, int x_dtype, int8_t* q, float* s, int M, int K,
                       hipStream_t st) {
    PIO_REQUIRE(x && q && s, "quantize_per_token: null pointer");
    PIO_REQUIRE(M >= 0 && K >= 1, "quantize_per_token: bad shape M=%d K=%d", M, K);
    PIO_REQUIRE(x_dtype == PIO_F32 || x_dtype == PIO_F16,
                "quantize_per_token: x must be fp32 or fp16");
    if (M == 0) return PIO_OK;
    const bool vec = (K % 8 == 0) && aligned16(x) && aligned16(q) &&
                     (x_dtype == PIO_F16 || aligned16(x));
    dim3 grid(ceil_div(M, 4)), block(256);
    if (x_dtype == PIO_F32) {
        if (vec) quant_per_token_kernel<float, true><<<grid, block, 0, st>>>((const float*)x, q, s, M, K);
        else quant_per_token_kernel<float, false><<<grid, block, 0, st>>>((const float*)x, q, s, M, K);
    } else {
        if (vec) quant_per_token_kernel<_Float16, true><<<grid, block, 0, st>>>((const _Float16*)x, q, s, M, K);
        else quant_per_token_kernel<_Float16, false><<<grid, block, 0, st>>>((const _Float16*)x, q, s, M, K);
    }
    PIO_LAUNCHED();
    return PIO_OK;
}

}  // namespace pio

using namespace pio;

PIO_EXPORT int pio_quantize_per_token(const void* x, int x_dtype, int8_t* q, float* s, int M,
                                      int K, void* stream) {
    return quantize_per_token(x, x_dtype, q, s, M, K, pick_stream(stream));
}

PIO_EXPORT int tensor_quantize_per_token_status(Tensor* x, Tensor* q, Tensor* s) {
    PIO_TRY(check_device_tensor(x, "quantize_per_token x"));
    PIO_TRY(check_device_tensor(q, "quantize_per_token q"));
    PIO_TRY(check_device_tensor(s, "quantize_per_token s"));
    const int K = last_dim(x);
    PIO_REQUIRE(K > 0, "quantize_per_token: empty last dim");
    const int M = x->size / K;
    PIO_REQUIRE(q->size == x->size, "quantize_per_token: q has %d elements, x has %d", q->size,
                x->size);
    PIO_REQUIRE(s->size == M, "quantize_per_token: s has %d elements, expected %d", s->size, M);
    PIO_REQUIRE(tensor_dtype_of(q) == PIO_I8 || tensor_dtype_of(q) == PIO_F32,
                "quantize_per_token: q must be int8 storage");
    PIO_REQUIRE(tensor_dtype_of(s) == PIO_F32, "quantize_per_token: s must be fp32");
    return quantize_per_token(x->data, tensor_dtype_of(x), (int8_t*)q->data, s->data, M, K,
                              current_stream());
}
PIO_EXPORT void tensor_quantize_per_token(Tensor* x, Tensor* q, Tensor* s) {
    tensor_quantize_per_token_status(x, q, s);
}
