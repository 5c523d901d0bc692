// Per-token symmetric int8 activation quantizer (the path's a7 op; the
// reference has no quantizer, so the definition is this library's):
//   amax[m] = max_k |x[m,k]|            (fp32; fmaxf, so NaNs are skipped)
//   s[m]    = amax[m] / 127.0f           (IEEE division), s = 1 when amax == 0
//   q[m,k]  = clamp(rint(x[m,k] / s[m]), -127, 127)   rint = round-half-even
// Division is the correctly rounded one (hipcc's default for fp32 '/', which
// emits the v_div_scale/v_div_fmas/v_div_fixup sequence), not a reciprocal
// multiply, so the host C restatement reproduces every byte.
//
// Few rows (M < 1024, K % 8 == 0, K <= 32768): a 256-thread block per row;
// each thread loads its up to 16 groups of 8 values once, all loads issued
// before the row maximum is reduced, and quantizes from registers. Other
// shapes: one wave per row in two passes (the second read hits L2).
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

template <typename XT, int TPR, int NV>
__global__ __launch_bounds__(256) void quant_rows_reg_kernel(const XT* __restrict__ x,
                                                             int8_t* __restrict__ q,
                                                             float* __restrict__ s, int M, int K) {
    constexpr int RPB = 256 / TPR;   // rows per block
    __shared__ float red[4];
    const int t = threadIdx.x % TPR;
    const int row = blockIdx.x * RPB + threadIdx.x / TPR;
    const bool live = row < M;   // (the block-wide reduction below needs every thread)
    const XT* xr = x + (int64_t)min(row, M - 1) * K;
    float v[NV][8];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k = (t + TPR * j) * 8;
        if (k < K) {
            load8<XT>(xr + k, v[j]);
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[j][i]));
        }
    }
    amax = wave_max(amax);
    if constexpr (TPR == 256) {
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
    if (!live) return;
    const float sc = amax == 0.f ? 1.f : amax / 127.0f;
    if (t == 0) s[row] = sc;
    int8_t* qr = q + (int64_t)row * K;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int k = (t + TPR * j) * 8;
        if (k < K) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) lo |= (uint32_t)(uint8_t)quant1(v[j][i], sc) << (8 * i);
#pragma unroll
            for (int i = 0; i < 4; i++) hi |= (uint32_t)(uint8_t)quant1(v[j][4 + i], sc) << (8 * i);
            *(uint2*)(qr + k) = make_uint2(lo, hi);
        }
    }
}

// Register path launch: TPR threads per row, NV = the groups of 8 a thread
// holds, rounded up to a power of two (<= 16); false if K does not fit.
template <typename XT, int TPR>
static bool launch_reg(const XT* x, int8_t* q, float* s, int M, int K, hipStream_t st) {
    const int nv = ceil_div(K, TPR * 8);
    const dim3 grid(ceil_div(M, 256 / TPR)), block(256);
    if (nv <= 1) quant_rows_reg_kernel<XT, TPR, 1><<<grid, block, 0, st>>>(x, q, s, M, K);
    else if (nv <= 2) quant_rows_reg_kernel<XT, TPR, 2><<<grid, block, 0, st>>>(x, q, s, M, K);
    else if (nv <= 4) quant_rows_reg_kernel<XT, TPR, 4><<<grid, block, 0, st>>>(x, q, s, M, K);
    else if (nv <= 8) quant_rows_reg_kernel<XT, TPR, 8><<<grid, block, 0, st>>>(x, q, s, M, K);
    else if (nv <= 16) quant_rows_reg_kernel<XT, TPR, 16><<<grid, block, 0, st>>>(x, q, s, M, K);
    else return false;
    return true;
}

// Few rows (a wave per row would leave most CUs without work): a block per
// row on the register path. Many rows: the two-pass kernel, which measured
// faster there (2048 x 3072 fp16: 7.6 vs 8.2 us).
template <typename XT>
static bool launch_reg_any(const XT* x, int8_t* q, float* s, int M, int K, hipStream_t st) {
    if (M < 1024) return launch_reg<XT, 256>(x, q, s, M, K, st);
    return false;
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
    if (vec) {
        const bool done = x_dtype == PIO_F32 ? launch_reg_any((const float*)x, q, s, M, K, st)
                                             : launch_reg_any((const _Float16*)x, q, s, M, K, st);
        if (done) {
            PIO_LAUNCHED();
            return PIO_OK;
        }
    }
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
