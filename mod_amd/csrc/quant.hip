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
        // U chunks of 8 per lane per batch, raw bits loaded together at
        // clamped offsets (a load-and-convert per loop trip waits for each
        // load in turn); a row of up to 64 U chunks stays in registers and is
        // quantized from them, a longer one is read again in the second pass
        constexpr int U = 8;
        const int nch = K / 8;
        for (int c0 = 0; c0 < nch; c0 += 64 * U) {
            Raw8<XT> raw[U];
#pragma unroll
            for (int u = 0; u < U; u++) raw[u] = raw8_load(xr + 8 * min(c0 + lane + 64 * u, nch - 1));
            float v[U][8];
#pragma unroll
            for (int u = 0; u < U; u++) {
                raw8_widen(raw[u], v[u]);
                if (c0 + lane + 64 * u < nch)
#pragma unroll
                    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[u][i]));
            }
            if (nch <= 64 * U) {   // the whole row is in v: quantize it from there
                amax = wave_max(amax);
                const float sc = amax == 0.f ? 1.f : amax / 127.0f;
                if (lane == 0) s[row] = sc;
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int c = lane + 64 * u;
                    if (c < nch) {
                        uint32_t lo = 0, hi = 0;
#pragma unroll
                        for (int i = 0; i < 4; i++) lo |= (uint32_t)(uint8_t)quant1(v[u][i], sc) << (8 * i);
#pragma unroll
                        for (int i = 0; i < 4; i++) hi |= (uint32_t)(uint8_t)quant1(v[u][4 + i], sc) << (8 * i);
                        *(uint2*)(qr + 8 * c) = make_uint2(lo, hi);
                    }
                }
                return;
            }
        }
    } else {
        for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(to_f32<XT>(xr[k])));
    }
    amax = wave_max(amax);
    const float sc = amax == 0.f ? 1.f : amax / 127.0f;
    if (lane == 0) s[row] = sc;

    if (VEC) {   // rows longer than 64 U chunks: second pass
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
    // every group's raw bits first, at clamped offsets (a load guarded by its
    // own branch and widened at once waits before the next one issues)
    Raw8<XT> raw[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) raw[j] = raw8_load(xr + min((t + TPR * j) * 8, K - 8));
    float v[NV][8];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        raw8_widen(raw[j], v[j]);
        if ((t + TPR * j) * 8 < K)
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[j][i]));
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


// ------------------------------------------ RMSNorm -> per-token quantizer
// The producer of a W8A8 linear's input in a prefill layer: RMSNorm
// (tensor_ops.c:369-383), optionally after the residual add of
// tensor_fused_add_rms_norm (tensor_ops_opencl.c:676-691), and the per-token
// quantizer above, in one pass over the row. Per row (K % 8 == 0):
//   v[k]  = x[k] (+ r[k], fp32 add, stored back in x's dtype; v is the stored value)
//   ss    = sum of v[k]^2 in one fixed order: chunk c = v[8c .. 8c+7], its
//           partial P[c] = fmaf(v, v, P) over the chunk in k order from 0;
//           P zero-padded to n = the next power of two >= K/8 chunks, then
//           for h = n/2, n/4, .., 1: P[c] += P[c + h] for c < h; ss = P[0]
//   scale = 1.0f / sqrtf(ss / K + eps)     (IEEE division and square root)
//   y[k]  = v[k] * scale * w[k]           (two roundings, in that order)
//   s, q  = the per-token quantizer of y
// The reference sums the squares in OpenMP's order, which no other
// implementation can reproduce; the pairwise order is this library's
// definition (the host restatement follows it, so q and s are bit-exact).
// Layout: T threads per row (64, 128 or 256; 256 / T rows per block); thread
// t holds chunks t + T i (i < n / T), so the tree levels h >= T run inside a
// thread, h = T/2 .. 64 through LDS and h = 32 .. 1 as a wave butterfly
// (lane t gets P[t] + P[t ^ h], which for t < h is the tree's P[t] + P[t + h]).
template <typename XT>
__device__ __forceinline__ void store8(XT* p, const float (&v)[8]);
template <>
__device__ __forceinline__ void store8<float>(float* p, const float (&v)[8]) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
template <>
__device__ __forceinline__ void store8<_Float16>(_Float16* p, const float (&v)[8]) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
    *(h8*)p = h;
}

template <typename XT, int T, int NV, bool RES>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const XT* __restrict__ x,
                                                            const XT* __restrict__ r,
                                                            XT* __restrict__ xs,
                                                            const float* __restrict__ w,
                                                            int8_t* __restrict__ q,
                                                            float* __restrict__ s, int M, int K,
                                                            float eps) {
    constexpr int RPB = 256 / T;
    __shared__ float red[256];
    __shared__ float bc[RPB][2];
    const int t = threadIdx.x % T, rg = threadIdx.x / T;
    const int row = blockIdx.x * RPB + rg;
    const bool live = row < M;                 // every thread joins the reductions
    const int64_t base = (int64_t)min(row, M - 1) * K;
    const int nch = K / 8;
    // every chunk's raw bits first, at clamped offsets (loads guarded by
    // their own branch would wait one by one)
    Raw8<XT> rx[NV], rr[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int cc = min(t + T * i, nch - 1);
        rx[i] = raw8_load(x + base + 8 * cc);
        if (RES) rr[i] = raw8_load(r + base + 8 * cc);
    }
    float v[NV][8];
    float part[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = t + T * i;
        part[i] = 0.f;
        if (c < nch) {
            raw8_widen(rx[i], v[i]);
            if (RES) {
                float rv[8];
                raw8_widen(rr[i], rv);
#pragma unroll
                for (int e = 0; e < 8; e++) v[i][e] = to_f32<XT>(from_f32<XT>(v[i][e] + rv[e]));
                if (live) store8<XT>(xs + base + 8 * c, v[i]);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) part[i] = __builtin_fmaf(v[i][e], v[i][e], part[i]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) v[i][e] = 0.f;
        }
    }
    // tree levels h >= T: inside the thread (chunk t + T i pairs with t + T (i + h/T))
#pragma unroll
    for (int hs = NV / 2; hs >= 1; hs >>= 1)
#pragma unroll
        for (int i = 0; i < hs; i++) part[i] += part[i + hs];
    float ss = part[0];
    // levels T/2 .. 64 through LDS
    if constexpr (T > 64) {
        float* rr = red + rg * T;
#pragma unroll
        for (int h = T / 2; h >= 64; h >>= 1) {
            rr[t] = ss;
            __syncthreads();
            if (t < h) ss = rr[t] + rr[t + h];
            __syncthreads();
        }
    }
    // levels 32 .. 1: wave butterfly (lanes >= h of the first wave carry copies)
#pragma unroll
    for (int h = 32; h >= 1; h >>= 1) ss += __shfl_xor(ss, h, 64);
    if (t == 0) bc[rg][0] = ss;
    __syncthreads();
    ss = bc[rg][0];
    const float scale = 1.0f / __builtin_sqrtf(ss / (float)K + eps);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = t + T * i;
        if (c < nch) {
            const float4 g0 = *(const float4*)(w + 8 * c), g1 = *(const float4*)(w + 8 * c + 4);
            const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float y = v[i][e] * scale;
                asm volatile("" : "+v"(y));       // two roundings, no fused form
                y = y * g[e];
                v[i][e] = y;
                amax = fmaxf(amax, fabsf(y));
            }
        }
    }
    amax = wave_max(amax);
    if constexpr (T > 64) {
        __syncthreads();
        if ((t & 63) == 0) red[rg * T + t / 64] = amax;
        __syncthreads();
        amax = red[rg * T];
#pragma unroll
        for (int k = 1; k < T / 64; k++) amax = fmaxf(amax, red[rg * T + k]);
    }
    if (!live) return;
    const float sc = amax == 0.f ? 1.f : amax / 127.0f;
    if (t == 0) s[row] = sc;
    int8_t* qr = q + (int64_t)row * K;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = t + T * i;
        if (c < nch) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) lo |= (uint32_t)(uint8_t)quant1(v[i][e], sc) << (8 * e);
#pragma unroll
            for (int e = 0; e < 4; e++) hi |= (uint32_t)(uint8_t)quant1(v[i][4 + e], sc) << (8 * e);
            *(uint2*)(qr + 8 * c) = make_uint2(lo, hi);
        }
    }
}

template <typename XT, int T, int NV>
static void launch_rq(const XT* x, const XT* r, XT* xs, const float* w, int8_t* q, float* s,
                      int M, int K, float eps, hipStream_t st) {
    const dim3 grid(ceil_div(M, 256 / T)), block(256);
    if (r) rmsnorm_quant_kernel<XT, T, NV, true><<<grid, block, 0, st>>>(x, r, xs, w, q, s, M, K, eps);
    else rmsnorm_quant_kernel<XT, T, NV, false><<<grid, block, 0, st>>>(x, r, xs, w, q, s, M, K, eps);
}

template <typename XT>
static void launch_rq_any(const XT* x, const XT* r, XT* xs, const float* w, int8_t* q, float* s,
                          int M, int K, float eps, hipStream_t st) {
    int n = 1;
    while (n < K / 8) n <<= 1;          // chunks, padded to a power of two
    if (n <= 64) launch_rq<XT, 64, 1>(x, r, xs, w, q, s, M, K, eps, st);
    else if (n == 128) launch_rq<XT, 128, 1>(x, r, xs, w, q, s, M, K, eps, st);
    else if (n == 256) launch_rq<XT, 256, 1>(x, r, xs, w, q, s, M, K, eps, st);
    else if (n == 512) launch_rq<XT, 256, 2>(x, r, xs, w, q, s, M, K, eps, st);
    else if (n == 1024) launch_rq<XT, 256, 4>(x, r, xs, w, q, s, M, K, eps, st);
    else if (n == 2048) launch_rq<XT, 256, 8>(x, r, xs, w, q, s, M, K, eps, st);
    else launch_rq<XT, 256, 16>(x, r, xs, w, q, s, M, K, eps, st);
}

int rmsnorm_quant(const void* x, int x_dtype, const void* residual, void* x_sum,
                  const float* gamma, float eps, int8_t* q, float* s, int M, int K,
                  hipStream_t st) {
    PIO_REQUIRE(x && gamma && q && s, "rmsnorm_quant: null pointer");
    PIO_REQUIRE((residual == nullptr) == (x_sum == nullptr),
                "rmsnorm_quant: residual and x_sum go together");
    PIO_REQUIRE(M >= 0 && K >= 8 && K % 8 == 0 && K <= 32768,
                "rmsnorm_quant: K=%d must be a multiple of 8 in [8, 32768] (M=%d)", K, M);
    PIO_REQUIRE(x_dtype == PIO_F32 || x_dtype == PIO_F16, "rmsnorm_quant: x must be fp32 or fp16");
    PIO_REQUIRE(aligned16(x) && aligned16(gamma) && aligned16(q) &&
                (!residual || (aligned16(residual) && aligned16(x_sum))),
                "rmsnorm_quant: pointers must be 16-byte aligned");
    PIO_REQUIRE(eps >= 0.f, "rmsnorm_quant: eps must be >= 0");
    if (M == 0) return PIO_OK;
    if (x_dtype == PIO_F32)
        launch_rq_any((const float*)x, (const float*)residual, (float*)x_sum, gamma, q, s, M, K, eps, st);
    else
        launch_rq_any((const _Float16*)x, (const _Float16*)residual, (_Float16*)x_sum, gamma, q, s, M,
                      K, eps, st);
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

PIO_EXPORT int pio_rmsnorm_quant(const void* x, int x_dtype, const void* residual, void* x_sum,
                                 const float* gamma, float eps, int8_t* q, float* s, int M, int K,
                                 void* stream) {
    return rmsnorm_quant(x, x_dtype, residual, x_sum, gamma, eps, q, s, M, K, pick_stream(stream));
}

// Shape checks shared by the two Tensor forms; r (the residual) may be null.
static int rmsnorm_quant_tensor(Tensor* x, Tensor* r, Tensor* weight, Tensor* q, Tensor* s,
                                float eps) {
    PIO_TRY(check_device_tensor(x, "rms_norm_quantize x"));
    PIO_TRY(check_device_tensor(weight, "rms_norm_quantize weight"));
    PIO_TRY(check_device_tensor(q, "rms_norm_quantize q"));
    PIO_TRY(check_device_tensor(s, "rms_norm_quantize s"));
    const int K = last_dim(x);
    PIO_REQUIRE(K > 0, "rms_norm_quantize: empty last dim");
    const int M = x->size / K;
    const int dt = tensor_dtype_of(x);
    if (r) {
        PIO_TRY(check_device_tensor(r, "fused_add_rms_norm_quantize residual"));
        PIO_REQUIRE(r->size == x->size && tensor_dtype_of(r) == dt,
                    "fused_add_rms_norm_quantize: residual must match x in size and dtype");
    }
    PIO_REQUIRE(weight->size == K && tensor_dtype_of(weight) == PIO_F32,
                "rms_norm_quantize: weight must be fp32 [%d]", K);
    PIO_REQUIRE(q->size == x->size && tensor_dtype_of(q) == PIO_I8,
                "rms_norm_quantize: q must be int8 with x's %d elements", x->size);
    PIO_REQUIRE(s->size == M && tensor_dtype_of(s) == PIO_F32,
                "rms_norm_quantize: s must be fp32 [%d]", M);
    return rmsnorm_quant(x->data, dt, r ? r->data : nullptr, r ? x->data : nullptr, weight->data,
                         eps, (int8_t*)q->data, s->data, M, K, current_stream());
}

PIO_EXPORT int tensor_rms_norm_quantize_status(Tensor* x, Tensor* weight, Tensor* q, Tensor* s,
                                               float eps) {
    return rmsnorm_quant_tensor(x, nullptr, weight, q, s, eps);
}
PIO_EXPORT void tensor_rms_norm_quantize(Tensor* x, Tensor* weight, Tensor* q, Tensor* s, float eps) {
    tensor_rms_norm_quantize_status(x, weight, q, s, eps);
}
PIO_EXPORT int tensor_fused_add_rms_norm_quantize_status(Tensor* x, Tensor* residual, Tensor* weight,
                                                         Tensor* q, Tensor* s, float eps) {
    return rmsnorm_quant_tensor(x, residual, weight, q, s, eps);
}
PIO_EXPORT void tensor_fused_add_rms_norm_quantize(Tensor* x, Tensor* residual, Tensor* weight,
                                                   Tensor* q, Tensor* s, float eps) {
    tensor_fused_add_rms_norm_quantize_status(x, residual, weight, q, s, eps);
}
