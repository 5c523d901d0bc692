// Drop-in Tensor* entry points for the int8 linear layers and dequantize.
// Shape rules follow the reference Tensor.linear (backend.py:458-467): x is
// [..., K], W is [N, K], out is [..., N], rows = x->size / K.
#include "pio_common.hpp"

namespace pio {
int gemv_w8(const void* x, int x_dtype, const int8_t* w, const float* s_w, const float* bias,
            void* y, int y_dtype, int M, int N, int K, hipStream_t st);
int gemm_w8a8(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
              const float* bias, void* y, int y_dtype, int M, int N, int K, hipStream_t st);
}  // namespace pio

using namespace pio;

// Int8 tensors may be typed PIO_I8 or be reference-style fp32 tensors whose
// buffer carries packed bytes (tensor_ops.c:227-228).
static bool int8_storage(const Tensor* t) {
    const int d = tensor_dtype_of(t);
    return d == PIO_I8 || d == PIO_F32;
}
static bool fp_act(const Tensor* t) {
    const int d = tensor_dtype_of(t);
    return d == PIO_F32 || d == PIO_F16;
}

static int check_linear_common(Tensor* w, Tensor* s_w, Tensor* bias, int* N, int* K) {
    PIO_TRY(check_device_tensor(w, "linear W"));
    PIO_TRY(check_device_tensor(s_w, "linear s_w"));
    PIO_REQUIRE(w->ndim == 2, "linear: W must be [N,K]");
    PIO_REQUIRE(int8_storage(w), "linear: W must hold int8");
    *N = w->shape[0];
    *K = w->shape[1];
    PIO_REQUIRE(s_w->size == *N && tensor_dtype_of(s_w) == PIO_F32,
                "linear: s_w must be fp32 [%d]", *N);
    if (bias) {
        PIO_TRY(check_device_tensor(bias, "linear bias"));
        PIO_REQUIRE(bias->size == *N && tensor_dtype_of(bias) == PIO_F32,
                    "linear: bias must be fp32 [%d]", *N);
    }
    return PIO_OK;
}

PIO_EXPORT int tensor_linear_w8_status(Tensor* x, Tensor* w, Tensor* s_w, Tensor* bias,
                                       Tensor* out) {
    int N, K;
    PIO_TRY(check_device_tensor(x, "linear_w8 x"));
    PIO_TRY(check_device_tensor(out, "linear_w8 out"));
    PIO_TRY(check_linear_common(w, s_w, bias, &N, &K));
    PIO_REQUIRE(fp_act(x) && fp_act(out), "linear_w8: x and out must be fp32 or fp16");
    PIO_REQUIRE(last_dim(x) == K, "linear_w8: x last dim %d != K %d", last_dim(x), K);
    const int M = x->size / K;
    PIO_REQUIRE(last_dim(out) == N && out->size == M * N, "linear_w8: out must be [..., %d]", N);
    return gemv_w8(x->data, tensor_dtype_of(x), (const int8_t*)w->data, s_w->data,
                   bias ? bias->data : nullptr, out->data, tensor_dtype_of(out), M, N, K,
                   current_stream());
}
PIO_EXPORT void tensor_linear_w8(Tensor* x, Tensor* w, Tensor* s_w, Tensor* bias, Tensor* out) {
    tensor_linear_w8_status(x, w, s_w, bias, out);
}

PIO_EXPORT int tensor_linear_w8a8_status(Tensor* q, Tensor* s_a, Tensor* w, Tensor* s_w,
                                         Tensor* bias, Tensor* out) {
    int N, K;
    PIO_TRY(check_device_tensor(q, "linear_w8a8 q"));
    PIO_TRY(check_device_tensor(s_a, "linear_w8a8 s_a"));
    PIO_TRY(check_device_tensor(out, "linear_w8a8 out"));
    PIO_TRY(check_linear_common(w, s_w, bias, &N, &K));
    PIO_REQUIRE(int8_storage(q), "linear_w8a8: q must hold int8");
    PIO_REQUIRE(last_dim(q) == K, "linear_w8a8: q last dim %d != K %d", last_dim(q), K);
    const int M = q->size / K;
    PIO_REQUIRE(s_a->size == M && tensor_dtype_of(s_a) == PIO_F32,
                "linear_w8a8: s_a must be fp32 [%d]", M);
    const int od = tensor_dtype_of(out);
    PIO_REQUIRE(od == PIO_F32 || od == PIO_F16 || od == PIO_I32,
                "linear_w8a8: out must be fp32, fp16 or int32");
    PIO_REQUIRE(last_dim(out) == N && out->size == M * N, "linear_w8a8: out must be [..., %d]",
                N);
    return gemm_w8a8((const int8_t*)q->data, s_a->data, (const int8_t*)w->data, s_w->data,
                     bias ? bias->data : nullptr, out->data, od, M, N, K, current_stream());
}
PIO_EXPORT void tensor_linear_w8a8(Tensor* q, Tensor* s_a, Tensor* w, Tensor* s_w, Tensor* bias,
                                   Tensor* out) {
    tensor_linear_w8a8_status(q, s_a, w, s_w, bias, out);
}

// out[i] = float(q[i]) * scale[i / cols]; per-tensor when scale has 1 element.
__global__ void dequant_kernel(const int8_t* __restrict__ q, const float* __restrict__ s,
                               float* __restrict__ out, int64_t n, int cols, int per_row) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (float)q[i] * s[per_row ? i / cols : 0];
}

PIO_EXPORT int tensor_dequantize_status(Tensor* q, Tensor* scale, Tensor* out) {
    PIO_TRY(check_device_tensor(q, "dequantize q"));
    PIO_TRY(check_device_tensor(scale, "dequantize scale"));
    PIO_TRY(check_device_tensor(out, "dequantize out"));
    PIO_REQUIRE(int8_storage(q), "dequantize: q must hold int8");
    PIO_REQUIRE(tensor_dtype_of(out) == PIO_F32 && out->size == q->size,
                "dequantize: out must be fp32 with q's element count");
    const int cols = last_dim(q);
    const int rows = cols ? q->size / cols : 0;
    int per_row;
    if (scale->size == 1) per_row = 0;
    else if (scale->size == rows) per_row = 1;
    else return set_error(PIO_ERR_INVALID, "dequantize: scale has %d elements; need 1 or %d",
                          scale->size, rows);
    if (q->size == 0) return PIO_OK;
    int64_t g = ((int64_t)q->size + 255) / 256;
    dequant_kernel<<<(int)(g > 8192 ? 8192 : g), 256, 0, current_stream()>>>(
        (const int8_t*)q->data, scale->data, out->data, q->size, cols, per_row);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_dequantize(Tensor* q, Tensor* scale, Tensor* out) {
    tensor_dequantize_status(q, scale, out);
}
