// W8 per-output-channel dequant GEMV / skinny GEMM (decode path):
//   y[m,n] = s_w[n] * sum_k x[m,k] * float(W[n,k]) (+ bias[n])
// W int8 [N,K] row-major, x fp32|fp16 [M,K], y fp32|fp16 [M,N].
//
// The op is HBM-bound: every weight byte is used M times (M <= 8 per launch).
// Mapping: a wavefront owns R consecutive output rows; lane l covers the 16
// bytes k = c*1024 + 16*l of each row in K-chunk c, so one 64-lane load
// instruction (global_load_dwordx4) fetches 1 KiB contiguous of one row and the
// R rows give R independent 16 B loads in flight per lane. The matching 16 x
// values are loaded once per chunk and reused across the R rows. Bytes are
// converted with v_cvt_f32_i32_sdwa (sign-extended byte select, 1 VALU op) and
// accumulated with fp32 FMA; the per-channel scale is applied once per output
// after the cross-lane reduction. Requires K % 16 == 0 and 16 B aligned rows.
#include "pio_common.hpp"

namespace pio {

typedef int v4i __attribute__((ext_vector_type(4)));

template <typename XT>
__device__ __forceinline__ void load_x16(const XT* p, float (&v)[16]);
template <>
__device__ __forceinline__ void load_x16<float>(const float* p, float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 a = *(const float4*)(p + 4 * i);
        v[4 * i + 0] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
    }
}
template <>
__device__ __forceinline__ void load_x16<_Float16>(const _Float16* p, float (&v)[16]) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
    for (int i = 0; i < 2; i++) {
        h8 h = *(const h8*)(p + 8 * i);
#pragma unroll
        for (int j = 0; j < 8; j++) v[8 * i + j] = (float)h[j];
    }
}

__device__ __forceinline__ float dot16(const float (&x)[16], v4i w, float acc) {
#pragma unroll
    for (int d = 0; d < 4; d++) {
        int u = w[d];
        acc = fmaf(x[4 * d + 0], (float)(int8_t)(u), acc);
        acc = fmaf(x[4 * d + 1], (float)(int8_t)(u >> 8), acc);
        acc = fmaf(x[4 * d + 2], (float)(int8_t)(u >> 16), acc);
        acc = fmaf(x[4 * d + 3], (float)(int8_t)(u >> 24), acc);
    }
    return acc;
}

// R rows per wave, MT x-rows per launch, 4 waves per block.
template <int R, int MT, typename XT, typename YT>
__global__ __launch_bounds__(256) void gemv_w8_kernel(const XT* __restrict__ x,
                                                      const int8_t* __restrict__ W,
                                                      const float* __restrict__ s_w,
                                                      const float* __restrict__ bias,
                                                      const float* residual,
                                                      YT* y, int N, int K, int ldy) {
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (n0 >= N) return;

    float acc[MT][R];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[m][r] = 0.f;

    const int8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; r++) wrow[r] = W + (int64_t)min(n0 + r, N - 1) * K;

    for (int k = lane * 16; k < K; k += 1024) {
        v4i w[R];
#pragma unroll
        for (int r = 0; r < R; r++) w[r] = __builtin_nontemporal_load((const v4i*)(wrow[r] + k));
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float xv[16];
            load_x16<XT>(x + (int64_t)m * K + k, xv);
#pragma unroll
            for (int r = 0; r < R; r++) acc[m][r] = dot16(xv, w[r], acc[m][r]);
        }
    }

#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[m][r] = wave_sum(acc[m][r]);

    // Lane (m*R + r) writes output (m, n0 + r).
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (lane == m * R + r && n0 + r < N) {
                float v = acc[m][r] * s_w[n0 + r];
                if (bias) v += bias[n0 + r];
                // residual may alias y (in-place x += W x'): same lane reads then writes.
                if (residual) v += residual[(int64_t)m * ldy + n0 + r];
                y[(int64_t)m * ldy + n0 + r] = from_f32<YT>(v);
            }
        }
}

template <int R, int MT, typename XT, typename YT>
static void launch_gemv(const XT* x, const int8_t* w, const float* s_w, const float* bias,
                        const float* res, YT* y, int N, int K, hipStream_t st) {
    dim3 grid(ceil_div(N, 4 * R)), block(256);
    gemv_w8_kernel<R, MT, XT, YT><<<grid, block, 0, st>>>(x, w, s_w, bias, res, y, N, K, N);
}

template <int R, typename XT, typename YT>
static void launch_rows(const XT* x, const int8_t* w, const float* s_w, const float* bias,
                        const float* res, YT* y, int M, int N, int K, hipStream_t st) {
    // x rows are processed in launches of up to 8; each launch re-streams W.
    for (int m0 = 0; m0 < M;) {
        const int left = M - m0;
        const XT* xm = x + (int64_t)m0 * K;
        YT* ym = y + (int64_t)m0 * N;
        const float* rm = res ? res + (int64_t)m0 * N : nullptr;
        if (left >= 8) { launch_gemv<R, 8>(xm, w, s_w, bias, rm, ym, N, K, st); m0 += 8; }
        else if (left >= 4) { launch_gemv<R, 4>(xm, w, s_w, bias, rm, ym, N, K, st); m0 += 4; }
        else if (left >= 2) { launch_gemv<R, 2>(xm, w, s_w, bias, rm, ym, N, K, st); m0 += 2; }
        else { launch_gemv<R, 1>(xm, w, s_w, bias, rm, ym, N, K, st); m0 += 1; }
    }
}

template <typename XT, typename YT>
static void dispatch_r(const XT* x, const int8_t* w, const float* s_w, const float* bias,
                       const float* res, YT* y, int M, int N, int K, hipStream_t st) {
    // Few rows -> fewer rows per wave so the grid still spreads over 256 CUs.
    if (N >= 32768) launch_rows<4>(x, w, s_w, bias, res, y, M, N, K, st);
    else launch_rows<2>(x, w, s_w, bias, res, y, M, N, K, st);
}

// GEMV with an optional fp32 residual added in the epilogue (y may alias it;
// y must then be fp32).
int gemv_w8_res(const void* x, int x_dtype, const int8_t* w, const float* s_w, const float* bias,
                const float* res, void* y, int y_dtype, int M, int N, int K, hipStream_t st) {
    PIO_REQUIRE(x && w && s_w && y, "gemv_w8: null pointer");
    PIO_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemv_w8: negative shape");
    PIO_REQUIRE(K % 16 == 0, "gemv_w8: K=%d must be a multiple of 16", K);
    PIO_REQUIRE(aligned16(x) && aligned16(w), "gemv_w8: x and W must be 16-byte aligned");
    PIO_REQUIRE(x_dtype == PIO_F32 || x_dtype == PIO_F16, "gemv_w8: x must be fp32 or fp16");
    PIO_REQUIRE(y_dtype == PIO_F32 || y_dtype == PIO_F16, "gemv_w8: y must be fp32 or fp16");
    if (M == 0 || N == 0) return PIO_OK;
    if (x_dtype == PIO_F32) {
        if (y_dtype == PIO_F32) dispatch_r((const float*)x, w, s_w, bias, res, (float*)y, M, N, K, st);
        else dispatch_r((const float*)x, w, s_w, bias, res, (_Float16*)y, M, N, K, st);
    } else {
        if (y_dtype == PIO_F32) dispatch_r((const _Float16*)x, w, s_w, bias, res, (float*)y, M, N, K, st);
        else dispatch_r((const _Float16*)x, w, s_w, bias, res, (_Float16*)y, M, N, K, st);
    }
    PIO_LAUNCHED();
    return PIO_OK;
}

int gemv_w8(const void* x, int x_dtype, const int8_t* w, const float* s_w, const float* bias,
            void* y, int y_dtype, int M, int N, int K, hipStream_t st) {
    return gemv_w8_res(x, x_dtype, w, s_w, bias, nullptr, y, y_dtype, M, N, K, st);
}

}  // namespace pio

using namespace pio;

PIO_EXPORT int pio_gemv_w8(const void* x, int x_dtype, const int8_t* w, const float* s_w,
                           const float* bias, void* y, int y_dtype, int M, int N, int K,
                           void* stream) {
    return gemv_w8(x, x_dtype, w, s_w, bias, y, y_dtype, M, N, K, pick_stream(stream));
}
