// W8 linear on the matrix cores for many activation rows (prefill, large M):
//   y[m,n] = s_w[n] * sum_k x[m,k] * float(W[n,k]) (+ bias[n]) (+ y[m,n])
// W int8 [N,K], x fp32 or fp16 [M,K], y fp32 or fp16 [M,N]. This is the same
// contract as the decode GEMV (gemv.hip), whose FMA kernels spend M fp32 FMAs
// per weight byte and re-stream W for every few rows. Here every weight byte
// is read once per launch from HBM: a 64 x 64 output tile per workgroup, and
// the tiles are dealt to the XCDs so that one XCD's tiles share weight panels
// through its L2.
//
// Exactness. An int8 weight is exact in bf16 and in fp16. fp16 x is used as
// it is (v_mfma_f32_32x32x16_f16). fp32 x is split exactly into three bf16
// parts, x = hi + mid + lo (the top, middle and low 8 significand bits: each
// subtraction below is exact by Sterbenz's lemma and the last remainder has
// at most 8 significant bits), and multiplied on v_mfma_f32_32x32x16_bf16.
// Every product of a part and a weight is exact in fp32, so, as in an fp32
// GEMV, only the fp32 accumulation rounds (in another order).
//
// Per K step of 64 elements each thread loads 16 x values and 16 weights of
// one row (registers, one step ahead), converts them and writes them to an LDS
// stage; rows are 128 B (64 two-byte elements) with the 16-byte chunks
// XOR-swizzled by row pair (chunk c of row r at c ^ ((r >> 1) & 7)), so the
// MFMA operand reads (16 consecutive rows per quarter wave, one chunk) are
// conflict-free. Two stages, one barrier per step. Tiles of 128 x 128 (each
// wave 2 x 2 MFMA tiles of 32 x 32, so each fragment read feeds two MFMAs)
// when they still give every CU a tile, else 64 x 64 (one MFMA tile per wave);
// when those leave CUs without two blocks, K is split and a reduce launch sums
// the fp32 partials in slice order.
#include "pio_common.hpp"

#include <type_traits>

namespace pio {

typedef __bf16 wf_bf8 __attribute__((ext_vector_type(8)));
typedef _Float16 wf_h8 __attribute__((ext_vector_type(8)));
typedef float wf_v16f __attribute__((ext_vector_type(16)));
typedef int wf_v4i __attribute__((ext_vector_type(4)));
typedef float wf_f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const wf_v4i wf_gv4i;
typedef __attribute__((address_space(1))) const wf_f4 wf_gf4;

constexpr int WF_BK = 64;
constexpr int WF_ROW = WF_BK * 2;   // LDS bytes per tile row

enum { WF_STORE = 0, WF_RESID = 1, WF_PARTIAL = 2 };

struct W8fParams {
    const void* x;
    const int8_t* w;
    const float* s_w;
    const float* bias;
    void* y;            // output, or the fp32 partials [splits][M][N] (WF_PARTIAL)
    int M, N, K;        // K: the whole reduction length
    int ks;             // K elements per split (a multiple of WF_BK)
    int64_t ldx, ldw, ldy;
    int m_tiles, n_tiles, per_xcd;
};

__device__ __forceinline__ int wf_swz(int r, int c) { return r * WF_ROW + ((c ^ ((r >> 1) & 7)) << 4); }

// The three bf16 parts of v (bit patterns in the low 16 bits).
__device__ __forceinline__ void wf_split3(float v, uint32_t& h, uint32_t& m, uint32_t& l) {
    const uint32_t bh = __float_as_uint(v) & 0xFFFF0000u;
    const float r1 = v - __uint_as_float(bh);
    const uint32_t bm = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(bm);
    h = bh >> 16;
    m = bm >> 16;
    l = __float_as_uint(r2) >> 16;
}

// 16 int8 weights (one 16-byte load) as 16 two-byte MFMA operands: bf16 for
// the fp32-x path (the high half of the exact fp32 value), fp16 otherwise.
template <int NL>
__device__ __forceinline__ void wf_widen(wf_v4i w, uint32_t (&o)[8]) {
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int u = w[d];
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; i++) f[i] = (float)(int8_t)(u >> (8 * i));
        if constexpr (NL == 3) {
            o[2 * d] = (__float_as_uint(f[0]) >> 16) | (__float_as_uint(f[1]) & 0xFFFF0000u);
            o[2 * d + 1] = (__float_as_uint(f[2]) >> 16) | (__float_as_uint(f[3]) & 0xFFFF0000u);
        } else {
            o[2 * d] = (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f[0]) |
                       (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f[1]) << 16;
            o[2 * d + 1] = (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f[2]) |
                           (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f[3]) << 16;
        }
    }
}

template <typename XT> struct WfXRegs;
template <> struct WfXRegs<float> { wf_f4 v[4]; };      // 16 fp32
template <> struct WfXRegs<_Float16> { wf_v4i v[2]; };  // 16 fp16

// Block tile BM x BN = 64 TM x 64 TN: 2 x 2 waves, each owning TM x TN MFMA
// tiles of 32 x 32 (a fragment read from LDS then feeds TN or TM MFMAs).
template <int NL, typename XT, typename YT, int EPI, int TM, int TN>
__global__ __launch_bounds__(256) void gemm_w8f_kernel(W8fParams p) {
    static_assert((NL == 3) == std::is_same<XT, float>::value, "three bf16 parts for fp32 x, one for fp16");
    extern __shared__ __attribute__((aligned(16))) int8_t wf_lds[];
    constexpr int BM = 64 * TM, BN = 64 * TN;
    constexpr int XB = BM * WF_ROW;                    // one part's x tile
    constexpr int STAGE = NL * XB + BN * WF_ROW;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // block b runs on XCD b % 8: each XCD takes a contiguous run of tiles,
    // M-fastest, so consecutive tiles of an XCD share a weight panel
    const int b = blockIdx.x;
    const int t = (b & 7) * p.per_xcd + (b >> 3);
    if (t >= p.m_tiles * p.n_tiles) return;
    const int nt = t / p.m_tiles, mt = t - nt * p.m_tiles;
    const int m0 = mt * BM, n0 = nt * BN;
    const int64_t kb = (int64_t)blockIdx.y * p.ks;
    const int klen = (int)min((int64_t)p.ks, (int64_t)p.K - kb);
    const int nk = (klen + WF_BK - 1) / WF_BK;

    // the epilogue's scales and biases first (clamped: loaded with no branch)
    const int col = lane & 31, h = lane >> 5;
    float sw[TN], bn[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int nc = min(n0 + 32 * TN * wn + 32 * j + col, p.N - 1);
        sw[j] = EPI == WF_PARTIAL ? 0.f : p.s_w[nc];
        bn[j] = (EPI != WF_PARTIAL && p.bias) ? p.bias[nc] : 0.f;
    }

    // loads: thread -> rows r + 64 i of the tile, elements 16 q .. 16 q + 15 of the step
    const int r = tid >> 2, q = tid & 3;
    const XT* xsrc[TM];
    const int8_t* wsrc[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) xsrc[i] = (const XT*)p.x + (int64_t)min(m0 + r + 64 * i, p.M - 1) * p.ldx + kb + 16 * q;
#pragma unroll
    for (int j = 0; j < TN; j++) wsrc[j] = p.w + (int64_t)min(n0 + r + 64 * j, p.N - 1) * p.ldw + kb + 16 * q;
    WfXRegs<XT> xr[TM];
    wf_v4i wr[TN];
    auto gload = [&](int kk) {
        // K % 16 == 0: a thread's 16 elements are all inside or all past the end
        const bool in = kk + 16 * q < klen;
        const int off = in ? kk : 0;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if constexpr (std::is_same<XT, float>::value) {
#pragma unroll
                for (int u = 0; u < 4; u++) xr[i].v[u] = *(wf_gf4*)(xsrc[i] + off + 4 * u);
                if (!in)
#pragma unroll
                    for (int u = 0; u < 4; u++) xr[i].v[u] = wf_f4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int u = 0; u < 2; u++) xr[i].v[u] = *(wf_gv4i*)(xsrc[i] + off + 8 * u);
                if (!in)
#pragma unroll
                    for (int u = 0; u < 2; u++) xr[i].v[u] = wf_v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            wr[j] = *(wf_gv4i*)(wsrc[j] + off);
            if (!in) wr[j] = wf_v4i{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
        int8_t* st = wf_lds + buf * STAGE;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int c0 = wf_swz(r + 64 * i, 2 * q), c1 = wf_swz(r + 64 * i, 2 * q + 1);
            if constexpr (NL == 3) {
                uint32_t pt[3][8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    uint32_t h0, m0_, l0, h1, m1, l1;
                    wf_split3(xr[i].v[u >> 1][2 * (u & 1)], h0, m0_, l0);
                    wf_split3(xr[i].v[u >> 1][2 * (u & 1) + 1], h1, m1, l1);
                    pt[0][u] = h0 | (h1 << 16);
                    pt[1][u] = m0_ | (m1 << 16);
                    pt[2][u] = l0 | (l1 << 16);
                }
#pragma unroll
                for (int L = 0; L < 3; L++) {
                    *(wf_v4i*)(st + L * XB + c0) = wf_v4i{(int)pt[L][0], (int)pt[L][1], (int)pt[L][2], (int)pt[L][3]};
                    *(wf_v4i*)(st + L * XB + c1) = wf_v4i{(int)pt[L][4], (int)pt[L][5], (int)pt[L][6], (int)pt[L][7]};
                }
            } else {
                *(wf_v4i*)(st + c0) = xr[i].v[0];
                *(wf_v4i*)(st + c1) = xr[i].v[1];
            }
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int c0 = wf_swz(r + 64 * j, 2 * q), c1 = wf_swz(r + 64 * j, 2 * q + 1);
            uint32_t o[8];
            wf_widen<NL>(wr[j], o);
            *(wf_v4i*)(st + NL * XB + c0) = wf_v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
            *(wf_v4i*)(st + NL * XB + c1) = wf_v4i{(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
        }
    };

    wf_v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * WF_BK);
        const int8_t* st = wf_lds + cur * STAGE;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int c = 2 * ks + h;   // elements 16 ks + 8 h .. + 8 of the step
            wf_v4i bw[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) bw[j] = *(const wf_v4i*)(st + NL * XB + wf_swz(32 * TN * wn + 32 * j + col, c));
            if constexpr (NL == 3) {
                // the low part first: the small products meet the smaller sums
#pragma unroll
                for (int L = 2; L >= 0; L--)
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        const wf_v4i a = *(const wf_v4i*)(st + L * XB + wf_swz(32 * TM * wm + 32 * i + col, c));
#pragma unroll
                        for (int j = 0; j < TN; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(wf_bf8, a), __builtin_bit_cast(wf_bf8, bw[j]), acc[i][j], 0, 0, 0);
                    }
            } else {
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const wf_v4i a = *(const wf_v4i*)(st + wf_swz(32 * TM * wm + 32 * i + col, c));
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(wf_h8, a), __builtin_bit_cast(wf_h8, bw[j]), acc[i][j], 0, 0, 0);
                }
            }
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // accumulator: element e of lane l is row 8 (e / 4) + 4 (l / 32) + e % 4 of
    // MFMA tile (i, j), column l % 32
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + 32 * TN * wn + 32 * j + col;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + 32 * TM * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
                if (m >= p.M) continue;
                if constexpr (EPI == WF_PARTIAL) {
                    ((float*)p.y)[((int64_t)blockIdx.y * p.M + m) * p.N + n] = acc[i][j][e];
                } else {
                    float v = acc[i][j][e] * sw[j];
                    if (p.bias) v += bn[j];
                    YT* yp = (YT*)p.y + (int64_t)m * p.ldy + n;
                    if constexpr (EPI == WF_RESID) v += to_f32<YT>(*yp);
                    *yp = from_f32<YT>(v);
                }
            }
    }
}

// y[m,n] = (sum over slices in order of part[z][m][n]) * s_w[n] (+ bias[n]) (+ y[m,n]).
template <typename YT, bool RESID>
__global__ __launch_bounds__(256) void gemm_w8f_reduce_kernel(const float* __restrict__ part, int splits, int M,
                                                              int N, const float* __restrict__ s_w,
                                                              const float* __restrict__ bias, YT* __restrict__ y,
                                                              int64_t ldy) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, MN = (int64_t)M * N;
    if (i >= MN) return;
    float acc = 0.f;
#pragma unroll 8
    for (int z = 0; z < splits; z++) acc += part[z * MN + i];   // unrolled: 8 slices' loads in flight
    const int n = (int)(i % N);
    const int64_t m = i / N;
    float v = acc * s_w[n];
    if (bias) v += bias[n];
    YT* yp = y + m * ldy + n;
    if (RESID) v += to_f32<YT>(*yp);
    *yp = from_f32<YT>(v);
}

template <int NL, typename XT, typename YT, int EPI, int TM, int TN>
static int launch_w8f(const W8fParams& p, int splits, hipStream_t st) {
    constexpr size_t lds = 2 * (size_t)(NL * 64 * TM + 64 * TN) * WF_ROW;
    PIO_TRY((allow_lds<gemm_w8f_kernel<NL, XT, YT, EPI, TM, TN>>(lds)));
    gemm_w8f_kernel<NL, XT, YT, EPI, TM, TN><<<dim3(8 * p.per_xcd, splits), 256, lds, st>>>(p);
    PIO_LAUNCHED();
    return PIO_OK;
}

// W8fSplit: a caller that finishes the K-slice sums itself (the prefill's
// fused epilogues). When the plan splits K, the slices' unscaled fp32 partials
// part[z][m][n] (z < splits) are left in `ws` and no reduce runs; otherwise
// y is written as usual and splits = 0.
struct W8fSplit {
    Scratch* ws;
    const float* part;
    int splits;
};

template <int NL, typename XT, typename YT, int TM, int TN>
static int run_tiles(W8fParams p, bool resid, const float* s_w, const float* bias, YT* y, int64_t ldy,
                     hipStream_t st, W8fSplit* out) {
    const int M = p.M, N = p.N, K = p.K;
    p.m_tiles = ceil_div(M, 64 * TM);
    p.n_tiles = ceil_div(N, 64 * TN);
    const int tiles = p.m_tiles * p.n_tiles;
    p.per_xcd = ceil_div(tiles, 8);
    // K slices while the blocks stay within two per CU and each slice keeps
    // >= 4 steps (the prefill's M = 127 linears: 2.64 -> 2.35 ms per prompt
    // against at most one block per CU and 8 steps)
    int splits = 1;
    const int steps = ceil_div(K, WF_BK);
    while (tiles * splits * 2 <= 512 && steps / (splits * 2) >= 4) splits *= 2;
    p.ks = ceil_div(steps, splits) * WF_BK;
    splits = ceil_div(K, p.ks);
    if (out) {
        out->part = nullptr;
        out->splits = 0;
    }
    if (splits == 1) {
        p.ks = K;
        return resid ? launch_w8f<NL, XT, YT, WF_RESID, TM, TN>(p, 1, st)
                     : launch_w8f<NL, XT, YT, WF_STORE, TM, TN>(p, 1, st);
    }
    Scratch own;
    Scratch& ws = out ? *out->ws : own;
    PIO_TRY(ws.get((size_t)splits * M * N * sizeof(float), st));
    p.y = ws.ptr;
    PIO_TRY((launch_w8f<NL, XT, YT, WF_PARTIAL, TM, TN>(p, splits, st)));
    if (out) {
        out->part = (const float*)ws.ptr;
        out->splits = splits;
        return PIO_OK;
    }
    const int64_t MN = (int64_t)M * N;
    if (resid)
        gemm_w8f_reduce_kernel<YT, true><<<(unsigned)ceil_div(MN, 256), 256, 0, st>>>((const float*)ws.ptr, splits, M,
                                                                                     N, s_w, bias, y, ldy);
    else
        gemm_w8f_reduce_kernel<YT, false><<<(unsigned)ceil_div(MN, 256), 256, 0, st>>>((const float*)ws.ptr, splits,
                                                                                      M, N, s_w, bias, y, ldy);
    PIO_LAUNCHED();
    return PIO_OK;
}

template <typename XT, typename YT>
static int run_w8f(const XT* x, int64_t ldx, const int8_t* w, const float* s_w, const float* bias, YT* y,
                   int64_t ldy, int M, int N, int K, bool resid, hipStream_t st, W8fSplit* out) {
    constexpr int NL = std::is_same<XT, float>::value ? 3 : 1;
    W8fParams p{};
    p.x = x; p.w = w; p.s_w = s_w; p.bias = bias; p.y = y;
    p.M = M; p.N = N; p.K = K;
    p.ldx = ldx; p.ldw = K; p.ldy = ldy;
    // 128 x 128 tiles (every fragment read feeds two MFMAs) when they still
    // give every CU a tile; 64 x 64 tiles (with K slices if needed) otherwise
    if ((int64_t)ceil_div(M, 128) * ceil_div(N, 128) >= 256)
        return run_tiles<NL, XT, YT, 2, 2>(p, resid, s_w, bias, y, ldy, st, out);
    return run_tiles<NL, XT, YT, 1, 1>(p, resid, s_w, bias, y, ldy, st, out);
}

static int check_w8f(const void* x, int x_dtype, int64_t ldx, const int8_t* w, const float* s_w, const void* y,
                     int y_dtype, int M, int N, int K) {
    PIO_REQUIRE(x && w && s_w && y, "gemm_w8f: null pointer");
    PIO_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemm_w8f: negative shape");
    PIO_REQUIRE(K % 16 == 0 && ldx % 8 == 0, "gemm_w8f: K=%d and the x row stride must be multiples of 16 and 8",
                K);
    PIO_REQUIRE(aligned16(x) && aligned16(w), "gemm_w8f: x and W must be 16-byte aligned");
    PIO_REQUIRE(x_dtype == PIO_F32 || x_dtype == PIO_F16, "gemm_w8f: x must be fp32 or fp16");
    PIO_REQUIRE(y_dtype == PIO_F32 || y_dtype == PIO_F16, "gemm_w8f: y must be fp32 or fp16");
    return PIO_OK;
}

// Row strides: ldx elements of x, ldy elements of y (W rows are K bytes).
// resid: y += the linear's output (y fp32 or fp16, read before it is written).
int gemm_w8f(const void* x, int x_dtype, int64_t ldx, const int8_t* w, const float* s_w, const float* bias,
             void* y, int y_dtype, int64_t ldy, int M, int N, int K, bool resid, hipStream_t st) {
    PIO_TRY(check_w8f(x, x_dtype, ldx, w, s_w, y, y_dtype, M, N, K));
    if (M == 0 || N == 0) return PIO_OK;
    if (x_dtype == PIO_F32) {
        if (y_dtype == PIO_F32)
            return run_w8f((const float*)x, ldx, w, s_w, bias, (float*)y, ldy, M, N, K, resid, st, nullptr);
        return run_w8f((const float*)x, ldx, w, s_w, bias, (_Float16*)y, ldy, M, N, K, resid, st, nullptr);
    }
    if (y_dtype == PIO_F32)
        return run_w8f((const _Float16*)x, ldx, w, s_w, bias, (float*)y, ldy, M, N, K, resid, st, nullptr);
    return run_w8f((const _Float16*)x, ldx, w, s_w, bias, (_Float16*)y, ldy, M, N, K, resid, st, nullptr);
}

// fp32 x and y. When the plan splits K, only the slices' unscaled partials
// are produced (*part, *splits, in `ws`; y untouched) for the caller to finish;
// otherwise y is written (scaled, + bias, + y when resid) and *splits = 0.
int gemm_w8f_split(const float* x, int64_t ldx, const int8_t* w, const float* s_w, const float* bias, float* y,
                   int64_t ldy, int M, int N, int K, bool resid, Scratch& ws, const float** part, int* splits,
                   hipStream_t st) {
    PIO_TRY(check_w8f(x, PIO_F32, ldx, w, s_w, y, PIO_F32, M, N, K));
    W8fSplit out{&ws, nullptr, 0};
    *part = nullptr;
    *splits = 0;
    if (M == 0 || N == 0) return PIO_OK;
    PIO_TRY(run_w8f(x, ldx, w, s_w, bias, y, ldy, M, N, K, resid, st, &out));
    *part = out.part;
    *splits = out.splits;
    return PIO_OK;
}

}  // namespace pio
