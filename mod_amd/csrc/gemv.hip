// W8 per-output-channel dequant GEMV / skinny GEMM (decode path):
//   y[m,n] = s_w[n] * sum_k x[m,k] * float(W[n,k]) (+ bias[n])
// W int8 [N,K] row-major, x fp32|fp16 [M,K], y fp32|fp16 [M,N].
//
// The op is HBM-bound: every weight byte is used M times (M <= 4 per launch).
// The stream kernel (gemv_w8_stream_kernel) keeps x in LDS and streams the
// weights with persistent waves; the direct kernel (gemv_w8_direct_kernel)
// takes small weights and the shapes whose x does not fit the LDS. Both
// convert each weight byte to fp32 once (v_cvt_f32_i32_sdwa, sign-extended
// byte select), accumulate in fp32 FMA, and apply the per-channel scale once
// per output after the cross-lane reduction. fp16 activations with
// 2 <= M <= 64 and K % 1024 == 0 go to the MFMA kernel (gemv_w8_mfma_kernel,
// below), where the FMA kernels would be VALU-bound; any other batch of more
// than 4 rows to the MFMA GEMM of gemm_w8f.hip, which reads W once. Requires
// K % 16 == 0 and 16 B aligned x and W rows.
#include "pio_common.hpp"
#include "gemm_core.hpp"

#include <algorithm>
#include <type_traits>

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

// Direct kernel: a wave owns R consecutive output rows; lane l covers the 16
// bytes k = c*1024 + 16*l of each row in K-chunk c (one 64-lane 16 B load
// fetches 1 KiB contiguous of a row), with the matching 16 x values loaded
// from global memory once per chunk and reused across the R rows. MT x-rows
// per launch, 4 waves per block.
template <int R, int MT, typename XT, typename YT>
__global__ __launch_bounds__(256) void gemv_w8_direct_kernel(const XT* __restrict__ x,
                                                             const int8_t* __restrict__ W,
                                                             const float* __restrict__ s_w,
                                                             const float* __restrict__ bias,
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
    // The scale and bias of the row this lane writes (lane m * R + r writes
    // row r), loaded with the first weights: loaded at the end, behind the
    // per-lane store branches, each waited for the previous one.
    const int rl = min(n0 + lane % R, N - 1);
    const float swl = s_w[rl];
    const float bl = bias ? bias[rl] : 0.f;

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
                float v = acc[m][r] * swl;
                if (bias) v += bl;
                y[(int64_t)m * ldy + n0 + r] = from_f32<YT>(v);
            }
        }
}

// ---------------------------------------------------------------- v2 ---
// Persistent weight stream. A block of GEMV_WAVES waves stages x once in LDS;
// each wave then walks its row groups (R rows each; group g goes to wave
// g % n_waves, so the waves in flight read neighbouring rows) and, per step,
// issues the 16 B loads of U 1 KiB chunks of each of its R rows -- every load
// unconditional, addresses clamped into the weight, so the compiler counts
// them and waits for each in order as the math consumes it -- then converts and
// accumulates them. Overlap of memory and math comes from the 16 resident
// waves per CU (4 per SIMD) rather than from software pipelining: plain
// 16 B loads into VGPRs stream from HBM faster here than LDS-DMA copies, and a
// loop-carried register double buffer makes the compiler wait for all loads.
// x in LDS is fp32 and lane-transposed: K-chunk c of x row m sits at
// xs[(m*nch + c)*1024], and within it the 4 floats a lane needs for its j-th
// 16 B read sit at j*256 + lane*4, so each of a lane's four ds_read_b128 per
// chunk reads 64 lanes' contiguous 16 B (no bank conflicts). Each weight byte
// is converted to fp32 once and used for the MT x rows.
constexpr int GEMV_WAVES = 16;                // waves per block = resident waves per CU
constexpr int GEMV_XLDS = 160 * 1024;         // x bytes the LDS stage takes (one block per CU)

template <typename XT>
__device__ __forceinline__ void load_x4(const XT* p, float (&v)[4]);
template <>
__device__ __forceinline__ void load_x4<float>(const float* p, float (&v)[4]) {
    const float4 a = *(const float4*)p;
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}
template <>
__device__ __forceinline__ void load_x4<_Float16>(const _Float16* p, float (&v)[4]) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = *(const h4*)p;
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = (float)h[j];
}

template <int R, int MT, typename XT, typename YT>
__global__ __launch_bounds__(64 * GEMV_WAVES) void gemv_w8_stream_kernel(const XT* __restrict__ x,
                                                                      const int8_t* __restrict__ W,
                                                                      const float* __restrict__ s_w,
                                                                      const float* __restrict__ bias,
                                                                      YT* y, int N, int K, int ldy) {
    constexpr int U = 4 / R;   // 1 KiB chunks per row per step: 4 loads per lane
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int nch = (K + 1023) >> 10;
    const int nst = (nch + U - 1) / U;
    const int ngroups = (N + R - 1) / R;
    // waves numbered block-fastest, so a grid with fewer row groups than waves
    // still spreads them over every block (CU)
    const int wave_id = (tid >> 6) * gridDim.x + blockIdx.x, n_waves = gridDim.x * GEMV_WAVES;

    // loads of U chunks of the R rows of group g at step st (addresses clamped
    // into the weight: every load is issued)
    auto load = [&](int g, int st, v4i (&w)[U][R]) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = min(min(st * U + u, nch - 1) * 1024 + lane * 16, K - 16);
#pragma unroll
            for (int r = 0; r < R; r++)
                w[u][r] = __builtin_nontemporal_load((const v4i*)(W + (int64_t)min(g * R + r, N - 1) * K + k));
        }
    };
    float acc[MT][R];
    auto math = [&](int st, const v4i (&w)[U][R]) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = st * U + u;
            if (c >= nch) continue;   // wave-uniform: a clamped duplicate chunk
            float xv[MT][16];
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const float* src = xs + (m * nch + c) * 1024 + lane * 4;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 q = *(const float4*)(src + j * 256);
                    xv[m][4 * j + 0] = q.x; xv[m][4 * j + 1] = q.y;
                    xv[m][4 * j + 2] = q.z; xv[m][4 * j + 3] = q.w;
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float wf[16];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int v = w[u][r][e];
                    wf[4 * e + 0] = (float)(int8_t)v;
                    wf[4 * e + 1] = (float)(int8_t)(v >> 8);
                    wf[4 * e + 2] = (float)(int8_t)(v >> 16);
                    wf[4 * e + 3] = (float)(v >> 24);
                }
#pragma unroll
                for (int m = 0; m < MT; m++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[m][r] = fmaf(xv[m][e], wf[e], acc[m][r]);
            }
        }
    };
    // The scale and bias of the row lane m*R + r writes in group g, loaded
    // when the group starts: loaded behind the store branch they were two
    // dependent round trips per group.
    auto scales = [&](int g, float& sw, float& bb) {
        const int rr = min(g * R + lane % R, N - 1);
        sw = s_w[rr];
        bb = bias ? bias[rr] : 0.f;
    };
    // lane m*R + r writes output (m, g*R + r)
    auto finish = [&](int g, float sw, float bb) {
        const int n0 = g * R;
        float mine = 0.f;
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float t = wsum(acc[m][r]);
                if (lane == m * R + r) mine = t;
                acc[m][r] = 0.f;
            }
        const int em = lane / R, er = lane % R;
        if (lane < MT * R && n0 + er < N) {
            float v = mine * sw;
            if (bias) v += bb;
            y[(int64_t)em * ldy + n0 + er] = from_f32<YT>(v);
        }
    };

    // the first step's weights are requested before x is staged, so the two
    // latencies overlap
    v4i w0[U][R];
    load(min(wave_id, ngroups - 1), 0, w0);
    float sw0, bb0;
    scales(min(wave_id, ngroups - 1), sw0, bb0);
    for (int q = tid; q < MT * nch * 256; q += 64 * GEMV_WAVES) {
        const int m = q / (nch * 256), k = (q - m * nch * 256) * 4;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (k < K) load_x4<XT>(x + (int64_t)m * K + k, v);
        float* d = xs + (m * nch + (k >> 10)) * 1024 + ((k & 15) >> 2) * 256 + ((k & 1023) >> 4) * 4;
        *(float4*)d = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    if (wave_id >= ngroups) return;

#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[m][r] = 0.f;
    math(0, w0);
    for (int st = 1; st < nst; st++) {
        v4i w[U][R];
        load(wave_id, st, w);
        math(st, w);
    }
    finish(wave_id, sw0, bb0);
    for (int g = wave_id + n_waves; g < ngroups; g += n_waves) {
        float sw, bb;
        scales(g, sw, bb);
        for (int st = 0; st < nst; st++) {
            v4i w[U][R];
            load(g, st, w);
            math(st, w);
        }
        finish(g, sw, bb);
    }
}

static int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

// Fraction of wave-rounds doing work when ceil(N/R) row groups are dealt to
// the resident waves round-robin.
static double stream_balance(int N, int R) {
    const int64_t waves = (int64_t)device_cus() * GEMV_WAVES;
    const int64_t groups = ceil_div(N, R);
    const int64_t rounds = (groups + waves - 1) / waves;
    return (double)groups / (double)(rounds * waves);
}

// Rows per group for the stream kernel: among R = 4, 2, 1 (U = 4/R chunks
// per step), those whose U divides the row's chunk count first (no duplicate
// chunk loads), then the best-balanced round-robin, ties to more rows (each x
// value read from LDS then serves more weight rows). 0: x does not fit the LDS.
static int stream_pick(int MT, int N, int K) {
    const int nch = (K + 1023) / 1024;
    if ((size_t)MT * nch * 4096 > (size_t)GEMV_XLDS) return 0;
    double best = -1;
    int pick = 0;
    for (int R : {4, 2, 1}) {
        if (R * MT > 8) continue;   // 4 rows x 4 x-rows: more registers than 16 waves per CU leave
        const int U = 4 / R;
        double e = stream_balance(N, R) - (nch % U ? 1.0 : 0.0);
        if (e > best + 1e-9) { best = e; pick = R; }
    }
    return pick;
}

template <int R, int MT, typename XT, typename YT>
static int launch_stream_r(const XT* x, const int8_t* w, const float* s_w, const float* bias, YT* y,
                           int N, int K, hipStream_t st) {
    const size_t lds = (size_t)MT * ((K + 1023) / 1024) * 4096;
    PIO_TRY(allow_lds<gemv_w8_stream_kernel<R, MT, XT, YT>>(lds));
    const int blocks = (int)std::min<int64_t>(ceil_div(N, R), device_cus());
    gemv_w8_stream_kernel<R, MT, XT, YT><<<blocks, 64 * GEMV_WAVES, lds, st>>>(x, w, s_w, bias, y, N, K, N);
    return PIO_OK;
}

template <int MT, typename XT, typename YT>
static int launch_stream(const XT* x, const int8_t* w, const float* s_w, const float* bias, YT* y,
                         int N, int K, int R, hipStream_t st) {
    if constexpr (MT * 4 <= 8) {
        if (R == 4) return launch_stream_r<4, MT>(x, w, s_w, bias, y, N, K, st);
    }
    if (R == 2) return launch_stream_r<2, MT>(x, w, s_w, bias, y, N, K, st);
    return launch_stream_r<1, MT>(x, w, s_w, bias, y, N, K, st);
}

template <int R, int MT, typename XT, typename YT>
static void launch_direct(const XT* x, const int8_t* w, const float* s_w, const float* bias, YT* y,
                          int N, int K, hipStream_t st) {
    gemv_w8_direct_kernel<R, MT, XT, YT><<<ceil_div(N, 4 * R), 256, 0, st>>>(x, w, s_w, bias, y, N, K, N);
}

template <int R, typename XT, typename YT>
static void launch_direct_rows(const XT* x, const int8_t* w, const float* s_w, const float* bias,
                               YT* y, int M, int N, int K, hipStream_t st) {
    // x rows in launches of up to 8; each launch re-streams W
    for (int m0 = 0; m0 < M;) {
        const int left = M - m0;
        const XT* xm = x + (int64_t)m0 * K;
        YT* ym = y + (int64_t)m0 * N;
        if (left >= 8) { launch_direct<R, 8>(xm, w, s_w, bias, ym, N, K, st); m0 += 8; }
        else if (left >= 4) { launch_direct<R, 4>(xm, w, s_w, bias, ym, N, K, st); m0 += 4; }
        else if (left >= 2) { launch_direct<R, 2>(xm, w, s_w, bias, ym, N, K, st); m0 += 2; }
        else { launch_direct<R, 1>(xm, w, s_w, bias, ym, N, K, st); m0 += 1; }
    }
}

// ------------------------------------------------------------- MFMA ---
// fp16 activations with 2 <= M <= 64 rows. The FMA kernels above spend M
// fp32 FMAs per weight byte, which makes them VALU-bound from M ~ 4 (M = 64:
// 2% of HBM). Here the products go to v_mfma_f32_16x16x32_f16: an int8 weight
// is exact in fp16, an fp16 x int8 product is exact in fp32, and the MFMA
// accumulates in fp32. The matrix core's accumulation does not round to
// nearest-even (a sign flip of W moves ~0.06% of outputs by 1-4 ulp, the
// negative side larger), so results match the FMA kernels to a few ulp, not
// bit for bit; they are deterministic run to run. The structure is the skinny W8A8 kernel's (gemm.hip):
// each wave owns 16 weight rows streamed from HBM into registers 4 blocks of
// 256 K ahead (lane: row r = lane % 16, K chunk q = lane / 16, 16 bytes at
// 64*i + 16*q), each 16-byte chunk widened to two 8 x fp16 operands; the
// workgroup's x slice (MT*16 rows x the slice's K, fp16) is copied once into
// LDS with direct-to-LDS loads and read with the same per-lane K chunks.
// Widening: byte b becomes the fp16 whose bits are 0x64 | (b ^ 0x80), i.e.
// 1024 + (b + 128) exactly, minus 1152 (one byte permute per two values and
// one packed fp16 subtract per two values; all values exact). K slices
// (grid y) write fp32 partials that gemv_split_reduce_kernel sums in slice
// order before the scale.
typedef _Float16 gm_v8h __attribute__((ext_vector_type(8)));
typedef _Float16 gm_v2h __attribute__((ext_vector_type(2)));
typedef float gm_v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const v4i gm_gv4i;

constexpr int GM_KB = 256;   // K per block: 4 x 64 (8 MFMAs of 32)
constexpr int GM_D = 4;      // weight blocks in flight per wave

template <int NB>
constexpr int gm_pitch() { return NB * GM_KB * 2 + 16; }   // LDS row pitch in bytes (fp16 x)
template <int MT, int NB>
constexpr size_t gm_lds_bytes() { return (size_t)MT * 16 * gm_pitch<NB>(); }

// Two fp16 (k and k+1 of dword d's bytes sel) from a dword of four int8.
__device__ __forceinline__ gm_v2h gm_widen2(uint32_t t, uint32_t sel) {
    const uint32_t u = __builtin_amdgcn_perm(0x64646464u, t, sel);
    return __builtin_bit_cast(gm_v2h, u) - gm_v2h{(_Float16)1152.0f, (_Float16)1152.0f};
}
// 16 int8 -> two operands of 8 fp16 (bytes 0..7, 8..15).
__device__ __forceinline__ void gm_widen16(v4i w, gm_v8h& lo, gm_v8h& hi) {
    gm_v2h h[8];
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const uint32_t t = (uint32_t)w[d] ^ 0x80808080u;
        h[2 * d] = gm_widen2(t, 0x04010400u);       // bytes 0, 1
        h[2 * d + 1] = gm_widen2(t, 0x04030402u);   // bytes 2, 3
    }
    lo = gm_v8h{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
    hi = gm_v8h{h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
}

struct GemvMfma {
    const _Float16* x;
    const int8_t* w;
    const float* s_w;
    const float* bias;
    void* y;          // YT [M][N], or fp32 partials [S][M][N] when split
    int M, N, K;      // K of one slice
    int ldx;          // row pitch of x and W (the full K)
};

template <int WV, int MT, int NB, typename YT, bool SPLIT>
__global__ __launch_bounds__(64 * WV) void gemv_w8_mfma_kernel(GemvMfma p) {
    typedef __attribute__((address_space(3))) void lds_t;
    constexpr int D = NB < GM_D ? NB : GM_D;
    constexpr int P = gm_pitch<NB>();
    constexpr int SEG = NB * GM_KB * 2 / 1024;   // 1 KB segments per x row
    constexpr int NCP = MT * 16 * SEG;
    extern __shared__ __attribute__((aligned(16))) int8_t gm_lds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * (16 * WV) + w * 16;
    const int64_t k0 = (int64_t)blockIdx.y * p.K;
    // the epilogue's scale and bias, loaded first (clamped column) so that
    // they are not a round trip after the K loop; older than every copy and
    // weight load, so the waits below cover them
    const int nc = min(n0 + r, p.N - 1);
    const float sw = SPLIT ? 0.f : p.s_w[nc];
    const float bn = (!SPLIT && p.bias) ? p.bias[nc] : 0.f;

    // x slice -> LDS (rows >= M re-read row M-1; their outputs are dropped)
#pragma unroll
    for (int j = 0; j < (NCP + WV - 1) / WV; j++) {
        const int u = w + WV * j;
        if (NCP % WV == 0 || u < NCP) {
            const int row = u / SEG, seg = u % SEG;
            const int8_t* src = (const int8_t*)(p.x + (int64_t)min(row, p.M - 1) * p.ldx + k0) + seg * 1024 + 16 * lane;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_t*)(gm_lds + row * P + seg * 1024), 16, 0, 0);
        }
    }
    // the copies must stay older than the weight prefetch (see the wait below)
    __builtin_amdgcn_sched_barrier(0);
    const int8_t* wp = p.w + (int64_t)min(n0 + r, p.N - 1) * p.ldx + k0 + 16 * q;
    v4i wr[D][4];
    auto load_w = [&](int b, v4i (&dst)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = *(gm_gv4i*)(wp + b * GM_KB + 64 * i);   // ordinary loads: see the streamed kernel below
    };
#pragma unroll
    for (int b = 0; b < D; b++) load_w(b, wr[b]);
    stage_barrier<4 * D>();   // the copies have landed; the weight loads stay in flight
    // The widening is register work the scheduler would hoist above the
    // barrier, with a full wait on every load issued so far.
    __builtin_amdgcn_sched_barrier(0);

    gm_v4f acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = gm_v4f{0.f, 0.f, 0.f, 0.f};
    const int8_t* xs = gm_lds + r * P + 32 * q;   // fp16 element 16*q of the K chunk
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            gm_v8h wlo, whi;
            gm_widen16(wr[b % D][i], wlo, whi);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int8_t* a = xs + t * 16 * P + (b * GM_KB + 64 * i) * 2;
                const gm_v8h alo = *(const gm_v8h*)a, ahi = *(const gm_v8h*)(a + 16);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, wlo, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, whi, acc[t], 0, 0, 0);
            }
        }
        if (b + D < NB) load_w(b + D, wr[b % D]);
        __builtin_amdgcn_sched_barrier(0);   // keep the reload here (see gemm.hip's skinny kernel)
    }

    // 16x16 accumulator: lane holds rows 4*q + v of M tile t, column r.
    const int n = n0 + r;
    if (n >= p.N) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int m = t * 16 + 4 * q + v;
            if (m >= p.M) continue;
            if constexpr (SPLIT) {
                ((float*)p.y)[((int64_t)blockIdx.y * p.M + m) * p.N + n] = acc[t][v];
            } else {
                float val = acc[t][v] * sw;
                if (p.bias) val += bn;
                ((YT*)p.y)[(int64_t)m * p.N + n] = from_f32<YT>(val);
            }
        }
    }
}

// Streamed MFMA GEMV for 16 < M <= 64: the one-pass kernel above keeps the
// workgroup's fp16 x slice in LDS, which at 64 rows holds only 1 KB of K and
// forces K slices of 1024 plus a reduce. Here x streams with the weights (as
// the streamed W8A8 kernel in gemm.hip), on v_mfma_f32_32x32x16_f16, which
// does 1.7x the work per cycle of the 16x16x32 form and reads half the x
// bytes from LDS per weight byte. Each wave owns 32 weight rows. Per K block
// of 256 it loads them into registers GS_DW blocks ahead, 64 contiguous bytes
// of 16 rows per load (4 lanes per row; the 32x32 operand layout would give
// each row only 2 lanes, 32 bytes per load, which measured 15-25% slower),
// and one v_permlane16_swap per dword pair moves them into the operand
// layout: lane l then holds bytes 64 s + 32 (l / 32) + 0..31 of row l % 32 for
// the block's 4 segments s. x streams GS_DX blocks ahead into an LDS ring
// stage (direct-to-LDS copies, 32 MT rows x 512 B); one barrier per block.
// (The wait for a block counts vector-memory operations in issue order, so
// the weights' effective lead is GS_DX too; running x as far ahead as the
// weights, in a deeper ring, measured slower.) The weights use ordinary
// loads: each load covers half of a 128-byte line per row, and nontemporal
// loads lose the other half before the next load asks for it (7% slower).
// LDS rows are 512 B with the 16-byte chunks XOR-swizzled by row (chunk c of
// row r at c ^ (r & 15)), so the operand reads (16 rows per quarter wave) are
// conflict-free; the copies pick their global chunk to land that way.
constexpr int GS_DW = 4;                     // weight blocks in flight per wave
constexpr int GS_DX = 2;                     // x blocks in flight per workgroup
constexpr int GS_TILE = 32 * GM_KB * 2;      // one 32-row x tile of a K block (16 KB)
template <int MT>
constexpr size_t gs_lds_bytes() { return (size_t)(GS_DX + 1) * MT * GS_TILE; }   // 48 or 96 KB

// Vector-memory operations a wave has issued after x block b (in the order
// the kernel issues them: per step j the weights of block j + DW, then the x
// copies of block j + DX), counted up to the wait at the top of step b.
template <int NB, int DW, int DX, int WOPS, int XOPS>
__device__ constexpr int gs_after_x(int b) {
    int n = 0;
    for (int j = b - DX + 1; j <= b - 1; j++) n += WOPS * (j + DW < NB) + XOPS * (j + DX < NB);
    return n;
}

// stage_barrier<n>() for a wave-uniform n in [0, MAXN] (constant-folded when
// n is known at compile time, as in fully unrolled loops).
template <int MAXN>
__device__ __forceinline__ void stage_barrier_n(int n) {
    if constexpr (MAXN > 0) {
        if (n >= MAXN) stage_barrier<MAXN>();
        else stage_barrier_n<MAXN - 1>(n);
    } else {
        stage_barrier<0>();
    }
}

typedef float gm_v16f __attribute__((ext_vector_type(16)));

template <int WV, int MT, int NB, typename YT, bool SPLIT>
__global__ __launch_bounds__(64 * WV) void gemv_w8_mfma_stream_kernel(GemvMfma p) {
    typedef __attribute__((address_space(3))) void lds_t;
    static_assert((16 * MT) % WV == 0, "16 MT x copies per block, shared evenly");
    constexpr int DW = NB < GS_DW ? NB : GS_DW;
    constexpr int DX = NB < GS_DX ? NB : GS_DX;
    constexpr int S = GS_DX + 1;
    constexpr int STAGE = MT * GS_TILE;
    constexpr int CPW = 16 * MT / WV;
    constexpr int WOPS = 8;
    constexpr int MAXW = (DX - 1) * (WOPS + CPW);   // the steady-state wait count
    static_assert(DW >= DX, "weights run at least as far ahead as x");
    static_assert(MAXW < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) int8_t gs_lds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int col = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * (32 * WV) + w * 32;
    const int64_t k0 = (int64_t)blockIdx.y * p.K;
    // the epilogue's scale and bias, loaded first (as in the one-pass kernel)
    const int nc = min(n0 + col, p.N - 1);
    const float sw = SPLIT ? 0.f : p.s_w[nc];
    const float bn = (!SPLIT && p.bias) ? p.bias[nc] : 0.f;

    // copy j moves x rows 2u, 2u + 1 (u = w + WV j): lane l lands 16 B at stage
    // offset 1024 u + 16 l = row 2u + l / 32, chunk position l % 32, which holds
    // the row's chunk (l % 32) ^ (row % 16)
    const int8_t* xsrc[CPW];
    int xdst[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const int u = w + WV * j, row = 2 * u + h, c = col ^ (row & 15);
        xsrc[j] = (const int8_t*)(p.x + (int64_t)min(row, p.M - 1) * p.ldx + k0) + c * 16;
        xdst[j] = u * 1024;
    }
    // load 2s + g of a block: rows n0 + 16 g + (l % 16), bytes 64 s + 16 (l / 16)
    const int8_t* wp[2];
#pragma unroll
    for (int g = 0; g < 2; g++)
        wp[g] = p.w + (int64_t)min(n0 + 16 * g + (lane & 15), p.N - 1) * p.ldx + k0 + 16 * (lane >> 4);
    v4i wr[DW][8];
    auto issue_w = [&](int b) {
#pragma unroll
        for (int i = 0; i < 8; i++) wr[b % DW][i] = *(gm_gv4i*)(wp[i & 1] + b * GM_KB + 64 * (i >> 1));
    };
    auto issue_x = [&](int b) {
        int8_t* st = gs_lds + (b % S) * STAGE;
#pragma unroll
        for (int j = 0; j < CPW; j++)
            __builtin_amdgcn_global_load_lds((const void*)(xsrc[j] + b * GM_KB * 2), (lds_t*)(st + xdst[j]), 16, 0, 0);
    };
    // steps -DW .. -1: the weights of blocks 0 .. DW-1, the x of blocks 0 .. DX-1
#pragma unroll
    for (int v = 0; v < DW; v++) {
        issue_w(v);
        if (v >= DW - DX) issue_x(v - (DW - DX));
    }
    __builtin_amdgcn_sched_barrier(0);

    gm_v16f acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[t][e] = 0.f;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        // x block b (and the older weights of block b) landed, then every wave's copies
        stage_barrier_n<MAXW>(gs_after_x<NB, DW, DX, WOPS, CPW>(b));
        // the widening is register work the scheduler would hoist above the barrier
        __builtin_amdgcn_sched_barrier(0);
        const int8_t* st = gs_lds + (b % S) * STAGE;
#pragma unroll
        for (int sg = 0; sg < 4; sg++) {
            // rows 0-15 (load 2s) and 16-31 (load 2s + 1), 16-lane groups swapped:
            // u[0] = chunk 2h, u[1] = chunk 2h + 1 of row col's 64-byte segment
            v4i u[2];
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const auto sw2 = __builtin_amdgcn_permlane16_swap((unsigned)wr[b % DW][2 * sg][d],
                                                                  (unsigned)wr[b % DW][2 * sg + 1][d], false, false);
                u[0][d] = (int)sw2[0];
                u[1][d] = (int)sw2[1];
            }
            gm_v8h wv[4];
            gm_widen16(u[0], wv[0], wv[1]);
            gm_widen16(u[1], wv[2], wv[3]);
            const int c = 8 * sg + 4 * h;   // 16-byte chunk of elements 64 s + 32 h
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int8_t* row = st + (32 * t + col) * (GM_KB * 2);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const gm_v8h a = *(const gm_v8h*)(row + (((c + e) ^ (col & 15)) << 4));
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, wv[e], acc[t], 0, 0, 0);
                }
            }
        }
        if (b + DW < NB) issue_w(b + DW);
        if (b + DX < NB) issue_x(b + DX);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 32x32 accumulator: element e of lane l is x row 8 (e / 4) + 4 (l / 32) + e % 4
    // of tile t, weight row n0 + l % 32.
    const int n = n0 + col;
    if (n >= p.N) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int m = 32 * t + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m >= p.M) continue;
            if constexpr (SPLIT) {
                ((float*)p.y)[((int64_t)blockIdx.y * p.M + m) * p.N + n] = acc[t][e];
            } else {
                float val = acc[t][e] * sw;
                if (p.bias) val += bn;
                ((YT*)p.y)[(int64_t)m * p.N + n] = from_f32<YT>(val);
            }
        }
    }
}

// y[m,n] = (sum over slices in order of ws[z][m][n]) * s_w[n] (+ bias[n]).
template <typename YT>
__global__ __launch_bounds__(256) void gemv_split_reduce_kernel(const float* __restrict__ ws, int splits, int M,
                                                                int N, const float* __restrict__ s_w,
                                                                const float* __restrict__ bias, YT* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, MN = (int64_t)M * N;
    if (i >= MN) return;
    // the scale and bias first, then the slices with their loop unrolled, so
    // every load is in flight together instead of one round trip each
    const int n = (int)(i % N);
    const float sw = s_w[n];
    const float bn = (bias ? bias : s_w)[n];
    float acc = 0.f;
#pragma unroll 8
    for (int z = 0; z < splits; z++) acc += ws[z * MN + i];
    float val = acc * sw;
    if (bias) val += bn;
    y[i] = from_f32<YT>(val);
}

struct GemvMfmaPlan {
    int wv = 0, nb = 0, splits = 1;
    bool stream = false;   // gemv_w8_mfma_stream_kernel
};

// Plan for the streamed kernel (16 < M <= 64), or wv == 0. A workgroup (one
// per CU: its LDS ring is 48 or 96 KB) moves its weights (32 WV rows) and x
// rows (32 or 64, fp16) at ~25 GB/s together, as measured over wv, nb and
// both C4 shapes; the cost is the busiest CU's bytes at that rate, plus for K
// slices the partials' write + read and the reduce launch.
static GemvMfmaPlan plan_gemv_stream(int M, int N, int K) {
    GemvMfmaPlan best;
    if (M <= 16 || M > 64 || K % 1024) return best;
    const int kb = K / GM_KB;
    double best_t = 0;
    for (int wv : {8, 4, 2}) {
        if (wv == 8 && M > 32) continue;
        for (int nb : {16, 12, 8, 6, 4}) {
            if (kb % nb) continue;
            const int sp = kb / nb;
            if (sp > 16) continue;
            const int64_t units = (int64_t)ceil_div(N, 32 * wv) * sp;
            const double per_cu = (double)((units + 255) / 256) * nb * GM_KB * (32.0 * wv + (M > 32 ? 128.0 : 64.0));
            double t = per_cu / 25.0e9;
            if (sp > 1) t += (double)sp * M * N * 8.0 / 4.0e12 + 2.0e-6;
            if (best.wv == 0 || t < best_t * 0.98) {
                best_t = t;
                best.wv = wv; best.nb = nb; best.splits = sp; best.stream = true;
            }
        }
    }
    return best;
}

// Same cost model as the skinny W8A8 plan; the fp16 x slice must fit the LDS
// (16 rows x 8 KB, or 64 rows x 2 KB).
static GemvMfmaPlan plan_gemv_mfma(int M, int N, int K) {
    GemvMfmaPlan best;
    if (M < 2 || M > 64 || K % 1024) return best;
    const int kb = K / GM_KB;
    double best_t = 0;
    for (int wv : {4, 3}) {
        for (int nb : {16, 12, 8, 4}) {
            if (kb % nb || kb / nb > 16 || (M > 16 && nb > 4)) continue;
            const int sp = kb / nb;
            const int64_t units = (int64_t)ceil_div(N, 16 * wv) * sp;
            const double rounds = (double)((units + 255) / 256);
            const double fill = std::min(1.0, (double)units / 256.0);
            double t = std::max((double)N * K / (6.0e12 * fill), rounds * 16.0 * wv * nb * GM_KB / 32.0e9);
            if (sp > 1) t += (double)sp * M * N * 8.0 / 4.0e12 + 2.0e-6;
            if (best.wv == 0 || t < best_t * 0.98) {
                best_t = t;
                best.wv = wv; best.nb = nb; best.splits = sp;
            }
        }
    }
    return best;
}

template <int WV, int MT, int NB, typename YT>
static int launch_gemv_mfma_nb(const GemvMfma& p, int splits, hipStream_t st) {
    constexpr size_t lds = gm_lds_bytes<MT, NB>();
    const dim3 grid(ceil_div(p.N, 16 * WV), splits);
    if (splits > 1) {
        PIO_TRY(allow_lds<gemv_w8_mfma_kernel<WV, MT, NB, YT, true>>(lds));
        gemv_w8_mfma_kernel<WV, MT, NB, YT, true><<<grid, 64 * WV, lds, st>>>(p);
    } else {
        PIO_TRY(allow_lds<gemv_w8_mfma_kernel<WV, MT, NB, YT, false>>(lds));
        gemv_w8_mfma_kernel<WV, MT, NB, YT, false><<<grid, 64 * WV, lds, st>>>(p);
    }
    PIO_LAUNCHED();
    return PIO_OK;
}

template <int WV, int MT, int NB, typename YT>
static int launch_gemv_stream_nb(const GemvMfma& p, int splits, hipStream_t st) {
    constexpr size_t lds = gs_lds_bytes<MT>();
    const dim3 grid(ceil_div(p.N, 32 * WV), splits);
    if (splits > 1) {
        PIO_TRY(allow_lds<gemv_w8_mfma_stream_kernel<WV, MT, NB, YT, true>>(lds));
        gemv_w8_mfma_stream_kernel<WV, MT, NB, YT, true><<<grid, 64 * WV, lds, st>>>(p);
    } else {
        PIO_TRY(allow_lds<gemv_w8_mfma_stream_kernel<WV, MT, NB, YT, false>>(lds));
        gemv_w8_mfma_stream_kernel<WV, MT, NB, YT, false><<<grid, 64 * WV, lds, st>>>(p);
    }
    PIO_LAUNCHED();
    return PIO_OK;
}
template <int WV, int MT, typename YT>
static int launch_gemv_stream_mt(const GemvMfma& p, const GemvMfmaPlan& pl, hipStream_t st) {
    switch (pl.nb) {
    case 16: return launch_gemv_stream_nb<WV, MT, 16, YT>(p, pl.splits, st);
    case 12: return launch_gemv_stream_nb<WV, MT, 12, YT>(p, pl.splits, st);
    case 8: return launch_gemv_stream_nb<WV, MT, 8, YT>(p, pl.splits, st);
    case 6: return launch_gemv_stream_nb<WV, MT, 6, YT>(p, pl.splits, st);
    case 4: return launch_gemv_stream_nb<WV, MT, 4, YT>(p, pl.splits, st);
    default: return set_error(PIO_ERR_INVALID, "gemv: streamed plan with %d blocks", pl.nb);
    }
}
template <int WV, typename YT>
static int launch_gemv_stream_wv(const GemvMfma& p, const GemvMfmaPlan& pl, hipStream_t st) {
    if (p.M <= 32) return launch_gemv_stream_mt<WV, 1, YT>(p, pl, st);
    // two x tiles and 8 waves would leave too few registers per wave
    if constexpr (WV == 8) return set_error(PIO_ERR_INVALID, "gemv: streamed plan with 8 waves for %d rows", p.M);
    else return launch_gemv_stream_mt<WV, 2, YT>(p, pl, st);
}

template <int WV, typename YT>
static int launch_gemv_mfma_wv(const GemvMfma& p, const GemvMfmaPlan& pl, hipStream_t st) {
    if (p.M <= 16) {
        switch (pl.nb) {
        case 16: return launch_gemv_mfma_nb<WV, 1, 16, YT>(p, pl.splits, st);
        case 12: return launch_gemv_mfma_nb<WV, 1, 12, YT>(p, pl.splits, st);
        case 8: return launch_gemv_mfma_nb<WV, 1, 8, YT>(p, pl.splits, st);
        default: return launch_gemv_mfma_nb<WV, 1, 4, YT>(p, pl.splits, st);
        }
    }
    if (pl.nb != 4) return set_error(PIO_ERR_INVALID, "gemv: MFMA plan with %d blocks for %d rows", pl.nb, p.M);
    return launch_gemv_mfma_nb<WV, 4, 4, YT>(p, pl.splits, st);
}

template <typename YT>
static int launch_gemv_mfma(const _Float16* x, const int8_t* w, const float* s_w, const float* bias, YT* y,
                            int M, int N, int K, const GemvMfmaPlan& pl, hipStream_t st) {
    GemvMfma p{x, w, s_w, bias, y, M, N, K / pl.splits, K};
    Scratch ws;
    if (pl.splits > 1) {
        PIO_TRY(ws.get((size_t)pl.splits * M * N * sizeof(float), st));
        p.y = ws.ptr;
    }
    int rc;
    if (pl.stream)
        rc = pl.wv == 8   ? launch_gemv_stream_wv<8, YT>(p, pl, st)
             : pl.wv == 4 ? launch_gemv_stream_wv<4, YT>(p, pl, st)
                          : launch_gemv_stream_wv<2, YT>(p, pl, st);
    else
        rc = pl.wv == 4 ? launch_gemv_mfma_wv<4, YT>(p, pl, st) : launch_gemv_mfma_wv<3, YT>(p, pl, st);
    if (rc != PIO_OK) return rc;
    if (pl.splits > 1) {
        const int64_t MN = (int64_t)M * N;
        gemv_split_reduce_kernel<YT><<<(int)ceil_div(MN, (int64_t)256), 256, 0, st>>>((const float*)ws.ptr, pl.splits,
                                                                                      M, N, s_w, bias, y);
        PIO_LAUNCHED();
    }
    return PIO_OK;
}

// The W8 linear on the matrix cores (gemm_w8f.hip), for more than 4 rows.
int gemm_w8f(const void* x, int x_dtype, int64_t ldx, const int8_t* w, const float* s_w, const float* bias,
             void* y, int y_dtype, int64_t ldy, int M, int N, int K, bool resid, hipStream_t st);
constexpr int GEMV_MAX_FMA_ROWS = 4;

// Below this weight size a launch is bounded by its start-up (one HBM round
// trip), not by streaming: the direct kernel's one-wave-per-row-group grid
// reaches its first weight bytes sooner than the stream kernel, which first
// stages x through LDS in 1024-thread blocks (3 MB: 3.05 vs 3.9 us).
constexpr size_t GEMV_STREAM_MIN_BYTES = 16u << 20;

template <typename XT, typename YT>
static int dispatch(const XT* x, const int8_t* w, const float* s_w, const float* bias, YT* y,
                    int M, int N, int K, hipStream_t st) {
    if constexpr (std::is_same<XT, _Float16>::value) {
        GemvMfmaPlan pl = plan_gemv_stream(M, N, K);
        if (!pl.wv) pl = plan_gemv_mfma(M, N, K);
        if (pl.wv) return launch_gemv_mfma(x, w, s_w, bias, y, M, N, K, pl, st);
    }
    // More rows than one FMA launch serves: the MFMA GEMM reads W once, where
    // the FMA kernels would re-stream it every few rows.
    if (M > GEMV_MAX_FMA_ROWS)
        return gemm_w8f(x, std::is_same<XT, float>::value ? PIO_F32 : PIO_F16, K, w, s_w, bias, y,
                        std::is_same<YT, float>::value ? PIO_F32 : PIO_F16, N, M, N, K, false, st);
    if ((size_t)N * K >= GEMV_STREAM_MIN_BYTES && stream_pick(1, N, K)) {
        // x rows in launches of up to 4 (as many as the LDS takes); each launch re-streams W
        for (int m0 = 0; m0 < M;) {
            const int left = M - m0;
            const XT* xm = x + (int64_t)m0 * K;
            YT* ym = y + (int64_t)m0 * N;
            int rc, R;
            if (left >= 4 && (R = stream_pick(4, N, K))) {
                rc = launch_stream<4>(xm, w, s_w, bias, ym, N, K, R, st); m0 += 4;
            } else if (left >= 2 && (R = stream_pick(2, N, K))) {
                rc = launch_stream<2>(xm, w, s_w, bias, ym, N, K, R, st); m0 += 2;
            } else {
                R = stream_pick(1, N, K);
                rc = launch_stream<1>(xm, w, s_w, bias, ym, N, K, R, st); m0 += 1;
            }
            if (rc != PIO_OK) return rc;
        }
        return PIO_OK;
    }
    // few rows -> fewer rows per wave so the grid still spreads over the CUs
    if (N >= 32768) launch_direct_rows<4>(x, w, s_w, bias, y, M, N, K, st);
    else launch_direct_rows<2>(x, w, s_w, bias, y, M, N, K, st);
    return PIO_OK;
}

int gemv_w8(const void* x, int x_dtype, const int8_t* w, const float* s_w, const float* bias,
            void* y, int y_dtype, int M, int N, int K, hipStream_t st) {
    PIO_REQUIRE(x && w && s_w && y, "gemv_w8: null pointer");
    PIO_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemv_w8: negative shape");
    PIO_REQUIRE(K % 16 == 0, "gemv_w8: K=%d must be a multiple of 16", K);
    PIO_REQUIRE(aligned16(x) && aligned16(w), "gemv_w8: x and W must be 16-byte aligned");
    PIO_REQUIRE(x_dtype == PIO_F32 || x_dtype == PIO_F16, "gemv_w8: x must be fp32 or fp16");
    PIO_REQUIRE(y_dtype == PIO_F32 || y_dtype == PIO_F16, "gemv_w8: y must be fp32 or fp16");
    if (M == 0 || N == 0) return PIO_OK;
    int rc;
    if (x_dtype == PIO_F32) {
        if (y_dtype == PIO_F32) rc = dispatch((const float*)x, w, s_w, bias, (float*)y, M, N, K, st);
        else rc = dispatch((const float*)x, w, s_w, bias, (_Float16*)y, M, N, K, st);
    } else {
        if (y_dtype == PIO_F32) rc = dispatch((const _Float16*)x, w, s_w, bias, (float*)y, M, N, K, st);
        else rc = dispatch((const _Float16*)x, w, s_w, bias, (_Float16*)y, M, N, K, st);
    }
    if (rc != PIO_OK) return rc;
    PIO_LAUNCHED();
    return PIO_OK;
}

}  // namespace pio

using namespace pio;

PIO_EXPORT int pio_gemv_w8(const void* x, int x_dtype, const int8_t* w, const float* s_w,
                           const float* bias, void* y, int y_dtype, int M, int N, int K,
                           void* stream) {
    return gemv_w8(x, x_dtype, w, s_w, bias, y, y_dtype, M, N, K, pick_stream(stream));
}
