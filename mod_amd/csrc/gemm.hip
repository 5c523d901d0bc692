// W8A8 int8 GEMM on gfx950 MFMA (dense prefill linears and tensor_matmul_int8).
//   acc[m,n] = sum_k A[m,k] * B[n,k]          int32, exact (|acc| < 2^31 for K < 133144)
//   C[m,n]   = cvt(float(acc) * s_a[m] * s_w[n] (+ bias[n]))   or raw acc / float(acc)
// A int8 [M,K] (quantized activations), B int8 [N,K] (weights, K contiguous),
// both "K-major", so one v_mfma_i32_32x32x32_i8 consumes 16 contiguous bytes per
// lane from each. The tile engines live in gemm_core.hpp; this file holds the
// dense kernel (XCD-aware tile order, scale epilogue), the tile-shape choice and
// the tensor_matmul_int8 adapter (B given as [K,N] is transposed once).
#include "gemm_core.hpp"

#include <stdlib.h>
#include <algorithm>
#include <mutex>

namespace pio {

enum { OUT_F32 = 0, OUT_F16 = 1, OUT_I32 = 2, OUT_F32_RAW = 3 };

struct GemmParams {
    const int8_t* A;
    int64_t lda, a_batch;
    const int8_t* B;
    int64_t ldb, b_batch;
    const float* s_a;
    const float* s_w;
    const float* bias;
    void* C;
    int64_t ldc, c_batch;
    int M, N, K;
    int xr, xc;   // XCD rectangles: tile rows split xr ways, tile columns xc ways (xr*xc == 8), or 0
    unsigned long long* trace;   // traced launches only (pio_probe_gemm_timeline): 4 stamps per block
};

// Scaled output value of one int32 accumulator. Each product and the bias add
// round to f32 separately, and the value is rounded to f32 before an f16
// store, as the reference computes them: the empty operand barriers stop the
// compiler from fusing the product and the add into one FMA, or the product
// and the f16 conversion into one v_fma_mix (each rounds once).
template <int OUT>
__device__ __forceinline__ float scaled_value(int a, float sa, float sw, float bn, bool bias) {
    float val = (float)a * sa * sw;
    if (bias) {
        asm volatile("" : "+v"(val));
        val += bn;
    }
    if (OUT == OUT_F16) asm volatile("" : "+v"(val));
    return val;
}

template <int WMT, int WNT, int ENG, int S>
constexpr size_t engine_lds() {
    if constexpr (ENG == 2) return TileV2<WMT, WNT>::LDS_BYTES;
    else if constexpr (ENG == 5) return TileV5<WMT, WNT, S>::LDS_BYTES;
    else return TileV4<WMT>::LDS_BYTES;
}

// ----------------------------------------------------------------- v2 ---
// Dense W8A8 on the 32x32x32 engine. Block b is mapped XCD-aware: the
// dispatcher places block b on XCD b % 8, so each XCD is given one rectangle
// of the tile grid (tile rows split xr ways, columns xc ways, chosen on the
// host to minimize the A + B panel bytes one XCD's L2 has to hold); inside it,
// the XCD's blocks walk the rectangle row by row. Identity map when the grid
// does not split into 8 rectangles.
// ENG 2: register-staged v2 engine (any K % 16 == 0); 4: direct-to-LDS v4
// engine, square tiles, half-step ring (K % 128 == 0); 5: direct-to-LDS v5
// engine, S-stage ring on the v4 schedule (K % 128 == 0).
// TR: the traced build (pio_probe_gemm_timeline): thread 0 of every block
// stamps the 100 MHz constant clock at its start, after the K loop, after the
// epilogue's stores are issued and once they have completed.
template <int WMT, int WNT, int OUT, int ENG, int S, bool TR = false>
__global__ __launch_bounds__(256, 1) void gemm_v2_kernel(GemmParams p, int tiles_n) {
    using T = TileV2<WMT, WNT>;
    extern __shared__ __attribute__((aligned(16))) int8_t lds_v2[];
    const int b = blockIdx.x;
    unsigned long long ts[2] = {0, 0};
    if constexpr (TR) ts[0] = wall_clock64();
    int tr, tc;
    if (p.xr) {
        const int x = b % 8, k = b / 8;
        const int R = ((int)gridDim.x / tiles_n) / p.xr, Cc = tiles_n / p.xc;
        tr = (x / p.xc) * R + k / Cc;
        tc = (x % p.xc) * Cc + k % Cc;
    } else {
        tr = b / tiles_n;
        tc = b % tiles_n;
    }
    const int m0 = tr * T::BM, n0 = tc * T::BN, z = blockIdx.z;
    constexpr bool SCALED = (OUT == OUT_F32 || OUT == OUT_F16);
    // Interior tiles (the common case) take a branch-free epilogue: with no
    // per-element bounds checks the stores issue back to back, while a
    // bounds-checked store sequence makes the compiler wait for every earlier
    // store (gfx9 counts stores in vmcnt). Epilogue operands are loaded before
    // the main loop so their latency hides behind it -- except for the
    // 256 x 256 tile, whose 256 accumulator registers per lane leave no room:
    // it loads them after the loop.
    constexpr bool LATE = WMT * WNT >= 16;
    const bool full = (m0 + T::BM <= p.M) && (n0 + T::BN <= p.N);
    float sa[WMT][16], sw[WNT], bn[WNT];
    auto load_scales = [&]() {
#pragma unroll
        for (int i = 0; i < WMT; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) sa[i][e] = p.s_a[min(m0 + v2_row<WMT>(i, e), p.M - 1)];
#pragma unroll
        for (int j = 0; j < WNT; j++) {
            const int n = min(n0 + v2_col<WNT>(j), p.N - 1);
            sw[j] = p.s_w[n];
            bn[j] = p.bias ? p.bias[n] : 0.f;
        }
    };
    if (SCALED && !LATE) load_scales();
    v16i acc[WMT][WNT];
    const int8_t* A = p.A + z * p.a_batch + (int64_t)m0 * p.lda;
    const int8_t* B = p.B + z * p.b_batch + (int64_t)n0 * p.ldb;
    if constexpr (ENG == 2) mma_tile_v2<WMT, WNT>(A, p.lda, p.M - m0, B, p.ldb, p.N - n0, p.K, lds_v2, acc);
    else if constexpr (ENG == 5) mma_tile_v5<WMT, WNT, S>(A, p.lda, p.M - m0, B, p.ldb, p.N - n0, p.K, lds_v2, acc);
    else mma_tile_v4<WMT>(A, p.lda, p.M - m0, B, p.ldb, p.N - n0, p.K, lds_v2, acc);
    if constexpr (TR) ts[1] = wall_clock64();
    if (SCALED && LATE) load_scales();
    char* C = (char*)p.C + z * p.c_batch * (OUT == OUT_F16 ? 2 : 4);
    const bool has_bias = SCALED && p.bias;
    // off = m * ldc + n in 32 bits when the whole output fits (it does at every
    // shape this path serves; the 64-bit form stays for the rest)
    const bool small = (int64_t)p.M * p.ldc < (int64_t)INT32_MAX;
    auto store = [&](int i, int j, int e, int m, int n, bool bias) {
        const int64_t off = small ? (int64_t)(m * (int)p.ldc + n) : (int64_t)m * p.ldc + n;
        const int a = acc[i][j][e];
        if (OUT == OUT_I32) {
            ((int32_t*)C)[off] = a;
        } else if (OUT == OUT_F32_RAW) {
            ((float*)C)[off] = (float)a;
        } else {
            const float val = scaled_value<OUT>(a, sa[i][e], sw[j], bn[j], bias);
            if (OUT == OUT_F32) ((float*)C)[off] = val;
            else ((_Float16*)C)[off] = (_Float16)val;
        }
    };
    // Full tiles of a 16-byte-aligned output go out through LDS: the scaled
    // tile is written to LDS in the accumulator layout, then read back as
    // 16-byte row pieces, so every global store writes 16 contiguous bytes per
    // lane and whole 128-byte lines (from the accumulators a half-wave writes
    // 32 consecutive values, half a line in f16). Rows are padded by 32 bytes
    // so that the two half-waves of an LDS write (rows r and r + 4) fall on
    // different banks. The ring is free once every wave is past the barrier.
    // The stores are nontemporal: whole lines stream out while other
    // workgroups still compute, instead of waiting in the L2 for the
    // end-of-kernel writeback (C3's (2048, 3072) f16 output: 15.3 -> 14.2 us
    // with the staging, 13.1 us with the hint; 2-byte stores of half-lines
    // with the hint were slower than without).
    // traced build: the stamps after the stores are issued, and once every
    // thread's have completed
    auto finish = [&]() {
        if constexpr (TR) {
            const unsigned long long t2 = wall_clock64();
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (threadIdx.x == 0) {
                unsigned long long* tr = p.trace + (int64_t)(blockIdx.z * gridDim.x + b) * 4;
                tr[0] = ts[0];
                tr[1] = ts[1];
                tr[2] = t2;
                tr[3] = wall_clock64();
            }
        }
    };
    constexpr int ES = OUT == OUT_F16 ? 2 : 4;
    constexpr int SROW = T::BN * ES + 32;
    constexpr int CPR = T::BN * ES / 16;   // 16-byte pieces per tile row
    if constexpr ((size_t)T::BM * SROW <= engine_lds<WMT, WNT, ENG, S>() && (T::BM * CPR) % 256 == 0) {
        if (full && (p.ldc * ES) % 16 == 0 && ((uintptr_t)C & 15) == 0) {
            __syncthreads();
            auto put = [&](bool bias) {
#pragma unroll
                for (int j = 0; j < WNT; j++)
#pragma unroll
                    for (int i = 0; i < WMT; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            int8_t* d = lds_v2 + v2_row<WMT>(i, e) * SROW + v2_col<WNT>(j) * ES;
                            const int a = acc[i][j][e];
                            if (OUT == OUT_I32) {
                                *(int32_t*)d = a;
                            } else if (OUT == OUT_F32_RAW) {
                                *(float*)d = (float)a;
                            } else {
                                const float val = scaled_value<OUT>(a, sa[i][e], sw[j], bn[j], bias);
                                if (OUT == OUT_F32) *(float*)d = val;
                                else *(_Float16*)d = (_Float16)val;
                            }
                        }
            };
            if (has_bias) put(true);
            else put(false);
            __syncthreads();
            char* Ct = C + ((int64_t)m0 * p.ldc + n0) * ES;
#pragma unroll
            for (int it = 0; it < T::BM * CPR / 256; it++) {
                const int q = it * 256 + (int)threadIdx.x, r = q / CPR, ch = q % CPR;
                __builtin_nontemporal_store(*(const v4i*)(lds_v2 + r * SROW + ch * 16),
                                            (v4i*)(Ct + (int64_t)r * p.ldc * ES + ch * 16));
            }
            finish();
            return;
        }
    }
    if (full) {
        auto all = [&](bool bias) {
#pragma unroll
            for (int j = 0; j < WNT; j++)
#pragma unroll
                for (int i = 0; i < WMT; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        store(i, j, e, m0 + v2_row<WMT>(i, e), n0 + v2_col<WNT>(j), bias);
        };
        if (has_bias) all(true);
        else all(false);
    } else {
#pragma unroll
        for (int j = 0; j < WNT; j++) {
            const int n = n0 + v2_col<WNT>(j);
            if (n >= p.N) continue;
#pragma unroll
            for (int i = 0; i < WMT; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = m0 + v2_row<WMT>(i, e);
                    if (m < p.M) store(i, j, e, m, n, has_bias);
                }
        }
    }
    finish();
}

template <int WMT, int WNT, int OUT, int ENG, int S>
static int launch_v2_out(const GemmParams& p, dim3 grid, int tn, hipStream_t st) {
    constexpr size_t lds = engine_lds<WMT, WNT, ENG, S>();
    if constexpr (OUT == OUT_F16 && ENG == 5) {
        // the traced build exists for the f16-out direct-to-LDS engine (C3)
        if (p.trace) {
            PIO_TRY((allow_lds<gemm_v2_kernel<WMT, WNT, OUT, ENG, S, true>>(lds)));
            gemm_v2_kernel<WMT, WNT, OUT, ENG, S, true><<<grid, 256, lds, st>>>(p, tn);
            PIO_LAUNCHED();
            return PIO_OK;
        }
    }
    PIO_REQUIRE(!p.trace, "gemm: the traced build covers the f16-out direct-to-LDS engine only");
    PIO_TRY(allow_lds<gemm_v2_kernel<WMT, WNT, OUT, ENG, S>>(lds));
    gemm_v2_kernel<WMT, WNT, OUT, ENG, S><<<grid, 256, lds, st>>>(p, tn);
    PIO_LAUNCHED();
    return PIO_OK;
}

template <int WMT, int WNT, int ENG, int S>
static int launch_v2_s(const GemmParams& p, int out_mode, dim3 grid, int tn, hipStream_t st) {
    switch (out_mode) {
    case OUT_F32: return launch_v2_out<WMT, WNT, OUT_F32, ENG, S>(p, grid, tn, st);
    case OUT_F16: return launch_v2_out<WMT, WNT, OUT_F16, ENG, S>(p, grid, tn, st);
    case OUT_I32: return launch_v2_out<WMT, WNT, OUT_I32, ENG, S>(p, grid, tn, st);
    case OUT_F32_RAW: return launch_v2_out<WMT, WNT, OUT_F32_RAW, ENG, S>(p, grid, tn, st);
    default: return set_error(PIO_ERR_INVALID, "gemm: bad output mode");
    }
}

// XCD rectangle split of a tm x tn tile grid: the (xr, xc), xr * xc = 8,
// with the fewest A + B rows per rectangle; (0, 0) if none divides the grid.
static void xcd_split(int tm, int tn, int BM, int BN, int& xr, int& xc) {
    xr = xc = 0;
    int64_t best = -1;
    for (int r = 1; r <= 8; r *= 2) {
        const int c = 8 / r;
        if (tm % r || tn % c) continue;
        const int64_t rows = (int64_t)(tm / r) * BM + (int64_t)(tn / c) * BN;
        if (best < 0 || rows < best) { best = rows; xr = r; xc = c; }
    }
}

// Direct-to-LDS engines need 16-byte aligned rows and K a multiple of the step.
static bool direct_ok(const GemmParams& p, int kstep) {
    return aligned16(p.A) && aligned16(p.B) && p.lda % 16 == 0 && p.ldb % 16 == 0 && p.K % kstep == 0;
}

template <int WMT, int WNT>
static int launch_v2(const GemmParams& p0, int out_mode, int batch, hipStream_t st) {
    using T = TileV2<WMT, WNT>;
    const int tn = ceil_div(p0.N, T::BN), tm = ceil_div(p0.M, T::BM);
    dim3 grid(tm * tn, 1, batch);
    GemmParams p = p0;
    xcd_split(tm, tn, T::BM, T::BN, p.xr, p.xc);
    if constexpr (WMT * WNT >= 16) {
        // 256 x 256: the half-step-ring engine (the caller checked its conditions)
        return launch_v2_s<WMT, WNT, 4, 0>(p, out_mode, grid, tn, st);
    } else {
        if (direct_ok(p, 128)) return launch_v2_s<WMT, WNT, 5, v5_stages<WMT, WNT>()>(p, out_mode, grid, tn, st);
        return launch_v2_s<WMT, WNT, 2, 0>(p, out_mode, grid, tn, st);
    }
}

// Picks the block tile: 256 x 256 when it fills every CU (its LDS and operand
// traffic per MFMA is the lowest), else among BM = 128 and BN in {64, 128,
// 192, 256} the one whose tile count best fills whole waves of the CUs (ties
// go to the larger tile).
static int launch_dense(const GemmParams& p, int out_mode, int batch, hipStream_t st) {
    const int64_t cus = 256;
    const int64_t big = (int64_t)ceil_div(p.M, 256) * ceil_div(p.N, 256) * batch;
    if (direct_ok(p, 128) && big >= cus && (double)big / (double)(((big + cus - 1) / cus) * cus) >= 0.9)
        return launch_v2<4, 4>(p, out_mode, batch, st);
    static const int cfg[][2] = {{2, 4}, {2, 3}, {2, 2}, {2, 1}};
    int best = 0;
    double best_eff = -1.0;
    for (int i = 0; i < 4; i++) {
        const int64_t tiles = (int64_t)ceil_div(p.M, 64 * cfg[i][0]) * ceil_div(p.N, 64 * cfg[i][1]) * batch;
        const int64_t rounds = (tiles + cus - 1) / cus;
        const double eff = (double)tiles / (double)(rounds * cus);
        if (eff > best_eff + 1e-9) { best_eff = eff; best = i; }
    }
    switch (best) {
    case 0: return launch_v2<2, 4>(p, out_mode, batch, st);
    case 1: return launch_v2<2, 3>(p, out_mode, batch, st);
    case 2: return launch_v2<2, 2>(p, out_mode, batch, st);
    default: return launch_v2<2, 1>(p, out_mode, batch, st);
    }
}

// ---------------------------------------------------------- split-K ---
// Skinny products (few tile rows: decode batches, MoE-free small-M linears)
// leave most CUs idle with one tile per output block. The split-K path runs
// `splits` K slices of every output tile as the batch dimension of the dense
// kernel (slice z reads A and B from column z*Kc, same row pitch) into int32
// partials ws[z][M][N], then splitk_reduce_kernel sums the slices in slice
// order and applies the epilogue. Integer sums are exact, so the result is
// bit-identical to the one-pass kernel's for every output type.
template <int OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const int32_t* __restrict__ ws, int splits,
                                                            int M, int N, const float* __restrict__ s_a,
                                                            const float* __restrict__ s_w,
                                                            const float* __restrict__ bias, void* C) {
    const int64_t MN = (int64_t)M * N;
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= MN) return;
    // Every load at a clamped index, with no branch around it (a guarded load
    // waits for the previous one): the epilogue operands first, then the
    // partials four slices at a time, added in slice order.
    float sa[4], sw[4], bb[4];
    if constexpr (OUT != OUT_I32) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int64_t i = min(i0 + u, MN - 1);
            const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
            sa[u] = s_a[m];
            sw[u] = s_w[n];
            bb[u] = bias ? bias[n] : 0.f;
        }
    }
    int acc[4] = {0, 0, 0, 0};
    const bool vec = (N % 4) == 0;   // then the four elements share a row and 16 B alignment
    for (int z0 = 0; z0 < splits; z0 += 4) {
        int v[4][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int32_t* src = ws + (int64_t)min(z0 + j, splits - 1) * MN;
            if (vec) {
                const int4 t = *(const int4*)(src + i0);
                v[j][0] = t.x; v[j][1] = t.y; v[j][2] = t.z; v[j][3] = t.w;
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++) v[j][u] = src[min(i0 + u, MN - 1)];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (z0 + j < splits)
#pragma unroll
                for (int u = 0; u < 4; u++) acc[u] += v[j][u];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int64_t i = i0 + u;
        if (i >= MN) break;
        if constexpr (OUT == OUT_I32) {
            ((int32_t*)C)[i] = acc[u];
        } else {
            const float val = scaled_value<OUT>(acc[u], sa[u], sw[u], bb[u], bias != nullptr);
            if constexpr (OUT == OUT_F32) ((float*)C)[i] = val;
            else ((_Float16*)C)[i] = (_Float16)val;
        }
    }
}

// ---------------------------------------------------------- skinny ---
// W8A8 with few activation rows (M <= 64: decode batches, small prefills).
// Such a product is bound by streaming the weights once (N*K bytes), not by
// the MFMA, so the kernel is built like the GEMV: each wave owns 16 weight
// rows and streams them from HBM straight into registers, SK_D blocks of 256 K
// ahead, already in the operand layout of v_mfma_i32_16x16x64_i8 (lane: row
// r = lane % 16 and K chunk q = lane / 16, i.e. the 16 bytes at 64*i + 16*q of
// MFMA i's 64-K step), so each load instruction reads 64 contiguous bytes of
// each of 16 rows. The workgroup's whole activation slice (MT*16 rows x the
// slice's K) is copied into LDS once, up front, with direct-to-LDS loads, and
// read there with the same per-lane K chunks, so each product pairs the same
// K. After that the loop only streams weights: no barriers, and the waits on
// the weight registers are exact (the K loop is unrolled per block count NB;
// vector-memory loads complete in order, so any activation load inside the
// loop would make its wait drain the weight prefetch). Grid x: weight row
// tiles of 16*WV; grid y: K slices (int32 partials for splitk_reduce_kernel
// when there is more than one).
constexpr int SK_KB = 256;                // K per block: 4 MFMAs of 64

// Epilogue operands of the skinny kernels' scaled outputs, loaded at the
// kernel's start with clamped indices (lane: column r = lane % 16, rows
// 16 t + 4 (lane / 16) + v): the store loop skips rows past M, and a load
// inside it waited for the previous one, MT x 4 round trips after the K loop.
template <int MT>
struct SkEpi {
    float sa[MT][4];
    float sw, bn;
};
template <int MT, int OUT>
__device__ __forceinline__ SkEpi<MT> sk_epi_load(const GemmParams& p, int n0, int lane) {
    SkEpi<MT> e;
    if constexpr (OUT == OUT_I32) {
        e.sw = e.bn = 0.f;
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) e.sa[t][v] = 0.f;
    } else {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) e.sa[t][v] = p.s_a[min(t * 16 + 4 * (lane >> 4) + v, p.M - 1)];
        const int n = min(n0 + (lane & 15), p.N - 1);
        e.sw = p.s_w[n];
        e.bn = p.bias ? p.bias[n] : 0.f;
    }
    return e;
}
constexpr int SK_D = 4;                   // weight blocks in flight per wave (8 measured no faster)

typedef __attribute__((address_space(1))) const v4i sk_gv4i;

// LDS row pitch of the activation slice: K + 16, so rows start 4 banks apart.
template <int NB>
constexpr int sk_pitch() { return NB * SK_KB + 16; }
template <int MT, int NB>
constexpr size_t sk_lds_bytes() { return (size_t)MT * 16 * sk_pitch<NB>(); }

template <int WV, int MT, int NB, int OUT>
__global__ __launch_bounds__(64 * WV) void skinny_w8a8_kernel(GemmParams p) {
    typedef __attribute__((address_space(3))) void lds_t;
    constexpr int D = NB < SK_D ? NB : SK_D;
    constexpr int P = sk_pitch<NB>();
    constexpr int SEG = NB * SK_KB / 1024;         // 1 KB segments per activation row
    constexpr int NCP = MT * 16 * SEG;             // copies (wave instructions) of the slice
    extern __shared__ __attribute__((aligned(16))) int8_t sk_lds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * (16 * WV) + w * 16;
    const int64_t k0 = (int64_t)blockIdx.y * p.K;          // p.K is the K of one slice
    // older than every copy and weight load, so the waits below cover them
    const SkEpi<MT> epi = sk_epi_load<MT, OUT>(p, n0, lane);

    // Activation slice -> LDS: copy u moves row u / SEG, segment u % SEG (lane l
    // lands 16 B at LDS offset 16*l of the segment). Rows >= M re-read row M-1;
    // they only feed accumulator rows that are never stored.
#pragma unroll
    for (int j = 0; j < (NCP + WV - 1) / WV; j++) {
        const int u = w + WV * j;
        if (NCP % WV == 0 || u < NCP) {
            const int row = u / SEG, seg = u % SEG;
            const int8_t* src = p.A + (int64_t)min(row, p.M - 1) * p.lda + k0 + seg * 1024 + 16 * lane;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_t*)(sk_lds + row * P + seg * 1024), 16, 0, 0);
        }
    }
    // The copies must be issued before the weight prefetch: loads complete in
    // order, and the wait below (at most 4*D loads outstanding) covers the
    // copies only if the 4*D weight loads are the youngest. Without this fence
    // the scheduler may hoist weight loads above the copies.
    __builtin_amdgcn_sched_barrier(0);
    // This lane's weight row, clamped: rows past N are computed, never stored.
    const int8_t* wp = p.B + (int64_t)min(n0 + r, p.N - 1) * p.ldb + k0 + 16 * q;
    v4i wr[D][4];
    // loads 2j and 2j + 1 read the two halves of one 128-byte line of each
    // row: the first an ordinary load, the second (the line's last use)
    // nontemporal; all-nontemporal loses the line's second half, all-ordinary
    // fills the L2 with dead lines (each measured up to 13% slower)
    auto load_w = [&](int b, v4i (&dst)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            dst[i] = (i & 1) ? __builtin_nontemporal_load((sk_gv4i*)(wp + b * SK_KB + 64 * i))
                             : *(sk_gv4i*)(wp + b * SK_KB + 64 * i);
    };
#pragma unroll
    for (int b = 0; b < D; b++) load_w(b, wr[b]);
    // The slice copies are older than the weight prefetch: wait for them only.
    stage_barrier<4 * D>();

    v4i acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = v4i{0, 0, 0, 0};
    const int8_t* as = sk_lds + r * P + 16 * q;
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i a = *(const v4i*)(as + t * 16 * P + b * SK_KB + 64 * i);
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wr[b % D][i], acc[t], 0, 0, 0);
            }
        }
        if (b + D < NB) load_w(b + D, wr[b % D]);
        // Keep the reload here, right after the block that freed its
        // registers: left alone, the scheduler sinks it next to its use (to
        // save registers), which leaves no weight loads in flight.
        __builtin_amdgcn_sched_barrier(0);
    }

    // 16x16 accumulator: lane holds rows 4*q + v (v < 4) of M tile t, column r.
    const int n = n0 + r;
    if (n >= p.N) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int m = t * 16 + 4 * q + v;
            if (m >= p.M) continue;
            const int64_t o = (int64_t)blockIdx.y * p.c_batch + (int64_t)m * p.ldc + n;
            if constexpr (OUT == OUT_I32) {
                ((int32_t*)p.C)[o] = acc[t][v];
            } else {
                const float val = scaled_value<OUT>(acc[t][v], epi.sa[t][v], epi.sw, epi.bn, p.bias != nullptr);
                if constexpr (OUT == OUT_F32) ((float*)p.C)[o] = val;
                else ((_Float16*)p.C)[o] = (_Float16)val;
            }
        }
    }
}

// ------------------------------------------------------ streamed skinny ---
// W8A8 for 16 < M <= 64 (prefill tails, small batches). The one-pass skinny
// kernel above keeps a workgroup's whole activation slice in LDS, which at 64
// rows holds only 2 KB of K and forces K slices plus a reduce. Here the
// activations stream with the weights instead: per K block of 256, every wave
// loads its 16 weight rows into registers (as above) and its share of the 64
// activation rows x 256 B into an LDS ring stage with direct-to-LDS copies,
// both SS_D blocks ahead, and one barrier per block makes the stage visible to
// the workgroup. The ring has SS_D + 1 stages: the stage a block's copies
// overwrite was last read one block earlier, which every wave has finished
// when it passes the current block's barrier. LDS rows are 256 B with the
// 16-byte chunks XOR-swizzled by row (chunk c of row r at c ^ (r & 15)), so
// the MFMA operand reads (16 rows, one chunk) are conflict-free; the copies
// pick their global chunk to land that way. The weights load as in the
// one-pass kernel: each load covers half of a 128-byte line per row, the
// first half with an ordinary load and the second (last use) nontemporal.
constexpr int SS_D = 3;                      // K blocks in flight (3-6 measured alike; 3 leaves LDS for 2 workgroups)
constexpr int SS_S = SS_D + 1;               // activation ring stages
constexpr int SS_STAGE = 64 * SK_KB;         // 64 rows x 256 B
constexpr size_t SS_LDS = (size_t)SS_S * SS_STAGE;

template <int WV, int NB, int OUT>
__global__ __launch_bounds__(64 * WV) void skinny_stream_kernel(GemmParams p) {
    typedef __attribute__((address_space(3))) void lds_t;
    static_assert(16 % WV == 0, "16 activation copies per block, shared evenly");
    constexpr int D = NB < SS_D ? NB : SS_D;
    constexpr int CPW = 16 / WV;                 // 1 KB copies per wave per block
    constexpr int L = 4 + CPW;                   // vector-memory ops per wave per block
    extern __shared__ __attribute__((aligned(16))) int8_t ss_lds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * (16 * WV) + w * 16;
    const int64_t k0 = (int64_t)blockIdx.y * p.K;          // p.K is the K of one slice
    // older than every copy and weight load, so the waits below cover them
    const SkEpi<4> epi = sk_epi_load<4, OUT>(p, n0, lane);

    // copy j of this wave moves activation rows 4u .. 4u + 3 (u = w + WV j):
    // lane l lands its 16 B at stage offset 1024 u + 16 l, i.e. row 4u + l / 16,
    // chunk position l % 16, holding the row's chunk (l % 16) ^ (row % 16)
    const int8_t* asrc[CPW];
    int adst[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const int u = w + WV * j, row = 4 * u + (lane >> 4), c = (lane & 15) ^ (row & 15);
        asrc[j] = p.A + (int64_t)min(row, p.M - 1) * p.lda + k0 + c * 16;
        adst[j] = u * 1024;
    }
    const int8_t* wp = p.B + (int64_t)min(n0 + r, p.N - 1) * p.ldb + k0 + 16 * q;
    v4i wr[D][4];
    auto issue = [&](int b) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            wr[b % D][i] = (i & 1) ? __builtin_nontemporal_load((sk_gv4i*)(wp + b * SK_KB + 64 * i))
                                   : *(sk_gv4i*)(wp + b * SK_KB + 64 * i);   // as the one-pass kernel
        int8_t* st = ss_lds + (b % SS_S) * SS_STAGE;
#pragma unroll
        for (int j = 0; j < CPW; j++)
            __builtin_amdgcn_global_load_lds((const void*)(asrc[j] + b * SK_KB), (lds_t*)(st + adst[j]), 16, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int b = 0; b < D; b++) issue(b);

    v4i acc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) acc[t] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < NB; b++) {
        // block b landed (this wave's loads and copies), then every wave's copies
        if (NB - 1 - b >= D - 1) stage_barrier<(D - 1) * L>();
        else stage_barrier_steps<L, (D > 1 ? D - 1 : 0)>(NB - 1 - b);
        const int8_t* st = ss_lds + (b % SS_S) * SS_STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int row = 16 * t + r;
                const v4i a = *(const v4i*)(st + row * SK_KB + (((4 * i + q) ^ r) << 4));
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wr[b % D][i], acc[t], 0, 0, 0);
            }
        }
        if (b + D < NB) issue(b + D);
    }

    // 16x16 accumulator: lane holds rows 4*q + v (v < 4) of M tile t, column r.
    const int n = n0 + r;
    if (n >= p.N) return;
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int m = t * 16 + 4 * q + v;
            if (m >= p.M) continue;
            const int64_t o = (int64_t)blockIdx.y * p.c_batch + (int64_t)m * p.ldc + n;
            if constexpr (OUT == OUT_I32) {
                ((int32_t*)p.C)[o] = acc[t][v];
            } else {
                const float val = scaled_value<OUT>(acc[t][v], epi.sa[t][v], epi.sw, epi.bn, p.bias != nullptr);
                if constexpr (OUT == OUT_F32) ((float*)p.C)[o] = val;
                else ((_Float16*)p.C)[o] = (_Float16)val;
            }
        }
    }
}

struct SkinnyPlan {
    int wv = 0, nb = 0, splits = 1;
    bool stream = false;   // the streamed kernel (16 < M <= 64)
};

// Streamed plan for 16 < M <= 64: the bytes a CU moves (each unit: 16*WV
// weight rows and the 64 activation rows, NB blocks of 256 B) at ~100 GB/s
// per CU, units spread over the 256 CUs (two workgroups fit a CU's LDS), plus
// the split path's int32 partials and reduce launch.
static SkinnyPlan plan_skinny_stream(const GemmParams& p) {
    SkinnyPlan best;
    if (p.M <= 16 || p.M > 64 || p.K % 1024 || !aligned16(p.A) || !aligned16(p.B) || p.lda % 16 ||
        p.ldb % 16)
        return best;
    const int kb = p.K / SK_KB;
    double best_t = 0;
    for (int wv : {8, 4, 2}) {
        for (int nb : {16, 12, 8, 6, 4}) {
            if (kb % nb) continue;
            const int sp = kb / nb;
            if (sp > 16) continue;
            const int64_t units = (int64_t)ceil_div(p.N, 16 * wv) * sp;
            const double per_cu = (double)((units + 255) / 256) * nb * SK_KB * (16.0 * wv + 64.0);
            double t = per_cu / 100.0e9;
            if (sp > 1) t += (double)sp * p.M * p.N * 8.0 / 4.0e12 + 2.0e-6;
            if (best.wv == 0 || t < best_t * 0.98) {
                best_t = t;
                best.wv = wv; best.nb = nb; best.splits = sp; best.stream = true;
            }
        }
    }
    return best;
}

template <int WV, int NB, int OUT>
static int launch_stream_out(const GemmParams& p, int splits, hipStream_t st) {
    PIO_TRY(allow_lds<skinny_stream_kernel<WV, NB, OUT>>(SS_LDS));
    skinny_stream_kernel<WV, NB, OUT><<<dim3(ceil_div(p.N, 16 * WV), splits), 64 * WV, SS_LDS, st>>>(p);
    PIO_LAUNCHED();
    return PIO_OK;
}
template <int WV, int NB>
static int launch_stream_nb(const GemmParams& p, int out_mode, int splits, hipStream_t st) {
    switch (out_mode) {
    case OUT_I32: return launch_stream_out<WV, NB, OUT_I32>(p, splits, st);
    case OUT_F32: return launch_stream_out<WV, NB, OUT_F32>(p, splits, st);
    case OUT_F16: return launch_stream_out<WV, NB, OUT_F16>(p, splits, st);
    default: return set_error(PIO_ERR_INVALID, "gemm: bad output mode");
    }
}
template <int WV>
static int launch_stream_wv(const GemmParams& p, int out_mode, const SkinnyPlan& sp, hipStream_t st) {
    switch (sp.nb) {
    case 16: return launch_stream_nb<WV, 16>(p, out_mode, sp.splits, st);
    case 12: return launch_stream_nb<WV, 12>(p, out_mode, sp.splits, st);
    case 8: return launch_stream_nb<WV, 8>(p, out_mode, sp.splits, st);
    case 6: return launch_stream_nb<WV, 6>(p, out_mode, sp.splits, st);
    case 4: return launch_stream_nb<WV, 4>(p, out_mode, sp.splits, st);
    default: return set_error(PIO_ERR_INVALID, "gemm: streamed plan with %d blocks", sp.nb);
    }
}
static int launch_stream_one(const GemmParams& p, int out_mode, const SkinnyPlan& sp, hipStream_t st) {
    if (sp.wv == 8) return launch_stream_wv<8>(p, out_mode, sp, st);
    if (sp.wv == 4) return launch_stream_wv<4>(p, out_mode, sp, st);
    return launch_stream_wv<2>(p, out_mode, sp, st);
}

// Plan for the skinny kernel, or wv == 0 when it does not apply (M > 64, K not
// a multiple of 1024, or unaligned operands). Cost model: the weights stream
// at ~6 TB/s when every CU has a workgroup (proportionally less on a partly
// filled grid), a workgroup moves its 16*WV rows x NB blocks at ~32 GB/s at
// most (its loads in flight over the HBM latency), and split K adds the
// partials' write + read and the reduce launch.
static SkinnyPlan plan_skinny(const GemmParams& p) {
    SkinnyPlan best;
    if (p.M < 1 || p.M > 64 || p.K % 1024 || !aligned16(p.A) || !aligned16(p.B) || p.lda % 16 || p.ldb % 16)
        return best;
    const int kb = p.K / SK_KB;
    double best_t = 0;
    for (int wv : {4, 3}) {
        for (int nb : {16, 12, 8, 4}) {
            // the activation slice lives in LDS: 64 rows x 2 KB at most
            if (kb % nb || kb / nb > 16 || (p.M > 16 && nb > 8)) continue;
            const int sp = kb / nb;
            const int64_t units = (int64_t)ceil_div(p.N, 16 * wv) * sp;
            const double rounds = (double)((units + 255) / 256);
            const double fill = std::min(1.0, (double)units / 256.0);
            double t = std::max((double)p.N * p.K / (6.0e12 * fill), rounds * 16.0 * wv * nb * SK_KB / 32.0e9);
            if (sp > 1) t += (double)sp * p.M * p.N * 8.0 / 4.0e12 + 2.0e-6;
            if (best.wv == 0 || t < best_t * 0.98) {
                best_t = t;
                best.wv = wv; best.nb = nb; best.splits = sp;
            }
        }
    }
    return best;
}

template <int WV, int MT, int NB, int OUT>
static int launch_skinny_out(const GemmParams& p, int splits, hipStream_t st) {
    constexpr size_t lds = sk_lds_bytes<MT, NB>();
    PIO_TRY(allow_lds<skinny_w8a8_kernel<WV, MT, NB, OUT>>(lds));
    skinny_w8a8_kernel<WV, MT, NB, OUT><<<dim3(ceil_div(p.N, 16 * WV), splits), 64 * WV, lds, st>>>(p);
    PIO_LAUNCHED();
    return PIO_OK;
}

template <int WV, int MT, int NB>
static int launch_skinny_nb(const GemmParams& p, int out_mode, int splits, hipStream_t st) {
    switch (out_mode) {
    case OUT_I32: return launch_skinny_out<WV, MT, NB, OUT_I32>(p, splits, st);
    case OUT_F32: return launch_skinny_out<WV, MT, NB, OUT_F32>(p, splits, st);
    case OUT_F16: return launch_skinny_out<WV, MT, NB, OUT_F16>(p, splits, st);
    default: return set_error(PIO_ERR_INVALID, "gemm: bad output mode");
    }
}

template <int WV, int MT>
static int launch_skinny_mt(const GemmParams& p, int out_mode, const SkinnyPlan& sp, hipStream_t st) {
    if constexpr (MT == 1) {
        if (sp.nb == 16) return launch_skinny_nb<WV, MT, 16>(p, out_mode, sp.splits, st);
        if (sp.nb == 12) return launch_skinny_nb<WV, MT, 12>(p, out_mode, sp.splits, st);
    }
    if (sp.nb == 8) return launch_skinny_nb<WV, MT, 8>(p, out_mode, sp.splits, st);
    if (sp.nb == 4) return launch_skinny_nb<WV, MT, 4>(p, out_mode, sp.splits, st);
    return set_error(PIO_ERR_INVALID, "gemm: skinny plan with %d blocks for %d rows", sp.nb, p.M);
}

static int launch_skinny_one(const GemmParams& p, int out_mode, const SkinnyPlan& sp, hipStream_t st) {
    if (sp.stream) return launch_stream_one(p, out_mode, sp, st);
    if (sp.wv == 4)
        return p.M <= 16 ? launch_skinny_mt<4, 1>(p, out_mode, sp, st) : launch_skinny_mt<4, 4>(p, out_mode, sp, st);
    return p.M <= 16 ? launch_skinny_mt<3, 1>(p, out_mode, sp, st) : launch_skinny_mt<3, 4>(p, out_mode, sp, st);
}

// Split-K plan: block tile (WMT x WNT waves of 32 x 32) and slice count.
struct SplitPlan {
    int wmt = 0, wnt = 0, splits = 1;
};

// Cost model for skinny products (M <= 256): a tile's time is its copy
// traffic per CU (BM + BN rows of Kc bytes through the LDS) plus a fixed
// start-up per round (the first copies' latency before the ring is full,
// ~1.5 us, counted as the 96 KB a CU copies meanwhile), times the rounds of
// units over the CUs, plus the split path's int32 partials (written and read
// back, spread over the CUs). The one-pass launch is costed with the tile
// launch_dense would choose; a split plan is taken when it is at least 10%
// cheaper. Slices are multiples of 128 bytes (the direct-to-LDS step) and at
// least 512 (4 steps, so the copy ring overlaps). 64-row tiles when M <= 64
// (a 128-row tile copies duplicated A rows).
static SplitPlan plan_split(const GemmParams& p, int cus) {
    SplitPlan best;
    if (!direct_ok(p, 128) || p.M > 256) return best;
    constexpr double RAMP = 96.0 * 1024;
    auto rounds = [&](int64_t units) { return (double)((units + cus - 1) / cus); };
    double base = 0, best_eff = -1.0;
    {
        static const int cfg[] = {4, 3, 2, 1};
        for (int wnt : cfg) {
            const int64_t tiles = (int64_t)ceil_div(p.M, 128) * ceil_div(p.N, 64 * wnt);
            const double eff = (double)tiles / (rounds(tiles) * cus);
            if (eff > best_eff + 1e-9) {
                best_eff = eff;
                base = rounds(tiles) * ((128.0 + 64.0 * wnt) * p.K + RAMP);
            }
        }
    }
    double best_cost = 0.9 * base;
    const int wmt = p.M <= 64 ? 1 : 2;
    for (int wnt : {4, 2, 1}) {
        const int64_t tiles = (int64_t)ceil_div(p.M, 64 * wmt) * ceil_div(p.N, 64 * wnt);
        for (int sp : {2, 3, 4, 6, 8}) {
            if (p.K % (sp * 128) || p.K / sp < 512) continue;
            const double cost = rounds(tiles * sp) * ((64.0 * (wmt + wnt)) * (p.K / sp) + RAMP) +
                                (double)sp * p.M * p.N * 8.0 / cus;
            if (cost < best_cost) {
                best_cost = cost;
                best.wmt = wmt; best.wnt = wnt; best.splits = sp;
            }
        }
    }
    return best;
}

template <int WMT, int WNT>
static int launch_split_tiles(const GemmParams& p, int splits, hipStream_t st) {
    using T = TileV5<WMT, WNT, v5_stages<WMT, WNT>()>;
    const int tn = ceil_div(p.N, T::BN), tm = ceil_div(p.M, T::BM);
    return launch_v2_out<WMT, WNT, OUT_I32, 5, v5_stages<WMT, WNT>()>(p, dim3(tm * tn, 1, splits), tn, st);
}

static int splitk_reduce(const int32_t* w, int splits, const GemmParams& p0, int out_mode, hipStream_t st);

// Workspace of one GEMM call: the caller's buffer when it brings one (`ext`,
// `cap` bytes), else a block from the caching allocator for the call's scope.
struct GemmWs {
    void* ext = nullptr;
    size_t cap = 0;
    const char* ext_name = "";
    Scratch own;
    void* ptr = nullptr;
    int get(size_t bytes, hipStream_t st) {
        if (!ext) {
            PIO_TRY(own.get(bytes, st));
            ptr = own.ptr;
            return PIO_OK;
        }
        if (bytes > cap)
            return set_error(PIO_ERR_INVALID, "%s: this shape's plan needs %zu B of workspace, "
                             "more than the %zu B it has", ext_name, bytes, cap);
        ptr = ext;
        return PIO_OK;
    }
};

static int launch_splitk(const GemmParams& p0, int out_mode, const SplitPlan& sp, GemmWs& ws,
                         hipStream_t st) {
    PIO_TRY(ws.get((size_t)sp.splits * p0.M * p0.N * sizeof(int32_t), st));
    GemmParams p = p0;
    p.a_batch = p.b_batch = p0.K / sp.splits;   // slice z starts at column z*Kc
    p.K = p0.K / sp.splits;
    p.C = ws.ptr;
    p.ldc = p0.N;
    p.c_batch = (int64_t)p0.M * p0.N;
    p.s_a = p.s_w = p.bias = nullptr;
    p.xr = p.xc = 0;
    int rc;
    if (sp.wmt == 1) {
        rc = sp.wnt == 4 ? launch_split_tiles<1, 4>(p, sp.splits, st)
           : sp.wnt == 2 ? launch_split_tiles<1, 2>(p, sp.splits, st)
                         : launch_split_tiles<1, 1>(p, sp.splits, st);
    } else {
        rc = sp.wnt == 4 ? launch_split_tiles<2, 4>(p, sp.splits, st)
           : sp.wnt == 2 ? launch_split_tiles<2, 2>(p, sp.splits, st)
                         : launch_split_tiles<2, 1>(p, sp.splits, st);
    }
    if (rc != PIO_OK) return rc;
    return splitk_reduce((const int32_t*)ws.ptr, sp.splits, p0, out_mode, st);
}

// Sums the int32 partials ws[splits][M][N] in slice order and applies the
// epilogue into p0.C (ldc == N).
static int splitk_reduce(const int32_t* w, int splits, const GemmParams& p0, int out_mode, hipStream_t st) {
    const int64_t MN = (int64_t)p0.M * p0.N;
    const int blocks = (int)ceil_div(MN, (int64_t)1024);
    switch (out_mode) {
    case OUT_I32: splitk_reduce_kernel<OUT_I32><<<blocks, 256, 0, st>>>(w, splits, p0.M, p0.N, nullptr, nullptr, nullptr, p0.C); break;
    case OUT_F32: splitk_reduce_kernel<OUT_F32><<<blocks, 256, 0, st>>>(w, splits, p0.M, p0.N, p0.s_a, p0.s_w, p0.bias, p0.C); break;
    case OUT_F16: splitk_reduce_kernel<OUT_F16><<<blocks, 256, 0, st>>>(w, splits, p0.M, p0.N, p0.s_a, p0.s_w, p0.bias, p0.C); break;
    default: return set_error(PIO_ERR_INVALID, "gemm: bad output mode");
    }
    PIO_LAUNCHED();
    return PIO_OK;
}

// Skinny product: one pass, or K slices into int32 partials plus the reduce.
static int launch_skinny(const GemmParams& p0, int out_mode, const SkinnyPlan& sp, GemmWs& ws,
                         hipStream_t st) {
    GemmParams p = p0;
    p.K = p0.K / sp.splits;
    if (sp.splits == 1) {
        p.c_batch = 0;
        return launch_skinny_one(p, out_mode, sp, st);
    }
    PIO_TRY(ws.get((size_t)sp.splits * p0.M * p0.N * sizeof(int32_t), st));
    p.C = ws.ptr;
    p.ldc = p0.N;
    p.c_batch = (int64_t)p0.M * p0.N;
    PIO_TRY(launch_skinny_one(p, OUT_I32, sp, st));
    return splitk_reduce((const int32_t*)ws.ptr, sp.splits, p0, out_mode, st);
}

// The W8A8 product with its workspace from `ws_ext` (`ws_cap` bytes) when
// given, else from the caching allocator; the plan (and so every output bit)
// is the same either way.
static int gemm_w8a8_ws(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
                        const float* bias, void* y, int y_dtype, int M, int N, int K,
                        void* ws_ext, size_t ws_cap, const char* ws_name, hipStream_t st) {
    PIO_REQUIRE(q && w && y, "gemm_w8a8: null pointer");
    PIO_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemm_w8a8: negative shape");
    PIO_REQUIRE(K % 16 == 0, "gemm_w8a8: K=%d must be a multiple of 16", K);
    PIO_REQUIRE(aligned16(q) && aligned16(w), "gemm_w8a8: operands must be 16-byte aligned");
    int mode;
    if (y_dtype == PIO_I32) mode = OUT_I32;
    else if (y_dtype == PIO_F32) mode = OUT_F32;
    else if (y_dtype == PIO_F16) mode = OUT_F16;
    else return set_error(PIO_ERR_INVALID, "gemm_w8a8: bad output dtype %d", y_dtype);
    if (mode != OUT_I32) PIO_REQUIRE(s_a && s_w, "gemm_w8a8: null scales");
    if (M == 0 || N == 0) return PIO_OK;
    GemmParams p{};
    p.A = q; p.lda = K;
    p.B = w; p.ldb = K;
    p.s_a = s_a; p.s_w = s_w; p.bias = bias;
    p.C = y; p.ldc = N;
    p.M = M; p.N = N; p.K = K;
    GemmWs ws;
    ws.ext = ws_ext;
    ws.cap = ws_cap;
    ws.ext_name = ws_name;
    SkinnyPlan kp = plan_skinny_stream(p);
    if (!kp.wv) kp = plan_skinny(p);
    if (kp.wv) return launch_skinny(p, mode, kp, ws, st);
    const SplitPlan sp = plan_split(p, 256);
    if (sp.splits > 1) return launch_splitk(p, mode, sp, ws, st);
    return launch_dense(p, mode, 1, st);
}

int gemm_w8a8(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
              const float* bias, void* y, int y_dtype, int M, int N, int K, hipStream_t st) {
    return gemm_w8a8_ws(q, s_a, w, s_w, bias, y, y_dtype, M, N, K, nullptr, 0, "", st);
}

// ---- the allocation-free variant ------------------------------------------
// Workspace of pio_gemm_w8a8_static: one array per GPU, loaded with this code
// object and held until the process ends. Host code uses the device address
// that hipGetSymbolAddress returns for it (per device), never the name.
constexpr size_t STATIC_SCRATCH_BYTES = size_t(16) << 20;
static __device__ __align__(256) char scratch[STATIC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES];

// Device address of this GPU's scratch array (looked up on the first call on
// each device, with that device current).
static int static_scratch(void** out) {
    int dev = 0;
    PIO_HIP(hipGetDevice(&dev));
    PIO_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "gemm_w8a8_static: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        PIO_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        PIO_REQUIRE(ptr, "gemm_w8a8_static: no device address for the scratch array");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return PIO_OK;
}

// [K,N] -> [N,Kp] int8 transpose, zero-filled for K <= k < Kp: one 64 x 64
// tile per block (per batch z). Thread (r, c) = (tid / 4, tid % 4) reads 16
// bytes of k row k0 + r (n0 + 16c ..) and writes 16 bytes of n row n0 + r
// (k0 + 16c ..), one 16-byte access each; the byte transpose happens in LDS,
// whose rows are 68 bytes apart so that the four k chunks a wave reads per
// byte fall in different banks. dst is 16-byte aligned and Kp % 16 == 0, so
// every write is one aligned chunk; the reads go byte by byte on the right and
// bottom edges and wherever vec is 0 (N % 16 != 0 or src unaligned).
__global__ __launch_bounds__(256) void transpose_i8_kernel(const int8_t* __restrict__ src,
                                                           int8_t* __restrict__ dst, int K, int N,
                                                           int Kp, int64_t sbatch, int64_t dbatch,
                                                           int vec) {
    constexpr int LS = 68;
    __shared__ __align__(16) uint32_t t[64 * LS / 4];
    const uint8_t* tb = (const uint8_t*)t;
    const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    src += blockIdx.z * sbatch;
    dst += blockIdx.z * dbatch;
    const int r = threadIdx.x >> 2, c = threadIdx.x & 3;
    {
        const int k = k0 + r, n = n0 + 16 * c;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (vec && k < K && n + 16 <= N) {
            const uint4 v = *(const uint4*)(src + (int64_t)k * N + n);
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else if (k < K) {
            for (int j = 0; j < 16; j++)
                if (n + j < N) w[j >> 2] |= (uint32_t)(uint8_t)src[(int64_t)k * N + n + j] << (8 * (j & 3));
        }
#pragma unroll
        for (int i = 0; i < 4; i++) t[r * (LS / 4) + 4 * c + i] = w[i];
    }
    __syncthreads();
    const int n = n0 + r, k = k0 + 16 * c;
    if (n < N && k < Kp) {   // Kp % 16 == 0, so the whole chunk is inside the row
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint8_t* col = tb + (16 * c + 4 * i) * LS + r;
            w[i] = (uint32_t)col[0] | (uint32_t)col[LS] << 8 | (uint32_t)col[2 * LS] << 16 |
                   (uint32_t)col[3 * LS] << 24;
        }
        *(uint4*)(dst + (int64_t)n * Kp + k) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

static int padded_k(int K) { return (K + 15) / 16 * 16; }

}  // namespace pio

using namespace pio;

PIO_EXPORT int pio_gemm_w8a8(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
                             const float* bias, void* y, int y_dtype, int M, int N, int K,
                             void* stream) {
    return gemm_w8a8(q, s_a, w, s_w, bias, y, y_dtype, M, N, K, pick_stream(stream));
}

// Per-block timeline of the dense W8A8 GEMM (f16 out, the direct-to-LDS
// engine: the C3 path): the same tile choice and launch as pio_gemm_w8a8 for
// a shape that runs dense, through the kernel's traced build. trace receives
// 4 stamps per block (100 MHz constant clock: start, K loop done, stores
// issued, stores complete), in block order. Returns how many 4-word entries
// to read -- the block count of the largest tile grid the launch can pick;
// entries of blocks the chosen grid does not have stay 0 -- or a negative
// status.
PIO_EXPORT int pio_probe_gemm_timeline(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
                                       void* y, int M, int N, int K, unsigned long long* trace, int trace_words,
                                       void* stream) {
    PIO_REQUIRE(q && s_a && w && s_w && y && trace, "pio_probe_gemm_timeline: null pointer");
    PIO_REQUIRE(M > 0 && N > 0 && K > 0 && K % 128 == 0 && aligned16(q) && aligned16(w),
                "pio_probe_gemm_timeline: shape or alignment outside the direct-to-LDS engine");
    GemmParams p{};
    p.A = q; p.lda = K;
    p.B = w; p.ldb = K;
    p.s_a = s_a; p.s_w = s_w;
    p.C = y; p.ldc = N;
    p.M = M; p.N = N; p.K = K;
    PIO_REQUIRE(!plan_skinny_stream(p).wv && !plan_skinny(p).wv && plan_split(p, 256).splits <= 1,
                "pio_probe_gemm_timeline: this shape does not run on the dense kernel");
    int64_t blocks = 0;
    for (int wnt : {4, 3, 2, 1}) blocks = std::max<int64_t>(blocks, (int64_t)ceil_div(M, 128) * ceil_div(N, 64 * wnt));
    blocks = std::max<int64_t>(blocks, (int64_t)ceil_div(M, 256) * ceil_div(N, 256));
    PIO_REQUIRE(trace_words >= 4 * blocks, "pio_probe_gemm_timeline: trace holds %d words, need %lld", trace_words,
                (long long)(4 * blocks));
    p.trace = trace;
    const hipStream_t st = pick_stream(stream);
    PIO_HIP(hipMemsetAsync(trace, 0, (size_t)trace_words * 8, st));
    PIO_TRY(launch_dense(p, OUT_F16, 1, st));
    return (int)blocks;
}

// pio_gemm_w8a8 without any allocation: the K-slice partials live in the
// library's per-GPU static scratch array (16 MiB). Same kernels, same bits.
// Calls that overlap on one GPU (different streams) share that array and race.
PIO_EXPORT int pio_gemm_w8a8_static(const int8_t* q, const float* s_a, const int8_t* w,
                                    const float* s_w, const float* bias, void* y, int y_dtype,
                                    int M, int N, int K, void* stream) {
    void* ptr = nullptr;
    PIO_TRY(static_scratch(&ptr));
    return gemm_w8a8_ws(q, s_a, w, s_w, bias, y, y_dtype, M, N, K, ptr, STATIC_SCRATCH_BYTES,
                        "pio_gemm_w8a8_static (static scratch; pio_gemm_w8a8 serves larger shapes)",
                        pick_stream(stream));
}

// Workspace: B repacked to [batch][N][Kp] (Kp = K rounded up to 16, zero
// padded) and, when K % 16 != 0, A repacked to [batch][M][Kp].
static size_t matmul_ws(int batch, int M, int K, int N) {
    const size_t Kp = padded_k(K);
    size_t b = (size_t)batch * N * Kp;
    size_t a = (K % 16) ? (size_t)batch * M * Kp : 0;
    return (b + 255) / 256 * 256 + a;
}

PIO_EXPORT size_t pio_matmul_int8_workspace(int batch, int M, int K, int N) {
    return matmul_ws(batch, M, K, N);
}

// Row copy of A [M,K] into [M,Kp] with zero padding (only when K % 16 != 0).
__global__ void pad_rows_i8_kernel(const int8_t* __restrict__ src, int8_t* __restrict__ dst, int M,
                                   int K, int Kp) {
    const int64_t n = (int64_t)M * Kp;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / Kp, c = i % Kp;
        dst[i] = c < K ? src[r * K + c] : (int8_t)0;
    }
}

static int matmul_int8_impl(const int8_t* a, const int8_t* b, void* c, int out_i32, int batch,
                            int M, int K, int N, void* ws, hipStream_t st) {
    PIO_REQUIRE(a && b && c, "matmul_int8: null pointer");
    PIO_REQUIRE(batch >= 1 && M >= 0 && K >= 0 && N >= 0, "matmul_int8: bad shape");
    if (M == 0 || N == 0) return PIO_OK;
    const int Kp = padded_k(K);
    Scratch own;
    if (!ws) {
        PIO_TRY(own.get(matmul_ws(batch, M, K, N), st));
        ws = own.ptr;
    }
    PIO_REQUIRE(aligned16(ws), "matmul_int8: the workspace must be 16-byte aligned");
    int8_t* bt = (int8_t*)ws;
    const size_t bt_bytes = ((size_t)batch * N * Kp + 255) / 256 * 256;
    dim3 tg(ceil_div(N, 64), ceil_div(Kp > 0 ? Kp : 1, 64), batch);
    transpose_i8_kernel<<<tg, 256, 0, st>>>(b, bt, K, N, Kp, (int64_t)K * N, (int64_t)N * Kp,
                                            aligned16(b) && N % 16 == 0);
    PIO_LAUNCHED();
    const int8_t* ap = a;
    if (K % 16) {
        int8_t* apad = bt + bt_bytes;
        for (int z = 0; z < batch; z++) {
            pad_rows_i8_kernel<<<256, 256, 0, st>>>(a + (int64_t)z * M * K,
                                                    apad + (int64_t)z * M * Kp, M, K, Kp);
            PIO_LAUNCHED();
        }
        ap = apad;
    }
    if (!aligned16(ap)) {
        // Unaligned A (a sub-view): repack through the workspace path.
        return set_error(PIO_ERR_INVALID, "matmul_int8: A must be 16-byte aligned");
    }
    GemmParams p{};
    p.A = ap; p.lda = Kp; p.a_batch = (int64_t)M * Kp;
    p.B = bt; p.ldb = Kp; p.b_batch = (int64_t)N * Kp;
    p.C = c; p.ldc = N; p.c_batch = (int64_t)M * N;
    p.M = M; p.N = N; p.K = Kp;
    return launch_dense(p, out_i32 ? OUT_I32 : OUT_F32_RAW, batch, st);
}

PIO_EXPORT int pio_matmul_int8(const int8_t* a, const int8_t* b, void* c, int out_i32, int batch,
                               int M, int K, int N, void* workspace, void* stream) {
    return matmul_int8_impl(a, b, c, out_i32, batch, M, K, N, workspace, pick_stream(stream));
}

static int matmul_int8_tensor(Tensor* a, Tensor* b, Tensor* out, int out_i32) {
    PIO_TRY(check_device_tensor(a, "matmul_int8 a"));
    PIO_TRY(check_device_tensor(b, "matmul_int8 b"));
    PIO_TRY(check_device_tensor(out, "matmul_int8 out"));
    PIO_REQUIRE(a->ndim >= 2 && b->ndim >= 2, "matmul_int8: operands must be >= 2-D");
    const int M = a->shape[a->ndim - 2], K = a->shape[a->ndim - 1];
    const int Kb = b->shape[b->ndim - 2], N = b->shape[b->ndim - 1];
    PIO_REQUIRE(K == Kb, "matmul_int8: inner dims differ (%d vs %d)", K, Kb);
    PIO_REQUIRE(M > 0 && N > 0, "matmul_int8: empty operand");
    const int batch = out->size / (M * N);   // tensor_ops.c:223
    PIO_REQUIRE(batch >= 1 && (int64_t)batch * M * N == out->size,
                "matmul_int8: out size %d is not a multiple of M*N", out->size);
    PIO_REQUIRE((int64_t)a->size >= (int64_t)batch * M * K && (int64_t)b->size >= (int64_t)batch * K * N,
                "matmul_int8: operands too small for batch %d", batch);
    return matmul_int8_impl((const int8_t*)a->data, (const int8_t*)b->data, out->data, out_i32,
                            batch, M, K, N, nullptr, current_stream());
}

PIO_EXPORT int tensor_matmul_int8_status(Tensor* a, Tensor* b, Tensor* out) {
    return matmul_int8_tensor(a, b, out, 0);
}
PIO_EXPORT void tensor_matmul_int8(Tensor* a, Tensor* b, Tensor* out) {
    matmul_int8_tensor(a, b, out, 0);
}
PIO_EXPORT int tensor_matmul_int8_i32_status(Tensor* a, Tensor* b, Tensor* out) {
    return matmul_int8_tensor(a, b, out, 1);
}
PIO_EXPORT void tensor_matmul_int8_i32(Tensor* a, Tensor* b, Tensor* out) {
    matmul_int8_tensor(a, b, out, 1);
}
