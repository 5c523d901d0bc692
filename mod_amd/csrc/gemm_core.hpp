// Int8 MFMA tile engine shared by the dense W8A8 GEMM and the grouped MoE GEMM.
//
// One 256-thread block computes a 128x128 int32 tile of A[M,K] * B[N,K]^T with
// v_mfma_i32_16x16x64_i8. 4 waves in a 2x2 grid each own 64x64 = 4x4 MFMA
// tiles. Operands go global -> registers -> LDS (double buffered, row stride
// padded 64 -> 80 B so one ds_read_b128 phase of 16 lanes touches 16 distinct
// 16-byte bank groups) and the next K step's global loads are in flight while
// the current step's 16 MFMAs run.
//
// MFMA operand layout (16x16xK, K = 64 per instruction): lane l supplies A row
// (l % 16) and B column (l % 16) with K bytes [16*(l/16), 16*(l/16)+16) of the
// step. A and B use the same per-lane K assignment, so every A[m,k] meets
// B[n,k] exactly once whatever order the unit sums in. Accumulator layout: lane
// l holds D[4*(l/16) + v][l % 16], v = 0..3.
#pragma once
#include "pio_common.hpp"

namespace pio {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int TM = 128, TN = 128, TK = 64, TLDS = 80;
constexpr int TILE_LDS_BYTES = 2 * (TM + TN) * TLDS;   // 40 KB

struct TileSrc {
    const int8_t* A;        // row 0 of the tile (ignored rows beyond m_rem)
    const int32_t* a_rows;  // optional: A row r of the tile is A_base + a_rows[r] * lda
    int64_t lda;
    int m_rem;              // valid rows in this tile (may exceed TM)
    const int8_t* B;        // row 0 (= output column n0) of the tile
    int64_t ldb;
    int n_rem;
    int K;                  // multiple of 16
};

// Computes acc (per the layout above) for one tile. `lds` must hold
// TILE_LDS_BYTES bytes, 16-byte aligned. Ends with a __syncthreads so the caller
// may reuse `lds` right away.
__device__ __forceinline__ void mma_tile_128(const TileSrc& s, int8_t* lds, v4i (&acc)[4][4]) {
    int8_t* As = lds;
    int8_t* Bs = lds + 2 * TM * TLDS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int8_t* ga[2];
    const int8_t* gb[2];
    bool va[2], vb[2];
    int soff[2], scol[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int idx = tid + 256 * j;
        const int row = idx >> 2;
        scol[j] = (idx & 3) * 16;
        soff[j] = row * TLDS + scol[j];
        va[j] = row < s.m_rem;
        vb[j] = row < s.n_rem;
        int64_t ar = va[j] ? (s.a_rows ? (int64_t)s.a_rows[row] : row) : 0;
        ga[j] = s.A + ar * s.lda + scol[j];
        gb[j] = s.B + (int64_t)(vb[j] ? row : 0) * s.ldb + scol[j];
    }

    v4i ra[2], rb[2];
    const int K = s.K;
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const bool kin = k0 + scol[j] < K;
            ra[j] = (va[j] && kin) ? *(const v4i*)(ga[j] + k0) : v4i{0, 0, 0, 0};
            rb[j] = (vb[j] && kin) ? *(const v4i*)(gb[j] + k0) : v4i{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            *(v4i*)&As[buf * TM * TLDS + soff[j]] = ra[j];
            *(v4i*)&Bs[buf * TN * TLDS + soff[j]] = rb[j];
        }
    };

#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = v4i{0, 0, 0, 0};

    const int nk = (K + TK - 1) / TK;
    gload(0);
    sstore(0);
    __syncthreads();

    const int fr = lane & 15, fk = (lane >> 4) * 16;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * TK);
        v4i a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            a[i] = *(const v4i*)&As[cur * TM * TLDS + (wm * 64 + i * 16 + fr) * TLDS + fk];
#pragma unroll
        for (int j = 0; j < 4; j++)
            b[j] = *(const v4i*)&Bs[cur * TN * TLDS + (wn * 64 + j * 16 + fr) * TLDS + fk];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }
}

// Tile-relative coordinates of accumulator element (i, j, v) for this lane.
__device__ __forceinline__ int acc_row(int i, int v) {
    const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) >> 1;
    return wm * 64 + i * 16 + (lane >> 4) * 4 + v;
}
__device__ __forceinline__ int acc_col(int j) {
    const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) & 1;
    return wn * 64 + j * 16 + (lane & 15);
}

}  // namespace pio
