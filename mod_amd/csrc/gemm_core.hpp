// Int8 MFMA tile engines shared by the dense W8A8 GEMM and the grouped MoE GEMM.
#pragma once
#include "pio_common.hpp"

namespace pio {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Dense tile engine v2: v_mfma_i32_32x32x32_i8, K step 128 bytes.
//
// Block = 256 threads = 2x2 waves; a wave owns WMT x WNT MFMA tiles of 32x32,
// so the block tile is BM = 64*WMT by BN = 64*WNT. LDS rows are 128 bytes (one
// K step) with no padding; 16-byte chunk c of row r is stored at slot
// c ^ ((r >> 1) & 7), which puts the 16 lanes of every ds_read_b128 phase (16
// consecutive rows, same chunk) on 16 distinct 4-bank groups.
//
// MFMA 32x32x32 operand layout: lane l supplies A row (l % 32) and B column
// (l % 32), 16 K bytes starting at 16 * (l / 32) of a 32-byte K slice (A and B
// identically, so the unit's internal K order cannot matter). Accumulator:
// lane l holds D[8*(i/4) + 4*(l/32) + (i%4)][l % 32], i = 0..15.
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

template <int WMT, int WNT>
struct TileV2 {
    static constexpr int BM = 64 * WMT, BN = 64 * WNT, BK = 128;
    static constexpr int A_CHUNKS = BM * 8 / 256;   // 16-byte chunks per thread per K step
    static constexpr int B_CHUNKS = BN * 8 / 256;
    static constexpr int STAGE = (BM + BN) * BK;     // bytes per LDS stage
    static constexpr int LDS_BYTES = 2 * STAGE;
};

// Computes the block tile's int32 accumulators. A rows [0, m_rem) and B rows
// [0, n_rem) are valid (others read as zero); K % 16 == 0.
template <int WMT, int WNT>
__device__ __forceinline__ void mma_tile_v2(const int8_t* __restrict__ A, int64_t lda, int m_rem,
                                            const int8_t* __restrict__ B, int64_t ldb, int n_rem,
                                            int K, int8_t* lds, v16i (&acc)[WMT][WNT]) {
    using T = TileV2<WMT, WNT>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // Global chunk assignment: chunk idx -> (row idx/8, col idx%8).
    const int8_t* ga[T::A_CHUNKS];
    const int8_t* gb[T::B_CHUNKS];
    int la[T::A_CHUNKS], lb[T::B_CHUNKS], ca[T::A_CHUNKS], cb[T::B_CHUNKS];
    bool va[T::A_CHUNKS], vb[T::B_CHUNKS];
#pragma unroll
    for (int j = 0; j < T::A_CHUNKS; j++) {
        const int idx = tid + 256 * j, r = idx >> 3, c = idx & 7;
        va[j] = r < m_rem;
        ga[j] = A + (int64_t)(va[j] ? r : 0) * lda + c * 16;
        ca[j] = c * 16;
        la[j] = swz(r, c);
    }
#pragma unroll
    for (int j = 0; j < T::B_CHUNKS; j++) {
        const int idx = tid + 256 * j, r = idx >> 3, c = idx & 7;
        vb[j] = r < n_rem;
        gb[j] = B + (int64_t)(vb[j] ? r : 0) * ldb + c * 16;
        cb[j] = c * 16;
        lb[j] = T::BM * 128 + swz(r, c);
    }
    v4i ra[T::A_CHUNKS], rb[T::B_CHUNKS];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < T::A_CHUNKS; j++)
            ra[j] = (va[j] && k0 + ca[j] < K) ? *(const v4i*)(ga[j] + k0) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < T::B_CHUNKS; j++)
            rb[j] = (vb[j] && k0 + cb[j] < K) ? *(const v4i*)(gb[j] + k0) : v4i{0, 0, 0, 0};
    };
    auto sstore = [&](int buf) {
        int8_t* base = lds + buf * T::STAGE;
#pragma unroll
        for (int j = 0; j < T::A_CHUNKS; j++) *(v4i*)(base + la[j]) = ra[j];
#pragma unroll
        for (int j = 0; j < T::B_CHUNKS; j++) *(v4i*)(base + lb[j]) = rb[j];
    };

#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int j = 0; j < WNT; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

    const int nk = (K + T::BK - 1) / T::BK;
    gload(0);
    sstore(0);
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * T::BK);
        const int8_t* base = lds + cur * T::STAGE;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int c = 2 * ks + fh;
            v4i a[WMT], b[WNT];
#pragma unroll
            for (int i = 0; i < WMT; i++) {
                const int r = wm * 32 * WMT + i * 32 + fr;
                a[i] = *(const v4i*)(base + swz(r, c));
            }
#pragma unroll
            for (int j = 0; j < WNT; j++) {
                const int r = wn * 32 * WNT + j * 32 + fr;
                b[j] = *(const v4i*)(base + T::BM * 128 + swz(r, c));
            }
#pragma unroll
            for (int i = 0; i < WMT; i++)
#pragma unroll
                for (int j = 0; j < WNT; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }
}

// Tile-relative row / column of accumulator element e of MFMA tile (i, j).
template <int WMT>
__device__ __forceinline__ int v2_row(int i, int e) {
    const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) >> 1;
    return wm * 32 * WMT + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
template <int WNT>
__device__ __forceinline__ int v2_col(int j) {
    const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) & 1;
    return wn * 32 * WNT + j * 32 + (lane & 31);
}

}  // namespace pio

namespace pio {

// ---------------------------------------------------------------------------
// Direct-to-LDS copies (engines v4 and v5): global_load_lds_dwordx4 moves a
// 1 KB block = 8 rows x 128 B per wave instruction, whole cache lines: lane l
// lands at LDS byte 16*l of the block, i.e. row l/8, slot l%8, so it fetches
// global chunk (l%8) ^ ((row >> 1) & 7) -- the v2 swizzle applied on the read
// side of the copy. Requires K % 128 == 0 (a K tail cannot be zero-filled on
// this path). Rows past m_rem / n_rem re-read the last valid row; they only
// feed output rows / columns the caller discards.

// Waits until at most N vector-memory loads of this wave are outstanding and
// all its LDS operations are done, then joins the workgroup barrier. Unlike
// __syncthreads() (whose workgroup fence waits for *every* outstanding load,
// vmcnt(0)), this keeps the later stages' global->LDS loads in flight. The
// empty asm statements stop the compiler from moving memory accesses across.
template <int N>
__device__ __forceinline__ void stage_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// stage_barrier<n * L>() for a wave-uniform n in [0, MAXN].
template <int L, int MAXN>
__device__ __forceinline__ void stage_barrier_steps(int n) {
    if constexpr (MAXN > 0) {
        if (n >= MAXN) {
            stage_barrier<MAXN * L>();
            return;
        }
        stage_barrier_steps<L, MAXN - 1>(n);
    } else {
        stage_barrier<0>();
    }
}

// ---------------------------------------------------------------------------
// Dense tile engine v4, for the big square block tile (256 x 256: each wave
// 128 x 128 = 4 x 4 MFMA tiles, so one ds_read_b128 fragment feeds 4 MFMAs).
// A K step is 128 bytes: a copy instruction moves 8 rows x 128 B, whole cache
// lines (copies of 16 rows x 64 B -- half lines -- fill the LDS at little
// more than half the rate). A full step of both operands is 64 KB, so
// the LDS holds the A slice and the B slice of a step as separate 32 KB
// halves in a ring of 5 (160 KB): half h = 2*step + (0: A, 1: B) sits in slot
// h % 5. While step kt is multiplied, the halves of steps kt+1 (B) and kt+2
// (A) are being copied -- the only slots not holding step kt or kt+1's A.
// Slot layout: 16-byte chunk c of row r at c ^ ((r >> 1) & 7).
template <int WT>
struct TileV4 {
    static constexpr int BM = 64 * WT, BN = 64 * WT, BK = 128, SLOTS = 5;
    static constexpr int BLK = BM / 8;                 // 1 KiB copies per half
    static constexpr int PER_WAVE = BLK / 4;            // per wave per half
    static constexpr int HALF = BM * BK;                // bytes per half
    static constexpr int LDS_BYTES = SLOTS * HALF;
    static_assert(BLK % 4 == 0, "tile rows per wave");
};

template <int WT>
__device__ __forceinline__ void mma_tile_v4(const int8_t* __restrict__ A, int64_t lda, int m_rem,
                                            const int8_t* __restrict__ B, int64_t ldb, int n_rem,
                                            int K, int8_t* lds, v16i (&acc)[WT][WT]) {
    using T = TileV4<WT>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int8_t* ga[T::PER_WAVE];
    const int8_t* gb[T::PER_WAVE];
#pragma unroll
    for (int j = 0; j < T::PER_WAVE; j++) {
        const int q = j * 4 + wave, r = q * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        ga[j] = A + (int64_t)min(r, m_rem - 1) * lda + c * 16;
        gb[j] = B + (int64_t)min(r, n_rem - 1) * ldb + c * 16;
    }
    typedef __attribute__((address_space(3))) void lds_t;
    const int nk = K / T::BK, nh = 2 * nk;
    // copy j of this wave's share of half h (A slice of step h/2 if h is even,
    // else B). Issued for every h, also past the end (the last step again, into
    // a slot nothing reads any more), so no copy sits behind a branch and the
    // wait counts stay constant.
    auto copy = [&](int h, int j) {
        int8_t* base = lds + (h % T::SLOTS) * T::HALF;
        const int k0 = min(h >> 1, nk - 1) * T::BK;
        __builtin_amdgcn_global_load_lds((const void*)(((h & 1) ? gb[j] : ga[j]) + k0),
                                         (lds_t*)(base + (j * 4 + wave) * 1024), 16, 0, 0);
    };

#pragma unroll
    for (int i = 0; i < WT; i++)
#pragma unroll
        for (int j = 0; j < WT; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

    if (nk <= 0) return;
#pragma unroll
    for (int h = 0; h < 3; h++)
#pragma unroll
        for (int j = 0; j < T::PER_WAVE; j++) copy(h, j);
    const int fr = lane & 31, fh = lane >> 5;
    // fragment q of sub-step ks: q < WT an A fragment, else a B fragment
    auto frag1 = [&](const int8_t* a_base, const int8_t* b_base, int ks, int q, v4i (&a)[WT], v4i (&b)[WT]) {
        const int c = 2 * ks + fh;
        if (q < WT) a[q] = *(const v4i*)(a_base + swz(wm * 32 * WT + q * 32 + fr, c));
        else b[q - WT] = *(const v4i*)(b_base + swz(wn * 32 * WT + (q - WT) * 32 + fr, c));
    };
    // One sub-step: its WT*WT MFMAs, with the next sub-step's 2*WT fragment
    // reads and (h >= 0) the PER_WAVE copies of half h placed one at a time
    // between MFMA pairs, in this order exactly (scheduling barriers): a burst
    // of copies stalls the wave, and with one wave per SIMD that idles the
    // MFMA unit.
    static_assert(2 * WT == T::PER_WAVE && WT * WT == 4 * WT, "one MFMA pair, read and copy per slot");
    auto substep = [&](const v4i (&a)[WT], const v4i (&b)[WT], const int8_t* na, const int8_t* nb, int nks,
                       v4i (&a2)[WT], v4i (&b2)[WT], int h) {
#pragma unroll
        for (int q = 0; q < 2 * WT; q++) {
            const int i = q >> 1, j0 = (q & 1) * 2;
            acc[i][j0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j0], acc[i][j0], 0, 0, 0);
            acc[i][j0 + 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j0 + 1], acc[i][j0 + 1], 0, 0, 0);
            // the reads go two per slot from the second slot on: they land long
            // before the next sub-step needs them, and the previous sub-step's
            // MFMAs (whose operand registers they overwrite) are long issued
            if (q >= 1 && q <= WT) {
                frag1(na, nb, nks, 2 * (q - 1), a2, b2);
                frag1(na, nb, nks, 2 * (q - 1) + 1, a2, b2);
            }
            if (h >= 0) copy(h, q);
            __builtin_amdgcn_sched_barrier(0);
        }
        // keep this sub-step's operands live to its end, so the register
        // allocator cannot give a next-sub-step read a register that an MFMA
        // issued just before still reads
#pragma unroll
        for (int i = 0; i < WT; i++) asm volatile("" ::"v"(a[i]), "v"(b[i]));
    };
    // One barrier per step, before its last sub-step: by then every wave has
    // read all of step kt's fragments (sub-step 3's were read during sub-step
    // 2), so step kt's slots may be refilled from the next step on, and step
    // kt+1's halves are waited for here and its first fragments read while
    // sub-step 3's MFMAs run.
    // Halves issued: 0..2 before the loop, 2kt+3 during sub-step 0 of step kt
    // and 2kt+4 during its sub-step 1; step j's halves are complete once only
    // the newest half (2j+4) may still be in flight.
    v4i fa[2][WT], fb[2][WT];
    stage_barrier<T::PER_WAVE>();
#pragma unroll
    for (int q = 0; q < 2 * WT; q++) frag1(lds, lds + T::HALF, 0, q, fa[0], fb[0]);
    for (int kt = 0; kt < nk; kt++) {
        const int8_t* a_base = lds + ((2 * kt) % T::SLOTS) * T::HALF;
        const int8_t* b_base = lds + ((2 * kt + 1) % T::SLOTS) * T::HALF;
        // B of kt+1 and A of kt+2 go into the slots of step kt-1, which every
        // wave finished reading before step kt-1's barrier
        substep(fa[0], fb[0], a_base, b_base, 1, fa[1], fb[1], 2 * kt + 3);
        substep(fa[1], fb[1], a_base, b_base, 2, fa[0], fb[0], 2 * kt + 4);
        substep(fa[0], fb[0], a_base, b_base, 3, fa[1], fb[1], -1);
        stage_barrier<T::PER_WAVE>();
        substep(fa[1], fb[1], lds + ((2 * kt + 2) % T::SLOTS) * T::HALF,
                lds + ((2 * kt + 3) % T::SLOTS) * T::HALF, 0, fa[0], fb[0], -1);
    }
    // the copies issued past the end must land before the wave moves on
    stage_barrier<0>();
}

// ---------------------------------------------------------------------------
// Dense tile engine v5: 2 x 2 waves of WMT x WNT MFMA tiles (the v2 tiling),
// an S-stage LDS ring of whole K steps filled by 8-row x 128 B direct copies,
// run on the v4 schedule:
//   - one barrier per K step, before its last sub-step: by then every wave has
//     read all of step kt's fragments, and step kt+1's stage is waited for, so
//     its first fragments are read while the last sub-step's MFMAs run;
//   - the copies of step kt+S-1 (into the slot of step kt-1, which every wave
//     finished reading before step kt-1's barrier) are spread over sub-steps
//     0-2 of step kt, and the next sub-step's fragment reads over the first
//     half of each sub-step, one at a time between the MFMAs (scheduling
//     barriers pin the order: a burst of copies stalls the only wave on the
//     SIMD);
//   - the loop runs in two parts: while step kt+S-1 exists every sub-step's
//     copies are issued unconditionally and the wait count is a constant; the
//     last S-1 steps copy nothing (a short K would otherwise spend a third of
//     its copy bandwidth on steps past the end) and wait for whatever is left.
// Fragments rotate through four register sets (sub-step ks uses set ks) and
// each sub-step keeps its own and the previous sub-step's operands alive to
// its end, so a fragment read never lands in a register an MFMA issued within
// the last sub-step still reads.
template <int WMT, int WNT, int S>
struct TileV5 {
    static constexpr int BM = 64 * WMT, BN = 64 * WNT, BK = 128, STAGES = S;
    static constexpr int A_PW = BM / 32, B_PW = BN / 32;   // 1 KiB copies per wave per step
    static constexpr int LOADS = A_PW + B_PW;
    static constexpr int STAGE = (BM + BN) * BK;
    static constexpr int LDS_BYTES = S * STAGE;
    static_assert(S >= 3 && (S - 2) * LOADS < 64, "ring depth / vmcnt range");
};

// ---------------------------------------------------------------------------
// Tile engine v6, for products that stream their weights from HBM (MoE
// experts): global_load_lds copies of 8 rows x 128 B reach ~4.4 TB/s from
// HBM, while plain 16-byte loads of the same rows into registers, written to
// LDS by the wave, reach ~6.1 TB/s with 8+ waves per CU. Block = 8 waves
// (2 x 4): wave (wm = w & 1, wn = w >> 1) owns WMT x WNT 32x32 MFMA tiles, so
// the block tile is BM = 64*WMT by BN = 128*WNT. Every wave loads L = (BM +
// BN) / 64 rows-of-8 blocks (1 KiB each) per K step, D steps ahead, into
// register sets; at step kt it multiplies LDS stage kt % 2, then writes step
// kt+1's set into the other stage (layout and swizzle as v4/v5) and refills
// the set with step kt+D+1. D steps are unrolled per loop iteration, so each
// register set has a static name; the compiler's vmcnt tracking waits for the
// set being written and keeps the later steps' loads in flight.
template <int WMT, int WNT, int D>
struct TileV6 {
    static constexpr int BM = 64 * WMT, BN = 128 * WNT, BK = 128;
    static constexpr int L = (BM + BN) / 64;   // 1 KiB copies per wave per step (8 waves)
    static constexpr int STAGE = (BM + BN) * BK;
    static constexpr int LDS_BYTES = 2 * STAGE;
    static_assert(D >= 2, "prefetch depth");
};

// LDS writes complete, then the workgroup barrier (no wait on vector memory).
__device__ __forceinline__ void v6_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Tile-relative row / column of accumulator element e of MFMA tile (i, j) in
// the v6 wave layout.
template <int WMT>
__device__ __forceinline__ int v6_row(int i, int e) {
    const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) & 1;
    return wm * 32 * WMT + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
template <int WNT>
__device__ __forceinline__ int v6_col(int j) {
    const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) >> 1;
    return wn * 32 * WNT + j * 32 + (lane & 31);
}

// Computes the block tile's int32 accumulators for K = 128 * NK exactly. A
// is read through a buffer resource of a_limit bytes from A: rows past m_rem
// get an offset beyond it, so their loads return zeros without touching
// memory (an expert's row tile is often half empty); B rows past n_rem re-read
// the last valid row. Their outputs are discarded by the caller. With a_rows,
// tile row r of A is A[a_rows[r]]. B (the weights) is read with nontemporal
// loads. The K loop is
// unrolled completely: with no loop-carried load results (a loop head makes
// the compiler wait for every load in flight) its vmcnt tracking waits
// exactly for the set being written and keeps the later steps' loads in
// flight.
template <int WMT, int WNT, int D, int NK>
__device__ __forceinline__ void mma_tile_v6(const int8_t* __restrict__ A, int64_t lda, int m_rem, uint32_t a_limit,
                                            const int8_t* __restrict__ B, int64_t ldb, int n_rem,
                                            int8_t* lds, v16i (&acc)[WMT][WNT],
                                            const int32_t* __restrict__ a_rows = nullptr,
                                            int b_jump = 0) {
    using T = TileV6<WMT, WNT, D>;
    constexpr int L = T::L, ABLK = T::BM / 8;
    static_assert(ABLK == 8 * WMT, "copies j < WMT are A blocks, the rest B blocks");
    static_assert(NK >= 1, "K steps");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int8_t* src[L];
    uint32_t aoff[WMT];
    int dst[L];
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)a_limit, 0x00020000);
#pragma unroll
    for (int j = 0; j < L; j++) {
        const int q = j * 8 + wave;   // block of 8 rows: A blocks first, then B blocks
        if (j < WMT) {
            const int r = q * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
            aoff[j] = r < m_rem ? (uint32_t)((int64_t)(a_rows ? a_rows[r] : r) * lda + c * 16) : 0x80000000u;
            src[j] = nullptr;
        } else {
            const int r = (q - ABLK) * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
            // b_jump: the tile's second half of columns reads B rows b_jump further on
            const int rb = r >= T::BN / 2 ? r + b_jump : r;
            src[j] = B + (int64_t)min(rb, n_rem - 1) * ldb + c * 16;
        }
        dst[j] = q * 1024 + lane * 16;
    }
    auto issue = [&](int step, v4i (&set)[L]) {
#pragma unroll
        for (int j = 0; j < L; j++) {
            if (j < WMT)
                set[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(arsrc, (int)(aoff[j < WMT ? j : 0] + step * T::BK), 0, 0));
            else
                set[j] = __builtin_nontemporal_load((const v4i*)(src[j] + step * T::BK));
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the loads where they are issued
    };
    auto put = [&](int stage, const v4i (&set)[L]) {
        int8_t* base = lds + stage * T::STAGE;
#pragma unroll
        for (int j = 0; j < L; j++) *(v4i*)(base + dst[j]) = set[j];
    };
    const int fr = lane & 31, fh = lane >> 5;
    auto mma = [&](int stage) {
        const int8_t* base = lds + stage * T::STAGE;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int c = 2 * ks + fh;
            v4i a[WMT], b[WNT];
#pragma unroll
            for (int i = 0; i < WMT; i++) a[i] = *(const v4i*)(base + swz(wm * 32 * WMT + i * 32 + fr, c));
#pragma unroll
            for (int j = 0; j < WNT; j++)
                b[j] = *(const v4i*)(base + T::BM * 128 + swz(wn * 32 * WNT + j * 32 + fr, c));
#pragma unroll
            for (int i = 0; i < WMT; i++)
#pragma unroll
                for (int j = 0; j < WNT; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int j = 0; j < WNT; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

    v4i rs[D][L];
#pragma unroll
    for (int s = 0; s < D; s++)
        if (s < NK) issue(s, rs[s]);
    put(0, rs[0]);
    if (D < NK) issue(D, rs[0]);
    v6_barrier();
#pragma unroll
    for (int kt = 0; kt < NK; kt++) {
        mma(kt & 1);
        if (kt + 1 < NK) {
            put((kt + 1) & 1, rs[(kt + 1) % D]);
            if (kt + D + 1 < NK) issue(kt + D + 1, rs[(kt + 1) % D]);
        }
        v6_barrier();
    }
}

// Stages of the v5 ring for a tile shape: as many as fit in 160 KB, at most 6.
template <int WMT, int WNT>
constexpr int v5_stages() {
    return (160 * 1024) / ((64 * WMT + 64 * WNT) * 128) >= 6 ? 6 : (160 * 1024) / ((64 * WMT + 64 * WNT) * 128);
}

template <int WMT, int WNT, int S>
__device__ __forceinline__ void mma_tile_v5(const int8_t* __restrict__ A, int64_t lda, int m_rem,
                                            const int8_t* __restrict__ B, int64_t ldb, int n_rem,
                                            int K, int8_t* lds, v16i (&acc)[WMT][WNT],
                                            const int32_t* __restrict__ a_rows = nullptr) {
    using T = TileV5<WMT, WNT, S>;
    constexpr int P = WMT * WNT, F = WMT + WNT, L = T::LOADS;
    constexpr int RS = (P + 1) / 2;   // slots that carry the fragment reads
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // copy j of this wave's share of a step: j < A_PW an A block, else a B
    // block; block q = (j % per-operand) * 4 + wave holds tile rows 8q..8q+7
    const int8_t* src[L];
    int dst[L];
#pragma unroll
    for (int j = 0; j < L; j++) {
        const bool is_a = j < T::A_PW;
        const int q = (is_a ? j : j - T::A_PW) * 4 + wave;
        const int r = q * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        if (is_a) {
            const int rr = min(r, m_rem - 1);   // A row r of the tile: A[a_rows[r]] when gathering
            src[j] = A + (int64_t)(a_rows ? a_rows[rr] : rr) * lda + c * 16;
            dst[j] = q * 1024;
        } else {
            src[j] = B + (int64_t)min(r, n_rem - 1) * ldb + c * 16;
            dst[j] = T::BM * 128 + q * 1024;
        }
    }
    typedef __attribute__((address_space(3))) void lds_t;
    const int nk = K / T::BK;
    auto copy = [&](int step, int j) {
        int8_t* base = lds + (step % S) * T::STAGE;
        __builtin_amdgcn_global_load_lds((const void*)(src[j] + step * T::BK), (lds_t*)(base + dst[j]), 16, 0,
                                         0);
    };

#pragma unroll
    for (int i = 0; i < WMT; i++)
#pragma unroll
        for (int j = 0; j < WNT; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
    if (nk <= 0) return;

#pragma unroll
    for (int s = 0; s < S - 1; s++)
        if (s < nk) {
#pragma unroll
            for (int j = 0; j < L; j++) copy(s, j);
        }

    const int fr = lane & 31, fh = lane >> 5;
    // fragment f of sub-step ks: f < WMT an A fragment, else a B fragment
    auto frag1 = [&](const int8_t* base, int ks, int f, v4i (&a)[WMT], v4i (&b)[WNT]) {
        const int c = 2 * ks + fh;
        if (f < WMT) a[f] = *(const v4i*)(base + swz(wm * 32 * WMT + f * 32 + fr, c));
        else b[f - WMT] = *(const v4i*)(base + T::BM * 128 + swz(wn * 32 * WNT + (f - WMT) * 32 + fr, c));
    };
    // One sub-step: MFMA q (A fragment q / WNT, B fragment q % WNT) in slot q;
    // the next sub-step's read f goes in slot f * RS / F; with part >= 0, the
    // step's copies [part*L/3, (part+1)*L/3) of step `cstep` are spread over
    // the slots.
    auto substep = [&](const v4i (&a)[WMT], const v4i (&b)[WNT], const v4i (&pa)[WMT],
                       const v4i (&pb)[WNT], const int8_t* nbase, int nks, v4i (&na)[WMT],
                       v4i (&nb)[WNT], int cstep, int part) {
#pragma unroll
        for (int q = 0; q < P; q++) {
            const int i = q / WNT, j = q % WNT;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);   // the MFMA first: reads issued before it would join its wait
#pragma unroll
            for (int f = 0; f < F; f++)
                if (f * RS / F == q) frag1(nbase, nks, f, na, nb);
            if (part >= 0) {
                const int c0 = part * L / 3, c1 = (part + 1) * L / 3;
#pragma unroll
                for (int c = 0; c < L; c++)
                    if (c >= c0 && c < c1 && (c - c0) * P / (c1 - c0) == q) copy(cstep, c);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < WMT; i++) asm volatile("" ::"v"(a[i]), "v"(pa[i]));
#pragma unroll
        for (int j = 0; j < WNT; j++) asm volatile("" ::"v"(b[j]), "v"(pb[j]));
    };

    v4i fa[4][WMT], fb[4][WNT];
#pragma unroll
    for (int i = 0; i < WMT; i++) fa[3][i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < WNT; j++) fb[3][j] = v4i{0, 0, 0, 0};
    // Steps copied: 0..min(S-1, nk)-1 before the loop, kt+S-1 during step kt
    // of the main part. Step kt+1 is complete once at most the steps copied
    // after it are in flight.
    stage_barrier_steps<L, S - 2>(min(S - 2, nk - 1));
#pragma unroll
    for (int f = 0; f < F; f++) frag1(lds, 0, f, fa[0], fb[0]);
    int kt = 0;
    for (; kt + S - 1 < nk; kt++) {
        const int8_t* cur = lds + (kt % S) * T::STAGE;
        const int8_t* nxt = lds + ((kt + 1) % S) * T::STAGE;
        const int cs = kt + S - 1;
        substep(fa[0], fb[0], fa[3], fb[3], cur, 1, fa[1], fb[1], cs, 0);
        substep(fa[1], fb[1], fa[0], fb[0], cur, 2, fa[2], fb[2], cs, 1);
        substep(fa[2], fb[2], fa[1], fb[1], cur, 3, fa[3], fb[3], cs, 2);
        stage_barrier<(S - 2) * L>();
        substep(fa[3], fb[3], fa[2], fb[2], nxt, 0, fa[0], fb[0], -1, -1);
    }
    for (; kt < nk; kt++) {
        const int8_t* cur = lds + (kt % S) * T::STAGE;
        const int8_t* nxt = lds + ((kt + 1) % S) * T::STAGE;
        substep(fa[0], fb[0], fa[3], fb[3], cur, 1, fa[1], fb[1], -1, -1);
        substep(fa[1], fb[1], fa[0], fb[0], cur, 2, fa[2], fb[2], -1, -1);
        substep(fa[2], fb[2], fa[1], fb[1], cur, 3, fa[3], fb[3], -1, -1);
        stage_barrier_steps<L, S - 2>(max(0, nk - 2 - kt));
        substep(fa[3], fb[3], fa[2], fb[2], nxt, 0, fa[0], fb[0], -1, -1);
    }
}

}  // namespace pio
