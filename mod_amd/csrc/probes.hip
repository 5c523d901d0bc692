// Measurement kernels (no counterpart in the reference; bench.py uses them to
// test what bounds a kernel, they compute nothing the path needs).
//
// Operand supply of the dense W8A8 GEMM: the GEMM's K loop with its copies
// only -- no MFMA, no epilogue, no output. Block b takes the tile of the
// GEMM's XCD-aware map (XCD b % 8 gets one rectangle of the tile grid) and
// moves its A rows (BM) and B rows (BN) global -> LDS with direct-to-LDS
// 16-byte copies, in K steps of `step` bytes per row (128 is the GEMM's), two
// steps in flight, one barrier per step; 8 rows x 128 B, 4 x 256 B or
// 2 x 512 B per wave instruction. The LDS destinations wrap in 64 KB (nothing
// reads them). Per-CU supply = (BM + BN) * K bytes / the block's time. Built
// for the 128 x 192 tile of the C3 shapes (320 rows per tile).
#include "pio_common.hpp"

namespace pio {

struct SupplyParams {
    const int8_t* A;
    const int8_t* B;
    int M, N, K, BM, BN;
    int tiles_n, xr, xc;
};

// s_waitcnt vmcnt(N), no wait on the other counters (gfx9 encoding)
template <int N>
__device__ __forceinline__ void probe_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

template <int STEP, int ROWS>
__global__ __launch_bounds__(256, 1) void gemm_supply_probe_kernel(SupplyParams p) {
    typedef __attribute__((address_space(3))) void lds_t;
    extern __shared__ __attribute__((aligned(16))) int8_t probe_lds[];
    constexpr int PER_INS = 1024 / STEP;             // rows per wave instruction
    constexpr int LANES_PER_ROW = STEP / 16;
    constexpr int INS = ROWS / PER_INS;              // wave instructions per step (all waves)
    static_assert(INS % 4 == 0, "the four waves share a step's copies evenly");
    constexpr int MINE = INS / 4;                    // this wave's copies per step
    const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int tr, tc;
    if (p.xr) {
        const int x = b % 8, k = b / 8;
        const int R = ((int)gridDim.x / p.tiles_n) / p.xr, Cc = p.tiles_n / p.xc;
        tr = (x / p.xc) * R + k / Cc;
        tc = (x % p.xc) * Cc + k % Cc;
    } else {
        tr = b / p.tiles_n;
        tc = b % p.tiles_n;
    }
    const int rl = lane / LANES_PER_ROW, cb = (lane % LANES_PER_ROW) * 16;
    const int8_t* src[MINE];
#pragma unroll
    for (int j = 0; j < MINE; j++) {
        const int r = (wave + 4 * j) * PER_INS + rl;
        src[j] = r < p.BM ? p.A + (int64_t)min(tr * p.BM + r, p.M - 1) * p.K + cb
                          : p.B + (int64_t)min(tc * p.BN + r - p.BM, p.N - 1) * p.K + cb;
    }
    const int nk = p.K / STEP;
    for (int s = 0; s < nk; s++) {
#pragma unroll
        for (int j = 0; j < MINE; j++)
            __builtin_amdgcn_global_load_lds((const void*)(src[j] + (int64_t)s * STEP),
                                             (lds_t*)(probe_lds + (((s * MINE + j) * 4 + wave) * 1024 & 65535)),
                                             16, 0, 0);
        // two steps in flight: wait for the step before this one, then meet
        if (s > 0) probe_wait_vm<MINE>();
        __builtin_amdgcn_s_barrier();
    }
    probe_wait_vm<0>();
}

}  // namespace pio

using namespace pio;

// `reps` back-to-back launches of the operand-supply probe for an M x N x K
// GEMM with BM x BN tiles and K steps of `step` bytes (128, 256 or 512), the
// tiles mapped to the XCDs as the GEMM maps them.
PIO_EXPORT int pio_probe_gemm_supply(const int8_t* A, const int8_t* B, int M, int N, int K, int BM, int BN,
                                     int step, int reps, void* stream) {
    PIO_REQUIRE(A && B, "pio_probe_gemm_supply: null pointer");
    PIO_REQUIRE(step == 128 || step == 256 || step == 512, "pio_probe_gemm_supply: step %d", step);
    PIO_REQUIRE(BM + BN == 320, "pio_probe_gemm_supply: the probe is built for the 128 x 192 tile");
    PIO_REQUIRE(K % step == 0 && M % BM == 0 && N % BN == 0,
                "pio_probe_gemm_supply: shape must divide into tiles and steps");
    SupplyParams p{A, B, M, N, K, BM, BN, N / BN, 0, 0};
    const int tm = M / BM, tn = N / BN;
    int64_t best = -1;
    for (int r = 1; r <= 8; r *= 2) {   // the GEMM's rectangle choice (gemm.hip xcd_split)
        const int c = 8 / r;
        if (tm % r || tn % c) continue;
        const int64_t rows = (int64_t)(tm / r) * BM + (int64_t)(tn / c) * BN;
        if (best < 0 || rows < best) { best = rows; p.xr = r; p.xc = c; }
    }
    const hipStream_t st = pick_stream(stream);
    for (int i = 0; i < reps; i++) {
        if (step == 128) gemm_supply_probe_kernel<128, 320><<<tm * tn, 256, 65536, st>>>(p);
        else if (step == 256) gemm_supply_probe_kernel<256, 320><<<tm * tn, 256, 65536, st>>>(p);
        else gemm_supply_probe_kernel<512, 320><<<tm * tn, 256, 65536, st>>>(p);
    }
    PIO_LAUNCHED();
    return PIO_OK;
}
