// Persistent int8 decode loop: one launch of one workgroup per CU runs n
// greedy decode steps of the Qwen3-style decoder, replacing the 143 kernel
// launches per token of the step graph (decode.hip) with in-kernel data flow.
// Same semantics as the step kernels (reference decode loop:
// ip/models/qwen3_0_6b/architecture.py:124-221, with the defects listed in
// decode.hip fixed).
//
// Why: at batch 1 every linear is a few MB of int8 weights, which HBM streams
// in well under a microsecond, but each kernel of the step graph costs ~1.6 us
// of launch overhead plus a full HBM latency before its first weight arrives.
// Here the weights of the next phases stream into LDS while the current phase
// waits for its input, and phases hand data to each other directly.
//
// Partitioning by XCD. MI355X has 8 XCDs of 32 CUs, each XCD with its own L2.
// The dispatcher deals a launch's workgroups to the XCDs round-robin, but from
// wherever the previous launch left off, so each workgroup reads its XCD from
// the hardware XCC id at start and takes the next free slot j of that XCD; the
// role (g, j) then fixes all its work. A value handed to another XCD travels
// through the memory side
// (~0.75 us one way, measured), one handed within an XCD stays closer. The
// layer is split so that only two hand-offs per layer cross XCDs:
//   XCD g owns KV head g (8 KV heads, 8 XCDs) and slice g of the MLP:
//   P1  x''[e] = x'[e] + sum_h dpart[h][e]   reduce the previous layer's 8
//       down partials; workgroup (g, j) reduces elements [32j, 32j+32) for
//       its XCD (every XCD keeps the full residual stream)        [cross-XCD]
//   P2  every workgroup of XCD g gathers the full x'', RMSNorm, and computes
//       8 of the 256 (row, row+64) pairs of KV head g's q/k/v rows, bias,
//       RoPE, KV-cache row                                        [intra-XCD]
//   P3  attention of KV head g (both query heads) in 8 position splits on
//       workgroups j < 8                                          [intra-XCD]
//   P4  every workgroup merges the 8 splits into the head output o_g (256
//       values) and computes the o_proj partial of rows [32j, 32j+32) over
//       o_g's 256 columns                                         [cross-XCD]
//   P5  x'[e] = x''[e] + sum_h opart[h][e] (like P1)
//   P6  gather x', RMSNorm, gate_up for 12 of XCD g's 384 intermediate
//       channels, SwiGLU                                          [intra-XCD]
//   P7  down partial of rows [32j, 32j+32) over XCD g's 384 channels
// After the last layer: P1, gather, final RMSNorm, lm_head rows + argmax key.
// The o_proj and down outputs are thus sums of 8 per-XCD partials, added in a
// fixed order (deterministic); each workgroup streams 60 KB of weights per
// layer, as evenly as before.
//
// Workgroup = 8 waves:
//   waves 4-7 ("stream waves") copy this workgroup's weight lines, in the order
//     the compute waves consume them, from a relaid copy of the weights
//     (built once, line-major over the workgroups) into an LDS ring of 1 KB lines with
//     global_load_lds_dwordx4; a line is published when its copy has landed.
//   waves 0-3 ("compute waves") run the phases; each polls whole input vectors
//     itself (no cross-wave rendezvous except around attention and the merge).
//
// Hand-off: every value a phase produces for other workgroups is stored as a
// tagged 64-bit word {tag:32 | fp32 bits:32}; a consumer polls the words it
// needs until every tag equals the producing phase's tag. Words bound for
// other XCDs (the opart/dpart partials) use device-scope stores and loads;
// words consumed within the producer's XCD go through that XCD's L2 (st_l2 /
// ld_l2_* below). Tags grow monotonically over the
// decoder's lifetime, so no buffer is ever reset and no barrier is needed. A
// buffer is rewritten one layer later, when every workgroup of every XCD has
// consumed it: each layer's gathers (P2, P6) need all workgroups of the XCD,
// and the cross-XCD reductions need all XCDs.
//
// Co-residency. The grid has exactly as many workgroups as the device has
// CUs, and each workgroup takes most of a CU's 160 KB of LDS, so on an idle
// device all of them are resident at once. The kernel needs no grid barrier,
// only that residency, so it is launched as an ordinary kernel: a cooperative
// launch would claim the device's global wave-sync resource, which only one
// process at a time can hold (a second process's cooperative launch fails).
// If other work holds some CUs, the workgroups waiting for them start when it
// drains; every wait below is bounded (a timeout records an error, read back
// by pio_qwen3_read, and makes every wave leave), so the kernel ends in any case.
#include "decode.hpp"

#include <math.h>
#include <algorithm>
#include <vector>

namespace pio {

typedef unsigned long long u64;
typedef int lp_v4i __attribute__((ext_vector_type(4)));

constexpr int LP_CW = 4;                   // compute waves
constexpr int LP_SW = 4;                   // stream waves
constexpr int LP_THREADS = 64 * (LP_CW + LP_SW);
constexpr int LP_RING = 64;                // LDS ring of 1 KB weight lines (power of two)
constexpr int LP_INFL = 12;                // lines in flight per stream wave
// The shape the kernel is built for (Qwen3-0.6B on an 8-XCD, 256-CU MI355X)
constexpr int LP_NX = 8;                   // XCDs = KV heads
constexpr int LP_WPX = 32;                 // workgroups per XCD
constexpr int LP_NBLK = LP_NX * LP_WPX;
constexpr int LP_D = 128;                  // head_dim
constexpr int LP_G = 2;                    // query heads per KV head
constexpr int LP_H = 1024;                 // hidden
constexpr int LP_KO = 2048;                // n_heads * head_dim
constexpr int LP_I = 3072;                 // intermediate
constexpr int LP_IX = LP_I / LP_NX;        // 384 intermediate channels per XCD
constexpr int LP_QKVX = (LP_G + 2) * LP_D; // 512 q/k/v values per KV head
constexpr int LP_S = 8;                    // attention splits over positions
constexpr int LP_NPF = 2;                  // attention passes whose K/V are prefetched
constexpr int LP_NPMAX = 8;                // attention passes (8 positions each) per wave
constexpr int LP_MAX_SEQ = LP_S * LP_CW * 8 * LP_NPMAX;   // 2048
constexpr int LP_PART = 2 + LP_D;          // (max, sum, o[128]) per split and head
static_assert(LP_S == 8, "the merge loads the partials of 8 splits in one batch");
constexpr int LP_LMAX = 48;                // layers whose per-wave constants LDS holds
constexpr int LP_NCST = 32;                // constants per layer and compute wave (30 used)
constexpr int LP_PH = 7;                   // tagged phases per layer
// weight lines per workgroup and layer, in consumption order
constexpr int LP_L_QKV = 16;               // 8 (row, row+64) pairs of 1 KB rows
constexpr int LP_L_O = 8;                  // 32 rows x 256 B (4 rows per line)
constexpr int LP_L_GU = 24;                // 12 (gate, up) pairs of 1 KB rows
constexpr int LP_L_DN = 12;                // 32 rows x 384 B (8 rows x 128 B per line)
constexpr int LP_OFF_O = LP_L_QKV, LP_OFF_GU = LP_OFF_O + LP_L_O, LP_OFF_DN = LP_OFF_GU + LP_L_GU;
constexpr int LP_LPL = LP_OFF_DN + LP_L_DN;   // 60
// Every wait gives up after LP_WAIT_TICKS of the 100 MHz constant clock
// (s_memrealtime): one time limit for every site, so a wait on an LDS counter
// outlasts the device poll of a sibling wave that it depends on.
constexpr uint64_t LP_WAIT_TICKS = 200000000ull;     // 2 s
// How long a workgroup waits at launch for all LP_NBLK to be resident.
constexpr uint64_t LP_ARRIVE_TICKS = 2000000ull;     // 20 ms

enum { PH_XR = 0, PH_QKV = 1, PH_ATT = 2, PH_OP = 3, PH_XR2 = 4, PH_ACT = 5, PH_DP = 6 };
enum { LP_ERR_TIMEOUT = 1, LP_ERR_XCD = 2, LP_ERR_RESIDENT = 3 };
// Error words (LoopState::err, 64 ints): [0] code, [1] site, [2] abort flag,
// [4] workgroups arrived, [8 + g] XCD g's next slot -- cleared before every
// launch; [16] set once a launch found the grid not co-resident (every later
// launch then leaves at once), [17] that launch's first position -- kept until
// the host has re-run those steps.
constexpr int LP_E_ARRIVED = 4, LP_E_STICKY = 16, LP_E_STICKY_POS = 17;

struct LoopLayer {
    const float *in_norm, *s_qkv, *b_qkv, *s_o, *post_norm, *s_gu, *s_down;
};

struct LoopParams {
    int L, V, max_seq;
    float eps, att_scale;
    const float* embed;
    const float* final_norm;
    const float* s_lm;
    const int8_t* lm_head;     // [V][H] int8, read directly by the lm phase
    const LoopLayer* layers;
    const int8_t* stream;      // [lpt][nblk][1024] weight lines in consumption order
    int lpt;                   // weight lines per token (n_layers * LP_LPL)
    void* kc;                  // KV cache [L][8][max_seq][128], fp32 or fp16 (kernel's KV16)
    void* vc;
    const float* cos_t;
    const float* sin_t;
    // tagged hand-off buffers
    u64* xr;      // [8][H]    P1 output, per XCD
    u64* xr2;     // [8][H]    P5 output, per XCD
    u64* qkv;     // [8][512]  q (2 heads), k, v of KV head g
    u64* att;     // [8][S][2][LP_PART] attention partials
    u64* act;     // [8][384]  SwiGLU output, XCD g's channels
    u64* opart;   // [8][H]    o_proj partials, per XCD
    u64* dpart;   // [8][H]    down partials, per XCD
    u64* keys;    // [nblk]    argmax keys
    int32_t* ids;
    float* logits;
    int32_t* state;
    int pos0, prompt_len, n_steps;
    uint32_t epoch0;
    uint64_t arrive_ticks;     // co-residency wait at launch (LP_ARRIVE_TICKS)
    int* err;                  // error words (see LP_E_*)
    u64* trace;                // traced launches: phase stamps (see lp_stamp)
    int tr_t0;                 // the first traced step of the launch
};

// Phase timeline of a traced launch (the kernel's TR instantiation): wave 0 of
// every workgroup stamps the 100 MHz constant clock at each phase boundary of
// LP_TR_TOK consecutive steps, trace[step][role][layer][slot]; layer L holds
// the last layer's reduction, the gather, the lm_head rows and the key store.
// Slots: 0 layer start, 1 P1 reduced, 2 P2 gathered, 3 q/k/v stored,
// 4 attention stored (its workgroups only), 5 merged, 6 o_proj partial stored,
// 7 P5 reduced, 8 P6 gathered, 9 act stored, 10 down partial stored; inside
// phases: 11 q/k/v weight lines landed, 12 attention's q arrived, 13 attention
// computed (before its workgroup combines the waves), 14 merge inputs
// arrived; in layer L: 0 start, 1 reduced, 2 gathered, 3 lm rows done, 4 key
// stored.
constexpr int LP_TR_TOK = 2, LP_TR_K = 16;

// LDS layout (dynamic): ring | per-wave x copies | merged head output |
// per-wave act copies | attention partials | attention staging | per-layer
// constants
constexpr size_t LP_LDS_RING = (size_t)LP_RING * 1024;
constexpr size_t LP_LDS_XW = (size_t)LP_CW * LP_H * 4;
static_assert(LP_LDS_XW == (LP_H / 64) * 64 * 16, "the lm phase's A operand fills the x-copy region");
constexpr size_t LP_LDS_OS = (size_t)LP_G * LP_D * 4;
constexpr size_t LP_LDS_ACT = (size_t)LP_CW * LP_IX * 4;
constexpr size_t LP_LDS_ATT = (size_t)LP_CW * LP_G * LP_D * 4 + 2 * LP_CW * LP_G * 4;
constexpr size_t LP_STG = LP_G * LP_D + 256;   // floats per wave: q heads + current k,v
constexpr size_t LP_LDS_STG = (size_t)LP_CW * LP_STG * 4;
constexpr size_t LP_LDS_CST = (size_t)LP_LMAX * LP_CW * LP_NCST * 4;
constexpr size_t LP_LDS_XS = (size_t)2 * LP_H * 4;   // the shared input vectors x'', x'
constexpr size_t LP_LDS_BYTES = LP_LDS_RING + LP_LDS_XW + LP_LDS_OS + LP_LDS_ACT + LP_LDS_ATT + LP_LDS_STG + LP_LDS_CST + LP_LDS_XS;

// ------------------------------------------------------------------ helpers
__device__ __forceinline__ u64 ll_load(const u64* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(u64* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// Loads through the global address space (not flat): a flat load also counts
// in lgkmcnt, so every later LDS wait of the wave (stage, rendezvous, ring
// checks) would wait for it too. Pointers read from the parameter block are
// generic to the compiler, hence the casts.
template <typename T>
__device__ __forceinline__ T gld(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}

// Hand-offs within one XCD go through that XCD's L2: the producer's store
// (sc0) lands in the L2, and the consumer's load (sc0 nt) misses the CU's L1
// and reads the L2 (~0.45 us one way between two CUs of an XCD, against ~0.75
// us through the memory side, measured). Every batch of polling loads is one
// asm statement that also waits for them, so no output register is used
// before its load has landed.
__device__ __forceinline__ void st_l2(u64* p, float v, uint32_t tag) {
    const u64 w = ((u64)tag << 32) | (u64)__float_as_uint(v);
    asm volatile("global_store_dwordx2 %0, %1, off sc0" ::"v"(p), "v"(w) : "memory");
}
#define LP_LD(i, off) "global_load_dwordx2 %" #i ", %[a], off offset:" #off " sc0 nt\n"
#define LP_LDB(i, off) "global_load_dwordx2 %" #i ", %[b], off offset:" #off " sc0 nt\n"
#define LP_LDC(i, off) "global_load_dwordx2 %" #i ", %[c], off offset:" #off " sc0 nt\n"
#define LP_LDD(i, off) "global_load_dwordx2 %" #i ", %[d], off offset:" #off " sc0 nt\n"
// 16 tagged words 64 words apart (lane-consecutive: coalesced), from two
// bases 512 words apart (immediate offsets reach 4 KB)
__device__ __forceinline__ void ld_l2_16s(const u64* a, const u64* b, u64 (&v)[16]) {
    asm volatile(LP_LD(0, 0) LP_LD(1, 512) LP_LD(2, 1024) LP_LD(3, 1536) LP_LD(4, 2048)
                 LP_LD(5, 2560) LP_LD(6, 3072) LP_LD(7, 3584) LP_LDB(8, 0) LP_LDB(9, 512)
                 LP_LDB(10, 1024) LP_LDB(11, 1536) LP_LDB(12, 2048) LP_LDB(13, 2560)
                 LP_LDB(14, 3072) LP_LDB(15, 3584) "s_waitcnt vmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
                   "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
                 : [a] "v"(a), [b] "v"(b)
                 : "memory");
}
// 2 tagged words 64 words apart
__device__ __forceinline__ void ld_l2_2s(const u64* p, u64 (&v)[2]) {
    asm volatile(LP_LD(0, 0) LP_LD(1, 512) "s_waitcnt vmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1])
                 : [a] "v"(p)
                 : "memory");
}
// 4 tagged words 64 words apart
__device__ __forceinline__ void ld_l2_4s(const u64* p, u64 (&v)[4]) {
    asm volatile(LP_LD(0, 0) LP_LD(1, 512) LP_LD(2, 1024) LP_LD(3, 1536) "s_waitcnt vmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                 : [a] "v"(p)
                 : "memory");
}
// 8 tagged words 64 words apart
__device__ __forceinline__ void ld_l2_8s(const u64* p, u64 (&v)[8]) {
    asm volatile(LP_LD(0, 0) LP_LD(1, 512) LP_LD(2, 1024) LP_LD(3, 1536) LP_LD(4, 2048)
                 LP_LD(5, 2560) LP_LD(6, 3072) LP_LD(7, 3584) "s_waitcnt vmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7])
                 : [a] "v"(p)
                 : "memory");
}
// The merge's words of 8 attention splits (split stride 130 words): max and
// sum of splits 0-3 from a, 4-7 from b (the same address in every lane), and
// o[d] of splits 0-3 from c, 4-7 from d (lane-consecutive d).
__device__ __forceinline__ void ld_l2_merge(const u64* a, const u64* b, const u64* c, const u64* d,
                                            u64 (&ml)[16], u64 (&o)[8]) {
    asm volatile(LP_LD(0, 0) LP_LD(1, 8) LP_LD(2, 1040) LP_LD(3, 1048) LP_LD(4, 2080) LP_LD(5, 2088)
                 LP_LD(6, 3120) LP_LD(7, 3128) LP_LDB(8, 0) LP_LDB(9, 8) LP_LDB(10, 1040)
                 LP_LDB(11, 1048) LP_LDB(12, 2080) LP_LDB(13, 2088) LP_LDB(14, 3120) LP_LDB(15, 3128)
                 LP_LDC(16, 0) LP_LDC(17, 1040) LP_LDC(18, 2080) LP_LDC(19, 3120)
                 LP_LDD(20, 0) LP_LDD(21, 1040) LP_LDD(22, 2080) LP_LDD(23, 3120) "s_waitcnt vmcnt(0)"
                 : "=&v"(ml[0]), "=&v"(ml[1]), "=&v"(ml[2]), "=&v"(ml[3]), "=&v"(ml[4]), "=&v"(ml[5]),
                   "=&v"(ml[6]), "=&v"(ml[7]), "=&v"(ml[8]), "=&v"(ml[9]), "=&v"(ml[10]),
                   "=&v"(ml[11]), "=&v"(ml[12]), "=&v"(ml[13]), "=&v"(ml[14]), "=&v"(ml[15]),
                   "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]),
                   "=&v"(o[6]), "=&v"(o[7])
                 : [a] "v"(a), [b] "v"(b), [c] "v"(c), [d] "v"(d)
                 : "memory");
}
template <int N>
__device__ __forceinline__ bool tags_ok(const u64 (&v)[N], uint32_t tag) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; i++) ok &= (uint32_t)(v[i] >> 32) == tag;
    return ok;
}

__device__ __forceinline__ void dev_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int lds_ld(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Same word in every lane: read it as a scalar so that loop exits on it are
// scalar branches (no exec-mask bookkeeping around every wait).
__device__ __forceinline__ int lds_ld_u(const int* p) { return __builtin_amdgcn_readfirstlane(lds_ld(p)); }
__device__ __forceinline__ void lds_st(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void cbar() { asm volatile("" ::: "memory"); }

// LDS store the compiler cannot see as one: a plain LDS store issued while
// this wave has global->LDS copies in flight makes the compiler wait for all
// of them first (it cannot tell the addresses apart), which would drain the
// stream waves' copy pipeline at every publish.
__device__ __forceinline__ void lds_st_raw(int* p, int v) {
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int*)p;
    asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory");
}

// s_waitcnt vmcnt(N), no wait on the other counters (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    cbar();
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
    cbar();
}

// ---- cross-lane ops on the VALU (DPP, permlane swaps, readlane; dpp, rlane,
// sum8, wsum and wmax come from pio_common.hpp). The LDS queue (where __shfl's
// ds_swizzle / ds_bpermute go) is busy with the stream waves' copies, so every
// reduction here avoids it.
// Four wave sums at once (each returned uniform): halves, then quarters are
// folded together with lane swaps so that lane rows 0..3 hold a, b, c, d, and a
// single 16-lane DPP reduction finishes all four.
//   permlane32_swap(x, y): r0 = [x lanes 0-31 | y lanes 0-31], r1 = [x 32-63 | y 32-63]
//   permlane16_swap(x, y): r0 = rows [x0, y0, x2, y2],         r1 = rows [x1, y1, x3, y3]
__device__ __forceinline__ void wsum4(float& a, float& b, float& c, float& d) {
    const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(c), false, false);
    const float pa = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);   // lanes 0-31: a, 32-63: c
    const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(b), __float_as_uint(d), false, false);
    const float pb = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);   // lanes 0-31: b, 32-63: d
    const auto s3 = __builtin_amdgcn_permlane16_swap(__float_as_uint(pa), __float_as_uint(pb), false, false);
    float r = __uint_as_float(s3[0]) + __uint_as_float(s3[1]);          // rows: a, b, c, d
    r += dpp<DPP_XOR1>(r);
    r += dpp<DPP_XOR2>(r);
    r += dpp<DPP_HMIRROR>(r);
    r += dpp<DPP_MIRROR>(r);
    a = rlane(r, 0);
    b = rlane(r, 16);
    c = rlane(r, 32);
    d = rlane(r, 48);
}
// Wave sums of N values (in place), four at a time.
template <int N>
__device__ __forceinline__ void wsum_n(float* v) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        float z1 = 0.f, z2 = 0.f, z3 = 0.f;
        wsum4(v[i], i + 1 < N ? v[i + 1] : z1, i + 2 < N ? v[i + 2] : z2, i + 3 < N ? v[i + 3] : z3);
    }
}

// Sum over the lanes i, i^8, i^16, i^32 (equal lane%8), in each of them.
__device__ __forceinline__ float sum_stride8(float x) {
    x += dpp<DPP_ROR8>(x);
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 16 int8 weights times 16 fp32 x with signed byte conversions (one
// v_cvt_f32_i32 with a sign-extending byte select each), 4 independent chains.
__device__ __forceinline__ void lp_dot16s(const float* x, lp_v4i w, float (&acc)[4]) {
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int u = w[d];
        acc[0] = fmaf(x[4 * d + 0], (float)(int8_t)(u), acc[0]);
        acc[1] = fmaf(x[4 * d + 1], (float)(int8_t)(u >> 8), acc[1]);
        acc[2] = fmaf(x[4 * d + 2], (float)(int8_t)(u >> 16), acc[2]);
        acc[3] = fmaf(x[4 * d + 3], (float)(int8_t)(u >> 24), acc[3]);
    }
}

// 16 int8 weights (one 16-byte lane slice of a line) times 16 fp32 x, into 4
// independent accumulator chains (byte position within each dword): with one
// compute wave per SIMD there is no other wave to hide a dependent chain's
// latency, so the chains have to be independent within the wave.
// The bytes are read as unsigned after flipping their sign bit (b + 128, one
// v_cvt_f32_ubyteN each); the caller removes the 128 * sum(x) offset once per
// row (lp_xsum gives the lane's sum of its 16 x values).
__device__ __forceinline__ void lp_dot16(const float* x, lp_v4i w, float (&acc)[4]) {
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const uint32_t u = (uint32_t)w[d] ^ 0x80808080u;
        acc[0] = fmaf(x[4 * d + 0], (float)(u & 0xFFu), acc[0]);
        acc[1] = fmaf(x[4 * d + 1], (float)((u >> 8) & 0xFFu), acc[1]);
        acc[2] = fmaf(x[4 * d + 2], (float)((u >> 16) & 0xFFu), acc[2]);
        acc[3] = fmaf(x[4 * d + 3], (float)(u >> 24), acc[3]);
    }
}
// -128 * (sum of the lane's 16 x values of one chunk): the offset lp_dot16 adds.
__device__ __forceinline__ float lp_xoff(const float* x) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += x[i];
    return -128.f * s;
}

__device__ __forceinline__ u64 lp_key(float v, int row, uint32_t tag) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((u64)b << 32) | ((u64)(0x3FFFFu - (uint32_t)row) << 14) | (u64)(tag & 0x3FFFu);
}
__device__ __forceinline__ u64 wave_max_u64(u64 v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const u64 other = __shfl_xor(v, o, 64);
        v = other > v ? other : v;
    }
    return v;
}

__device__ __forceinline__ bool lm_needed(const LoopParams& p, int t) {
    return p.pos0 + t + 1 >= p.prompt_len || t == p.n_steps - 1;
}
__device__ __forceinline__ uint32_t tag_of(const LoopParams& p, int t, int l, int ph) {
    return p.epoch0 + (uint32_t)t * (uint32_t)(p.L * LP_PH + 2) + (uint32_t)(l * LP_PH + ph);
}

struct Cx {
    int lane, w, nsync, fail_where;
    uint64_t wt0;    // s_memrealtime at the current wait's first check
    int g, j, role;  // XCD, slot within it, role index j * 8 + g
    int tt, tl;      // current step and layer (for the traced build's stamps)
    int uv0, nuv;    // lm_head rows of this workgroup
    int* ready;      // [LP_SW] lines landed per stream wave
    int* done;       // [LP_CW] first line each compute wave may still need
    int* csync;      // compute-wave rendezvous counter
    int* abort;      // workgroup abort flag
    int8_t* ring;
    float* xw;       // 16 KB: the lm phase's A operand (16 MFMAs x 64 lanes x 16 B)
    float* os;       // [256] merged attention output of KV head g
    float* acts;     // [384] the workgroup's copy of XCD g's act slice
    float* attp;     // [LP_CW][LP_G][128] attention partials
    float* attm;     // [2][LP_CW][LP_G] wave max, wave sum
    float* stg;      // [LP_CW][LP_STG]
    float* cst;      // [LP_LMAX][LP_CW][LP_NCST] per-layer constants of each compute wave
    float* xs;       // [2][H] the workgroup's copies of x'' (0) and x' (1)
    u64* wkeys;      // [LP_CW]
};

template <bool TR>
__device__ __forceinline__ void lp_stamp(const LoopParams& p, const Cx& c, int t, int l, int k) {
    if constexpr (TR) {
        const int tt = t - p.tr_t0;
        if (c.w == 0 && c.lane == 0 && tt >= 0 && tt < LP_TR_TOK)
            p.trace[(((int64_t)tt * LP_NBLK + c.role) * (p.L + 1) + l) * LP_TR_K + k] = wall_clock64();
    }
}

// A stamp inside a phase, at the step and layer compute_role is in.
template <bool TR>
__device__ __forceinline__ void lp_stamp_in(const LoopParams& p, const Cx& c, int k) {
    lp_stamp<TR>(p, c, c.tt, c.tl, k);
}

// Records a timed-out wait (site `where`) and tells every workgroup to stop.
__device__ void lp_fail(const LoopParams& p, int code, int where) {
    if (atomicCAS(&p.err[0], 0, code) == 0) atomicExch(&p.err[1], where);
    __hip_atomic_store(&p.err[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One more iteration of a bounded wait? Also leaves when another wave or
// workgroup gave up. A wave that runs out of patience only notes where (and
// raises the workgroup's abort flag); the kernel reports it once on the way
// out -- the kernel has to fit the instruction cache, so no calls or long
// paths sit inside the wait loops. The clock is read every 64th iteration;
// the first read starts the wait's LP_WAIT_TICKS.
__device__ __forceinline__ bool keep_waiting(const LoopParams& p, Cx& c, uint32_t it, int where) {
    // the abort flag every 16 iterations: an LDS read in every iteration
    // lengthens each poll by a round trip
    if ((it & 15) == 15 && lds_ld_u(c.abort)) return false;
    if ((it & 63) != 63) return true;
    const uint64_t now = __builtin_amdgcn_s_memrealtime();
    if (it == 63) c.wt0 = now;
    const bool late = now - c.wt0 > LP_WAIT_TICKS;
    if (__hip_atomic_load(&p.err[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || late) {
        if (late) c.fail_where = where;
        lds_st(c.abort, 1);
        return false;
    }
    return true;
}

// Polls N tagged words per lane (addr(i), i < N) until every tag of the wave
// matches; returns their values.
template <int N, typename F>
__device__ __forceinline__ bool poll(const LoopParams& p, Cx& c, F addr, uint32_t tag,
                                     float (&out)[N], int where) {
    for (uint32_t it = 0;; it++) {
        u64 v[N];
#pragma unroll
        for (int i = 0; i < N; i++) v[i] = ll_load(addr(i));
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++) ok &= (uint32_t)(v[i] >> 32) == tag;
        if (__all(ok)) {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)v[i]);
            return true;
        }
        if (!keep_waiting(p, c, it, where)) return false;
    }
}

// Rendezvous of the four compute waves of this workgroup.
__device__ __forceinline__ bool csync(const LoopParams& p, Cx& c, int where) {
    c.nsync++;
    cbar();
    if (c.lane == 0) __hip_atomic_fetch_add(c.csync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int target = LP_CW * c.nsync;
    // no sleep between the reads: the four waves arrive within a few hundred
    // cycles, and a sleep delays the last wave's exit (+0.4% tok/s without)
    for (uint32_t it = 0; lds_ld_u(c.csync) < target; it++)
        if (!keep_waiting(p, c, it, where)) return false;
    cbar();
    return true;
}

// One LDS word, read without the compiler's knowledge: the stream waves' own
// global->LDS copies in flight then need no wait before it.
__device__ __forceinline__ int lds_ld_asm(const int* p) {
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const int*)p;
    int v;
    asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
    return __builtin_amdgcn_readfirstlane(v);
}

// Four LDS counters in one read (the stream waves' landed lines ready[], or
// the compute waves' done[]; both 16-byte aligned): four separate atomic
// reads each waited for the previous one, four LDS round trips per check.
static_assert(LP_SW == 4 && LP_CW == 4, "the ready[] / done[] counters are read as one 16-byte word");
__device__ __forceinline__ lp_v4i lds_ld_ready(const int* ready) {
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const int*)ready;
    lp_v4i v;
    asm volatile("ds_read_b128 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
    return v;
}

// Waits until every ring line up to `last` has landed (stream wave r copies
// lines r, r+4, ... in order and counts them in ready[r]).
__device__ __forceinline__ bool wait_upto(const LoopParams& p, Cx& c, int last, int where) {
    for (uint32_t it = 0;; it++) {
        const lp_v4i rd = lds_ld_ready(c.ready);
        bool ok = true;
#pragma unroll
        for (int r = 0; r < LP_SW; r++)
            ok &= last < r || __builtin_amdgcn_readfirstlane(rd[r]) >= ((last - r) >> 2) + 1;
        if (ok) break;
        if (!keep_waiting(p, c, it, where)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    cbar();
    return true;
}

__device__ __forceinline__ void set_done(Cx& c, int line) {
    cbar();
    if (c.lane == 0) lds_st(&c.done[c.w], line);
    cbar();
}

__device__ __forceinline__ lp_v4i ring_line(const Cx& c, int line) {
    return *(const lp_v4i*)(c.ring + (size_t)(line % LP_RING) * 1024 + c.lane * 16);
}

// Sum over each group of 16 consecutive lanes, in every lane of the group.
__device__ __forceinline__ float sum16(float x) {
    x = sum8(x);
    return x + dpp<DPP_ROR8>(x);
}

// ------------------------------------------------------------ phase bodies
__device__ __forceinline__ void load_row16(const float* src, float (&d)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 a = *(const float4*)(src + 4 * i);
        d[4 * i] = a.x; d[4 * i + 1] = a.y; d[4 * i + 2] = a.z; d[4 * i + 3] = a.w;
    }
}
typedef float lp_f4 __attribute__((ext_vector_type(4)));
// A KV cache element. Its readers are the attention workgroups of KV head g
// in later tokens, which run on the same XCD as the writer (XCD g owns head
// g in every launch), so the store goes to that XCD's L2 (sc0), like the
// hand-off words; a row is never read before it is written within a launch
// (rows < pos come from the cache, the current one from the tagged copy), so
// no reader's L1 can hold it stale, and a kernel boundary writes the L2 back
// for the next launch or the graph path. A device-scope 2-byte store here
// (fp16 KV) went to the memory side and held the wave's following stores, the
// tagged q/k/v words, back by ~2.4 us per layer.
// kv_put2(row, i, a, b) stores elements i and i + 64 of a cache row: fp32
// rows are in dimension order; fp16 rows are paired (slot 2i holds dim i,
// slot 2i + 1 dim i + 64), so the two halves go out as one dword -- 2-byte
// stores measured ~4x slower loads of the lines they touched afterwards.
__device__ __forceinline__ void kv_put2(float* row, int i, float a, float b) {
    asm volatile("global_store_dword %0, %1, off sc0" ::"v"(row + i), "v"(a) : "memory");
    asm volatile("global_store_dword %0, %1, off sc0" ::"v"(row + i + 64), "v"(b) : "memory");
}
__device__ __forceinline__ void kv_put2(_Float16* row, int i, float a, float b) {
    const unsigned w = (unsigned)__builtin_bit_cast(unsigned short, (_Float16)a) |
                       (unsigned)__builtin_bit_cast(unsigned short, (_Float16)b) << 16;
    asm volatile("global_store_dword %0, %1, off sc0" ::"v"(row + 2 * i), "v"(w) : "memory");
}
// Storage slots 16 part .. 16 part + 15 of a row as dims: the q (or current
// k) values to pair with them, from a dimension-ordered vector.
__device__ __forceinline__ void slots16(const float* src, int part, float (&d)[16], float*) {
    load_row16(src + part * 16, d);
}
__device__ __forceinline__ void slots16(const float* src, int part, float (&d)[16], _Float16*) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        d[2 * j] = src[part * 8 + j];
        d[2 * j + 1] = src[64 + part * 8 + j];
    }
}
// The value the cache holds for v.
__device__ __forceinline__ float kv_round(float v, float*) { return v; }
__device__ __forceinline__ float kv_round(float v, _Float16*) { return (float)(_Float16)v; }

// The full input vector (H values) into the workgroup's LDS copy xs: each of
// the four compute waves polls one quarter (words 256 w + lane + 64 i, i < 4:
// coalesced), so the XCD's L2 serves each word once per workgroup rather than
// once per wave, and a poll is 4 loads per lane instead of 16; after the
// waves meet, each reads the vector in the lane layout of a 1 KB weight line
// (lane l holds x[16 l .. 16 l + 15]). Returns the RMSNorm scale of g * x
// (g = gamma). xs is one of two buffers that alternate between the two
// gathers of a layer: the other still holds the previous vector, the base of
// the reduction that precedes the next gather, and the rendezvous here
// orders every wave's reads of a buffer before the writes that reuse it.
__device__ __forceinline__ bool gather_x(const LoopParams& p, Cx& c, const u64* src, uint32_t tag,
                                         const float (&gam)[16], float (&xv)[16], float& nscale,
                                         float* xs, int where) {
    const u64* base = src + c.g * LP_H + 256 * c.w + c.lane;
    for (uint32_t it = 0;; it++) {
        u64 v[4];
        ld_l2_4s(base, v);
        if (__all(tags_ok(v, tag))) {
#pragma unroll
            for (int i = 0; i < 4; i++) xs[256 * c.w + c.lane + 64 * i] = __uint_as_float((uint32_t)v[i]);
            break;
        }
        if (!keep_waiting(p, c, it, where)) return false;
    }
    if (!csync(p, c, where + 200)) return false;
    load_row16(xs + 16 * c.lane, xv);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 4)
        ss += xv[i] * xv[i] + xv[i + 1] * xv[i + 1] + xv[i + 2] * xv[i + 2] + xv[i + 3] * xv[i + 3];
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] *= gam[i];
    nscale = rsqrtf(wsum(ss) * (1.0f / (float)LP_H) + p.eps);
    return true;
}

// Cross-XCD reduction (P1 / P5): x_new[e] = base[e] + sum over the 8 XCDs'
// partials part[h][e], for this wave's 8 elements e = 32 j + 8 w + (lane >> 3)
// (lane & 7 = h); the 8-lane sum has one fixed order. xb is the workgroup's
// copy of the previous input vector. Stored tagged for the XCD's gather.
__device__ __forceinline__ bool reduce_x(const LoopParams& p, Cx& c, const u64* part, uint32_t ptag,
                                         u64* out, uint32_t otag, const float* xb, int where) {
    const int e = 32 * c.j + 8 * c.w + (c.lane >> 3);
    const u64* src = part + (c.lane & 7) * LP_H + e;
    float v[1];
    if (!poll<1>(p, c, [&](int) { return src; }, ptag, v, where)) return false;
    const float s = sum8(v[0]);
    if ((c.lane & 7) == 0) st_l2(out + c.g * LP_H + e, xb[e] + s, otag);
    return true;
}

// Per-unit constants of a phase are loaded one per lane before the phase
// waits for its input and read back with readlane.
struct Pre {
    float a = 0.f, b = 0.f, cs = 0.f, sn = 0.f;
};

// q/k/v unit u (0..255) of KV head g: the row pair (r, r + 64) of a 128-row
// head block: u < 128: query head 2g + u/64; u < 192: key head g; else value
// head g. Returns the first row of the pair in W_qkv.
__device__ __forceinline__ int qkv_row(int g, int u) {
    if (u < 128) return (LP_G * g + (u >> 6)) * LP_D + (u & 63);
    if (u < 192) return LP_KO + g * LP_D + (u - 128);
    return LP_KO + LP_NX * LP_D + g * LP_D + (u - 192);
}

// Per-layer constants of a compute wave, loaded into LDS once per launch
// (load_constants) so that no phase waits for them: every poll waits for all
// loads issued before it, and these scales (a few words per workgroup, read
// once per token) missed the caches. Value i of layer l:
//   0-3    q/k/v scale, lane 2m + r: row r of the wave's unit m (qkv_row)
//   4-7    the same rows' bias (0 without one)
//   8-13   gate_up scale, lane 2m + r: channel i_m, gate (r = 0) or up row
//   14-21  o_proj scale of row 32 j + 8 w + k, k = i - 14
//   22-29  down scale of row 32 j + 8 w + k, k = i - 22
__device__ __forceinline__ float layer_constant(const LoopParams& p, const Cx& c, int l, int i) {
    const LoopLayer& Lw = p.layers[l];
    if (i < 8) {
        const int u = 8 * c.j + c.w + LP_CW * ((i & 3) >> 1);
        const int row = qkv_row(c.g, u) + (i & 1) * 64;
        if (i < 4) return gld(Lw.s_qkv + row);
        return Lw.b_qkv ? gld(Lw.b_qkv + row) : 0.f;
    }
    if (i < 14) {
        const int k = i - 8;
        return gld(Lw.s_gu + LP_IX * c.g + 12 * c.j + c.w + LP_CW * (k >> 1) + (k & 1) * LP_I);
    }
    if (i < 22) return gld(Lw.s_o + 32 * c.j + 8 * c.w + (i - 14));
    if (i < 30) return gld(Lw.s_down + 32 * c.j + 8 * c.w + (i - 22));
    return 0.f;
}
__device__ __forceinline__ void load_constants(const LoopParams& p, Cx& c) {
    float* dst = c.cst + c.w * LP_NCST + c.lane;
    for (int l = 0; l < p.L; l++)
        if (c.lane < LP_NCST) dst[l * LP_CW * LP_NCST] = layer_constant(p, c, l, c.lane);
}
__device__ __forceinline__ const float* layer_cst(const Cx& c, int l) {
    return c.cst + (l * LP_CW + c.w) * LP_NCST;
}

__device__ __forceinline__ Pre pre_qkv(const Cx& c, int l, float rcs, float rsn) {
    const float* k = layer_cst(c, l);
    Pre q;
    if (c.lane < 4) {   // lane 2m + r: row r of this wave's unit m
        q.a = k[c.lane];
        q.b = k[4 + c.lane];
    }
    q.cs = rcs;   // lane m: RoPE angle of unit m
    q.sn = rsn;
    return q;
}

// qkv (P2): this wave's 2 units, from ring lines line0 + 2 (w + 4 m) + r.
// KT = the KV cache element type.
template <typename KT, bool TR>
__device__ bool phase_qkv(const LoopParams& p, Cx& c, int l, int pos, int line0, uint32_t tag,
                          const float (&xv)[16], float nscale, const Pre& pre) {
    if (!wait_upto(p, c, line0 + 2 * (c.w + LP_CW) + 1, 10)) return false;
    lp_stamp_in<TR>(p, c, 11);
    lp_v4i wv[2][2];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int r = 0; r < 2; r++) wv[m][r] = ring_line(c, line0 + 2 * (c.w + LP_CW * m) + r);
    float acc[4];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int r = 0; r < 2; r++) {
            float s[4] = {0.f, 0.f, 0.f, 0.f};
            lp_dot16s(xv, wv[m][r], s);
            acc[2 * m + r] = (s[0] + s[1]) + (s[2] + s[3]);
        }
    wsum4(acc[0], acc[1], acc[2], acc[3]);
    u64* dst = p.qkv + c.g * LP_QKVX;
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int u = 8 * c.j + c.w + LP_CW * m, i = u & 63;
        const float v0 = acc[2 * m] * rlane(pre.a, 2 * m) * nscale + rlane(pre.b, 2 * m);
        const float v1 = acc[2 * m + 1] * rlane(pre.a, 2 * m + 1) * nscale + rlane(pre.b, 2 * m + 1);
        const float cs = rlane(pre.cs, m), sn = rlane(pre.sn, m);
        if (c.lane != 0) continue;
        if (u < 192) {
            const float o0 = v0 * cs - v1 * sn, o1 = v0 * sn + v1 * cs;
            if (u < 128) {
                st_l2(dst + (u >> 6) * LP_D + i, o0, tag);
                st_l2(dst + (u >> 6) * LP_D + i + 64, o1, tag);
            } else {
                KT* kr = (KT*)p.kc + (((int64_t)l * LP_NX + c.g) * p.max_seq + pos) * LP_D;
                kv_put2(kr, i, o0, o1);
                st_l2(dst + 256 + i, o0, tag);
                st_l2(dst + 256 + i + 64, o1, tag);
            }
        } else {
            KT* vr = (KT*)p.vc + (((int64_t)l * LP_NX + c.g) * p.max_seq + pos) * LP_D;
            kv_put2(vr, i, v0, v1);
            st_l2(dst + 384 + i, v0, tag);
            st_l2(dst + 384 + i + 64, v1, tag);
        }
    }
    return true;
}

// gate_up (P6): this wave's 3 pairs (i, i + I), i = 384 g + 12 j + w + 4 m,
// lines line0 + 2 (w + 4 m) + r -> act = silu(g) * u.
__device__ __forceinline__ Pre pre_gu(const Cx& c, int l) {
    Pre q;
    if (c.lane < 6) q.a = layer_cst(c, l)[8 + c.lane];
    return q;
}

__device__ bool phase_gu(const LoopParams& p, Cx& c, int line0, uint32_t tag, const float (&xv)[16],
                         float nscale, const Pre& pre) {
    if (!wait_upto(p, c, line0 + 2 * (c.w + 2 * LP_CW) + 1, 40)) return false;
    lp_v4i wv[3][2];
#pragma unroll
    for (int m = 0; m < 3; m++)
#pragma unroll
        for (int r = 0; r < 2; r++) wv[m][r] = ring_line(c, line0 + 2 * (c.w + LP_CW * m) + r);
    float acc[6];
#pragma unroll
    for (int m = 0; m < 3; m++)
#pragma unroll
        for (int r = 0; r < 2; r++) {
            float s[4] = {0.f, 0.f, 0.f, 0.f};
            lp_dot16s(xv, wv[m][r], s);
            acc[2 * m + r] = (s[0] + s[1]) + (s[2] + s[3]);
        }
    wsum_n<6>(acc);
#pragma unroll
    for (int m = 0; m < 3; m++) {
        const float g = acc[2 * m] * rlane(pre.a, 2 * m) * nscale;
        const float up = acc[2 * m + 1] * rlane(pre.a, 2 * m + 1) * nscale;
        if (c.lane == 0)
            st_l2(p.act + c.g * LP_IX + 12 * c.j + c.w + LP_CW * m,
                  g * __frcp_rn(1.0f + __expf(-g)) * up, tag);
    }
    return true;
}

// o_proj partial (P4): rows 32 j + 8 w + 4 c' + (lane >> 4) (c' = 0, 1) over the
// 256 columns of KV head g's query heads; lane holds columns 16 (lane & 15) ..
// +16 of its row in line line0 + 2 w + c'. x = the merged head output in LDS;
// so[c'] = the row's output scale.
__device__ bool phase_opart(const LoopParams& p, Cx& c, int line0, uint32_t tag, const float (&so)[2]) {
    if (!wait_upto(p, c, line0 + 2 * c.w + 1, 32)) return false;
    float xv[16];
    load_row16(c.os + 16 * (c.lane & 15), xv);
    float acc[2];
#pragma unroll
    for (int cc = 0; cc < 2; cc++) {
        const lp_v4i wv = ring_line(c, line0 + 2 * c.w + cc);
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        lp_dot16s(xv, wv, s);
        acc[cc] = sum16((s[0] + s[1]) + (s[2] + s[3]));
    }
#pragma unroll
    for (int cc = 0; cc < 2; cc++) {
        const int r = 4 * cc + (c.lane >> 4);                 // row within the wave's 8
        const float v = acc[cc] * so[cc];
        if ((c.lane & 15) == 0) ll_store(p.opart + c.g * LP_H + 32 * c.j + 8 * c.w + r, v, tag);
    }
    return true;
}

// down partial (P7): rows 32 j + 8 w + (lane >> 3) over XCD g's 384 channels;
// line line0 + 3 w + cc holds channels 128 cc .. +128 of the wave's 8 rows,
// lane: 16 channels 128 cc + 16 (lane & 7).
__device__ bool phase_dpart(const LoopParams& p, Cx& c, int line0, uint32_t atag, uint32_t tag,
                            float sd) {
    // XCD g's 384 act values into the workgroup's LDS copy: waves 0-2 poll
    // 128 words each (2 per lane, coalesced), then the four waves meet
    static_assert(LP_IX == 3 * 128, "three waves poll the act slice");
    float* aw = c.acts;
    if (c.w < 3) {
        const u64* src = p.act + c.g * LP_IX + 128 * c.w + c.lane;
        for (uint32_t it = 0;; it++) {
            u64 v[2];
            ld_l2_2s(src, v);
            if (__all(tags_ok(v, atag))) {
                aw[128 * c.w + c.lane] = __uint_as_float((uint32_t)v[0]);
                aw[128 * c.w + c.lane + 64] = __uint_as_float((uint32_t)v[1]);
                break;
            }
            if (!keep_waiting(p, c, it, 7)) return false;
        }
    }
    if (!csync(p, c, 207)) return false;
    if (!wait_upto(p, c, line0 + 3 * c.w + 2, 50)) return false;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 3; cc++) {
        float xv[16];
        load_row16(aw + 128 * cc + 16 * (c.lane & 7), xv);
        lp_dot16s(xv, ring_line(c, line0 + 3 * c.w + cc), s);
    }
    const float v = sum8((s[0] + s[1]) + (s[2] + s[3])) * sd;
    if ((c.lane & 7) == 0) ll_store(p.dpart + c.g * LP_H + 32 * c.j + 8 * c.w + (c.lane >> 3), v, tag);
    return true;
}

// ------------------------------------------------------------- attention
struct AttRange {
    int t0, n, tw0, tw1;
};

// Positions of attention split s (workgroup j = s of XCD g) and of wave w in it.
__device__ __forceinline__ AttRange att_range(int s, int w, int pos) {
    AttRange r;
    const int Lc = pos + 1, cs = (Lc + LP_S - 1) / LP_S;
    r.t0 = s * cs;
    r.n = min(cs, Lc - r.t0);
    const int nw = r.n > 0 ? (r.n + LP_CW - 1) / LP_CW : 0;
    r.tw0 = r.t0 + w * nw;
    r.tw1 = r.n > 0 ? min(r.t0 + r.n, r.tw0 + nw) : r.tw0;
    return r;
}

// A pass's cache data as loaded (raw bits; fp16 is widened only after the q
// poll, so no conversion sits right behind a load and makes the wave wait for
// it): a lane's 16 key slots and its 2 value slots of each of 8 positions.
template <typename KT>
struct KvRaw {
    static constexpr int KQ = 16 * (int)sizeof(KT) / 16;   // 16-byte key pieces
    static constexpr int VW = (int)sizeof(KT) / 2;         // dwords per value pair
    lp_v4i k[KQ];
    uint32_t v[8][VW];
};
template <typename KT>
__device__ __forceinline__ void kv_load_k(const KT* src, KvRaw<KT>& r) {
#pragma unroll
    for (int q = 0; q < KvRaw<KT>::KQ; q++) r.k[q] = gld((const lp_v4i*)src + q);
}
template <typename KT>
__device__ __forceinline__ void kv_zero_k(KvRaw<KT>& r) {
#pragma unroll
    for (int q = 0; q < KvRaw<KT>::KQ; q++) r.k[q] = lp_v4i{0, 0, 0, 0};
}
template <typename KT>
__device__ __forceinline__ void kv_load_v(const KT* src, KvRaw<KT>& r, int i) {
#pragma unroll
    for (int w = 0; w < KvRaw<KT>::VW; w++) r.v[i][w] = gld((const uint32_t*)src + w);
}
__device__ __forceinline__ void kv_widen(const KvRaw<float>& r, float (&kk)[16], float (&vv)[8][2]) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) kk[4 * q + e] = __int_as_float(r.k[q][e]);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        vv[i][0] = __uint_as_float(r.v[i][0]);
        vv[i][1] = __uint_as_float(r.v[i][1]);
    }
}
__device__ __forceinline__ float h2f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
}
__device__ __forceinline__ void kv_widen(const KvRaw<_Float16>& r, float (&kk)[16], float (&vv)[8][2]) {
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t w = (uint32_t)r.k[q][e];
            kk[8 * q + 2 * e] = h2f(w & 0xFFFFu);
            kk[8 * q + 2 * e + 1] = h2f(w >> 16);
        }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        vv[i][0] = h2f(r.v[i][0] & 0xFFFFu);
        vv[i][1] = h2f(r.v[i][0] >> 16);
    }
}

// Partial attention (P3) of split s = j over this workgroup's positions, for
// both query heads of KV head g. A wave takes its positions 8 per pass. Scores
// use 8 lanes per position (lane group jj = position slot, 16 dims per lane);
// the value rows are read in the accumulation layout instead (lane l holds
// row slots 2l, 2l+1 of each of the pass's 8 positions, one coalesced row per
// load), so with the pass's 8 weights broadcast from their lane groups every
// lane accumulates its own two output dims: the softmax state (max, sum) is
// wave-uniform and no cross-lane combine of the outputs is needed. The current
// position's k/v (this step's, from the tagged copy) is one extra pass with
// slot 0 only. The waves' partials go to LDS and one pass over them combines
// the four waves; the split's (max, sum, o) is stored tagged.
template <typename KT, bool TR>
__device__ bool phase_att(const LoopParams& p, Cx& c, int l, int pos, uint32_t qtag, uint32_t tag) {
    constexpr int G = LP_G;
    // fp16 rows are paired (kv_put2): lane l's two value slots are dims l, l + 64
    constexpr bool VPAIR = sizeof(KT) == 2;
    const AttRange r = att_range(c.j, c.w, pos);
    if (r.n <= 0) return true;
    const int jj = c.lane >> 3, part = c.lane & 7;
    const int npos = max(0, r.tw1 - r.tw0), passes = (npos + 7) / 8;
    float* stg = c.stg + c.w * LP_STG;
    const bool has_cur = pos >= r.tw0 && pos < r.tw1;
    // Keys/values of the earlier positions (final since the steps that wrote
    // them): issued before the q poll, so their latency hides behind it.
    const KT* kb = (const KT*)p.kc + ((int64_t)l * LP_NX + c.g) * p.max_seq * LP_D;
    const KT* vb = (const KT*)p.vc + ((int64_t)l * LP_NX + c.g) * p.max_seq * LP_D;
    auto load_pass = [&](int ps, KvRaw<KT>& raw) {
        const int tp = r.tw0 + ps * 8 + jj;
        if (tp < r.tw1 && tp != pos) kv_load_k(kb + (int64_t)tp * LP_D + part * 16, raw);
        else kv_zero_k(raw);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int tv = r.tw0 + ps * 8 + i;   // the same in every lane
            if (tv < r.tw1 && tv != pos) {
                kv_load_v(vb + (int64_t)tv * LP_D + 2 * c.lane, raw, i);
            } else {
#pragma unroll
                for (int w = 0; w < KvRaw<KT>::VW; w++) raw.v[i][w] = 0u;
            }
        }
    };
    KvRaw<KT> pre[LP_NPF];
#pragma unroll
    for (int ps = 0; ps < LP_NPF; ps++) load_pass(ps, pre[ps]);
    {
        // q of the two query heads and the current k/v row, in one poll
        // (words lane + 64 i: q for i < 4, then k, v)
        const u64* src = p.qkv + c.g * LP_QKVX + c.lane;
        for (uint32_t it = 0;; it++) {
            u64 v[8];
            ld_l2_8s(src, v);
            bool ok = true;
#pragma unroll
            for (int i = 0; i < 8; i++) ok &= (i < 2 * G || has_cur) ? (uint32_t)(v[i] >> 32) == qtag : true;
            if (__all(ok)) {
#pragma unroll
                for (int i = 0; i < 8; i++) stg[c.lane + 64 * i] = __uint_as_float((uint32_t)v[i]);
                break;
            }
            if (!keep_waiting(p, c, it, 20)) return false;
        }
    }
    lp_stamp_in<TR>(p, c, 12);
    cbar();
    float qv[G][16];
#pragma unroll
    for (int h = 0; h < G; h++) slots16(stg + h * LP_D, part, qv[h], (KT*)nullptr);
    float m[G], lsum[G], o[G][2];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = -INFINITY;
        lsum[h] = 0.f;
        o[h][0] = o[h][1] = 0.f;
    }
    // One pass: slot jj's score in its lane group (-inf when invalid), the
    // wave's running max and sum, and every lane's two output dims. The two
    // heads are independent chains, written side by side and branch-free so
    // that their latencies overlap.
    auto pass = [&](const float (&kk)[16], const float (&vv)[8][2], bool valid) {
        float sc[G], mx[G], corr[G], e[G];
#pragma unroll
        for (int h = 0; h < G; h++) {
            float d4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 16; i++) d4[i & 3] = fmaf(qv[h][i], kk[i], d4[i & 3]);
            sc[h] = valid ? sum8((d4[0] + d4[1]) + (d4[2] + d4[3])) * p.att_scale : -INFINITY;
        }
#pragma unroll
        for (int h = 0; h < G; h++) mx[h] = fmaxf(m[h], wmax(sc[h]));   // wave-uniform
#pragma unroll
        for (int h = 0; h < G; h++) {
            corr[h] = mx[h] == -INFINITY ? 0.f : __expf(m[h] - mx[h]);
            e[h] = sc[h] == -INFINITY ? 0.f : __expf(sc[h] - mx[h]);
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
            float o0 = o[h][0] * corr[h], o1 = o[h][1] * corr[h], es = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float ei = rlane(e[h], 8 * i);
                o0 = fmaf(ei, vv[i][0], o0);
                o1 = fmaf(ei, vv[i][1], o1);
                es += ei;
            }
            o[h][0] = o0;
            o[h][1] = o1;
            lsum[h] = fmaf(lsum[h], corr[h], es);
            m[h] = mx[h];
        }
    };
#pragma unroll
    for (int ps = 0; ps < LP_NPF; ps++) {
        if (ps >= passes) break;   // wave-uniform: no work for an empty pass
        const int tp = r.tw0 + ps * 8 + jj;
        float kk[16], vv[8][2];
        kv_widen(pre[ps], kk, vv);
        pass(kk, vv, tp < r.tw1 && tp != pos);
    }
    for (int ps = LP_NPF; ps < passes; ps++) {
        const int tp = r.tw0 + ps * 8 + jj;
        KvRaw<KT> raw;
        load_pass(ps, raw);
        float kk[16], vv[8][2];
        kv_widen(raw, kk, vv);
        pass(kk, vv, tp < r.tw1 && tp != pos);
    }
    if (has_cur) {
        // this step's k/v as the cache holds them, in slot 0
        float kk[16], vv[8][2];
        slots16(stg + G * LP_D, part, kk, (KT*)nullptr);
#pragma unroll
        for (int i = 0; i < 16; i++) kk[i] = kv_round(kk[i], (KT*)nullptr);
        const int d0 = VPAIR ? c.lane : 2 * c.lane, d1 = VPAIR ? c.lane + 64 : 2 * c.lane + 1;
        vv[0][0] = kv_round(stg[G * LP_D + LP_D + d0], (KT*)nullptr);
        vv[0][1] = kv_round(stg[G * LP_D + LP_D + d1], (KT*)nullptr);
#pragma unroll
        for (int i = 1; i < 8; i++) vv[i][0] = vv[i][1] = 0.f;
        pass(kk, vv, jj == 0);
    }
    // the wave's partial o[h][128] (relative to its max) and its max / sum
#pragma unroll
    for (int h = 0; h < G; h++) {
        float* ap = c.attp + (c.w * G + h) * LP_D;
        if (VPAIR) {
            ap[c.lane] = o[h][0];
            ap[c.lane + 64] = o[h][1];
        } else {
            *(float2*)(ap + 2 * c.lane) = make_float2(o[h][0], o[h][1]);
        }
        if (c.lane == 0) {
            c.attm[c.w * G + h] = m[h];
            c.attm[LP_CW * G + c.w * G + h] = lsum[h];
        }
    }
    lp_stamp_in<TR>(p, c, 13);
    if (!csync(p, c, 22)) return false;
    // combine: one (head, dim) per thread of the four waves; partial layout
    // att[g][h][split][max, sum, o[128]]
    u64* dst = p.att + ((int64_t)c.g * G * LP_S + c.j) * LP_PART;
    for (int e = c.w * 64 + c.lane; e < G * LP_D; e += LP_CW * 64) {
        const int h = e >> 7, d = e & 127;
        float M = -INFINITY;
#pragma unroll
        for (int wv = 0; wv < LP_CW; wv++) M = fmaxf(M, c.attm[wv * G + h]);
        float acc = 0.f, den = 0.f;
#pragma unroll
        for (int wv = 0; wv < LP_CW; wv++) {
            const float mw = c.attm[wv * G + h];
            const float F = mw == -INFINITY ? 0.f : __expf(mw - M);
            acc = fmaf(F, c.attp[(wv * G + h) * LP_D + d], acc);
            den = fmaf(F, c.attm[LP_CW * G + wv * G + h], den);
        }
        st_l2(dst + h * LP_S * LP_PART + 2 + d, acc, tag);
        if (d == 0) {
            st_l2(dst + h * LP_S * LP_PART, M, tag);
            st_l2(dst + h * LP_S * LP_PART + 1, den, tag);
        }
    }
    return true;
}

// Merge (start of P4) of the active splits of KV head g's query heads into the
// head output o_g [2][128] in LDS: wave w merges head w >> 1, dims
// 64 (w & 1) + lane, in split order; then the four waves meet.
template <bool TR>
__device__ bool merge_heads(const LoopParams& p, Cx& c, int pos, uint32_t ptag) {
    const int hh = c.w >> 1, d = 64 * (c.w & 1) + c.lane;
    const int Lc = pos + 1, cs = (Lc + LP_S - 1) / LP_S, sact = (Lc + cs - 1) / cs;
    float mm[LP_S], ll[LP_S], oo[LP_S];
    const u64* base = p.att + (int64_t)(c.g * LP_G + hh) * LP_S * LP_PART;
    for (uint32_t it = 0;; it++) {
        u64 ml[16], ov[8];   // (max, sum) of split s at ml[2s], ml[2s+1]; o[d] of split s at ov[s]
        ld_l2_merge(base, base + 4 * LP_PART, base + 2 + d, base + 4 * LP_PART + 2 + d, ml, ov);
        bool ok = true;
#pragma unroll
        for (int s = 0; s < LP_S; s++) {
            if (s >= sact) continue;
            ok &= (uint32_t)(ml[2 * s] >> 32) == ptag && (uint32_t)(ml[2 * s + 1] >> 32) == ptag &&
                  (uint32_t)(ov[s] >> 32) == ptag;
            mm[s] = __uint_as_float((uint32_t)ml[2 * s]);
            ll[s] = __uint_as_float((uint32_t)ml[2 * s + 1]);
            oo[s] = __uint_as_float((uint32_t)ov[s]);
        }
        if (__all(ok)) break;
        if (!keep_waiting(p, c, it, 30)) return false;
    }
    lp_stamp_in<TR>(p, c, 14);
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < LP_S; s++)
        if (s < sact) M = fmaxf(M, mm[s]);
    float den = 0.f, a = 0.f;
#pragma unroll
    for (int s = 0; s < LP_S; s++) {
        if (s >= sact) continue;
        const float f = mm[s] == -INFINITY ? 0.f : __expf(mm[s] - M);
        den += f * ll[s];
        a += f * oo[s];
    }
    c.os[hh * LP_D + d] = a * __frcp_rn(den);
    return csync(p, c, 31);
}

typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) const int8_t lds_i8;
typedef __attribute__((address_space(3))) u64 lds_u64;
typedef __attribute__((address_space(1))) const lp_v4i glb_v4i;   // global (not flat) loads
typedef __attribute__((address_space(1))) const float glb_f32;

// ----------------------------------------------------- lm_head on MFMA
// The lm phase multiplies one vector by 151936 x 1024 int8 rows. On the VALU
// that is a byte conversion and an fp32 FMA per weight (one compute wave per
// SIMD: ~14 us of issue per token); here the rows go to the matrix cores
// (v_mfma_i32_16x16x64_i8) untouched, against an exact int8 decomposition of
// the vector. v = gamma * x (the RMSNorm scale nscale multiplies the sums) is
// split under one power-of-two scale S = 2^(E - 6), where max |v| = m 2^E with
// m in [0.5, 1): u = v / S (exact, |u| < 64), q1 = rint(u) and
// q_{i+1} = rint(128 (u_i - q_i)) (every step exact), so every part is in
// [-64, 64] and v = S (q1 + q2/128 + q3/128^2 + q4/128^3) + e with
// |e| <= S 2^-22 (about 2^-27 max |v|, far below fp32 rounding of the sums).
// A row's four sums c_i = sum_k W[row][k] q_i[k] are exact int32
// (|c_i| <= 64 * 127 * 1024 < 2^23), and its value is
// S (((c4 / 128 + c3) / 128 + c2) / 128 + c1): a few fp32 roundings in all,
// where the FMA chain rounded once per weight.
//
// Operand layout (as the skinny W8A8 kernel's): lane l = r + 16 q supplies the
// 16 bytes at K = 64 i + 16 q of MFMA i (16 per 1024-byte row); for B that is
// lm_head row r of the group, for A part r of the vector (r < 4) or zeros.
// The A operand lives in LDS, [16 MFMAs][64 lanes][16 B], and is read back
// whole lines at a time; the C rows 0-3 (lanes 0-15) are the four sums of
// row r = lane.

// Writes this wave's share of the A operand (the 4-byte column 4 w of every
// part slot, and the zero rows of MFMAs 4 w .. 4 w + 3) from gamma * x in
// xv (lane l: elements 16 l .. 16 l + 15, the whole vector in every wave);
// returns S. The caller's rendezvous then makes the operand whole.
__device__ __forceinline__ float lm_split(const Cx& c, const float (&xv)[16], int8_t* A) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(xv[i]));
    amax = wmax(amax);
    int E;
    (void)frexpf(amax, &E);   // amax = 0: E = 0, every part 0
    // u = x 2^(6 - E) by exponent arithmetic (v_ldexp_f32): exact, and unlike
    // a multiply by 2^(6 - E) it cannot overflow when amax is below 2^-121
    // this wave's elements 16 l + 4 w + t: MFMA i = l / 4, lane chunk q = l % 4,
    // byte 4 w + t of the chunk
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const float x = c.w == 0 ? xv[t] : c.w == 1 ? xv[4 + t] : c.w == 2 ? xv[8 + t] : xv[12 + t];
        float u = ldexpf(x, 6 - E);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float q = rintf(u);
            pk[m] |= ((uint32_t)(int)q & 0xFFu) << (8 * t);
            u = (u - q) * 128.f;
        }
    }
    typedef __attribute__((address_space(3))) uint32_t lds_u32w;
    typedef __attribute__((address_space(3))) lp_v4i lds_v4w;
    typedef __attribute__((address_space(3))) int8_t lds_i8w;
    lds_i8w* L = (lds_i8w*)A;
    const int i = c.lane >> 2, q = c.lane & 3;
#pragma unroll
    for (int m = 0; m < 4; m++) *(lds_u32w*)(L + i * 1024 + (m + 16 * q) * 16 + 4 * c.w) = pk[m];
    // zero rows 4..15 of MFMAs 4 w .. 4 w + 3: 192 slots of 16 bytes, 3 per lane
#pragma unroll
    for (int s = 0; s < 3; s++) {
        const int slot = c.lane + 64 * s, r = slot % 48;
        *(lds_v4w*)(L + (4 * c.w + slot / 48) * 1024 + (4 + r % 12 + 16 * (r / 12)) * 16) = lp_v4i{0, 0, 0, 0};
    }
    return ldexpf(1.f, E - 6);
}

// 16 lm_head rows (group g of this wave: rows w + 4 (16 g + r)) into the B
// operand registers, and their scales.
__device__ __forceinline__ void lm_load(const int8_t* lm, const float* s_lm, int uv0, int w, int nk, int lane,
                                        int g, lp_v4i (&wr)[16], float& s) {
    const int k = min(16 * g + (lane & 15), nk - 1);   // past the end: re-read the last row
    const int row = uv0 + w + 4 * k;
    const int8_t* src = lm + (int64_t)row * LP_H + 16 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 16; i++) wr[i] = *(glb_v4i*)(src + 64 * i);
    s = *(glb_f32*)(s_lm + row);
}

// One group: 16 MFMAs on two accumulators, then lanes 0-15 hold the four sums
// of row r = lane; its value, the lane's running maximum (rows ascend within a
// lane, ties keep the first) and, on the last step, its logit.
__device__ __forceinline__ void lm_group(const lds_i8* A, int g, int uv0, int w, int nk, int lane, float sn,
                                         const lp_v4i (&wr)[16], float s, float* logits, float& bestv,
                                         int& besti) {
    lp_v4i c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
        const lp_v4i a0 = *(const __attribute__((address_space(3))) lp_v4i*)(A + i * 1024 + lane * 16);
        const lp_v4i a1 = *(const __attribute__((address_space(3))) lp_v4i*)(A + (i + 1) * 1024 + lane * 16);
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, wr[i], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, wr[i + 1], c1, 0, 0, 0);
    }
    const lp_v4i cs = c0 + c1;   // |c| < 2^24
    const float y = (((float)cs[3] * 0.0078125f + (float)cs[2]) * 0.0078125f + (float)cs[1]) * 0.0078125f +
                    (float)cs[0];
    const float v = y * sn * s;
    const int k = 16 * g + lane;
    const bool in = lane < 16 && k < nk;
    const int row = uv0 + w + 4 * k;
    if (in && v > bestv) {
        bestv = v;
        besti = row;
    }
    // a global (not flat) store: a pending flat store makes the compiler's
    // next wait drain every load in flight
    if (in && logits) *(__attribute__((address_space(1))) float*)(logits + row) = v;
}

// lm_head: the one phase that is pure streaming (155 MB at the Qwen3-0.6B
// shape) and waits on no other workgroup, so the compute waves read its rows
// straight from HBM into the B operand registers, 16 rows (16 KB) per group,
// two groups in flight. This wave's rows: uv0 + w + 4 k. Out of line, so that
// its registers are its own. sn = S * nscale. Writes the wave's argmax key.
__device__ __noinline__ void phase_lm(const int8_t* lm, const float* s_lm, float* logits, int uv0, int nuv, int w,
                                      int lane, const lds_i8* A, float sn, uint32_t tag, lds_u64* wkey) {
    const int nk = nuv > w ? (nuv - w + LP_CW - 1) / LP_CW : 0;   // rows of this wave
    const int ng = (nk + 15) / 16;
    float bestv = -INFINITY;
    int besti = -1;
    lp_v4i wa[16], wb[16];
    float sa = 0.f, sb = 0.f;
    // Every load below is unconditional within its block, so the compiler's
    // waits count exactly (a load behind a branch makes it wait for all).
    if (ng > 0) {
        lm_load(lm, s_lm, uv0, w, nk, lane, 0, wa, sa);
        int g = 0;
        for (; g + 2 < ng; g += 2) {
            lm_load(lm, s_lm, uv0, w, nk, lane, g + 1, wb, sb);
            __builtin_amdgcn_sched_barrier(0);
            lm_group(A, g, uv0, w, nk, lane, sn, wa, sa, logits, bestv, besti);
            __builtin_amdgcn_sched_barrier(0);
            lm_load(lm, s_lm, uv0, w, nk, lane, g + 2, wa, sa);
            __builtin_amdgcn_sched_barrier(0);
            lm_group(A, g + 1, uv0, w, nk, lane, sn, wb, sb, logits, bestv, besti);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (g + 1 < ng) {
            lm_load(lm, s_lm, uv0, w, nk, lane, g + 1, wb, sb);
            __builtin_amdgcn_sched_barrier(0);
            lm_group(A, g, uv0, w, nk, lane, sn, wa, sa, logits, bestv, besti);
            __builtin_amdgcn_sched_barrier(0);
            lm_group(A, g + 1, uv0, w, nk, lane, sn, wb, sb, logits, bestv, besti);
        } else {
            lm_group(A, g, uv0, w, nk, lane, sn, wa, sa, logits, bestv, besti);
        }
    }
    const u64 key = wave_max_u64(besti >= 0 ? lp_key(bestv, besti, tag) : 0);
    if (lane == 0) *wkey = key;
}

// Argmax over the workgroups' keys of the lm phase tagged `tag` (first max,
// tensor_ops.c:649-662).
// The keys are polled four per lane with no branch between the loads, so the
// four cross-XCD round trips overlap (a guarded load in a loop waited for each
// load before the next one issued: 21 us per token).
static_assert(LP_NBLK % 64 == 0, "argmax keys: whole waves");
__device__ bool argmax_id(const LoopParams& p, Cx& c, uint32_t tag, int& id) {
    constexpr int n = LP_NBLK / 64;
    for (uint32_t it = 0;; it++) {
        u64 k[n];
#pragma unroll
        for (int i = 0; i < n; i++) k[i] = ll_load(p.keys + c.lane + 64 * i);
        u64 best = 0;
        bool ok = true;
#pragma unroll
        for (int i = 0; i < n; i++) {
            ok &= (uint32_t)(k[i] & 0x3FFF) == (tag & 0x3FFFu);
            best = k[i] > best ? k[i] : best;
        }
        if (__all(ok)) {
            best = wave_max_u64(best);
            id = (int)(0x3FFFFu - (uint32_t)((best >> 14) & 0x3FFFF));
            return true;
        }
        if (!keep_waiting(p, c, it, 70)) return false;
    }
}

__device__ void stream_role(const LoopParams& p, Cx& c) {
    const int sw = c.w - LP_CW;
    const int8_t* src = p.stream + (int64_t)c.role * 1024 + c.lane * 16;
    typedef __attribute__((address_space(3))) void lds_t;
    int G = 0, inflight = 0, published = 0;
    bool ok = true;
    for (int t = 0; t < p.n_steps && ok; t++) {
        const int nl = p.lpt;
        for (int j = ((sw - G) % LP_SW + LP_SW) % LP_SW; j < nl; j += LP_SW) {
            const int Lg = G + j;
            // every 8th line; an asm read, so the compiler does not first wait
            // for every copy in flight (it cannot tell the flag from the ring)
            if (((j / LP_SW) & 7) == 0 && lds_ld_asm(c.abort)) { ok = false; break; }
            // the slot of line Lg held line Lg - LP_RING: free once every
            // compute wave has moved past it
            auto room = [&]() {
                const lp_v4i dn = lds_ld_ready(c.done);   // done[] is 16-byte aligned too
                return min(min(dn[0], dn[1]), min(dn[2], dn[3])) > Lg - LP_RING;
            };
            if (!room()) {
                wait_vm<0>();
                published += inflight;
                inflight = 0;
                lds_st_raw(&c.ready[sw], published);
                for (uint32_t it = 0; !room(); it++) {
                    if (!keep_waiting(p, c, it, 80)) { ok = false; break; }
                    __builtin_amdgcn_s_sleep(2);
                }
                if (!ok) break;
                cbar();
            }
            // nt: the weights are read once per token; keep them out of the caches
            __builtin_amdgcn_global_load_lds((const void*)(src + (int64_t)j * (LP_NBLK * 1024)),
                                             (lds_t*)(c.ring + (size_t)(Lg % LP_RING) * 1024), 16,
                                             0, 2);
            if (++inflight == LP_INFL) {
                wait_vm<LP_INFL - 1>();
                inflight--;
                published++;
                lds_st_raw(&c.ready[sw], published);
            }
        }
        G += nl;
    }
    wait_vm<0>();
    lds_st(&c.ready[sw], published + inflight);
}

// ----------------------------------------------------------- compute waves
__device__ __forceinline__ void gld16(const float* src, float (&d)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const lp_f4 a = gld((const lp_f4*)(src + 4 * i));
        d[4 * i] = a[0]; d[4 * i + 1] = a[1]; d[4 * i + 2] = a[2]; d[4 * i + 3] = a[3];
    }
}

template <typename KT, bool TR>
__device__ void compute_role(const LoopParams& p, Cx& c) {
    __builtin_amdgcn_s_setprio(2);
    load_constants(p, c);
    const bool att_blk = c.j < LP_S;
    int Gl = 0;        // first ring line of the current token
    int id = 0;
    for (int t = 0; t < p.n_steps; t++) {
        asm volatile("" : "+v"(c.lane));
        const int pos = p.pos0 + t;
        const bool lm = lm_needed(p, t);
        if (t == 0 || pos < p.prompt_len) {
            id = p.ids[pos];
        } else {
            if (!argmax_id(p, c, tag_of(p, t - 1, p.L, 1), id)) return;
            if (c.role == 0 && c.w == 0 && c.lane == 0) p.ids[pos] = id;
        }
        if (id < 0 || id >= p.V) id = 0;
        // RoPE angles of this wave's two q/k units at this position (lane m:
        // unit m), the same in every layer of the token
        float rcs = 0.f, rsn = 0.f;
        if (c.lane < 2) {
            const int u = 8 * c.j + c.w + LP_CW * c.lane;
            rcs = gld(p.cos_t + (int64_t)pos * 64 + (u & 63));
            rsn = gld(p.sin_t + (int64_t)pos * 64 + (u & 63));
        }
        const float* emb = p.embed + (int64_t)id * LP_H;
        for (int l = 0; l < p.L; l++) {
            // Opaque per-iteration copy of the lane id: keeps the compiler from
            // hoisting every per-lane address of the loop body out of the loop
            // (they would stay live across all phases and spill).
            asm volatile("" : "+v"(c.lane));
            c.tt = t;
            c.tl = l;
            const LoopLayer& Lw = p.layers[l];
            const int lb = Gl + l * LP_LPL;
            // ---- P1 + P2: x'' (embedding row or reduced), RMSNorm, q/k/v of head g
            {
                // A poll waits for every load issued before it, so what a
                // phase needs from memory is loaded where it has time to land:
                // the norm weights (L2 hits after the first workgroup of the
                // XCD) before the reduction, the scales from LDS.
                cbar();   // nothing may move above the previous phase
                lp_stamp<TR>(p, c, t, l, 0);
                float gam[16], xv[16], nscale;
                gld16(Lw.in_norm + 16 * c.lane, gam);
                if (l > 0 && !reduce_x(p, c, p.dpart, tag_of(p, t, l - 1, PH_DP), p.xr, tag_of(p, t, l, PH_XR),
                                       c.xs + LP_H, 1))
                    return;
                lp_stamp<TR>(p, c, t, l, 1);
                cbar();
                if (l == 0) {
                    gld16(emb + 16 * c.lane, xv);
                    float ss = 0.f;
                    // every wave writes the same row: x'' of layer 0
                    float* xw = c.xs + 16 * c.lane;
#pragma unroll
                    for (int i = 0; i < 16; i += 4) {
                        *(float4*)(xw + i) = make_float4(xv[i], xv[i + 1], xv[i + 2], xv[i + 3]);
                        ss += xv[i] * xv[i] + xv[i + 1] * xv[i + 1] + xv[i + 2] * xv[i + 2] +
                              xv[i + 3] * xv[i + 3];
                    }
#pragma unroll
                    for (int i = 0; i < 16; i++) xv[i] *= gam[i];
                    nscale = rsqrtf(wsum(ss) * (1.0f / (float)LP_H) + p.eps);
                } else {
                    if (!gather_x(p, c, p.xr, tag_of(p, t, l, PH_XR), gam, xv, nscale, c.xs, 2)) return;
                }
                // the q/k/v constants (LDS) after the gather: +0.15% over reading them before it
                const Pre pq = pre_qkv(c, l, rcs, rsn);
                lp_stamp<TR>(p, c, t, l, 2);
                if (!phase_qkv<KT, TR>(p, c, l, pos, lb, tag_of(p, t, l, PH_QKV), xv, nscale, pq)) return;
                lp_stamp<TR>(p, c, t, l, 3);
                set_done(c, lb + LP_OFF_O);
            }
            // ---- P3: attention partials of head g's splits
            if (att_blk && !phase_att<KT, TR>(p, c, l, pos, tag_of(p, t, l, PH_QKV), tag_of(p, t, l, PH_ATT)))
                return;
            if (att_blk) lp_stamp<TR>(p, c, t, l, 4);
            // ---- P4: merge, o_proj partial over head g's columns
            {
                const float* lk = layer_cst(c, l) + 14 + (c.lane >> 4);
                const float so[2] = {lk[0], lk[4]};
                if (!merge_heads<TR>(p, c, pos, tag_of(p, t, l, PH_ATT))) return;
                lp_stamp<TR>(p, c, t, l, 5);
                if (!phase_opart(p, c, lb + LP_OFF_O, tag_of(p, t, l, PH_OP), so)) return;
                lp_stamp<TR>(p, c, t, l, 6);
                set_done(c, lb + LP_OFF_GU);
            }
            // ---- P5 + P6: x' (reduced), RMSNorm, gate_up + SwiGLU for XCD g's channels
            {
                cbar();
                const Pre pg = pre_gu(c, l);
                float gam[16], xv[16], nscale;
                gld16(Lw.post_norm + 16 * c.lane, gam);
                if (!reduce_x(p, c, p.opart, tag_of(p, t, l, PH_OP), p.xr2, tag_of(p, t, l, PH_XR2), c.xs, 3))
                    return;
                lp_stamp<TR>(p, c, t, l, 7);
                if (!gather_x(p, c, p.xr2, tag_of(p, t, l, PH_XR2), gam, xv, nscale, c.xs + LP_H, 4)) return;
                lp_stamp<TR>(p, c, t, l, 8);
                if (!phase_gu(p, c, lb + LP_OFF_GU, tag_of(p, t, l, PH_ACT), xv, nscale, pg)) return;
                lp_stamp<TR>(p, c, t, l, 9);
                set_done(c, lb + LP_OFF_DN);
            }
            // ---- P7: down partial over XCD g's channels
            {
                const float sd = layer_cst(c, l)[22 + (c.lane >> 3)];
                if (!phase_dpart(p, c, lb + LP_OFF_DN, tag_of(p, t, l, PH_ACT), tag_of(p, t, l, PH_DP), sd))
                    return;
                lp_stamp<TR>(p, c, t, l, 10);
                set_done(c, lb + LP_LPL);
            }
        }
        if (lm) {
            lp_stamp<TR>(p, c, t, p.L, 0);
            float gam[16], xv[16], nscale;
            gld16(p.final_norm + 16 * c.lane, gam);
            if (!reduce_x(p, c, p.dpart, tag_of(p, t, p.L - 1, PH_DP), p.xr, tag_of(p, t, p.L, PH_XR),
                          c.xs + LP_H, 9))
                return;
            lp_stamp<TR>(p, c, t, p.L, 1);
            if (!gather_x(p, c, p.xr, tag_of(p, t, p.L, PH_XR), gam, xv, nscale, c.xs, 11)) return;
            lp_stamp<TR>(p, c, t, p.L, 2);
            // gamma * x as the lm phase's int8 matrix operand (in the x-copy region
            // of LDS), each wave writing its share; the rendezvous makes it whole
            int8_t* A = (int8_t*)c.xw;
            const float S = lm_split(c, xv, A);
            if (!csync(p, c, 60)) return;
            const uint32_t tl = tag_of(p, t, p.L, 1);
            phase_lm(p.lm_head, p.s_lm, t == p.n_steps - 1 ? p.logits : nullptr, c.uv0, c.nuv, c.w, c.lane,
                     (const lds_i8*)A, S * nscale, tl, (lds_u64*)(c.wkeys + c.w));
            lp_stamp<TR>(p, c, t, p.L, 3);
            if (!csync(p, c, 61)) return;
            if (c.w == 0 && c.lane == 0) {
                u64 b = c.wkeys[0];
                for (int i = 1; i < LP_CW; i++) b = c.wkeys[i] > b ? c.wkeys[i] : b;
                b = (b & ~(u64)0x3FFF) | (u64)(tl & 0x3FFFu);
                __hip_atomic_store(p.keys + c.role, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            lp_stamp<TR>(p, c, t, p.L, 4);
        }
        Gl += p.lpt;
    }
    // The last step's argmax -> ids[pos+1] and the device position/state.
    if (c.role == 0 && c.w == 0) {
        const int pos = p.pos0 + p.n_steps - 1;
        int last = id;
        if (pos + 1 >= p.prompt_len) {
            if (!argmax_id(p, c, tag_of(p, p.n_steps - 1, p.L, 1), last)) return;
            if (c.lane == 0 && pos + 1 < p.max_seq + 1) p.ids[pos + 1] = last;
        }
        if (c.lane == 0) {
            p.state[0] = pos + 1;
            p.state[2] = last;
        }
    }
}

template <typename KT, bool TR>
__global__ __launch_bounds__(LP_THREADS, 1) void decode_loop_kernel(LoopParams p) {
    extern __shared__ __attribute__((aligned(16))) int8_t lp_lds[];
    __shared__ __attribute__((aligned(16))) int ready[LP_SW];
    __shared__ __attribute__((aligned(16))) int done[LP_CW];
    __shared__ int sync_ctr, abort_flag, role;
    __shared__ u64 wkeys[LP_CW];
    if (threadIdx.x < LP_SW) ready[threadIdx.x] = 0;
    if (threadIdx.x < LP_CW) done[threadIdx.x] = 0;
    if (threadIdx.x == 0) {
        sync_ctr = 0;
        abort_flag = 0;
        role = -1;
        // An earlier launch of this decoder found the grid not co-resident:
        // its steps have not run, so this one leaves too (the host re-runs
        // them all in graph mode).
        if (!__hip_atomic_load(p.err + LP_E_STICKY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            // this workgroup's XCD and the next free slot in it
            unsigned xcc;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 16)" : "=s"(xcc));
            int slot = LP_WPX;
            if (xcc < (unsigned)LP_NX)
                slot = __hip_atomic_fetch_add(p.err + 8 + xcc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            role = slot < LP_WPX ? slot * LP_NX + (int)xcc : -1;
            if (role < 0) lp_fail(p, LP_ERR_XCD, 100 + (int)xcc);
            // Co-residency: every wait below assumes all LP_NBLK workgroups
            // run at once. Other work holding CUs would leave some waiting
            // for them, so each workgroup counts in and waits (briefly) for
            // the rest before it writes anything; if they do not come, the
            // launch is marked and computes nothing.
            __hip_atomic_fetch_add(p.err + LP_E_ARRIVED, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            while (role >= 0) {
                const int n = __hip_atomic_load(p.err + LP_E_ARRIVED, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
                if (__hip_atomic_load(p.err + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    role = -1;
                } else if (n >= LP_NBLK && p.arrive_ticks > 0) {
                    break;
                } else if (__builtin_amdgcn_s_memrealtime() - t0 > p.arrive_ticks) {
                    if (atomicCAS(p.err + LP_E_STICKY, 0, 1) == 0) atomicExch(p.err + LP_E_STICKY_POS, p.pos0);
                    lp_fail(p, LP_ERR_RESIDENT, n);
                    role = -1;
                } else {
                    __builtin_amdgcn_s_sleep(2);
                }
            }
        }
    }
    __syncthreads();
    if (role < 0) return;   // every wave of the workgroup leaves together
    Cx c;
    c.lane = threadIdx.x & 63;
    c.w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
    c.role = __builtin_amdgcn_readfirstlane(role);
    c.g = c.role % LP_NX;
    c.j = c.role / LP_NX;
    {
        const int V = p.V;
        c.uv0 = (int)(((uint32_t)c.role * (uint32_t)V) / (uint32_t)LP_NBLK);
        c.nuv = (int)(((uint32_t)(c.role + 1) * (uint32_t)V) / (uint32_t)LP_NBLK) - c.uv0;
    }
    c.nsync = 0;
    c.fail_where = 0;
    c.wt0 = 0;
    c.tt = c.tl = 0;
    c.ready = ready;
    c.done = done;
    c.csync = &sync_ctr;
    c.abort = &abort_flag;
    c.ring = lp_lds;
    c.xw = (float*)(lp_lds + LP_LDS_RING);
    c.os = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XW);
    c.acts = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XW + LP_LDS_OS);
    c.attp = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XW + LP_LDS_OS + LP_LDS_ACT);
    c.attm = c.attp + LP_CW * LP_G * LP_D;
    c.stg = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XW + LP_LDS_OS + LP_LDS_ACT + LP_LDS_ATT);
    c.cst = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XW + LP_LDS_OS + LP_LDS_ACT + LP_LDS_ATT + LP_LDS_STG);
    c.xs = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XW + LP_LDS_OS + LP_LDS_ACT + LP_LDS_ATT + LP_LDS_STG + LP_LDS_CST);
    c.wkeys = wkeys;
    if (c.w >= LP_CW) {
        stream_role(p, c);
    } else {
        compute_role<KT, TR>(p, c);
        // a compute wave that leaves early must not hold the ring
        cbar();
        if (c.lane == 0) lds_st(&done[c.w], 0x7fffffff);
    }
    if (c.fail_where && c.lane == 0) lp_fail(p, LP_ERR_TIMEOUT, c.fail_where);
}

// ------------------------------------------------------------------ host
struct LoopState {
    int nblk = 0;
    int lpt = 0;
    void* stream = nullptr;      // relaid weights
    void* tab = nullptr;         // source address of every 128-byte piece of them (the caller's weights)
    int64_t nlines = 0;
    void* small = nullptr;       // tagged buffers + layer table + error words
    size_t small_bytes = 0, ll_bytes = 0;
    LoopLayer* layers = nullptr;
    u64 *xr, *xr2, *qkv, *att, *act, *opart, *dpart, *keys;
    int* err = nullptr;
    uint32_t epoch = 1;
    bool ran = false;
    int replays = 0;    // launches re-run in graph mode (grid not co-resident)
    int trace_t0 = -1;  // the next launch is traced from this step (-1: not traced)
    u64* trace = nullptr;
};

// The kernel's dynamic LDS exceeds the 64 KB default limit.
static int loop_lds_attr() {
    const void* k[] = {(const void*)decode_loop_kernel<float, false>, (const void*)decode_loop_kernel<_Float16, false>,
                       (const void*)decode_loop_kernel<float, true>, (const void*)decode_loop_kernel<_Float16, true>};
    for (const void* f : k)
        PIO_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LP_LDS_BYTES));
    return PIO_OK;
}

int loop_check(const Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    int dev = 0, cus = 0, per_cu = 0;
    PIO_HIP(hipGetDevice(&dev));
    PIO_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    PIO_TRY(loop_lds_attr());
    if (d->kv16)
        PIO_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_loop_kernel<_Float16, false>,
                                                             LP_THREADS, LP_LDS_BYTES));
    else
        PIO_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_loop_kernel<float, false>,
                                                             LP_THREADS, LP_LDS_BYTES));
    const bool ok = c.head_dim == LP_D && c.hidden == LP_H && c.n_heads * LP_D == LP_KO &&
                    c.n_kv_heads == LP_NX && c.intermediate == LP_I && cus == LP_NBLK &&
                    c.max_seq <= LP_MAX_SEQ && c.vocab <= (1 << 18) && c.n_layers <= LP_LMAX &&
                    per_cu >= 1;
    if (!ok)
        return set_error(PIO_ERR_UNSUPPORTED,
                         "persistent decode is built for the Qwen3-0.6B layer shape on a %d-CU, "
                         "%d-XCD device: head_dim %d, hidden %d, %d query / %d KV heads, "
                         "intermediate %d, max_seq <= %d, vocab <= 262144, layers <= %d (device has %d CUs)",
                         LP_NBLK, LP_NX, LP_D, LP_H, LP_KO / LP_D, LP_NX, LP_I, LP_MAX_SEQ, LP_LMAX, cus);
    return PIO_OK;
}

// One 1 KB line per 64 threads from 8 sources of 128 B each (chunk k of the
// line = lanes 8k .. 8k+7).
__global__ void loop_gather_kernel(const int8_t* const* __restrict__ src, int8_t* __restrict__ dst,
                                   int64_t nlines) {
    const int64_t line = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (line >= nlines) return;
    const int lane = threadIdx.x & 63;
    const lp_v4i v = *(const lp_v4i*)(src[line * 8 + (lane >> 3)] + (lane & 7) * 16);
    const int64_t lpt = nlines / LP_NBLK;                    // table: [nblk][lpt] lines
    const int64_t dl = (line % lpt) * LP_NBLK + line / lpt;  // copy: [lpt][nblk]
    *(lp_v4i*)(dst + dl * 1024 + lane * 16) = v;
}

// Lays out every workgroup's weight lines in the order its compute waves
// consume them (the partition of the kernel above), line-major: line L of all
// workgroups sits together, so the lines in flight across the grid at one
// moment form one contiguous region (0.4% faster than one contiguous block
// per workgroup, whose equal 1.7 MB strides share their low address bits).
static int loop_build(Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    LoopState* s = new LoopState();
    d->loop = s;
    s->nblk = LP_NBLK;
    s->lpt = c.n_layers * LP_LPL;
    const int64_t nlines = (int64_t)LP_NBLK * s->lpt;
    std::vector<const int8_t*> tab((size_t)nlines * 8);
    for (int b = 0; b < LP_NBLK; b++) {
        const int g = b % LP_NX, j = b / LP_NX;
        for (int l = 0; l < c.n_layers; l++) {
            const pio_qwen3_layer& L = d->layers[l];
            const int64_t lb = ((int64_t)b * s->lpt + (int64_t)l * LP_LPL) * 8;
            auto row_line = [&](int64_t line, const int8_t* row) {   // a whole 1 KB row
                for (int k = 0; k < 8; k++) tab[lb + line * 8 + k] = row + 128 * k;
            };
            // qkv: unit ub = w + 4m of this workgroup's 8 -> lines 2 ub (+1 for row + 64)
            for (int ub = 0; ub < 8; ub++) {
                const int u = 8 * j + ub;
                int r0;
                if (u < 128) r0 = (LP_G * g + (u >> 6)) * LP_D + (u & 63);
                else if (u < 192) r0 = LP_KO + g * LP_D + (u - 128);
                else r0 = LP_KO + LP_NX * LP_D + g * LP_D + (u - 192);
                row_line(2 * ub, L.w_qkv + (int64_t)r0 * LP_H);
                row_line(2 * ub + 1, L.w_qkv + (int64_t)(r0 + 64) * LP_H);
            }
            // o_proj partial: line c holds rows 32 j + 4 c + r (r < 4), columns 256 g .. +256
            for (int cc = 0; cc < LP_L_O; cc++)
                for (int k = 0; k < 8; k++) {
                    const int row = 32 * j + 4 * cc + (k >> 1);
                    tab[lb + (LP_OFF_O + cc) * 8 + k] =
                        L.w_o + (int64_t)row * LP_KO + 256 * g + 128 * (k & 1);
                }
            // gate_up: unit ub -> channel i = 384 g + 12 j + ub; lines gate row i, up row i + I
            for (int ub = 0; ub < 12; ub++) {
                const int i = LP_IX * g + 12 * j + ub;
                row_line(LP_OFF_GU + 2 * ub, L.w_gu + (int64_t)i * LP_H);
                row_line(LP_OFF_GU + 2 * ub + 1, L.w_gu + (int64_t)(i + LP_I) * LP_H);
            }
            // down partial: wave w, line 3 w + cc, chunk k = row 32 j + 8 w + k,
            // channels 384 g + 128 cc .. +128
            for (int w = 0; w < LP_CW; w++)
                for (int cc = 0; cc < 3; cc++)
                    for (int k = 0; k < 8; k++) {
                        const int row = 32 * j + 8 * w + k;
                        tab[lb + (LP_OFF_DN + 3 * w + cc) * 8 + k] =
                            L.w_down + (int64_t)row * LP_I + LP_IX * g + 128 * cc;
                    }
        }
    }
    PIO_TRY(device_alloc(&s->stream, (size_t)nlines * 1024, d->st));
    // the table stays (nlines * 64 B): pio_qwen3_refresh_weights gathers again from it
    PIO_TRY(device_alloc(&s->tab, tab.size() * sizeof(void*), d->st));
    s->nlines = nlines;
    PIO_HIP(hipMemcpyAsync(s->tab, tab.data(), tab.size() * sizeof(void*), hipMemcpyHostToDevice, d->st));
    loop_gather_kernel<<<(unsigned)((nlines + 3) / 4), 256, 0, d->st>>>((const int8_t* const*)s->tab,
                                                                        (int8_t*)s->stream, nlines);
    PIO_LAUNCHED();

    // tagged buffers, layer table, error words
    const size_t n_ll[] = {(size_t)LP_NX * LP_H, (size_t)LP_NX * LP_H, (size_t)LP_NX * LP_QKVX,
                           (size_t)LP_NX * LP_S * LP_G * LP_PART, (size_t)LP_NX * LP_IX,
                           (size_t)LP_NX * LP_H, (size_t)LP_NX * LP_H, (size_t)LP_NBLK};
    constexpr int NB = 8;
    size_t off[NB + 1];
    off[0] = 0;
    for (int i = 0; i < NB; i++) off[i + 1] = off[i] + (n_ll[i] * 8 + 255) / 256 * 256;
    s->ll_bytes = off[NB];
    const size_t lay_off = s->ll_bytes;
    const size_t err_off = lay_off + (c.n_layers * sizeof(LoopLayer) + 255) / 256 * 256;
    s->small_bytes = err_off + 256;
    PIO_TRY(device_alloc(&s->small, s->small_bytes, d->st));
    char* sp = (char*)s->small;
    u64** dst[] = {&s->xr, &s->xr2, &s->qkv, &s->att, &s->act, &s->opart, &s->dpart, &s->keys};
    for (int i = 0; i < NB; i++) *dst[i] = (u64*)(sp + off[i]);
    s->layers = (LoopLayer*)(sp + lay_off);
    s->err = (int*)(sp + err_off);
    std::vector<LoopLayer> lt(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        const pio_qwen3_layer& L = d->layers[l];
        lt[l] = LoopLayer{L.in_norm, L.s_qkv, L.b_qkv, L.s_o, L.post_norm, L.s_gu, L.s_down};
    }
    PIO_HIP(hipMemsetAsync(s->small, 0, s->small_bytes, d->st));
    PIO_HIP(hipMemcpyAsync(s->layers, lt.data(), lt.size() * sizeof(LoopLayer), hipMemcpyHostToDevice,
                           d->st));
    PIO_HIP(hipStreamSynchronize(d->st));   // the host tables go out of scope
    s->epoch = 1;
    return PIO_OK;
}

// Copies the caller's int8 layer weights into the relaid copy again (after the
// caller changed them in place), ordered on the decoder's stream.
int loop_refresh(Qwen3Dec* d) {
    LoopState* s = d->loop;
    if (!s) return PIO_OK;   // no copy yet: the first persistent run makes it
    loop_gather_kernel<<<(unsigned)((s->nlines + 3) / 4), 256, 0, d->st>>>((const int8_t* const*)s->tab,
                                                                           (int8_t*)s->stream, s->nlines);
    PIO_LAUNCHED();
    return PIO_OK;
}

void loop_destroy(Qwen3Dec* d) {
    if (!d || !d->loop) return;
    if (d->loop->stream) device_free(d->loop->stream);
    if (d->loop->tab) device_free(d->loop->tab);
    if (d->loop->small) device_free(d->loop->small);
    if (d->loop->trace) device_free(d->loop->trace);
    delete d->loop;
    d->loop = nullptr;
}

int loop_run(Qwen3Dec* d, int n_steps) {
    if (n_steps <= 0) return PIO_OK;
    PIO_TRY(loop_check(d));
    if (!d->loop) {
        const int rc = loop_build(d);
        if (rc != PIO_OK) {
            loop_destroy(d);
            return rc;
        }
    }
    LoopState* s = d->loop;
    const pio_qwen3_config& c = d->c;
    const uint32_t per_tok = (uint32_t)(c.n_layers * LP_PH + 2);
    if ((uint64_t)s->epoch + (uint64_t)n_steps * per_tok + 1 >= 0xFFFFFFFFull) {
        // tags would wrap: clear every tagged word and start over
        PIO_HIP(hipMemsetAsync(s->small, 0, s->ll_bytes, d->st));
        s->epoch = 1;
    }
    // abort flag, arrival and XCD slot counters; the error code and site stay
    // until loop_status reads them, so the first error since then is reported
    PIO_HIP(hipMemsetAsync(s->err + 2, 0, 14 * sizeof(int), d->st));
    LoopParams p{};
    p.L = c.n_layers; p.V = c.vocab; p.max_seq = c.max_seq;
    p.eps = c.rms_eps;
    p.att_scale = 1.0f / sqrtf((float)c.head_dim);
    p.embed = d->embed; p.final_norm = d->final_norm; p.s_lm = d->s_lm;
    p.layers = s->layers;
    p.stream = (const int8_t*)s->stream;
    p.lpt = s->lpt;
    p.lm_head = d->lm_head;
    p.kc = d->kc; p.vc = d->vc; p.cos_t = d->cos_t; p.sin_t = d->sin_t;
    p.xr = s->xr; p.xr2 = s->xr2; p.qkv = s->qkv; p.att = s->att; p.act = s->act;
    p.opart = s->opart; p.dpart = s->dpart; p.keys = s->keys;
    p.ids = d->ids; p.logits = d->logits; p.state = d->state;
    p.pos0 = d->host_pos;
    p.prompt_len = d->prompt_len;
    p.n_steps = n_steps;
    p.epoch0 = s->epoch;
    // PIO_LOOP_ARRIVE_TICKS overrides the co-residency wait (ticks of 10 ns);
    // 0 makes every launch act as if the grid never became resident, which is
    // how the tests reach the graph-mode re-run
    p.arrive_ticks = LP_ARRIVE_TICKS;
    if (const char* e = getenv("PIO_LOOP_ARRIVE_TICKS")) p.arrive_ticks = strtoull(e, nullptr, 10);
    p.err = s->err;
    PIO_TRY(loop_lds_attr());
    const dim3 grid(LP_NBLK), block(LP_THREADS);
    if (s->trace_t0 >= 0) {
        // one traced launch: the phase stamps of steps trace_t0 .. + LP_TR_TOK
        const size_t tb = loop_trace_bytes(d);
        if (!s->trace) PIO_TRY(device_alloc((void**)&s->trace, tb, d->st));
        PIO_HIP(hipMemsetAsync(s->trace, 0, tb, d->st));
        p.trace = s->trace;
        p.tr_t0 = s->trace_t0;
        s->trace_t0 = -1;
        if (d->kv16) decode_loop_kernel<_Float16, true><<<grid, block, LP_LDS_BYTES, d->st>>>(p);
        else decode_loop_kernel<float, true><<<grid, block, LP_LDS_BYTES, d->st>>>(p);
    } else {
        if (d->kv16) decode_loop_kernel<_Float16, false><<<grid, block, LP_LDS_BYTES, d->st>>>(p);
        else decode_loop_kernel<float, false><<<grid, block, LP_LDS_BYTES, d->st>>>(p);
    }
    PIO_LAUNCHED();
    s->epoch += (uint32_t)n_steps * per_tok;
    s->ran = true;
    return PIO_OK;
}

bool loop_pending(const Qwen3Dec* d) { return d->loop && d->loop->ran; }

size_t loop_trace_bytes(const Qwen3Dec* d) {
    return (size_t)LP_TR_TOK * LP_NBLK * (d->c.n_layers + 1) * LP_TR_K * sizeof(u64);
}
int loop_trace_next(Qwen3Dec* d, int first_step) {
    PIO_TRY(loop_check(d));
    if (!d->loop) {
        const int rc = loop_build(d);
        if (rc != PIO_OK) {
            loop_destroy(d);
            return rc;
        }
    }
    d->loop->trace_t0 = first_step;
    return PIO_OK;
}
int loop_trace_read(Qwen3Dec* d, void* out, size_t bytes) {
    PIO_REQUIRE(d->loop && d->loop->trace, "pio_qwen3_trace_read: no traced launch has run");
    PIO_REQUIRE(bytes == loop_trace_bytes(d), "pio_qwen3_trace_read: %zu bytes, the trace has %zu", bytes,
                loop_trace_bytes(d));
    PIO_HIP(hipStreamSynchronize(d->st));
    PIO_HIP(hipMemcpy(out, d->loop->trace, bytes, hipMemcpyDeviceToHost));
    return PIO_OK;
}
int loop_replays(const Qwen3Dec* d) { return d->loop ? d->loop->replays : 0; }

// Error words of the persistent launches since the last call (after the
// stream has drained). A launch that found the grid not co-resident, and every
// launch after it, computed nothing: returns LOOP_REPLAY with *replay_pos = the
// first position whose step has to be run again; the words are cleared.
int loop_status(Qwen3Dec* d, int* replay_pos) {
    if (!d->loop || !d->loop->ran) return PIO_OK;
    int e[18] = {};
    PIO_HIP(hipMemcpy(e, d->loop->err, sizeof(e), hipMemcpyDeviceToHost));
    d->loop->ran = false;
    const int zero[2] = {0, 0};
    PIO_HIP(hipMemcpy(d->loop->err, zero, sizeof(zero), hipMemcpyHostToDevice));
    if (e[LP_E_STICKY]) {
        PIO_HIP(hipMemcpy(d->loop->err + LP_E_STICKY, zero, sizeof(zero), hipMemcpyHostToDevice));
        d->loop->replays++;
        *replay_pos = e[LP_E_STICKY_POS];
        return LOOP_REPLAY;
    }
    if (e[0] == LP_ERR_XCD)
        return set_error(PIO_ERR_HIP, "persistent decode: more than %d workgroups on XCD %d (or no "
                                      "such XCD); results of that run are invalid",
                         LP_WPX, e[1] - 100);
    if (e[0])
        return set_error(PIO_ERR_HIP, "persistent decode: a wait timed out (site %d); results of "
                                      "that run are invalid", e[1]);
    return PIO_OK;
}

}  // namespace pio
