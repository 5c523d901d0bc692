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
// Co-residency. The grid has exactly as many workgroups as the device has
// CUs, and each workgroup takes 131 KB of a CU's 160 KB of LDS, so on an idle
// device all of them are resident at once. The kernel needs no grid barrier,
// only that residency, so it is launched as an ordinary kernel: a cooperative
// launch would claim the device's global wave-sync resource, which only one
// process at a time can hold (a second process's cooperative launch fails).
// If other work holds some CUs, the workgroups waiting for them start when it
// drains; every wait below is bounded, so the kernel ends in any case.
//
// Workgroup = 8 waves:
//   waves 4-7 ("stream waves") copy this workgroup's weight lines, in the order
//     the compute waves consume them, from a per-workgroup contiguous copy of
//     the weights (built once) into an LDS ring of 1 KB lines with
//     global_load_lds_dwordx4; a line is published when its copy has landed.
//   waves 0-3 ("compute waves") run the phases of every token:
//       qkv -> attention -> merge -> o_proj -> gate_up -> down   (per layer)
//       -> lm_head + argmax
//     reading x from LDS, weights from the ring, and writing outputs.
//
// Cross-workgroup hand-off uses tagged 64-bit words: every value a phase
// produces for other workgroups is stored as {tag:32 | fp32 bits:32} with a
// device-scope (L2-bypassing) store; a consumer polls the words it needs with
// device-scope loads until every tag equals the producing phase's tag. Tags
// grow monotonically over the decoder's lifetime, so no buffer is ever reset
// and no barrier is needed: one memory round trip per hand-off. A buffer is
// rewritten only one layer later, by which time every consumer has read it
// (each phase needs all of the previous phase's outputs, so no workgroup can
// be two phases ahead of any other's reads).
//
// The KV cache rows are written with device-scope stores; rows are read only
// after the token that wrote them (the current row is read from the tagged
// copy), so ordinary cached loads never see a stale line.
//
// Every wait is bounded: a wait that exceeds its limit records an error
// (read back by pio_qwen3_read) and makes every wave leave its loops, so the
// kernel always terminates.
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
constexpr int LP_S = ATT_SPLITS;           // attention splits over positions
constexpr int LP_NPF = 2;                  // attention passes whose K/V are prefetched
constexpr int LP_NPMAX = 8;                // attention passes (8 positions each) per wave
constexpr int LP_CMAX = 3;                 // K <= 3 * 1024
// The layer shape the kernel is instantiated for, in 1 KB weight lines per
// row: hidden (qkv, gate_up, lm_head rows), n_heads*head_dim (o_proj rows),
// intermediate (down rows). Qwen3-0.6B: 1024, 2048, 3072.
constexpr int LP_CH = 1, LP_CO = 2, LP_CI = 3;
constexpr int LP_G = 2;                    // query heads per KV head the kernel is built for
// Units per wave and phase the kernel is unrolled for (Qwen3-0.6B on 256 CUs:
// qkv 2048 pairs, gate_up 3072 pairs, o_proj/down 1024 rows over 1024 waves).
constexpr int LP_MU_QKV = 2, LP_MU_GU = 3, LP_MU_ROW = 1;
constexpr int LP_LM_B = 6;                 // lm_head rows per wave and batch (double-buffered)
constexpr int LP_PH = 6;                   // tagged phases per layer
constexpr int LP_MAX_SEQ = LP_S * LP_CW * 8 * LP_NPMAX;   // 2048
constexpr int LP_PART = 2 + 128;           // (max, sum, o[128]) per split and head
constexpr uint32_t LP_POLL_LIMIT = 1u << 21;   // device-scope polls (~0.5-1 us each)
constexpr uint32_t LP_LDS_LIMIT = 1u << 24;    // LDS polls

enum { PH_QKV = 0, PH_ATT = 1, PH_MERGE = 2, PH_O = 3, PH_GU = 4, PH_DN = 5 };
enum { LP_ERR_TIMEOUT = 1 };

struct LoopLayer {
    const float *in_norm, *s_qkv, *b_qkv, *s_o, *post_norm, *s_gu, *s_down;
};

struct LoopParams {
    int L, H, nq, nkv, I, V, max_seq, nblk;
    float eps, att_scale;
    const float* embed;
    const float* final_norm;
    const float* s_lm;
    const int8_t* lm_head;     // [V][H] int8, read directly by the lm phase
    const LoopLayer* layers;
    const int8_t* stream;      // [nblk][lpt][1024] weight lines in consumption order
    int lpl;                   // lines per layer (per workgroup)
    int off_o, off_gu, off_dn; // phase offsets inside a layer
    int lpt;                   // weight lines per token (n_layers * lpl)
    float* kc;
    float* vc;
    const float* cos_t;
    const float* sin_t;
    u64 *xa, *xb, *q, *kv, *part, *merged, *act, *keys;
    int32_t* ids;
    float* logits;
    int32_t* state;
    int pos0, prompt_len, n_steps;
    uint32_t epoch0;
    int* err;                  // [0] code, [1] where, [2] abort flag
};

// LDS layout (dynamic): ring | xs[2][3072] | att partials | per-wave staging
constexpr int LP_XS = LP_CMAX * 1024;
constexpr size_t LP_LDS_RING = (size_t)LP_RING * 1024;
constexpr size_t LP_LDS_XS = 2 * LP_XS * 4;
// attention partials: [wave][head][lane group][128] + per (wave, head) max and sum
constexpr size_t LP_LDS_ATT = (size_t)LP_CW * LP_G * 8 * 128 * 4 + 2 * LP_CW * LP_G * 4;
constexpr size_t LP_STG = LP_G * 128 + 256;   // floats per wave: q heads + current k,v
constexpr size_t LP_LDS_STG = (size_t)LP_CW * LP_STG * 4;
constexpr size_t LP_LDS_BYTES = LP_LDS_RING + LP_LDS_XS + LP_LDS_ATT + LP_LDS_STG;

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
    return p.epoch0 + (uint32_t)t * (uint32_t)(p.L * LP_PH + 1) + (uint32_t)(l * LP_PH + ph);
}

struct Units;
struct Cx {
    int lane, w, nsync, fail_where;
    int uq0, nuq, uh0, nuh, ui0, nui, uv0, nuv;   // unit ranges: qkv pairs, H rows, I pairs, V rows
    int* ready;      // [LP_SW] lines landed per stream wave
    int* done;       // [LP_CW] first line each compute wave may still need
    int* csync;      // compute-wave rendezvous counter
    int* abort;      // workgroup abort flag
    int8_t* ring;
    float* xs;       // [2][LP_XS]
    float* ss;       // [2][LP_CW] partial sums of squares
    float* attp;     // [LP_CW][LP_G][8][128] attention partials
    float* attm;     // [2][LP_CW][LP_G] wave max, wave sum
    float* stg;      // [LP_CW][LP_STG]
    u64* wkeys;      // [LP_CW]
};

// Records a timed-out wait (site `where`) and tells every workgroup to stop.
__device__ void lp_fail(const LoopParams& p, int where) {
    if (atomicCAS(&p.err[0], 0, LP_ERR_TIMEOUT) == 0) atomicExch(&p.err[1], where);
    __hip_atomic_store(&p.err[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One more iteration of a bounded wait? Also leaves when another wave or
// workgroup gave up. A wave that runs out of patience only notes where (and
// raises the workgroup's abort flag); its role function reports the error
// once, on the way out -- the kernel has to fit the instruction cache, so no
// calls or long paths sit inside the wait loops.
__device__ __forceinline__ bool keep_waiting(const LoopParams& p, Cx& c, uint32_t it, uint32_t limit,
                                             int where) {
    if (lds_ld_u(c.abort)) return false;
    if ((it & 63) != 63) return true;
    if (__hip_atomic_load(&p.err[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || it > limit) {
        if (it > limit) c.fail_where = where;
        lds_st(c.abort, 1);
        return false;
    }
    return true;
}

// Polls n tagged words per lane (src[lane + 64 i], i < n) until every tag
// matches; returns their values.
template <int NMAX>
__device__ __forceinline__ bool ll_poll(const LoopParams& p, Cx& c, const u64* src, int n,
                                        uint32_t tag, float (&out)[NMAX], int where) {
    for (uint32_t it = 0;; it++) {
        u64 v[NMAX];
#pragma unroll
        for (int i = 0; i < NMAX; i++) v[i] = i < n ? ll_load(src + c.lane + 64 * i) : ((u64)tag << 32);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < NMAX; i++) ok &= (uint32_t)(v[i] >> 32) == tag;
        if (__all(ok)) {
#pragma unroll
            for (int i = 0; i < NMAX; i++) out[i] = __uint_as_float((uint32_t)v[i]);
            return true;
        }
        if (!keep_waiting(p, c, it, LP_POLL_LIMIT, where)) return false;
    }
}

// One tagged word (same address in every lane).
__device__ __forceinline__ bool ll_poll1(const LoopParams& p, Cx& c, const u64* src, uint32_t tag,
                                         float& out, int where) {
    for (uint32_t it = 0;; it++) {
        const u64 v = ll_load(src);
        if ((uint32_t)(v >> 32) == tag) {
            out = __uint_as_float((uint32_t)v);
            return true;
        }
        if (!keep_waiting(p, c, it, LP_POLL_LIMIT, where)) return false;
    }
}

// Rendezvous of the four compute waves of this workgroup.
__device__ __forceinline__ bool csync(const LoopParams& p, Cx& c, int where) {
    c.nsync++;
    cbar();
    if (c.lane == 0) __hip_atomic_fetch_add(c.csync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int target = LP_CW * c.nsync;
    for (uint32_t it = 0; lds_ld_u(c.csync) < target; it++) {
        if (!keep_waiting(p, c, it, LP_LDS_LIMIT, where)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    cbar();
    return true;
}

// Waits until every ring line up to `last` has landed (stream wave r copies
// lines r, r+4, ... in order and counts them in ready[r]).
__device__ __forceinline__ bool wait_upto(const LoopParams& p, Cx& c, int last, int where) {
    for (uint32_t it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < LP_SW; r++) ok &= last < r || lds_ld_u(&c.ready[r]) >= ((last - r) >> 2) + 1;
        if (ok) break;
        if (!keep_waiting(p, c, it, LP_LDS_LIMIT, where)) return false;
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

// Stage one quarter of a K-vector (this wave's values v[i] = x[w*K/4 + lane + 64 i])
// into LDS buffer `buf`, times gamma if given, with this wave's partial sum of
// squares; after the rendezvous load the whole vector into the lane layout
// xr[c][j] = x[c*1024 + 16 lane + j] and return the RMSNorm scale (1 without gamma).
template <int NMAX, int C>
__device__ __forceinline__ bool stage_x(const LoopParams& p, Cx& c, int buf, int K,
                                        const float (&v)[NMAX], const float (&g)[NMAX], bool norm,
                                        float (&xr)[LP_CMAX][16], float& nscale, int where) {
    const int n = K / 256;
    float* xs = c.xs + buf * LP_XS;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NMAX; i++) {
        if (i >= n) continue;
        const int e = c.w * (K / 4) + c.lane + 64 * i;
        s += v[i] * v[i];
        xs[e] = norm ? v[i] * g[i] : v[i];
    }
    if (norm) {
        s = wsum(s);
        if (c.lane == 0) c.ss[buf * LP_CW + c.w] = s;
    }
    if (!csync(p, c, where)) return false;
#pragma unroll
    for (int ch = 0; ch < C; ch++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 a = *(const float4*)&xs[ch * 1024 + c.lane * 16 + 4 * i];
            xr[ch][4 * i] = a.x; xr[ch][4 * i + 1] = a.y; xr[ch][4 * i + 2] = a.z; xr[ch][4 * i + 3] = a.w;
        }
    }
    nscale = 1.f;
    if (norm) {
        const float* ss = c.ss + buf * LP_CW;
        nscale = rsqrtf((ss[0] + ss[1] + ss[2] + ss[3]) * (1.0f / (float)K) + p.eps);
    }
    return true;
}

// Units of a phase owned by this workgroup: [u0, u0 + nu), u0 = b*U/nblk.
// Computed once per kernel (a division is a long instruction sequence).
struct Units {
    int u0, nu;
};
__device__ __forceinline__ Units blk_units(int U, int nblk) {
    const uint32_t b = blockIdx.x;
    const int u0 = (int)((b * (uint32_t)U) / (uint32_t)nblk);
    return Units{u0, (int)(((b + 1) * (uint32_t)U) / (uint32_t)nblk) - u0};
}

// Dot products of this wave's units of a phase: units ub = w + 4m (m < MU,
// ub < nu), each R rows of C 1 KB lines at ring lines line0 + ub*R*C + r*C + ch.
// One wait covers all of them; every ring read is issued before the first dot
// product, and the reductions are independent chains.
template <int C, int R, int MU>
__device__ __forceinline__ bool phase_dots(const LoopParams& p, Cx& c, int line0, int nu,
                                           const float (&xr)[LP_CMAX][16], float (&acc)[MU][R],
                                           int& nmy, int where) {
    const int lpu = R * C;
    nmy = nu > c.w ? min(MU, (nu - c.w + LP_CW - 1) / LP_CW) : 0;
    if (nmy == 0) return true;
    if (!wait_upto(p, c, line0 + (c.w + LP_CW * (nmy - 1)) * lpu + lpu - 1, where)) return false;
    // Every MU unit is computed (a unit past nmy reads a stale ring line, and
    // its result is never used): straight-line code, no per-unit branches.
    lp_v4i wv[MU][R][C];
#pragma unroll
    for (int m = 0; m < MU; m++)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int ch = 0; ch < C; ch++)
                wv[m][r][ch] = ring_line(c, line0 + (c.w + LP_CW * m) * lpu + r * C + ch);
#pragma unroll
    for (int m = 0; m < MU; m++) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ch = 0; ch < C; ch++) lp_dot16s(xr[ch], wv[m][r][ch], s);
            acc[m][r] = (s[0] + s[1]) + (s[2] + s[3]);
        }
    }
    wsum_n<MU * R>(&acc[0][0]);
    return true;
}

// ------------------------------------------------------------ phase bodies
// Per-unit constants of a phase are loaded one per lane before the phase
// waits for its input (lane k holds the value of this wave's unit k, or of
// row k&1 of unit k>>1 for paired units) and read back with readlane.
struct Pre {
    float a = 0.f, b = 0.f, cs = 0.f, sn = 0.f;
    u64 r = 0;
};

// qkv: pairs (n, n + 64) of one head; bias + rotate-half RoPE at pos;
// q -> tagged q, k/v -> tagged current row + cache row pos.
__device__ __forceinline__ Pre pre_qkv(const LoopParams& p, const Cx& c, int l, int pos) {
    const LoopLayer& Lw = p.layers[l];
    const int u0 = c.uq0, nu = c.nuq;
    Pre q;
    const int ub = c.w + LP_CW * (c.lane >> 1);
    if (ub < nu) {
        const int u = u0 + ub, row = (u >> 6) * 128 + (u & 63) + (c.lane & 1) * 64;
        q.a = gld(Lw.s_qkv + row);
        q.b = Lw.b_qkv ? gld(Lw.b_qkv + row) : 0.f;
    }
    const int ubc = c.w + LP_CW * c.lane;
    if (ubc < nu) {
        const int i = (u0 + ubc) & 63;
        q.cs = gld(p.cos_t + (int64_t)pos * 64 + i);
        q.sn = gld(p.sin_t + (int64_t)pos * 64 + i);
    }
    return q;
}

template <int C>
__device__ bool phase_qkv(const LoopParams& p, Cx& c, int l, int pos, int line0, uint32_t tag,
                          const float (&xr)[LP_CMAX][16], float nscale, const Pre& pre) {
    int nmy;
    const int u0 = c.uq0, nu = c.nuq;
    float acc[LP_MU_QKV][2];
    if (!phase_dots<C, 2, LP_MU_QKV>(p, c, line0, nu, xr, acc, nmy, 10)) return false;
#pragma unroll
    for (int m = 0; m < LP_MU_QKV; m++) {
        if (m >= nmy) break;
        const int u = u0 + c.w + LP_CW * m, hd = u >> 6, i = u & 63;
        const float v0 = acc[m][0] * rlane(pre.a, 2 * m) * nscale + rlane(pre.b, 2 * m);
        const float v1 = acc[m][1] * rlane(pre.a, 2 * m + 1) * nscale + rlane(pre.b, 2 * m + 1);
        const float cs = rlane(pre.cs, m), sn = rlane(pre.sn, m);
        if (c.lane != 0) continue;
        if (hd < p.nq + p.nkv) {
            const float o0 = v0 * cs - v1 * sn, o1 = v0 * sn + v1 * cs;
            if (hd < p.nq) {
                ll_store(p.q + hd * 128 + i, o0, tag);
                ll_store(p.q + hd * 128 + i + 64, o1, tag);
            } else {
                const int kvh = hd - p.nq;
                float* kr = p.kc + (((int64_t)l * p.nkv + kvh) * p.max_seq + pos) * 128;
                dev_store(kr + i, o0);
                dev_store(kr + i + 64, o1);
                ll_store(p.kv + kvh * 256 + i, o0, tag);
                ll_store(p.kv + kvh * 256 + i + 64, o1, tag);
            }
        } else {
            const int kvh = hd - p.nq - p.nkv;
            float* vr = p.vc + (((int64_t)l * p.nkv + kvh) * p.max_seq + pos) * 128;
            dev_store(vr + i, v0);
            dev_store(vr + i + 64, v1);
            ll_store(p.kv + kvh * 256 + 128 + i, v0, tag);
            ll_store(p.kv + kvh * 256 + 128 + i + 64, v1, tag);
        }
    }
    return true;
}

// Residual row phase: y[n] = res[n] + s[n] * (W x)[n] for this wave's rows.
// res comes from the tagged vector `rin` (tag rtag) or, when rin is null, from
// the embedding row emb.
__device__ __forceinline__ Pre pre_resid(const LoopParams& p, const Cx& c, const float* s_w,
                                         const u64* rin) {
    const int u0 = c.uh0, nu = c.nuh;
    Pre q;
    const int ub = c.w + LP_CW * c.lane;
    if (ub < nu) {
        q.a = gld(s_w + u0 + ub);
        if (rin) q.r = ll_load(rin + u0 + ub);
    }
    return q;
}

template <int C>
__device__ bool phase_resid(const LoopParams& p, Cx& c, int line0, const u64* rin, uint32_t rtag,
                            const float* emb, u64* out, uint32_t tag,
                            const float (&xr)[LP_CMAX][16], const Pre& pre, int where) {
    int nmy;
    const int u0 = c.uh0, nu = c.nuh;
    float acc[LP_MU_ROW][1];
    if (!phase_dots<C, 1, LP_MU_ROW>(p, c, line0, nu, xr, acc, nmy, where)) return false;
#pragma unroll
    for (int m = 0; m < LP_MU_ROW; m++) {
        if (m >= nmy) break;
        const int n = u0 + c.w + LP_CW * m;
        float res;
        if (rin) {
            const uint32_t rt = (uint32_t)__builtin_amdgcn_readlane((int)(pre.r >> 32), m);
            res = __int_as_float(__builtin_amdgcn_readlane((int)(uint32_t)pre.r, m));
            if (rt != rtag && !ll_poll1(p, c, rin + n, rtag, res, where + 1)) return false;
        } else {
            res = gld(emb + n);
        }
        const float v = res + acc[m][0] * rlane(pre.a, m);
        if (c.lane == 0) ll_store(out + n, v, tag);
    }
    return true;
}

// gate_up: pairs (i, i + I) -> act[i] = silu(g) * u.
__device__ __forceinline__ Pre pre_gu(const LoopParams& p, const Cx& c, int l) {
    const int u0 = c.ui0, nu = c.nui;
    Pre q;
    const int ub = c.w + LP_CW * (c.lane >> 1);
    if (ub < nu) q.a = gld(p.layers[l].s_gu + u0 + ub + (c.lane & 1) * p.I);
    return q;
}

template <int C>
__device__ bool phase_gu(const LoopParams& p, Cx& c, int line0, uint32_t tag,
                         const float (&xr)[LP_CMAX][16], float nscale, const Pre& pre) {
    int nmy;
    const int u0 = c.ui0, nu = c.nui;
    float acc[LP_MU_GU][2];
    if (!phase_dots<C, 2, LP_MU_GU>(p, c, line0, nu, xr, acc, nmy, 40)) return false;
#pragma unroll
    for (int m = 0; m < LP_MU_GU; m++) {
        if (m >= nmy) break;
        const float g = acc[m][0] * rlane(pre.a, 2 * m) * nscale;
        const float up = acc[m][1] * rlane(pre.a, 2 * m + 1) * nscale;
        if (c.lane == 0) ll_store(p.act + u0 + c.w + LP_CW * m, g * __frcp_rn(1.0f + __expf(-g)) * up, tag);
    }
    return true;
}

typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) u64 lds_u64;
typedef __attribute__((address_space(1))) const lp_v4i glb_v4i;   // global (not flat) loads
typedef __attribute__((address_space(1))) const float glb_f32;

template <int C>
__device__ __forceinline__ void lm_load(const int8_t* lm, int H, int uv0, int nuv, int w, int lane,
                                        int k0, lp_v4i (&wr)[LP_LM_B][C]) {
#pragma unroll
    for (int m = 0; m < LP_LM_B; m++) {
        const int ub = min(w + LP_CW * (k0 + m), nuv - 1);   // past the end: re-read the last row
        const int8_t* row = lm + (int64_t)(uv0 + ub) * H + lane * 16;
#pragma unroll
        for (int ch = 0; ch < C; ch++) wr[m][ch] = *(glb_v4i*)(row + ch * 1024);
    }
}

// One batch of LP_LM_B rows (k0 .. k0 + LP_LM_B - 1 of this wave).
template <int C>
__device__ __forceinline__ void lm_batch(int k0, int nk, int sbase, float sv, float nscale,
                                         float* logits, int row0, int lane,
                                         const float (&xr)[C][16], float xoff,
                                         const lp_v4i (&wr)[LP_LM_B][C], float& bestv, int& besti) {
    float acc[LP_LM_B];
#pragma unroll
    for (int m = 0; m < LP_LM_B; m++) {
        float s[4] = {xoff, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ch = 0; ch < C; ch++) lp_dot16(xr[ch], wr[m][ch], s);
        acc[m] = (s[0] + s[1]) + (s[2] + s[3]);
    }
    wsum_n<LP_LM_B>(acc);
#pragma unroll
    for (int m = 0; m < LP_LM_B; m++) {
        const int row = row0 + LP_CW * (k0 + m);
        const float v = acc[m] * rlane(sv, k0 + m - sbase) * nscale;
        const bool in = k0 + m < nk;
        if (in && v > bestv) {   // rows ascend: ties keep the first
            bestv = v;
            besti = row;
        }
        if (in && logits && lane == 0) logits[row] = v;
    }
}

// lm_head: the one phase that is pure streaming (155 MB at the Qwen3-0.6B
// shape) and waits on no other workgroup, so the compute waves read its rows
// straight from HBM into registers, LP_LM_B rows per batch, double-buffered
// (the next batch's loads are in flight while the current one is reduced).
// This wave's rows: uv0 + w + 4k. Out of line, so that its registers are its
// own; x comes from the staged LDS copy. Writes the wave's argmax key.
template <int C>
__device__ __noinline__ void phase_lm(const int8_t* lm, const float* s_lm, float* logits, int H,
                                      int uv0, int nuv, int w, int lane, const lds_f32* xs,
                                      float nscale, uint32_t tag, lds_u64* wkey) {
    float xr[C][16];
#pragma unroll
    for (int ch = 0; ch < C; ch++)
#pragma unroll
        for (int i = 0; i < 16; i++) xr[ch][i] = xs[ch * 1024 + lane * 16 + i];
    float xoff = 0.f;
#pragma unroll
    for (int ch = 0; ch < C; ch++) xoff += lp_xoff(xr[ch]);
    const int nk = nuv > w ? (nuv - w + LP_CW - 1) / LP_CW : 0;   // rows of this wave
    const int row0 = uv0 + w;
    float bestv = -INFINITY;
    int besti = 0;
    int sbase = 0;
    float sv = w + LP_CW * lane < nuv ? *(glb_f32*)(s_lm + row0 + LP_CW * lane) : 0.f;
    lp_v4i wa[LP_LM_B][C], wb[LP_LM_B][C];
    if (nk > 0) lm_load<C>(lm, H, uv0, nuv, w, lane, 0, wa);
    for (int k0 = 0; k0 < nk; k0 += 2 * LP_LM_B) {
        if (k0 - sbase > 64 - 2 * LP_LM_B) {
            sbase = k0;
            const int ub = w + LP_CW * (k0 + lane);
            sv = ub < nuv ? *(glb_f32*)(s_lm + uv0 + ub) : 0.f;
        }
        // sched_barrier: keep each batch's conversions next to its FMAs (the
        // scheduler would otherwise convert the in-flight batch too, and spill)
        if (k0 + LP_LM_B < nk) lm_load<C>(lm, H, uv0, nuv, w, lane, k0 + LP_LM_B, wb);
        __builtin_amdgcn_sched_barrier(0);
        lm_batch<C>(k0, nk, sbase, sv, nscale, logits, row0, lane, xr, xoff, wa, bestv, besti);
        __builtin_amdgcn_sched_barrier(0);
        if (k0 + LP_LM_B >= nk) break;
        if (k0 + 2 * LP_LM_B < nk) lm_load<C>(lm, H, uv0, nuv, w, lane, k0 + 2 * LP_LM_B, wa);
        __builtin_amdgcn_sched_barrier(0);
        lm_batch<C>(k0 + LP_LM_B, nk, sbase, sv, nscale, logits, row0, lane, xr, xoff, wb, bestv, besti);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (lane == 0) *wkey = nk > 0 ? lp_key(bestv, besti, tag) : 0;
}

// Argmax over the workgroups' keys of the lm phase tagged `tag` (first max,
// tensor_ops.c:649-662).
__device__ bool argmax_id(const LoopParams& p, Cx& c, uint32_t tag, int& id) {
    const int n = (p.nblk + 63) / 64;
    for (uint32_t it = 0;; it++) {
        u64 best = 0;
        bool ok = true;
        for (int i = 0; i < n; i++) {
            const int j = c.lane + 64 * i;
            if (j >= p.nblk) continue;
            const u64 k = ll_load(p.keys + j);
            ok &= (uint32_t)(k & 0x3FFF) == (tag & 0x3FFFu);
            best = k > best ? k : best;
        }
        if (__all(ok)) {
            best = wave_max_u64(best);
            id = (int)(0x3FFFFu - (uint32_t)((best >> 14) & 0x3FFFF));
            return true;
        }
        if (!keep_waiting(p, c, it, LP_POLL_LIMIT, 70)) return false;
    }
}

// ------------------------------------------------------------- attention
struct AttRange {
    int s, kvh, t0, n, tw0, tw1;
};

__device__ __forceinline__ AttRange att_range(const LoopParams& p, int w, int pos) {
    AttRange r;
    r.kvh = blockIdx.x / LP_S;
    r.s = blockIdx.x % LP_S;
    const int Lc = pos + 1, cs = (Lc + LP_S - 1) / LP_S;
    r.t0 = r.s * cs;
    r.n = min(cs, Lc - r.t0);
    const int nw = r.n > 0 ? (r.n + LP_CW - 1) / LP_CW : 0;
    r.tw0 = r.t0 + w * nw;
    r.tw1 = r.n > 0 ? min(r.t0 + r.n, r.tw0 + nw) : r.tw0;
    return r;
}

__device__ __forceinline__ void load_row16(const float* src, float (&d)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 a = *(const float4*)(src + 4 * i);
        d[4 * i] = a.x; d[4 * i + 1] = a.y; d[4 * i + 2] = a.z; d[4 * i + 3] = a.w;
    }
}
// The same from global memory (the KV cache), through the global address space.
typedef float lp_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void load_row16g(const float* src, float (&d)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const lp_f4 a = gld((const lp_f4*)(src + 4 * i));
        d[4 * i] = a[0]; d[4 * i + 1] = a[1]; d[4 * i + 2] = a[2]; d[4 * i + 3] = a[3];
    }
}

// Partial attention of split s over this workgroup's positions. Lane layout:
// 8 lanes per position (16 dims each), 8 positions per pass, both query heads
// of the KV head per pass; online softmax per lane group. The current
// position's k/v (this step's, from the tagged copy) is one extra step, done by
// lane group 0 of the wave whose range holds it. The per-lane-group partials
// (scaled to the wave's max) go to LDS and one pass over them combines the 32
// lane groups of the workgroup; the split's (max, sum, o) is stored tagged.
__device__ bool phase_att(const LoopParams& p, Cx& c, int l, int pos, uint32_t qtag, uint32_t tag) {
    constexpr int G = LP_G;
    const AttRange r = att_range(p, c.w, pos);
    if (r.n <= 0) return true;
    const int j = c.lane >> 3, part = c.lane & 7;
    const int npos = max(0, r.tw1 - r.tw0), passes = (npos + 7) / 8;
    float* stg = c.stg + c.w * LP_STG;
    const bool has_cur = pos >= r.tw0 && pos < r.tw1;
    // Keys/values of the earlier positions (final since the steps that wrote
    // them): issued before the q poll, so their latency hides behind it.
    const float* kb = p.kc + ((int64_t)l * p.nkv + r.kvh) * p.max_seq * 128;
    const float* vb = p.vc + ((int64_t)l * p.nkv + r.kvh) * p.max_seq * 128;
    float kp[LP_NPF][16], vp[LP_NPF][16];
#pragma unroll
    for (int ps = 0; ps < LP_NPF; ps++) {
        const int tp = r.tw0 + ps * 8 + j;
        if (tp < r.tw1 && tp != pos) {
            load_row16g(kb + (int64_t)tp * 128 + part * 16, kp[ps]);
            load_row16g(vb + (int64_t)tp * 128 + part * 16, vp[ps]);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) { kp[ps][i] = 0.f; vp[ps][i] = 0.f; }
        }
    }
    {
        // q of this KV head's G query heads, and the current k/v row, in one poll
        for (uint32_t it = 0;; it++) {
            u64 v[2 * G + 4];
            bool ok = true;
#pragma unroll
            for (int i = 0; i < 2 * G; i++) {
                v[i] = ll_load(p.q + r.kvh * G * 128 + c.lane + 64 * i);
                ok &= (uint32_t)(v[i] >> 32) == qtag;
            }
            if (has_cur) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[2 * G + i] = ll_load(p.kv + r.kvh * 256 + c.lane + 64 * i);
                    ok &= (uint32_t)(v[2 * G + i] >> 32) == qtag;
                }
            }
            if (__all(ok)) {
#pragma unroll
                for (int i = 0; i < 2 * G; i++) stg[c.lane + 64 * i] = __uint_as_float((uint32_t)v[i]);
                if (has_cur) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        stg[G * 128 + c.lane + 64 * i] = __uint_as_float((uint32_t)v[2 * G + i]);
                }
                break;
            }
            if (!keep_waiting(p, c, it, LP_POLL_LIMIT, 20)) return false;
        }
    }
    cbar();
    float qv[G][16];
#pragma unroll
    for (int h = 0; h < G; h++) load_row16(stg + h * 128 + part * 16, qv[h]);
    float m[G], lsum[G], o[G][16];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = -INFINITY;
        lsum[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) o[h][i] = 0.f;
    }
    auto step = [&](const float (&kk)[16], const float (&vv)[16], bool valid) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            float d4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 16; i++) d4[i & 3] = fmaf(qv[h][i], kk[i], d4[i & 3]);
            float s = sum8((d4[0] + d4[1]) + (d4[2] + d4[3])) * p.att_scale;
            s = valid ? s : -INFINITY;
            const float mn = fmaxf(m[h], s);
            const float corr = mn == -INFINITY ? 1.f : __expf(m[h] - mn);
            const float e = s == -INFINITY ? 0.f : __expf(s - mn);
            lsum[h] = fmaf(lsum[h], corr, e);
#pragma unroll
            for (int i = 0; i < 16; i++) o[h][i] = fmaf(o[h][i], corr, e * vv[i]);
            m[h] = mn;
        }
    };
#pragma unroll
    for (int ps = 0; ps < LP_NPF; ps++) {
        const int tp = r.tw0 + ps * 8 + j;
        step(kp[ps], vp[ps], ps < passes && tp < r.tw1 && tp != pos);
    }
    for (int ps = LP_NPF; ps < passes; ps++) {
        const int tp = r.tw0 + ps * 8 + j;
        const bool valid = tp < r.tw1 && tp != pos;
        float kk[16], vv[16];
        if (valid) {
            load_row16g(kb + (int64_t)tp * 128 + part * 16, kk);
            load_row16g(vb + (int64_t)tp * 128 + part * 16, vv);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) { kk[i] = 0.f; vv[i] = 0.f; }
        }
        step(kk, vv, valid);
    }
    if (has_cur) {
        float kk[16], vv[16];
        load_row16(stg + G * 128 + part * 16, kk);
        load_row16(stg + G * 128 + 128 + part * 16, vv);
        step(kk, vv, j == 0);
    }
    // Scale every lane group to the wave's max; partials to LDS:
    // po[w][h][j][128], wave max / sum in pm / pl.
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float mw = wmax(m[h]);
        const float f = m[h] == -INFINITY ? 0.f : __expf(m[h] - mw);
        const float lw = wsum(part == 0 ? lsum[h] * f : 0.f);
        float* dst = c.attp + ((c.w * G + h) * 8 + j) * 128 + part * 16;
#pragma unroll
        for (int i = 0; i < 16; i += 4)
            *(float4*)(dst + i) = make_float4(o[h][i] * f, o[h][i + 1] * f, o[h][i + 2] * f, o[h][i + 3] * f);
        if (c.lane == 0) {
            c.attm[c.w * G + h] = mw;
            c.attm[LP_CW * G + c.w * G + h] = lw;
        }
    }
    if (!csync(p, c, 22)) return false;
    // combine: one (head, dim) per thread of the four waves
    u64* dst = p.part + (int64_t)(r.kvh * LP_S + r.s) * G * LP_PART;
    for (int e = c.w * 64 + c.lane; e < G * 128; e += LP_CW * 64) {
        const int h = e >> 7, d = e & 127;
        float M = -INFINITY;
#pragma unroll
        for (int wv = 0; wv < LP_CW; wv++) M = fmaxf(M, c.attm[wv * G + h]);
        float acc = 0.f, den = 0.f;
#pragma unroll
        for (int wv = 0; wv < LP_CW; wv++) {
            const float mw = c.attm[wv * G + h];
            const float F = mw == -INFINITY ? 0.f : __expf(mw - M);
            const float* src = c.attp + (wv * G + h) * 8 * 128 + d;
            float sj = 0.f;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) sj += src[jj * 128];
            acc = fmaf(F, sj, acc);
            den = fmaf(F, c.attm[LP_CW * G + wv * G + h], den);
        }
        ll_store(dst + h * LP_PART + 2 + d, acc, tag);
        if (d == 0) {
            ll_store(dst + h * LP_PART, M, tag);
            ll_store(dst + h * LP_PART + 1, den, tag);
        }
    }
    return true;
}

// Merge of the active splits of query head h = kvh*G + w (wave w < G of the
// split-0 workgroup of each KV head), in split order; tagged head output.
__device__ bool phase_merge(const LoopParams& p, Cx& c, int pos, uint32_t ptag, uint32_t tag) {
    const int G = p.nq / p.nkv;
    const int kvh = blockIdx.x / LP_S;
    const int h = kvh * G + c.w;
    const int Lc = pos + 1, cs = (Lc + LP_S - 1) / LP_S, sact = (Lc + cs - 1) / cs;
    float mm[LP_S], ll[LP_S], o0[LP_S], o1[LP_S];
    for (uint32_t it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int s = 0; s < LP_S; s++) {
            if (s >= sact) continue;
            const u64* src = p.part + ((int64_t)(kvh * LP_S + s) * G + c.w) * LP_PART;
            const u64 a = ll_load(src), b = ll_load(src + 1), x0 = ll_load(src + 2 + c.lane),
                      x1 = ll_load(src + 2 + 64 + c.lane);
            ok &= (uint32_t)(a >> 32) == ptag && (uint32_t)(b >> 32) == ptag &&
                  (uint32_t)(x0 >> 32) == ptag && (uint32_t)(x1 >> 32) == ptag;
            mm[s] = __uint_as_float((uint32_t)a);
            ll[s] = __uint_as_float((uint32_t)b);
            o0[s] = __uint_as_float((uint32_t)x0);
            o1[s] = __uint_as_float((uint32_t)x1);
        }
        if (__all(ok)) break;
        if (!keep_waiting(p, c, it, LP_POLL_LIMIT, 30)) return false;
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < LP_S; s++)
        if (s < sact) M = fmaxf(M, mm[s]);
    float den = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int s = 0; s < LP_S; s++) {
        if (s >= sact) continue;
        const float f = mm[s] == -INFINITY ? 0.f : __expf(mm[s] - M);
        den += f * ll[s];
        a0 += f * o0[s];
        a1 += f * o1[s];
    }
    const float inv = __frcp_rn(den);
    ll_store(p.merged + h * 128 + c.lane, a0 * inv, tag);
    ll_store(p.merged + h * 128 + 64 + c.lane, a1 * inv, tag);
    return true;
}

// ----------------------------------------------------------- wave roles
__device__ void stream_role(const LoopParams& p, Cx& c) {
    const int sw = c.w - LP_CW;
    const int8_t* src = p.stream + (int64_t)blockIdx.x * p.lpt * 1024 + c.lane * 16;
    typedef __attribute__((address_space(3))) void lds_t;
    int G = 0, inflight = 0, published = 0;
    bool ok = true;
    for (int t = 0; t < p.n_steps && ok; t++) {
        const int nl = p.lpt;
        for (int j = ((sw - G) % LP_SW + LP_SW) % LP_SW; j < nl; j += LP_SW) {
            const int Lg = G + j;
            if (lds_ld(c.abort)) { ok = false; break; }
            // the slot of line Lg held line Lg - LP_RING: free once every
            // compute wave has moved past it
            auto room = [&]() {
                int mn = lds_ld(&c.done[0]);
#pragma unroll
                for (int i = 1; i < LP_CW; i++) mn = min(mn, lds_ld(&c.done[i]));
                return mn > Lg - LP_RING;
            };
            if (!room()) {
                wait_vm<0>();
                published += inflight;
                inflight = 0;
                lds_st_raw(&c.ready[sw], published);
                for (uint32_t it = 0; !room(); it++) {
                    if (!keep_waiting(p, c, it, LP_LDS_LIMIT, 80)) { ok = false; break; }
                    __builtin_amdgcn_s_sleep(2);
                }
                if (!ok) break;
                cbar();
            }
            // nt: the weights are read once per token; keep them out of the caches
            __builtin_amdgcn_global_load_lds((const void*)(src + (int64_t)j * 1024),
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

template <int CH, int CO, int CI>
__device__ void compute_role(const LoopParams& p, Cx& c) {
    __builtin_amdgcn_s_setprio(2);
    const int H = p.H, KO = p.nq * 128, I = p.I;
    const bool att_blk = (int)blockIdx.x < p.nkv * LP_S;
    const bool merger = att_blk && (blockIdx.x % LP_S) == 0 && c.w < p.nq / p.nkv;
    int Gl = 0;        // first ring line of the current token
    int buf = 0;
    int id = 0;
    for (int t = 0; t < p.n_steps; t++) {
        asm volatile("" : "+v"(c.lane));
        const int pos = p.pos0 + t;
        const bool lm = lm_needed(p, t);
        if (t == 0 || pos < p.prompt_len) {
            id = p.ids[pos];
        } else {
            if (!argmax_id(p, c, tag_of(p, t - 1, p.L, 0), id)) return;
            if (blockIdx.x == 0 && c.w == 0 && c.lane == 0) p.ids[pos] = id;
        }
        if (id < 0 || id >= p.V) id = 0;
        const float* emb = p.embed + (int64_t)id * H;
        for (int l = 0; l < p.L; l++) {
            // Opaque per-iteration copy of the lane id: keeps the compiler from
            // hoisting every per-lane address of the loop body out of the loop
            // (they would stay live across all phases and spill).
            asm volatile("" : "+v"(c.lane));
            const LoopLayer& Lw = p.layers[l];
            const int lb = Gl + l * p.lpl;
            const uint32_t tq = tag_of(p, t, l, PH_QKV);
            // ---- qkv: x = embed row (layer 0) or the previous layer's output
            {
                constexpr int NX = CH * 4;
                cbar();   // the preloads must not move above the previous phase
                const Pre pq = pre_qkv(p, c, l, pos);
                float v[NX], g[NX], xr[LP_CMAX][16], nscale;
#pragma unroll
                for (int i = 0; i < NX; i++) g[i] = gld(Lw.in_norm + c.w * (H / 4) + c.lane + 64 * i);
                if (l == 0) {
#pragma unroll
                    for (int i = 0; i < NX; i++) v[i] = gld(emb + c.w * (H / 4) + c.lane + 64 * i);
                } else if (!ll_poll<NX>(p, c, p.xa + c.w * (H / 4), NX, tag_of(p, t, l - 1, PH_DN), v, 1)) {
                    return;
                }
                if (!stage_x<NX, CH>(p, c, buf, H, v, g, true, xr, nscale, 2)) return;
                buf ^= 1;
                if (!phase_qkv<CH>(p, c, l, pos, lb, tq, xr, nscale, pq)) return;
                set_done(c, lb + p.off_o);
            }
            // ---- attention partials and merge
            if (att_blk && !phase_att(p, c, l, pos, tq, tag_of(p, t, l, PH_ATT))) return;
            if (merger && !phase_merge(p, c, pos, tag_of(p, t, l, PH_ATT), tag_of(p, t, l, PH_MERGE)))
                return;
            // ---- o_proj (+ residual)
            {
                constexpr int NX = CO * 4;
                float v[NX], g[NX], xr[LP_CMAX][16], nscale;
                const u64* rin = l == 0 ? nullptr : p.xa;
                cbar();   // the preloads must not move above the previous phase
                const Pre pr = pre_resid(p, c, Lw.s_o, rin);
                if (!ll_poll<NX>(p, c, p.merged + c.w * (KO / 4), NX, tag_of(p, t, l, PH_MERGE), v, 3))
                    return;
                if (!stage_x<NX, CO>(p, c, buf, KO, v, g, false, xr, nscale, 4)) return;
                buf ^= 1;
                if (!phase_resid<CO>(p, c, lb + p.off_o, rin, tag_of(p, t, l - 1, PH_DN), emb, p.xb,
                                     tag_of(p, t, l, PH_O), xr, pr, 32))
                    return;
                set_done(c, lb + p.off_gu);
            }
            // ---- gate_up + SwiGLU
            {
                constexpr int NX = CH * 4;
                float v[NX], g[NX], xr[LP_CMAX][16], nscale;
#pragma unroll
                for (int i = 0; i < NX; i++) g[i] = gld(Lw.post_norm + c.w * (H / 4) + c.lane + 64 * i);
                cbar();   // the preloads must not move above the previous phase
                const Pre pg = pre_gu(p, c, l);
                if (!ll_poll<NX>(p, c, p.xb + c.w * (H / 4), NX, tag_of(p, t, l, PH_O), v, 5)) return;
                if (!stage_x<NX, CH>(p, c, buf, H, v, g, true, xr, nscale, 6)) return;
                buf ^= 1;
                if (!phase_gu<CH>(p, c, lb + p.off_gu, tag_of(p, t, l, PH_GU), xr, nscale, pg)) return;
                set_done(c, lb + p.off_dn);
            }
            // ---- down (+ residual)
            {
                constexpr int NX = CI * 4;
                float v[NX], g[NX], xr[LP_CMAX][16], nscale;
                cbar();   // the preloads must not move above the previous phase
                const Pre pd = pre_resid(p, c, Lw.s_down, p.xb);
                if (!ll_poll<NX>(p, c, p.act + c.w * (I / 4), NX, tag_of(p, t, l, PH_GU), v, 7)) return;
                if (!stage_x<NX, CI>(p, c, buf, I, v, g, false, xr, nscale, 8)) return;
                buf ^= 1;
                if (!phase_resid<CI>(p, c, lb + p.off_dn, p.xb, tag_of(p, t, l, PH_O), nullptr, p.xa,
                                     tag_of(p, t, l, PH_DN), xr, pd, 50))
                    return;
                set_done(c, lb + p.lpl);
            }
        }
        if (lm) {
            constexpr int NX = CH * 4;
            float v[NX], g[NX], xr[LP_CMAX][16], nscale;
#pragma unroll
            for (int i = 0; i < NX; i++) g[i] = gld(p.final_norm + c.w * (H / 4) + c.lane + 64 * i);
            if (!ll_poll<NX>(p, c, p.xa + c.w * (H / 4), NX, tag_of(p, t, p.L - 1, PH_DN), v, 9)) return;
            if (!stage_x<NX, CH>(p, c, buf, H, v, g, true, xr, nscale, 11)) return;
            const uint32_t tl = tag_of(p, t, p.L, 0);
            phase_lm<CH>(p.lm_head, p.s_lm, t == p.n_steps - 1 ? p.logits : nullptr, H, c.uv0, c.nuv,
                         c.w, c.lane, (const lds_f32*)(c.xs + buf * LP_XS), nscale, tl,
                         (lds_u64*)(c.wkeys + c.w));
            buf ^= 1;
            if (!csync(p, c, 61)) return;
            if (c.w == 0 && c.lane == 0) {
                u64 b = c.wkeys[0];
                for (int i = 1; i < LP_CW; i++) b = c.wkeys[i] > b ? c.wkeys[i] : b;
                b = (b & ~(u64)0x3FFF) | (u64)(tl & 0x3FFFu);
                __hip_atomic_store(p.keys + blockIdx.x, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        Gl += p.lpt;
    }
    // The last step's argmax -> ids[pos+1] and the device position/state.
    if (blockIdx.x == 0 && c.w == 0) {
        const int pos = p.pos0 + p.n_steps - 1;
        int last = id;
        if (pos + 1 >= p.prompt_len) {
            if (!argmax_id(p, c, tag_of(p, p.n_steps - 1, p.L, 0), last)) return;
            if (c.lane == 0 && pos + 1 < p.max_seq + 1) p.ids[pos + 1] = last;
        }
        if (c.lane == 0) {
            p.state[0] = pos + 1;
            p.state[2] = last;
        }
    }
}

template <int CH, int CO, int CI>
__global__ __launch_bounds__(LP_THREADS, 1) void decode_loop_kernel(LoopParams p) {
    extern __shared__ __attribute__((aligned(16))) int8_t lp_lds[];
    __shared__ int ready[LP_SW], done[LP_CW], sync_ctr, abort_flag;
    __shared__ u64 wkeys[LP_CW];
    __shared__ float ss[2 * LP_CW];
    if (threadIdx.x < LP_SW) ready[threadIdx.x] = 0;
    if (threadIdx.x < LP_CW) done[threadIdx.x] = 0;
    if (threadIdx.x == 0) { sync_ctr = 0; abort_flag = 0; }
    __syncthreads();
    Cx c;
    c.lane = threadIdx.x & 63;
    c.w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
    {
        const Units q = blk_units((p.nq + 2 * p.nkv) * 64, p.nblk), h = blk_units(p.H, p.nblk),
                    i = blk_units(p.I, p.nblk), v = blk_units(p.V, p.nblk);
        c.uq0 = q.u0; c.nuq = q.nu; c.uh0 = h.u0; c.nuh = h.nu;
        c.ui0 = i.u0; c.nui = i.nu; c.uv0 = v.u0; c.nuv = v.nu;
    }
    c.nsync = 0;
    c.fail_where = 0;
    c.ready = ready;
    c.done = done;
    c.csync = &sync_ctr;
    c.abort = &abort_flag;
    c.ring = lp_lds;
    c.xs = (float*)(lp_lds + LP_LDS_RING);
    c.ss = ss;
    c.attp = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XS);
    c.attm = c.attp + LP_CW * LP_G * 8 * 128;
    c.stg = (float*)(lp_lds + LP_LDS_RING + LP_LDS_XS + LP_LDS_ATT);
    c.wkeys = wkeys;
    if (c.w >= LP_CW) {
        stream_role(p, c);
    } else {
        compute_role<CH, CO, CI>(p, c);
        // a compute wave that leaves early must not hold the ring
        cbar();
        if (c.lane == 0) lds_st(&done[c.w], 0x7fffffff);
    }
    if (c.fail_where && c.lane == 0) lp_fail(p, c.fail_where);
}

// ------------------------------------------------------------------ host
struct LoopState {
    int nblk = 0;
    int lpl = 0, off_o = 0, off_gu = 0, off_dn = 0, lpt = 0;
    void* stream = nullptr;      // relaid weights
    void* small = nullptr;       // tagged buffers + layer table + error words
    size_t small_bytes = 0, ll_bytes = 0;
    LoopLayer* layers = nullptr;
    u64 *xa, *xb, *q, *kv, *part, *merged, *act, *keys;
    int* err = nullptr;
    uint32_t epoch = 1;
    bool ran = false;
};

// Unit counts and lines per unit of the five weight phases.
struct PhaseShape {
    int U, lpu;
};

static int seg_lines(const PhaseShape& s, int nblk) { return ceil_div(s.U, nblk) * s.lpu; }

// The kernel's dynamic LDS exceeds the 64 KB default limit.
static int loop_lds_attr() {
    PIO_HIP(hipFuncSetAttribute((const void*)decode_loop_kernel<LP_CH, LP_CO, LP_CI>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)LP_LDS_BYTES));
    return PIO_OK;
}

int loop_check(const Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    int dev = 0, cus = 0, per_cu = 0;
    PIO_HIP(hipGetDevice(&dev));
    PIO_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    PIO_TRY(loop_lds_attr());
    PIO_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, decode_loop_kernel<LP_CH, LP_CO, LP_CI>, LP_THREADS, LP_LDS_BYTES));
    if (per_cu < 1)
        return set_error(PIO_ERR_UNSUPPORTED, "persistent decode: a %d-thread workgroup with %zu B "
                         "of LDS does not fit a CU", LP_THREADS, LP_LDS_BYTES);
    const int G = c.n_heads / c.n_kv_heads;
    const bool ok = c.head_dim == 128 && c.hidden == LP_CH * 1024 &&
                    c.n_heads * 128 == LP_CO * 1024 && c.intermediate == LP_CI * 1024 && G == LP_G &&
                    c.n_kv_heads * LP_S <= cus && c.max_seq <= LP_MAX_SEQ && c.vocab <= (1 << 18);
    // per-wave unit counts must fit the one-value-per-lane preloads
    auto per_wave = [&](int U) { return ceil_div(ceil_div(U, cus), LP_CW); };
    const bool fits = per_wave((c.n_heads + 2 * c.n_kv_heads) * 64) <= LP_MU_QKV &&
                      per_wave(c.intermediate) <= LP_MU_GU && per_wave(c.hidden) <= LP_MU_ROW;
    if (!ok || !fits)
        return set_error(PIO_ERR_UNSUPPORTED,
                         "persistent decode is built for the Qwen3-0.6B layer shape: head_dim 128, "
                         "hidden %d, n_heads*head_dim %d, intermediate %d, %d query heads per KV "
                         "head, n_kv_heads*%d <= %d CUs, max_seq <= %d, vocab <= 262144",
                         LP_CH * 1024, LP_CO * 1024, LP_CI * 1024, LP_G, LP_S, cus, LP_MAX_SEQ);
    return PIO_OK;
}

__global__ void loop_gather_kernel(const int8_t* const* __restrict__ src, int8_t* __restrict__ dst,
                                   int64_t nlines) {
    const int64_t line = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (line >= nlines) return;
    const int lane = threadIdx.x & 63;
    const lp_v4i v = *(const lp_v4i*)(src[line] + lane * 16);
    *(lp_v4i*)(dst + line * 1024 + lane * 16) = v;
}

// Lays every workgroup's weight lines out contiguously, in the order its
// compute waves consume them (the same unit split as the kernel's blk_units).
static int loop_build(Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    LoopState* s = new LoopState();
    d->loop = s;
    int dev = 0;
    PIO_HIP(hipGetDevice(&dev));
    PIO_HIP(hipDeviceGetAttribute(&s->nblk, hipDeviceAttributeMultiprocessorCount, dev));
    const int nb = s->nblk, H = c.hidden, I = c.intermediate, KO = c.n_heads * 128;
    const int CH = H / 1024, CO = KO / 1024, CI = I / 1024;
    const PhaseShape qkv{(c.n_heads + 2 * c.n_kv_heads) * 64, 2 * CH}, o{H, CO}, gu{I, 2 * CH},
        dn{H, CI};
    s->off_o = seg_lines(qkv, nb);
    s->off_gu = s->off_o + seg_lines(o, nb);
    s->off_dn = s->off_gu + seg_lines(gu, nb);
    s->lpl = s->off_dn + seg_lines(dn, nb);
    s->lpt = c.n_layers * s->lpl;

    // source line table
    void* zero = nullptr;
    PIO_TRY(device_alloc(&zero, 1024, d->st));
    Scratch zero_guard;
    zero_guard.ptr = zero;
    PIO_HIP(hipMemsetAsync(zero, 0, 1024, d->st));
    const int64_t nlines = (int64_t)nb * s->lpt;
    std::vector<const int8_t*> tab((size_t)nlines, (const int8_t*)zero);
    auto blk = [&](int U, int b, int& u0, int& nu) {
        u0 = (int)(((int64_t)b * U) / nb);
        nu = (int)(((int64_t)(b + 1) * U) / nb) - u0;
    };
    for (int b = 0; b < nb; b++) {
        const int64_t base = (int64_t)b * s->lpt;
        int u0, nu;
        for (int l = 0; l < c.n_layers; l++) {
            const pio_qwen3_layer& L = d->layers[l];
            const int64_t lb = base + (int64_t)l * s->lpl;
            blk(qkv.U, b, u0, nu);
            for (int ub = 0; ub < nu; ub++) {
                const int u = u0 + ub, r0 = (u >> 6) * 128 + (u & 63), r1 = r0 + 64;
                for (int ch = 0; ch < CH; ch++) {
                    tab[lb + ub * qkv.lpu + ch] = L.w_qkv + (int64_t)r0 * H + ch * 1024;
                    tab[lb + ub * qkv.lpu + CH + ch] = L.w_qkv + (int64_t)r1 * H + ch * 1024;
                }
            }
            blk(o.U, b, u0, nu);
            for (int ub = 0; ub < nu; ub++)
                for (int ch = 0; ch < CO; ch++)
                    tab[lb + s->off_o + ub * CO + ch] = L.w_o + (int64_t)(u0 + ub) * KO + ch * 1024;
            blk(gu.U, b, u0, nu);
            for (int ub = 0; ub < nu; ub++)
                for (int ch = 0; ch < CH; ch++) {
                    tab[lb + s->off_gu + ub * gu.lpu + ch] = L.w_gu + (int64_t)(u0 + ub) * H + ch * 1024;
                    tab[lb + s->off_gu + ub * gu.lpu + CH + ch] =
                        L.w_gu + (int64_t)(u0 + ub + I) * H + ch * 1024;
                }
            blk(dn.U, b, u0, nu);
            for (int ub = 0; ub < nu; ub++)
                for (int ch = 0; ch < CI; ch++)
                    tab[lb + s->off_dn + ub * CI + ch] = L.w_down + (int64_t)(u0 + ub) * I + ch * 1024;
        }
    }
    PIO_TRY(device_alloc(&s->stream, (size_t)nlines * 1024, d->st));
    void* dtab = nullptr;
    PIO_TRY(device_alloc(&dtab, (size_t)nlines * sizeof(void*), d->st));
    Scratch tab_guard;
    tab_guard.ptr = dtab;
    PIO_HIP(hipMemcpyAsync(dtab, tab.data(), (size_t)nlines * sizeof(void*), hipMemcpyHostToDevice,
                           d->st));
    loop_gather_kernel<<<(unsigned)((nlines + 3) / 4), 256, 0, d->st>>>((const int8_t* const*)dtab,
                                                                        (int8_t*)s->stream, nlines);
    PIO_LAUNCHED();

    // tagged buffers, layer table, error words
    const int G = c.n_heads / c.n_kv_heads;
    const size_t n_ll[] = {(size_t)H, (size_t)H, (size_t)KO, (size_t)c.n_kv_heads * 256,
                           (size_t)c.n_kv_heads * LP_S * G * LP_PART, (size_t)KO, (size_t)I,
                           (size_t)nb};
    size_t off[9];
    off[0] = 0;
    for (int i = 0; i < 8; i++) off[i + 1] = off[i] + (n_ll[i] * 8 + 255) / 256 * 256;
    s->ll_bytes = off[8];
    const size_t lay_off = s->ll_bytes;
    const size_t err_off = lay_off + (c.n_layers * sizeof(LoopLayer) + 255) / 256 * 256;
    s->small_bytes = err_off + 256;
    PIO_TRY(device_alloc(&s->small, s->small_bytes, d->st));
    char* sp = (char*)s->small;
    u64** dst[] = {&s->xa, &s->xb, &s->q, &s->kv, &s->part, &s->merged, &s->act, &s->keys};
    for (int i = 0; i < 8; i++) *dst[i] = (u64*)(sp + off[i]);
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
    PIO_HIP(hipStreamSynchronize(d->st));   // the host table and guards go out of scope
    s->epoch = 1;
    return PIO_OK;
}

void loop_destroy(Qwen3Dec* d) {
    if (!d || !d->loop) return;
    if (d->loop->stream) device_free(d->loop->stream);
    if (d->loop->small) device_free(d->loop->small);
    delete d->loop;
    d->loop = nullptr;
}

template <int CH, int CO, int CI>
static int launch_loop(LoopParams& p, hipStream_t st) {
    PIO_TRY(loop_lds_attr());
    decode_loop_kernel<CH, CO, CI><<<dim3(p.nblk), dim3(LP_THREADS), LP_LDS_BYTES, st>>>(p);
    PIO_LAUNCHED();
    return PIO_OK;
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
    const uint32_t per_tok = (uint32_t)(c.n_layers * LP_PH + 1);
    if ((uint64_t)s->epoch + (uint64_t)n_steps * per_tok + 1 >= 0xFFFFFFFFull) {
        // tags would wrap: clear every tagged word and start over
        PIO_HIP(hipMemsetAsync(s->small, 0, s->ll_bytes, d->st));
        s->epoch = 1;
    }
    PIO_HIP(hipMemsetAsync(s->err, 0, 16, d->st));
    LoopParams p{};
    p.L = c.n_layers; p.H = c.hidden; p.nq = c.n_heads; p.nkv = c.n_kv_heads;
    p.I = c.intermediate; p.V = c.vocab; p.max_seq = c.max_seq; p.nblk = s->nblk;
    p.eps = c.rms_eps;
    p.att_scale = 1.0f / sqrtf((float)c.head_dim);
    p.embed = d->embed; p.final_norm = d->final_norm; p.s_lm = d->s_lm;
    p.layers = s->layers;
    p.stream = (const int8_t*)s->stream;
    p.lpl = s->lpl; p.off_o = s->off_o; p.off_gu = s->off_gu; p.off_dn = s->off_dn;
    p.lpt = s->lpt;
    p.lm_head = d->lm_head;
    p.kc = d->kc; p.vc = d->vc; p.cos_t = d->cos_t; p.sin_t = d->sin_t;
    p.xa = s->xa; p.xb = s->xb; p.q = s->q; p.kv = s->kv; p.part = s->part; p.merged = s->merged;
    p.act = s->act; p.keys = s->keys;
    p.ids = d->ids; p.logits = d->logits; p.state = d->state;
    p.pos0 = d->host_pos;
    p.prompt_len = d->prompt_len;
    p.n_steps = n_steps;
    p.epoch0 = s->epoch;
    p.err = s->err;
    PIO_TRY((launch_loop<LP_CH, LP_CO, LP_CI>(p, d->st)));
    s->epoch += (uint32_t)n_steps * per_tok;
    s->ran = true;
    return PIO_OK;
}

// Error words of the last persistent run (after the stream has drained).
int loop_status(Qwen3Dec* d) {
    if (!d->loop || !d->loop->ran) return PIO_OK;
    int e[2] = {0, 0};
    PIO_HIP(hipMemcpy(e, d->loop->err, sizeof(e), hipMemcpyDeviceToHost));
    d->loop->ran = false;
    if (e[0])
        return set_error(PIO_ERR_HIP, "persistent decode: a wait timed out (site %d); results of "
                                      "that run are invalid", e[1]);
    return PIO_OK;
}

}  // namespace pio
