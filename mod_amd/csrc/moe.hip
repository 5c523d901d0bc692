// Int8 MoE expert layer. Replaces the reference's per-expert Python loop
// (Qwen3Coder30BMoE.forward, ip/models/qwen3_coder_30b/model.py:308-353: a
// D2H sync per slot, one gather/MLP/scatter call chain per expert, an atomic
// and therefore order-dependent scatter-add) with six launches and a
// deterministic combine:
//
//  1. route:   p = softmax(logits) exactly as tensor_softmax (tensor_ops.c:351-368:
//              max seeded with -1e9, exp(x - max), multiply by 1/sum); top-k by
//              tensor_topk's rule (tensor_ops.c:719-738: strict '>', so equal
//              probabilities keep the lower expert id first); weights = the top-k
//              probabilities, optionally renormalized to sum 1. The same launch
//              quantizes x per token (the rows are shared by all k slots).
//  2. group:   (token, slot) pairs are sorted by expert, tokens ascending inside
//              an expert (one block per expert: its offset is the count of pairs
//              routed below it, its tokens ranked by ballots), so every expert's
//              rows are one contiguous run of an index list.
//  3. gate_up: grouped W8A8 GEMM, one block per (expert, 64 gate + 64 up
//              rows); the block walks its expert's row tiles, so each weight
//              tile is read from HBM once. Its epilogue applies SwiGLU,
//              h = silu(g) * u (tensor_ops.c:588-604 formula), writes h (fp32)
//              and the row's max |h| (atomic max).
//  4. requant: h per row to int8 with that max.
//  5. down:    grouped W8A8 GEMM over the contiguous h rows, fp32 output.
//  6. combine: out[t] = sum_{k=0..top_k-1} w[t,k] * down[pos(t,k)], in k order.
#include "gemm_core.hpp"

namespace pio {

// Minimum over the 64 lanes (in every lane), on DPP lane moves and readlane.
template <int CTRL>
__device__ __forceinline__ int dppi(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int wmin_i(int x) {
    x = min(x, dppi<DPP_XOR1>(x));
    x = min(x, dppi<DPP_XOR2>(x));
    x = min(x, dppi<DPP_HMIRROR>(x));
    x = min(x, dppi<DPP_MIRROR>(x));
    return min(min(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
               min(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// ------------------------------------------------------------------ route ---
// One wave per token, 4 tokens per block; the token's E probabilities live in LDS.
constexpr int ROUTE_MAX_E = 1024;

// Routing of one token by one wave: p (LDS, E floats) receives the
// probabilities; lanes < top_k write the token's weights and ids.
__device__ __forceinline__ void route_token(const float* __restrict__ lr, float* p, int lane, int E,
                                            int top_k, int renorm, float* __restrict__ w_out,
                                            int32_t* __restrict__ id_out) {
    float mx = -1e9f;
    for (int e0 = 0; e0 < E; e0 += 256) {
        float lv[4];   // four loads in flight (clamped index, not a guarded load each)
#pragma unroll
        for (int u = 0; u < 4; u++) lv[u] = lr[min(e0 + lane + 64 * u, E - 1)];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = e0 + lane + 64 * u;
            if (e < E) {
                p[e] = lv[u];
                mx = fmaxf(mx, lv[u]);
            }
        }
    }
    mx = wave_max(mx);
    float sum = 0.f;
    for (int e = lane; e < E; e += 64) {
        float v = expf(p[e] - mx);
        p[e] = v;
        sum += v;
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    for (int e = lane; e < E; e += 64) p[e] *= inv;

    // k rounds of (max value, then min index) selection; chosen entries are
    // retired by setting them to -inf (probabilities are >= 0). Each lane's
    // best (strict '>' over ascending e: its lowest index among equals), then
    // the wave max and the lowest index holding it, both as DPP reductions
    // (no LDS-queue shuffles in the dependent chain).
    float wsum = 0.f;
    float myw = 0.f;
    int myid = 0;
    for (int kk = 0; kk < top_k; kk++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int e = lane; e < E; e += 64) {
            const float v = p[e];
            if (v > bv) { bv = v; bi = e; }
        }
        const float m = wmax(bv);
        const int mi = wmin_i(bv == m ? bi : 0x7fffffff);
        if (lane == kk) { myw = m; myid = mi; }
        wsum += m;
        if (lane == (mi & 63)) p[mi] = -INFINITY;
    }
    if (lane < top_k) {
        w_out[lane] = renorm ? myw / wsum : myw;
        id_out[lane] = myid;
    }
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits,
                                                        float* __restrict__ topk_w,
                                                        int32_t* __restrict__ topk_id, int T,
                                                        int E, int top_k, int renorm) {
    __shared__ float sp[4][ROUTE_MAX_E];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + w;
    if (t >= T) return;
    route_token(logits + (int64_t)t * E, sp[w], lane, E, top_k, renorm, topk_w + (int64_t)t * top_k,
                topk_id + (int64_t)t * top_k);
}

// The layer's first launch: block b takes tokens 2b and 2b + 1; waves 0-1
// route them, waves 2-3 quantize their x rows per token (the quantizer of
// quant.hip: amax / 127, IEEE division, round-half-even), each row loaded once
// into registers, lane l holding the 8-element chunks l, l + 64, ...
// (H % 8 == 0, H <= 512 ROUTE_XG).
constexpr int ROUTE_XG = 8;
template <typename XT>
__global__ __launch_bounds__(256) void moe_route_quant_kernel(const float* __restrict__ logits,
                                                              const XT* __restrict__ x, int H,
                                                              float* __restrict__ topk_w,
                                                              int32_t* __restrict__ topk_id,
                                                              int8_t* __restrict__ qx,
                                                              float* __restrict__ sx, int T,
                                                              int E, int top_k, int renorm,
                                                              unsigned* __restrict__ hmax) {
    __shared__ float sp[2][ROUTE_MAX_E];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    // the gate_up epilogue's per-row max starts from 0 (grid >= 128 T threads >= T * top_k)
    {
        const int i = blockIdx.x * 256 + threadIdx.x;
        if (i < T * top_k) hmax[i] = 0u;
    }
    const int t = blockIdx.x * 2 + (w & 1);
    if (t >= T) return;
    if (w < 2) {
        route_token(logits + (int64_t)t * E, sp[w], lane, E, top_k, renorm,
                    topk_w + (int64_t)t * top_k, topk_id + (int64_t)t * top_k);
        return;
    }
    const XT* xr = x + (int64_t)t * H;
    const int nch = H / 8;
    // every group's raw bits first (clamped chunk index), widened afterwards
    Raw8<XT> raw[ROUTE_XG];
#pragma unroll
    for (int g = 0; g < ROUTE_XG; g++) raw[g] = raw8_load(xr + 8 * min(lane + 64 * g, nch - 1));
    float v[ROUTE_XG][8];
#pragma unroll
    for (int g = 0; g < ROUTE_XG; g++) raw8_widen(raw[g], v[g]);
    float amax = 0.f;
#pragma unroll
    for (int g = 0; g < ROUTE_XG; g++)
        if (lane + 64 * g < nch)
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[g][i]));
    amax = wmax(amax);
    const float sc = amax == 0.f ? 1.f : amax / 127.0f;
    if (lane == 0) sx[t] = sc;
    int8_t* qr = qx + (int64_t)t * H;
#pragma unroll
    for (int g = 0; g < ROUTE_XG; g++)
        if (lane + 64 * g < nch) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) lo |= (uint32_t)(uint8_t)quant1(v[g][i], sc) << (8 * i);
#pragma unroll
            for (int i = 0; i < 4; i++) hi |= (uint32_t)(uint8_t)quant1(v[g][4 + i], sc) << (8 * i);
            *(uint2*)(qr + 8 * (lane + 64 * g)) = make_uint2(lo, hi);
        }
}

// ------------------------------------------------------------------ group ---
// One 512-thread block per expert e, all blocks independent:
//  1. offsets[e] = the number of (token, slot) pairs routed to experts < e
//     (a count over all T * top_k ids);
//  2. the tokens that chose e, in ascending order, take the rows
//     offsets[e], offsets[e] + 1, ...: 512 tokens per round, a ballot per
//     wave and a prefix over the 8 waves give each its rank.
// The layout equals a serial walk over (expert, token). A token's top-k ids
// are distinct, so at most one of its slots names e.
__global__ __launch_bounds__(512) void moe_group_kernel(const int32_t* __restrict__ topk_id, int T,
                                                        int E, int top_k,
                                                        int32_t* __restrict__ offsets,
                                                        int32_t* __restrict__ row_token,
                                                        int32_t* __restrict__ pos_of_pair) {
    __shared__ int wcount[8];
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int P = T * top_k;
    // The first round's ids of this thread's token load together with the
    // count's, so every load of the block is in flight at once. Indices are
    // clamped, not branched around: a guarded load becomes a branch with a
    // wait of its own, one round trip per load.
    auto token_hit = [&](int t) {
        int hit = -1;
        const int tc = min(t, T - 1);
        for (int k0 = 0; k0 < top_k; k0 += 8) {
            int id[8];
#pragma unroll
            for (int j = 0; j < 8; j++) id[j] = topk_id[(int64_t)tc * top_k + min(k0 + j, top_k - 1)];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (t < T && k0 + j < top_k && id[j] == e) hit = k0 + j;
        }
        return hit;
    };
    int hit0 = token_hit(tid);
    int c = 0;
    for (int r0 = 0; r0 < P; r0 += 8 * 512) {
        int id[8];
#pragma unroll
        for (int j = 0; j < 8; j++) id[j] = topk_id[min(r0 + 8 * tid + j, P - 1)];
#pragma unroll
        for (int j = 0; j < 8; j++) c += (r0 + 8 * tid + j < P) & (id[j] < e);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
    if (lane == 0) wcount[wv] = c;
    __syncthreads();
    int run = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) run += wcount[k];
    if (tid == 0) {
        offsets[e] = run;
        if (e == E - 1) offsets[E] = P;
    }
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int t0 = 0; t0 < T; t0 += 512) {
        const int t = t0 + tid;
        const int hit = t0 == 0 ? hit0 : token_hit(t);
        const unsigned long long m = __ballot(hit >= 0);
        __syncthreads();   // wcount is free again
        if (lane == 0) wcount[wv] = __popcll(m);
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            before += k < wv ? wcount[k] : 0;
            total += wcount[k];
        }
        if (hit >= 0) {
            const int pos = run + before + __popcll(m & below);
            row_token[pos] = t;
            pos_of_pair[(int64_t)t * top_k + hit] = pos;
        }
        run += total;
    }
}

// ------------------------------------------------------- grouped W8A8 GEMM ---
struct GroupedParams {
    const int8_t* A;          // quantized activations, lda = K
    const int32_t* a_rows;    // gathered row ids (gate_up) or nullptr (down: rows = positions)
    const float* s_a;         // per A row (indexed by gathered id, or by position)
    const int8_t* W;          // [E][N][K]
    const float* s_w;         // [E][N]
    const int32_t* offsets;   // [E+1]
    float* C;                 // [rows][N] (row = position); with SwiGLU [rows][N / 2] of h
    unsigned* amax;           // SwiGLU: per position, max |h| as float bits (zeroed beforehand)
    int64_t a_bytes;          // extent of A (< 2^31: rows past a tile's count read as zeros)
    int N, K;
};

// Block (n-tile, expert) on the register-staged v6 engine (the expert layer
// streams its weights from HBM once): 64 x 128 tiles, 8 waves, 4 K steps of
// loads in flight per wave, 48 KB of LDS (two blocks per CU), A rows gathered
// through the expert's token list. The block walks its expert's row tiles, so
// each weight tile is streamed from HBM once per 64 tokens.
// SWIGLU (gate_up): the tile's 128 columns are gate rows c0 .. c0 + 63 and
// the matching up rows I + c0 .. I + c0 + 63 (I = N / 2), so the epilogue has
// both halves of h = silu(g) * u for 64 channels: it writes h (fp32, half the
// bytes of g and u) and raises the row's max |h| with an atomic max, which is
// exact and order-free; the requantization then needs no second look at g, u.
constexpr int MOE_WMT = 1, MOE_WNT = 1, MOE_D = 4;
using MoeTile = TileV6<MOE_WMT, MOE_WNT, MOE_D>;
constexpr int MOE_THREADS = 512;

// silu(g) * u with the deterministic exp (the host oracle evaluates the same
// operations, so h and its requantized bytes are bit-identical).
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * (1.0f / (1.0f + exp_det(-g))) * u;
}

template <int NK, bool SWIGLU>
__global__ __launch_bounds__(MOE_THREADS, 2) void moe_grouped_gemm_kernel(GroupedParams p) {
    extern __shared__ __attribute__((aligned(16))) int8_t lds_moe[];
    const int e = blockIdx.y;
    // n0: first weight row of the tile; SwiGLU tiles take 64 gate + 64 up rows
    const int n0 = SWIGLU ? blockIdx.x * (MoeTile::BN / 2) : blockIdx.x * MoeTile::BN;
    const int I = p.N / 2;
    const int beg = p.offsets[e], cnt = p.offsets[e + 1] - beg;
    const int8_t* W = p.W + ((int64_t)e * p.N + n0) * p.K;
    const float* sw = p.s_w + (int64_t)e * p.N;
    for (int m0 = 0; m0 < cnt; m0 += MoeTile::BM) {
        // Epilogue scales: thread r < BM fetches row r's activation scale (through
        // the token gather), thread BM + c fetches column c's weight scale,
        // before the main loop so the latency overlaps it. After the loop they
        // go through LDS, so the bounds-checked stores below consume only
        // LDS/VALU results and issue without waiting on one another.
        const int tid = threadIdx.x;
        float my_scale = 0.f;
        if (tid < MoeTile::BM) {
            const int pos = beg + min(m0 + tid, cnt - 1);
            my_scale = p.s_a[p.a_rows ? p.a_rows[pos] : pos];
        } else if (tid < MoeTile::BM + MoeTile::BN) {
            const int c = tid - MoeTile::BM;
            const int row = SWIGLU && c >= MoeTile::BN / 2 ? I + n0 + c - MoeTile::BN / 2 : n0 + c;
            my_scale = sw[min(row, p.N - 1)];
        }
        v16i acc[MOE_WMT][MOE_WNT];
        if (p.a_rows)
            mma_tile_v6<MOE_WMT, MOE_WNT, MOE_D, NK>(p.A, p.K, cnt - m0, (uint32_t)p.a_bytes, W, p.K, p.N - n0,
                                                     lds_moe, acc, p.a_rows + beg + m0,
                                                     SWIGLU ? I - MoeTile::BN / 2 : 0);
        else
            mma_tile_v6<MOE_WMT, MOE_WNT, MOE_D, NK>(p.A + (int64_t)(beg + m0) * p.K, p.K, cnt - m0,
                                                     (uint32_t)(p.a_bytes - (int64_t)(beg + m0) * p.K), W, p.K,
                                                     p.N - n0, lds_moe, acc);
        float* scl = (float*)lds_moe;   // the stages are free once every wave is past this barrier
        __syncthreads();
        if (tid < MoeTile::BM + MoeTile::BN) scl[tid] = my_scale;
        __syncthreads();
        if constexpr (SWIGLU) {
            // scaled tile -> LDS; then h of (row, channel), 4 channels per thread
            constexpr int TP = MoeTile::BN + 4;
            float* tile = scl + MoeTile::BM + MoeTile::BN;
            static_assert((MoeTile::BM + MoeTile::BN + MoeTile::BM * TP) * 4 <= MoeTile::LDS_BYTES,
                          "epilogue tile fits in the stages");
#pragma unroll
            for (int j = 0; j < MOE_WNT; j++) {
                const int c = v6_col<MOE_WNT>(j);
                const float swn = scl[MoeTile::BM + c];
#pragma unroll
                for (int i = 0; i < MOE_WMT; i++)
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int rl = v6_row<MOE_WMT>(i, v);
                        tile[rl * TP + c] = (float)acc[i][j][v] * scl[rl] * swn;
                    }
            }
            __syncthreads();
            constexpr int HC = MoeTile::BN / 2;          // channels per tile
#pragma unroll
            for (int it = 0; it < MoeTile::BM * (HC / 4) / MOE_THREADS; it++) {
                const int q = it * MOE_THREADS + tid, rl = q / (HC / 4), c4 = (q % (HC / 4)) * 4;
                const float4 g = *(const float4*)(tile + rl * TP + c4);
                const float4 u = *(const float4*)(tile + rl * TP + HC + c4);
                const float4 h = make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z),
                                             silu_mul(g.w, u.w));
                // max |h| over the row's 64 channels: 16 consecutive lanes
                float mx = fmaxf(fmaxf(fabsf(h.x), fabsf(h.y)), fmaxf(fabsf(h.z), fabsf(h.w)));
                mx = fmaxf(mx, dpp<DPP_XOR1>(mx));
                mx = fmaxf(mx, dpp<DPP_XOR2>(mx));
                mx = fmaxf(mx, dpp<DPP_HMIRROR>(mx));
                mx = fmaxf(mx, dpp<DPP_MIRROR>(mx));
                if (m0 + rl < cnt) {
                    const int64_t pos = beg + m0 + rl;
                    *(float4*)(p.C + pos * I + n0 + c4) = h;
                    if ((q % (HC / 4)) == 0) atomicMax(p.amax + pos, __float_as_uint(mx));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < MOE_WNT; j++) {
                const int c = v6_col<MOE_WNT>(j), n = n0 + c;
                const float swn = scl[MoeTile::BM + c];
#pragma unroll
                for (int i = 0; i < MOE_WMT; i++)
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int rl = v6_row<MOE_WMT>(i, v), r = m0 + rl;
                        const float val = (float)acc[i][j][v] * scl[rl] * swn;
                        if (r < cnt && n < p.N) p.C[(int64_t)(beg + r) * p.N + n] = val;
                    }
            }
        }
        __syncthreads();   // the next row tile reuses the LDS stages
    }
}

// Launches the instance for K = 128 * nk (1 <= nk <= MOE_MAX_NK).
constexpr int MOE_MAX_NK = 32;
template <int NK, bool SWIGLU>
static void launch_grouped(const GroupedParams& g, dim3 grid, int nk, hipStream_t st) {
    if constexpr (NK <= MOE_MAX_NK) {
        if (nk == NK) moe_grouped_gemm_kernel<NK, SWIGLU><<<grid, MOE_THREADS, MoeTile::LDS_BYTES, st>>>(g);
        else launch_grouped<NK + 1, SWIGLU>(g, grid, nk, st);
    }
}

// --------------------------------------------------------------- requant ---
// Requantization of h per row: s = max|h| / 127 (1 when 0), q = rint(h / s)
// clamped to +-127, the per-token quantizer's rule; max|h| comes from the
// gate_up epilogue's atomic max. One wave per row, 4 consecutive values per
// lane and step.
__global__ __launch_bounds__(256) void moe_requant_kernel(const float* __restrict__ h,
                                                          const unsigned* __restrict__ amax,
                                                          int8_t* __restrict__ q,
                                                          float* __restrict__ s, int rows, int I) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float am = __uint_as_float(amax[r]);
    const float4* h4 = (const float4*)(h + (int64_t)r * I);
    uint32_t* qr = (uint32_t*)(q + (int64_t)r * I);
    const int n4 = I / 4;
    // up to 256 float4 per round, all loaded before the scale is used (the
    // max and the row's values arrive together)
    for (int c0 = 0; c0 < n4; c0 += 256) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = h4[min(c0 + lane + 64 * u, n4 - 1)];   // clamped, not branched
        const float sc = am == 0.f ? 1.f : am / 127.0f;
        if (c0 == 0 && lane == 0) s[r] = sc;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int c = c0 + lane + 64 * u;
            if (c < n4)
                qr[c] = (uint32_t)(uint8_t)quant1(v[u].x, sc) | (uint32_t)(uint8_t)quant1(v[u].y, sc) << 8 |
                        (uint32_t)(uint8_t)quant1(v[u].z, sc) << 16 | (uint32_t)(uint8_t)quant1(v[u].w, sc) << 24;
        }
    }
}

// ---------------------------------------------------------------- combine ---
// Four consecutive columns per thread (H % 4 == 0), summed in k order with
// one fused multiply-add per term.
template <typename OT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ d,
                                                          const float* __restrict__ topk_w,
                                                          const int32_t* __restrict__ pos_of_pair,
                                                          OT* __restrict__ out, int T, int H,
                                                          int top_k) {
    const int t = blockIdx.y;
    const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= H) return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    // 8 slots per round: their positions and weights, then their rows, in flight together
    for (int k0 = 0; k0 < top_k; k0 += 8) {
        int pos[8];
        float wk[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {   // clamped indices: guarded loads would wait one by one
            const int pr = t * top_k + min(k0 + j, top_k - 1);
            pos[j] = pos_of_pair[pr];
            wk[j] = topk_w[pr];
        }
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = *(const float4*)(d + (int64_t)pos[j] * H + n);
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (k0 + j < top_k) {
                acc[0] = __builtin_fmaf(wk[j], v[j].x, acc[0]);
                acc[1] = __builtin_fmaf(wk[j], v[j].y, acc[1]);
                acc[2] = __builtin_fmaf(wk[j], v[j].z, acc[2]);
                acc[3] = __builtin_fmaf(wk[j], v[j].w, acc[3]);
            }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) out[(int64_t)t * H + n + e] = from_f32<OT>(acc[e]);
}

// --------------------------------------------------------------- workspace ---
struct MoeWs {
    float* topk_w;
    int32_t* topk_id;
    int32_t* offsets;
    int32_t* row_token;
    int32_t* pos_of_pair;
    int8_t* qx;
    float* sx;
    float* h;            // [P][I] SwiGLU output (fp32)
    unsigned* amax;      // [P] max |h| per row, float bits
    int8_t* qh;
    float* sh;
    float* d;
    size_t total;
};

static size_t al(size_t b) { return (b + 255) / 256 * 256; }

static MoeWs moe_layout(char* base, int T, int H, int I, int E, int k) {
    MoeWs w{};
    const size_t P = (size_t)T * k;
    size_t o = 0;
    auto take = [&](size_t bytes) { char* p = base ? base + o : nullptr; o += al(bytes); return p; };
    w.topk_w = (float*)take(P * 4);
    w.topk_id = (int32_t*)take(P * 4);
    w.offsets = (int32_t*)take((size_t)(E + 1) * 4);
    w.row_token = (int32_t*)take(P * 4);
    w.pos_of_pair = (int32_t*)take(P * 4);
    w.qx = (int8_t*)take((size_t)T * H);
    w.sx = (float*)take((size_t)T * 4);
    w.h = (float*)take(P * I * 4);
    w.amax = (unsigned*)take(P * 4);
    w.qh = (int8_t*)take(P * I);
    w.sh = (float*)take(P * 4);
    w.d = (float*)take(P * H * 4);
    w.total = o;
    return w;
}

int moe_route(const float* logits, float* topk_w, int32_t* topk_id, int T, int E, int top_k,
              int renorm, hipStream_t st) {
    PIO_REQUIRE(logits && topk_w && topk_id, "moe_route: null pointer");
    PIO_REQUIRE(T >= 0 && E >= 1 && E <= ROUTE_MAX_E, "moe_route: need 1 <= E <= %d", ROUTE_MAX_E);
    PIO_REQUIRE(top_k >= 1 && top_k <= E && top_k <= 64, "moe_route: bad top_k %d", top_k);
    if (T == 0) return PIO_OK;
    moe_route_kernel<<<ceil_div(T, 4), 256, 0, st>>>(logits, topk_w, topk_id, T, E, top_k, renorm);
    PIO_LAUNCHED();
    return PIO_OK;
}

int moe_w8a8(const void* x, int x_dtype, const float* logits, const int8_t* w_gu,
             const float* s_gu, const int8_t* w_down, const float* s_down, void* out,
             int out_dtype, int T, int H, int I, int E, int top_k, int renorm, void* ws,
             hipStream_t st) {
    PIO_REQUIRE(x && logits && w_gu && s_gu && w_down && s_down && out, "moe: null pointer");
    PIO_REQUIRE(T >= 0 && H > 0 && I > 0, "moe: bad shape");
    PIO_REQUIRE(H % 128 == 0 && I % 128 == 0, "moe: H=%d and I=%d must be multiples of 128", H, I);
    PIO_REQUIRE(H <= 128 * MOE_MAX_NK && I <= 128 * MOE_MAX_NK, "moe: H=%d and I=%d must be <= %d", H,
                I, 128 * MOE_MAX_NK);
    PIO_REQUIRE(out_dtype == PIO_F32 || out_dtype == PIO_F16, "moe: out must be fp32 or fp16");
    PIO_REQUIRE(x_dtype == PIO_F32 || x_dtype == PIO_F16, "moe: x must be fp32 or fp16");
    PIO_REQUIRE(E >= 1 && E <= ROUTE_MAX_E && top_k >= 1 && top_k <= E && top_k <= 64,
                "moe: E=%d experts (<= %d) and top_k=%d (<= min(E, 64))", E, ROUTE_MAX_E, top_k);
    PIO_REQUIRE((int64_t)T * top_k <= INT32_MAX / 4, "moe: T * top_k too large");
    PIO_REQUIRE((int64_t)T * H < (1ll << 31) && (int64_t)T * top_k * I < (1ll << 31),
                "moe: the quantized activations (T*H, T*top_k*I bytes) must stay below 2 GiB");
    PIO_REQUIRE(H <= 64 * 8 * ROUTE_XG, "moe: H=%d must be <= %d", H, 64 * 8 * ROUTE_XG);
    PIO_REQUIRE(aligned16(w_gu) && aligned16(w_down) && aligned16(x),
                "moe: x and the weights must be 16-byte aligned");
    if (T == 0) return PIO_OK;
    Scratch own;
    if (!ws) {
        PIO_TRY(own.get(moe_layout(nullptr, T, H, I, E, top_k).total, st));
        ws = own.ptr;
    }
    MoeWs w = moe_layout((char*)ws, T, H, I, E, top_k);
    const int P = T * top_k;

    if (x_dtype == PIO_F32)
        moe_route_quant_kernel<float><<<ceil_div(T, 2), 256, 0, st>>>(
            logits, (const float*)x, H, w.topk_w, w.topk_id, w.qx, w.sx, T, E, top_k, renorm, w.amax);
    else
        moe_route_quant_kernel<_Float16><<<ceil_div(T, 2), 256, 0, st>>>(
            logits, (const _Float16*)x, H, w.topk_w, w.topk_id, w.qx, w.sx, T, E, top_k, renorm, w.amax);
    PIO_LAUNCHED();
    moe_group_kernel<<<E, 512, 0, st>>>(w.topk_id, T, E, top_k, w.offsets, w.row_token,
                                        w.pos_of_pair);
    PIO_LAUNCHED();

    GroupedParams g{};
    g.A = w.qx; g.a_rows = w.row_token; g.s_a = w.sx;
    g.W = w_gu; g.s_w = s_gu; g.offsets = w.offsets; g.C = w.h; g.amax = w.amax;
    g.N = 2 * I; g.K = H; g.a_bytes = (int64_t)T * H;
    launch_grouped<1, true>(g, dim3(I / (MoeTile::BN / 2), E), H / 128, st);
    PIO_LAUNCHED();

    moe_requant_kernel<<<ceil_div(P, 4), 256, 0, st>>>(w.h, w.amax, w.qh, w.sh, P, I);
    PIO_LAUNCHED();

    GroupedParams d{};
    d.A = w.qh; d.a_rows = nullptr; d.s_a = w.sh;
    d.W = w_down; d.s_w = s_down; d.offsets = w.offsets; d.C = w.d;
    d.N = H; d.K = I; d.a_bytes = (int64_t)P * I;
    launch_grouped<1, false>(d, dim3(ceil_div(H, MoeTile::BN), E), I / 128, st);
    PIO_LAUNCHED();

    dim3 cg(ceil_div(H, 1024), T);
    if (out_dtype == PIO_F32)
        moe_combine_kernel<float><<<cg, 256, 0, st>>>(w.d, w.topk_w, w.pos_of_pair, (float*)out, T, H, top_k);
    else
        moe_combine_kernel<_Float16><<<cg, 256, 0, st>>>(w.d, w.topk_w, w.pos_of_pair, (_Float16*)out, T, H, top_k);
    PIO_LAUNCHED();
    return PIO_OK;
}

}  // namespace pio

using namespace pio;

PIO_EXPORT size_t pio_moe_workspace(int T, int H, int I, int E, int top_k) {
    return moe_layout(nullptr, T, H, I, E, top_k).total;
}

PIO_EXPORT int pio_moe_route(const float* logits, float* topk_w, int32_t* topk_id, int T, int E,
                             int top_k, int renorm, void* stream) {
    return moe_route(logits, topk_w, topk_id, T, E, top_k, renorm, pick_stream(stream));
}

PIO_EXPORT int pio_moe_w8a8(const void* x, int x_dtype, const float* logits, const int8_t* w_gu,
                            const float* s_gu, const int8_t* w_down, const float* s_down, void* out,
                            int out_dtype, int T, int H, int I, int E, int top_k, int renorm,
                            void* workspace, void* stream) {
    return moe_w8a8(x, x_dtype, logits, w_gu, s_gu, w_down, s_down, out, out_dtype, T, H, I, E,
                    top_k, renorm, workspace, pick_stream(stream));
}

PIO_EXPORT int tensor_moe_w8a8_status(Tensor* x, Tensor* logits, Tensor* w_gu, Tensor* s_gu,
                                      Tensor* w_down, Tensor* s_down, int top_k, int renorm,
                                      Tensor* out) {
    PIO_TRY(check_device_tensor(x, "moe x"));
    PIO_TRY(check_device_tensor(logits, "moe logits"));
    PIO_TRY(check_device_tensor(w_gu, "moe w_gu"));
    PIO_TRY(check_device_tensor(s_gu, "moe s_gu"));
    PIO_TRY(check_device_tensor(w_down, "moe w_down"));
    PIO_TRY(check_device_tensor(s_down, "moe s_down"));
    PIO_TRY(check_device_tensor(out, "moe out"));
    PIO_REQUIRE(w_gu->ndim == 3 && w_down->ndim == 3, "moe: expert weights must be 3-D");
    const int E = w_gu->shape[0], I2 = w_gu->shape[1], H = w_gu->shape[2];
    PIO_REQUIRE(I2 % 2 == 0, "moe: gate_up rows must be even");
    const int I = I2 / 2;
    PIO_REQUIRE(w_down->shape[0] == E && w_down->shape[1] == H && w_down->shape[2] == I,
                "moe: w_down must be [%d,%d,%d]", E, H, I);
    PIO_REQUIRE(s_gu->size == E * I2 && s_down->size == E * H, "moe: scale sizes mismatch");
    PIO_REQUIRE(last_dim(x) == H, "moe: x last dim must be %d", H);
    const int T = x->size / H;
    PIO_REQUIRE(logits->size == T * E, "moe: logits must be [%d,%d]", T, E);
    PIO_REQUIRE(out->size == T * H, "moe: out must be [%d,%d]", T, H);
    return moe_w8a8(x->data, tensor_dtype_of(x), logits->data, (const int8_t*)w_gu->data,
                    s_gu->data, (const int8_t*)w_down->data, s_down->data, out->data,
                    tensor_dtype_of(out), T, H, I, E, top_k, renorm, nullptr, current_stream());
}
PIO_EXPORT void tensor_moe_w8a8(Tensor* x, Tensor* logits, Tensor* w_gu, Tensor* s_gu,
                                Tensor* w_down, Tensor* s_down, int top_k, int renorm,
                                Tensor* out) {
    tensor_moe_w8a8_status(x, logits, w_gu, s_gu, w_down, s_down, top_k, renorm, out);
}
