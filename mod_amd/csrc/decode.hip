// Int8 Qwen3-style decoder, batch 1 greedy (see pio_qwen3_* in tensor_rocm.h).
//
// One decode step is a fixed sequence of kernels whose only varying inputs --
// the position and the token ids -- live in device memory, so the whole step is
// captured once as a HIP graph and replayed per token with no host round trip:
//
//   embed -> L x [ rmsnorm+W8 qkv+bias+RoPE+kv-write -> attention ->
//                  W8 o(+residual) -> rmsnorm+W8 gate_up+SwiGLU -> W8 down(+residual) ]
//         -> rmsnorm+W8 lm_head+block argmax -> finish (argmax, next id, pos += 1)
//
// The W8 GEMVs are the HBM-bound kernels (596 MB of int8 weights per token at
// the Qwen3-0.6B shape); everything else is latency. Semantics follow the
// reference model code with its defects fixed: causal attention over the whole
// cache (tensor_ops.c:536-578 attends only to matching positions and has no
// mask), GQA without materializing repeated heads (architecture.py:57-66),
// residual adds kept (architecture.py:129-132 drops one on CPU), RoPE on the
// key heads' own count (tensor_ops.c:390 indexes k with q's head count).
#include "decode.hpp"

#include <math.h>
#include <algorithm>
#include <vector>

namespace pio {


// x = embed[ids[pos]] (an out-of-range id reads row 0, as tensor_embed,
// tensor_ops.c:663-671).
__global__ void dec_embed_kernel(const float* __restrict__ embed, const int32_t* __restrict__ ids,
                                 const int32_t* __restrict__ state, float* __restrict__ x, int H,
                                 int V, int max_seq) {
    const int pos = state[0];
    if (pos >= max_seq) return;
    int id = ids[pos];
    if (id < 0 || id >= V) id = 0;
    for (int i = threadIdx.x; i < H; i += blockDim.x) x[i] = embed[(int64_t)id * H + i];
}

// ----------------------------------------------------------- fused GEMV ---
// One kernel template for every decode linear: y = W8(x) with
//   prologue  optional RMSNorm: x' = x * g, and the row sum of x^2 -- each wave
//             covers all of x, so the norm costs one extra wave reduction;
//             the scale 1/sqrt(mean(x^2)+eps) is applied to the dot products
//             (tensor_ops.c:369-383 applies it to x first; same value up to rounding);
//   epilogue  PLAIN y = v; RESID y += v (y is the residual stream);
//             ROPE   rows (n, n+D/2) of one head: bias, rotate-half RoPE at pos
//                    (tensor_ops.c:384-415 formula), q -> q_out, k/v -> cache row pos;
//             SWIGLU rows (i, i+I): act[i] = silu(g)*u (tensor_ops.c:588-604);
//             LOGITS y = v and a per-block argmax key (value, lowest index).
// A wave owns R rows; paired modes give it R/2 pairs (n, n+half).
enum { EPI_PLAIN = 0, EPI_RESID = 1, EPI_ROPE = 2, EPI_SWIGLU = 3, EPI_LOGITS = 4 };

struct DecGemv {
    const float* x;
    const float* norm_w;   // RMSNorm weight or nullptr
    float eps;
    const int8_t* W;
    const float* s_w;
    const float* bias;
    int N, K, half;
    float* y;
    const float* cos_t;
    const float* sin_t;
    const int32_t* state;
    float* q_out;
    void* kc;              // KV cache rows of this layer: fp32, or fp16 when kv16
    void* vc;
    int kv16;
    int nq, nkv, max_seq;
    unsigned long long* part_keys;
    // o_proj prologue: merge the attention splits into x (x must be nullptr)
    const float* att_o;    // [S][nq*D] unnormalized sum_t p v per split
    const float* att_ml;   // [S][nq][2] (max, sum) per split
};

typedef int v4i_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot16i8(const float (&x)[16], v4i_t w, float acc) {
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int u = w[d];
        acc = fmaf(x[4 * d + 0], (float)(int8_t)(u), acc);
        acc = fmaf(x[4 * d + 1], (float)(int8_t)(u >> 8), acc);
        acc = fmaf(x[4 * d + 2], (float)(int8_t)(u >> 16), acc);
        acc = fmaf(x[4 * d + 3], (float)(int8_t)(u >> 24), acc);
    }
    return acc;
}

// Two elements (i, i + half) of a KV cache row starting at element `row`.
// fp16 rows are paired: slot 2i holds dim i and slot 2i + 1 dim i + half, so
// the pair is one dword store (2-byte stores slowed the later loads of the
// lines they touched ~4x); fp32 rows are in dimension order.
__device__ __forceinline__ void kv_store(void* base, int64_t row, int i, int half, float a, float b,
                                         int kv16) {
    if (kv16) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        h2 v;
        v[0] = (_Float16)a;
        v[1] = (_Float16)b;
        *(h2*)((_Float16*)base + row + 2 * i) = v;
    } else {
        float* d = (float*)base + row;
        d[i] = a;
        d[i + half] = b;
    }
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i);
}

// KC = number of 1024-wide K chunks a lane covers (K <= KC * 1024). The first
// row group's weight loads are issued before the x prologue so their HBM
// latency overlaps it; x (times the norm weight) is staged once per block in
// LDS; waves that own several row groups prefetch the next group's weights
// before reducing the current one.
template <int EPI, int R, int KC>
__global__ __launch_bounds__(256) void dec_gemv_kernel(DecGemv p) {
    constexpr bool PAIRED = (EPI == EPI_ROPE || EPI == EPI_SWIGLU);
    __shared__ __attribute__((aligned(16))) float xs[KC * 1024];
    __shared__ float red[4];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int K = p.K, N = p.N;
    const int waves = gridDim.x * 4;
    const int groups = (N + R - 1) / R;

    auto rows_of = [&](int g, int (&row)[R], bool (&ok)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            int n;
            if (PAIRED) {
                const int pi = g * (R / 2) + r / 2;
                n = (pi / p.half) * 2 * p.half + (pi % p.half) + (r & 1) * p.half;
            } else {
                n = g * R + r;
            }
            ok[r] = n < N;
            row[r] = ok[r] ? n : N - 1;
        }
    };
    auto load_w = [&](const int (&row)[R], v4i_t (&w)[KC][R]) {
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * 1024 + lane * 16;
#pragma unroll
            for (int r = 0; r < R; r++)
                w[c][r] = k < K ? __builtin_nontemporal_load((const v4i_t*)(p.W + (int64_t)row[r] * K + k))
                                : v4i_t{0, 0, 0, 0};
        }
    };

    // A group's epilogue operands (scale, bias; for RoPE the angles at the
    // current position) are loaded with its weights, not after its math: there
    // they were dependent round trips at the end of every group (the position,
    // then cos / sin). Indices are clamped so every load is issued.
    constexpr int RP = R / 2 > 0 ? R / 2 : 1;
    int pos = 0;
    if constexpr (EPI == EPI_ROPE) pos = p.state[0];   // first, so the angle loads wait for it alone
    const int tpos = EPI == EPI_ROPE ? min(pos, p.max_seq - 1) : 0;
    auto epi_ops = [&](const int (&row)[R], float (&sw)[R], float (&bb)[R], float (&cs)[RP], float (&sn)[RP]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            sw[r] = p.s_w[row[r]];
            bb[r] = (p.bias ? p.bias : p.s_w)[row[r]];
        }
        if constexpr (EPI == EPI_ROPE) {
#pragma unroll
            for (int j = 0; j < RP; j++) {
                const int i = row[2 * j] % (2 * p.half);
                const int64_t t = (int64_t)tpos * p.half + min(i, p.half - 1);
                cs[j] = p.cos_t[t];
                sn[j] = p.sin_t[t];
            }
        }
    };

    int g = blockIdx.x * 4 + wid;
    int row[R];
    bool ok[R];
    v4i_t w[KC][R];
    float sw[R], bb[R], cs[RP], sn[RP];
    rows_of(g < groups ? g : 0, row, ok);
    if (g < groups) {
        load_w(row, w);
        epi_ops(row, sw, bb, cs, sn);
    }

    // Block prologue: xs = x * norm_w (or x, or the merged attention output),
    // and the RMSNorm scale. The loop over K in steps of 1024 issues the loads
    // of several steps (4 of x, 2 of the split merge) before it uses any, at
    // clamped indices: one step at a time, each step's loads waited for the
    // previous step's math (two extra round trips at K = 3072).
    float ss = 0.f;
    auto put = [&](int k, float4 a, float4 gw) {
        if (p.norm_w) {
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
            a.x *= gw.x; a.y *= gw.y; a.z *= gw.z; a.w *= gw.w;
        }
        *(float4*)&xs[k] = a;
    };
    if (p.att_o) {
        // softmax-merge of the splits for q head k/128, in split order
        const int nh = K >> 7;
        for (int k0 = threadIdx.x * 4; k0 < K; k0 += 2048) {
            float m[2][ATT_SPLITS], l[2][ATT_SPLITS];
            float4 o[2][ATT_SPLITS], gw[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int k = min(k0 + 1024 * u, K - 4), h = k >> 7;
#pragma unroll
                for (int i = 0; i < ATT_SPLITS; i++) {
                    m[u][i] = p.att_ml[(i * nh + h) * 2];
                    l[u][i] = p.att_ml[(i * nh + h) * 2 + 1];
                    o[u][i] = *(const float4*)(p.att_o + (int64_t)i * K + k);
                }
                gw[u] = p.norm_w ? *(const float4*)(p.norm_w + k) : make_float4(1.f, 1.f, 1.f, 1.f);
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                if (k0 + 1024 * u >= K) continue;
                float M = m[u][0];
#pragma unroll
                for (int i = 1; i < ATT_SPLITS; i++) M = fmaxf(M, m[u][i]);
                float den = 0.f;
                float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int i = 0; i < ATT_SPLITS; i++) {
                    const float f = m[u][i] == -INFINITY ? 0.f : expf(m[u][i] - M);
                    den += f * l[u][i];
                    a.x += f * o[u][i].x; a.y += f * o[u][i].y; a.z += f * o[u][i].z; a.w += f * o[u][i].w;
                }
                const float inv = 1.0f / den;
                a.x *= inv; a.y *= inv; a.z *= inv; a.w *= inv;
                put(k0 + 1024 * u, a, gw[u]);
            }
        }
    } else {
        for (int k0 = threadIdx.x * 4; k0 < K; k0 += 4096) {
            float4 a[4], gw[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int k = min(k0 + 1024 * u, K - 4);
                a[u] = *(const float4*)(p.x + k);
                gw[u] = p.norm_w ? *(const float4*)(p.norm_w + k) : make_float4(1.f, 1.f, 1.f, 1.f);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (k0 + 1024 * u < K) put(k0 + 1024 * u, a[u], gw[u]);
        }
    }
    float nscale = 1.f;
    if (p.norm_w) {
        ss = wave_sum(ss);
        if (lane == 0) red[wid] = ss;
    }
    __syncthreads();
    if (p.norm_w) nscale = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + p.eps);

    unsigned long long best = 0ull;
    while (g < groups) {
        const int gn = g + waves;
        int rown[R];
        bool okn[R];
        v4i_t wn[KC][R];
        float swn[R], bbn[R], csn[RP], snn[RP];
        if (gn < groups) {
            rows_of(gn, rown, okn);
            load_w(rown, wn);
            epi_ops(rown, swn, bbn, csn, snn);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * 1024 + lane * 16;
            if (k < K) {
                float xv[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 a = *(const float4*)&xs[k + 4 * i];
                    xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
                }
#pragma unroll
                for (int r = 0; r < R; r++) acc[r] = dot16i8(xv, w[c][r], acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
        float v[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            v[r] = acc[r] * sw[r] * nscale;
            if (p.bias) v[r] += bb[r];
        }

        if (EPI == EPI_PLAIN || EPI == EPI_RESID || EPI == EPI_LOGITS) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (lane == r && ok[r]) {
                    if (EPI == EPI_RESID) p.y[row[r]] += v[r];
                    else p.y[row[r]] = v[r];
                }
        }
        if (EPI == EPI_LOGITS) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (ok[r]) {
                    const unsigned long long kk = argmax_key(v[r], row[r]);
                    best = kk > best ? kk : best;
                }
        }
        if (EPI == EPI_SWIGLU) {
#pragma unroll
            for (int j = 0; j < R / 2; j++)
                if (lane == j && ok[2 * j]) {
                    const float gg = v[2 * j], u = v[2 * j + 1];
                    p.y[row[2 * j]] = gg * (1.0f / (1.0f + expf(-gg))) * u;
                }
        }
        if (EPI == EPI_ROPE) {
            const int D = 2 * p.half;
#pragma unroll
            for (int j = 0; j < R / 2; j++) {
                if (lane != j || !ok[2 * j] || pos >= p.max_seq) continue;
                const int n0 = row[2 * j];
                const int head = n0 / D, i = n0 % D;
                const float re = v[2 * j], im = v[2 * j + 1];
                if (head < p.nq + p.nkv) {
                    const float c = cs[j], sj = sn[j];
                    const float o0 = re * c - im * sj, o1 = re * sj + im * c;
                    if (head < p.nq) {
                        float* dst = p.q_out + (int64_t)head * D;
                        dst[i] = o0;
                        dst[i + p.half] = o1;
                    } else {
                        kv_store(p.kc, ((int64_t)(head - p.nq) * p.max_seq + pos) * D, i, p.half, o0, o1, p.kv16);
                    }
                } else {
                    kv_store(p.vc, ((int64_t)(head - p.nq - p.nkv) * p.max_seq + pos) * D, i, p.half, re, im,
                             p.kv16);
                }
            }
        }
        if (gn >= groups) break;
#pragma unroll
        for (int r = 0; r < R; r++) { row[r] = rown[r]; ok[r] = okn[r]; }
#pragma unroll
        for (int c = 0; c < KC; c++)
#pragma unroll
            for (int r = 0; r < R; r++) w[c][r] = wn[c][r];
#pragma unroll
        for (int r = 0; r < R; r++) { sw[r] = swn[r]; bb[r] = bbn[r]; }
#pragma unroll
        for (int j = 0; j < RP; j++) { cs[j] = csn[j]; sn[j] = snn[j]; }
        g = gn;
    }
    if (EPI == EPI_LOGITS) {
        __shared__ unsigned long long wbest[4];
        if (lane == 0) wbest[wid] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int i = 1; i < 4; i++) best = wbest[i] > best ? wbest[i] : best;
            p.part_keys[blockIdx.x] = best;
        }
    }
}

// ------------------------------------------------------------ attention ---
// Causal GQA decode attention, split ATT_SPLITS ways over the L = pos+1 cached
// positions: block (s, kv head) takes positions [s*c, s*c + c), c = ceil(L/S),
// for the G = nq/nkv query heads sharing that KV head (each K/V row is read
// once per step), and writes unnormalized partials (sum_t p v, max, sum).
// The o_proj GEMV that consumes them merges the splits in split order in its
// block prologue, so no block waits on another and no cache flush is needed.
//   scores  8 threads per key row (16 dims each), 32 rows per pass;
//   values  32 dim-groups (float4) x 8 position-groups, LDS reduction.
constexpr int ATT_MAX_G = 4;

// Four consecutive cache elements as fp32.
__device__ __forceinline__ float4 kv_ld4(const float* p) { return *(const float4*)p; }
__device__ __forceinline__ float4 kv_ld4(const _Float16* p) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = *(const h4*)p;
    return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

template <typename KT>
__global__ __launch_bounds__(256) void dec_attn_kernel(
    const float* __restrict__ q, const KT* __restrict__ kc, const KT* __restrict__ vc,
    const int32_t* __restrict__ state, float* __restrict__ att_o, float* __restrict__ att_ml,
    int nq, int nkv, int max_seq, float scale) {
    constexpr int D = 128;
    extern __shared__ __attribute__((aligned(16))) float att_lds[];
    const int G = nq / nkv;
    const int cmax = (max_seq + ATT_SPLITS - 1) / ATT_SPLITS;
    float* sc = att_lds;                              // [G][cmax]
    float* po = att_lds + G * cmax;                   // [8][G][D]
    __shared__ float red[ATT_MAX_G][2][4];
    const int pos = state[0];
    if (pos >= max_seq) return;
    const int L = pos + 1;
    const int s = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int c = (L + ATT_SPLITS - 1) / ATT_SPLITS;
    const int t0 = s * c, n = min(c, L - t0);
    if (n <= 0) {
        // empty split: contributes exp(-inf) = 0 to the merge
        if (tid < G * D) att_o[(int64_t)s * nq * D + (int64_t)kvh * G * D + tid] = 0.f;
        if (tid < G) {
            att_ml[((int64_t)s * nq + kvh * G + tid) * 2] = -INFINITY;
            att_ml[((int64_t)s * nq + kvh * G + tid) * 2 + 1] = 0.f;
        }
        return;
    }
    const KT* kb = kc + ((int64_t)kvh * max_seq + t0) * D;
    const KT* vb = vc + ((int64_t)kvh * max_seq + t0) * D;
    const float* qg = q + (int64_t)kvh * G * D;
    // fp16 rows are paired (kv_store): storage slot s holds dim s / 2 + 64 (s & 1)
    constexpr bool PAIR = sizeof(KT) == 2;
    auto dim_of = [](int slot) { return PAIR ? (slot >> 1) + 64 * (slot & 1) : slot; };
    // values: thread (dg, pg) = (tid % 32, tid / 32) owns dims 4 dg .. 4 dg + 3
    // of positions pg + 8 u (+ 32 per pass). The first pass's values load with
    // the keys (both depend only on pos): one memory round trip fewer than
    // loading them after the softmax. Rows past the split's end are clamped.
    const int dg = tid & 31, pg = tid >> 5;
    float4 vv0[4];
#pragma unroll
    for (int u = 0; u < 4; u++) vv0[u] = kv_ld4(vb + (int64_t)min(pg + 8 * u, n - 1) * D + 4 * dg);

    {
        const int part = tid & 7, sub = tid >> 3;
        float qv[ATT_MAX_G][16];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++)
#pragma unroll
            for (int i = 0; i < 16; i++)   // q in the rows' slot order; heads past G re-read the last
                qv[h][i] = qg[min(h, G - 1) * D + dim_of(part * 16 + i)];
        for (int tb = 0; tb < n; tb += 64) {
            // rows past the split's end load its last row (clamped, no branch:
            // a guarded load waits for the previous one); their scores are not
            // stored
            float kv[2][16];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = min(tb + sub + 32 * u, n - 1);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 a = kv_ld4(kb + (int64_t)t * D + part * 16 + 4 * i);
                    kv[u][4 * i] = a.x; kv[u][4 * i + 1] = a.y; kv[u][4 * i + 2] = a.z; kv[u][4 * i + 3] = a.w;
                }
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = tb + sub + 32 * u;
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++) {
                    if (h >= G) continue;
                    float d = 0.f;
#pragma unroll
                    for (int i = 0; i < 16; i++) d += qv[h][i] * kv[u][i];
                    d += __shfl_xor(d, 1, 64);
                    d += __shfl_xor(d, 2, 64);
                    d += __shfl_xor(d, 4, 64);
                    if (part == 0 && t < n) sc[h * cmax + t] = d * scale;
                }
            }
        }
    }
    __syncthreads();
    for (int h = 0; h < G; h++) {
        float m = -INFINITY;
        for (int t = tid; t < n; t += 256) m = fmaxf(m, sc[h * cmax + t]);
        m = wave_max(m);
        if (lane == 0) red[h][0][wid] = m;
    }
    __syncthreads();
    for (int h = 0; h < G; h++) {
        const float m = fmaxf(fmaxf(red[h][0][0], red[h][0][1]), fmaxf(red[h][0][2], red[h][0][3]));
        float l = 0.f;
        for (int t = tid; t < n; t += 256) {
            const float e = expf(sc[h * cmax + t] - m);
            sc[h * cmax + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) red[h][1][wid] = l;
    }
    __syncthreads();
    {
        float4 o[ATT_MAX_G];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) o[h] = make_float4(0.f, 0.f, 0.f, 0.f);
        auto accum = [&](int tb, const float4 (&vv)[4]) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int t = tb + 8 * u;
                if (t >= n) continue;
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++) {
                    if (h >= G) continue;
                    const float pt = sc[h * cmax + t];
                    o[h].x += pt * vv[u].x; o[h].y += pt * vv[u].y; o[h].z += pt * vv[u].z; o[h].w += pt * vv[u].w;
                }
            }
        };
        accum(pg, vv0);
        for (int tb = pg + 32; tb < n; tb += 32) {
            float4 vv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) vv[u] = kv_ld4(vb + (int64_t)min(tb + 8 * u, n - 1) * D + 4 * dg);
            accum(tb, vv);
        }
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++)
            if (h < G) *(float4*)&po[(pg * G + h) * D + 4 * dg] = o[h];
    }
    __syncthreads();
    if (tid < G * D) {
        const int h = tid / D, d = tid % D;
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) o += po[(i * G + h) * D + (PAIR ? (d < 64 ? 2 * d : 2 * (d - 64) + 1) : d)];
        att_o[(int64_t)s * nq * D + (int64_t)(kvh * G + h) * D + d] = o;
    }
    if (tid < G) {
        att_ml[((int64_t)s * nq + kvh * G + tid) * 2] =
            fmaxf(fmaxf(red[tid][0][0], red[tid][0][1]), fmaxf(red[tid][0][2], red[tid][0][3]));
        att_ml[((int64_t)s * nq + kvh * G + tid) * 2 + 1] =
            red[tid][1][0] + red[tid][1][1] + red[tid][1][2] + red[tid][1][3];
    }
}

// Argmax over the lm_head blocks' keys (reference tie rule: first maximum,
// tensor_ops.c:649-662), then ids[pos+1] = argmax unless pos+1 is a prompt
// position, and pos += 1.
__global__ __launch_bounds__(1024) void dec_finish_kernel(int32_t* state,
                                                          const unsigned long long* part_keys,
                                                          int nparts, int32_t* ids, int max_seq) {
    __shared__ unsigned long long wb[16];
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) best = part_keys[i] > best ? part_keys[i] : best;
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
    }
    if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) best = wb[i] > best ? wb[i] : best;
    const int pos = state[0];
    if (pos >= max_seq) return;
    const int id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
    if (pos + 1 >= state[1]) ids[pos + 1] = id;
    state[2] = id;
    state[0] = pos + 1;
}

// Every launch gives each wave one row group (grid covers N); the kernel also
// supports fewer blocks, whose waves then stride over the row groups.

template <int EPI, int R>
static int launch_dec_gemv(const DecGemv& p, int blocks, hipStream_t st) {
    switch ((p.K + 1023) / 1024) {
    case 1: dec_gemv_kernel<EPI, R, 1><<<blocks, 256, 0, st>>>(p); break;
    case 2: dec_gemv_kernel<EPI, R, 2><<<blocks, 256, 0, st>>>(p); break;
    case 3: dec_gemv_kernel<EPI, R, 3><<<blocks, 256, 0, st>>>(p); break;
    case 4: dec_gemv_kernel<EPI, R, 4><<<blocks, 256, 0, st>>>(p); break;
    default: return set_error(PIO_ERR_UNSUPPORTED, "decoder GEMV: K=%d > 4096", p.K);
    }
    PIO_LAUNCHED();
    return PIO_OK;
}

// One decode step: 1 + 5 per layer + 2 launches.
static int enqueue_step(Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    const int H = c.hidden, D = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, I = c.intermediate;
    const int nqkv = (nq + 2 * nkv) * D;
    hipStream_t st = d->st;
    dec_embed_kernel<<<1, 256, 0, st>>>(d->embed, d->ids, d->state, d->x, H, c.vocab, c.max_seq);
    PIO_LAUNCHED();
    const float scale = 1.0f / sqrtf((float)D);
    DecGemv base{};
    base.eps = c.rms_eps;
    base.cos_t = d->cos_t;
    base.sin_t = d->sin_t;
    base.state = d->state;
    base.nq = nq;
    base.nkv = nkv;
    base.max_seq = c.max_seq;
    for (int l = 0; l < c.n_layers; l++) {
        const pio_qwen3_layer& L = d->layers[l];
        const int64_t lkv = (int64_t)l * nkv * c.max_seq * D * (d->kv16 ? 2 : 4);   // bytes
        void* kc = (char*)d->kc + lkv;
        void* vc = (char*)d->vc + lkv;
        // qkv: rmsnorm(x) -> W8 + bias -> RoPE -> q, k/v cache
        DecGemv g = base;
        g.x = d->x; g.norm_w = L.in_norm; g.W = L.w_qkv; g.s_w = L.s_qkv; g.bias = L.b_qkv;
        g.N = nqkv; g.K = H; g.half = D / 2; g.q_out = d->q; g.kc = kc; g.vc = vc; g.kv16 = d->kv16;
        PIO_TRY((launch_dec_gemv<EPI_ROPE, 2>(g, ceil_div(g.N, 8), st)));
        if (d->kv16)
            dec_attn_kernel<_Float16><<<dim3(ATT_SPLITS, nkv), 256, d->att_lds, st>>>(
                d->q, (const _Float16*)kc, (const _Float16*)vc, d->state, d->att_o, d->att_ml, nq, nkv,
                c.max_seq, scale);
        else
            dec_attn_kernel<float><<<dim3(ATT_SPLITS, nkv), 256, d->att_lds, st>>>(
                d->q, (const float*)kc, (const float*)vc, d->state, d->att_o, d->att_ml, nq, nkv,
                c.max_seq, scale);
        PIO_LAUNCHED();
        // o_proj: x += W8(attn)
        g = base;
        g.att_o = d->att_o; g.att_ml = d->att_ml;
        g.W = L.w_o; g.s_w = L.s_o; g.N = H; g.K = nq * D; g.y = d->x;
        PIO_TRY((launch_dec_gemv<EPI_RESID, 1>(g, ceil_div(g.N, 4), st)));
        // gate_up: rmsnorm(x) -> W8 -> silu(g)*u
        g = base;
        g.x = d->x; g.norm_w = L.post_norm; g.W = L.w_gu; g.s_w = L.s_gu; g.N = 2 * I; g.K = H;
        g.half = I; g.y = d->act;
        PIO_TRY((launch_dec_gemv<EPI_SWIGLU, 2>(g, ceil_div(g.N, 8), st)));
        // down: x += W8(act)
        g = base;
        g.x = d->act; g.W = L.w_down; g.s_w = L.s_down; g.N = H; g.K = I; g.y = d->x;
        PIO_TRY((launch_dec_gemv<EPI_RESID, 1>(g, ceil_div(g.N, 4), st)));
    }
    return enqueue_lm(d);
}

// The step's tail: logits = W8_lm_head(rmsnorm(x) * w_final), the argmax, and
// finish (ids[pos + 1] unless still inside the prompt, pos += 1).
int enqueue_lm(Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    DecGemv g{};
    g.eps = c.rms_eps;
    g.state = d->state;
    g.max_seq = c.max_seq;
    g.x = d->x; g.norm_w = d->final_norm; g.W = d->lm_head; g.s_w = d->s_lm; g.N = c.vocab;
    g.K = c.hidden; g.y = d->logits; g.part_keys = d->part_keys;
    PIO_TRY((launch_dec_gemv<EPI_LOGITS, 4>(g, d->lm_blocks, d->st)));
    dec_finish_kernel<<<1, 1024, 0, d->st>>>(d->state, d->part_keys, d->lm_blocks, d->ids, c.max_seq);
    PIO_LAUNCHED();
    return PIO_OK;
}

static size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// Frees the decoder's memory into the cache of its stream. A stream the
// decoder created is drained first and its cached blocks (the state block and
// the persistent kernel's weight copy among them) are released with it, so
// nothing stays cached under a stream that no longer exists.
static void destroy(Qwen3Dec* d) {
    if (!d) return;
    loop_destroy(d);
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    if (d->block) device_free(d->block);
    if (d->own_stream && d->st) {
        release_stream(d->st);
        (void)hipStreamDestroy(d->st);
    }
    delete d;
}

}  // namespace pio

using namespace pio;

PIO_EXPORT void* pio_qwen3_create(const pio_qwen3_config* cfg, const float* embed,
                                  const float* final_norm, const int8_t* lm_head,
                                  const float* s_lm_head, const pio_qwen3_layer* layers,
                                  void* stream) {
    if (!cfg || !embed || !final_norm || !lm_head || !s_lm_head || !layers) {
        set_error(PIO_ERR_INVALID, "pio_qwen3_create: null argument");
        return nullptr;
    }
    const pio_qwen3_config& c = *cfg;
    // The attention kernel is specialized for head_dim 128 (the Qwen3 family's);
    // every GEMV K (hidden, heads*head_dim, intermediate) must be a multiple of 16.
    if (c.n_layers < 1 || c.hidden < 16 || c.hidden % 16 || c.n_heads < 1 || c.n_kv_heads < 1 ||
        c.n_heads % c.n_kv_heads || c.head_dim != 128 || c.intermediate % 16 ||
        c.intermediate < 16 || c.vocab < 1 || c.max_seq < 1 || c.max_seq > DEC_MAX_SEQ ||
        (c.kv_dtype != PIO_F32 && c.kv_dtype != PIO_F16)) {
        set_error(PIO_ERR_INVALID, "pio_qwen3_create: unsupported config (head_dim must be 128; "
                                   "hidden and intermediate multiples of 16; max_seq <= %d; "
                                   "kv_dtype PIO_F32 or PIO_F16)",
                  DEC_MAX_SEQ);
        return nullptr;
    }
    for (int l = 0; l < c.n_layers; l++) {
        const pio_qwen3_layer& L = layers[l];
        if (!L.in_norm || !L.w_qkv || !L.s_qkv || !L.w_o || !L.s_o || !L.post_norm || !L.w_gu ||
            !L.s_gu || !L.w_down || !L.s_down) {
            set_error(PIO_ERR_INVALID, "pio_qwen3_create: layer %d has a null weight", l);
            return nullptr;
        }
    }
    Qwen3Dec* d = new Qwen3Dec();
    d->c = c;
    d->embed = embed;
    d->final_norm = final_norm;
    d->lm_head = lm_head;
    d->s_lm = s_lm_head;
    d->layers.assign(layers, layers + c.n_layers);
    if (stream) {
        d->st = (hipStream_t)stream;
    } else {
        if (hipStreamCreateWithFlags(&d->st, hipStreamNonBlocking) != hipSuccess) {
            set_error(PIO_ERR_HIP, "pio_qwen3_create: stream creation failed");
            delete d;
            return nullptr;
        }
        d->own_stream = true;
    }
    const int D = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads;
    const size_t kv = (size_t)c.n_layers * nkv * c.max_seq * D;
    const size_t half = D / 2;
    // lm_head GEMV blocks: each wave walks 4-row groups, loading the next
    // group's rows before it reduces the current one; capped so that each block's
    // prologue (x, its norm and the RMSNorm scale) serves several groups:
    // vocab / 16 blocks (one group per wave) ran C2 graph mode at 1278 tok/s,
    // 2048 blocks at 1303
    d->lm_blocks = std::min(ceil_div(c.vocab, 16), 2048);
    // attention LDS: scores [G][ceil(max_seq/S)] + value partials [8][G][128], <= 64 KB
    d->att_lds = (size_t)(nq / nkv) * (ceil_div(c.max_seq, ATT_SPLITS) + 8 * D) * 4;
    if (nq / nkv > ATT_MAX_G || d->att_lds > 65536) {
        set_error(PIO_ERR_UNSUPPORTED, "pio_qwen3_create: %d query heads per KV head and max_seq "
                  "%d need %zu B of attention LDS (limits: %d heads, 65536 B)", nq / nkv,
                  c.max_seq, d->att_lds, ATT_MAX_G);
        destroy(d);
        return nullptr;
    }
    size_t sizes[] = {
        al256((size_t)c.hidden * 4),                      // x
        al256((size_t)nq * D * 4),                        // q
        al256((size_t)ATT_SPLITS * nq * D * 4),           // attention partial o
        al256((size_t)ATT_SPLITS * nq * 2 * 4),           // attention partial (max, sum)
        al256((size_t)c.intermediate * 4),                // act
        al256((size_t)c.vocab * 4),                       // logits
        al256(kv * (c.kv_dtype == PIO_F16 ? 2 : 4)),      // k cache
        al256(kv * (c.kv_dtype == PIO_F16 ? 2 : 4)),      // v cache
        al256(c.max_seq * half * 4), al256(c.max_seq * half * 4),   // cos, sin
        al256(16 * 4),                                    // state
        al256((size_t)(c.max_seq + 1) * 4),               // ids
        al256((size_t)d->lm_blocks * 8)};                 // argmax partial keys
    size_t total = 0;
    for (size_t sz : sizes) total += sz;
    if (device_alloc(&d->block, total, d->st) != PIO_OK) {
        destroy(d);
        return nullptr;
    }
    char* p = (char*)d->block;
    size_t o = 0;
    auto take = [&](int i) { char* r = p + o; o += sizes[i]; return r; };
    d->x = (float*)take(0);
    d->q = (float*)take(1);
    d->att_o = (float*)take(2);
    d->att_ml = (float*)take(3);
    d->act = (float*)take(4);
    d->logits = (float*)take(5);
    d->kc = take(6);
    d->vc = take(7);
    d->kv16 = c.kv_dtype == PIO_F16;
    d->cos_t = (float*)take(8);
    d->sin_t = (float*)take(9);
    d->state = (int32_t*)take(10);
    d->ids = (int32_t*)take(11);
    d->part_keys = (unsigned long long*)take(12);
    // RoPE table: angle(pos, j) = pos * theta^(-2j/D), computed in double.
    std::vector<float> ct((size_t)c.max_seq * half), stt((size_t)c.max_seq * half);
    for (int pos = 0; pos < c.max_seq; pos++)
        for (size_t j = 0; j < half; j++) {
            const double inv = pow((double)c.rope_theta, -(double)(2 * j) / (double)D);
            const double a = (double)pos * inv;
            ct[pos * half + j] = (float)cos(a);
            stt[pos * half + j] = (float)sin(a);
        }
    hipError_t e = hipMemcpyAsync(d->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice, d->st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->sin_t, stt.data(), stt.size() * 4, hipMemcpyHostToDevice, d->st);
    if (e == hipSuccess) e = hipStreamSynchronize(d->st);
    if (e != hipSuccess) {
        set_error(PIO_ERR_HIP, "pio_qwen3_create: table upload failed: %s", hipGetErrorString(e));
        destroy(d);
        return nullptr;
    }
    return d;
}

PIO_EXPORT void pio_qwen3_destroy(void* h) { destroy((Qwen3Dec*)h); }

PIO_EXPORT int pio_qwen3_reset(void* h, const int32_t* ids, int prompt_len) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d && ids, "pio_qwen3_reset: null argument");
    PIO_REQUIRE(prompt_len >= 1 && prompt_len <= d->c.max_seq,
                "pio_qwen3_reset: prompt length %d outside [1, %d]", prompt_len, d->c.max_seq);
    for (int i = 0; i < prompt_len; i++)
        PIO_REQUIRE(ids[i] >= 0 && ids[i] < d->c.vocab, "pio_qwen3_reset: token %d out of range",
                    i);
    // Host staging keeps the copies and the state init in stream order; no memset
    // (a graph replay must not follow a memset node).
    // persistent launches still queued run first; their results are dropped
    PIO_HIP(hipStreamSynchronize(d->st));
    int from = 0;
    (void)loop_status(d, &from);
    clear_error();
    std::vector<int32_t> st(16, 0);
    st[0] = 0;
    st[1] = prompt_len;
    PIO_HIP(hipMemcpyAsync(d->ids, ids, (size_t)prompt_len * 4, hipMemcpyHostToDevice, d->st));
    PIO_HIP(hipMemcpyAsync(d->state, st.data(), 16 * 4, hipMemcpyHostToDevice, d->st));
    PIO_HIP(hipStreamSynchronize(d->st));
    d->host_pos = 0;
    d->prompt_len = prompt_len;
    return PIO_OK;
}

// n_steps decode steps of the step kernels: one captured graph per step
// (use_graph) or the kernels launched one by one.
static int run_stepwise(Qwen3Dec* d, int n_steps, bool use_graph) {
    if (use_graph && !d->exec && n_steps > 0) {
        PIO_HIP(hipStreamBeginCapture(d->st, hipStreamCaptureModeRelaxed));
        int rc = enqueue_step(d);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(d->st, &g);
        if (rc != PIO_OK) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        PIO_HIP(e);
        d->graph = g;
        PIO_HIP(hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0));
    }
    for (int i = 0; i < n_steps; i++) {
        if (use_graph) PIO_HIP(hipGraphLaunch(d->exec, d->st));
        else PIO_TRY(enqueue_step(d));
    }
    d->host_pos += n_steps;
    return PIO_OK;
}

// Drains the stream and checks the persistent launches since the last check.
// Launches that found the grid not co-resident (other work held CUs when they
// started) computed nothing, nor did any launch after them: their steps run
// again here in graph mode, from the first position that did not run.
static int settle(Qwen3Dec* d) {
    PIO_HIP(hipStreamSynchronize(d->st));
    int from = 0;
    const int rc = loop_status(d, &from);
    if (rc != LOOP_REPLAY) return rc;
    const int n = d->host_pos - from;
    d->host_pos = from;
    PIO_TRY(run_stepwise(d, n, true));
    PIO_HIP(hipStreamSynchronize(d->st));
    return PIO_OK;
}

PIO_EXPORT int pio_qwen3_run(void* h, int n_steps, int mode) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_run: null handle");
    PIO_REQUIRE(n_steps >= 0 && d->host_pos + n_steps <= d->c.max_seq,
                "pio_qwen3_run: %d more steps exceed max_seq %d (at %d)", n_steps, d->c.max_seq,
                d->host_pos);
    PIO_REQUIRE(mode >= PIO_DECODE_EAGER && mode <= PIO_DECODE_PERSISTENT,
                "pio_qwen3_run: unknown mode %d", mode);
    if (mode == PIO_DECODE_PERSISTENT) {
        PIO_TRY(loop_run(d, n_steps));
        d->host_pos += n_steps;
        return PIO_OK;
    }
    // the step kernels continue from the device position: persistent launches
    // queued before must have run (or been re-run) first
    if (loop_pending(d)) PIO_TRY(settle(d));
    return run_stepwise(d, n_steps, mode == PIO_DECODE_GRAPH);
}

PIO_EXPORT int pio_qwen3_prefill(void* h, int n_steps, int logits) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_prefill: null handle");
    PIO_REQUIRE(n_steps >= 1 && d->host_pos + n_steps <= d->c.max_seq,
                "pio_qwen3_prefill: %d more positions exceed max_seq %d (at %d)", n_steps, d->c.max_seq,
                d->host_pos);
    // the batch continues from the device position and cache
    if (loop_pending(d)) PIO_TRY(settle(d));
    return prefill(d, n_steps, logits != 0);
}

PIO_EXPORT int pio_qwen3_trace_next(void* h, int first_step) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d && first_step >= 0, "pio_qwen3_trace_next: null handle or negative step");
    return loop_trace_next(d, first_step);
}

PIO_EXPORT size_t pio_qwen3_trace_bytes(void* h) { return h ? loop_trace_bytes((Qwen3Dec*)h) : 0; }

PIO_EXPORT int pio_qwen3_trace_read(void* h, void* out, size_t bytes) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d && out, "pio_qwen3_trace_read: null argument");
    return loop_trace_read(d, out, bytes);
}

PIO_EXPORT int pio_qwen3_persistent_replays(void* h) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_persistent_replays: null handle");
    return loop_replays(d);
}

PIO_EXPORT int pio_qwen3_refresh_weights(void* h) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_refresh_weights: null handle");
    return loop_refresh(d);
}

PIO_EXPORT int pio_qwen3_persistent_supported(void* h) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_persistent_supported: null handle");
    return loop_check(d) == PIO_OK ? 1 : 0;
}

PIO_EXPORT int pio_qwen3_read(void* h, int32_t* ids, int n, float* logits) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_read: null handle");
    PIO_REQUIRE(n >= 0 && n <= d->c.max_seq + 1, "pio_qwen3_read: n=%d out of range", n);
    PIO_TRY(settle(d));
    if (n > 0) {
        PIO_REQUIRE(ids, "pio_qwen3_read: null ids");
        PIO_HIP(hipMemcpyAsync(ids, d->ids, (size_t)n * 4, hipMemcpyDeviceToHost, d->st));
    }
    if (logits)
        PIO_HIP(hipMemcpyAsync(logits, d->logits, (size_t)d->c.vocab * 4, hipMemcpyDeviceToHost,
                               d->st));
    PIO_HIP(hipStreamSynchronize(d->st));
    return PIO_OK;
}

PIO_EXPORT const float* pio_qwen3_logits(void* h) { return h ? ((Qwen3Dec*)h)->logits : nullptr; }
