// Batched prompt (prefill) for the int8 Qwen3-style decoder: M consecutive
// prompt positions in one pass per layer, as the reference model forwards the
// whole prompt at its first generate step (ip/models/qwen3_0_6b/
// architecture.py:204-213: every Linear sees all prompt rows at once). The
// decode step kernels and the persistent decode consume one position per
// step; here each int8 linear runs once over all M rows on the matrix cores
// (gemm_w8f.hip: every weight byte read once per launch), and the attention,
// RoPE and KV-cache writes cover every position of the batch:
//
//   x = embed[ids[pos0 .. pos0 + M)]
//   per layer:  h = rmsnorm(x) * w_in;  qkv = W8(h) + b_qkv;
//               RoPE on q and k at each row's position; k, v -> cache rows;
//               o = causal GQA attention (row m sees positions 0 .. pos0 + m);
//               x += W8_o(o);  h = rmsnorm(x) * w_post;  [g|u] = W8_gu(h);
//               x += W8_down(silu(g) * u)
//   optionally: the last row's logits (lm_head, argmax) through the step
//   kernels' tail, exactly as a step at that position would produce them.
//
// The arithmetic is the step's (fp32 activations, int8 weights with
// per-channel scales, fp32 accumulation; the same KV element type and layout),
// so decode steps and the persistent decode continue from it.
#include "decode.hpp"

#include <math.h>

namespace pio {

int gemm_w8f(const void* x, int x_dtype, int64_t ldx, const int8_t* w, const float* s_w, const float* bias,
             void* y, int y_dtype, int64_t ldy, int M, int N, int K, bool resid, hipStream_t st);
int gemm_w8f_split(const float* x, int64_t ldx, const int8_t* w, const float* s_w, const float* bias, float* y,
                   int64_t ldy, int M, int N, int K, bool resid, Scratch& ws, const float** part, int* splits,
                   hipStream_t st);

// x[m] = embed[ids[pos0 + m]] (an out-of-range id reads row 0, as the step).
__global__ __launch_bounds__(256) void pf_embed_kernel(const float* __restrict__ embed, const int32_t* __restrict__ ids,
                                                       int pos0, float* __restrict__ x, int H, int V) {
    const int m = blockIdx.x;
    int id = ids[pos0 + m];
    if (id < 0 || id >= V) id = 0;
    const float4* src = (const float4*)(embed + (int64_t)id * H);
    float4* dst = (float4*)(x + (int64_t)m * H);
    for (int i = threadIdx.x; i < H / 4; i += 256) dst[i] = src[i];
}

// h[m] = x[m] * (1 / sqrt(mean(x[m]^2) + eps)) * w, one block per row.
__global__ __launch_bounds__(256) void pf_rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         float* __restrict__ h, int H, float eps) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)m * H;
    float ss = 0.f;
    for (int i = tid * 4; i < H; i += 1024) {
        const float4 a = *(const float4*)(xr + i);
        ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float r = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
    float* hr = h + (int64_t)m * H;
    for (int i = tid * 4; i < H; i += 1024) {
        const float4 a = *(const float4*)(xr + i);
        const float4 g = *(const float4*)(w + i);
        *(float4*)(hr + i) = make_float4(a.x * r * g.x, a.y * r * g.y, a.z * r * g.z, a.w * r * g.w);
    }
}

// Rotate-half RoPE at each row's position on the q and k heads of qkv (row m,
// position pos0 + m; q rotated in place), then k and v into the cache rows of
// that position, fp32 or fp16 in the step kernels' layout (fp16 rows paired:
// slot 2i holds dim i, slot 2i + 1 dim i + 64). Thread i of (m, head) takes
// dims (i, i + 64) with values a, b.
template <typename KT>
__device__ __forceinline__ void pf_rope_kv_put(float* __restrict__ qkv, int ldq, int pos0, int nq, int nkv,
                                               const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                               KT* __restrict__ kc, KT* __restrict__ vc, int max_seq, int m, int head,
                                               int i, float a, float b) {
    constexpr int D = 128, HALF = 64;
    const int pos = pos0 + m;
    if (head < nq + nkv) {
        const float c = cos_t[(int64_t)pos * HALF + i], s = sin_t[(int64_t)pos * HALF + i];
        const float a2 = a * c - b * s, b2 = a * s + b * c;
        a = a2;
        b = b2;
    }
    if (head < nq) {
        float* row = qkv + (int64_t)m * ldq + head * D;
        row[i] = a;
        row[i + HALF] = b;
        return;
    }
    const bool is_k = head < nq + nkv;
    const int kvh = is_k ? head - nq : head - nq - nkv;
    KT* dst = (is_k ? kc : vc) + ((int64_t)kvh * max_seq + pos) * D;
    if constexpr (sizeof(KT) == 2) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        h2 v;
        v[0] = (_Float16)a;
        v[1] = (_Float16)b;
        *(h2*)(dst + 2 * i) = v;
    } else {
        dst[i] = a;
        dst[i + HALF] = b;
    }
}

// Block (m, head), 64 threads: RoPE and KV rows from the stored q/k/v.
template <typename KT>
__global__ __launch_bounds__(64) void pf_rope_kv_kernel(float* __restrict__ qkv, int ldq, int pos0, int nq, int nkv,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, KT* __restrict__ kc,
                                                        KT* __restrict__ vc, int max_seq) {
    const int m = blockIdx.x, head = blockIdx.y, i = threadIdx.x;
    const float* row = qkv + (int64_t)m * ldq + head * 128;
    pf_rope_kv_put<KT>(qkv, ldq, pos0, nq, nkv, cos_t, sin_t, kc, vc, max_seq, m, head, i, row[i], row[i + 64]);
}

// The q/k/v linear's K slices finished here instead of by the GEMM's reduce:
// y = (sum over slices in order) * s + bias, exactly as that reduce forms it,
// then RoPE and the KV rows as pf_rope_kv_kernel (one launch instead of two).
template <typename KT>
__global__ __launch_bounds__(64) void pf_qkv_finish_kernel(const float* __restrict__ part, int splits, int N,
                                                           const float* __restrict__ s_w,
                                                           const float* __restrict__ bias, float* __restrict__ qkv,
                                                           int ldq, int pos0, int nq, int nkv,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t, KT* __restrict__ kc,
                                                           KT* __restrict__ vc, int max_seq, int M) {
    const int m = blockIdx.x, head = blockIdx.y, i = threadIdx.x;
    const int c0 = head * 128 + i, c1 = c0 + 64;
    const int64_t MN = (int64_t)M * N, r = (int64_t)m * N;
    float a = 0.f, b = 0.f;
#pragma unroll 8
    for (int z = 0; z < splits; z++) {
        a += part[z * MN + r + c0];
        b += part[z * MN + r + c1];
    }
    a = a * s_w[c0];
    b = b * s_w[c1];
    if (bias) {
        a += bias[c0];
        b += bias[c1];
    }
    pf_rope_kv_put<KT>(qkv, ldq, pos0, nq, nkv, cos_t, sin_t, kc, vc, max_seq, m, head, i, a, b);
}

// The gate_up linear's K slices finished with SwiGLU: act[m][i] = silu(g) * u
// for g, u formed as the GEMM's reduce forms them (no bias), the arithmetic of
// pf_swiglu_kernel.
__global__ __launch_bounds__(256) void pf_gu_finish_kernel(const float* __restrict__ part, int splits, int M, int I,
                                                           const float* __restrict__ s_w, float* __restrict__ act) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)M * I) return;
    const int64_t m = e / I, i = e - m * I, MN = (int64_t)M * 2 * I, r = m * 2 * I;
    float g = 0.f, u = 0.f;
#pragma unroll 8
    for (int z = 0; z < splits; z++) {
        g += part[z * MN + r + i];
        u += part[z * MN + r + I + i];
    }
    g = g * s_w[i];
    u = u * s_w[I + i];
    act[e] = g / (1.0f + expf(-g)) * u;
}

// A residual linear's K slices finished into x (x += slices * s, as the
// GEMM's reduce forms it), then -- when w is given -- the RMSNorm of the new
// row into h with pf_rmsnorm_kernel's arithmetic. One block per row; H % 4 == 0.
__global__ __launch_bounds__(256) void pf_resid_norm_kernel(const float* __restrict__ part, int splits, int M, int H,
                                                            const float* __restrict__ s_w, float* __restrict__ x,
                                                            const float* __restrict__ w, float* __restrict__ h,
                                                            float eps) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int64_t MN = (int64_t)M * H;
    float* xr = x + (int64_t)m * H;
    float ss = 0.f;
    for (int i = tid * 4; i < H; i += 1024) {
        // the slices' 4 columns as one 16-byte load each, unrolled so that the
        // loads of up to 8 slices are in flight together (a load per slice and
        // column, each waited for, was most of this kernel's time)
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int z = 0; z < splits; z++) {
            const float4 q = *(const float4*)(part + z * MN + (int64_t)m * H + i);
            acc.x += q.x;
            acc.y += q.y;
            acc.z += q.z;
            acc.w += q.w;
        }
        const float4 xo = *(const float4*)(xr + i);
        const float4 sw = *(const float4*)(s_w + i);
        const float4 a = make_float4(acc.x * sw.x + xo.x, acc.y * sw.y + xo.y, acc.z * sw.z + xo.z, acc.w * sw.w + xo.w);
        *(float4*)(xr + i) = a;
        ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    if (!w) return;
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float r = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
    float* hr = h + (int64_t)m * H;
    for (int i = tid * 4; i < H; i += 1024) {
        const float4 a = *(const float4*)(xr + i);
        const float4 g = *(const float4*)(w + i);
        *(float4*)(hr + i) = make_float4(a.x * r * g.x, a.y * r * g.y, a.z * r * g.z, a.w * r * g.w);
    }
}

constexpr int ATT_MAX_G_PF = 4;   // query heads per KV head

// Causal GQA attention of row m (position p = pos0 + m) for the G query heads
// of KV head g over cache positions 0 .. p, with an online softmax over
// passes of 32 positions. Per pass: 8 threads per position score it (16 dims
// each); the first G half-waves fold the pass's scores into each head's
// running max and sum (the scores become exp(s - max) in place); then every
// thread folds the pass into two output dims (d and d + 64) of one or two
// heads, over half the pass's positions. Block (m, g), 256 threads.
template <typename KT>
__global__ __launch_bounds__(256) void pf_attn_kernel(const float* __restrict__ qkv, int ldq, int pos0, int nq,
                                                      int nkv, const KT* __restrict__ kc, const KT* __restrict__ vc,
                                                      int max_seq, float scale, float* __restrict__ out, int ldo) {
    constexpr int D = 128, P = 32, GM = ATT_MAX_G_PF;
    constexpr bool PAIR = sizeof(KT) == 2;
    __shared__ float sc[GM][P];
    __shared__ float qs[GM][D];
    __shared__ float part[2][GM][D];
    __shared__ float run_m[GM], run_l[GM], corr_s[GM];
    const int m = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int G = nq / nkv, pos = pos0 + m, L = pos + 1;
    const float* qrow = qkv + (int64_t)m * ldq + (int64_t)g * G * D;
    // q in the cache's slot order (fp16 rows are paired)
    for (int e = tid; e < G * D; e += 256) {
        const int h = e / D, sl = e % D;
        const int dim = PAIR ? (sl >> 1) + 64 * (sl & 1) : sl;
        qs[h][sl] = qrow[h * D + dim];
    }
    if (tid < GM) {
        run_m[tid] = -INFINITY;
        run_l[tid] = 0.f;
    }
    const KT* kb = kc + (int64_t)g * max_seq * D;
    const KT* vb = vc + (int64_t)g * max_seq * D;
    // output dims of this thread: dims d and d + 64 of heads hh and hh + 2,
    // over the pass positions of parity ph
    const int ph = tid >> 7, hh = (tid >> 6) & 1, d = tid & 63;
    float o0[2] = {0.f, 0.f}, o1[2] = {0.f, 0.f};
    __syncthreads();
    const int part8 = tid & 7, sub = tid >> 3;   // 32 positions x 8 slices of 16 slots
    for (int t0 = 0; t0 < L; t0 += P) {
        const int np = min(P, L - t0);
        // the pass's values of this thread's two output dims, loaded with the
        // keys (positions clamped, used only below np): all in flight at once,
        // their latency behind the scores (one load round trip per pass; a
        // load per position in the value loop was one round trip each)
        float v_lo[P / 2], v_hi[P / 2];
#pragma unroll
        for (int jj = 0; jj < P / 2; jj++) {
            const KT* vr = vb + (int64_t)(t0 + min(ph + 2 * jj, np - 1)) * D;
            v_lo[jj] = PAIR ? (float)vr[2 * d] : (float)vr[d];
            v_hi[jj] = PAIR ? (float)vr[2 * d + 1] : (float)vr[d + 64];
        }
        {
            const int t = t0 + sub;
            float kv[16];
            const KT* kr = kb + (int64_t)min(t, L - 1) * D + part8 * 16;
#pragma unroll
            for (int i = 0; i < 16; i++) kv[i] = (float)kr[i];
            for (int h = 0; h < G; h++) {
                float sdot = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) sdot = fmaf(qs[h][part8 * 16 + i], kv[i], sdot);
                sdot += __shfl_xor(sdot, 1, 64);
                sdot += __shfl_xor(sdot, 2, 64);
                sdot += __shfl_xor(sdot, 4, 64);
                if (part8 == 0) sc[h][sub] = sub < np ? sdot * scale : -INFINITY;
            }
        }
        __syncthreads();
        if (tid < 32 * G) {
            // half-wave h: the pass's max, the running max and sum of head h
            const int h = tid >> 5, j = tid & 31;
            const float sv = sc[h][j];
            float pm = sv;
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) pm = fmaxf(pm, __shfl_xor(pm, o, 64));
            const float om = run_m[h], nm = fmaxf(om, pm);
            const float e = j < np ? expf(sv - nm) : 0.f;
            float es = e;
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) es += __shfl_xor(es, o, 64);
            sc[h][j] = e;
            if (j == 0) {
                const float cr = om == -INFINITY ? 0.f : expf(om - nm);
                corr_s[h] = cr;
                run_l[h] = run_l[h] * cr + es;
                run_m[h] = nm;
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int h = hh + 2 * k;
            if (h < G) {
                o0[k] *= corr_s[h];
                o1[k] *= corr_s[h];
            }
        }
#pragma unroll
        for (int jj = 0; jj < P / 2; jj++) {
            const int j = ph + 2 * jj;
            if (j >= np) continue;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int h = hh + 2 * k;
                if (h >= G) continue;
                const float e = sc[h][j];
                o0[k] = fmaf(e, v_lo[jj], o0[k]);
                o1[k] = fmaf(e, v_hi[jj], o1[k]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int h = hh + 2 * k;
        if (h < G) {
            part[ph][h][d] = o0[k];
            part[ph][h][d + 64] = o1[k];
        }
    }
    __syncthreads();
    for (int e = tid; e < G * D; e += 256) {
        const int h = e / D, dd = e % D;
        out[(int64_t)m * ldo + (int64_t)(g * G + h) * D + dd] = (part[0][h][dd] + part[1][h][dd]) / run_l[h];
    }
}

// act[m][i] = silu(g) * u with g = gu[m][i], u = gu[m][I + i].
__global__ __launch_bounds__(256) void pf_swiglu_kernel(const float* __restrict__ gu, float* __restrict__ act, int M,
                                                        int I) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)M * I) return;
    const int64_t m = e / I, i = e - m * I;
    const float g = gu[m * 2 * I + i], u = gu[m * 2 * I + I + i];
    act[e] = g / (1.0f + expf(-g)) * u;
}

// The decoder's x = row `m` of the batch, and its position = pos (so that
// the step tail, which advances it, leaves pos + 1).
__global__ void pf_handoff_kernel(const float* __restrict__ xb, int m, int H, float* __restrict__ x,
                                  int32_t* __restrict__ state, int pos) {
    for (int i = threadIdx.x; i < H; i += blockDim.x) x[i] = xb[(int64_t)m * H + i];
    if (threadIdx.x == 0) state[0] = pos;
}

int prefill(Qwen3Dec* d, int M, bool logits) {
    const pio_qwen3_config& c = d->c;
    const int H = c.hidden, D = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, I = c.intermediate;
    const int nqkv = (nq + 2 * nkv) * D, pos0 = d->host_pos;
    PIO_REQUIRE(M >= 1 && pos0 + M <= d->prompt_len,
                "pio_qwen3_prefill: positions %d..%d are not all prompt positions (prompt length %d)", pos0,
                pos0 + M - 1, d->prompt_len);
    PIO_REQUIRE(nq / nkv <= ATT_MAX_G_PF, "pio_qwen3_prefill: %d query heads per KV head (at most %d)", nq / nkv,
                ATT_MAX_G_PF);
    PIO_REQUIRE(H % 16 == 0 && I % 16 == 0, "pio_qwen3_prefill: hidden and intermediate must be multiples of 16");
    hipStream_t st = d->st;
    // activations of the batch: x, h (normed), qkv, attention out, [g|u], act
    const size_t n_x = (size_t)M * H, n_qkv = (size_t)M * nqkv, n_o = (size_t)M * nq * D;
    const size_t n_gu = (size_t)M * 2 * I, n_act = (size_t)M * I;
    Scratch ws;
    PIO_TRY(ws.get((2 * n_x + n_qkv + n_o + n_gu + n_act) * sizeof(float), st));
    float* x = (float*)ws.ptr;
    float* h = x + n_x;
    float* qkv = h + n_x;
    float* o = qkv + n_qkv;
    float* gu = o + n_o;
    float* act = gu + n_gu;
    pf_embed_kernel<<<M, 256, 0, st>>>(d->embed, d->ids, pos0, x, H, c.vocab);
    PIO_LAUNCHED();
    const float scale = 1.0f / sqrtf((float)D);
    // When a linear's plan splits K, its slices are finished by the next step's
    // own kernel (RoPE + KV rows, SwiGLU, residual + the next RMSNorm) instead
    // of by the GEMM's reduce launch; h_ready: h already holds this layer's
    // input RMSNorm (the previous layer's down finish wrote it).
    bool h_ready = false;
    for (int l = 0; l < c.n_layers; l++) {
        const pio_qwen3_layer& L = d->layers[l];
        const int64_t lkv = (int64_t)l * nkv * c.max_seq * D;   // elements
        if (!h_ready) {
            pf_rmsnorm_kernel<<<M, 256, 0, st>>>(x, L.in_norm, h, H, c.rms_eps);
            PIO_LAUNCHED();
        }
        {
            Scratch pw;
            const float* part;
            int sp;
            PIO_TRY(gemm_w8f_split(h, H, L.w_qkv, L.s_qkv, L.b_qkv, qkv, nqkv, M, nqkv, H, false, pw, &part, &sp, st));
            const dim3 g(M, nq + 2 * nkv);
            if (d->kv16) {
                _Float16* kc = (_Float16*)d->kc + lkv;
                _Float16* vc = (_Float16*)d->vc + lkv;
                if (sp)
                    pf_qkv_finish_kernel<_Float16><<<g, 64, 0, st>>>(part, sp, nqkv, L.s_qkv, L.b_qkv, qkv, nqkv, pos0,
                                                                     nq, nkv, d->cos_t, d->sin_t, kc, vc, c.max_seq, M);
                else
                    pf_rope_kv_kernel<_Float16><<<g, 64, 0, st>>>(qkv, nqkv, pos0, nq, nkv, d->cos_t, d->sin_t, kc, vc,
                                                                  c.max_seq);
                PIO_LAUNCHED();
                pf_attn_kernel<_Float16><<<dim3(M, nkv), 256, 0, st>>>(qkv, nqkv, pos0, nq, nkv, kc, vc, c.max_seq,
                                                                         scale, o, nq * D);
            } else {
                float* kc = (float*)d->kc + lkv;
                float* vc = (float*)d->vc + lkv;
                if (sp)
                    pf_qkv_finish_kernel<float><<<g, 64, 0, st>>>(part, sp, nqkv, L.s_qkv, L.b_qkv, qkv, nqkv, pos0, nq,
                                                                  nkv, d->cos_t, d->sin_t, kc, vc, c.max_seq, M);
                else
                    pf_rope_kv_kernel<float><<<g, 64, 0, st>>>(qkv, nqkv, pos0, nq, nkv, d->cos_t, d->sin_t, kc, vc,
                                                               c.max_seq);
                PIO_LAUNCHED();
                pf_attn_kernel<float><<<dim3(M, nkv), 256, 0, st>>>(qkv, nqkv, pos0, nq, nkv, kc, vc, c.max_seq,
                                                                      scale, o, nq * D);
            }
            PIO_LAUNCHED();
        }
        {
            Scratch pw;
            const float* part;
            int sp;
            PIO_TRY(gemm_w8f_split(o, nq * D, L.w_o, L.s_o, nullptr, x, H, M, H, nq * D, true, pw, &part, &sp, st));
            if (sp)
                pf_resid_norm_kernel<<<M, 256, 0, st>>>(part, sp, M, H, L.s_o, x, L.post_norm, h, c.rms_eps);
            else
                pf_rmsnorm_kernel<<<M, 256, 0, st>>>(x, L.post_norm, h, H, c.rms_eps);
            PIO_LAUNCHED();
        }
        {
            Scratch pw;
            const float* part;
            int sp;
            PIO_TRY(gemm_w8f_split(h, H, L.w_gu, L.s_gu, nullptr, gu, 2 * I, M, 2 * I, H, false, pw, &part, &sp, st));
            if (sp)
                pf_gu_finish_kernel<<<ceil_div((int64_t)M * I, 256), 256, 0, st>>>(part, sp, M, I, L.s_gu, act);
            else
                pf_swiglu_kernel<<<ceil_div((int64_t)M * I, 256), 256, 0, st>>>(gu, act, M, I);
            PIO_LAUNCHED();
        }
        {
            Scratch pw;
            const float* part;
            int sp;
            PIO_TRY(gemm_w8f_split(act, I, L.w_down, L.s_down, nullptr, x, H, M, H, I, true, pw, &part, &sp, st));
            const bool next = l + 1 < c.n_layers;
            h_ready = sp && next;
            if (sp) {
                pf_resid_norm_kernel<<<M, 256, 0, st>>>(part, sp, M, H, L.s_down, x,
                                                        next ? d->layers[l + 1].in_norm : nullptr, h, c.rms_eps);
                PIO_LAUNCHED();
            }
        }
    }
    // the last row as the decoder's x; the device position: the step tail
    // (logits, argmax, next id) advances it from the last row's position
    pf_handoff_kernel<<<1, 256, 0, st>>>(x, M - 1, H, d->x, d->state, logits ? pos0 + M - 1 : pos0 + M);
    PIO_LAUNCHED();
    if (logits) PIO_TRY(enqueue_lm(d));
    d->host_pos = pos0 + M;
    return PIO_OK;
}

}  // namespace pio
