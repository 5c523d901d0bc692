/*
 * int8_ref.c -- CPU oracle for the int8 quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests, the
 * smoke test and the benchmark's CPU-baseline leg compare the HIP library
 * against. Nothing in the product (mod_amd/) links, loads or calls it.
 *
 * Each function restates one reference function (cited file:line under
 * /root/reference/src/inference_pio/) or, where the reference has no such
 * function, states the definition the HIP kernels implement. Built with
 * -ffp-contract=off so every fp operation rounds where the source says.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 --- */
/* IEEE binary16 conversion, round-to-nearest-even, with subnormals, inf, nan. */
uint16_t ref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* below 2^-14: half subnormal or zero */
        const uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign; /* < 2^-25 */
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e; /* 14..24 */
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u; /* rebias exponent 127 -> 15 */
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

float ref_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void ref_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = ref_f32_to_f16(in[i]);
}

static inline float load_act(const void* x, int x_f16, int64_t i) {
    return x_f16 ? ref_f16_to_f32(((const uint16_t*)x)[i]) : ((const float*)x)[i];
}
static inline void store_out(void* y, int y_f16, int64_t i, float v) {
    if (y_f16) ((uint16_t*)y)[i] = ref_f32_to_f16(v);
    else ((float*)y)[i] = v;
}

/* ------------------------------------------------------- int8 matmul (a1) --- */
/* plugins/cpu/c_src/tensor_ops.c:217-246: A [batch,m,k] int8, B [batch,k,n]
 * int8 (n contiguous), int accumulator, C = (float)sum; OpenMP over batch. */
void ref_matmul_int8(const int8_t* A, const int8_t* B, float* C, int batch, int m, int k, int n) {
#pragma omp parallel for
    for (int b = 0; b < batch; b++) {
        const int8_t* a = A + (int64_t)b * m * k;
        const int8_t* bb = B + (int64_t)b * k * n;
        float* c = C + (int64_t)b * m * n;
        for (int i = 0; i < m; i++)
            for (int j = 0; j < n; j++) {
                int sum = 0;
                for (int p = 0; p < k; p++) sum += a[i * k + p] * bb[p * n + j];
                c[i * n + j] = (float)sum;
            }
    }
}

/* Same loop nest, int32 accumulators stored raw. */
void ref_matmul_int8_i32(const int8_t* A, const int8_t* B, int32_t* C, int batch, int m, int k,
                         int n) {
#pragma omp parallel for
    for (int b = 0; b < batch; b++) {
        const int8_t* a = A + (int64_t)b * m * k;
        const int8_t* bb = B + (int64_t)b * k * n;
        int32_t* c = C + (int64_t)b * m * n;
        for (int i = 0; i < m; i++)
            for (int j = 0; j < n; j++) {
                int sum = 0;
                for (int p = 0; p < k; p++) sum += a[i * k + p] * bb[p * n + j];
                c[i * n + j] = sum;
            }
    }
}

/* The same integer sums with B given in the Linear layout W [n,k] (k
 * contiguous); integer addition is order-free, so C equals ref_matmul_int8_i32
 * on (A, W^T). Parallel over rows so checker runs at full shapes stay short. */
void ref_matmul_nt_i32(const int8_t* A, const int8_t* W, int32_t* C, int m, int n, int k) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < m; i++) {
        const int8_t* a = A + (int64_t)i * k;
        for (int j = 0; j < n; j++) {
            const int8_t* w = W + (int64_t)j * k;
            int32_t sum = 0;
            for (int p = 0; p < k; p++) sum += (int32_t)a[p] * (int32_t)w[p];
            C[(int64_t)i * n + j] = sum;
        }
    }
}

/* ---------------------------------------------------- fp32 linear (a5) --- */
/* tensor_ops.c:301-335 (tensor_matmul_transposed + bias loop): y[i,j] =
 * sum_p x[i,p]*W[j,p] in fp32, then y += bias[j]. */
void ref_linear_f32(const float* x, const float* W, const float* bias, float* y, int m, int n,
                    int k) {
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            float sum = 0.f;
            for (int p = 0; p < k; p++) sum += x[(int64_t)i * k + p] * W[(int64_t)j * k + p];
            y[(int64_t)i * n + j] = sum;
        }
    if (bias)
        for (int i = 0; i < m; i++)
            for (int j = 0; j < n; j++) y[(int64_t)i * n + j] += bias[j];
}

/* ------------------------------------------------------ W8 GEMV (a6) --- */
/* y[i,j] = s_w[j] * sum_p x[i,p]*float(W[j,p]) (+ bias[j]). The checker sums in
 * double (the products are exact in double) and rounds once at the end, so it
 * sits closer to the exact value than any fp32 summation order. */
void ref_gemv_w8(const void* x, int x_f16, const int8_t* W, const float* s_w, const float* bias,
                 void* y, int y_f16, int m, int n, int k) {
#pragma omp parallel for schedule(static)
    for (int j = 0; j < n; j++) {
        const int8_t* w = W + (int64_t)j * k;
        for (int i = 0; i < m; i++) {
            double acc = 0.0;
            for (int p = 0; p < k; p++) acc += (double)load_act(x, x_f16, (int64_t)i * k + p) * (double)w[p];
            double v = acc * (double)s_w[j];
            if (bias) v += (double)bias[j];
            store_out(y, y_f16, (int64_t)i * n + j, (float)v);
        }
    }
}

/* -------------------------------------------- per-token quantizer (a7) --- */
/* amax = max |x| (fmaxf), s = amax / 127.0f (IEEE division; 1 when amax == 0),
 * q = clamp(rintf(x / s), -127, 127) under round-to-nearest-even. */
void ref_quant_per_token(const void* x, int x_f16, int8_t* q, float* s, int m, int k) {
    for (int i = 0; i < m; i++) {
        float amax = 0.f;
        for (int p = 0; p < k; p++) amax = fmaxf(amax, fabsf(load_act(x, x_f16, (int64_t)i * k + p)));
        const float sc = amax == 0.f ? 1.f : amax / 127.0f;
        s[i] = sc;
        for (int p = 0; p < k; p++) {
            float r = rintf(load_act(x, x_f16, (int64_t)i * k + p) / sc);
            r = fminf(fmaxf(r, -127.f), 127.f);
            q[(int64_t)i * k + p] = (int8_t)(int)r;
        }
    }
}

/* --------------------------------- RMSNorm -> per-token quantizer (f2) --- */
/* Row i (K % 8 == 0), following tensor_rms_norm (tensor_ops.c:369-383) and the
 * residual add of tensor_fused_add_rms_norm (tensor_ops_opencl.c:676-691):
 *   v[k]  = x[k] (+ r[k] in fp32, rounded to x's dtype and stored to x_sum)
 *   ss    = pairwise sum over the chunk partials P[c] = fmaf(v, v, P) over
 *           v[8c .. 8c+7] in k order from 0, P zero-padded to a power of two n,
 *           for h = n/2 .. 1: P[c] += P[c+h] (c < h); ss = P[0]
 *   scale = 1.0f / sqrtf(ss / K + eps)      (tensor_ops.c:380)
 *   y[k]  = v[k] * scale * w[k]             (tensor_ops.c:382, left to right)
 *   q, s  = ref_quant_per_token(y)
 * The reference's own sum order is OpenMP's; this fixed order is the one the
 * GPU kernel uses. */
void ref_rmsnorm_quant(const void* x, int x_f16, const void* r, void* x_sum, const float* w,
                       float eps, int8_t* q, float* s, float* y_out, int m, int k) {
    const int nch = k / 8;
    int n = 1;
    while (n < nch) n <<= 1;
    float* P = (float*)malloc(sizeof(float) * (size_t)n);
    float* v = (float*)malloc(sizeof(float) * (size_t)k);
    float* y = (float*)malloc(sizeof(float) * (size_t)k);
    if (!P || !v || !y) { free(P); free(v); free(y); return; }
    for (int i = 0; i < m; i++) {
        const int64_t b = (int64_t)i * k;
        for (int p = 0; p < k; p++) {
            float a = load_act(x, x_f16, b + p);
            if (r) {
                a = a + load_act(r, x_f16, b + p);
                store_out(x_sum, x_f16, b + p, a);
                a = load_act(x_sum, x_f16, b + p);
            }
            v[p] = a;
        }
        for (int c = 0; c < n; c++) {
            P[c] = 0.f;
            if (c < nch)
                for (int e = 0; e < 8; e++) P[c] = fmaf(v[8 * c + e], v[8 * c + e], P[c]);
        }
        for (int h = n / 2; h >= 1; h /= 2)
            for (int c = 0; c < h; c++) P[c] = P[c] + P[c + h];
        const float scale = 1.0f / sqrtf(P[0] / (float)k + eps);
        for (int p = 0; p < k; p++) {
            const float t = v[p] * scale;
            y[p] = t * w[p];
        }
        if (y_out) memcpy(y_out + b, y, sizeof(float) * (size_t)k);
        ref_quant_per_token(y, 0, q + b, s + i, 1, k);
    }
    free(P);
    free(v);
    free(y);
}

/* -------------------------------------------------- W8A8 linear (a8) --- */
/* acc = int32 sum (ref_matmul_nt_i32); y = float(acc) * s_a[i] * s_w[j]
 * (+ bias[j]) in that order, stored fp32 / fp16 (RNE) / raw int32. */
enum { REF_F32 = 0, REF_F16 = 1, REF_I32 = 3 };
void ref_w8a8(const int8_t* q, const float* s_a, const int8_t* W, const float* s_w,
              const float* bias, void* y, int y_kind, int m, int n, int k) {
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)m * n);
    if (!acc) return;
    ref_matmul_nt_i32(q, W, acc, m, n, k);
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            const int64_t o = (int64_t)i * n + j;
            if (y_kind == REF_I32) { ((int32_t*)y)[o] = acc[o]; continue; }
            float v = (float)acc[o] * s_a[i] * s_w[j];
            if (bias) v += bias[j];
            store_out(y, y_kind == REF_F16, o, v);
        }
    free(acc);
}

/* ------------------------------------------------------ routing (a9) --- */
/* tensor_ops.c:351-368: per row, max seeded with -1e9f, out = expf(x - max),
 * sum in index order, out *= 1/sum. */
void ref_softmax(const float* in, float* out, int rows, int cols) {
    for (int i = 0; i < rows; i++) {
        const float* ip = in + (int64_t)i * cols;
        float* op = out + (int64_t)i * cols;
        float mx = -1e9f;
        for (int j = 0; j < cols; j++) if (ip[j] > mx) mx = ip[j];
        float sum = 0.f;
        for (int j = 0; j < cols; j++) { op[j] = expf(ip[j] - mx); sum += op[j]; }
        const float inv = 1.0f / sum;
        for (int j = 0; j < cols; j++) op[j] *= inv;
    }
}

/* tensor_ops.c:719-738: insertion into a descending list seeded with -1e18 /
 * -1, strict '>' (an equal later value never displaces an earlier one). */
void ref_topk(const float* in, int rows, int cols, int k, float* vals, int32_t* idx) {
    for (int b = 0; b < rows; b++) {
        const float* ip = in + (int64_t)b * cols;
        float* vp = vals + (int64_t)b * k;
        int32_t* xp = idx + (int64_t)b * k;
        for (int i = 0; i < k; i++) { vp[i] = -1e18f; xp[i] = -1; }
        for (int i = 0; i < cols; i++) {
            const float v = ip[i];
            int pos = -1;
            for (int j = 0; j < k; j++) if (v > vp[j]) { pos = j; break; }
            if (pos != -1) {
                for (int j = k - 1; j > pos; j--) { vp[j] = vp[j - 1]; xp[j] = xp[j - 1]; }
                vp[pos] = v;
                xp[pos] = i;
            }
        }
    }
}

/* Router of the MoE layer: softmax, top-k, weights = the top-k probabilities
 * (Qwen3Coder30BMoE.forward, models/qwen3_coder_30b/model.py:311-317), divided
 * by their fp32 sum when renorm != 0. */
void ref_moe_route(const float* logits, int T, int E, int k, int renorm, float* w, int32_t* id) {
    float* p = (float*)malloc(sizeof(float) * (size_t)E);
    for (int t = 0; t < T; t++) {
        ref_softmax(logits + (int64_t)t * E, p, 1, E);
        ref_topk(p, 1, E, k, w + (int64_t)t * k, id + (int64_t)t * k);
        if (renorm) {
            float s = 0.f;
            for (int j = 0; j < k; j++) s += w[(int64_t)t * k + j];
            for (int j = 0; j < k; j++) w[(int64_t)t * k + j] = w[(int64_t)t * k + j] / s;
        }
    }
    free(p);
}

/* e^x as a fixed sequence of fp32 operations (Cody-Waite reduction by ln2 in
 * two parts, degree-7 Taylor polynomial, Horner with explicit fmaf, ldexpf),
 * the same steps as the GPU's exp_det, so both give the same bits. Pinned in
 * tests against float64 exp (<= 2 ulp) and special values. */
float ref_exp_det(float x) {
    if (!(x < 88.72283935546875f)) return x != x ? x : INFINITY;
    if (x < -103.97208f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.428606765330187045e-06f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333377e-3f);
    p = fmaf(p, r, 4.16666679e-2f);
    p = fmaf(p, r, 1.66666672e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}
void ref_exp_det_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ref_exp_det(x[i]);
}

/* tensor_ops.c:588-604 (tensor_fused_gate_up_swiglu): h = g*(1/(1+exp(-g)))*u
 * for the halves [g | u] of one gate_up row, with the reference's expf
 * replaced by ref_exp_det (same value to 2 ulp; bit-reproducible on the GPU). */
static inline float silu_mul(float g, float u) {
    return g * (1.0f / (1.0f + ref_exp_det(-g))) * u;
}

/* --------------------------------------------------- MoE layer (a9/a10) --- */
/* For every token t and slot kk (expert e = id[t,kk], weight w[t,kk]):
 *   gu  = float(int32(q_x[t] . W_gu[e]^T)) * s_x[t] * s_gu[e]      (fp32, [2I])
 *   h   = silu(gu[:I]) * gu[I:]                                      (fp32, [I])
 *   q_h, s_h = per-token quantization of h
 *   d   = float(int32(q_h . W_down[e]^T)) * s_h * s_down[e]          (fp32, [H])
 *   out[t] = sum over kk = 0..k-1, in order, of w[t,kk] * d          (fp32,
 *            one fmaf per term)
 * q_x, s_x = per-token quantization of x. The reference's own combine
 * (model.py:348, elementwise tensor_mul of [n,H] by [n,1]) reads out of bounds
 * and scatter-adds atomically, so this deterministic definition replaces it. */
void ref_moe_w8a8(const void* x, int x_f16, const float* logits, const int8_t* w_gu,
                  const float* s_gu, const int8_t* w_down, const float* s_down, void* out,
                  int out_f16, int T, int H, int I, int E, int k, int renorm) {
    float* tw = (float*)malloc(sizeof(float) * (size_t)T * k);
    int32_t* tid = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * k);
    int8_t* qx = (int8_t*)malloc((size_t)T * H);
    float* sx = (float*)malloc(sizeof(float) * (size_t)T);
    ref_moe_route(logits, T, E, k, renorm, tw, tid);
    ref_quant_per_token(x, x_f16, qx, sx, T, H);
#pragma omp parallel
    {
        int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(2 * I > H ? 2 * I : H));
        float* h = (float*)malloc(sizeof(float) * (size_t)I);
        int8_t* qh = (int8_t*)malloc((size_t)I);
        float* d = (float*)malloc(sizeof(float) * (size_t)H);
        float* o = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(dynamic)
        for (int t = 0; t < T; t++) {
            for (int n = 0; n < H; n++) o[n] = 0.f;
            for (int kk = 0; kk < k; kk++) {
                const int e = tid[(int64_t)t * k + kk];
                const int8_t* wg = w_gu + (int64_t)e * 2 * I * H;
                const float* sg = s_gu + (int64_t)e * 2 * I;
                ref_matmul_nt_i32(qx + (int64_t)t * H, wg, acc, 1, 2 * I, H);
                for (int i = 0; i < I; i++) {
                    const float g = (float)acc[i] * sx[t] * sg[i];
                    const float u = (float)acc[I + i] * sx[t] * sg[I + i];
                    h[i] = silu_mul(g, u);
                }
                float sh;
                ref_quant_per_token(h, 0, qh, &sh, 1, I);
                const int8_t* wd = w_down + (int64_t)e * H * I;
                const float* sd = s_down + (int64_t)e * H;
                ref_matmul_nt_i32(qh, wd, acc, 1, H, I);
                const float wt = tw[(int64_t)t * k + kk];
                for (int n = 0; n < H; n++) {
                    d[n] = (float)acc[n] * sh * sd[n];
                    o[n] = fmaf(wt, d[n], o[n]);
                }
            }
            for (int n = 0; n < H; n++) store_out(out, out_f16, (int64_t)t * H + n, o[n]);
        }
        free(acc); free(h); free(qh); free(d); free(o);
    }
    free(tw); free(tid); free(qx); free(sx);
}

/* Grouping used by the MoE kernels: pairs (t, kk) ordered by expert, then by
 * token. offsets[E+1], row_token[T*k], pos_of_pair[T*k]. */
void ref_moe_group(const int32_t* id, int T, int E, int k, int32_t* offsets, int32_t* row_token,
                   int32_t* pos_of_pair) {
    int32_t* cnt = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    for (int i = 0; i < T * k; i++) cnt[id[i]]++;
    int run = 0;
    for (int e = 0; e < E; e++) { offsets[e] = run; run += cnt[e]; }
    offsets[E] = run;
    for (int e = 0; e < E; e++) cnt[e] = offsets[e];
    for (int t = 0; t < T; t++)
        for (int e = 0; e < E; e++)
            for (int kk = 0; kk < k; kk++)
                if (id[t * k + kk] == e) {
                    row_token[cnt[e]] = t;
                    pos_of_pair[t * k + kk] = cnt[e]++;
                }
    free(cnt);
}

int ref_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
