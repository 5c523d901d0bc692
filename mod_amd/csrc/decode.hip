// Int8 Qwen3-style decoder, batch 1 greedy (see pio_qwen3_* in tensor_rocm.h).
//
// One decode step is a fixed sequence of kernels whose only varying inputs --
// the position and the token ids -- live in device memory, so the whole step is
// captured once as a HIP graph and replayed per token with no host round trip:
//
//   embed -> L x [ rmsnorm -> W8 qkv(+bias) -> rope+kv-write -> attention ->
//                  W8 o(+residual) -> rmsnorm -> W8 gate_up -> swiglu ->
//                  W8 down(+residual) ] -> rmsnorm -> W8 lm_head -> argmax -> finish
//
// The W8 GEMVs are the HBM-bound kernels (596 MB of int8 weights per token at
// the Qwen3-0.6B shape); everything else is latency. Semantics follow the
// reference model code with its defects fixed: causal attention over the whole
// cache (tensor_ops.c:536-578 attends only to matching positions and has no
// mask), GQA without materializing repeated heads (architecture.py:57-66),
// residual adds kept (architecture.py:129-132 drops one on CPU), RoPE on the
// key heads' own count (tensor_ops.c:390 indexes k with q's head count).
#include "pio_common.hpp"

#include <math.h>
#include <vector>

namespace pio {

int gemv_w8_res(const void* x, int x_dtype, const int8_t* w, const float* s_w, const float* bias,
                const float* res, void* y, int y_dtype, int M, int N, int K, hipStream_t st);

constexpr int DEC_MAX_SEQ = 8192;

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}

// x = embed[ids[pos]] (an out-of-range id reads row 0, as tensor_embed,
// tensor_ops.c:663-671); also clears the argmax key for this step.
__global__ void dec_embed_kernel(const float* __restrict__ embed, const int32_t* __restrict__ ids,
                                 const int32_t* __restrict__ state, float* __restrict__ x, int H,
                                 int V, int max_seq, unsigned long long* key) {
    const int pos = state[0];
    if (pos >= max_seq) return;
    int id = ids[pos];
    if (id < 0 || id >= V) id = 0;
    for (int i = threadIdx.x; i < H; i += blockDim.x) x[i] = embed[(int64_t)id * H + i];
    if (threadIdx.x == 0) *key = 0ull;
}

// out = x * (1/sqrt(mean(x^2) + eps)) * w   (tensor_ops.c:369-383)
__global__ __launch_bounds__(1024) void dec_rmsnorm_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           float* __restrict__ out, int H,
                                                           float eps) {
    __shared__ float red[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float sc = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += blockDim.x) out[i] = x[i] * sc * w[i];
}

// Rotate-half RoPE on q (nq heads) and k (nkv heads) at `pos`, q -> q_out,
// k and v -> the cache row `pos` ([kv_head][max_seq][D] layout).
__global__ void dec_rope_cache_kernel(const float* __restrict__ qkv, const float* __restrict__ cos_t,
                                      const float* __restrict__ sin_t,
                                      const int32_t* __restrict__ state, float* __restrict__ q_out,
                                      float* __restrict__ kc, float* __restrict__ vc, int nq,
                                      int nkv, int D, int max_seq) {
    const int pos = state[0];
    if (pos >= max_seq) return;
    const int half = D / 2;
    const float* c = cos_t + (int64_t)pos * half;
    const float* s = sin_t + (int64_t)pos * half;
    const int pairs = (nq + nkv) * half;
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < pairs; i += blockDim.x * gridDim.x) {
        const int h = i / half, j = i % half;
        const float* src = qkv + (int64_t)h * D;   // q heads then k heads, contiguous
        const float r = src[j], im = src[j + half];
        const float o0 = r * c[j] - im * s[j];
        const float o1 = r * s[j] + im * c[j];
        if (h < nq) {
            q_out[(int64_t)h * D + j] = o0;
            q_out[(int64_t)h * D + j + half] = o1;
        } else {
            float* dst = kc + ((int64_t)(h - nq) * max_seq + pos) * D;
            dst[j] = o0;
            dst[j + half] = o1;
        }
    }
    const float* vsrc = qkv + (int64_t)(nq + nkv) * D;
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < nkv * D; i += blockDim.x * gridDim.x) {
        const int h = i / D, d = i % D;
        vc[((int64_t)h * max_seq + pos) * D + d] = vsrc[i];
    }
}

// Causal GQA attention for one query position: block = one q head, 256 threads.
__global__ __launch_bounds__(256) void dec_attn_kernel(const float* __restrict__ q,
                                                       const float* __restrict__ kc,
                                                       const float* __restrict__ vc,
                                                       const int32_t* __restrict__ state,
                                                       float* __restrict__ out, int nq, int nkv,
                                                       int D, int max_seq, float scale) {
    __shared__ float sc[DEC_MAX_SEQ];
    __shared__ float red[16];
    __shared__ float part[256];
    const int pos = state[0];
    if (pos >= max_seq) return;
    const int L = pos + 1;
    const int h = blockIdx.x, kvh = h / (nq / nkv);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float* qh = q + (int64_t)h * D;
    const float* kb = kc + (int64_t)kvh * max_seq * D;
    const float* vb = vc + (int64_t)kvh * max_seq * D;

    for (int t = w; t < L; t += 4) {
        float dot = 0.f;
        for (int d = lane; d < D; d += 64) dot += qh[d] * kb[(int64_t)t * D + d];
        dot = wave_sum(dot);
        if (lane == 0) sc[t] = dot * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < L; t += blockDim.x) mx = fmaxf(mx, sc[t]);
    mx = block_max(mx, red);
    float sum = 0.f;
    for (int t = threadIdx.x; t < L; t += blockDim.x) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    __syncthreads();
    // out[d] = sum_t p[t] * v[t][d]; the block's threads split (t-slices x d).
    const int slices = blockDim.x / D > 0 ? blockDim.x / D : 1;
    const int d = threadIdx.x % D, sl = threadIdx.x / D;
    float acc = 0.f;
    if (sl < slices)
        for (int t = sl; t < L; t += slices) acc += sc[t] * vb[(int64_t)t * D + d];
    part[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < D) {
        float o = 0.f;
        for (int i = 0; i < slices; i++) o += part[i * D + threadIdx.x];
        out[(int64_t)h * D + threadIdx.x] = o * inv;
    }
}

// a[i] = silu(g[i]) * u[i] with [g | u] = gu  (tensor_ops.c:588-604)
__global__ void dec_swiglu_kernel(const float* __restrict__ gu, float* __restrict__ a, int I) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < I; i += gridDim.x * blockDim.x) {
        const float g = gu[i], u = gu[I + i];
        a[i] = g * (1.0f / (1.0f + expf(-g))) * u;
    }
}

// Argmax with the reference tie rule (strict '>', the first maximum wins,
// tensor_ops.c:649-662): each block reduces to (value, lowest index), then one
// 64-bit atomicMax on (order-preserving value bits << 32 | ~index).
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i);
}
__global__ __launch_bounds__(256) void dec_argmax_kernel(const float* __restrict__ logits, int V,
                                                         unsigned long long* key) {
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < V; i += gridDim.x * blockDim.x) {
        const unsigned long long k = argmax_key(logits[i], i);
        best = k > best ? k : best;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
    }
    __shared__ unsigned long long wb[4];
    if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 4; i++) best = wb[i] > best ? wb[i] : best;
        best = wb[0] > best ? wb[0] : best;
        atomicMax(key, best);
    }
}

// ids[pos+1] = argmax unless pos+1 is still a prompt position; pos += 1.
__global__ void dec_finish_kernel(int32_t* state, const unsigned long long* key, int32_t* ids,
                                  int max_seq) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const int pos = state[0];
    if (pos >= max_seq) return;
    const int id = (int)(0xffffffffu - (uint32_t)(*key & 0xffffffffull));
    if (pos + 1 >= state[1]) ids[pos + 1] = id;
    state[2] = id;
    state[0] = pos + 1;
}

struct Qwen3Dec {
    pio_qwen3_config c{};
    const float* embed = nullptr;
    const float* final_norm = nullptr;
    const int8_t* lm_head = nullptr;
    const float* s_lm = nullptr;
    std::vector<pio_qwen3_layer> layers;
    hipStream_t st = nullptr;
    bool own_stream = false;
    void* block = nullptr;
    float *x, *xn, *qkv, *q, *attn, *gu, *act, *logits, *kc, *vc, *cos_t, *sin_t;
    int32_t *state, *ids;
    unsigned long long* key;
    int host_pos = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

static int enqueue_step(Qwen3Dec* d) {
    const pio_qwen3_config& c = d->c;
    const int H = c.hidden, D = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, I = c.intermediate;
    const int nqkv = (nq + 2 * nkv) * D;
    hipStream_t st = d->st;
    dec_embed_kernel<<<1, 256, 0, st>>>(d->embed, d->ids, d->state, d->x, H, c.vocab, c.max_seq,
                                        d->key);
    PIO_LAUNCHED();
    const float scale = 1.0f / sqrtf((float)D);
    for (int l = 0; l < c.n_layers; l++) {
        const pio_qwen3_layer& L = d->layers[l];
        float* kc = d->kc + (int64_t)l * nkv * c.max_seq * D;
        float* vc = d->vc + (int64_t)l * nkv * c.max_seq * D;
        dec_rmsnorm_kernel<<<1, 1024, 0, st>>>(d->x, L.in_norm, d->xn, H, c.rms_eps);
        PIO_LAUNCHED();
        PIO_TRY(gemv_w8_res(d->xn, PIO_F32, L.w_qkv, L.s_qkv, L.b_qkv, nullptr, d->qkv, PIO_F32, 1,
                            nqkv, H, st));
        dec_rope_cache_kernel<<<4, 256, 0, st>>>(d->qkv, d->cos_t, d->sin_t, d->state, d->q, kc, vc,
                                                 nq, nkv, D, c.max_seq);
        PIO_LAUNCHED();
        dec_attn_kernel<<<nq, 256, 0, st>>>(d->q, kc, vc, d->state, d->attn, nq, nkv, D, c.max_seq,
                                            scale);
        PIO_LAUNCHED();
        PIO_TRY(gemv_w8_res(d->attn, PIO_F32, L.w_o, L.s_o, nullptr, d->x, d->x, PIO_F32, 1, H,
                            nq * D, st));
        dec_rmsnorm_kernel<<<1, 1024, 0, st>>>(d->x, L.post_norm, d->xn, H, c.rms_eps);
        PIO_LAUNCHED();
        PIO_TRY(gemv_w8_res(d->xn, PIO_F32, L.w_gu, L.s_gu, nullptr, nullptr, d->gu, PIO_F32, 1,
                            2 * I, H, st));
        dec_swiglu_kernel<<<ceil_div(I, 256), 256, 0, st>>>(d->gu, d->act, I);
        PIO_LAUNCHED();
        PIO_TRY(gemv_w8_res(d->act, PIO_F32, L.w_down, L.s_down, nullptr, d->x, d->x, PIO_F32, 1,
                            H, I, st));
    }
    dec_rmsnorm_kernel<<<1, 1024, 0, st>>>(d->x, d->final_norm, d->xn, H, c.rms_eps);
    PIO_LAUNCHED();
    PIO_TRY(gemv_w8_res(d->xn, PIO_F32, d->lm_head, d->s_lm, nullptr, nullptr, d->logits, PIO_F32,
                        1, c.vocab, H, st));
    dec_argmax_kernel<<<256, 256, 0, st>>>(d->logits, c.vocab, d->key);
    PIO_LAUNCHED();
    dec_finish_kernel<<<1, 64, 0, st>>>(d->state, d->key, d->ids, c.max_seq);
    PIO_LAUNCHED();
    return PIO_OK;
}

static size_t al256(size_t b) { return (b + 255) / 256 * 256; }

static void destroy(Qwen3Dec* d) {
    if (!d) return;
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    if (d->block) device_free(d->block);
    if (d->own_stream && d->st) (void)hipStreamDestroy(d->st);
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
    if (c.n_layers < 1 || c.hidden < 16 || c.hidden % 16 || c.n_heads < 1 || c.n_kv_heads < 1 ||
        c.n_heads % c.n_kv_heads || c.head_dim < 2 || c.head_dim % 2 || c.head_dim > 256 ||
        c.intermediate % 16 || c.intermediate < 16 || c.vocab < 1 || c.max_seq < 1 ||
        c.max_seq > DEC_MAX_SEQ || (c.n_heads * c.head_dim) % 16) {
        set_error(PIO_ERR_INVALID, "pio_qwen3_create: unsupported config");
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
    const int H = c.hidden, D = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads;
    const size_t nqkv = (size_t)(nq + 2 * nkv) * D;
    const size_t kv = (size_t)c.n_layers * nkv * c.max_seq * D;
    const size_t half = D / 2;
    size_t sizes[] = {
        al256(H * 4), al256(H * 4), al256(nqkv * 4), al256((size_t)nq * D * 4),
        al256((size_t)nq * D * 4), al256((size_t)2 * c.intermediate * 4),
        al256((size_t)c.intermediate * 4), al256((size_t)c.vocab * 4), al256(kv * 4),
        al256(kv * 4), al256(c.max_seq * half * 4), al256(c.max_seq * half * 4), al256(16 * 4),
        al256((size_t)(c.max_seq + 1) * 4), al256(8)};
    size_t total = 0;
    for (size_t s : sizes) total += s;
    if (device_alloc(&d->block, total) != PIO_OK) {
        destroy(d);
        return nullptr;
    }
    char* p = (char*)d->block;
    size_t o = 0;
    auto take = [&](int i) { char* r = p + o; o += sizes[i]; return r; };
    d->x = (float*)take(0);
    d->xn = (float*)take(1);
    d->qkv = (float*)take(2);
    d->q = (float*)take(3);
    d->attn = (float*)take(4);
    d->gu = (float*)take(5);
    d->act = (float*)take(6);
    d->logits = (float*)take(7);
    d->kc = (float*)take(8);
    d->vc = (float*)take(9);
    d->cos_t = (float*)take(10);
    d->sin_t = (float*)take(11);
    d->state = (int32_t*)take(12);
    d->ids = (int32_t*)take(13);
    d->key = (unsigned long long*)take(14);
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
    std::vector<int32_t> st(16, 0);
    st[0] = 0;
    st[1] = prompt_len;
    PIO_HIP(hipMemcpyAsync(d->ids, ids, (size_t)prompt_len * 4, hipMemcpyHostToDevice, d->st));
    PIO_HIP(hipMemcpyAsync(d->state, st.data(), 16 * 4, hipMemcpyHostToDevice, d->st));
    PIO_HIP(hipStreamSynchronize(d->st));
    d->host_pos = 0;
    return PIO_OK;
}

PIO_EXPORT int pio_qwen3_run(void* h, int n_steps, int use_graph) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_run: null handle");
    PIO_REQUIRE(n_steps >= 0 && d->host_pos + n_steps <= d->c.max_seq,
                "pio_qwen3_run: %d more steps exceed max_seq %d (at %d)", n_steps, d->c.max_seq,
                d->host_pos);
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

PIO_EXPORT int pio_qwen3_read(void* h, int32_t* ids, int n, float* logits) {
    Qwen3Dec* d = (Qwen3Dec*)h;
    PIO_REQUIRE(d, "pio_qwen3_read: null handle");
    PIO_REQUIRE(n >= 0 && n <= d->c.max_seq + 1, "pio_qwen3_read: n=%d out of range", n);
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
