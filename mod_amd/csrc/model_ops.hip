// Device-side companion ops of the reference model layers: the fp32 ops a
// decoder layer written against the reference Tensor API calls around its
// linears (RMSNorm, RoPE, attention, SwiGLU, embedding, argmax and the data
// movement that slices q/k/v and fills a KV cache), so that such a layer runs
// on rocm:N with the int8 linears of this library. Each op follows the
// reference CPU backend's loop (tensor_ops.c, cited per op); where that loop
// reads out of bounds or ignores a shape the model hands it, the op takes the
// shape from its own operand instead, and says so. fp32 device tensors only;
// every op runs on the library's current stream and returns a status
// (PIO_OK or a negative code with the message in tensor_last_error).
#include "pio_common.hpp"

#include <climits>

namespace pio {

constexpr int MO_THREADS = 256;
constexpr int MO_MAX_DIMS = 8;

static int need_f32(const Tensor* t, const char* what) {
    PIO_TRY(check_device_tensor(t, what));
    PIO_REQUIRE(tensor_dtype_of(t) == PIO_F32, "%s: fp32 tensor required", what);
    return PIO_OK;
}
static int same_device(const Tensor* a, const Tensor* b, const char* what) {
    PIO_REQUIRE(a->device_id == b->device_id, "%s: tensors on devices %d and %d", what, a->device_id,
                b->device_id);
    return PIO_OK;
}
static unsigned blocks_for(int64_t n) {
    const int64_t g = (n + MO_THREADS - 1) / MO_THREADS;
    return (unsigned)(g > 65535 ? 65535 : (g < 1 ? 1 : g));
}

// Sum / max over the block (256 threads = 4 waves); every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ------------------------------------------------------------ RMSNorm ------
// One block per row: y = x * (1 / sqrt(sum(x^2) / cols + eps)) * w
// (tensor_ops.c:369-383). With res: x <- x + res first, stored back in place
// (tensor_ops_cuda.cu:220-240, the fused_add_rms_norm the reference layer
// calls when the backend has it).
__global__ __launch_bounds__(MO_THREADS) void mo_rms_norm_kernel(float* x, const float* __restrict__ res,
                                                                const float* __restrict__ w, float* y, int cols,
                                                                float eps) {
    __shared__ float red[4];
    float* xr = x + (int64_t)blockIdx.x * cols;
    float* yr = y + (int64_t)blockIdx.x * cols;
    float ss = 0.f;
    for (int i = threadIdx.x; i < cols; i += MO_THREADS) {
        float v = xr[i];
        if (res) {
            v += res[(int64_t)blockIdx.x * cols + i];
            xr[i] = v;
        }
        ss += v * v;
    }
    const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)cols + eps);
    for (int i = threadIdx.x; i < cols; i += MO_THREADS) yr[i] = xr[i] * scale * w[i];
}

static int rms_norm_impl(Tensor* x, Tensor* res, Tensor* w, Tensor* out, float eps, const char* nm) {
    PIO_TRY(need_f32(x, nm));
    PIO_TRY(need_f32(w, nm));
    PIO_TRY(need_f32(out, nm));
    if (res) PIO_TRY(need_f32(res, nm));
    PIO_TRY(same_device(x, out, nm));
    PIO_TRY(same_device(x, w, nm));
    const int cols = last_dim(x);
    PIO_REQUIRE(cols > 0 && x->size % cols == 0, "%s: bad input shape", nm);
    PIO_REQUIRE(w->size >= cols, "%s: weight has %d elements, rows have %d", nm, w->size, cols);
    PIO_REQUIRE(out->size >= x->size, "%s: out smaller than the input", nm);
    PIO_REQUIRE(!res || res->size >= x->size, "%s: residual smaller than the input", nm);
    const int rows = x->size / cols;
    if (rows == 0) return PIO_OK;
    mo_rms_norm_kernel<<<rows, MO_THREADS, 0, current_stream()>>>(x->data, res ? res->data : nullptr, w->data,
                                                                  out->data, cols, eps);
    PIO_LAUNCHED();
    return PIO_OK;
}

// --------------------------------------------------------------- RoPE ------
// q [.., S, Hq, D], k [.., S, Hk, D]; cos / sin rows s of [>= S, D/2]:
//   o[i] = r cs - m sn, o[i + D/2] = r sn + m cs with r = x[i], m = x[i + D/2]
// (tensor_ops.c:384-413). k keeps its own head count: the reference loop
// walks k with q's (one pointer per q head), which for a grouped-query k
// reads past its end; with Hk == Hq the two agree.
// q / k may be out_q / out_k (in place): each thread reads its element pair
// before it writes the same pair, so neither is marked __restrict__.
__global__ __launch_bounds__(MO_THREADS) void mo_rope_kernel(const float* q, const float* k,
                                                             const float* __restrict__ cs, const float* __restrict__ sn,
                                                             float* oq, float* ok, int64_t tok, int S, int Hq, int Hk,
                                                             int half) {
    const int64_t per = (int64_t)(Hq + Hk) * half;
    for (int64_t e = (int64_t)blockIdx.x * MO_THREADS + threadIdx.x; e < tok * per;
         e += (int64_t)gridDim.x * MO_THREADS) {
        const int64_t t = e / per;         // (batch, position)
        const int r = (int)(e - t * per);
        const int h = r / half, i = r - h * half;
        const int s = (int)(t % S);
        const float c = cs[(int64_t)s * half + i], n = sn[(int64_t)s * half + i];
        const float* x;
        float* o;
        if (h < Hq) {
            x = q + (t * Hq + h) * 2 * half;
            o = oq + (t * Hq + h) * 2 * half;
        } else {
            x = k + (t * Hk + (h - Hq)) * 2 * half;
            o = ok + (t * Hk + (h - Hq)) * 2 * half;
        }
        const float re = x[i], im = x[i + half];
        o[i] = re * c - im * n;
        o[i + half] = re * n + im * c;
    }
}

// ------------------------------------------------- SiLU / SwiGLU family ----
// silu(x) = x * (1 / (1 + exp(-x))) (tensor_ops.c:336-342); swiglu:
// silu(gate) * up (:579-587); fused: row r's gate is gate_up[r][0..h), its up
// gate_up[r][h..2h) (:588-604).
__device__ __forceinline__ float mo_silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

// silu and swiglu may run in place (out == a or b: each element is read and
// written by one thread); the fused form may not (act_impl refuses an out that
// overlaps gate_up: an output row lands on input rows other threads read).
__global__ __launch_bounds__(MO_THREADS) void mo_act_kernel(const float* a, const float* b, float* out, int64_t n,
                                                            int hidden, int mode) {
    for (int64_t i = (int64_t)blockIdx.x * MO_THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * MO_THREADS) {
        if (mode == 0) {
            out[i] = mo_silu(a[i]);
        } else if (mode == 1) {
            out[i] = mo_silu(a[i]) * b[i];
        } else {
            const int64_t r = i / hidden, j = i - r * hidden;
            const float* row = a + r * 2 * hidden;
            out[i] = mo_silu(row[j]) * row[j + hidden];
        }
    }
}

// ------------------------------------------------------------ softmax ------
// One block per row: m = max(-1e9, row); e = exp(x - m); out = e * (1 / sum e)
// (tensor_ops.c:351-367).
__global__ __launch_bounds__(MO_THREADS) void mo_softmax_kernel(const float* x, float* y, int cols) {   // y may be x
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * cols;
    float* yr = y + (int64_t)blockIdx.x * cols;
    float m = -1e9f;
    for (int i = threadIdx.x; i < cols; i += MO_THREADS) m = fmaxf(m, xr[i]);
    m = block_max(m, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < cols; i += MO_THREADS) {
        const float e = expf(xr[i] - m);
        yr[i] = e;
        s += e;
    }
    const float inv = 1.0f / block_sum(s, red);
    for (int i = threadIdx.x; i < cols; i += MO_THREADS) yr[i] *= inv;
}

// ------------------------------------------------------------- argmax ------
// One block per row: the first index of the largest value above -1e9, 0 when
// none is (the reference scan starts from max = -1e9 and moves on a strictly
// larger value, tensor_ops.c:649-661); written as a float.
__device__ __forceinline__ void mo_better(float v, int i, float& bv, int& bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}
__global__ __launch_bounds__(MO_THREADS) void mo_argmax_kernel(const float* __restrict__ x, float* out, int cols) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const float* xr = x + (int64_t)blockIdx.x * cols;
    float bv = -1e9f;
    int bi = INT_MAX;
    for (int i = threadIdx.x; i < cols; i += MO_THREADS) {
        const float v = xr[i];
        if (v > -1e9f) mo_better(v, i, bv, bi);   // NaN and values <= -1e9 never win
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mo_better(__shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64), bv, bi);
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) mo_better(rv[w], ri[w], bv, bi);
        out[blockIdx.x] = (float)(bi == INT_MAX ? 0 : bi);
    }
}

// -------------------------------------------------------------- embed ------
// out[i] = weight[(int)indices[i]], rows outside [0, V) read row 0
// (tensor_ops.c:663-671).
__global__ __launch_bounds__(MO_THREADS) void mo_embed_kernel(const float* __restrict__ w, const float* __restrict__ idx,
                                                              float* out, int V, int E) {
    const float f = idx[blockIdx.x];
    int r = (int)f;
    if (!(f > -2147483648.f && f < 2147483648.f) || r < 0 || r >= V) r = 0;
    const float* src = w + (int64_t)r * E;
    float* dst = out + (int64_t)blockIdx.x * E;
    for (int j = threadIdx.x; j < E; j += MO_THREADS) dst[j] = src[j];
}

// ---------------------------------------------------------- attention ------
// One block per (batch, query position, head): q [B, S, H, D], k / v
// [B, T, Hk, D], out [B, S, H, D]. Scores q.k * scale over all T keys (no
// mask, as the reference), softmax with max from -1e9 and the weights
// normalised before the weighted sum of v (tensor_ops.c:536-578). T and Hk
// come from k's own shape: the reference loop uses q's sequence length for
// the keys too, which equals T only when the whole sequence is attended at
// once; query head h reads kv head h / (H / Hk), the head repeat_kv
// (qwen3_0_6b/architecture.py:57-66) would have put there.
__global__ __launch_bounds__(MO_THREADS) void mo_sdpa_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                             const float* __restrict__ v, float* out, int S, int T,
                                                             int H, int Hk, int D, float scale) {
    extern __shared__ float sc[];   // [T]
    __shared__ float red[4];
    const int h = blockIdx.x % H;
    const int64_t bs = blockIdx.x / H;   // batch * S + position
    const int64_t b = bs / S;
    const int hk = h / (H / Hk);
    const float* qr = q + (bs * H + h) * D;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int t = wv; t < T; t += MO_THREADS / 64) {
        const float* kr = k + ((b * T + t) * Hk + hk) * D;
        float d = 0.f;
        for (int i = lane; i < D; i += 64) d += qr[i] * kr[i];
        d = wave_sum(d);
        if (lane == 0) sc[t] = d * scale;
    }
    __syncthreads();
    float m = -1e9f;
    for (int t = threadIdx.x; t < T; t += MO_THREADS) m = fmaxf(m, sc[t]);
    m = block_max(m, red);
    float s = 0.f;
    for (int t = threadIdx.x; t < T; t += MO_THREADS) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        s += e;
    }
    const float inv = 1.0f / block_sum(s, red);   // its barriers order the sc writes before the reads below
    float* orow = out + (bs * H + h) * D;
    for (int i = threadIdx.x; i < D; i += MO_THREADS) {
        float acc = 0.f;
        for (int t = 0; t < T; t++) acc += (sc[t] * inv) * v[((b * T + t) * Hk + hk) * D + i];
        orow[i] = acc;
    }
}

// ------------------------------------------------- slices and copies ------
// Element i of the source (its coordinates by the source's strides) goes to
// the offset sum((start[d] + coord[d]) * dst_stride[d]); offsets outside the
// destination are skipped (tensor_ops.c:605-637 slice, :504-535 set_slice;
// for a slice the source walk is over out's coordinates and the offset is
// into the input).
struct SliceGeom {
    int ndim;
    int walk[MO_MAX_DIMS];   // strides of the tensor walked element by element
    int jump[MO_MAX_DIMS];   // strides of the other tensor
    int start[MO_MAX_DIMS];
};
__global__ __launch_bounds__(MO_THREADS) void mo_slice_kernel(const float* __restrict__ src, float* dst, int n,
                                                              int other_size, SliceGeom g, int gather) {
    for (int64_t i = (int64_t)blockIdx.x * MO_THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * MO_THREADS) {
        int rem = (int)i;
        int64_t off = 0;
        for (int d = 0; d < g.ndim; d++) {
            if (g.walk[d] == 0) continue;
            const int c = rem / g.walk[d];
            rem -= c * g.walk[d];
            off += (int64_t)(g.start[d] + c) * g.jump[d];
        }
        if (off < 0 || off >= other_size) continue;
        if (gather) dst[i] = src[off];   // slice: walk out, read the input
        else dst[off] = src[i];          // set_slice: walk src, write dst
    }
}
static void strides_of(const Tensor* t, int* st) {
    st[t->ndim - 1] = 1;
    for (int d = t->ndim - 2; d >= 0; d--) st[d] = st[d + 1] * t->shape[d + 1];
}
static int slice_impl(Tensor* walked, Tensor* other, const int* start, bool gather, const char* nm) {
    PIO_TRY(need_f32(walked, nm));
    PIO_TRY(need_f32(other, nm));
    PIO_TRY(same_device(walked, other, nm));
    PIO_REQUIRE(start, "%s: null start indices", nm);
    PIO_REQUIRE(walked->ndim == other->ndim && walked->ndim >= 1 && walked->ndim <= MO_MAX_DIMS,
                "%s: both tensors need the same rank (1..%d)", nm, MO_MAX_DIMS);
    SliceGeom g{};
    g.ndim = walked->ndim;
    strides_of(walked, g.walk);
    strides_of(other, g.jump);
    for (int d = 0; d < g.ndim; d++) g.start[d] = start[d];
    if (walked->size == 0) return PIO_OK;
    hipStream_t st = current_stream();
    if (gather)
        mo_slice_kernel<<<blocks_for(walked->size), MO_THREADS, 0, st>>>(other->data, walked->data, walked->size,
                                                                       other->size, g, 1);
    else
        mo_slice_kernel<<<blocks_for(walked->size), MO_THREADS, 0, st>>>(walked->data, other->data, walked->size,
                                                                       other->size, g, 0);
    PIO_LAUNCHED();
    return PIO_OK;
}

}  // namespace pio

using namespace pio;

PIO_EXPORT int tensor_rms_norm_status(Tensor* input, Tensor* weight, Tensor* out, float eps) {
    return rms_norm_impl(input, nullptr, weight, out, eps, "tensor_rms_norm");
}
PIO_EXPORT void tensor_rms_norm(Tensor* input, Tensor* weight, Tensor* out, float eps) {
    tensor_rms_norm_status(input, weight, out, eps);
}
PIO_EXPORT int tensor_fused_add_rms_norm_status(Tensor* x, Tensor* residual, Tensor* weight, Tensor* out, float eps) {
    PIO_REQUIRE(residual, "tensor_fused_add_rms_norm: null residual");
    return rms_norm_impl(x, residual, weight, out, eps, "tensor_fused_add_rms_norm");
}
PIO_EXPORT void tensor_fused_add_rms_norm(Tensor* x, Tensor* residual, Tensor* weight, Tensor* out, float eps) {
    tensor_fused_add_rms_norm_status(x, residual, weight, out, eps);
}

PIO_EXPORT int tensor_rope_status(Tensor* q, Tensor* k, Tensor* cos, Tensor* sin, Tensor* out_q, Tensor* out_k) {
    const char* nm = "tensor_rope";
    for (Tensor* t : {q, k, cos, sin, out_q, out_k}) PIO_TRY(need_f32(t, nm));
    for (Tensor* t : {k, cos, sin, out_q, out_k}) PIO_TRY(same_device(q, t, nm));
    PIO_REQUIRE(q->ndim >= 3 && k->ndim == q->ndim, "tensor_rope: q and k need the same rank >= 3");
    const int D = last_dim(q), Hq = q->shape[q->ndim - 2], S = q->shape[q->ndim - 3];
    const int Hk = k->shape[k->ndim - 2];
    PIO_REQUIRE(D > 0 && D % 2 == 0 && last_dim(k) == D && k->shape[k->ndim - 3] == S,
                "tensor_rope: q and k need one even head_dim and one sequence length");
    PIO_REQUIRE(Hq > 0 && Hk > 0 && S > 0, "tensor_rope: empty head or sequence dimension");
    const int64_t tok = (int64_t)q->size / ((int64_t)S * Hq * D) * S;
    PIO_REQUIRE(tok * Hk * D == k->size, "tensor_rope: q and k disagree on the batch");
    PIO_REQUIRE((int64_t)cos->size >= (int64_t)S * (D / 2) && (int64_t)sin->size >= (int64_t)S * (D / 2),
                "tensor_rope: cos / sin need %d rows of %d", S, D / 2);
    PIO_REQUIRE(out_q->size >= q->size && out_k->size >= k->size, "tensor_rope: outputs too small");
    if (tok == 0) return PIO_OK;
    mo_rope_kernel<<<blocks_for(tok * (Hq + Hk) * (D / 2)), MO_THREADS, 0, current_stream()>>>(
        q->data, k->data, cos->data, sin->data, out_q->data, out_k->data, tok, S, Hq, Hk, D / 2);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_rope(Tensor* q, Tensor* k, Tensor* cos, Tensor* sin, Tensor* out_q, Tensor* out_k) {
    tensor_rope_status(q, k, cos, sin, out_q, out_k);
}

static int act_impl(Tensor* a, Tensor* b, Tensor* out, int mode, const char* nm) {
    PIO_TRY(need_f32(a, nm));
    PIO_TRY(need_f32(out, nm));
    PIO_TRY(same_device(a, out, nm));
    int hidden = 0;
    if (mode == 1) {
        PIO_TRY(need_f32(b, nm));
        PIO_TRY(same_device(a, b, nm));
        PIO_REQUIRE(a->size >= out->size && b->size >= out->size, "%s: operands smaller than out", nm);
    } else if (mode == 2) {
        hidden = last_dim(out);
        PIO_REQUIRE(hidden > 0 && out->size % hidden == 0 && a->size >= 2 * (int64_t)out->size,
                    "%s: gate_up needs 2 x %d columns per row of out", nm, hidden);
        const float *o0 = out->data, *o1 = out->data + out->size, *a0 = a->data, *a1 = a->data + a->size;
        PIO_REQUIRE(o1 <= a0 || a1 <= o0, "%s: out overlaps gate_up (threads would overwrite rows others read)", nm);
    } else {
        PIO_REQUIRE(a->size >= out->size, "%s: input smaller than out", nm);
    }
    if (out->size == 0) return PIO_OK;
    mo_act_kernel<<<blocks_for(out->size), MO_THREADS, 0, current_stream()>>>(a->data, b ? b->data : nullptr,
                                                                            out->data, out->size, hidden, mode);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT int tensor_silu_status(Tensor* input, Tensor* out) { return act_impl(input, nullptr, out, 0, "tensor_silu"); }
PIO_EXPORT void tensor_silu(Tensor* input, Tensor* out) { tensor_silu_status(input, out); }
PIO_EXPORT int tensor_swiglu_status(Tensor* gate, Tensor* up, Tensor* out) {
    return act_impl(gate, up, out, 1, "tensor_swiglu");
}
PIO_EXPORT void tensor_swiglu(Tensor* gate, Tensor* up, Tensor* out) { tensor_swiglu_status(gate, up, out); }
PIO_EXPORT int tensor_fused_gate_up_swiglu_status(Tensor* gate_up, Tensor* out) {
    return act_impl(gate_up, nullptr, out, 2, "tensor_fused_gate_up_swiglu");
}
PIO_EXPORT void tensor_fused_gate_up_swiglu(Tensor* gate_up, Tensor* out) {
    tensor_fused_gate_up_swiglu_status(gate_up, out);
}

PIO_EXPORT int tensor_softmax_status(Tensor* input, Tensor* out) {
    const char* nm = "tensor_softmax";
    PIO_TRY(need_f32(input, nm));
    PIO_TRY(need_f32(out, nm));
    PIO_TRY(same_device(input, out, nm));
    const int cols = last_dim(input);
    PIO_REQUIRE(cols > 0 && input->size % cols == 0 && out->size >= input->size, "tensor_softmax: bad shapes");
    if (input->size == 0) return PIO_OK;
    mo_softmax_kernel<<<input->size / cols, MO_THREADS, 0, current_stream()>>>(input->data, out->data, cols);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_softmax(Tensor* input, Tensor* out) { tensor_softmax_status(input, out); }

PIO_EXPORT int tensor_argmax_status(Tensor* input, Tensor* out) {
    const char* nm = "tensor_argmax";
    PIO_TRY(need_f32(input, nm));
    PIO_TRY(need_f32(out, nm));
    PIO_TRY(same_device(input, out, nm));
    const int cols = last_dim(input);
    PIO_REQUIRE(cols > 0 && input->size % cols == 0, "tensor_argmax: bad input shape");
    const int rows = input->size / cols;
    PIO_REQUIRE(out->size >= rows, "tensor_argmax: out has %d elements for %d rows", out->size, rows);
    if (rows == 0) return PIO_OK;
    mo_argmax_kernel<<<rows, MO_THREADS, 0, current_stream()>>>(input->data, out->data, cols);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_argmax(Tensor* input, Tensor* out) { tensor_argmax_status(input, out); }

PIO_EXPORT int tensor_embed_status(Tensor* weight, Tensor* indices, Tensor* out) {
    const char* nm = "tensor_embed";
    for (Tensor* t : {weight, indices, out}) PIO_TRY(need_f32(t, nm));
    PIO_TRY(same_device(weight, out, nm));
    PIO_TRY(same_device(indices, out, nm));
    PIO_REQUIRE(weight->ndim == 2, "tensor_embed: weight must be [vocab, dim]");
    const int V = weight->shape[0], E = weight->shape[1];
    PIO_REQUIRE((int64_t)out->size >= (int64_t)indices->size * E, "tensor_embed: out too small");
    if (indices->size == 0 || E == 0) return PIO_OK;
    PIO_REQUIRE(indices->size <= INT_MAX / 2, "tensor_embed: too many indices");
    mo_embed_kernel<<<indices->size, MO_THREADS, 0, current_stream()>>>(weight->data, indices->data, out->data, V, E);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_embed(Tensor* weight, Tensor* indices, Tensor* out) {
    tensor_embed_status(weight, indices, out);
}

constexpr int MO_SDPA_MAX_T = 32768;   // keys held in LDS (128 KB of scores)

PIO_EXPORT int tensor_scaled_dot_product_attention_status(Tensor* q, Tensor* k, Tensor* v, Tensor* out,
                                                          float scale) {
    const char* nm = "tensor_scaled_dot_product_attention";
    for (Tensor* t : {q, k, v, out}) PIO_TRY(need_f32(t, nm));
    for (Tensor* t : {k, v, out}) PIO_TRY(same_device(q, t, nm));
    PIO_REQUIRE(q->ndim == 4 && k->ndim == 4 && v->ndim == 4,
                "tensor_scaled_dot_product_attention: q, k, v must be [batch, seq, heads, head_dim]");
    const int B = q->shape[0], S = q->shape[1], H = q->shape[2], D = q->shape[3];
    const int T = k->shape[1], Hk = k->shape[2];
    for (int d = 0; d < 4; d++)
        PIO_REQUIRE(k->shape[d] == v->shape[d], "tensor_scaled_dot_product_attention: k and v shapes differ");
    PIO_REQUIRE(k->shape[0] == B && k->shape[3] == D && Hk > 0 && H % Hk == 0,
                "tensor_scaled_dot_product_attention: k [B, T, Hk, D] with Hk dividing q's %d heads", H);
    PIO_REQUIRE(T > 0 && T <= MO_SDPA_MAX_T, "tensor_scaled_dot_product_attention: %d keys (1..%d)", T,
                MO_SDPA_MAX_T);
    PIO_REQUIRE(out->size >= q->size, "tensor_scaled_dot_product_attention: out too small");
    const int64_t blocks = (int64_t)B * S * H;
    PIO_REQUIRE(blocks <= INT_MAX, "tensor_scaled_dot_product_attention: too many query rows");
    if (blocks == 0 || D == 0) return PIO_OK;
    const size_t lds = (size_t)T * sizeof(float);
    PIO_TRY(allow_lds<mo_sdpa_kernel>(lds));
    mo_sdpa_kernel<<<(unsigned)blocks, MO_THREADS, lds, current_stream()>>>(q->data, k->data, v->data, out->data, S, T,
                                                                          H, Hk, D, scale);
    PIO_LAUNCHED();
    return PIO_OK;
}
PIO_EXPORT void tensor_scaled_dot_product_attention(Tensor* q, Tensor* k, Tensor* v, Tensor* out, float scale) {
    tensor_scaled_dot_product_attention_status(q, k, v, out, scale);
}

PIO_EXPORT int tensor_slice_status(Tensor* input, Tensor* out, int* start_indices, int* slice_shapes) {
    (void)slice_shapes;   // the reference ignores it too: out's shape is the slice's
    return slice_impl(out, input, start_indices, true, "tensor_slice");
}
PIO_EXPORT void tensor_slice(Tensor* input, Tensor* out, int* start_indices, int* slice_shapes) {
    tensor_slice_status(input, out, start_indices, slice_shapes);
}
PIO_EXPORT int tensor_set_slice_status(Tensor* dst, Tensor* src, int* start_indices) {
    return slice_impl(src, dst, start_indices, false, "tensor_set_slice");
}
PIO_EXPORT void tensor_set_slice(Tensor* dst, Tensor* src, int* start_indices) {
    tensor_set_slice_status(dst, src, start_indices);
}

// tensor_ops.c:672: out <- the input's elements in order (a reshape copies).
PIO_EXPORT int tensor_reshape_status(Tensor* input, Tensor* out) {
    PIO_TRY(need_f32(input, "tensor_reshape"));
    PIO_TRY(need_f32(out, "tensor_reshape"));
    PIO_TRY(same_device(input, out, "tensor_reshape"));
    PIO_REQUIRE(out->size >= input->size, "tensor_reshape: out has %d elements for %d", out->size, input->size);
    if (input->size == 0) return PIO_OK;
    PIO_HIP(hipMemcpyAsync(out->data, input->data, (size_t)input->size * 4, hipMemcpyDeviceToDevice,
                           current_stream()));
    return PIO_OK;
}
PIO_EXPORT void tensor_reshape(Tensor* input, Tensor* out) { tensor_reshape_status(input, out); }

// tensor_ops.c:702-718: the inputs one after the other along `axis`, each a
// 2-D copy of outer rows of (its extent x inner) elements.
PIO_EXPORT int tensor_cat_status(Tensor** inputs, int count, int axis, Tensor* out) {
    const char* nm = "tensor_cat";
    PIO_REQUIRE(inputs && count >= 0, "tensor_cat: null inputs");
    PIO_TRY(need_f32(out, nm));
    PIO_REQUIRE(axis >= 0 && axis < out->ndim, "tensor_cat: axis %d of a rank-%d output", axis, out->ndim);
    int64_t outer = 1, inner = 1, total = 0;
    for (int d = 0; d < axis; d++) outer *= out->shape[d];
    for (int d = axis + 1; d < out->ndim; d++) inner *= out->shape[d];
    for (int i = 0; i < count; i++) {
        Tensor* t = inputs[i];
        PIO_TRY(need_f32(t, nm));
        PIO_TRY(same_device(t, out, nm));
        PIO_REQUIRE(t->ndim == out->ndim, "tensor_cat: input %d has rank %d, out %d", i, t->ndim, out->ndim);
        for (int d = 0; d < out->ndim; d++)
            PIO_REQUIRE(d == axis || t->shape[d] == out->shape[d], "tensor_cat: input %d differs off the axis", i);
        total += t->shape[axis];
    }
    PIO_REQUIRE(total == out->shape[axis], "tensor_cat: inputs add up to %lld along the axis, out has %d",
                (long long)total, out->shape[axis]);
    hipStream_t st = current_stream();
    int64_t at = 0;
    for (int i = 0; i < count; i++) {
        const int64_t w = (int64_t)inputs[i]->shape[axis] * inner;
        if (w > 0 && outer > 0)
            PIO_HIP(hipMemcpy2DAsync(out->data + at * inner, (size_t)out->shape[axis] * inner * 4, inputs[i]->data,
                                     (size_t)w * 4, (size_t)w * 4, (size_t)outer, hipMemcpyDeviceToDevice, st));
        at += inputs[i]->shape[axis];
    }
    return PIO_OK;
}
PIO_EXPORT void tensor_cat(Tensor** inputs, int count, int axis, Tensor* out) {
    tensor_cat_status(inputs, count, axis, out);
}
