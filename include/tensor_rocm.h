/*
 * tensor_rocm.h — C ABI of libtensor_ops_rocm.so, the MI355X (gfx950) int8
 * quantized-linear backend for Inference-PIO.
 *
 * Two layers, both extern "C", plain pointers and sizes only:
 *
 *  1. Drop-in `Tensor*` layer. Same struct, same calling convention as the
 *     reference ABI (src/inference_pio/plugins/common/tensor.h:19-69): inputs
 *     first, caller-allocated `out` last, `void` return. A Python binding written
 *     for the reference (src/inference_pio/core/engine/backend.py:46-160) can
 *     load this library unchanged. Errors never abort the process: the `void`
 *     entry points record a message readable through tensor_last_error(), and
 *     every new op also has an `int`-returning `*_status` twin.
 *
 *  2. Raw-pointer layer (`pio_*`). Device pointers, explicit element types,
 *     explicit stream (NULL = the library's current stream). The drop-in layer
 *     is a thin wrapper over it; tests and the benchmark drive it directly with
 *     device memory they own.
 *
 * Data layout (all row-major, innermost dimension contiguous):
 *   weights   W   int8  [N, K]   one row per output channel (reference Linear
 *                                layout, backend.py:698; tensor_ops.c:316)
 *   w scales  s_w fp32  [N]      per output channel
 *   act.      x   fp32|fp16 [M, K]
 *   quant act q   int8  [M, K],  s_a fp32 [M]  (per token, symmetric)
 *   outputs   y   fp32|fp16 [M, N]
 * Non-fp32 data rides in `Tensor.data` byte-packed, as the reference does for
 * int8 (tensor_ops.c:227-228).
 */
#ifndef INFERENCE_PIO_TENSOR_ROCM_H
#define INFERENCE_PIO_TENSOR_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference struct, field for field: tensor.h:19-25; Python mirror CTensor,
 * backend.py:37-44. `size` is the element count; device_id -1 = host, >=0 = GPU. */
typedef struct {
    float* data;
    int* shape;
    int ndim;
    int size;
    int device_id;
} Tensor;

/* Element types for the typed allocator and the raw layer. */
enum {
    PIO_F32 = 0,
    PIO_F16 = 1,
    PIO_I8 = 2,
    PIO_I32 = 3,
};

/* Status codes returned by every `int` entry point. */
enum {
    PIO_OK = 0,
    PIO_ERR_INVALID = -1,   /* bad shape / dtype / null pointer / device mismatch */
    PIO_ERR_HIP = -2,       /* a HIP runtime call failed                           */
    PIO_ERR_OOM = -3,       /* device or pool allocation failed                    */
    PIO_ERR_UNSUPPORTED = -4,
};

/* ---------------------------------------------------------------------------
 * Drop-in: memory and data movement. Required unconditionally by the reference
 * binding (backend.py:49-55, 67-68).
 * ------------------------------------------------------------------------- */

/* tensor.h:28; tensor_ops.c:95-133. fp32 elements (4 B each); device_id >= 0
 * allocates in HBM through the caching allocator / pool, -1 on the host. */
Tensor* create_tensor(int* shape, int ndim, int device_id);
/* tensor.h:29; tensor_ops.c:135-162. Pool-owned memory is returned to the pool,
 * never handed to hipFree. */
void free_tensor(Tensor* t);
/* tensor.h:32; tensor_ops.c:280-283. */
void tensor_fill(Tensor* t, float value);
/* tensor.h:33-34; tensor_ops.c:287-288. `size` counts 4-byte words, exactly as
 * the reference (an int8 [N,K] tensor is loaded as ceil(N*K/4) "floats"). */
void tensor_load_data(Tensor* t, float* buffer, int size);
void tensor_get_data(Tensor* t, float* buffer, int size);
/* tensor.h:37-38; tensor_ops.c:289-296 (elementwise fp32). */
void tensor_add(Tensor* a, Tensor* b, Tensor* out);
void tensor_mul(Tensor* a, Tensor* b, Tensor* out);

/* New: typed allocation (no reference counterpart: the reference has no dtype
 * and over-allocates int8 at 4 B/elem). Allocates size*elem_bytes(dtype). */
Tensor* create_tensor_typed(int* shape, int ndim, int device_id, int dtype);
int tensor_dtype(Tensor* t);
/* New: byte-count loaders next to the float-count ones (tensor_ops.c:287-288). */
void tensor_load_bytes(Tensor* t, const void* src, size_t nbytes);
void tensor_get_bytes(Tensor* t, void* dst, size_t nbytes);
int tensor_load_bytes_status(Tensor* t, const void* src, size_t nbytes);
int tensor_get_bytes_status(Tensor* t, void* dst, size_t nbytes);

/* ---------------------------------------------------------------------------
 * Drop-in: allocator (tensor_ops.c:69-93; bound at backend.py:88-91, 150-154,
 * used by UnifiedMemoryManager.malloc_pinned, unified_manager.py:16-28).
 * ------------------------------------------------------------------------- */

/* tensor_ops.c:74-89: reserve one HBM arena on the current device; later
 * device tensors are bump-allocated from it (256 B aligned) until it is full,
 * then fall back to the caching allocator. Second call is a no-op. */
void init_memory_pool(size_t size_bytes);
/* tensor_ops.c:91-93: rewind the arena. Tensors still pointing into it become
 * dangling, exactly as in the reference. */
void reset_memory_pool(void);
/* backend.py:150-154 (pinned host memory, hipHostMalloc). */
void* allocate_pinned_memory(size_t size);
void free_pinned_memory(void* ptr);
/* New: stats[0]=bytes hipMalloc'd, [1]=bytes in live tensors, [2]=bytes cached
 * for reuse, [3]=peak live bytes, [4]=hipMalloc calls, [5]=arena size,
 * [6]=arena bytes used. */
void tensor_pool_stats(size_t* stats7);
/* New: hipFree every cached (not live) block. */
void tensor_empty_cache(void);
/* New: bytes of op workspaces freed while their stream was capturing a graph
 * and still held for that graph's replays. begin_capture/end_capture's graph
 * returns them to the cache when it is replaced; graphs captured by other
 * means keep them for the life of the process. */
size_t tensor_pool_graph_bytes(void);

/* ---------------------------------------------------------------------------
 * Drop-in: streams and graphs (probed by hasattr at backend.py:82-87, 139-149;
 * CUDAGraph wrapper backend.py:801-810). One in-order HIP stream per device is
 * the library default; set_current_stream(NULL) restores it. destroy_stream
 * drains the stream and releases the memory cached for it. A workspace an op
 * frees while its stream captures stays reserved for the captured graph (see
 * tensor_pool_graph_bytes), so no later tensor can alias it.
 * ------------------------------------------------------------------------- */
void* create_stream(void);
void destroy_stream(void* stream);
void stream_synchronize(void* stream);
void set_current_stream(void* stream);
void* get_current_stream(void);
void device_synchronize(void);
void begin_capture(void);
void end_capture(void);
void replay_graph(void);

/* New, for layer offloading (HybridScheduler, hybrid_scheduler.py:10-177,
 * whose CUDAStream use at :22-23 and :49-72 notes that events are needed for
 * its prefetch): a host tensor in pinned memory (device_id -1; freed by
 * free_tensor), an asynchronous copy between any two tensors of equal bytes
 * and dtype on a stream (NULL: the current one; a DMA that overlaps other
 * streams' kernels when the host side is pinned), and events to order one
 * stream after another. event_query returns 1 when the event has completed, 0
 * when not, < 0 on error. */
Tensor* create_tensor_pinned(int* shape, int ndim, int dtype);
int tensor_is_pinned(Tensor* t);
int tensor_copy_async(Tensor* dst, Tensor* src, void* stream);
void* create_event(void);
void destroy_event(void* event);
int record_event(void* event, void* stream);
int stream_wait_event(void* stream, void* event);
int event_synchronize(void* event);
int event_query(void* event);

/* New: error channel (the reference has none; its CUDA path exit()s,
 * tensor_ops_cuda.cu:10-18). Message of the last failed call on this thread,
 * "" if none; tensor_clear_error() resets it. */
const char* tensor_last_error(void);
void tensor_clear_error(void);

/* ---------------------------------------------------------------------------
 * Drop-in: int8 path.
 * ------------------------------------------------------------------------- */

/* tensor_ops.c:217-246, identical semantics: A [..,M,K] int8, B [..,K,N] int8
 * (N contiguous), out fp32 [..,M,N] = (float) int32 sum; batch = out->size/(M*N),
 * A and B both offset per batch. */
void tensor_matmul_int8(Tensor* a, Tensor* b, Tensor* out);
int tensor_matmul_int8_status(Tensor* a, Tensor* b, Tensor* out);
/* Same, int32 accumulators written raw (out must be PIO_I32 or fp32-sized). */
void tensor_matmul_int8_i32(Tensor* a, Tensor* b, Tensor* out);
int tensor_matmul_int8_i32_status(Tensor* a, Tensor* b, Tensor* out);

/* tensor_ops_cuda.cu:923-929 / tensor_ops_opencl.c:1429-1438 (per-tensor
 * scale, scale->size == 1), extended to per-row scales when scale->size equals
 * the row count of a 2-D int8 input: out[r,c] = float(q[r,c]) * scale[r]. */
void tensor_dequantize(Tensor* q, Tensor* scale, Tensor* out);
int tensor_dequantize_status(Tensor* q, Tensor* scale, Tensor* out);

/* W8 per-output-channel dequant linear (replaces tensor_linear, tensor_ops.c:
 * 323-335, for int8 weights): out[m,n] = s_w[n] * sum_k x[m,k]*W[n,k] + bias[n].
 * x fp32|fp16 [..,K]; W int8 [N,K]; s_w fp32 [N]; bias fp32 [N] or NULL;
 * out fp32|fp16 [..,N]. Decode (small M) runs the HBM-streaming GEMV. */
void tensor_linear_w8(Tensor* x, Tensor* w, Tensor* s_w, Tensor* bias, Tensor* out);
int tensor_linear_w8_status(Tensor* x, Tensor* w, Tensor* s_w, Tensor* bias, Tensor* out);

/* Per-token symmetric activation quantizer (no reference counterpart):
 * amax = max_k |x[m,k]|; s[m] = amax/127 (IEEE division; s=1 when amax==0);
 * q[m,k] = clamp(rint(x[m,k]/s[m]), -127, 127), round-half-even.
 * x fp32|fp16 [..,K]; q int8 [..,K]; s fp32 [..]. */
void tensor_quantize_per_token(Tensor* x, Tensor* q, Tensor* s);
int tensor_quantize_per_token_status(Tensor* x, Tensor* q, Tensor* s);

/* RMSNorm -> per-token quantizer in one pass (the producer of a prefill
 * W8A8 linear's input): y = RMSNorm(x) * weight as tensor_rms_norm
 * (tensor_ops.c:369-383; its sum of squares in a fixed pairwise order, stated
 * in quant.hip), then q, s = the per-token quantizer of y, without writing y.
 * x fp32|fp16 [..,K] with K % 8 == 0 and K <= 32768; weight fp32 [K]; q int8
 * [..,K]; s fp32 [..]. No reference counterpart fuses these: it replaces the
 * pair tensor_rms_norm + tensor_quantize_per_token. */
void tensor_rms_norm_quantize(Tensor* x, Tensor* weight, Tensor* q, Tensor* s, float eps);
int tensor_rms_norm_quantize_status(Tensor* x, Tensor* weight, Tensor* q, Tensor* s, float eps);

/* The same after the residual add of tensor_fused_add_rms_norm
 * (tensor_ops_opencl.c:1471-1483, bound at backend.py:157-158): x <- x +
 * residual (in x's dtype, in place, as the reference updates x), then the
 * RMSNorm -> quantizer of the sum. */
void tensor_fused_add_rms_norm_quantize(Tensor* x, Tensor* residual, Tensor* weight, Tensor* q,
                                        Tensor* s, float eps);
int tensor_fused_add_rms_norm_quantize_status(Tensor* x, Tensor* residual, Tensor* weight,
                                              Tensor* q, Tensor* s, float eps);

/* W8A8 linear: acc = sum_k q[m,k]*W[n,k] (int32, bit-exact vs tensor_ops.c:
 * 217-246); out[m,n] = cvt(float(acc)*s_a[m]*s_w[n] (+ bias[n])).
 * out fp32|fp16 [..,N]. Runs on int8 MFMA. */
void tensor_linear_w8a8(Tensor* q, Tensor* s_a, Tensor* w, Tensor* s_w, Tensor* bias, Tensor* out);
int tensor_linear_w8a8_status(Tensor* q, Tensor* s_a, Tensor* w, Tensor* s_w, Tensor* bias, Tensor* out);

/* Int8 MoE expert layer (replaces Qwen3Coder30BMoE.forward, ip/models/
 * qwen3_coder_30b/model.py:308-353, with a deterministic combine):
 *   p = softmax(logits) (tensor_ops.c:351-368); top_k by tensor_topk's rule
 *   (tensor_ops.c:719-738, strict '>' so ties keep the lower expert id);
 *   weights = top-k probabilities, divided by their sum when renorm != 0;
 *   per (token, slot): h = silu(g)*u of the W8A8 gate_up output (fp32),
 *   requantized per row, then the W8A8 down projection;
 *   out[t] = sum over slots in order k = 0..top_k-1 of w[t,k] * down(t,k).
 * x fp32|fp16 [T,H]; logits fp32 [T,E]; w_gu int8 [E,2I,H] (gate rows first,
 * then up rows); s_gu fp32 [E,2I]; w_down int8 [E,H,I]; s_down fp32 [E,H];
 * out fp32|fp16 [T,H]. Device scratch comes from the caching allocator. */
void tensor_moe_w8a8(Tensor* x, Tensor* logits, Tensor* w_gu, Tensor* s_gu, Tensor* w_down,
                     Tensor* s_down, int top_k, int renorm, Tensor* out);
int tensor_moe_w8a8_status(Tensor* x, Tensor* logits, Tensor* w_gu, Tensor* s_gu, Tensor* w_down,
                           Tensor* s_down, int top_k, int renorm, Tensor* out);

/* ---------------------------------------------------------------------------
 * Raw-pointer layer. All pointers are device pointers; `stream` is a
 * hipStream_t (NULL = library current stream). Return PIO_OK or an error code.
 * ------------------------------------------------------------------------- */

/* y[m,n] = s_w[n]*sum_k x[m,k]*W[n,k] (+bias[n]); x_dtype, y_dtype in {F32,F16}.
 * Requirements: K % 16 == 0, pointers 16-byte aligned. Any M >= 1. Products
 * and sums in fp32 on every path: fp32 FMA kernels in general; fp16 x with
 * 2 <= M <= 64 and K % 1024 == 0 runs on fp16 MFMAs with exact products and
 * fp32 accumulation inside the matrix core, whose rounding is not
 * round-to-nearest-even (measured: results within a few ulp of the FMA
 * kernels'; deterministic run to run). */
int pio_gemv_w8(const void* x, int x_dtype, const int8_t* w, const float* s_w, const float* bias,
                void* y, int y_dtype, int M, int N, int K, void* stream);

/* Per-token quantizer as tensor_quantize_per_token. Any K >= 1. */
int pio_quantize_per_token(const void* x, int x_dtype, int8_t* q, float* s, int M, int K,
                           void* stream);

/* RMSNorm -> quantizer as tensor_rms_norm_quantize on raw pointers. With
 * residual != NULL, x_sum receives x + residual (x's dtype; may equal x) and
 * the norm is taken of that sum (tensor_fused_add_rms_norm_quantize).
 * Pointers 16-byte aligned. */
int pio_rmsnorm_quant(const void* x, int x_dtype, const void* residual, void* x_sum,
                      const float* gamma, float eps, int8_t* q, float* s, int M, int K,
                      void* stream);

/* W8A8 GEMM as tensor_linear_w8a8; y_dtype in {F32,F16,I32}. With y_dtype ==
 * PIO_I32 the raw int32 accumulators are written and s_a/s_w/bias are ignored.
 * Requirements: K % 16 == 0, pointers 16-byte aligned. */
int pio_gemm_w8a8(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
                  const float* bias, void* y, int y_dtype, int M, int N, int K, void* stream);

/* No counterpart in the reference. pio_gemm_w8a8 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same kernels and bit-identical
 * results, with the K-slice int32 partials kept in the library's per-GPU
 * static scratch array (16 MiB, held until the process ends) instead of
 * allocator memory. It calls no hipMalloc/hipFree. Shapes whose plan needs
 * more than 16 MiB of partials (splits x M x N x 4 B) are refused with an
 * error. Every call on a GPU shares that GPU's array: calls that overlap on
 * one GPU (different streams, no ordering between them) race. */
int pio_gemm_w8a8_static(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w,
                         const float* bias, void* y, int y_dtype, int M, int N, int K,
                         void* stream);

/* tensor_matmul_int8 semantics on raw pointers (B is [K,N]); `out_i32` != 0
 * writes int32 instead of fp32. `workspace` needs pio_matmul_int8_workspace()
 * bytes, 16-byte aligned (B is repacked to [N,K] there); null makes the
 * library take its own. */
size_t pio_matmul_int8_workspace(int batch, int M, int K, int N);
int pio_matmul_int8(const int8_t* a, const int8_t* b, void* c, int out_i32, int batch, int M,
                    int K, int N, void* workspace, void* stream);

/* Router: probs = softmax(logits[T,E]) (reference formula), top-k selection
 * (strict '>'), optional renormalization. topk_w fp32 [T,k], topk_id int32 [T,k]. */
int pio_moe_route(const float* logits, float* topk_w, int32_t* topk_id, int T, int E, int top_k,
                  int renorm, void* stream);

/* Full MoE layer on raw pointers; workspace needs pio_moe_workspace() bytes. */
size_t pio_moe_workspace(int T, int H, int I, int E, int top_k);
int pio_moe_w8a8(const void* x, int x_dtype, const float* logits, const int8_t* w_gu,
                 const float* s_gu, const int8_t* w_down, const float* s_down, void* out,
                 int out_dtype, int T, int H, int I, int E, int top_k, int renorm, void* workspace,
                 void* stream);

/* ---------------------------------------------------------------------------
 * Int8 Qwen3-style decoder (greedy decode at batch 1). Replaces the decode
 * loop of Qwen3ForCausalLM.generate / Qwen3DecoderLayer.forward
 * (ip/models/qwen3_0_6b/architecture.py:124-221) with one device-driven step:
 *   x = embed[id[pos]]; per layer: h = rmsnorm(x)*w_in; qkv = W8(h) + b_qkv;
 *   rotate-half RoPE on q and k at `pos` (tensor_ops.c:384-415 formula);
 *   k, v -> cache; causal GQA attention over positions 0..pos; x += W8_o(attn);
 *   h = rmsnorm(x)*w_post; x += W8_down(silu(g)*u) with [g|u] = W8_gate_up(h);
 *   logits = W8_lm_head(rmsnorm(x)*w_final); id[pos+1] = argmax (first max,
 *   tensor_ops.c:649-662) unless pos+1 is still inside the prompt; pos += 1.
 * Position and token ids live in device memory, so a step is replayable as a
 * captured HIP graph. The handle owns activations, KV cache
 * ([layer][kv_head][max_seq][head_dim], fp32 or fp16 by `kv_dtype`) and the
 * RoPE table; weights are the caller's device pointers and must outlive the
 * handle.
 * ------------------------------------------------------------------------- */
typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab, max_seq;
    float rms_eps, rope_theta;
    /* KV cache element type: PIO_F32 (0, the reference's) or PIO_F16 (1: k and
     * v rounded to fp16 when they are written, half the cache bytes read per
     * token). A caller that zero-initializes the struct gets fp32.
     * This field was appended to the struct: a C host built against an
     * earlier copy of this header passes a smaller struct and must be rebuilt
     * against this one. */
    int kv_dtype;
} pio_qwen3_config;

typedef struct {
    const float* in_norm;    /* [hidden]                                        */
    const int8_t* w_qkv;     /* [(n_heads + 2*n_kv_heads)*head_dim, hidden]      */
    const float* s_qkv;      /* [rows of w_qkv]                                  */
    const float* b_qkv;      /* [rows of w_qkv] or NULL                          */
    const int8_t* w_o;       /* [hidden, n_heads*head_dim]                       */
    const float* s_o;        /* [hidden]                                         */
    const float* post_norm;  /* [hidden]                                         */
    const int8_t* w_gu;      /* [2*intermediate, hidden]  (gate rows, then up)   */
    const float* s_gu;       /* [2*intermediate]                                 */
    const int8_t* w_down;    /* [hidden, intermediate]                           */
    const float* s_down;     /* [hidden]                                         */
} pio_qwen3_layer;

/* Creates a decoder on the current device. `layers` is a host array of
 * cfg->n_layers entries. Returns NULL on error (see tensor_last_error). */
void* pio_qwen3_create(const pio_qwen3_config* cfg, const float* embed, const float* final_norm,
                       const int8_t* lm_head, const float* s_lm_head,
                       const pio_qwen3_layer* layers, void* stream);
void pio_qwen3_destroy(void* dec);
/* Loads `ids` (host, prompt_len tokens) and rewinds to position 0. */
int pio_qwen3_reset(void* dec, const int32_t* ids, int prompt_len);
/* Enqueues n decode steps. mode PIO_DECODE_EAGER launches the step kernels,
 * PIO_DECODE_GRAPH replays one captured step graph per token, and
 * PIO_DECODE_PERSISTENT runs all n steps in one kernel launch (one
 * workgroup per CU; weights stream through LDS while each phase waits for its
 * input). The modes share the KV cache and position, so they can alternate.
 * Persistent mode builds a per-workgroup copy of the int8 layer weights on
 * first use (their size; scales, norms, embeddings and the lm_head are read
 * from the caller's buffers in every mode) and needs the config checked by
 * pio_qwen3_persistent_supported. After the caller changes those int8
 * weights in place, pio_qwen3_refresh_weights copies them again. It needs every CU at once: a launch whose
 * workgroups do not all become resident within 20 ms (other work on the
 * device) computes nothing, nor does any persistent launch after it; the next
 * pio_qwen3_read, or a run in another mode, re-runs those steps in graph mode
 * (pio_qwen3_persistent_replays counts such launches). */
#define PIO_DECODE_EAGER 0
#define PIO_DECODE_GRAPH 1
#define PIO_DECODE_PERSISTENT 2
int pio_qwen3_run(void* dec, int n_steps, int mode);
/* Batched prompt: runs the next n_steps positions, all of them prompt
 * positions (position + n_steps <= prompt_len), in one pass per layer -- each
 * int8 linear once over all n_steps rows on the matrix cores, causal
 * attention, RoPE and KV-cache rows for every position -- as the reference
 * forwards the whole prompt at its first step (architecture.py:204-213);
 * the step modes then continue from the cache and position it leaves. With
 * logits != 0 the last position's logits (and, at the prompt's end, the next
 * id) are produced as its step would produce them. */
int pio_qwen3_prefill(void* dec, int n_steps, int logits);
/* 1 if the persistent mode supports this decoder's config on the current
 * device, else 0 (the reason is in tensor_last_error). No counterpart in the
 * reference. */
int pio_qwen3_persistent_supported(void* dec);
/* Copies the caller's int8 layer weights into the persistent mode's
 * per-workgroup copy again, on the decoder's stream (after earlier work on it,
 * before later). Call it after changing those weights in place; without a
 * copy yet (no persistent run so far) it does nothing. No counterpart in the
 * reference, whose layers read their weights on every call. */
int pio_qwen3_refresh_weights(void* dec);
/* Phase timeline of the persistent decode (measurement; no counterpart in the
 * reference). pio_qwen3_trace_next makes the next persistent launch of this
 * decoder run the kernel's traced build, which stamps the 100 MHz constant
 * clock at every phase boundary of that launch's steps first_step and
 * first_step + 1 (wave 0 of each workgroup); pio_qwen3_trace_read waits for
 * the stream and copies the stamps out: uint64 [2][256 workgroups]
 * [n_layers + 1][16] (pio_qwen3_trace_bytes bytes; 0 = not reached). Slots
 * per layer: 0 start, 1 cross-XCD reduction, 2 gather, 3 q/k/v stored,
 * 4 attention stored, 5 merged, 6 o_proj partial, 7 reduction, 8 gather,
 * 9 act stored, 10 down partial, 11 q/k/v weight lines landed, 12 the
 * attention's q arrived, 13 attention computed, 14 merge inputs arrived;
 * layer n_layers: 0 start, 1 reduction, 2 gather, 3 lm_head rows, 4 argmax
 * key stored. */
int pio_qwen3_trace_next(void* dec, int first_step);
size_t pio_qwen3_trace_bytes(void* dec);
int pio_qwen3_trace_read(void* dec, void* out, size_t bytes);
/* Measurement only (no counterpart in the reference): `reps` back-to-back
 * launches of the dense W8A8 GEMM's K loop with its copies only (no MFMA, no
 * output) for an M x N x K problem in 128 x 192 tiles (BM + BN = 320) mapped to
 * the XCDs as the GEMM maps them, in K steps of `step` = 128 (the GEMM's), 256
 * or 512 bytes per row. bench.py --gemm-supply times it. */
int pio_probe_gemm_supply(const int8_t* A, const int8_t* B, int M, int N, int K, int BM, int BN, int step,
                          int reps, void* stream);
/* Measurement, no reference counterpart: the per-block timeline of the dense
 * W8A8 GEMM with f16 output (the C3 path), through the kernel's traced build
 * and the tile choice pio_gemm_w8a8 makes for the shape (which must run the
 * dense direct-to-LDS engine: K % 128 == 0, not a skinny or split-K shape).
 * trace gets 4 stamps per block of the 100 MHz constant clock (start, K loop
 * done, stores issued, stores complete); returns how many 4-word entries to
 * read (entries of blocks the chosen grid lacks stay 0), or a negative
 * status. */
int pio_probe_gemm_timeline(const int8_t* q, const float* s_a, const int8_t* w, const float* s_w, void* y, int M,
                            int N, int K, unsigned long long* trace, int trace_words, void* stream);
/* Persistent launches of this decoder that were re-run in graph mode because
 * the device could not hold their grid at once. No counterpart in the
 * reference. */
int pio_qwen3_persistent_replays(void* dec);
/* Waits for the stream (re-running steps of persistent launches that could
 * not start, see pio_qwen3_run), then copies out ids[0..n) and, if
 * logits != NULL, the last step's logits [vocab]. Reports an error if a
 * persistent run since the last read gave up on a wait (its results are then
 * invalid). */
int pio_qwen3_read(void* dec, int32_t* ids, int n, float* logits);
/* Device pointer of the last step's logits ([vocab] fp32). */
const float* pio_qwen3_logits(void* dec);

/* ---------------------------------------------------------------------------
 * int8 on-disk weights: safetensors reading.
 *
 * The reference loads checkpoints through plugins/cpu/c_src/safetensors_loader.c
 * (bound at core/engine/backend.py:120-126, driven by load_safetensors,
 * backend.py:812-835). That loader searches the header text for the name and
 * picks F32 or F16 from the byte count, so BF16 is misread and I8 is refused.
 * Here the header is parsed into a table and conversions follow the stored
 * dtype; the three reference entry points keep their signatures and return
 * conventions. A context is read-only after open and may be shared by threads.
 * ------------------------------------------------------------------------- */

/* safetensors_loader.c:40-120. Maps the file read-only and parses its header;
 * NULL on any error (missing file, header length beyond the file, malformed
 * JSON, an entry whose offsets leave the data region or whose byte count is
 * not dtype size x shape, a duplicate name); the reason is in
 * tensor_last_error. */
void* open_safetensors(const char* filepath);
/* safetensors_loader.c:147-243. Converts tensor `name` to fp32 into `buffer`
 * (`size` fp32 elements, which must equal the tensor's element count). Reads
 * F32, F16, BF16, I8, U8, BOOL, I16 and I32 by their stored dtype (the
 * reference reads only F32 and, by byte count, F16). 1 on success, 0 if the
 * name is absent, the size differs or the dtype has no fp32 conversion. */
int load_tensor_data(void* ctx, const char* name, float* buffer, int size);
/* safetensors_loader.c:245-265. Unmaps the file; NULL is a no-op. */
void close_safetensors(void* ctx);

/* Stored dtype codes reported by pio_safetensors_info. */
enum {
    PIO_ST_F64 = 0, PIO_ST_F32 = 1, PIO_ST_F16 = 2, PIO_ST_BF16 = 3, PIO_ST_I64 = 4,
    PIO_ST_I32 = 5, PIO_ST_I16 = 6, PIO_ST_I8 = 7, PIO_ST_U8 = 8, PIO_ST_BOOL = 9,
    PIO_ST_U16 = 10, PIO_ST_U32 = 11, PIO_ST_U64 = 12,
};
/* Number of tensors in the file (__metadata__ excluded); the i-th name in
 * header order (NULL when out of range; valid until close). No reference
 * counterpart: the reference can only probe names it already knows. */
int pio_safetensors_count(void* ctx);
const char* pio_safetensors_name(void* ctx, int i);
/* Stored dtype (PIO_ST_*), rank, up to max_dims dims and byte count of
 * `name`; any output pointer may be NULL. PIO_OK or PIO_ERR_INVALID. */
int pio_safetensors_info(void* ctx, const char* name, int* dtype, int64_t* shape, int max_dims,
                         int* ndim, int64_t* nbytes);
/* The stored bytes of `name` into host memory; nbytes must equal the stored
 * size. */
int pio_safetensors_read(void* ctx, const char* name, void* dst, int64_t nbytes);
/* The stored bytes of `name` into device memory `dst` on `stream` (NULL =
 * current); returns once the bytes have landed. The bytes are read with
 * pread by up to 8 threads into two pinned 16 MiB staging buffers, one
 * filling while the other's DMA runs; the buffers and threads are
 * process-wide, made on first use and kept until exit, and device loads
 * serialize on them. */
int pio_safetensors_to_device(void* ctx, const char* name, void* dst, int64_t nbytes,
                              void* stream);
/* `name` converted to fp32 into device memory (`count` elements, which must
 * equal the tensor's): F32 is copied; BF16, F16, I8, U8, BOOL, I16 and I32
 * land raw in device scratch and are widened on the GPU (bit-exact; a
 * signalling F16 NaN comes back quiet). Returns once done. */
int pio_safetensors_to_device_f32(void* ctx, const char* name, float* dst, int64_t count,
                                  void* stream);
/* Drop-in load of `name` into a device Tensor (the tensor_load_data step of
 * backend.py:822-826 without the host fp32 round trip): an int8 tensor takes
 * I8 / U8 bytes, an fp16 tensor F16 bytes, an fp32 tensor any dtype
 * pio_safetensors_to_device_f32 converts. Element counts must match. */
void tensor_load_safetensors(void* ctx, const char* name, Tensor* out);
int tensor_load_safetensors_status(void* ctx, const char* name, Tensor* out);

/* ---------------------------------------------------------------------------
 * Drop-in: companion ops of the reference model layers on rocm:N, fp32 device
 * tensors (bound by hasattr at backend.py:60-111, 157; called by
 * qwen3_0_6b/architecture.py:16-135 through backend.py:385-600, 740-790).
 * Each follows the reference CPU loop cited; the void forms drop the status,
 * as the reference's do, and leave the message for tensor_last_error.
 * ------------------------------------------------------------------------- */

/* tensor.h:46; backend.py:63, 502; tensor_ops.c:369-383: per row of the last dimension,
 * out = x * (1 / sqrt(sum(x^2) / cols + eps)) * weight. */
void tensor_rms_norm(Tensor* input, Tensor* weight, Tensor* out, float eps);
int tensor_rms_norm_status(Tensor* input, Tensor* weight, Tensor* out, float eps);
/* backend.py:157, 515; tensor_ops_cuda.cu:914-921: x <- x + residual (in
 * place), out = rms_norm(x). */
void tensor_fused_add_rms_norm(Tensor* x, Tensor* residual, Tensor* weight, Tensor* out, float eps);
int tensor_fused_add_rms_norm_status(Tensor* x, Tensor* residual, Tensor* weight, Tensor* out,
                                     float eps);
/* tensor.h:47; backend.py:64, 508; tensor_ops.c:384-413: q [.., S, Hq, D], k [.., S, Hk, D],
 * cos / sin [>= S, D/2] (row s for position s): rotate-half RoPE. k keeps its
 * own head count (the reference walks k with q's). */
void tensor_rope(Tensor* q, Tensor* k, Tensor* cos, Tensor* sin, Tensor* out_q, Tensor* out_k);
int tensor_rope_status(Tensor* q, Tensor* k, Tensor* cos, Tensor* sin, Tensor* out_q,
                       Tensor* out_k);
/* tensor.h:44; backend.py:61, 490; tensor_ops.c:336-342: x * (1 / (1 + exp(-x))). */
void tensor_silu(Tensor* input, Tensor* out);
int tensor_silu_status(Tensor* input, Tensor* out);
/* backend.py:103, 385; tensor_ops.c:579-587: silu(gate) * up. */
void tensor_swiglu(Tensor* gate, Tensor* up, Tensor* out);
int tensor_swiglu_status(Tensor* gate, Tensor* up, Tensor* out);
/* backend.py:105, 395; tensor_ops.c:588-604: rows of [gate | up] (2h columns) ->
 * silu(gate) * up (h columns). */
void tensor_fused_gate_up_swiglu(Tensor* gate_up, Tensor* out);
int tensor_fused_gate_up_swiglu_status(Tensor* gate_up, Tensor* out);
/* tensor.h:43; backend.py:60, 484; tensor_ops.c:351-367: per row, max from -1e9, exp(x - max),
 * times 1 / sum. */
void tensor_softmax(Tensor* input, Tensor* out);
int tensor_softmax_status(Tensor* input, Tensor* out);
/* tensor.h:55; backend.py:70, 552; tensor_ops.c:649-661: per row the first index of the largest
 * value above -1e9 (0 when none), as a float. */
void tensor_argmax(Tensor* input, Tensor* out);
int tensor_argmax_status(Tensor* input, Tensor* out);
/* tensor.h:56; backend.py:71, 559; tensor_ops.c:663-671: out[i] = weight[(int)indices[i]]
 * ([vocab, dim] weight); indices outside [0, vocab) read row 0. */
void tensor_embed(Tensor* weight, Tensor* indices, Tensor* out);
int tensor_embed_status(Tensor* weight, Tensor* indices, Tensor* out);
/* backend.py:109, 771; tensor_ops.c:536-578: q [B, S, H, D], k / v [B, T, Hk, D]
 * (Hk divides H; query head h reads kv head h / (H / Hk)), out [B, S, H, D]:
 * softmax(q.k * scale) over all T keys (no mask, as the reference), the
 * weights normalised before the sum over v. T comes from k (the reference
 * loop takes q's sequence length for the keys; equal when S == T);
 * T <= 32768. */
void tensor_scaled_dot_product_attention(Tensor* q, Tensor* k, Tensor* v, Tensor* out,
                                         float scale);
int tensor_scaled_dot_product_attention_status(Tensor* q, Tensor* k, Tensor* v, Tensor* out,
                                               float scale);
/* tensor.h:50; backend.py:74, 566; tensor_ops.c:605-637: out's elements from the input at
 * start_indices + out's coordinates (offsets outside the input are
 * skipped); slice_shapes is unused, as in the reference. Rank <= 8. */
void tensor_slice(Tensor* input, Tensor* out, int* start_indices, int* slice_shapes);
int tensor_slice_status(Tensor* input, Tensor* out, int* start_indices, int* slice_shapes);
/* backend.py:78, 594; tensor_ops.c:504-535: src written into dst at
 * start_indices (the KV-cache update, architecture.py:95-96). */
void tensor_set_slice(Tensor* dst, Tensor* src, int* start_indices);
int tensor_set_slice_status(Tensor* dst, Tensor* src, int* start_indices);
/* backend.py:111; tensor_ops.c:672: out <- input's elements in order. */
void tensor_reshape(Tensor* input, Tensor* out);
int tensor_reshape_status(Tensor* input, Tensor* out);
/* tensor.h:57; backend.py:72, 740; tensor_ops.c:702-718: the inputs in order along `axis`. */
void tensor_cat(Tensor** inputs, int count, int axis, Tensor* out);
int tensor_cat_status(Tensor** inputs, int count, int axis, Tensor* out);

/* Library version string and the gfx target it was built for. */
const char* pio_version(void);

#ifdef __cplusplus
}
#endif

#endif /* INFERENCE_PIO_TENSOR_ROCM_H */
