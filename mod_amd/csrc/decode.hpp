// Decoder state shared by the step kernels (decode.hip) and the persistent
// decode loop (decode_loop.hip).
#pragma once

#include "pio_common.hpp"

#include <vector>

namespace pio {

constexpr int DEC_MAX_SEQ = 8192;
constexpr int ATT_SPLITS = 8;   // attention splits over key positions

struct LoopState;               // decode_loop.hip

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
    float *x, *q, *att_o, *att_ml, *act, *logits, *cos_t, *sin_t;
    void *kc, *vc;         // KV cache, fp32 or fp16 elements (kv16)
    bool kv16 = false;
    int32_t *state, *ids;
    unsigned long long* part_keys;
    int lm_blocks = 0;
    size_t att_lds = 0;
    int host_pos = 0;
    int prompt_len = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    LoopState* loop = nullptr;   // persistent-loop resources, built on first use
};

// Persistent decode loop (decode_loop.hip): one launch (a workgroup per CU) runs
// n_steps tokens. loop_check() says whether the config fits its kernel.
int loop_check(const Qwen3Dec* d);
int loop_run(Qwen3Dec* d, int n_steps);
// Error words of the persistent launches since the last call; call after the
// stream has drained. LOOP_REPLAY: a launch found the grid not co-resident
// (other work held CUs), so it and every launch after it computed nothing;
// *replay_pos is the first position to run again.
constexpr int LOOP_REPLAY = 1;
int loop_status(Qwen3Dec* d, int* replay_pos);
int loop_replays(const Qwen3Dec* d);
bool loop_pending(const Qwen3Dec* d);   // persistent launches not yet checked
// Phase timeline: the next persistent launch runs the traced kernel and stamps
// steps first_step, first_step + 1 of it (u64 [2][256][n_layers + 1][12]).
size_t loop_trace_bytes(const Qwen3Dec* d);
int loop_trace_next(Qwen3Dec* d, int first_step);
int loop_trace_read(Qwen3Dec* d, void* out, size_t bytes);
int loop_refresh(Qwen3Dec* d);
void loop_destroy(Qwen3Dec* d);

// The step kernels' tail (decode.hip): lm_head on the decoder's x with the
// final RMSNorm, argmax, then ids[pos + 1] (past the prompt) and pos += 1.
int enqueue_lm(Qwen3Dec* d);

// Batched prompt (prefill.hip): the next M positions (all prompt positions) in
// one pass per layer; with `logits`, the last one's logits and argmax as its
// step would produce them. Advances the position by M.
int prefill(Qwen3Dec* d, int M, bool logits);

}  // namespace pio
