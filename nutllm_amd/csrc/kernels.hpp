// kernels.hpp — host-side launchers of the gfx950 kernels (internal API).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.hpp"

namespace nut {

// Device step state of a decode loop: the token being decoded, whether the
// loop reached eos, and how many tokens it emitted.
struct StepState {
    int token;
    int done;
    int count;
    int pad;
};

// Standalone kernels (matvec.hip).
void launch_matvec_q(const QMat &m, const float *x, float *y,
                     hipStream_t stream);
void launch_matvec_f32(const float *w, int rows, int cols, const float *x,
                       float *y, hipStream_t stream);
void launch_matmul_f32(const float *a, const float *b, float *c, int m, int k,
                       int n, hipStream_t stream);
size_t matvec_q_lds_bytes(const QMat &m);

// Decode-step kernels (decode.hip).
struct LayerView {
    QMat query, key, value, output, gate, up, down;
    const float *attention_norm, *ffn_norm;
};

// Byte layout of one layer in the model's weight arena (every layer
// identical, pieces 256-byte aligned, block size 32): for query, key,
// value, output, gate, up, down in turn the packed data then the fp16
// scales, then the attention and ffn norm vectors. Layer l starts at
// l * bytes, so a kernel addresses any weight without loading pointers.
struct LayerLayout {
    size_t data[7], scales[7], attention_norm, ffn_norm, bytes;
};

__host__ __device__ constexpr size_t align256(size_t v)
{
    return (v + 255) / 256 * 256;
}

__host__ __device__ constexpr LayerLayout layer_layout(int type, size_t dim,
                                                       size_t ffn, size_t kvd)
{
    LayerLayout l{};
    const size_t rows[7] = {dim, kvd, kvd, dim, ffn, ffn, dim};
    const size_t cols[7] = {dim, dim, dim, dim, dim, dim, ffn};
    size_t total = 0;
    for (int i = 0; i < 7; i++) {
        const size_t n = rows[i] * cols[i];
        l.data[i] = total;
        total = align256(total + (type == 1 ? (n + 1) / 2 : n));
        l.scales[i] = total;
        total = align256(total + 2 * ((n + 31) / 32));
    }
    l.attention_norm = total;
    l.ffn_norm = total + dim * 4;
    l.bytes = align256(total + 2 * dim * 4);
    return l;
}

struct DecodeShape {
    int dim, heads, kv_heads, head_dim, ffn_dim, vocab, max_seq, eos;
    float attn_scale;
};

void launch_embed(const DecodeShape &s, const float *embeddings,
                  const int *token_ptr, const StepState *state, float *hidden,
                  hipStream_t stream);
void launch_layer(const DecodeShape &s, const LayerView &w,
                  const float2 *rope, const int *length, float *k_layer,
                  float *v_layer, float *hidden, float *query, float *context,
                  float *act, const StepState *state, hipStream_t stream);
void launch_finish_step(const StepState *state, int *length,
                        hipStream_t stream);
// GQA attention of one decode step (attention_step's softmax and context,
// src/quant_model.cpp:68-105): query [heads][head_dim] at position *length
// over cached positions 0..*length, context [heads][head_dim].
void launch_attention(const DecodeShape &s, const float *query, const float *k_layer,
                      const float *v_layer, const int *length, float *context,
                      const StepState *state, hipStream_t stream);
// Final rmsnorm + fp32 classifier; logits may be null. Writes per-block
// argmax partials (value, index) for launch_pick_token.
int classifier_blocks(const DecodeShape &s);
void launch_classifier(const DecodeShape &s, const float *hidden,
                       const float *final_norm, const float *weights,
                       float *logits, float *part_val, int *part_idx,
                       const StepState *state, hipStream_t stream);
// The classifier's screening copy for the token kernels' argmax: INT8
// block-32 codes (vocab x dim) and fp16 block scales (vocab x dim / 32),
// each scale the smallest fp16 >= the block's max |w| / 127.
void launch_classifier_screen(const float *weights, int vocab, int dim, int8_t *codes,
                              uint16_t *scales, hipStream_t stream);
// Reduce the partials to the first maximal index; on eos set done, else
// append to tokens and make it the next input token.
void launch_pick_token(const DecodeShape &s, const float *part_val,
                       const int *part_idx, int parts, StepState *state,
                       int *tokens, hipStream_t stream);
// Fast step kernels (step.hip): layers whose matrices all use 32-wide
// blocks along whole rows, head_dim 64 or 128, 1, 2, 4 or 8 query heads per
// KV head. One launch runs 1 .. kStepTokensMax consecutive tokens at
// positions *length, *length + 1, ...: hidden, query and context hold a
// [tokens][dim] row per token, act a [tokens][ffn] row. attn_part holds
// step_attn_part_words(s) words, every byte 0xff before the first step;
// attn_count holds 2 * heads * kStepTokensMax ints, zero before the first
// step (the kernels keep both consistent from then on). 31 tokens: one
// chunk costs about 0.55 ms plus 0.09 ms per token on the TinyLlama INT4
// shape, so a prompt below the batched-prefill threshold runs as one chunk
// (15-token chunks took 2.81 ms for 20 tokens, one chunk 2.28 ms).
constexpr int kStepTokensMax = 31;
struct StepBuffers {
    float *hidden, *query, *context, *act;
    uint64_t *attn_part;
    int *attn_count;
};
bool step_fast_supported(const DecodeShape &s, const LayerView &w);
size_t step_attn_part_words(const DecodeShape &s);
void launch_layer_fast(const DecodeShape &s, const LayerView &w,
                       const float2 *rope, const int *length, float *k_layer,
                       float *v_layer, const StepBuffers &b, int tokens,
                       const StepState *state, hipStream_t stream);

// Tiny state writers, enqueued on the stream (graph-safe, no memset).
void launch_set_int(int *target, int value, hipStream_t stream);
void launch_reset_state(StepState *state, int token, hipStream_t stream);

} // namespace nut
