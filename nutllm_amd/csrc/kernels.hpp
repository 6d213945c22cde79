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
// Final rmsnorm + fp32 classifier; logits may be null. Writes per-block
// argmax partials (value, index) for launch_pick_token.
int classifier_blocks(const DecodeShape &s);
void launch_classifier(const DecodeShape &s, const float *hidden,
                       const float *final_norm, const float *weights,
                       float *logits, float *part_val, int *part_idx,
                       const StepState *state, hipStream_t stream);
// Reduce the partials to the first maximal index; on eos set done, else
// append to tokens and make it the next input token.
void launch_pick_token(const DecodeShape &s, const float *part_val,
                       const int *part_idx, int parts, StepState *state,
                       int *tokens, hipStream_t stream);
// Tiny state writers, enqueued on the stream (graph-safe, no memset).
void launch_set_int(int *target, int value, hipStream_t stream);
void launch_reset_state(StepState *state, int token, hipStream_t stream);

} // namespace nut
