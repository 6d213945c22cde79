// fmodel.hpp — the fp32 model path on the device: ModelWeights
// (include/loader.hpp) in HBM, and decode_token / prefill_tokens
// (src/kvcache.cpp:237-284) over the device KV cache.
#pragma once

#include <vector>

#include "model.hpp"

// ModelWeights resident in HBM. Projections keep the reference's [in x out]
// layout (LayerWeights, src/attention.cpp:29-40): query dim x dim, key and
// value dim x kv_dim, output dim x dim, gate and up dim x ffn, down
// ffn x dim.
struct nut_fmodel {
    struct Layer {
        nut::DeviceBuffer w[7]; // query, key, value, output, gate, up, down
        nut::DeviceBuffer attention_norm, ffn_norm;
        bool set = false;
    };
    nut_config config{};
    bool tied = false;
    bool globals_set = false;
    nut::DecodeShape shape{};
    std::vector<Layer> layers;
    nut::DeviceBuffer embeddings, final_norm, lm_head, rope;
    // workspace of one decode step
    nut::DeviceBuffer hidden, query, context, act, partial, state, token;
    hipStream_t stream = nullptr;
    ~nut_fmodel();
};

namespace nut {

nut_fmodel *create_fmodel(const nut_config &config, bool tied);
void set_fglobals(nut_fmodel &m, const float *embeddings, const float *final_norm,
                  const float *lm_head);
void set_flayer(nut_fmodel &m, size_t layer, const float *const w[7],
                const float *attention_norm, const float *ffn_norm);
// decode_token: the hidden state after every layer (not normalised) to
// hidden (host, may be null); the cache length grows by one.
void decode_token(nut_fmodel &m, nut_kvcache &kv, int token, float *hidden);
// prefill_tokens: resets the cache, runs the tokens in order and writes
// every token's hidden state to rows [count x dim] (host, may be null).
void prefill_tokens(nut_fmodel &m, nut_kvcache &kv, const int *tokens, size_t count,
                    float *rows);

} // namespace nut
