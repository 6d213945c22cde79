// model.hpp — device-resident model, KV cache and token loop behind the C
// ABI (the objects nut_model / nut_kvcache point to).
#pragma once

#include <memory>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

struct nut_model;
struct nut_kvcache;

namespace nut {

struct DeviceLayer {
    // Own storage of a layer whose blocks are not 32 wide; layers with
    // 32-wide blocks live in the model's arena instead.
    DeviceBuffer storage;
    LayerView view{};
    // The prefill GEMM's stage-major copy of the seven matrices' scales
    // (query, key, value, output, gate, up, down), when every matrix has
    // 32-wide blocks in whole 64-wide stages.
    DeviceBuffer stage_scales;
    const uint32_t *stage_scale[7]{};
    bool in_arena = false;
    size_t storage_bytes = 0; // reference storage accounting
    bool set = false;
};

} // namespace nut

// KVCache on the device (include/kvcache.hpp:8-31): keys and values are
// [layer][kv_head][position][head_dim] fp32, as src/kvcache.cpp:196-205.
struct nut_kvcache {
    nut_config config{};
    nut::DeviceBuffer keys, values;
    nut::DeviceBuffer device_length; // int, read by the step kernels
    size_t length = 0;               // host copy, authoritative

    size_t kv_heads() const
    {
        return config.kv_heads == 0 ? config.heads : config.kv_heads;
    }
    size_t layer_elements() const
    {
        return kv_heads() * config.max_seq * config.head_dim;
    }
    void sync_length(hipStream_t stream);
};

struct nut_model {
    nut_config config{};
    int type = 0;
    bool tied = false;
    nut::DecodeShape shape{};
    std::vector<nut::DeviceLayer> layers;
    nut::DeviceBuffer embeddings, final_norm, lm_head, rope;
    // The classifier's INT8 screening copy (codes, block scales) for the
    // token kernels' argmax, built at the first generate after set_globals.
    nut::DeviceBuffer classifier8, classifier8_scales;
    bool screen_ready = false;
    // Weight arena: layer l at arena + l * layout.bytes (LayerLayout).
    nut::DeviceBuffer arena;
    nut::LayerLayout layout{};
    bool globals_set = false;

    // Step workspace.
    nut::DeviceBuffer hidden, query, context, act, logits, scratch_hidden;
    nut::DeviceBuffer attn_part, attn_count; // fast step kernels
    // Prompt chunks on the step kernels: kStepTokensMax rows each.
    nut::DeviceBuffer mt_hidden, mt_query, mt_context, mt_act;
    // One greedy iteration (classifier, argmax, decode step) captured as a
    // graph for the generation cache; replayed once per generated token.
    hipGraphExec_t step_graph = nullptr;
    nut::DeviceBuffer part_val, part_idx, state, tokens, prompt;
    hipStream_t stream = nullptr;
    hipEvent_t decode_begin = nullptr, decode_end = nullptr;
    // Cooperative token kernel state.
    int path = 0; // 0 auto, 1 step kernels, 2 token kernel
    nut::DeviceBuffer exchange, token_error, timeline;
    nut::DeviceBuffer exchange_once; // write-once words of fused-attention launches
    // Prefill GEMM path: activations of a whole prompt, max_seq rows each.
    nut::DeviceBuffer pf_h, pf_x, pf_q, pf_ctx, pf_act;
    nut::DeviceBuffer pf_kv; // the batch's K and V as f16 limbs (prefill attention)
    nut::DeviceBuffer sample_ws; // sampling: numerators, sort buffers
    size_t timeline_entries = 0; // > 0 when the phase timeline is recorded
    int timeline_wgs = 0;        // workgroups it covers
    unsigned launch_count = 0;
    int fault = 0; // nut_model_inject_fault
    double last_decode_device_ms = 0.0; // events around the decode loop
    std::unique_ptr<nut_kvcache> generation_cache;

    ~nut_model();
    const float *output_weights() const
    {
        return tied ? embeddings.as<float>() : lm_head.as<float>();
    }
};

namespace nut {

nut_model *create_model(const nut_config &config, int type, bool tied);
void set_globals(nut_model &m, const float *embeddings,
                 const float *final_norm, const float *lm_head);
void set_layer(nut_model &m, size_t layer, const nut_qmatrix *const mats[7],
               const float *attention_norm, const float *ffn_norm);
size_t storage_bytes(const nut_model &m);

nut_kvcache *create_kv(const nut_config &config);
bool kv_compatible(const nut_kvcache &kv, const nut_config &config);

void decode(nut_model &m, nut_kvcache &kv, int token, float *hidden);
// decode on the step kernels with the attention workspace in the
// per-device scratch array (noalloc.hpp); d_hidden is a device pointer.
void decode_noalloc(nut_model &m, nut_kvcache &kv, int token, float *d_hidden);
void prefill(nut_model &m, nut_kvcache &kv, const int *tokens, size_t count,
             float *hidden);
void logits(nut_model &m, const float *hidden, float *out);
void generate_greedy(nut_model &m, const int *prompt, size_t prompt_len,
                     size_t max_tokens, int *out, size_t *out_count,
                     nut_generation_stats *stats);
// generate_tokens_cached with temperature / top-p sampling: device logits,
// numerators and sort (sample.hip), the reference's sequential nucleus sum
// and std::mt19937 draw on the host.
void generate_sampled(nut_model &m, const int *prompt, size_t prompt_len,
                      size_t max_tokens, float temperature, float top_p, uint32_t seed,
                      int *out, size_t *out_count, nut_generation_stats *stats);

bool config_valid(const nut_config &c);

// RoPE cos/sin table [max_seq][head_dim / 2] of (cos, sin) as fp32, from the
// reference's double-precision formula (src/quant_model.cpp:26-37).
std::vector<float> rope_table(const nut_config &c);

// load_llama2c_quantized_model (src/llama2.cpp:339-412) into a device model;
// *seconds gets the wall time of the whole load (may be null).
nut_model *load_llama2c(const char *path, int type, double *seconds);

} // namespace nut
