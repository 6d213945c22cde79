/* nutllm_hip.h — C ABI of the MI355X (gfx950) token loop.
 *
 * This is the drop-in boundary under nutllm's C++17 host API: the
 * generate_tokens_cached / prefill_quantized / decode_quantized_token /
 * matvec_quantized_threaded entry points call these functions instead of the
 * reference's CPU kernels. Every function returns a status (never throws);
 * the status names the exception type the reference would have thrown, and
 * nut_last_error() gives its message ("quantized decode: token out of
 * range", ...). Citations are MokiMeow/nutllm path:line.
 *
 * Pointers named d_* are device pointers; all others are host pointers.
 * One host thread drives a handle at a time (the reference serialises calls
 * the same way, src/threading.cpp:50).
 */
#ifndef NUTLLM_HIP_H
#define NUTLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status -- */

enum {
    NUT_OK = 0,
    NUT_EINVAL = 1,      /* std::invalid_argument */
    NUT_EOUTOFRANGE = 2, /* std::out_of_range */
    NUT_ELENGTH = 3,     /* std::length_error */
    NUT_ERANGE = 4,      /* std::range_error */
    NUT_ERUNTIME = 5,    /* std::runtime_error */
    NUT_EDEVICE = 6      /* HIP runtime error or no gfx950 device */
};

/* Message of the last failing call on this thread ("" after success). */
const char *nut_last_error(void);

/* ------------------------------------------------------------- types -- */

/* QuantType (include/quant.hpp:9-12). */
enum { NUT_INT8 = 0, NUT_INT4 = 1 };

/* ModelConfig (include/model.hpp:8-24); kv_heads == 0 means heads. */
typedef struct nut_config {
    size_t layers, heads, dim, head_dim, ffn_dim, vocab_size, max_seq,
        eos_token, kv_heads;
} nut_config;

/* Host view of a QuantizedMatrix's storage (include/quant.hpp:40-49):
 * flattened row-major blocks of block_size weights; INT8 bytes or INT4
 * nibbles (even flattened index in the low nibble), fp16 scale bits. */
typedef struct nut_qmatrix {
    const uint8_t *data;
    const uint16_t *scales;
    size_t rows, cols, block_size;
    int type;
} nut_qmatrix;

/* GenerationStats (include/generate.hpp:19-24). */
typedef struct nut_generation_stats {
    size_t prefill_tokens, generated_tokens;
    double prefill_seconds, decode_seconds;
} nut_generation_stats;

/* ------------------------------------------- host utilities (no GPU) -- */

/* QuantizedMatrix::quantize (src/quant.cpp:154-197), bit-exact: data gets
 * nut_quant_data_bytes bytes, scales nut_quant_scale_count fp16 words.
 * NUT_EINVAL on non-finite weights or bad shape, NUT_ERANGE when a scale
 * exceeds fp16 (src/quant.cpp:24-27,44-45). Runs on host threads. */
int nut_quantize(const float *source, size_t rows, size_t cols, int type,
                 size_t block_size, uint8_t *data, uint16_t *scales);
size_t nut_quant_data_bytes(size_t rows, size_t cols, int type);
size_t nut_quant_scale_count(size_t rows, size_t cols, size_t block_size);
/* QuantizedMatrix::storage_bytes (src/quant.cpp:235-241). */
size_t nut_quant_storage_bytes(size_t rows, size_t cols, int type,
                               size_t block_size);
/* positive_float_to_half / positive_half_to_float (src/quant.cpp:23-56). */
int nut_float_to_half(float value, uint16_t *bits);
float nut_half_to_float(uint16_t bits);
/* ModelConfig::validate (src/attention.cpp:15-27): 1 when valid. */
int nut_config_valid(const nut_config *config);

/* Synthetic workload generator (no reference counterpart: the reference
 * loads checkpoints). N(0, sigma^2) fp32 values from a counter-based
 * splitmix64 + Box-Muller stream keyed by (seed, stream); element i depends
 * only on (seed, stream, i), so any thread count gives the same array. */
int nut_synth_normal(uint64_t seed, uint64_t stream, float sigma, float *out,
                     size_t count);
/* Uniform token ids in [0, vocab) (rejection sampled) from seed. */
int nut_synth_tokens(uint64_t seed, size_t vocab, int *out, size_t count);

/* ------------------------------------------------- device and memory -- */

/* Number of visible gfx950 devices (0 on a host without a GPU). */
int nut_device_count(int *count);
/* Select the device this thread's calls use (default 0). */
int nut_set_device(int device);
int nut_malloc(void **d_ptr, size_t bytes);
int nut_free(void *d_ptr);
/* Device allocations (hipMalloc calls) this library has made since it was
 * loaded, its own and nut_malloc's (no reference counterpart: a
 * diagnostic, for checking that nut_decode_noalloc allocates nothing). */
int nut_device_allocations(unsigned long long *count);
int nut_memcpy_h2d(void *d_dst, const void *src, size_t bytes);
int nut_memcpy_d2h(void *dst, const void *d_src, size_t bytes);
/* Device-to-device copy (synchronous); also the known-size copy that
 * calibrates HBM traffic counters. */
int nut_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes);
int nut_memset(void *d_dst, int value, size_t bytes);
int nut_synchronize(void);

/* --------------------------------------------- standalone kernels -- */

/* A QuantizedMatrix uploaded to HBM (weights verbatim, fp16 scales). */
typedef struct nut_qweight nut_qweight;
int nut_qweight_create(const nut_qmatrix *host, nut_qweight **out);
int nut_qweight_destroy(nut_qweight *w);
size_t nut_qweight_device_bytes(const nut_qweight *w);

/* y = W x on the device: matvec_quantized_threaded (src/quant.cpp:262-321).
 * stream may be NULL (the null stream). */
int nut_matvec_q(const nut_qweight *w, const float *d_x, float *d_y,
                 void *stream);
/* fp32 y = W x, W [rows x cols] row-major: matvec_threaded
 * (src/threading.cpp:183-198), the classifier kernel. */
int nut_matvec_f32(const float *d_w, size_t rows, size_t cols,
                   const float *d_x, float *d_y, void *stream);
/* fp32 C = A B, row-major A [m x k], B [k x n]: matmul_threaded
 * (src/threading.cpp:163-181). */
int nut_matmul_f32(const float *d_a, const float *d_b, float *d_c, size_t m,
                   size_t k, size_t n, void *stream);

/* Launch-time of the last nut_matvec_q / nut_matvec_f32 / nut_matmul_f32
 * batch measured with HIP events: call nut_timer_begin(stream), launch,
 * then nut_timer_end(stream, &ms) waits and returns elapsed milliseconds on
 * that stream. (No reference counterpart; the reference times with
 * std::chrono around whole calls.) */
int nut_timer_begin(void *stream);
int nut_timer_end(void *stream, double *milliseconds);

/* ------------------------------------------------------------- model -- */

typedef struct nut_model nut_model;

/* QuantizedModelWeights (include/quant_model.hpp:32-46): validates config,
 * allocates device storage for every layer; tied selects embeddings as the
 * classifier (output_weights(), include/quant_model.hpp:42-44). */
int nut_model_create(const nut_config *config, int type, int tied,
                     nut_model **out);
/* fp32 embeddings [vocab x dim], final_norm [dim], lm_head [vocab x dim]
 * (ignored when tied). */
int nut_model_set_globals(nut_model *m, const float *embeddings,
                          const float *final_norm, const float *lm_head);
/* QuantizedLayerWeights (include/quant_model.hpp:9-30): projections in
 * [out x in] layout: query dim x dim, key/value kv_dim x dim, output
 * dim x dim, gate/up ffn x dim, down dim x ffn. */
int nut_model_set_layer(nut_model *m, size_t layer, const nut_qmatrix *query,
                        const nut_qmatrix *key, const nut_qmatrix *value,
                        const nut_qmatrix *output, const nut_qmatrix *gate,
                        const nut_qmatrix *up, const nut_qmatrix *down,
                        const float *attention_norm, const float *ffn_norm);
/* QuantizedModelWeights::storage_bytes (src/quant_model.cpp:140-156). */
size_t nut_model_storage_bytes(const nut_model *m);
/* load_llama2c_quantized_model (src/llama2.cpp:339-412) straight into a
 * device model: the reference's header and size checks and messages
 * (src/llama2.cpp:199-296, run before the device is touched), pread of one
 * projection at a time, the product quantiser (bit-exact with
 * QuantizedMatrix::quantize) on a worker thread overlapping the upload of
 * the previous layer. A positive vocabulary in the header ties the
 * classifier to the embeddings; eos_token is 1. *load_seconds (may be
 * NULL) gets the load's wall time, the reference CLI's load_s
 * (src/cli.cpp:165-169). */
int nut_model_load_llama2c(const char *path, int type, nut_model **out,
                           double *load_seconds);
/* The configuration, quant type and tied flag a model was created with. */
int nut_model_config(const nut_model *m, nut_config *config, int *type,
                     int *tied);
int nut_model_destroy(nut_model *m);

/* ---------------------------------------------------------- KV cache -- */

/* KVCache (include/kvcache.hpp:8-31, src/kvcache.cpp:173-235): fp32 K and
 * V in HBM, [layer][kv_head][position][head_dim]. */
typedef struct nut_kvcache nut_kvcache;
int nut_kv_create(const nut_config *config, nut_kvcache **out);
int nut_kv_destroy(nut_kvcache *kv);
size_t nut_kv_length(const nut_kvcache *kv);
size_t nut_kv_capacity(const nut_kvcache *kv);
size_t nut_kv_memory_bytes(const nut_kvcache *kv);
int nut_kv_compatible(const nut_kvcache *kv, const nut_config *config);
int nut_kv_reset(nut_kvcache *kv);
int nut_kv_set_length(nut_kvcache *kv, size_t length);
/* KVCache::key / value: copy one [head_dim] row to the host. */
int nut_kv_read(const nut_kvcache *kv, size_t layer, size_t head,
                size_t position, float *key, float *value);
/* KVCache::store: key/value are [kv_heads x head_dim] host vectors. */
int nut_kv_store(nut_kvcache *kv, size_t layer, size_t position,
                 const float *key, const float *value);
/* KVCache::key / value / store over a run of positions at once (one
 * strided copy each way): host arrays [layer][kv_head][end - begin]
 * [head_dim]. Read-back or upload only: the length is not changed. Either
 * output of the read may be NULL. */
int nut_kv_read_positions(const nut_kvcache *kv, size_t begin, size_t end,
                          float *keys, float *values);
int nut_kv_write_positions(nut_kvcache *kv, size_t begin, size_t end,
                           const float *keys, const float *values);

/* -------------------------------------------------------- token loop -- */

/* decode_quantized_token (src/quant_model.cpp:158-206): one token through
 * every layer at position = length; writes the pre-final-norm hidden state
 * [dim] to hidden (host, may be NULL) and increments the length. */
int nut_decode(nut_model *m, nut_kvcache *kv, int token, float *hidden);
/* nut_decode without allocating (no reference counterpart): for callers
 * that cannot call hipMalloc (tight serving loops, harnesses that forbid
 * it). It allocates nothing, but it is not itself capturable: it runs
 * eagerly on the model's own stream and synchronizes it before returning.
 * Same validation and result as nut_decode on the step kernels
 * (NUT_PATH_STEPS); the split-attention partials and arrival counters live
 * in a per-device 2 MiB scratch array instead of model-owned allocations,
 * and the hidden state goes to the device pointer d_hidden (may be NULL). Limit: heads x splits x
 * (head_dim + 2) words of 8 bytes plus 2 x heads counters must fit 2 MiB,
 * else NUT_EINVAL (TinyLlama needs 0.55 MiB, Llama-2-7B 0.27). Every call
 * on one GPU shares that GPU's array and clears it first: calls that
 * overlap on one GPU (other host threads, other streams) race. */
int nut_decode_noalloc(nut_model *m, nut_kvcache *kv, int token,
                       float *d_hidden);
/* prefill_quantized (src/quant_model.cpp:208-220): resets the cache and
 * runs the prompt; hidden gets the last token's hidden state. */
int nut_prefill(nut_model *m, nut_kvcache *kv, const int *tokens,
                size_t count, float *hidden);
/* Final rmsnorm + fp32 classifier (src/generate.cpp:197-200) on a host
 * hidden state; logits [vocab] to the host. */
int nut_logits(nut_model *m, const float *hidden, float *logits);
/* Greedy generate_tokens_cached (src/generate.cpp:174-216) with its
 * GenerationStats timing; out receives up to max_tokens ids, stopping at
 * eos_token or a full cache. The loop runs on the device: the argmax of
 * each step feeds the next step without a host round trip. */
int nut_generate_greedy(nut_model *m, const int *prompt, size_t prompt_len,
                        size_t max_tokens, int *out, size_t *out_count,
                        nut_generation_stats *stats);

/* generate_tokens_cached with SamplingConfig{max_tokens, temperature,
 * top_p, seed} (src/generate.cpp:31-72,174-216): temperature <= 0 is the
 * greedy loop above; otherwise each step's logits, softmax numerators
 * p = exp((logit - max) / temperature) and their sort (p descending, token
 * ascending) run on the device, and the host walks the sorted prefix with
 * the reference's sequential nucleus sum and draws with std::mt19937(seed)
 * and uniform_real_distribution<double>, as choose_token does. Errors as
 * the reference's: "sampling: invalid temperature or top-p"
 * (NUT_EINVAL), "sampling: non-finite probability" and "sampling: zero
 * probability mass" (NUT_ERUNTIME). */
int nut_generate_sampled(nut_model *m, const int *prompt, size_t prompt_len,
                         size_t max_tokens, float temperature, float top_p,
                         uint32_t seed, int *out, size_t *out_count,
                         nut_generation_stats *stats);

/* ---------------------------------------------------- fp32 model path -- */

/* ModelWeights (include/loader.hpp:46-60) in HBM: fp32 embeddings
 * [vocab x dim], final_norm [dim], lm_head [vocab x dim] (ignored when
 * tied), and per layer the projections in the reference's [in x out]
 * layout (LayerWeights, src/attention.cpp:29-40): query dim x dim, key and
 * value dim x kv_dim, output dim x dim, gate and up dim x ffn, down
 * ffn x dim. The KV cache is the same nut_kvcache. */
typedef struct nut_fmodel nut_fmodel;
int nut_fmodel_create(const nut_config *config, int tied, nut_fmodel **out);
int nut_fmodel_set_globals(nut_fmodel *m, const float *embeddings,
                           const float *final_norm, const float *lm_head);
int nut_fmodel_set_layer(nut_fmodel *m, size_t layer, const float *query,
                         const float *key, const float *value,
                         const float *output, const float *gate,
                         const float *up, const float *down,
                         const float *attention_norm, const float *ffn_norm);
int nut_fmodel_destroy(nut_fmodel *m);
/* decode_token (src/kvcache.cpp:264-284): one token at position = length;
 * hidden (host, may be NULL) gets the hidden state after the last layer. */
int nut_decode_token(nut_fmodel *m, nut_kvcache *kv, int token,
                     float *hidden);
/* prefill_tokens (src/kvcache.cpp:237-262): resets the cache and runs the
 * tokens; rows (host, may be NULL) gets every token's hidden state,
 * [count x dim]. */
int nut_prefill_tokens(nut_fmodel *m, nut_kvcache *kv, const int *tokens,
                       size_t count, float *rows);

/* Execution path of decode / prefill / generate (no reference counterpart;
 * every path computes the same function): NUT_PATH_AUTO picks the
 * cooperative token kernel when the shape has an instantiation and the
 * context fits its attention (fused up to 44-48 positions, split over the
 * grid up to 4,096), else per-phase step kernels; NUT_PATH_STEPS forces the
 * step kernels; NUT_PATH_TOKEN forces the token kernel and fails with
 * NUT_EINVAL where it does not apply. */
enum { NUT_PATH_AUTO = 0, NUT_PATH_STEPS = 1, NUT_PATH_TOKEN = 2 };
int nut_model_set_path(nut_model *m, int path);

/* Phase timeline of the cooperative token kernel, for profiling (no
 * reference counterpart). mode 0 records nothing, 1 workgroup 0, 2 every
 * workgroup of the grid (256): each stamps the device's constant 100 MHz
 * clock at each phase boundary; per decode iteration 4 + 13 * layers
 * entries: iteration start, classifier input staged, classifier pass done,
 * token known (the generate loop; zero in the prefill loop), then per
 * layer the times its QKV
 * input is staged, QKV published, Wo/K/V DMA issued, attention input
 * staged, attention done, Wo published, gate/up DMA issued, FFN input
 * staged, gate/up published, down DMA issued, down input staged, down
 * published and next QKV DMA issued. Entries are
 * [workgroup][max_seq iterations][marks].
 * nut_model_timeline copies up to capacity entries of the last launch's
 * timeline. */
int nut_model_record_timeline(nut_model *m, int mode);
int nut_model_timeline(const nut_model *m, uint64_t *ticks, size_t capacity,
                       size_t *count);

/* Exchange-tag schedule of the cooperative token kernel (no reference
 * counterpart). Every launch polls words tagged with its own base; a base
 * is never 0 and never repeats until the exchange buffer has been zeroed.
 * nut_token_tag_base advances *launch_count and returns the next launch's
 * base, with *clear = 1 when the buffer must be zeroed first (the counter
 * ran out and restarted); it needs no GPU. nut_model_set_launch_count
 * presets a model's counter (a test hook, to cross the restart quickly). */
int nut_token_tag_base(unsigned *launch_count, unsigned *base, int *clear);
int nut_model_set_launch_count(nut_model *m, unsigned launch_count);
/* Test hook of the cooperative token kernel's bounded waits (no reference
 * counterpart): with fault = 1, workgroup 0 of every later launch leaves
 * its words of the first step's h after W2 unpublished, so every wait for
 * them runs into its spin limit; the launch must still end, and the call
 * fail with NUT_EDEVICE ("token kernel: phase exchange timed out").
 * fault = 0 restores normal launches. */
int nut_model_inject_fault(nut_model *m, int fault);

/* Device time (HIP events on the model's stream) of the decode loop of the
 * last nut_generate_greedy call: every classifier, argmax and decode step
 * after the prefill. (No reference counterpart: GenerationStats carries
 * host wall time only.) */
int nut_model_last_decode_ms(const nut_model *m, double *milliseconds);

#ifdef __cplusplus
}
#endif
#endif
