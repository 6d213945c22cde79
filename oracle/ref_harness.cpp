/* ref_harness.cpp — C entry points over the compiled reference.
 *
 * TEST INFRASTRUCTURE. oracle/Makefile compiles this file together with the
 * reference's own sources, where they lie, into oracle/_ref/libnutref.so.
 * It is used to pin the C oracle (golden vectors) and as the "reference"
 * CPU baseline. Nothing here is product code, and no reference source is
 * copied: the reference headers are included from the reference tree.
 *
 * QuantizedMatrix keeps data_/scales_ private (include/quant.hpp:39-49); the
 * harness opens them with a preprocessor switch so golden bytes and fp16
 * scale bits can be read exactly.
 */
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <vector>

#define private public
#include "quant.hpp"
#undef private
#include "generate.hpp"
#include "kvcache.hpp"
#include "loader.hpp"
#include "matmul.hpp"
#include "ops.hpp"
#include "quant_model.hpp"

namespace {

int status_of(const std::exception &e)
{
    if (dynamic_cast<const std::out_of_range *>(&e))
        return 2;
    if (dynamic_cast<const std::length_error *>(&e))
        return 3;
    if (dynamic_cast<const std::range_error *>(&e))
        return 4;
    if (dynamic_cast<const std::invalid_argument *>(&e))
        return 1;
    return 5;
}

QuantType qtype(int type) { return type == 0 ? QuantType::int8 : QuantType::int4; }

ModelConfig config_of(const size_t *c)
{
    ModelConfig config;
    config.layers = c[0];
    config.heads = c[1];
    config.dim = c[2];
    config.head_dim = c[3];
    config.ffn_dim = c[4];
    config.vocab_size = c[5];
    config.max_seq = c[6];
    config.eos_token = c[7];
    config.kv_heads = c[8];
    return config;
}

Matrix matrix_of(const float *source, size_t rows, size_t cols)
{
    Matrix m(rows, cols);
    std::memcpy(m.data(), source, rows * cols * sizeof(float));
    return m;
}

} // namespace

#define GUARD_BEGIN try {
#define GUARD_END                                                            \
    }                                                                        \
    catch (const std::exception &e) { return status_of(e); }                 \
    return 0;

extern "C" {

/* Quantise with the reference; copy out the raw bytes, fp16 scale bits,
 * storage_bytes() and error_bound() per element (bounds may be null). */
int ref_quantize(const float *source, size_t rows, size_t cols, int type,
                 size_t block_size, uint8_t *data, uint16_t *scales,
                 size_t *storage, float *bounds)
{
    GUARD_BEGIN
    QuantizedMatrix q =
        QuantizedMatrix::quantize(source, rows, cols, qtype(type), block_size);
    std::memcpy(data, q.data_.data(), q.data_.size());
    std::memcpy(scales, q.scales_.data(), q.scales_.size() * sizeof(uint16_t));
    *storage = q.storage_bytes();
    if (bounds != nullptr)
        for (size_t r = 0; r < rows; r++)
            for (size_t c = 0; c < cols; c++)
                bounds[r * cols + c] = q.error_bound(r, c);
    GUARD_END
}

/* matvec_quantized_threaded on a matrix quantised by the reference. */
int ref_matvec_q(const float *source, size_t rows, size_t cols, int type,
                 size_t block_size, const float *x, float *y, size_t threads)
{
    GUARD_BEGIN
    QuantizedMatrix q =
        QuantizedMatrix::quantize(source, rows, cols, qtype(type), block_size);
    matvec_quantized_threaded(q, x, y, threads);
    GUARD_END
}

int ref_matvec_f32(const float *w, size_t rows, size_t cols, const float *x,
                   float *y, size_t threads)
{
    GUARD_BEGIN
    Matrix m = matrix_of(w, rows, cols);
    matvec_threaded(m, x, y, threads);
    GUARD_END
}

int ref_matmul(const float *a, const float *b, float *c, size_t m, size_t k,
               size_t n, size_t threads)
{
    GUARD_BEGIN
    Matrix left = matrix_of(a, m, k), right = matrix_of(b, k, n), out(m, n);
    matmul_threaded(left, right, out, threads);
    std::memcpy(c, out.data(), m * n * sizeof(float));
    GUARD_END
}

/* Time matmul_threaded on resident matrices: returns the median seconds of
 * `repeats` calls. */
int ref_matmul_time(const float *a, const float *b, size_t m, size_t k,
                    size_t n, size_t threads, size_t repeats, double *median)
{
    GUARD_BEGIN
    Matrix left = matrix_of(a, m, k), right = matrix_of(b, k, n), out(m, n);
    std::vector<double> times;
    for (size_t i = 0; i < repeats; i++) {
        const auto t0 = std::chrono::steady_clock::now();
        matmul_threaded(left, right, out, threads);
        times.push_back(std::chrono::duration<double>(
                            std::chrono::steady_clock::now() - t0)
                            .count());
    }
    std::sort(times.begin(), times.end());
    *median = times[times.size() / 2];
    GUARD_END
}

/* Time matvec_quantized_threaded on a matrix quantised once by the
 * reference: the median seconds of `repeats` calls. */
int ref_matvec_q_time(const float *source, size_t rows, size_t cols, int type,
                      const float *x, size_t threads, size_t repeats, double *median)
{
    GUARD_BEGIN
    QuantizedMatrix q = QuantizedMatrix::quantize(source, rows, cols, qtype(type), 32);
    std::vector<float> y(rows);
    std::vector<double> times;
    matvec_quantized_threaded(q, x, y.data(), threads);
    for (size_t i = 0; i < repeats; i++) {
        const auto t0 = std::chrono::steady_clock::now();
        matvec_quantized_threaded(q, x, y.data(), threads);
        times.push_back(std::chrono::duration<double>(std::chrono::steady_clock::now() - t0)
                            .count());
    }
    std::sort(times.begin(), times.end());
    *median = times[times.size() / 2];
    GUARD_END
}

int ref_rmsnorm(const float *x, const float *w, float *out, size_t n,
                float eps)
{
    GUARD_BEGIN
    rmsnorm(x, w, out, n, eps);
    GUARD_END
}

float ref_silu(float v) { return silu(v); }

struct RefModel {
    std::unique_ptr<QuantizedModelWeights> weights;
};

int ref_model_create(const size_t *config, int type, int tied,
                     const float *embeddings, const float *final_norm,
                     const float *lm_head, void **out)
{
    GUARD_BEGIN
    const ModelConfig c = config_of(config);
    auto model = std::make_unique<RefModel>();
    model->weights = std::make_unique<QuantizedModelWeights>(c, qtype(type),
                                                             tied == 0);
    QuantizedModelWeights &m = *model->weights;
    m.tied_embeddings = tied != 0;
    std::memcpy(m.embeddings.data(), embeddings,
                c.vocab_size * c.dim * sizeof(float));
    std::memcpy(m.final_norm.data(), final_norm, c.dim * sizeof(float));
    if (!tied)
        std::memcpy(m.lm_head.data(), lm_head,
                    c.vocab_size * c.dim * sizeof(float));
    *out = model.release();
    GUARD_END
}

/* Append one layer, quantising its fp32 [out x in] projections with the
 * reference quantiser. */
int ref_model_add_layer(void *handle, const float *query, const float *key,
                        const float *value, const float *output,
                        const float *gate, const float *up, const float *down,
                        const float *attention_norm, const float *ffn_norm)
{
    GUARD_BEGIN
    QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    const ModelConfig &c = m.config;
    const QuantType t = m.quant_type;
    m.layers.emplace_back(
        QuantizedMatrix::quantize(query, c.dim, c.dim, t),
        QuantizedMatrix::quantize(key, c.kv_dim(), c.dim, t),
        QuantizedMatrix::quantize(value, c.kv_dim(), c.dim, t),
        QuantizedMatrix::quantize(output, c.dim, c.dim, t),
        QuantizedMatrix::quantize(gate, c.ffn_dim, c.dim, t),
        QuantizedMatrix::quantize(up, c.ffn_dim, c.dim, t),
        QuantizedMatrix::quantize(down, c.dim, c.ffn_dim, t),
        std::vector<float>(attention_norm, attention_norm + c.dim),
        std::vector<float>(ffn_norm, ffn_norm + c.dim));
    GUARD_END
}

/* Append one layer from already-quantised storage (bytes + fp16 scale bits
 * in the reference layout, e.g. from a quantiser shown bit-identical to
 * QuantizedMatrix::quantize). mats[i] = {data, scales} for query, key,
 * value, output, gate, up, down. */
int ref_model_add_layer_quantized(void *handle, const void *const *data,
                                  const void *const *scales,
                                  const float *attention_norm,
                                  const float *ffn_norm)
{
    GUARD_BEGIN
    QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    const ModelConfig &c = m.config;
    const size_t shapes[7][2] = {{c.dim, c.dim},     {c.kv_dim(), c.dim},
                                 {c.kv_dim(), c.dim}, {c.dim, c.dim},
                                 {c.ffn_dim, c.dim}, {c.ffn_dim, c.dim},
                                 {c.dim, c.ffn_dim}};
    std::vector<QuantizedMatrix> mats;
    for (int i = 0; i < 7; i++) {
        QuantizedMatrix q(shapes[i][0], shapes[i][1], 32, m.quant_type);
        std::memcpy(q.data_.data(), data[i], q.data_.size());
        std::memcpy(q.scales_.data(), scales[i],
                    q.scales_.size() * sizeof(uint16_t));
        mats.push_back(std::move(q));
    }
    m.layers.emplace_back(std::move(mats[0]), std::move(mats[1]),
                          std::move(mats[2]), std::move(mats[3]),
                          std::move(mats[4]), std::move(mats[5]),
                          std::move(mats[6]),
                          std::vector<float>(attention_norm, attention_norm + c.dim),
                          std::vector<float>(ffn_norm, ffn_norm + c.dim));
    GUARD_END
}

void ref_model_free(void *handle) { delete static_cast<RefModel *>(handle); }

size_t ref_model_storage_bytes(void *handle)
{
    return static_cast<RefModel *>(handle)->weights->storage_bytes();
}

/* Run prefill_quantized over tokens[0..n) one decode at a time, recording
 * each step's hidden state (n x dim) and, if given, the final K/V cache. */
int ref_decode_trace(void *handle, const int *tokens, size_t n,
                     size_t threads, float *hidden, float *keys,
                     float *values)
{
    GUARD_BEGIN
    const QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    const ModelConfig &c = m.config;
    KVCache cache(c);
    for (size_t t = 0; t < n; t++) {
        std::vector<float> h =
            decode_quantized_token(m, tokens[t], cache, threads);
        std::memcpy(hidden + t * c.dim, h.data(), c.dim * sizeof(float));
    }
    if (keys != nullptr && values != nullptr) {
        const size_t kv = c.effective_kv_heads(), hd = c.head_dim;
        for (size_t l = 0; l < c.layers; l++)
            for (size_t h = 0; h < kv; h++)
                for (size_t p = 0; p < cache.length(); p++) {
                    const size_t o = ((l * kv + h) * c.max_seq + p) * hd;
                    std::memcpy(keys + o, cache.key(l, h, p), hd * sizeof(float));
                    std::memcpy(values + o, cache.value(l, h, p),
                                hd * sizeof(float));
                }
    }
    GUARD_END
}

/* Final rmsnorm + fp32 classifier, as generate_tokens_cached does. */
int ref_logits(void *handle, const float *hidden, float *logits,
               size_t threads)
{
    GUARD_BEGIN
    const QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    std::vector<float> normalized(m.config.dim);
    rmsnorm(hidden, m.final_norm.data(), normalized.data(), m.config.dim,
            1e-5f);
    matvec_threaded(m.output_weights(), normalized.data(), logits, threads);
    GUARD_END
}

int ref_generate(void *handle, const int *prompt, size_t n, size_t max_tokens,
                 size_t threads, int *out, size_t *count,
                 double *prefill_seconds, double *decode_seconds)
{
    GUARD_BEGIN
    const QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    SamplingConfig sampling;
    sampling.max_tokens = max_tokens;
    sampling.threads = threads;
    GenerationStats stats;
    const std::vector<int> ids = generate_tokens_cached(
        m, std::vector<int>(prompt, prompt + n), sampling, &stats);
    std::memcpy(out, ids.data(), ids.size() * sizeof(int));
    *count = ids.size();
    *prefill_seconds = stats.prefill_seconds;
    *decode_seconds = stats.decode_seconds;
    GUARD_END
}

/* The decode loop of generate_tokens_cached (src/generate.cpp:194-207:
 * final rmsnorm, classifier, argmax, decode_quantized_token) for n steps
 * from a cache whose length is set to start_length (a decode step costs the
 * same whatever the cached rows hold), feeding tokens[i]; seconds gets the
 * wall time of the n steps. */
int ref_decode_time(void *handle, size_t start_length, const int *tokens, size_t n,
                    size_t threads, double *seconds)
{
    GUARD_BEGIN
    const QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    const ModelConfig &c = m.config;
    KVCache cache(c);
    cache.set_length(start_length);
    std::vector<float> last(c.dim, 0.01f), normalized(c.dim), logits(c.vocab_size);
    const auto t0 = std::chrono::steady_clock::now();
    for (size_t i = 0; i < n; i++) {
        rmsnorm(last.data(), m.final_norm.data(), normalized.data(), c.dim, 1e-5f);
        matvec_threaded(m.output_weights(), normalized.data(), logits.data(), threads);
        volatile size_t best =
            size_t(std::max_element(logits.begin(), logits.end()) - logits.begin());
        (void)best;
        last = decode_quantized_token(m, tokens[i], cache, threads);
    }
    *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    GUARD_END
}

/* generate_tokens_cached with temperature / top-p sampling. */
int ref_generate_sampled(void *handle, const int *prompt, size_t n, size_t max_tokens,
                         size_t threads, float temperature, float top_p, unsigned seed,
                         int *out, size_t *count)
{
    GUARD_BEGIN
    const QuantizedModelWeights &m = *static_cast<RefModel *>(handle)->weights;
    SamplingConfig sampling;
    sampling.max_tokens = max_tokens;
    sampling.threads = threads;
    sampling.temperature = temperature;
    sampling.top_p = top_p;
    sampling.seed = seed;
    const std::vector<int> ids = generate_tokens_cached(
        m, std::vector<int>(prompt, prompt + n), sampling, nullptr);
    std::memcpy(out, ids.data(), ids.size() * sizeof(int));
    *count = ids.size();
    GUARD_END
}

/* ------------------------------------------------ fp32 model path --- */

struct RefFModel {
    std::unique_ptr<ModelWeights> weights;
    size_t filled = 0; // layers set so far (the constructor makes them all)
};

/* ModelWeights with fp32 embeddings, final norm and (unless tied) lm_head;
 * layers appended by ref_fmodel_add_layer. */
int ref_fmodel_create(const size_t *config, int tied, const float *embeddings,
                      const float *final_norm, const float *lm_head, void **out)
{
    GUARD_BEGIN
    const ModelConfig c = config_of(config);
    auto model = std::make_unique<RefFModel>();
    model->weights = std::make_unique<ModelWeights>(c, tied == 0);
    ModelWeights &m = *model->weights;
    m.tied_embeddings = tied != 0;
    std::memcpy(m.embeddings.data(), embeddings, c.vocab_size * c.dim * sizeof(float));
    m.final_norm.assign(final_norm, final_norm + c.dim);
    if (!tied)
        std::memcpy(m.lm_head.data(), lm_head, c.vocab_size * c.dim * sizeof(float));
    *out = model.release();
    GUARD_END
}

/* The next layer's [in x out] fp32 projections (LayerWeights). */
int ref_fmodel_add_layer(void *handle, const float *query, const float *key,
                         const float *value, const float *output, const float *gate,
                         const float *up, const float *down, const float *attention_norm,
                         const float *ffn_norm)
{
    GUARD_BEGIN
    RefFModel &r = *static_cast<RefFModel *>(handle);
    ModelWeights &m = *r.weights;
    if (r.filled >= m.layers.size())
        throw std::out_of_range("harness: too many layers");
    LayerWeights &l = m.layers[r.filled++];
    const float *src[7] = {query, key, value, output, gate, up, down};
    Matrix *dst[7] = {&l.query, &l.key, &l.value, &l.output, &l.gate, &l.up, &l.down};
    for (int i = 0; i < 7; i++)
        std::memcpy(dst[i]->data(), src[i], dst[i]->size() * sizeof(float));
    l.attention_norm.assign(attention_norm, attention_norm + m.config.dim);
    l.ffn_norm.assign(ffn_norm, ffn_norm + m.config.dim);
    GUARD_END
}

void ref_fmodel_free(void *handle) { delete static_cast<RefFModel *>(handle); }

/* prefill_tokens over the prompt (every row of its output), then
 * decode_token for each of `tokens` (each hidden state), then the cache. */
int ref_fmodel_run(void *handle, const int *prompt, size_t n, const int *tokens, size_t m,
                   size_t threads, float *rows, float *hidden, float *keys, float *values)
{
    GUARD_BEGIN
    const ModelWeights &w = *static_cast<RefFModel *>(handle)->weights;
    const ModelConfig &c = w.config;
    KVCache cache(c);
    const Matrix out = prefill_tokens(w, std::vector<int>(prompt, prompt + n), cache, threads);
    std::memcpy(rows, out.data(), n * c.dim * sizeof(float));
    for (size_t t = 0; t < m; t++) {
        const std::vector<float> h = decode_token(w, tokens[t], cache, threads);
        std::memcpy(hidden + t * c.dim, h.data(), c.dim * sizeof(float));
    }
    const size_t kv = c.effective_kv_heads(), hd = c.head_dim;
    for (size_t l = 0; l < c.layers; l++)
        for (size_t h = 0; h < kv; h++)
            for (size_t p = 0; p < cache.length(); p++) {
                const size_t o = ((l * kv + h) * c.max_seq + p) * hd;
                std::memcpy(keys + o, cache.key(l, h, p), hd * sizeof(float));
                std::memcpy(values + o, cache.value(l, h, p), hd * sizeof(float));
            }
    GUARD_END
}

} // extern "C"
