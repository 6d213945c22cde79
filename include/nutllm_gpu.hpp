// nutllm_gpu.hpp — C++17 host API of the gfx950 token loop, over the C ABI
// of libnutllm_hip.so (nutllm_hip.h).
//
// Mirrors the declarations of nutllm's quantised path with the same names,
// argument meaning, exception types and messages:
//   QuantType, QuantizedMatrix           include/quant.hpp:9-57
//   ModelConfig                          include/model.hpp:8-24
//   QuantizedLayerWeights / QuantizedModelWeights
//                                        include/quant_model.hpp:9-46
//   prefill_quantized / decode_quantized_token
//                                        include/quant_model.hpp:48-53
//   KVCache                              include/kvcache.hpp:8-31
//   SamplingConfig, GenerationStats, generate_tokens_cached
//                                        include/generate.hpp:11-36
//   matvec_quantized[_threaded]          include/quant.hpp:53-57
//
// Differences a caller sees, all forced by device residency:
//   * QuantizedModelWeights holds host storage; DeviceModel is its copy in
//     HBM, built once and passed where the reference passes the weights.
//   * KVCache lives in HBM; key()/value() return a host copy of the row.
//   * generate_tokens_cached samples with temperature / top-p through
//     nut_generate_sampled (device numerators and sort, the reference's
//     std::mt19937 draw on the host).
//   * thread_count is validated as the reference does and otherwise unused.
// Header-only: link with -lnutllm_hip.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "nutllm_hip.h"

namespace nutgpu {

// Throws the exception the status names, with the library's message.
inline void check(int status)
{
    if (status == NUT_OK)
        return;
    const std::string message = nut_last_error();
    switch (status) {
    case NUT_EINVAL:
        throw std::invalid_argument(message);
    case NUT_EOUTOFRANGE:
        throw std::out_of_range(message);
    case NUT_ELENGTH:
        throw std::length_error(message);
    case NUT_ERANGE:
        throw std::range_error(message);
    default:
        throw std::runtime_error(message);
    }
}

enum class QuantType { int8, int4 };

inline int c_type(QuantType t) { return t == QuantType::int8 ? NUT_INT8 : NUT_INT4; }

struct ModelConfig {
    size_t layers = 0;
    size_t heads = 0;
    size_t dim = 0;
    size_t head_dim = 0;
    size_t ffn_dim = 0;
    size_t vocab_size = 0;
    size_t max_seq = 0;
    size_t eos_token = 0;
    size_t kv_heads = 0;

    nut_config c_config() const
    {
        return nut_config{layers,     heads,   dim,       head_dim, ffn_dim,
                          vocab_size, max_seq, eos_token, kv_heads};
    }
    void validate() const
    {
        const nut_config c = c_config();
        if (!nut_config_valid(&c))
            throw std::invalid_argument("model config: invalid dimensions");
    }
    size_t effective_kv_heads() const { return kv_heads == 0 ? heads : kv_heads; }
    size_t kv_dim() const { return effective_kv_heads() * head_dim; }
};

// Host storage of a quantised matrix, bit-identical to the reference's:
// flattened blocks, INT8 bytes or INT4 nibbles (even index low), fp16
// scale bits.
class QuantizedMatrix {
public:
    static QuantizedMatrix quantize(const float *source, size_t rows,
                                    size_t cols, QuantType type,
                                    size_t block_size = 32)
    {
        QuantizedMatrix m;
        m.rows_ = rows;
        m.cols_ = cols;
        m.block_size_ = block_size;
        m.type_ = type;
        // Invalid shapes still pass real buffers, so the library reports
        // the reference's error for the shape rather than a null pointer.
        const bool shaped = rows != 0 && cols != 0 && block_size != 0 &&
                            rows <= SIZE_MAX / cols;
        m.data_.resize(shaped ? nut_quant_data_bytes(rows, cols, c_type(type)) : 1);
        m.scales_.resize(shaped ? nut_quant_scale_count(rows, cols, block_size) : 1);
        check(nut_quantize(source, rows, cols, c_type(type), block_size,
                           m.data_.data(), m.scales_.data()));
        return m;
    }

    size_t rows() const { return rows_; }
    size_t cols() const { return cols_; }
    size_t size() const { return rows_ * cols_; }
    size_t block_size() const { return block_size_; }
    size_t blocks() const { return scales_.size(); }
    QuantType type() const { return type_; }
    size_t storage_bytes() const
    {
        return nut_quant_storage_bytes(rows_, cols_, c_type(type_), block_size_);
    }
    uint8_t packed_byte(size_t index) const
    {
        if (type_ != QuantType::int4 || index >= data_.size())
            throw std::out_of_range("quantized matrix: packed byte out of range");
        return data_[index];
    }
    float value(size_t row, size_t column) const
    {
        if (row >= rows_ || column >= cols_)
            throw std::out_of_range("quantized matrix: index out of range");
        const size_t index = row * cols_ + column;
        return float(quantized_value(index)) *
               nut_half_to_float(scales_[index / block_size_]);
    }
    float error_bound(size_t row, size_t column) const
    {
        if (row >= rows_ || column >= cols_)
            throw std::out_of_range("quantized matrix: index out of range");
        const float stored =
            nut_half_to_float(scales_[(row * cols_ + column) / block_size_]);
        const float floor_half = 2.98023223876953125e-08f; // 2^-25
        const float half_rounding =
            stored / 2047.0f > floor_half ? stored / 2047.0f : floor_half;
        const float limit = type_ == QuantType::int8 ? 127.0f : 7.0f;
        const float product = (limit + 0.5f) * half_rounding;
        return stored * 0.5f + product;
    }

    // Raw storage for upload (the reference keeps it private).
    const std::vector<uint8_t> &raw_data() const { return data_; }
    const std::vector<uint16_t> &raw_scales() const { return scales_; }
    nut_qmatrix view() const
    {
        return nut_qmatrix{data_.data(), scales_.data(), rows_, cols_,
                           block_size_, c_type(type_)};
    }

private:
    QuantizedMatrix() = default;
    int quantized_value(size_t index) const
    {
        if (type_ == QuantType::int8)
            return int(int8_t(data_[index]));
        const unsigned byte = data_[index / 2];
        const unsigned nibble = index % 2 == 0 ? byte & 0x0fu : byte >> 4;
        return nibble >= 8 ? int(nibble) - 16 : int(nibble);
    }

    size_t rows_ = 0, cols_ = 0, block_size_ = 32;
    QuantType type_ = QuantType::int8;
    std::vector<uint8_t> data_;
    std::vector<uint16_t> scales_;
};

struct QuantizedLayerWeights {
    QuantizedLayerWeights(QuantizedMatrix query_weight,
                          QuantizedMatrix key_weight,
                          QuantizedMatrix value_weight,
                          QuantizedMatrix output_weight,
                          QuantizedMatrix gate_weight,
                          QuantizedMatrix up_weight,
                          QuantizedMatrix down_weight,
                          std::vector<float> attention_norm_weight,
                          std::vector<float> ffn_norm_weight)
        : query(std::move(query_weight)), key(std::move(key_weight)),
          value(std::move(value_weight)), output(std::move(output_weight)),
          gate(std::move(gate_weight)), up(std::move(up_weight)),
          down(std::move(down_weight)),
          attention_norm(std::move(attention_norm_weight)),
          ffn_norm(std::move(ffn_norm_weight))
    {
    }

    QuantizedMatrix query, key, value, output, gate, up, down;
    std::vector<float> attention_norm, ffn_norm;
};

// Host weights; embeddings and lm_head are [vocab_size x dim] row-major.
struct QuantizedModelWeights {
    ModelConfig config;
    std::vector<float> embeddings;
    std::vector<QuantizedLayerWeights> layers;
    std::vector<float> final_norm;
    std::vector<float> lm_head;
    bool tied_embeddings = false;
    QuantType quant_type;

    QuantizedModelWeights(const ModelConfig &model_config, QuantType type,
                          bool allocate_lm_head)
        : config(model_config), quant_type(type)
    {
        config.validate();
        embeddings.assign(config.vocab_size * config.dim, 0.0f);
        final_norm.assign(config.dim, 1.0f);
        if (allocate_lm_head)
            lm_head.assign(config.vocab_size * config.dim, 0.0f);
    }
    const std::vector<float> &output_weights() const
    {
        return tied_embeddings ? embeddings : lm_head;
    }
};

// QuantizedModelWeights resident in HBM (upload once, decode many).
class DeviceModel {
public:
    explicit DeviceModel(const QuantizedModelWeights &weights)
        : config_(weights.config)
    {
        if (weights.layers.size() != weights.config.layers)
            throw std::invalid_argument("quantized decode: layer count mismatch");
        const nut_config c = config_.c_config();
        check(nut_model_create(&c, c_type(weights.quant_type),
                               weights.tied_embeddings ? 1 : 0, &model_));
        try {
            check(nut_model_set_globals(
                model_, weights.embeddings.data(), weights.final_norm.data(),
                weights.tied_embeddings ? nullptr : weights.lm_head.data()));
            for (size_t l = 0; l < weights.layers.size(); l++) {
                const QuantizedLayerWeights &w = weights.layers[l];
                const nut_qmatrix q = w.query.view(), k = w.key.view(),
                                  v = w.value.view(), o = w.output.view(),
                                  g = w.gate.view(), u = w.up.view(),
                                  d = w.down.view();
                check(nut_model_set_layer(model_, l, &q, &k, &v, &o, &g, &u,
                                          &d, w.attention_norm.data(),
                                          w.ffn_norm.data()));
            }
        } catch (...) {
            nut_model_destroy(model_);
            throw;
        }
    }
    ~DeviceModel()
    {
        if (model_ != nullptr)
            nut_model_destroy(model_);
    }
    DeviceModel(const DeviceModel &) = delete;
    DeviceModel &operator=(const DeviceModel &) = delete;

    const ModelConfig &config() const { return config_; }
    nut_model *handle() const { return model_; }
    size_t storage_bytes() const { return nut_model_storage_bytes(model_); }

private:
    ModelConfig config_;
    nut_model *model_ = nullptr;
};

class KVCache {
public:
    explicit KVCache(const ModelConfig &config) : config_(config)
    {
        const nut_config c = config.c_config();
        check(nut_kv_create(&c, &cache_));
    }
    ~KVCache()
    {
        if (cache_ != nullptr)
            nut_kv_destroy(cache_);
    }
    KVCache(const KVCache &) = delete;
    KVCache &operator=(const KVCache &) = delete;

    size_t length() const { return nut_kv_length(cache_); }
    size_t capacity() const { return nut_kv_capacity(cache_); }
    size_t memory_bytes() const { return nut_kv_memory_bytes(cache_); }
    bool compatible(const ModelConfig &config) const
    {
        const nut_config c = config.c_config();
        return nut_kv_compatible(cache_, &c) != 0;
    }
    void reset() { check(nut_kv_reset(cache_)); }
    void set_length(size_t length) { check(nut_kv_set_length(cache_, length)); }
    std::vector<float> key(size_t layer, size_t head, size_t position) const
    {
        std::vector<float> row(config_.head_dim);
        check(nut_kv_read(cache_, layer, head, position, row.data(), nullptr));
        return row;
    }
    std::vector<float> value(size_t layer, size_t head, size_t position) const
    {
        std::vector<float> row(config_.head_dim);
        check(nut_kv_read(cache_, layer, head, position, nullptr, row.data()));
        return row;
    }
    void store(size_t layer, size_t position, const float *key_data,
               const float *value_data)
    {
        check(nut_kv_store(cache_, layer, position, key_data, value_data));
    }
    nut_kvcache *handle() const { return cache_; }

private:
    ModelConfig config_;
    nut_kvcache *cache_ = nullptr;
};

struct SamplingConfig {
    size_t max_tokens = 32;
    float temperature = 0.0f;
    float top_p = 1.0f;
    uint32_t seed = 1;
    size_t threads = 1;
};

struct GenerationStats {
    size_t prefill_tokens = 0;
    size_t generated_tokens = 0;
    double prefill_seconds = 0.0;
    double decode_seconds = 0.0;
};

inline std::vector<float> decode_quantized_token(DeviceModel &model,
                                                 int token, KVCache &cache,
                                                 size_t thread_count)
{
    model.config().validate();
    if (!cache.compatible(model.config()))
        throw std::invalid_argument(
            "quantized decode: cache configuration mismatch");
    if (thread_count == 0)
        throw std::invalid_argument("quantized decode: zero threads");
    std::vector<float> hidden(model.config().dim);
    check(nut_decode(model.handle(), cache.handle(), token, hidden.data()));
    return hidden;
}

inline std::vector<float> prefill_quantized(DeviceModel &model,
                                            const std::vector<int> &tokens,
                                            KVCache &cache,
                                            size_t thread_count)
{
    if (tokens.empty() || tokens.size() > cache.capacity())
        throw std::invalid_argument("quantized prefill: invalid prompt");
    model.config().validate();
    if (!cache.compatible(model.config()))
        throw std::invalid_argument(
            "quantized decode: cache configuration mismatch");
    if (thread_count == 0)
        throw std::invalid_argument("quantized decode: zero threads");
    std::vector<float> hidden(model.config().dim);
    check(nut_prefill(model.handle(), cache.handle(), tokens.data(),
                      tokens.size(), hidden.data()));
    return hidden;
}

inline std::vector<int> generate_tokens_cached(DeviceModel &model,
                                               const std::vector<int> &prompt,
                                               const SamplingConfig &sampling,
                                               GenerationStats *stats = nullptr)
{
    model.config().validate();
    if (prompt.empty() || prompt.size() > model.config().max_seq)
        throw std::invalid_argument("generation: invalid prompt length");
    if (sampling.threads == 0)
        throw std::invalid_argument("generation: zero threads");
    std::vector<int> out(sampling.max_tokens > 0 ? sampling.max_tokens : 1);
    size_t count = 0;
    nut_generation_stats s{};
    check(nut_generate_sampled(model.handle(), prompt.data(), prompt.size(),
                               sampling.max_tokens, sampling.temperature, sampling.top_p,
                               sampling.seed, out.data(), &count, &s));
    out.resize(count);
    if (stats != nullptr) {
        stats->prefill_tokens = s.prefill_tokens;
        stats->generated_tokens = s.generated_tokens;
        stats->prefill_seconds = s.prefill_seconds;
        stats->decode_seconds = s.decode_seconds;
    }
    return out;
}

// y = W x with host x / y: uploads W for this call. Keep a DeviceMatrix for
// repeated products with resident weights.
class DeviceMatrix {
public:
    explicit DeviceMatrix(const QuantizedMatrix &m) : rows_(m.rows()), cols_(m.cols())
    {
        const nut_qmatrix v = m.view();
        check(nut_qweight_create(&v, &weight_));
    }
    ~DeviceMatrix()
    {
        if (weight_ != nullptr)
            nut_qweight_destroy(weight_);
    }
    DeviceMatrix(const DeviceMatrix &) = delete;
    DeviceMatrix &operator=(const DeviceMatrix &) = delete;

    // y = W x, device pointers, on stream (may be null).
    void matvec(const float *d_x, float *d_y, void *stream = nullptr) const
    {
        check(nut_matvec_q(weight_, d_x, d_y, stream));
    }
    size_t rows() const { return rows_; }
    size_t cols() const { return cols_; }

private:
    size_t rows_, cols_;
    nut_qweight *weight_ = nullptr;
};

// Device memory owned for the duration of a call.
class DeviceBuffer {
public:
    explicit DeviceBuffer(size_t bytes) { check(nut_malloc(&ptr_, bytes)); }
    ~DeviceBuffer()
    {
        if (ptr_ != nullptr)
            nut_free(ptr_);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    void *get() const { return ptr_; }

private:
    void *ptr_ = nullptr;
};

inline void matvec_quantized_threaded(const QuantizedMatrix &matrix,
                                      const float *vector, float *output,
                                      size_t thread_count)
{
    if (vector == nullptr || output == nullptr)
        throw std::invalid_argument("quantized matvec: null pointer");
    if (thread_count == 0)
        throw std::invalid_argument("quantized matvec: zero threads");
    const DeviceMatrix w(matrix);
    const DeviceBuffer x(matrix.cols() * sizeof(float));
    const DeviceBuffer y(matrix.rows() * sizeof(float));
    check(nut_memcpy_h2d(x.get(), vector, matrix.cols() * sizeof(float)));
    w.matvec(static_cast<const float *>(x.get()), static_cast<float *>(y.get()));
    check(nut_memcpy_d2h(output, y.get(), matrix.rows() * sizeof(float)));
}

inline void matvec_quantized(const QuantizedMatrix &matrix,
                             const float *vector, float *output)
{
    matvec_quantized_threaded(matrix, vector, output, 1);
}

} // namespace nutgpu
