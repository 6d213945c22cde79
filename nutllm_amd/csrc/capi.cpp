// capi.cpp — the extern "C" entry points declared in include/nutllm_hip.h.
// Each one validates its arguments, runs under nut::guarded (exceptions
// become status codes plus nut_last_error()), and forwards to the runtime.
#include <cstring>
#include <unordered_map>

#include "fmodel.hpp"
#include "kernels.hpp"
#include "model.hpp"
#include "persistent.hpp"
#include <algorithm>

namespace nut {
int select_device(int device);
const char *last_error();
} // namespace nut

struct nut_qweight {
    nut::DeviceBuffer data, scales;
    nut::QMat view{};
    size_t device_bytes = 0;
};

namespace {

hipStream_t as_stream(void *stream) { return static_cast<hipStream_t>(stream); }

struct TimerPair {
    hipEvent_t start = nullptr, stop = nullptr;
};

thread_local std::unordered_map<void *, TimerPair> g_timers;

} // namespace

extern "C" {

const char *nut_last_error(void) { return nut::last_error(); }

int nut_config_valid(const nut_config *config)
{
    return config != nullptr && nut::config_valid(*config) ? 1 : 0;
}

int nut_device_count(int *count)
{
    return nut::guarded([&]() {
        nut::require(count != nullptr, NUT_EINVAL, "device count: null output");
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess)
            n = 0;
        int gfx950 = 0;
        for (int d = 0; d < n; d++) {
            hipDeviceProp_t props;
            if (hipGetDeviceProperties(&props, d) == hipSuccess &&
                std::strncmp(props.gcnArchName, "gfx950", 6) == 0)
                gfx950++;
        }
        *count = gfx950;
    });
}

int nut_set_device(int device)
{
    return nut::guarded([&]() { nut::select_device(device); });
}

int nut_malloc(void **d_ptr, size_t bytes)
{
    return nut::guarded([&]() {
        nut::require(d_ptr != nullptr, NUT_EINVAL, "malloc: null output");
        nut::ensure_device();
        nut::hip_check(hipMalloc(d_ptr, bytes == 0 ? 1 : bytes), "hipMalloc");
        nut::count_device_allocation();
    });
}

int nut_device_allocations(unsigned long long *count)
{
    return nut::guarded([&]() {
        nut::require(count != nullptr, NUT_EINVAL, "device allocations: null output");
        *count = nut::device_allocations();
    });
}

int nut_free(void *d_ptr)
{
    return nut::guarded([&]() {
        if (d_ptr != nullptr)
            nut::hip_check(hipFree(d_ptr), "hipFree");
    });
}

int nut_memcpy_h2d(void *d_dst, const void *src, size_t bytes)
{
    return nut::guarded([&]() {
        nut::ensure_device();
        nut::hip_check(hipMemcpy(d_dst, src, bytes, hipMemcpyHostToDevice),
                       "hipMemcpy to device");
    });
}

int nut_memcpy_d2h(void *dst, const void *d_src, size_t bytes)
{
    return nut::guarded([&]() {
        nut::ensure_device();
        nut::hip_check(hipMemcpy(dst, d_src, bytes, hipMemcpyDeviceToHost),
                       "hipMemcpy to host");
    });
}

int nut_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes)
{
    return nut::guarded([&]() {
        nut::ensure_device();
        nut::hip_check(hipMemcpy(d_dst, d_src, bytes, hipMemcpyDeviceToDevice),
                       "hipMemcpy device to device");
    });
}

int nut_memset(void *d_dst, int value, size_t bytes)
{
    return nut::guarded([&]() {
        nut::ensure_device();
        nut::hip_check(hipMemset(d_dst, value, bytes), "hipMemset");
    });
}

int nut_synchronize(void)
{
    return nut::guarded([&]() {
        nut::ensure_device();
        nut::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    });
}

int nut_qweight_create(const nut_qmatrix *host, nut_qweight **out)
{
    return nut::guarded([&]() {
        nut::require(host != nullptr && out != nullptr && host->data != nullptr &&
                         host->scales != nullptr,
                     NUT_EINVAL, "quantized matvec: null pointer");
        nut::require(host->rows != 0 && host->cols != 0 && host->block_size != 0 &&
                         host->rows <= 0x7fffffff && host->cols <= 0x7fffffff,
                     NUT_EINVAL, "quantize: invalid dimensions");
        nut::require(host->type == NUT_INT8 || host->type == NUT_INT4, NUT_EINVAL,
                     "quantize: unknown quant type");
        nut::ensure_device();
        std::unique_ptr<nut_qweight> w(new nut_qweight());
        const size_t data = nut_quant_data_bytes(host->rows, host->cols, host->type);
        const size_t scales =
            2 * nut_quant_scale_count(host->rows, host->cols, host->block_size);
        w->data.allocate(data);
        w->scales.allocate(scales);
        nut::hip_check(hipMemcpy(w->data.get(), host->data, data, hipMemcpyHostToDevice),
                       "hipMemcpy to device");
        nut::hip_check(hipMemcpy(w->scales.get(), host->scales, scales,
                                 hipMemcpyHostToDevice),
                       "hipMemcpy to device");
        w->view = nut::QMat{w->data.as<uint8_t>(), w->scales.as<uint16_t>(),
                            int(host->rows), int(host->cols), int(host->block_size),
                            host->type};
        w->device_bytes = data + scales;
        *out = w.release();
    });
}

int nut_qweight_destroy(nut_qweight *w)
{
    return nut::guarded([&]() { delete w; });
}

size_t nut_qweight_device_bytes(const nut_qweight *w)
{
    return w == nullptr ? 0 : w->device_bytes;
}

int nut_matvec_q(const nut_qweight *w, const float *d_x, float *d_y, void *stream)
{
    return nut::guarded([&]() {
        nut::require(w != nullptr && d_x != nullptr && d_y != nullptr, NUT_EINVAL,
                     "quantized matvec: null pointer");
        nut::ensure_device();
        nut::launch_matvec_q(w->view, d_x, d_y, as_stream(stream));
    });
}

int nut_matvec_f32(const float *d_w, size_t rows, size_t cols, const float *d_x,
                   float *d_y, void *stream)
{
    return nut::guarded([&]() {
        nut::require(d_w != nullptr && d_x != nullptr && d_y != nullptr, NUT_EINVAL,
                     "threaded matvec: null pointer");
        nut::require(rows != 0 && cols != 0 && rows <= 0x7fffffff && cols <= 0x7fffffff,
                     NUT_EINVAL, "threaded kernel: zero rows");
        nut::ensure_device();
        nut::launch_matvec_f32(d_w, int(rows), int(cols), d_x, d_y, as_stream(stream));
    });
}

int nut_matmul_f32(const float *d_a, const float *d_b, float *d_c, size_t m, size_t k,
                   size_t n, void *stream)
{
    return nut::guarded([&]() {
        nut::require(d_a != nullptr && d_b != nullptr && d_c != nullptr, NUT_EINVAL,
                     "threaded matmul: null pointer");
        nut::require(m != 0 && k != 0 && n != 0 && m <= 0x7fffffff && k <= 0x7fffffff &&
                         n <= 0x7fffffff,
                     NUT_EINVAL, "threaded matmul: shape mismatch");
        nut::ensure_device();
        nut::launch_matmul_f32(d_a, d_b, d_c, int(m), int(k), int(n), as_stream(stream));
    });
}

int nut_timer_begin(void *stream)
{
    return nut::guarded([&]() {
        nut::ensure_device();
        TimerPair &t = g_timers[stream];
        if (t.start == nullptr) {
            nut::hip_check(hipEventCreate(&t.start), "hipEventCreate");
            nut::hip_check(hipEventCreate(&t.stop), "hipEventCreate");
        }
        nut::hip_check(hipEventRecord(t.start, as_stream(stream)), "hipEventRecord");
    });
}

int nut_timer_end(void *stream, double *milliseconds)
{
    return nut::guarded([&]() {
        nut::require(milliseconds != nullptr, NUT_EINVAL, "timer: null output");
        auto it = g_timers.find(stream);
        nut::require(it != g_timers.end(), NUT_EINVAL, "timer: not started");
        nut::hip_check(hipEventRecord(it->second.stop, as_stream(stream)),
                       "hipEventRecord");
        nut::hip_check(hipEventSynchronize(it->second.stop), "hipEventSynchronize");
        float ms = 0.0f;
        nut::hip_check(hipEventElapsedTime(&ms, it->second.start, it->second.stop),
                       "hipEventElapsedTime");
        *milliseconds = ms;
    });
}

int nut_model_create(const nut_config *config, int type, int tied, nut_model **out)
{
    return nut::guarded([&]() {
        nut::require(config != nullptr && out != nullptr, NUT_EINVAL,
                     "quantized model: null pointer");
        *out = nut::create_model(*config, type, tied != 0);
    });
}

int nut_model_set_globals(nut_model *m, const float *embeddings, const float *final_norm,
                          const float *lm_head)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "quantized model: null model");
        nut::ensure_device();
        nut::set_globals(*m, embeddings, final_norm, lm_head);
    });
}

int nut_model_set_layer(nut_model *m, size_t layer, const nut_qmatrix *query,
                        const nut_qmatrix *key, const nut_qmatrix *value,
                        const nut_qmatrix *output, const nut_qmatrix *gate,
                        const nut_qmatrix *up, const nut_qmatrix *down,
                        const float *attention_norm, const float *ffn_norm)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "quantized model: null model");
        nut::ensure_device();
        const nut_qmatrix *mats[7] = {query, key, value, output, gate, up, down};
        nut::set_layer(*m, layer, mats, attention_norm, ffn_norm);
    });
}

int nut_model_set_path(nut_model *m, int path)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "quantized model: null model");
        nut::require(path >= 0 && path <= 2, NUT_EINVAL, "quantized model: unknown path");
        m->path = path;
    });
}

int nut_model_record_timeline(nut_model *m, int mode)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "quantized model: null model");
        nut::require(mode >= 0 && mode <= 2, NUT_EINVAL, "timeline: unknown mode");
        nut::ensure_device();
        m->timeline.release();
        m->timeline_entries = 0;
        m->timeline_wgs = 0;
        if (mode != 0) {
            const int wgs = mode == 1 ? 1 : nut::kTokenGrid;
            const size_t n = size_t(wgs) * m->config.max_seq *
                             size_t(nut::marks_per_iteration(int(m->config.layers)));
            m->timeline.allocate(n * sizeof(unsigned long long));
            nut::hip_check(hipMemset(m->timeline.get(), 0, n * sizeof(unsigned long long)),
                           "hipMemset");
            m->timeline_entries = n;
            m->timeline_wgs = wgs;
        }
    });
}

int nut_model_timeline(const nut_model *m, uint64_t *ticks, size_t capacity, size_t *count)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && count != nullptr, NUT_EINVAL, "timeline: null pointer");
        const size_t n = std::min(capacity, m->timeline_entries);
        if (n > 0 && ticks != nullptr)
            nut::hip_check(hipMemcpy(ticks, m->timeline.get(), n * sizeof(uint64_t),
                                     hipMemcpyDeviceToHost),
                           "hipMemcpy to host");
        *count = n;
    });
}

int nut_model_last_decode_ms(const nut_model *m, double *milliseconds)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && milliseconds != nullptr, NUT_EINVAL,
                     "generation: null pointer");
        *milliseconds = m->last_decode_device_ms;
    });
}

int nut_token_tag_base(unsigned *launch_count, unsigned *base, int *clear)
{
    return nut::guarded([&]() {
        nut::require(launch_count != nullptr && base != nullptr && clear != nullptr,
                     NUT_EINVAL, "tag schedule: null pointer");
        bool c = false;
        *base = nut::next_tag_base(*launch_count, c);
        *clear = c ? 1 : 0;
    });
}

int nut_model_set_launch_count(nut_model *m, unsigned launch_count)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "quantized model: null model");
        nut::require(launch_count <= nut::kTagBases, NUT_EINVAL,
                     "tag schedule: launch count beyond the tag range");
        m->launch_count = launch_count;
    });
}

int nut_model_inject_fault(nut_model *m, int fault)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "quantized model: null model");
        nut::require(fault == 0 || fault == 1, NUT_EINVAL, "fault: unknown kind");
        m->fault = fault;
    });
}

int nut_model_load_llama2c(const char *path, int type, nut_model **out,
                           double *load_seconds)
{
    return nut::guarded([&]() {
        nut::require(out != nullptr, NUT_EINVAL, "llama2 checkpoint: null output");
        *out = nullptr;
        *out = nut::load_llama2c(path, type, load_seconds);
    });
}

int nut_model_config(const nut_model *m, nut_config *config, int *type, int *tied)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && config != nullptr, NUT_EINVAL,
                     "quantized model: null pointer");
        *config = m->config;
        if (type != nullptr)
            *type = m->type;
        if (tied != nullptr)
            *tied = m->tied ? 1 : 0;
    });
}

size_t nut_model_storage_bytes(const nut_model *m)
{
    return m == nullptr ? 0 : nut::storage_bytes(*m);
}

int nut_model_destroy(nut_model *m)
{
    return nut::guarded([&]() { delete m; });
}

int nut_kv_create(const nut_config *config, nut_kvcache **out)
{
    return nut::guarded([&]() {
        nut::require(config != nullptr && out != nullptr, NUT_EINVAL,
                     "kv cache: null pointer");
        *out = nut::create_kv(*config);
    });
}

int nut_kv_destroy(nut_kvcache *kv)
{
    return nut::guarded([&]() { delete kv; });
}

size_t nut_kv_length(const nut_kvcache *kv) { return kv == nullptr ? 0 : kv->length; }

size_t nut_kv_capacity(const nut_kvcache *kv) { return kv == nullptr ? 0 : kv->config.max_seq; }

size_t nut_kv_memory_bytes(const nut_kvcache *kv)
{
    // KVCache::memory_bytes (src/kvcache.cpp:179-185): keys + values.
    return kv == nullptr ? 0 : 2 * kv->config.layers * kv->layer_elements() * sizeof(float);
}

int nut_kv_compatible(const nut_kvcache *kv, const nut_config *config)
{
    return kv != nullptr && config != nullptr && nut::kv_compatible(*kv, *config) ? 1 : 0;
}

int nut_kv_reset(nut_kvcache *kv)
{
    return nut::guarded([&]() {
        nut::require(kv != nullptr, NUT_EINVAL, "kv cache: null cache");
        kv->length = 0;
    });
}

int nut_kv_set_length(nut_kvcache *kv, size_t length)
{
    return nut::guarded([&]() {
        nut::require(kv != nullptr, NUT_EINVAL, "kv cache: null cache");
        nut::require(length <= kv->config.max_seq, NUT_ELENGTH,
                     "kv cache: context exceeds capacity");
        kv->length = length;
    });
}

int nut_kv_read(const nut_kvcache *kv, size_t layer, size_t head, size_t position,
                float *key, float *value)
{
    return nut::guarded([&]() {
        nut::require(kv != nullptr, NUT_EINVAL, "kv cache: null cache");
        nut::require(layer < kv->config.layers && head < kv->kv_heads() &&
                         position < kv->config.max_seq,
                     NUT_EOUTOFRANGE, "kv cache: index out of range");
        nut::ensure_device();
        const size_t hd = kv->config.head_dim;
        const size_t offset =
            layer * kv->layer_elements() + (head * kv->config.max_seq + position) * hd;
        if (key != nullptr)
            nut::hip_check(hipMemcpy(key, kv->keys.as<float>() + offset, hd * sizeof(float),
                                     hipMemcpyDeviceToHost),
                           "hipMemcpy to host");
        if (value != nullptr)
            nut::hip_check(hipMemcpy(value, kv->values.as<float>() + offset,
                                     hd * sizeof(float), hipMemcpyDeviceToHost),
                           "hipMemcpy to host");
    });
}

int nut_kv_store(nut_kvcache *kv, size_t layer, size_t position, const float *key,
                 const float *value)
{
    return nut::guarded([&]() {
        nut::require(kv != nullptr, NUT_EINVAL, "kv cache: null cache");
        nut::require(key != nullptr && value != nullptr, NUT_EINVAL,
                     "kv cache: null source");
        nut::require(layer < kv->config.layers && position < kv->config.max_seq,
                     NUT_EOUTOFRANGE, "kv cache: index out of range");
        nut::ensure_device();
        const size_t hd = kv->config.head_dim;
        for (size_t head = 0; head < kv->kv_heads(); head++) {
            const size_t offset = layer * kv->layer_elements() +
                                  (head * kv->config.max_seq + position) * hd;
            nut::hip_check(hipMemcpy(kv->keys.as<float>() + offset, key + head * hd,
                                     hd * sizeof(float), hipMemcpyHostToDevice),
                           "hipMemcpy to device");
            nut::hip_check(hipMemcpy(kv->values.as<float>() + offset, value + head * hd,
                                     hd * sizeof(float), hipMemcpyHostToDevice),
                           "hipMemcpy to device");
        }
    });
}

namespace {

// Positions [begin, end) of every (layer, kv head) row as one strided copy:
// host [layer][kv_head][end - begin][head_dim], device rows max_seq apart.
void kv_rows_copy(nut_kvcache *kv, size_t begin, size_t end, float *keys, float *values,
                  const float *src_keys, const float *src_values, bool to_host)
{
    nut::require(kv != nullptr, NUT_EINVAL, "kv cache: null cache");
    nut::require(begin <= end && end <= kv->config.max_seq, NUT_EOUTOFRANGE,
                 "kv cache: index out of range");
    nut::ensure_device();
    if (begin == end)
        return;
    const size_t hd = kv->config.head_dim;
    const size_t width = (end - begin) * hd * sizeof(float);
    const size_t pitch = kv->config.max_seq * hd * sizeof(float);
    const size_t rows = kv->config.layers * kv->kv_heads();
    float *dk = kv->keys.as<float>() + begin * hd;
    float *dv = kv->values.as<float>() + begin * hd;
    if (to_host) {
        if (keys != nullptr)
            nut::hip_check(hipMemcpy2D(keys, width, dk, pitch, width, rows, hipMemcpyDeviceToHost),
                           "hipMemcpy2D to host");
        if (values != nullptr)
            nut::hip_check(hipMemcpy2D(values, width, dv, pitch, width, rows,
                                       hipMemcpyDeviceToHost),
                           "hipMemcpy2D to host");
    } else {
        nut::require(src_keys != nullptr && src_values != nullptr, NUT_EINVAL,
                     "kv cache: null source");
        nut::hip_check(hipMemcpy2D(dk, pitch, src_keys, width, width, rows, hipMemcpyHostToDevice),
                       "hipMemcpy2D to device");
        nut::hip_check(hipMemcpy2D(dv, pitch, src_values, width, width, rows,
                                   hipMemcpyHostToDevice),
                       "hipMemcpy2D to device");
    }
}

} // namespace

int nut_kv_read_positions(const nut_kvcache *kv, size_t begin, size_t end, float *keys,
                          float *values)
{
    return nut::guarded([&]() {
        kv_rows_copy(const_cast<nut_kvcache *>(kv), begin, end, keys, values, nullptr, nullptr,
                     true);
    });
}

int nut_kv_write_positions(nut_kvcache *kv, size_t begin, size_t end, const float *keys,
                           const float *values)
{
    return nut::guarded([&]() {
        kv_rows_copy(kv, begin, end, nullptr, nullptr, keys, values, false);
    });
}

int nut_generate_sampled(nut_model *m, const int *prompt, size_t prompt_len,
                         size_t max_tokens, float temperature, float top_p, uint32_t seed,
                         int *out, size_t *out_count, nut_generation_stats *stats)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "generation: null model");
        nut::ensure_device();
        nut::generate_sampled(*m, prompt, prompt_len, max_tokens, temperature, top_p, seed, out,
                              out_count, stats);
    });
}

int nut_fmodel_create(const nut_config *config, int tied, nut_fmodel **out)
{
    return nut::guarded([&]() {
        nut::require(config != nullptr && out != nullptr, NUT_EINVAL,
                     "fp32 model: null pointer");
        *out = nullptr;
        *out = nut::create_fmodel(*config, tied != 0);
    });
}

int nut_fmodel_set_globals(nut_fmodel *m, const float *embeddings, const float *final_norm,
                           const float *lm_head)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "fp32 model: null model");
        nut::ensure_device();
        nut::set_fglobals(*m, embeddings, final_norm, lm_head);
    });
}

int nut_fmodel_set_layer(nut_fmodel *m, size_t layer, const float *query, const float *key,
                         const float *value, const float *output, const float *gate,
                         const float *up, const float *down, const float *attention_norm,
                         const float *ffn_norm)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "fp32 model: null model");
        nut::ensure_device();
        const float *const w[7] = {query, key, value, output, gate, up, down};
        nut::set_flayer(*m, layer, w, attention_norm, ffn_norm);
    });
}

int nut_fmodel_destroy(nut_fmodel *m)
{
    return nut::guarded([&]() { delete m; });
}

int nut_decode_token(nut_fmodel *m, nut_kvcache *kv, int token, float *hidden)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && kv != nullptr, NUT_EINVAL, "kv cache: null pointer");
        nut::ensure_device();
        nut::decode_token(*m, *kv, token, hidden);
    });
}

int nut_prefill_tokens(nut_fmodel *m, nut_kvcache *kv, const int *tokens, size_t count,
                       float *rows)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && kv != nullptr, NUT_EINVAL, "kv cache: null pointer");
        nut::ensure_device();
        nut::prefill_tokens(*m, *kv, tokens, count, rows);
    });
}

int nut_decode(nut_model *m, nut_kvcache *kv, int token, float *hidden)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && kv != nullptr, NUT_EINVAL,
                     "quantized decode: null pointer");
        nut::ensure_device();
        nut::decode(*m, *kv, token, hidden);
    });
}

int nut_decode_noalloc(nut_model *m, nut_kvcache *kv, int token, float *d_hidden)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && kv != nullptr, NUT_EINVAL,
                     "quantized decode: null pointer");
        nut::ensure_device();
        nut::decode_noalloc(*m, *kv, token, d_hidden);
    });
}

int nut_prefill(nut_model *m, nut_kvcache *kv, const int *tokens, size_t count,
                float *hidden)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr && kv != nullptr, NUT_EINVAL,
                     "quantized prefill: null pointer");
        nut::ensure_device();
        nut::prefill(*m, *kv, tokens, count, hidden);
    });
}

int nut_logits(nut_model *m, const float *hidden, float *logits)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "logits: null model");
        nut::ensure_device();
        nut::logits(*m, hidden, logits);
    });
}

int nut_generate_greedy(nut_model *m, const int *prompt, size_t prompt_len,
                        size_t max_tokens, int *out, size_t *out_count,
                        nut_generation_stats *stats)
{
    return nut::guarded([&]() {
        nut::require(m != nullptr, NUT_EINVAL, "generation: null model");
        nut::ensure_device();
        nut::generate_greedy(*m, prompt, prompt_len, max_tokens, out, out_count, stats);
    });
}

} // extern "C"
