// reference_dropin.cpp — nutllm's quantised token-loop entry points with the
// reference's own signatures, running on the gfx950 device through the C ABI
// of libnutllm_hip.so (include/nutllm_hip.h).
//
// Added to the reference tree, this file replaces the CPU definitions of
//   matvec_quantized_threaded, matvec_quantized       src/quant.cpp:257-321
//   decode_quantized_token, prefill_quantized         src/quant_model.cpp:158-220
//   generate_tokens_cached(const QuantizedModelWeights&, ...)
//                                                     src/generate.cpp:174-216
//   matmul_threaded, matvec_threaded                  src/threading.cpp:163-198
// and compiles against the reference's headers unchanged: build it with
// -I<reference>/include -I<this repository>/include, link with -lnutllm_hip,
// and leave those CPU definitions out of the link.
//
// Device state is kept per host object, behind one lock (the reference
// serialises its calls the same way, src/threading.cpp:50):
//   * a QuantizedModelWeights is uploaded at its first use, keyed by its
//     address and a fingerprint of its storage; a QuantizedMatrix or a
//     classifier Matrix likewise;
//   * a KVCache gets a device twin, made for the cache's configuration and
//     remade when a cache of another configuration turns up at the address.
//     Rows the device writes are copied back into the host cache, so
//     KVCache::key()/value()/length() read what the reference would hold
//     (to the fp32 bar, rel-L2 1e-5); rows the host cache gained some other
//     way (KVCache::store + set_length) are uploaded before the next device
//     step. A fingerprint of the first and last shared rows catches a new
//     cache at a reused address and a reset; rows the host rewrites inside
//     the shared run (KVCache::store below length()) are not detected: call
//     nutgpu_release_cache(cache) after such a rewrite. At most kMaxTwins
//     twins are kept; the least recently used one is dropped beyond that
//     (its cache uploads every row at its next use).
// nutgpu_release_device_state() drops every device copy: call it before
// changing or freeing host weights that were used here.
// nutgpu_release_cache(cache) drops one cache's twin: call it before the
// cache is destroyed, or after rewriting its rows on the host.
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "generate.hpp"
#include "kvcache.hpp"
#include "matmul.hpp"
#include "quant.hpp"
#include "quant_model.hpp"

#include "nutllm_hip.h"

void nutgpu_release_device_state();
void nutgpu_release_cache(const KVCache &cache);
size_t nutgpu_cache_twins();

namespace {

std::mutex g_lock;

// Throws the exception the status names, with the library's message (the
// reference's own text for the reference's own errors).
void check(int status)
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

int c_type(QuantType t) { return t == QuantType::int8 ? NUT_INT8 : NUT_INT4; }

nut_config c_config(const ModelConfig &c)
{
    return nut_config{c.layers,     c.heads,   c.dim,       c.head_dim, c.ffn_dim,
                      c.vocab_size, c.max_seq, c.eos_token, c.kv_heads};
}

// ---------------------------------------------------------------- storage --

// QuantizedMatrix keeps its bytes and fp16 scale bits private and grants
// access only to matvec_quantized_threaded (include/quant.hpp:35-37). That
// function is defined below, so it is also where the upload reads the
// storage: with a probe armed on this thread it records the storage
// instead of multiplying.
struct StorageProbe {
    const uint8_t *data = nullptr;
    const uint16_t *scales = nullptr;
    size_t data_bytes = 0, scale_count = 0;
};
thread_local StorageProbe *g_probe = nullptr;

nut_qmatrix storage_of(const QuantizedMatrix &m, StorageProbe &probe)
{
    g_probe = &probe;
    matvec_quantized_threaded(m, nullptr, nullptr, 1);
    g_probe = nullptr;
    return nut_qmatrix{probe.data, probe.scales, m.rows(), m.cols(), m.block_size(),
                       c_type(m.type())};
}

// A cheap fingerprint of a byte range (its size, ends and a stride sample):
// a different object at a reused address shows up as a different value.
uint64_t fingerprint(const void *p, size_t bytes, uint64_t h = 1469598103934665603ull)
{
    const auto *b = static_cast<const uint8_t *>(p);
    auto mix = [&h](uint64_t v) { h = (h ^ v) * 1099511628211ull; };
    mix(bytes);
    mix(reinterpret_cast<uintptr_t>(p));
    if (bytes == 0 || p == nullptr)
        return h;
    const size_t step = std::max<size_t>(1, bytes / 61);
    for (size_t i = 0; i < bytes; i += step)
        mix(b[i]);
    mix(b[bytes - 1]);
    return h;
}

uint64_t fingerprint(const QuantizedMatrix &m)
{
    StorageProbe probe;
    const nut_qmatrix q = storage_of(m, probe);
    uint64_t h = fingerprint(q.data, probe.data_bytes);
    return fingerprint(q.scales, probe.scale_count * sizeof(uint16_t), h);
}

// --------------------------------------------------------- device buffers --

struct DeviceVec {
    void *ptr = nullptr;
    size_t bytes = 0;
    void ensure(size_t n)
    {
        if (n <= bytes)
            return;
        if (ptr != nullptr)
            check(nut_free(ptr));
        ptr = nullptr;
        bytes = 0;
        check(nut_malloc(&ptr, n));
        bytes = n;
    }
    void release()
    {
        if (ptr != nullptr)
            (void)nut_free(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

DeviceVec g_in, g_out, g_aux;

struct UploadedMatrix {
    nut_qweight *w = nullptr;
    uint64_t print = 0;
};
std::map<const QuantizedMatrix *, UploadedMatrix> g_matrices;

struct UploadedDense {
    DeviceVec data;
    uint64_t print = 0;
};
std::map<const float *, UploadedDense> g_dense;

// ------------------------------------------------------------------ model --

struct UploadedModel {
    nut_model *model = nullptr;
    uint64_t print = 0;
};
std::map<const QuantizedModelWeights *, UploadedModel> g_models;

uint64_t fingerprint(const QuantizedModelWeights &w)
{
    const ModelConfig &c = w.config;
    uint64_t h = fingerprint(&c, sizeof c);
    h = fingerprint(w.embeddings.data(), w.embeddings.size() * sizeof(float), h);
    h = fingerprint(w.final_norm.data(), w.final_norm.size() * sizeof(float), h);
    if (!w.tied_embeddings)
        h = fingerprint(w.lm_head.data(), w.lm_head.size() * sizeof(float), h);
    h ^= uint64_t(w.tied_embeddings) * 0x9e3779b97f4a7c15ull + uint64_t(c_type(w.quant_type));
    for (const QuantizedLayerWeights &l : w.layers) {
        for (const QuantizedMatrix *m :
             {&l.query, &l.key, &l.value, &l.output, &l.gate, &l.up, &l.down})
            h = h * 31 + fingerprint(*m);
        h = fingerprint(l.attention_norm.data(), l.attention_norm.size() * sizeof(float), h);
        h = fingerprint(l.ffn_norm.data(), l.ffn_norm.size() * sizeof(float), h);
    }
    return h;
}

nut_model *device_model(const QuantizedModelWeights &w)
{
    const uint64_t print = fingerprint(w);
    UploadedModel &u = g_models[&w];
    if (u.model != nullptr && u.print == print)
        return u.model;
    if (u.model != nullptr) {
        (void)nut_model_destroy(u.model);
        u.model = nullptr;
    }
    const ModelConfig &c = w.config;
    const nut_config cfg = c_config(c);
    nut_model *m = nullptr;
    check(nut_model_create(&cfg, c_type(w.quant_type), w.tied_embeddings ? 1 : 0, &m));
    try {
        check(nut_model_set_globals(m, w.embeddings.data(), w.final_norm.data(),
                                    w.tied_embeddings ? nullptr : w.lm_head.data()));
        for (size_t i = 0; i < w.layers.size(); i++) {
            const QuantizedLayerWeights &l = w.layers[i];
            StorageProbe pq, pk, pv, po, pg, pu, pd;
            const nut_qmatrix q = storage_of(l.query, pq), k = storage_of(l.key, pk),
                              v = storage_of(l.value, pv), o = storage_of(l.output, po),
                              g = storage_of(l.gate, pg), up = storage_of(l.up, pu),
                              d = storage_of(l.down, pd);
            check(nut_model_set_layer(m, i, &q, &k, &v, &o, &g, &up, &d,
                                      l.attention_norm.data(), l.ffn_norm.data()));
        }
    } catch (...) {
        (void)nut_model_destroy(m);
        g_models.erase(&w);
        throw;
    }
    u.model = m;
    u.print = print;
    return m;
}

// --------------------------------------------------------------- KV cache --

// The device twin of a host KVCache: the configuration it was made for,
// the positions both hold alike, a fingerprint of the host rows at the ends
// of that run (a different cache at a reused address, or a reset, shows up
// as a different value and makes the next use upload every row again), and
// when it was last used.
struct Twin {
    nut_kvcache *kv = nullptr;
    nut_config config{};
    size_t synced = 0;
    uint64_t print = 0;
    uint64_t used = 0;
};
std::map<const KVCache *, Twin> g_caches;
uint64_t g_cache_clock = 0;
constexpr size_t kMaxTwins = 8;

bool same_config(const nut_config &a, const nut_config &b)
{
    return a.layers == b.layers && a.heads == b.heads && a.dim == b.dim &&
           a.head_dim == b.head_dim && a.ffn_dim == b.ffn_dim && a.vocab_size == b.vocab_size &&
           a.max_seq == b.max_seq && a.eos_token == b.eos_token && a.kv_heads == b.kv_heads;
}

// Drops the least recently used twins other than `keep` until at most
// kMaxTwins - 1 remain besides it.
void evict_twins(const KVCache *keep)
{
    while (g_caches.size() >= kMaxTwins) {
        auto oldest = g_caches.end();
        for (auto it = g_caches.begin(); it != g_caches.end(); ++it)
            if (it->first != keep && (oldest == g_caches.end() || it->second.used < oldest->second.used))
                oldest = it;
        if (oldest == g_caches.end())
            return;
        (void)nut_kv_destroy(oldest->second.kv);
        g_caches.erase(oldest);
    }
}

size_t kv_elements(const ModelConfig &c, size_t positions)
{
    return c.layers * c.effective_kv_heads() * positions * c.head_dim;
}

uint64_t fingerprint(const KVCache &cache, const ModelConfig &c, size_t synced)
{
    uint64_t h = fingerprint(cache.key(0, 0, 0), 0);
    if (synced == 0)
        return h;
    const size_t bytes = c.head_dim * sizeof(float);
    for (size_t l : {size_t(0), c.layers - 1})
        for (size_t hd = 0; hd < c.effective_kv_heads(); hd++)
            for (size_t p : {size_t(0), synced - 1}) {
                h = fingerprint(cache.key(l, hd, p), bytes, h);
                h = fingerprint(cache.value(l, hd, p), bytes, h);
            }
    return h;
}

// Bring the twin to the host cache's length: positions the host holds
// beyond what the twin shares are uploaded.
nut_kvcache *device_cache(const KVCache &cache, const ModelConfig &c)
{
    const nut_config cfg = c_config(c);
    if (g_caches.find(&cache) == g_caches.end())
        evict_twins(&cache);
    Twin &t = g_caches[&cache];
    t.used = ++g_cache_clock;
    if (t.kv != nullptr && !same_config(t.config, cfg)) {
        // another cache, of another configuration, at a reused address
        (void)nut_kv_destroy(t.kv);
        t.kv = nullptr;
    }
    if (t.kv == nullptr) {
        check(nut_kv_create(&cfg, &t.kv));
        t.config = cfg;
        t.synced = 0;
    } else if (t.print != fingerprint(cache, c, t.synced)) {
        t.synced = 0;
    }
    const size_t host = cache.length();
    if (host < t.synced)
        t.synced = host;
    if (host > t.synced) {
        const size_t n = host - t.synced, kvh = c.effective_kv_heads(), hd = c.head_dim;
        std::vector<float> keys(kv_elements(c, n)), values(keys.size());
        for (size_t l = 0; l < c.layers; l++)
            for (size_t h = 0; h < kvh; h++)
                for (size_t p = 0; p < n; p++) {
                    const size_t o = ((l * kvh + h) * n + p) * hd;
                    std::memcpy(&keys[o], cache.key(l, h, t.synced + p), hd * sizeof(float));
                    std::memcpy(&values[o], cache.value(l, h, t.synced + p), hd * sizeof(float));
                }
        check(nut_kv_write_positions(t.kv, t.synced, host, keys.data(), values.data()));
    }
    check(nut_kv_set_length(t.kv, host));
    t.synced = host;
    t.print = fingerprint(cache, c, host);
    return t.kv;
}

// Copy the twin's positions [begin, end) into the host cache and set its
// length to end.
void copy_back(KVCache &cache, const ModelConfig &c, size_t begin, size_t end)
{
    Twin &t = g_caches[&cache];
    const size_t n = end - begin, kvh = c.effective_kv_heads(), hd = c.head_dim;
    if (n > 0) {
        std::vector<float> keys(kv_elements(c, n)), values(keys.size());
        check(nut_kv_read_positions(t.kv, begin, end, keys.data(), values.data()));
        std::vector<float> k(kvh * hd), v(kvh * hd);
        for (size_t l = 0; l < c.layers; l++)
            for (size_t p = 0; p < n; p++) {
                for (size_t h = 0; h < kvh; h++) {
                    const size_t o = ((l * kvh + h) * n + p) * hd;
                    std::memcpy(&k[h * hd], &keys[o], hd * sizeof(float));
                    std::memcpy(&v[h * hd], &values[o], hd * sizeof(float));
                }
                cache.store(l, begin + p, k.data(), v.data());
            }
    }
    cache.set_length(end);
    t.synced = end;
    t.print = fingerprint(cache, c, end);
}

// decode_quantized_token's checks, in its order (src/quant_model.cpp:161-172).
void check_decode(const QuantizedModelWeights &model, int token, const KVCache &cache,
                  size_t thread_count)
{
    model.config.validate();
    if (!cache.compatible(model.config))
        throw std::invalid_argument("quantized decode: cache configuration mismatch");
    if (model.layers.size() != model.config.layers)
        throw std::invalid_argument("quantized decode: layer count mismatch");
    if (thread_count == 0)
        throw std::invalid_argument("quantized decode: zero threads");
    if (token < 0 || size_t(token) >= model.config.vocab_size)
        throw std::out_of_range("quantized decode: token out of range");
    if (cache.length() >= cache.capacity())
        throw std::length_error("quantized decode: context is full");
}

} // namespace

void nutgpu_release_cache(const KVCache &cache)
{
    std::lock_guard<std::mutex> lock(g_lock);
    const auto it = g_caches.find(&cache);
    if (it == g_caches.end())
        return;
    (void)nut_kv_destroy(it->second.kv);
    g_caches.erase(it);
}

size_t nutgpu_cache_twins()
{
    std::lock_guard<std::mutex> lock(g_lock);
    return g_caches.size();
}

void nutgpu_release_device_state()
{
    std::lock_guard<std::mutex> lock(g_lock);
    for (auto &e : g_models)
        (void)nut_model_destroy(e.second.model);
    g_models.clear();
    for (auto &e : g_caches)
        (void)nut_kv_destroy(e.second.kv);
    g_caches.clear();
    for (auto &e : g_matrices)
        (void)nut_qweight_destroy(e.second.w);
    g_matrices.clear();
    for (auto &e : g_dense)
        e.second.data.release();
    g_dense.clear();
    g_in.release();
    g_out.release();
    g_aux.release();
}

// ------------------------------------------------------------- entry points --

void matvec_quantized_threaded(const QuantizedMatrix &matrix, const float *vector,
                               float *output, size_t thread_count)
{
    if (g_probe != nullptr) {
        g_probe->data = matrix.data_.data();
        g_probe->scales = matrix.scales_.data();
        g_probe->data_bytes = matrix.data_.size();
        g_probe->scale_count = matrix.scales_.size();
        return;
    }
    if (vector == nullptr || output == nullptr)
        throw std::invalid_argument("quantized matvec: null pointer");
    if (thread_count == 0)
        throw std::invalid_argument("quantized matvec: zero threads");
    std::lock_guard<std::mutex> lock(g_lock);
    const uint64_t print = fingerprint(matrix);
    UploadedMatrix &u = g_matrices[&matrix];
    if (u.w == nullptr || u.print != print) {
        if (u.w != nullptr)
            (void)nut_qweight_destroy(u.w);
        u.w = nullptr;
        StorageProbe probe;
        const nut_qmatrix q = storage_of(matrix, probe);
        check(nut_qweight_create(&q, &u.w));
        u.print = print;
    }
    g_in.ensure(matrix.cols() * sizeof(float));
    g_out.ensure(matrix.rows() * sizeof(float));
    check(nut_memcpy_h2d(g_in.ptr, vector, matrix.cols() * sizeof(float)));
    check(nut_matvec_q(u.w, static_cast<const float *>(g_in.ptr),
                       static_cast<float *>(g_out.ptr), nullptr));
    check(nut_memcpy_d2h(output, g_out.ptr, matrix.rows() * sizeof(float)));
}

void matvec_quantized(const QuantizedMatrix &matrix, const float *vector, float *output)
{
    matvec_quantized_threaded(matrix, vector, output, 1);
}

void matvec_threaded(const Matrix &matrix, const float *vector, float *output,
                     size_t thread_count)
{
    if (vector == nullptr || output == nullptr)
        throw std::invalid_argument("threaded matvec: null pointer");
    if (matrix.rows() == 0)
        throw std::invalid_argument("threaded kernel: zero rows");
    if (thread_count == 0)
        throw std::invalid_argument("threaded kernel: zero threads");
    std::lock_guard<std::mutex> lock(g_lock);
    const size_t bytes = matrix.size() * sizeof(float);
    const uint64_t print = fingerprint(matrix.data(), bytes);
    UploadedDense &u = g_dense[matrix.data()];
    if (u.data.ptr == nullptr || u.print != print) {
        u.data.ensure(bytes);
        check(nut_memcpy_h2d(u.data.ptr, matrix.data(), bytes));
        u.print = print;
    }
    g_in.ensure(matrix.cols() * sizeof(float));
    g_out.ensure(matrix.rows() * sizeof(float));
    check(nut_memcpy_h2d(g_in.ptr, vector, matrix.cols() * sizeof(float)));
    check(nut_matvec_f32(static_cast<const float *>(u.data.ptr), matrix.rows(), matrix.cols(),
                         static_cast<const float *>(g_in.ptr), static_cast<float *>(g_out.ptr),
                         nullptr));
    check(nut_memcpy_d2h(output, g_out.ptr, matrix.rows() * sizeof(float)));
}

void matmul_threaded(const Matrix &a, const Matrix &b, Matrix &c, size_t thread_count)
{
    if (a.cols() != b.rows() || c.rows() != a.rows() || c.cols() != b.cols())
        throw std::invalid_argument("threaded matmul: shape mismatch");
    if (a.rows() == 0)
        throw std::invalid_argument("threaded kernel: zero rows");
    if (thread_count == 0)
        throw std::invalid_argument("threaded kernel: zero threads");
    std::lock_guard<std::mutex> lock(g_lock);
    g_in.ensure(a.size() * sizeof(float));
    g_aux.ensure(b.size() * sizeof(float));
    g_out.ensure(c.size() * sizeof(float));
    check(nut_memcpy_h2d(g_in.ptr, a.data(), a.size() * sizeof(float)));
    check(nut_memcpy_h2d(g_aux.ptr, b.data(), b.size() * sizeof(float)));
    check(nut_matmul_f32(static_cast<const float *>(g_in.ptr),
                         static_cast<const float *>(g_aux.ptr), static_cast<float *>(g_out.ptr),
                         a.rows(), a.cols(), b.cols(), nullptr));
    check(nut_memcpy_d2h(c.data(), g_out.ptr, c.size() * sizeof(float)));
}

std::vector<float> decode_quantized_token(const QuantizedModelWeights &model, int token,
                                          KVCache &cache, size_t thread_count)
{
    check_decode(model, token, cache, thread_count);
    std::lock_guard<std::mutex> lock(g_lock);
    nut_model *m = device_model(model);
    nut_kvcache *kv = device_cache(cache, model.config);
    const size_t position = cache.length();
    std::vector<float> hidden(model.config.dim);
    check(nut_decode(m, kv, token, hidden.data()));
    copy_back(cache, model.config, position, position + 1);
    return hidden;
}

std::vector<float> prefill_quantized(const QuantizedModelWeights &model,
                                     const std::vector<int> &tokens, KVCache &cache,
                                     size_t thread_count)
{
    if (tokens.empty() || tokens.size() > cache.capacity())
        throw std::invalid_argument("quantized prefill: invalid prompt");
    cache.reset();
    // the first decode's checks (the reference decodes token by token)
    check_decode(model, tokens[0], cache, thread_count);
    std::lock_guard<std::mutex> lock(g_lock);
    nut_model *m = device_model(model);
    nut_kvcache *kv = device_cache(cache, model.config);
    std::vector<float> hidden(model.config.dim);
    const int status = nut_prefill(m, kv, tokens.data(), tokens.size(), hidden.data());
    // a bad id fails after the valid prefix is in the cache, as in the
    // reference's token-by-token loop
    copy_back(cache, model.config, 0, nut_kv_length(kv));
    check(status);
    return hidden;
}

std::vector<int> generate_tokens_cached(const QuantizedModelWeights &model,
                                        const std::vector<int> &prompt,
                                        const SamplingConfig &sampling, GenerationStats *stats)
{
    model.config.validate();
    if (prompt.empty() || prompt.size() > model.config.max_seq)
        throw std::invalid_argument("generation: invalid prompt length");
    if (sampling.threads == 0)
        throw std::invalid_argument("generation: zero threads");
    if (model.layers.size() != model.config.layers)
        throw std::invalid_argument("quantized decode: layer count mismatch");
    std::lock_guard<std::mutex> lock(g_lock);
    nut_model *m = device_model(model);
    std::vector<int> out(std::max<size_t>(1, sampling.max_tokens));
    size_t count = 0;
    nut_generation_stats s{};
    check(nut_generate_sampled(m, prompt.data(), prompt.size(), sampling.max_tokens,
                               sampling.temperature, sampling.top_p, sampling.seed, out.data(),
                               &count, &s));
    out.resize(count);
    if (stats != nullptr) {
        stats->prefill_tokens = s.prefill_tokens;
        stats->generated_tokens = s.generated_tokens;
        stats->prefill_seconds = s.prefill_seconds;
        stats->decode_seconds = s.decode_seconds;
    }
    return out;
}
