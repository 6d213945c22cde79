// host_api_test.cpp — the C++ host API (include/nutllm_gpu.hpp) exercised
// the way nutllm's own selftests exercise the reference API:
//   quantiser KATs          src/quant_selftest.cpp:80-101,155-159
//   llama2.c fixture "Hi!"  src/loader_selftest.cpp (file lines 81-116):
//                           prompt [1, 0, 3] -> [4, 5] in INT8 and INT4
//   decode / prefill / generate errors
//                           src/quant_model.cpp:161-172,212-213,
//                           src/generate.cpp:177-181
//
// usage: host_api_test <dir holding tiny-llama2.bin> [--cpu-only]
// Exit status 0 when every check passes.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "nutllm_gpu.hpp"

using namespace nutgpu;

namespace {

int failures = 0;

void report(bool ok, const char *name)
{
    std::printf("  %s %s\n", ok ? "ok" : "FAIL", name);
    if (!ok)
        failures++;
}

// Runs f; true when it throws E whose message equals `message`.
template <class E>
bool throws(const std::function<void()> &f, const char *message)
{
    try {
        f();
    } catch (const E &e) {
        return std::strcmp(e.what(), message) == 0;
    } catch (...) {
        return false;
    }
    return false;
}

void quantiser_checks()
{
    const float kat[] = {-7.0f, -1.0f, 2.0f, 7.0f};
    const QuantizedMatrix q = QuantizedMatrix::quantize(kat, 1, 4, QuantType::int4);
    report(q.packed_byte(0) == 0xf9 && q.packed_byte(1) == 0x72 &&
               q.value(0, 0) == -7.0f && q.value(0, 3) == 7.0f,
           "int4 packing KAT f9 72");

    std::vector<float> zeros(64, 0.0f);
    const QuantizedMatrix z = QuantizedMatrix::quantize(zeros.data(), 2, 32,
                                                        QuantType::int8);
    report(z.value(1, 31) == 0.0f && z.raw_scales()[0] == 0x0001 &&
               z.error_bound(0, 0) > 0.0f,
           "zero block scale 2^-24");

    bool storage = true;
    for (size_t rows : {1, 3, 5, 64})
        for (size_t cols : {1, 7, 37, 172}) {
            const size_t n = rows * cols, blocks = (n + 31) / 32;
            std::vector<float> w(n, 0.5f);
            storage = storage &&
                      QuantizedMatrix::quantize(w.data(), rows, cols, QuantType::int8)
                              .storage_bytes() == n + 2 * blocks &&
                      QuantizedMatrix::quantize(w.data(), rows, cols, QuantType::int4)
                              .storage_bytes() == (n + 1) / 2 + 2 * blocks;
        }
    report(storage, "storage formula");

    // dequantised values stay within error_bound of the source
    std::vector<float> w(5 * 37);
    for (size_t i = 0; i < w.size(); i++)
        w[i] = std::sin(0.37f * float(i)) * (1.0f + float(i % 5));
    bool bounded = true;
    for (QuantType t : {QuantType::int8, QuantType::int4}) {
        const QuantizedMatrix m = QuantizedMatrix::quantize(w.data(), 5, 37, t);
        for (size_t r = 0; r < 5; r++)
            for (size_t c = 0; c < 37; c++)
                bounded = bounded && std::fabs(m.value(r, c) - w[r * 37 + c]) <=
                                         m.error_bound(r, c);
    }
    report(bounded, "round trip within error_bound");

    std::vector<float> bad(32, 1.0f);
    bad[5] = NAN;
    report(throws<std::invalid_argument>(
               [&] { QuantizedMatrix::quantize(bad.data(), 1, 32, QuantType::int8); },
               "quantize: non-finite source weight") &&
               throws<std::invalid_argument>(
                   [&] { QuantizedMatrix::quantize(w.data(), 0, 4, QuantType::int8); },
                   "quantize: invalid dimensions") &&
               throws<std::invalid_argument>(
                   [&] { QuantizedMatrix::quantize(nullptr, 1, 4, QuantType::int8); },
                   "quantize: null source") &&
               throws<std::out_of_range>([&] { z.packed_byte(0); },
                                         "quantized matrix: packed byte out of range"),
           "quantiser errors");

    ModelConfig bad_config{2, 4, 64, 16, 172, 256, 64, 1, 3};
    report(throws<std::invalid_argument>([&] { bad_config.validate(); },
                                         "model config: invalid dimensions"),
           "config validation");
}

// llama2.c checkpoint (src/llama2.cpp:199-296) quantised into host weights.
QuantizedModelWeights load_llama2c(const std::string &path, QuantType type)
{
    std::ifstream in(path, std::ios::binary);
    if (!in)
        throw std::runtime_error("cannot open " + path);
    int32_t h[7];
    in.read(reinterpret_cast<char *>(h), sizeof h);
    const size_t dim = size_t(h[0]), ffn = size_t(h[1]), layers = size_t(h[2]);
    const size_t heads = size_t(h[3]), kv_heads = size_t(h[4]);
    const bool shared = h[5] > 0;
    const size_t vocab = size_t(shared ? h[5] : -h[5]), max_seq = size_t(h[6]);
    const size_t hd = dim / heads, kvd = kv_heads * hd;
    auto take = [&](size_t n) {
        std::vector<float> v(n);
        in.read(reinterpret_cast<char *>(v.data()), std::streamsize(n * 4));
        return v;
    };
    ModelConfig config{layers, heads, dim, hd, ffn, vocab, max_seq, 1, kv_heads};
    QuantizedModelWeights model(config, type, !shared);
    model.tied_embeddings = shared;
    model.embeddings = take(vocab * dim);
    const auto att_norm = take(layers * dim);
    const auto wq = take(layers * dim * dim), wk = take(layers * kvd * dim),
               wv = take(layers * kvd * dim), wo = take(layers * dim * dim);
    const auto ffn_norm = take(layers * dim);
    const auto w1 = take(layers * ffn * dim), w2 = take(layers * dim * ffn),
               w3 = take(layers * ffn * dim);
    model.final_norm = take(dim);
    take(max_seq * hd);
    if (!shared)
        model.lm_head = take(vocab * dim);
    if (!in)
        throw std::runtime_error("truncated checkpoint " + path);
    auto quant = [&](const std::vector<float> &all, size_t l, size_t rows,
                     size_t cols) {
        return QuantizedMatrix::quantize(all.data() + l * rows * cols, rows,
                                         cols, type);
    };
    for (size_t l = 0; l < layers; l++)
        model.layers.emplace_back(
            quant(wq, l, dim, dim), quant(wk, l, kvd, dim),
            quant(wv, l, kvd, dim), quant(wo, l, dim, dim),
            quant(w1, l, ffn, dim), quant(w3, l, ffn, dim),
            quant(w2, l, dim, ffn),
            std::vector<float>(att_norm.begin() + long(l * dim),
                               att_norm.begin() + long((l + 1) * dim)),
            std::vector<float>(ffn_norm.begin() + long(l * dim),
                               ffn_norm.begin() + long((l + 1) * dim)));
    return model;
}

void device_checks(const std::string &dir)
{
    const std::vector<int> prompt = {1, 0, 3};
    SamplingConfig greedy;
    greedy.max_tokens = 8;
    for (QuantType t : {QuantType::int8, QuantType::int4}) {
        const QuantizedModelWeights weights =
            load_llama2c(dir + "/tiny-llama2.bin", t);
        DeviceModel model(weights);
        GenerationStats stats;
        const std::vector<int> ids =
            generate_tokens_cached(model, prompt, greedy, &stats);
        report(ids == std::vector<int>({4, 5}) && stats.prefill_tokens == 3 &&
                   stats.generated_tokens == 2,
               t == QuantType::int8 ? "llama2.c fixture int8 says Hi!"
                                    : "llama2.c fixture int4 says Hi!");
    }

    const QuantizedModelWeights weights =
        load_llama2c(dir + "/tiny-llama2.bin", QuantType::int8);
    DeviceModel model(weights);
    KVCache cache(weights.config);
    const std::vector<float> h = prefill_quantized(model, prompt, cache, 1);
    KVCache other(weights.config);
    std::vector<float> last;
    for (int token : prompt)
        last = decode_quantized_token(model, token, other, 1);
    bool same = h.size() == last.size();
    for (size_t i = 0; same && i < h.size(); i++)
        same = std::fabs(h[i] - last[i]) <= 1e-6f * (1.0f + std::fabs(last[i]));
    report(same && cache.length() == 3 && other.length() == 3 &&
               cache.key(1, 0, 2) == other.key(1, 0, 2),
           "prefill equals the decode loop");

    report(throws<std::out_of_range>(
               [&] { decode_quantized_token(model, 6, cache, 1); },
               "quantized decode: token out of range") &&
               throws<std::invalid_argument>(
                   [&] { decode_quantized_token(model, 2, cache, 0); },
                   "quantized decode: zero threads") &&
               throws<std::invalid_argument>(
                   [&] { prefill_quantized(model, {}, cache, 1); },
                   "quantized prefill: invalid prompt") &&
               throws<std::invalid_argument>(
                   [&] { generate_tokens_cached(model, {}, greedy); },
                   "generation: invalid prompt length"),
           "decode / prefill / generate errors");

    cache.set_length(cache.capacity());
    report(throws<std::length_error>(
               [&] { decode_quantized_token(model, 2, cache, 1); },
               "quantized decode: context is full") &&
               throws<std::length_error>(
                   [&] { cache.set_length(cache.capacity() + 1); },
                   "kv cache: context exceeds capacity"),
           "full context");

    // blocks straddle rows (37 columns): the generic device path
    std::vector<float> w(5 * 37);
    for (size_t i = 0; i < w.size(); i++)
        w[i] = std::cos(0.21f * float(i)) * (0.5f + float(i % 3));
    bool column = true;
    for (QuantType t : {QuantType::int8, QuantType::int4}) {
        const QuantizedMatrix m = QuantizedMatrix::quantize(w.data(), 5, 37, t);
        for (size_t k : {0, 13, 36}) {
            std::vector<float> x(37, 0.0f), y(5, -1.0f);
            x[k] = 1.0f;
            matvec_quantized_threaded(m, x.data(), y.data(), 2);
            for (size_t r = 0; r < 5; r++)
                column = column && y[r] == m.value(r, k);
        }
    }
    report(column, "matvec unit vectors give columns");
}

} // namespace

int main(int argc, char **argv)
{
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <fixture dir> [--cpu-only]\n", argv[0]);
        return 2;
    }
    const bool cpu_only = argc > 2 && std::strcmp(argv[2], "--cpu-only") == 0;
    std::printf("host API checks\n");
    quantiser_checks();
    if (!cpu_only) {
        int devices = 0;
        if (nut_device_count(&devices) != NUT_OK || devices == 0) {
            std::printf("  FAIL no gfx950 device\n");
            return 1;
        }
        try {
            device_checks(argv[1]);
        } catch (const std::exception &e) {
            std::printf("  FAIL unexpected exception: %s\n", e.what());
            failures++;
        }
    }
    std::printf("%s\n", failures == 0 ? "all passed" : "FAILED");
    return failures == 0 ? 0 : 1;
}
