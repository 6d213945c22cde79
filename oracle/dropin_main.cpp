/* dropin_main.cpp — TEST INFRASTRUCTURE: the reference's own entry points
 * resolved to the device drop-in (nutllm_amd/adapter/reference_dropin.cpp),
 * checked against the reference's CPU definitions of the same functions.
 *
 * oracle/Makefile (target dropin) compiles the reference's sources where
 * they lie with the replaced functions renamed to cpu_* (so both versions
 * live in one program) and links this file, the adapter and
 * libnutllm_hip.so into oracle/_ref/dropin_test. The calls below are the
 * reference's own signatures (include/quant.hpp:53-57,
 * include/quant_model.hpp:48-53, include/generate.hpp:33-36,
 * include/matmul.hpp:32-35) on the reference's own types, including its
 * llama2.c loader (src/llama2.cpp:339-412) on the reference fixture.
 *
 *   dropin_test <tiny-llama2.bin>              every check (needs the GPU)
 *   dropin_test <tiny-llama2.bin> --no-device  host-side checks only, and
 *                                              that a device call fails
 *                                              with std::runtime_error
 */
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <new>
#include <random>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "generate.hpp"
#include "kvcache.hpp"
#include "llama2.hpp"
#include "matmul.hpp"
#include "quant.hpp"
#include "quant_model.hpp"

// The reference's CPU definitions, renamed at compile time.
std::vector<float> cpu_decode_quantized_token(const QuantizedModelWeights &, int, KVCache &,
                                              size_t);
std::vector<float> cpu_prefill_quantized(const QuantizedModelWeights &, const std::vector<int> &,
                                         KVCache &, size_t);
std::vector<int> cpu_generate_tokens_cached(const QuantizedModelWeights &,
                                            const std::vector<int> &, const SamplingConfig &,
                                            GenerationStats *);
void cpu_matvec_quantized_threaded(const QuantizedMatrix &, const float *, float *, size_t);
void cpu_matvec_threaded(const Matrix &, const float *, float *, size_t);
void cpu_matmul_threaded(const Matrix &, const Matrix &, Matrix &, size_t);
void nutgpu_release_device_state();
void nutgpu_release_cache(const KVCache &cache);
size_t nutgpu_cache_twins();

namespace {

int g_failures = 0;

void expect(bool ok, const std::string &what)
{
    std::printf("  %s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    std::fflush(stdout);
    if (!ok)
        g_failures++;
}

double rel_l2(const float *a, const float *b, size_t n)
{
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double d = double(a[i]) - double(b[i]);
        num += d * d;
        den += double(b[i]) * double(b[i]);
    }
    return std::sqrt(num) / std::max(std::sqrt(den), 1e-30);
}

template <class E>
void expect_throw(const std::function<void()> &f, const std::string &message,
                  const std::string &what)
{
    try {
        f();
    } catch (const E &e) {
        expect(message.empty() || std::string(e.what()) == message,
               what + " (" + e.what() + ")");
        return;
    } catch (const std::exception &e) {
        expect(false, what + ": wrong exception: " + e.what());
        return;
    }
    expect(false, what + ": no exception");
}

std::vector<float> uniform(std::mt19937 &rng, size_t n, float scale)
{
    std::uniform_real_distribution<float> d(-scale, scale);
    std::vector<float> v(n);
    for (float &x : v)
        x = d(rng);
    return v;
}

// A two-layer model at a shape the device's fast step kernels run (head_dim
// 64, two query heads per KV head), weights U(-0.05, 0.05) from mt19937.
QuantizedModelWeights synthetic(QuantType type, unsigned seed, size_t max_seq = 96)
{
    ModelConfig c;
    c.layers = 2;
    c.heads = 4;
    c.dim = 256;
    c.head_dim = 64;
    c.ffn_dim = 512;
    c.vocab_size = 512;
    c.max_seq = max_seq;
    c.eos_token = 1;
    c.kv_heads = 2;
    std::mt19937 rng(seed);
    QuantizedModelWeights m(c, type, true);
    const std::vector<float> emb = uniform(rng, c.vocab_size * c.dim, 0.5f);
    std::memcpy(m.embeddings.data(), emb.data(), emb.size() * sizeof(float));
    const std::vector<float> head = uniform(rng, c.vocab_size * c.dim, 0.05f);
    std::memcpy(m.lm_head.data(), head.data(), head.size() * sizeof(float));
    for (float &x : m.final_norm)
        x = 1.0f + 0.25f * std::uniform_real_distribution<float>(-1.0f, 1.0f)(rng);
    const size_t kvd = c.kv_dim();
    auto q = [&](size_t rows, size_t cols) {
        const std::vector<float> w = uniform(rng, rows * cols, 0.05f);
        return QuantizedMatrix::quantize(w.data(), rows, cols, type);
    };
    for (size_t l = 0; l < c.layers; l++) {
        QuantizedMatrix wq = q(c.dim, c.dim), wk = q(kvd, c.dim), wv = q(kvd, c.dim),
                        wo = q(c.dim, c.dim), wg = q(c.ffn_dim, c.dim),
                        wu = q(c.ffn_dim, c.dim), wd = q(c.dim, c.ffn_dim);
        std::vector<float> an = uniform(rng, c.dim, 0.25f), fn = uniform(rng, c.dim, 0.25f);
        for (float &x : an)
            x += 1.0f;
        for (float &x : fn)
            x += 1.0f;
        m.layers.emplace_back(std::move(wq), std::move(wk), std::move(wv), std::move(wo),
                              std::move(wg), std::move(wu), std::move(wd), std::move(an),
                              std::move(fn));
    }
    return m;
}

void host_checks(const QuantizedModelWeights &model)
{
    KVCache cache(model.config);
    expect_throw<std::invalid_argument>(
        [&] { (void)prefill_quantized(model, {}, cache, 1); },
        "quantized prefill: invalid prompt", "prefill_quantized rejects an empty prompt");
    expect_throw<std::out_of_range>(
        [&] { (void)decode_quantized_token(model, int(model.config.vocab_size), cache, 1); },
        "quantized decode: token out of range", "decode_quantized_token rejects a bad token");
    expect_throw<std::invalid_argument>(
        [&] { (void)decode_quantized_token(model, 0, cache, 0); },
        "quantized decode: zero threads", "decode_quantized_token rejects zero threads");
    SamplingConfig zero;
    zero.threads = 0;
    expect_throw<std::invalid_argument>(
        [&] { (void)generate_tokens_cached(model, {1, 2}, zero); }, "generation: zero threads",
        "generate_tokens_cached rejects zero threads");
    std::vector<float> x(model.config.dim), y(model.config.dim);
    expect_throw<std::invalid_argument>(
        [&] { matvec_quantized_threaded(model.layers[0].query, nullptr, y.data(), 1); },
        "quantized matvec: null pointer", "matvec_quantized_threaded rejects null input");
    Matrix a(3, 4), b(5, 6), c(3, 6);
    expect_throw<std::invalid_argument>([&] { matmul_threaded(a, b, c, 1); },
                                        "threaded matmul: shape mismatch",
                                        "matmul_threaded rejects mismatched shapes");
}

// Hidden state of one more decode on `dev` against the same decode on the
// CPU copy `cpu` of its cache.
double decode_both(const QuantizedModelWeights &m, int token, KVCache &dev, KVCache &cpu)
{
    const std::vector<float> hd = decode_quantized_token(m, token, dev, 2);
    const std::vector<float> hc = cpu_decode_quantized_token(m, token, cpu, 2);
    return rel_l2(hd.data(), hc.data(), m.config.dim);
}

// The device twins of host caches: a cache of another configuration at a
// reused address, an interior row rewritten on the host, more caches than
// the adapter keeps twins for.
void cache_twin_checks()
{
    const QuantizedModelWeights a = synthetic(QuantType::int8, 21, 96);
    const QuantizedModelWeights b = synthetic(QuantType::int8, 22, 64);
    const std::vector<int> prompt = {5, 9, 200, 17};
    alignas(KVCache) unsigned char storage[sizeof(KVCache)];
    {
        KVCache *first = new (storage) KVCache(a.config);
        KVCache cpu(a.config);
        prefill_quantized(a, prompt, *first, 2);
        cpu_prefill_quantized(a, prompt, cpu, 2);
        const double e = decode_both(a, 33, *first, cpu);
        first->~KVCache();
        // no release call: the next cache at this address has another
        // configuration (max_seq 64)
        KVCache *second = new (storage) KVCache(b.config);
        KVCache cpu_b(b.config);
        prefill_quantized(b, prompt, *second, 2);
        cpu_prefill_quantized(b, prompt, cpu_b, 2);
        const double eb = decode_both(b, 34, *second, cpu_b);
        expect(e <= 1e-5 && eb <= 1e-5,
               "a cache of another configuration at a reused address gets a twin of its own");
        nutgpu_release_cache(*second);
        second->~KVCache();
    }
    {
        // an interior row rewritten on the host, then the twin released
        KVCache dev(a.config), cpu(a.config);
        prefill_quantized(a, prompt, dev, 2);
        cpu_prefill_quantized(a, prompt, cpu, 2);
        const ModelConfig &c = a.config;
        std::vector<float> k(c.effective_kv_heads() * c.head_dim, 0.25f),
            v(c.effective_kv_heads() * c.head_dim, -0.5f);
        for (KVCache *x : {&dev, &cpu}) {
            const size_t length = x->length();
            x->store(0, 1, k.data(), v.data());
            x->set_length(length);
        }
        nutgpu_release_cache(dev);
        expect(decode_both(a, 40, dev, cpu) <= 1e-5,
               "after nutgpu_release_cache, a host rewrite inside the cache reaches the device");
        nutgpu_release_cache(dev);
    }
    {
        // more caches than twins: the least recently used twin is dropped,
        // and its cache uploads every row at its next use
        std::vector<std::unique_ptr<KVCache>> dev, cpu;
        for (int i = 0; i < 10; i++) {
            dev.emplace_back(new KVCache(a.config));
            cpu.emplace_back(new KVCache(a.config));
            prefill_quantized(a, {int(i + 2), 7}, *dev.back(), 2);
            cpu_prefill_quantized(a, {int(i + 2), 7}, *cpu.back(), 2);
        }
        const size_t twins = nutgpu_cache_twins();
        double worst = 0.0;
        for (int i = 0; i < 10; i++)
            worst = std::max(worst, decode_both(a, 100 + i, *dev[i], *cpu[i]));
        expect(twins <= 8 && nutgpu_cache_twins() <= 8 && worst <= 1e-5,
               "cache twins stay bounded (" + std::to_string(twins) +
                   " after ten caches); evicted caches decode from a fresh upload");
        for (auto &d : dev)
            nutgpu_release_cache(*d);
    }
}

void device_checks(const std::string &fixture)
{
    // the reference's llama2.c fixture through its own loader: "H" -> [4, 5]
    // (src/loader_selftest.cpp, file lines 96-116)
    for (QuantType t : {QuantType::int8, QuantType::int4}) {
        const char *tag = t == QuantType::int8 ? "INT8" : "INT4";
        QuantizedModelWeights m = load_llama2c_quantized_model(fixture, t);
        SamplingConfig greedy;
        greedy.max_tokens = 8;
        GenerationStats stats;
        const std::vector<int> ids = generate_tokens_cached(m, {1, 0, 3}, greedy, &stats);
        const std::vector<int> ref = cpu_generate_tokens_cached(m, {1, 0, 3}, greedy, nullptr);
        expect(ids == std::vector<int>({4, 5}) && ids == ref,
               std::string("llama2.c fixture ") + tag + ": generate_tokens_cached gives [4, 5]");
        expect(stats.prefill_tokens == 3 && stats.generated_tokens == 2,
               std::string("llama2.c fixture ") + tag + ": GenerationStats counts");
    }

    for (QuantType t : {QuantType::int8, QuantType::int4}) {
        const std::string tag = t == QuantType::int8 ? "INT8" : "INT4";
        const QuantizedModelWeights m = synthetic(t, t == QuantType::int8 ? 11u : 12u);
        const ModelConfig &c = m.config;
        std::mt19937 rng(5);
        std::vector<int> prompt(9);
        for (int &p : prompt)
            p = int(rng() % c.vocab_size);

        // prefill + three decodes: hidden states and cache rows, device
        // cache against the CPU cache
        KVCache dev(c), cpu(c);
        std::vector<float> hd = prefill_quantized(m, prompt, dev, 4);
        std::vector<float> hc = cpu_prefill_quantized(m, prompt, cpu, 4);
        double worst = rel_l2(hd.data(), hc.data(), c.dim);
        for (int token : {7, 300, 511}) {
            hd = decode_quantized_token(m, token, dev, 4);
            hc = cpu_decode_quantized_token(m, token, cpu, 4);
            worst = std::max(worst, rel_l2(hd.data(), hc.data(), c.dim));
        }
        double kv = 0.0;
        for (size_t l = 0; l < c.layers; l++)
            for (size_t h = 0; h < c.effective_kv_heads(); h++)
                for (size_t p = 0; p < cpu.length(); p++) {
                    kv = std::max(kv, rel_l2(dev.key(l, h, p), cpu.key(l, h, p), c.head_dim));
                    kv = std::max(kv, rel_l2(dev.value(l, h, p), cpu.value(l, h, p), c.head_dim));
                }
        expect(worst <= 1e-5 && kv <= 1e-5 && dev.length() == cpu.length(),
               tag + ": prefill_quantized + decode_quantized_token hidden rel-L2 " +
                   std::to_string(worst) + ", KVCache rows " + std::to_string(kv));

        // a host cache the device has not seen: the CPU cache, one more step
        hd = decode_quantized_token(m, 42, cpu, 1);
        KVCache fresh(c);
        cpu_prefill_quantized(m, prompt, fresh, 1);
        for (int token : {7, 300, 511})
            cpu_decode_quantized_token(m, token, fresh, 1);
        hc = cpu_decode_quantized_token(m, 42, fresh, 1);
        expect(rel_l2(hd.data(), hc.data(), c.dim) <= 1e-5,
               tag + ": decode_quantized_token continues a cache filled on the CPU");

        SamplingConfig greedy;
        greedy.max_tokens = 12;
        expect(generate_tokens_cached(m, prompt, greedy) ==
                   cpu_generate_tokens_cached(m, prompt, greedy, nullptr),
               tag + ": greedy generate_tokens_cached ids");
        for (const auto &cfg : {std::make_tuple(0.8f, 0.9f, 3u), std::make_tuple(1.5f, 1.0f, 9u)}) {
            SamplingConfig sampled;
            sampled.max_tokens = 12;
            sampled.temperature = std::get<0>(cfg);
            sampled.top_p = std::get<1>(cfg);
            sampled.seed = std::get<2>(cfg);
            expect(generate_tokens_cached(m, prompt, sampled) ==
                       cpu_generate_tokens_cached(m, prompt, sampled, nullptr),
                   tag + ": sampled generate_tokens_cached ids (temperature " +
                       std::to_string(sampled.temperature) + ", top-p " +
                       std::to_string(sampled.top_p) + ")");
        }
        SamplingConfig bad;
        bad.temperature = 1.0f;
        bad.top_p = 0.0f;
        expect_throw<std::invalid_argument>([&] { (void)generate_tokens_cached(m, prompt, bad); },
                                            "sampling: invalid temperature or top-p",
                                            tag + ": top-p 0 rejected");

        // matvec_quantized_threaded / matvec_quantized on the layer matrices
        std::vector<float> x = uniform(rng, c.ffn_dim, 1.0f), y(c.ffn_dim), yr(c.ffn_dim);
        double mv = 0.0;
        for (const QuantizedMatrix *q : {&m.layers[0].gate, &m.layers[1].down}) {
            matvec_quantized_threaded(*q, x.data(), y.data(), 3);
            cpu_matvec_quantized_threaded(*q, x.data(), yr.data(), 3);
            mv = std::max(mv, rel_l2(y.data(), yr.data(), q->rows()));
            matvec_quantized(*q, x.data(), y.data());
            mv = std::max(mv, rel_l2(y.data(), yr.data(), q->rows()));
        }
        expect(mv <= 1e-5, tag + ": matvec_quantized_threaded rel-L2 " + std::to_string(mv));
    }

    cache_twin_checks();

    // the fp32 classifier matvec and the fp32 GEMM
    std::mt19937 rng(8);
    Matrix w(300, 257), a(65, 33), b(33, 130), c(65, 130), cr(65, 130);
    const std::vector<float> wv = uniform(rng, w.size(), 1.0f), av = uniform(rng, a.size(), 1.0f),
                             bv = uniform(rng, b.size(), 1.0f), xv = uniform(rng, 257, 1.0f);
    std::memcpy(w.data(), wv.data(), wv.size() * sizeof(float));
    std::memcpy(a.data(), av.data(), av.size() * sizeof(float));
    std::memcpy(b.data(), bv.data(), bv.size() * sizeof(float));
    std::vector<float> y(300), yr(300);
    matvec_threaded(w, xv.data(), y.data(), 2);
    cpu_matvec_threaded(w, xv.data(), yr.data(), 2);
    expect(rel_l2(y.data(), yr.data(), 300) <= 1e-5, "matvec_threaded (fp32)");
    matmul_threaded(a, b, c, 2);
    cpu_matmul_threaded(a, b, cr, 2);
    expect(rel_l2(c.data(), cr.data(), c.size()) <= 1e-5, "matmul_threaded (fp32)");
    nutgpu_release_device_state();
}

} // namespace

int main(int argc, char **argv)
{
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <tiny-llama2.bin> [--no-device]\n", argv[0]);
        return 2;
    }
    const bool no_device = argc > 2 && std::string(argv[2]) == "--no-device";
    std::printf("reference entry points on the device drop-in\n");
    try {
        const QuantizedModelWeights m = synthetic(QuantType::int8, 3);
        host_checks(m);
        if (no_device) {
            SamplingConfig greedy;
            greedy.max_tokens = 2;
            expect_throw<std::runtime_error>([&] { (void)generate_tokens_cached(m, {1}, greedy); },
                                             "", "without a device, a device call raises "
                                                 "std::runtime_error");
        } else {
            device_checks(argv[1]);
        }
    } catch (const std::exception &e) {
        expect(false, std::string("unexpected exception: ") + e.what());
    }
    std::printf("%s: %d failure(s)\n", g_failures == 0 ? "PASS" : "FAIL", g_failures);
    return g_failures == 0 ? 0 : 1;
}
