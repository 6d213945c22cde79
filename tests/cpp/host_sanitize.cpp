// host_sanitize.cpp — the product's host-side code under ThreadSanitizer
// and AddressSanitizer + UndefinedBehaviorSanitizer (no GPU): the threaded
// block quantiser (nut_quantize, which splits blocks over host threads), the
// synthetic generator and the fp16 scale codec, each driven from several
// caller threads at once, with every result compared bit for bit against a
// serial run. Built from the sources by tests/cpp/Makefile (sanitize
// target) and run by tests/test_cpu_host_sanitize.py. Also the sampled
// loop's nucleus cut (host/nucleus.hpp) against the reference's order of
// summation.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "host/nucleus.hpp"
#include "nutllm_hip.h"

// The C ABI's thread-local last-error message, as the library keeps it
// (runtime.cpp and capi.cpp, which also need the HIP runtime).
namespace nut {
namespace {
thread_local std::string g_message;
}
void set_last_error(const char *message) { g_message = message; }
} // namespace nut

extern "C" const char *nut_last_error(void) { return nut::g_message.c_str(); }

namespace {

int failures = 0;

void expect(bool ok, const char *what)
{
    if (!ok) {
        std::printf("FAIL: %s\n", what);
        failures++;
    }
}

struct Shape {
    size_t rows, cols;
    int type;
};

struct Quantized {
    std::vector<uint8_t> data;
    std::vector<uint16_t> scales;
    int status = -1;
};

Quantized quantize(const std::vector<float> &w, const Shape &s)
{
    Quantized q;
    q.data.resize(nut_quant_data_bytes(s.rows, s.cols, s.type));
    q.scales.resize(nut_quant_scale_count(s.rows, s.cols, 32));
    q.status = nut_quantize(w.data(), s.rows, s.cols, s.type, 32, q.data.data(),
                            q.scales.data());
    return q;
}

std::vector<float> normal(uint64_t seed, uint64_t stream, size_t n, float sigma)
{
    std::vector<float> v(n);
    if (nut_synth_normal(seed, stream, sigma, v.data(), n) != NUT_OK)
        v.clear();
    return v;
}

// choose_token's nucleus (src/generate.cpp:63-68) with the total summed in
// 128 strided blocks, as the device sums it, against the total summed in
// token order, as the reference sums it: wherever nucleus_count does not
// flag the cut as ambiguous, the count and the nucleus equal the ones the
// token-order total gives (model.cpp recomputes the total in token order
// for the flagged cuts).
void nucleus_checks()
{
    std::mt19937 rng(17);
    std::uniform_real_distribution<float> u01(0.0f, 1.0f);
    int decided = 0, flagged = 0;
    for (int trial = 0; trial < 600; trial++) {
        const size_t n = 300 + rng() % 3000;
        // spreads from a few e-folds to far below a double ulp of the total
        const float spread = trial % 3 == 0 ? 80.0f : trial % 3 == 1 ? 12.0f : 3.0f;
        std::vector<float> p(n);
        for (float &x : p)
            x = std::exp(-spread * u01(rng));
        double sequential = 0.0;
        for (float x : p)
            sequential += x;
        double blocks = 0.0;
        for (size_t b = 0; b < 128; b++) {
            double t = 0.0;
            for (size_t i = b; i < n; i += 128)
                t += p[i];
            blocks += t;
        }
        std::vector<float> sorted(p);
        std::sort(sorted.begin(), sorted.end(), std::greater<float>());
        const float top_p = trial % 2 == 0 ? 1.0f : 0.05f + 0.95f * u01(rng);
        auto next = [&](size_t i) { return double(sorted[i]); };
        double nucleus_ref = 0.0, nucleus = 0.0;
        bool unused = false, ambiguous = false;
        const size_t ref = nut::nucleus_count(next, n, top_p, sequential, 0.0, nucleus_ref, unused);
        const double slack = blocks * double(n) * 0x1p-52 * 1.01;
        expect(std::fabs(blocks - sequential) <= slack, "nucleus: block total within slack");
        const size_t got = nut::nucleus_count(next, n, top_p, blocks, slack, nucleus, ambiguous);
        if (ambiguous) {
            flagged++;
        } else {
            decided++;
            expect(got == ref && nucleus == nucleus_ref,
                   "nucleus: an unflagged cut equals the token-order total's");
        }
    }
    expect(decided > 300, "nucleus: most cuts decided from the block total");
    expect(flagged > 0, "nucleus: cuts within the slack flagged");
}

} // namespace

int main()
{
    nucleus_checks();

    const Shape shapes[] = {{256, 2048, NUT_INT4}, {256, 2048, NUT_INT8}, {300, 96, NUT_INT4},
                            {7, 4096, NUT_INT8}, {1, 33, NUT_INT4}, {5632, 64, NUT_INT4}};
    constexpr int kCallers = 4;

    // serial results first
    std::vector<std::vector<float>> weights;
    std::vector<Quantized> serial;
    for (size_t i = 0; i < sizeof shapes / sizeof shapes[0]; i++) {
        weights.push_back(normal(2, 100 + i, shapes[i].rows * shapes[i].cols, 0.02f));
        expect(!weights.back().empty(), "synth");
        serial.push_back(quantize(weights.back(), shapes[i]));
        expect(serial.back().status == NUT_OK, "serial quantize");
    }
    std::vector<float> synth_serial = normal(9, 3, 1 << 20, 1.0f);

    // the same calls from several threads at once
    std::vector<std::thread> pool;
    std::vector<int> ok(kCallers, 1);
    for (int t = 0; t < kCallers; t++) {
        pool.emplace_back([&, t]() {
            for (size_t i = 0; i < serial.size(); i++) {
                const size_t k = (i + size_t(t)) % serial.size();
                const Quantized q = quantize(weights[k], shapes[k]);
                ok[t] &= q.status == NUT_OK && q.data == serial[k].data &&
                         q.scales == serial[k].scales;
            }
            ok[t] &= normal(9, 3, 1 << 20, 1.0f) == synth_serial;
            // an error on this thread leaves its own message
            std::vector<float> bad(64, 1.0f);
            bad[t] = NAN;
            Quantized q = quantize(bad, {2, 32, NUT_INT8});
            ok[t] &= q.status == NUT_EINVAL && std::strlen(nut_last_error()) > 0;
            q = quantize(weights[0], shapes[0]);
            ok[t] &= q.status == NUT_OK && std::strlen(nut_last_error()) == 0;
        });
    }
    for (std::thread &th : pool)
        th.join();
    for (int t = 0; t < kCallers; t++)
        expect(ok[t] == 1, "concurrent callers");

    // the fp16 scale codec over a sweep of magnitudes
    for (int e = -30; e <= 15; e++)
        for (int m = 0; m < 64; m++) {
            const float v = std::ldexp(1.0f + float(m) / 64.0f, e);
            uint16_t bits = 0;
            if (nut_float_to_half(v, &bits) == NUT_OK)
                expect(std::isfinite(nut_half_to_float(bits)), "fp16 decode");
        }

    if (failures == 0)
        std::printf("all passed\n");
    return failures == 0 ? 0 : 1;
}
