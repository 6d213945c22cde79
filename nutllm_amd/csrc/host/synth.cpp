// synth.cpp — the synthetic workload generator shared by tests, smoke and
// the benchmark (the reference has none: it loads checkpoints).
//
// Counter-based so that any thread split gives the same array: element pair
// j of stream (seed, stream) takes two 64-bit words
//   a = mix(key + 2j), b = mix(key + 2j + 1), key = mix(mix(seed) ^ stream)
// where mix is the splitmix64 finaliser, then Box-Muller in double:
//   u1 = (a>>11 + 0.5) 2^-53, u2 = (b>>11) 2^-53,
//   r = sqrt(-2 ln u1), out[2j] = fp32(sigma r cos 2pi u2),
//   out[2j+1] = fp32(sigma r sin 2pi u2).
// Token ids use rejection sampling on mix(key + i) for an unbiased
// [0, vocab) draw.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

#include "../status.hpp"

namespace {

inline uint64_t mix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return mix64(mix64(seed) ^ stream);
}

void normal_range(uint64_t key, double sigma, float *out, size_t count,
                  size_t first_pair, size_t last_pair)
{
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t j = first_pair; j < last_pair; j++) {
        const uint64_t a = mix64(key + 2 * uint64_t(j));
        const uint64_t b = mix64(key + 2 * uint64_t(j) + 1);
        const double u1 = (double(a >> 11) + 0.5) * 0x1p-53;
        const double u2 = double(b >> 11) * 0x1p-53;
        const double radius = std::sqrt(-2.0 * std::log(u1));
        const double angle = two_pi * u2;
        out[2 * j] = float(sigma * radius * std::cos(angle));
        if (2 * j + 1 < count)
            out[2 * j + 1] = float(sigma * radius * std::sin(angle));
    }
}

} // namespace

extern "C" {

int nut_synth_normal(uint64_t seed, uint64_t stream, float sigma, float *out,
                     size_t count)
{
    return nut::guarded([&]() {
        nut::require(out != nullptr || count == 0, NUT_EINVAL,
                     "synth: null output");
        const uint64_t key = stream_key(seed, stream);
        const size_t pairs = (count + 1) / 2;
        unsigned threads = std::max(1u, std::min(std::thread::hardware_concurrency(), 16u));
        if (pairs < (1u << 16))
            threads = 1;
        std::vector<std::thread> pool;
        for (unsigned t = 0; t < threads; t++)
            pool.emplace_back(normal_range, key, double(sigma), out, count,
                              pairs * t / threads, pairs * (t + 1) / threads);
        for (std::thread &worker : pool)
            worker.join();
    });
}

int nut_synth_tokens(uint64_t seed, size_t vocab, int *out, size_t count)
{
    return nut::guarded([&]() {
        nut::require(vocab > 0 && vocab <= 0x7fffffffu, NUT_EINVAL,
                     "synth: invalid vocabulary");
        nut::require(out != nullptr || count == 0, NUT_EINVAL,
                     "synth: null output");
        const uint64_t key = stream_key(seed, 0x70726f6d7074ull);
        const uint64_t span = UINT64_MAX - (UINT64_MAX % vocab);
        uint64_t counter = 0;
        for (size_t i = 0; i < count; i++) {
            uint64_t draw;
            do
                draw = mix64(key + counter++);
            while (draw >= span);
            out[i] = int(draw % vocab);
        }
    });
}

} // extern "C"
