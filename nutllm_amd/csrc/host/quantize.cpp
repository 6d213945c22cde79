// quantize.cpp — the product's block quantiser and fp16 scale format.
//
// Bit-exact with QuantizedMatrix::quantize (src/quant.cpp:154-197): per
// block of block_size weights along the flattened row-major index,
// scale = max|w| / limit (limit 127 for INT8, 7 for INT4; 2^-24 for an
// all-zero block), stored as fp16 by positive_float_to_half
// (src/quant.cpp:23-47), whose rounding differs from IEEE: the 10-bit
// mantissa is rounded half-up (lround on a positive value) and values below
// 2^-14 become round(value * 2^24) clamped to [1, 1023] rather than carrying
// into the smallest normal. q = clamp(lround(w / stored_scale), +-limit).
// INT4 packs the even flattened index in the low nibble.
//
// Blocks are independent, so the work is split over host threads by block
// ranges; the output does not depend on the thread count.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../status.hpp"

namespace nut {

namespace {

// The fp16 encoding of a positive finite scale, from its fp32 fields.
// Returns -1 for non-positive or non-finite input, -2 when it exceeds fp16.
int encode_scale(float value, uint16_t &bits)
{
    if (!(value > 0.0f) || !std::isfinite(value))
        return -1;
    if (value > 65504.0f)
        return -2;
    uint32_t word;
    std::memcpy(&word, &value, sizeof word);
    const uint32_t field = word >> 23;
    const uint32_t fraction = word & 0x7fffffu;
    // value = significand * 2^(power - 23)
    const int power = field == 0 ? -126 : int(field) - 127;
    const uint64_t significand = field == 0 ? fraction : (fraction | 0x800000u);
    if (power <= -15) {
        const int drop = -power - 1; // value * 2^24 = significand >> drop
        uint64_t rounded =
            drop >= 40 ? 0 : (significand + (uint64_t(1) << (drop - 1))) >> drop;
        rounded = std::min<uint64_t>(std::max<uint64_t>(rounded, 1), 1023);
        bits = uint16_t(rounded);
        return 0;
    }
    uint32_t mantissa = (fraction >> 13) + ((fraction >> 12) & 1u);
    int exponent = power;
    if (mantissa == 1024) {
        mantissa = 0;
        exponent += 1;
    }
    if (exponent > 15)
        return -2;
    bits = uint16_t((uint32_t(exponent + 15) << 10) | mantissa);
    return 0;
}

float decode_scale(uint16_t bits)
{
    const uint32_t exponent = (bits >> 10) & 0x1fu;
    const uint32_t mantissa = bits & 0x3ffu;
    if (exponent == 0)
        return std::ldexp(float(mantissa), -24);
    const uint32_t word = ((exponent + 112u) << 23) | (mantissa << 13);
    float value;
    std::memcpy(&value, &word, sizeof value);
    return value;
}

struct BlockJob {
    const float *source;
    size_t count, block_size;
    int limit;
    bool int4;
    uint8_t *data;
    uint16_t *scales;
};

// Quantise blocks [first, last). INT4 blocks of even size start on a byte
// boundary, so disjoint block ranges write disjoint bytes when block_size
// is even; odd block sizes run on one thread (see quantize()).
int quantize_blocks(const BlockJob &job, size_t first, size_t last)
{
    for (size_t block = first; block < last; block++) {
        const size_t begin = block * job.block_size;
        const size_t end = std::min(begin + job.block_size, job.count);
        float peak = 0.0f;
        for (size_t i = begin; i < end; i++) {
            if (!std::isfinite(job.source[i]))
                return -1;
            peak = std::max(peak, std::fabs(job.source[i]));
        }
        const float exact =
            peak == 0.0f ? std::ldexp(1.0f, -24) : peak / float(job.limit);
        uint16_t bits = 0;
        const int status = encode_scale(exact, bits);
        if (status != 0)
            return status;
        job.scales[block] = bits;
        const float stored = decode_scale(bits);
        for (size_t i = begin; i < end; i++) {
            long q = std::lround(job.source[i] / stored);
            q = std::max<long>(-job.limit, std::min<long>(job.limit, q));
            const uint8_t code = uint8_t(q);
            if (!job.int4) {
                job.data[i] = code;
            } else if ((i & 1) == 0) {
                job.data[i >> 1] = uint8_t((job.data[i >> 1] & 0xf0u) | (code & 0x0fu));
            } else {
                job.data[i >> 1] = uint8_t((job.data[i >> 1] & 0x0fu) | uint8_t(code << 4));
            }
        }
    }
    return 0;
}

unsigned host_threads()
{
    const unsigned n = std::thread::hardware_concurrency();
    return std::max(1u, std::min(n == 0 ? 1u : n, 16u));
}

} // namespace

int encode_scale_bits(float value, uint16_t &bits) { return encode_scale(value, bits); }
float decode_scale_bits(uint16_t bits) { return decode_scale(bits); }

void quantize(const float *source, size_t rows, size_t cols, int type,
              size_t block_size, uint8_t *data, uint16_t *scales)
{
    require(source != nullptr && data != nullptr && scales != nullptr,
            NUT_EINVAL, "quantize: null source");
    require(rows != 0 && cols != 0 && rows <= SIZE_MAX / cols, NUT_EINVAL,
            "quantize: invalid dimensions");
    require(block_size != 0, NUT_EINVAL, "quantize: zero block size");
    require(type == NUT_INT8 || type == NUT_INT4, NUT_EINVAL,
            "quantize: unknown quant type");
    const size_t count = rows * cols;
    const size_t blocks = (count + block_size - 1) / block_size;
    const bool int4 = type == NUT_INT4;
    std::memset(data, 0, int4 ? (count + 1) / 2 : count);
    const BlockJob job{source, count, block_size, int4 ? 7 : 127, int4, data,
                       scales};

    unsigned threads = host_threads();
    if ((int4 && (block_size & 1)) || blocks < 4096)
        threads = 1;
    std::vector<int> status(threads, 0);
    if (threads == 1) {
        status[0] = quantize_blocks(job, 0, blocks);
    } else {
        std::vector<std::thread> pool;
        for (unsigned t = 0; t < threads; t++)
            pool.emplace_back([&, t]() {
                status[t] = quantize_blocks(job, blocks * t / threads,
                                            blocks * (t + 1) / threads);
            });
        for (std::thread &worker : pool)
            worker.join();
    }
    // Report the failure the reference would hit first (lowest block).
    for (int s : status) {
        if (s == -1)
            fail(NUT_EINVAL, "quantize: non-finite source weight");
        if (s == -2)
            fail(NUT_ERANGE, "quantize: scale exceeds fp16");
    }
}

} // namespace nut

extern "C" {

int nut_quantize(const float *source, size_t rows, size_t cols, int type,
                 size_t block_size, uint8_t *data, uint16_t *scales)
{
    return nut::guarded([&]() {
        nut::quantize(source, rows, cols, type, block_size, data, scales);
    });
}

size_t nut_quant_data_bytes(size_t rows, size_t cols, int type)
{
    const size_t n = rows * cols;
    return type == NUT_INT8 ? n : (n + 1) / 2;
}

size_t nut_quant_scale_count(size_t rows, size_t cols, size_t block_size)
{
    return block_size == 0 ? 0 : (rows * cols + block_size - 1) / block_size;
}

size_t nut_quant_storage_bytes(size_t rows, size_t cols, int type,
                               size_t block_size)
{
    return nut_quant_data_bytes(rows, cols, type) +
           2 * nut_quant_scale_count(rows, cols, block_size);
}

int nut_float_to_half(float value, uint16_t *bits)
{
    return nut::guarded([&]() {
        nut::require(bits != nullptr, NUT_EINVAL, "float_to_half: null output");
        const int s = nut::encode_scale_bits(value, *bits);
        if (s == -1)
            nut::fail(NUT_EINVAL, "quantize: scale must be finite positive");
        if (s == -2)
            nut::fail(NUT_ERANGE, "quantize: scale exceeds fp16");
    });
}

float nut_half_to_float(uint16_t bits) { return nut::decode_scale_bits(bits); }

} // extern "C"
