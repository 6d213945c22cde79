// kernel_bench.cpp — standalone kernel timing through the C ABI.
//
//   nutllm_amd/lib/nut_kernel_bench [--iters N]
//
// Launches come from C++ back to back, so the timed loop measures the
// kernels and not the cost of a Python call per launch (which exceeds a
// small matvec).
//  * Quantised matvec (nut_matvec_q; matvec_quantized_threaded,
//    src/quant.cpp:257-321) for the five standalone shapes, INT4 and INT8:
//    x ~ N(0, 1), W ~ N(0, 0.02) from seed 2 (streams 200 + i and 100 + i).
//    Each timed loop rotates through enough uploaded copies of W (at least
//    300 MB) that the 256 MB MALL cannot hold them. Algorithmic bytes =
//    packed weights + fp16 scales + 4 in (x) + 4 out (y); GB/s = bytes /
//    average launch time (HIP events on the launch stream) against the
//    8 TB/s HBM peak.
//  * fp32 GEMM 768 x 768 x 768 (nut_matmul_f32; matmul_threaded,
//    src/threading.cpp:163-181), A, B ~ N(0, 1) from seed 7:
//    905,969,664 FLOP per call against the 157.3 TFLOP/s fp32 matrix peak.
// Prints one JSON object per measurement.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "nutllm_hip.h"

namespace {

constexpr double kHbmPeakGBs = 8000.0;
constexpr double kFp32MatrixPeakTflops = 157.3;
constexpr size_t kRotateBytes = size_t(300) << 20;

void check(int status, const char *what)
{
    if (status != 0) {
        std::fprintf(stderr, "%s failed (%d): %s\n", what, status, nut_last_error());
        std::exit(1);
    }
}

std::vector<float> synth(uint64_t seed, uint64_t stream, float sigma, size_t n)
{
    std::vector<float> v(n);
    check(nut_synth_normal(seed, stream, sigma, v.data(), n), "nut_synth_normal");
    return v;
}

void matvec_case(size_t rows, size_t cols, int type, int index, int iters)
{
    const std::vector<float> w = synth(2, 100 + index, 0.02f, rows * cols);
    const std::vector<float> x = synth(2, 200 + index, 1.0f, cols);
    std::vector<uint8_t> data(nut_quant_data_bytes(rows, cols, type));
    std::vector<uint16_t> scales(nut_quant_scale_count(rows, cols, 32));
    check(nut_quantize(w.data(), rows, cols, type, 32, data.data(), scales.data()),
          "nut_quantize");
    const size_t weight_bytes = data.size() + 2 * scales.size();
    const size_t copies = std::max<size_t>(2, (kRotateBytes + weight_bytes - 1) / weight_bytes);
    const nut_qmatrix host{data.data(), scales.data(), rows, cols, 32, type};
    std::vector<nut_qweight *> mats(copies);
    for (auto &m : mats)
        check(nut_qweight_create(&host, &m), "nut_qweight_create");
    void *dx = nullptr, *dy = nullptr;
    check(nut_malloc(&dx, 4 * cols), "nut_malloc");
    check(nut_malloc(&dy, 4 * rows), "nut_malloc");
    check(nut_memcpy_h2d(dx, x.data(), 4 * cols), "nut_memcpy_h2d");
    for (size_t i = 0; i < 4; i++)
        check(nut_matvec_q(mats[i % copies], static_cast<float *>(dx),
                           static_cast<float *>(dy), nullptr), "nut_matvec_q");
    const size_t launches = std::max<size_t>(iters, copies);
    check(nut_timer_begin(nullptr), "nut_timer_begin");
    for (size_t i = 0; i < launches; i++)
        check(nut_matvec_q(mats[i % copies], static_cast<float *>(dx),
                           static_cast<float *>(dy), nullptr), "nut_matvec_q");
    double ms = 0.0;
    check(nut_timer_end(nullptr, &ms), "nut_timer_end");
    const double per_launch_s = ms * 1e-3 / double(launches);
    const double algorithmic = double(weight_bytes + 4 * cols + 4 * rows);
    const double gbs = algorithmic / per_launch_s / 1e9;
    std::printf("{\"kernel\": \"matvec_q\", \"shape\": [%zu, %zu], \"type\": \"%s\", "
                "\"bytes_per_launch\": %.0f, \"copies_rotated\": %zu, "
                "\"us_per_launch\": %.3f, \"GBps\": %.1f, \"roofline_frac\": %.4f}\n",
                rows, cols, type == 1 ? "int4" : "int8", algorithmic, copies,
                per_launch_s * 1e6, gbs, gbs / kHbmPeakGBs);
    std::fflush(stdout);
    for (auto *m : mats)
        check(nut_qweight_destroy(m), "nut_qweight_destroy");
    check(nut_free(dx), "nut_free");
    check(nut_free(dy), "nut_free");
}

void gemm_case(size_t n, int iters)
{
    const std::vector<float> a = synth(7, 1, 1.0f, n * n), b = synth(7, 2, 1.0f, n * n);
    void *da = nullptr, *db = nullptr, *dc = nullptr;
    check(nut_malloc(&da, 4 * n * n), "nut_malloc");
    check(nut_malloc(&db, 4 * n * n), "nut_malloc");
    check(nut_malloc(&dc, 4 * n * n), "nut_malloc");
    check(nut_memcpy_h2d(da, a.data(), 4 * n * n), "nut_memcpy_h2d");
    check(nut_memcpy_h2d(db, b.data(), 4 * n * n), "nut_memcpy_h2d");
    auto call = [&]() {
        check(nut_matmul_f32(static_cast<float *>(da), static_cast<float *>(db),
                             static_cast<float *>(dc), n, n, n, nullptr), "nut_matmul_f32");
    };
    for (int i = 0; i < 3; i++)
        call();
    check(nut_timer_begin(nullptr), "nut_timer_begin");
    for (int i = 0; i < iters; i++)
        call();
    double ms = 0.0;
    check(nut_timer_end(nullptr, &ms), "nut_timer_end");
    const double flop = 2.0 * double(n) * double(n) * double(n);
    const double per_call = ms * 1e-3 / iters;
    const double tflops = flop / per_call / 1e12;
    std::printf("{\"kernel\": \"matmul_f32\", \"shape\": [%zu, %zu, %zu], "
                "\"flop_per_call\": %.0f, \"us_per_call\": %.2f, \"TFLOPs\": %.2f, "
                "\"roofline_frac\": %.4f}\n",
                n, n, n, flop, per_call * 1e6, tflops, tflops / kFp32MatrixPeakTflops);
    std::fflush(stdout);
    check(nut_free(da), "nut_free");
    check(nut_free(db), "nut_free");
    check(nut_free(dc), "nut_free");
}

} // namespace

int main(int argc, char **argv)
{
    int iters = 200;
    for (int i = 1; i < argc; i++)
        if (std::strcmp(argv[i], "--iters") == 0 && i + 1 < argc)
            iters = std::atoi(argv[++i]);
    int devices = 0;
    check(nut_device_count(&devices), "nut_device_count");
    if (devices < 1) {
        std::fprintf(stderr, "no gfx950 device\n");
        return 1;
    }
    const size_t shapes[5][2] = {{2048, 2048}, {256, 2048}, {5632, 2048}, {2048, 5632},
                                 {4096, 4096}};
    for (int i = 0; i < 5; i++)
        for (int type : {1, 0})
            matvec_case(shapes[i][0], shapes[i][1], type, i, iters);
    gemm_case(768, iters);
    return 0;
}
