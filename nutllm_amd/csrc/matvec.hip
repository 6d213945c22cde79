// matvec.hip — standalone quantised and fp32 matvec kernels for gfx950.
//
// Bandwidth-bound, no MFMA: each wave streams whole rows with 128-bit
// loads (lane l reads bytes [16l, 16l+16) of every 1 KB stretch of a row),
// dequantises in registers and reduces across the wave. x is staged once
// per workgroup in LDS with its per-chunk sums.
#include "kernels.hpp"
#include "runtime.hpp"

namespace nut {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 2; // rows per wave tile

__global__ __launch_bounds__(kThreads) void matvec_q_kernel(QMat m,
                                                            const float *x,
                                                            float *y)
{
    extern __shared__ float lds[];
    const int cw = chunk_weights(m.type);
    float *xs = lds;
    float *xsum = lds + m.cols;
    stage_x(x, xs, xsum, m.cols, cw);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    if (fast_layout(m)) {
        const int tiles = (m.rows + kRows - 1) / kRows;
        for (int t = blockIdx.x * kWaves + wave; t < tiles;
             t += gridDim.x * kWaves) {
            const int row0 = t * kRows;
            float out[kRows];
            qrows_fast<kRows>(m, row0, xs, xsum, out);
#pragma unroll
            for (int r = 0; r < kRows; r++)
                if (lane == r && row0 + r < m.rows)
                    y[row0 + r] = out[r];
        }
    } else {
        for (int row = blockIdx.x * kWaves + wave; row < m.rows;
             row += gridDim.x * kWaves) {
            const float v = qrow_generic(m, row, xs);
            if (lane == 0)
                y[row] = v;
        }
    }
}

// fp32 rows: lane l reads float4 chunks l, l+64, ... of each row.
__global__ __launch_bounds__(kThreads) void matvec_f32_kernel(
    const float *w, int rows, int cols, const float *x, float *y)
{
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < cols; i += blockDim.x)
        xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    for (int row = blockIdx.x * kWaves + wave; row < rows;
         row += gridDim.x * kWaves) {
        const float *wr = w + size_t(row) * cols;
        float acc = 0.0f;
        if ((cols & 3) == 0) {
            for (int c = lane; c < cols / 4; c += kWave) {
                const float4 v = reinterpret_cast<const float4 *>(wr)[c];
                const float *xc = xs + 4 * c;
                acc = fmaf(v.x, xc[0], acc);
                acc = fmaf(v.y, xc[1], acc);
                acc = fmaf(v.z, xc[2], acc);
                acc = fmaf(v.w, xc[3], acc);
            }
        } else {
            for (int c = lane; c < cols; c += kWave)
                acc = fmaf(wr[c], xs[c], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0)
            y[row] = acc;
    }
}

int grid_for(int work_items)
{
    const int blocks = (work_items + kWaves - 1) / kWaves;
    return blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
}

} // namespace

size_t matvec_q_lds_bytes(const QMat &m)
{
    const int cw = chunk_weights(m.type);
    return sizeof(float) * (size_t(m.cols) + (m.cols + cw - 1) / cw);
}

void launch_matvec_q(const QMat &m, const float *x, float *y,
                     hipStream_t stream)
{
    const size_t lds = matvec_q_lds_bytes(m);
    require(lds <= 64 * 1024, NUT_EINVAL,
            "quantized matvec: input dimension exceeds LDS staging");
    const int work = fast_layout(m) ? (m.rows + kRows - 1) / kRows : m.rows;
    hipLaunchKernelGGL(matvec_q_kernel, dim3(grid_for(work)), dim3(kThreads),
                       lds, stream, m, x, y);
    check_launch("quantized matvec");
}

void launch_matvec_f32(const float *w, int rows, int cols, const float *x,
                       float *y, hipStream_t stream)
{
    const size_t lds = sizeof(float) * size_t(cols);
    require(lds <= 64 * 1024, NUT_EINVAL,
            "threaded matvec: input dimension exceeds LDS staging");
    hipLaunchKernelGGL(matvec_f32_kernel, dim3(grid_for(rows)),
                       dim3(kThreads), lds, stream, w, rows, cols, x, y);
    check_launch("threaded matvec");
}

} // namespace nut
