// matvec.hip — standalone quantised and fp32 matvec kernels for gfx950.
//
// Bandwidth-bound, no MFMA. Fast layout (block 32, cols % 32 == 0): a wave
// owns R consecutive rows; lane l handles 16-byte chunks l, l + 64, ... of
// each row (one INT4 block or half an INT8 block per chunk) and the R row
// sums are reduced with DPP at the end. Two variants:
//   staged  the workgroup stages x once in LDS (rows.hpp) and each lane
//           reads its x chunk from there; the first weight chunk of every
//           row is requested before the staging, so it loads meanwhile;
//   direct  each lane reads its x chunk from global memory (through L1);
//           used when x does not fit 64 KB of LDS.
// Other layouts (blocks straddling rows, other block sizes) run one row
// per wave from an LDS copy of x.
#include "kernels.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace nut {

namespace {

constexpr int kThreads = kRowThreads;
constexpr int kWaves = kRowWaves;

template <int QT, int R>
__global__ __launch_bounds__(kThreads) void matvec_q_fast(QMat m,
                                                          const float *__restrict__ x,
                                                          float *__restrict__ y)
{
    constexpr int CW = QT == 1 ? 32 : 16; // weights per 16-byte chunk
    constexpr float kBias = QT == 1 ? 8.0f : 128.0f;
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = (blockIdx.x * kWaves + threadIdx.x / kWave) * R;
    if (row0 >= m.rows)
        return; // wave-uniform
    const int row_bytes = QT == 1 ? m.cols / 2 : m.cols;
    const int chunks = row_bytes / 16;
    const int blocks_per_row = m.cols / 32;
    const uint8_t *rows[R];
    const uint16_t *scales[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int rr = min(row0 + r, m.rows - 1); // tail rows re-read the last
        rows[r] = m.data + size_t(rr) * row_bytes;
        scales[r] = m.scales + size_t(rr) * blocks_per_row;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++)
        acc[r] = 0.0f;
    for (int c = lane; c < chunks; c += kWave) {
        const int block = QT == 1 ? c : (c >> 1);
        uint4 w[R];
        float s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = load_stream(rows[r] + 16 * c);
            s[r] = half_bits_to_float(scales[r][block]);
        }
        float xc[CW];
        const float4 *x4 = reinterpret_cast<const float4 *>(x + c * CW);
#pragma unroll
        for (int q = 0; q < CW / 4; q++) {
            const float4 v = x4[q];
            xc[4 * q] = v.x;
            xc[4 * q + 1] = v.y;
            xc[4 * q + 2] = v.z;
            xc[4 * q + 3] = v.w;
        }
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < CW; i++)
            xsum += xc[i];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = QT == 1 ? dot_int4_chunk(w[r], xc) : dot_int8_chunk(w[r], xc);
            acc[r] = fmaf(s[r], d - kBias * xsum, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = wave_total(acc[r]);
        if (lane == 0 && row0 + r < m.rows)
            y[row0 + r] = v;
    }
}

template <int QT, int R>
__global__ __launch_bounds__(kThreads) void matvec_q_staged(QMat m, const float *x,
                                                            float *y)
{
    extern __shared__ float xs[];
    const int row0 = (blockIdx.x * kWaves + threadIdx.x / kWave) * R;
    const uint8_t *rp[R];
    const uint16_t *sp[R];
    row_ptrs<QT, R>(m, row0, 0, R, rp, sp);
    float out[R];
    rows_matvec<QT, R, false>(rp, sp, m.cols, x, nullptr, row0 < m.rows, xs, nullptr, out);
    if (row0 < m.rows && (threadIdx.x & (kWave - 1)) == 0)
#pragma unroll
        for (int r = 0; r < R; r++)
            if (row0 + r < m.rows)
                y[row0 + r] = out[r];
}

__global__ __launch_bounds__(kThreads) void matvec_q_generic(QMat m,
                                                             const float *x,
                                                             float *y)
{
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < m.cols; i += blockDim.x)
        xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    for (int row = blockIdx.x * kWaves + wave; row < m.rows;
         row += gridDim.x * kWaves) {
        const float v = qrow_generic(m, row, xs);
        if (lane == 0)
            y[row] = v;
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

// LDS of a kernel that stages x and its per-chunk sums (the step kernels).
size_t matvec_q_lds_bytes(const QMat &m)
{
    const int cw = chunk_weights(m.type);
    return sizeof(float) * (size_t(m.cols) + (m.cols + cw - 1) / cw);
}

template <int QT, int R>
void launch_fast(const QMat &m, const float *x, float *y, hipStream_t stream)
{
    const int waves = (m.rows + R - 1) / R;
    const int blocks = (waves + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((matvec_q_fast<QT, R>), dim3(blocks), dim3(kThreads), 0,
                       stream, m, x, y);
}

template <int QT, int R>
void launch_staged(const QMat &m, const float *x, float *y, hipStream_t stream)
{
    const int waves = (m.rows + R - 1) / R;
    const int blocks = (waves + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((matvec_q_staged<QT, R>), dim3(blocks), dim3(kThreads),
                       staged_x_bytes<QT>(m.cols), stream, m, x, y);
}

void launch_matvec_q(const QMat &m, const float *x, float *y,
                     hipStream_t stream)
{
    // INT4 chunks need 32 floats of x per 16 bytes of weights, which keeps
    // L1 busier than HBM unless x comes from LDS; INT8 chunks need 16, and
    // below 4096 rows the staging latency costs more than it saves
    // (measured per shape with rocprofv3)
    const bool staged = m.type == 1 ? staged_x_bytes<1>(m.cols) <= 65536
                                    : m.rows >= 4096 && staged_x_bytes<0>(m.cols) <= 65536;
    if (fast_layout(m) && staged) {
        // two rows per wave, one where that leaves fewer than 256 workgroups
        if (m.rows >= 2048)
            m.type == 1 ? launch_staged<1, 2>(m, x, y, stream)
                        : launch_staged<0, 2>(m, x, y, stream);
        else
            m.type == 1 ? launch_staged<1, 1>(m, x, y, stream)
                        : launch_staged<0, 1>(m, x, y, stream);
    } else if (fast_layout(m)) {
        // rows per wave: enough waves to fill 256 CUs, as many rows in
        // flight per wave as that allows
        const int r = m.rows >= 4096 ? 4 : m.rows >= 1024 ? 2 : 1;
        if (m.type == 1)
            r == 4 ? launch_fast<1, 4>(m, x, y, stream)
                   : r == 2 ? launch_fast<1, 2>(m, x, y, stream)
                            : launch_fast<1, 1>(m, x, y, stream);
        else
            r == 4 ? launch_fast<0, 4>(m, x, y, stream)
                   : r == 2 ? launch_fast<0, 2>(m, x, y, stream)
                            : launch_fast<0, 1>(m, x, y, stream);
    } else {
        const size_t lds = sizeof(float) * size_t(m.cols);
        require(lds <= 64 * 1024, NUT_EINVAL,
                "quantized matvec: input dimension exceeds LDS staging");
        hipLaunchKernelGGL(matvec_q_generic, dim3(grid_for(m.rows)), dim3(kThreads),
                           lds, stream, m, x, y);
    }
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
