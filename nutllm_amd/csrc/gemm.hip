// gemm.hip — fp32 C = A B on gfx950 matrix cores (matmul_threaded,
// src/threading.cpp:163-181).
//
// v_mfma_f32_16x16x4f32 keeps fp32 inputs and accumulation. A workgroup of
// four waves owns a 64x64 tile of C; each wave a 32x32 quarter (2x2 MFMA
// tiles). K advances 16 at a time through LDS. Edges are zero-filled, so any
// M, K, N works.
#include "kernels.hpp"
#include "runtime.hpp"

namespace nut {

namespace {

constexpr int BM = 64, BN = 64, BK = 16;
constexpr int kThreads = 256;

typedef float floatx4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void matmul_f32_kernel(
    const float *a, const float *b, float *c, int m, int k, int n)
{
    __shared__ float as[BM][BK + 1];
    __shared__ float bs[BK][BN + 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int k0 = 0; k0 < k; k0 += BK) {
        // A tile 64x16: thread -> (row tid/4, cols 4*(tid%4) .. +3).
        {
            const int r = tid >> 2, c4 = (tid & 3) * 4;
            const int gr = row0 + r;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int gc = k0 + c4 + q;
                as[r][c4 + q] = (gr < m && gc < k) ? a[size_t(gr) * k + gc] : 0.0f;
            }
        }
        // B tile 16x64: thread -> (row tid/16, cols 4*(tid%16) .. +3).
        {
            const int r = tid >> 4, c4 = (tid & 15) * 4;
            const int gr = k0 + r;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int gc = col0 + c4 + q;
                bs[r][c4 + q] = (gr < k && gc < n) ? b[size_t(gr) * n + gc] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            const int ka = kk + (lane >> 4);
            float af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                af[i] = as[wr + i * 16 + (lane & 15)][ka];
#pragma unroll
            for (int j = 0; j < 2; j++)
                bf[j] = bs[ka][wc + j * 16 + (lane & 15)];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // D layout: lane holds rows 4*(lane/16)+v, column lane%16.
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = row0 + wr + i * 16 + 4 * (lane >> 4) + v;
                const int col = col0 + wc + j * 16 + (lane & 15);
                if (r < m && col < n)
                    c[size_t(r) * n + col] = acc[i][j][v];
            }
}

} // namespace

void launch_matmul_f32(const float *a, const float *b, float *c, int m, int k,
                       int n, hipStream_t stream)
{
    const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    hipLaunchKernelGGL(matmul_f32_kernel, grid, dim3(kThreads), 0, stream, a,
                       b, c, m, k, n);
    check_launch("threaded matmul");
}

} // namespace nut
