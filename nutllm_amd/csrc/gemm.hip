// gemm.hip — fp32 C = A B on gfx950 matrix cores (matmul_threaded,
// src/threading.cpp:163-181).
//
// v_mfma_f32_16x16x4f32 keeps fp32 inputs and accumulation. A workgroup of
// four waves owns a 64x64 tile of C; each wave a 32x32 quarter (2x2 MFMA
// tiles).
//   tiled    M, N, K multiples of 64, 16-byte aligned rows: K advances 64
//            at a time; the next slice is loaded (float4) into registers
//            while the MFMAs run on the current one in LDS; A is stored
//            transposed so fragment reads are bank-conflict free.
//   generic  any M, K, N: K advances 16 at a time, edges zero-filled.
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

constexpr int TK = 64;

__global__ __launch_bounds__(kThreads) void matmul_f32_tiled(
    const float *__restrict__ a, const float *__restrict__ b,
    float *__restrict__ c, int m, int k, int n)
{
    __shared__ float at[TK][BM + 4]; // A slice, transposed: at[k][row]
    __shared__ float bs[TK][BN + 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    // loader mapping: A slice 64x64 = 1024 float4, B slice 64x64 = 1024
    // float4; four of each per thread
    const int ar = tid >> 4, ac = (tid & 15) * 4;  // A: rows ar + 16 h
    const int br = tid >> 4, bc = (tid & 15) * 4;  // B: rows br + 16 h
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    const size_t lda4 = size_t(k) / 4, ldb4 = size_t(n) / 4;
    auto load = [&](int k0, float4 (&ra)[4], float4 (&rb)[4]) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
            ra[h] = a4[size_t(row0 + ar + 16 * h) * lda4 + (k0 + ac) / 4];
            rb[h] = b4[size_t(k0 + br + 16 * h) * ldb4 + (col0 + bc) / 4];
        }
    };
    auto store = [&](const float4 (&ra)[4], const float4 (&rb)[4]) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const int r = ar + 16 * h;
            at[ac][r] = ra[h].x;
            at[ac + 1][r] = ra[h].y;
            at[ac + 2][r] = ra[h].z;
            at[ac + 3][r] = ra[h].w;
            *reinterpret_cast<float4 *>(&bs[br + 16 * h][bc]) = rb[h];
        }
    };
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float4 ra[4], rb[4];
    load(0, ra, rb);
    for (int k0 = 0; k0 < k; k0 += TK) {
        store(ra, rb);
        __syncthreads();
        if (k0 + TK < k)
            load(k0 + TK, ra, rb); // in flight during the MFMAs below
        // fragments of four k-steps are read together, then 16 MFMAs
        // issue back to back
#pragma unroll
        for (int kq = 0; kq < TK; kq += 16) {
            float af[4][2], bf[4][2];
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++) {
                const int ka = kq + 4 * s4 + (lane >> 4);
#pragma unroll
                for (int i = 0; i < 2; i++)
                    af[s4][i] = at[ka][wr + i * 16 + (lane & 15)];
#pragma unroll
                for (int j = 0; j < 2; j++)
                    bf[s4][j] = bs[ka][wc + j * 16 + (lane & 15)];
            }
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            af[s4][i], bf[s4][j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = row0 + wr + i * 16 + 4 * (lane >> 4) + v;
                const int col = col0 + wc + j * 16 + (lane & 15);
                c[size_t(r) * n + col] = acc[i][j][v];
            }
}

} // namespace

void launch_matmul_f32(const float *a, const float *b, float *c, int m, int k,
                       int n, hipStream_t stream)
{
    const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) |
                           reinterpret_cast<uintptr_t>(b)) & 15) == 0;
    if (aligned && m % BM == 0 && n % BN == 0 && k % TK == 0)
        hipLaunchKernelGGL(matmul_f32_tiled, grid, dim3(kThreads), 0, stream,
                           a, b, c, m, k, n);
    else
        hipLaunchKernelGGL(matmul_f32_kernel, grid, dim3(kThreads), 0, stream,
                           a, b, c, m, k, n);
    check_launch("threaded matmul");
}

} // namespace nut
