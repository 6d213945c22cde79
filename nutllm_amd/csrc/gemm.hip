// gemm.hip — fp32 C = A B on gfx950 matrix cores (matmul_threaded,
// src/threading.cpp:163-181).
//
// v_mfma_f32_16x16x4f32 keeps fp32 inputs and accumulation. Three kernels:
//   ksplit   grids where 64x64 tiles would not give every CU one, M and N
//            multiples of 32, K of 128, 16-byte aligned rows: a 32x32 tile
//            per workgroup of eight waves, each wave the whole tile over
//            an eighth of K, operands straight from L2 into registers, the
//            eight partial tiles added in LDS in a fixed order;
//   tiled    M, N, K multiples of 64 (or 32 x 32 tiles when the ksplit
//            shape rules fail), 16-byte aligned rows: four waves each own a
//            quarter of the tile; K advances 64 at a time through LDS, the
//            next slice in flight in registers (A stored transposed);
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

// The tiled kernel for a TBM x TBN tile of C (64 x 64, or 32 x 32 when the
// 64 x 64 grid would leave CUs idle): waves in a 2 x 2 grid, each a
// (TBM / 2) x (TBN / 2) block of 16 x 16 MFMA tiles. The next D k-slices
// are in flight in registers while one is multiplied from LDS (a slice's
// MFMAs take far less than a load's latency for the small tile).
template <int TBM, int TBN, int D>
__global__ __launch_bounds__(kThreads) void matmul_f32_tiled(
    const float *__restrict__ a, const float *__restrict__ b,
    float *__restrict__ c, int m, int k, int n)
{
    constexpr int TI = TBM / 32, TJ = TBN / 32; // MFMA tiles per wave
    constexpr int AH = TBM * TK / 4 / kThreads; // A float4 per thread
    constexpr int BH = TK * TBN / 4 / kThreads; // B float4 per thread
    static_assert(TI >= 1 && TJ >= 1 && AH >= 1 && BH >= 1, "tile shape");
    __shared__ float at[TK][TBM + 4]; // A slice, transposed: at[k][row]
    __shared__ float bs[TK][TBN + 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.y * TBM, col0 = blockIdx.x * TBN;
    const int wr = (wave >> 1) * (TBM / 2), wc = (wave & 1) * (TBN / 2);
    // loader mapping: A slice TBM x 64 (16 float4 per row), B slice
    // 64 x TBN (TBN / 4 float4 per row)
    const int ar = tid >> 4, ac = (tid & 15) * 4;   // A: rows ar + 16 h
    constexpr int BQ = TBN / 4;                      // float4 per B row
    const int br = tid / BQ, bc = (tid % BQ) * 4;   // B: rows br + (kThreads / BQ) h
    constexpr int BRS = kThreads / BQ;
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    const size_t lda4 = size_t(k) / 4, ldb4 = size_t(n) / 4;
    auto load = [&](int k0, float4 (&ra)[AH], float4 (&rb)[BH]) {
#pragma unroll
        for (int h = 0; h < AH; h++)
            ra[h] = a4[size_t(row0 + ar + 16 * h) * lda4 + (k0 + ac) / 4];
#pragma unroll
        for (int h = 0; h < BH; h++)
            rb[h] = b4[size_t(k0 + br + BRS * h) * ldb4 + (col0 + bc) / 4];
    };
    auto store = [&](const float4 (&ra)[AH], const float4 (&rb)[BH]) {
#pragma unroll
        for (int h = 0; h < AH; h++) {
            const int r = ar + 16 * h;
            at[ac][r] = ra[h].x;
            at[ac + 1][r] = ra[h].y;
            at[ac + 2][r] = ra[h].z;
            at[ac + 3][r] = ra[h].w;
        }
#pragma unroll
        for (int h = 0; h < BH; h++)
            *reinterpret_cast<float4 *>(&bs[br + BRS * h][bc]) = rb[h];
    };
    floatx4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++)
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float4 ra[D][AH], rb[D][BH];
#pragma unroll
    for (int j = 0; j < D; j++)
        if (j * TK < k)
            load(j * TK, ra[j], rb[j]);
    auto slice = [&](int k0, float4 (&sa)[AH], float4 (&sb)[BH]) {
        store(sa, sb);
        __syncthreads();
        if (k0 + D * TK < k)
            load(k0 + D * TK, sa, sb); // in flight during the MFMAs below
        // fragments of four k-steps are read together, then the MFMAs
        // issue back to back
#pragma unroll
        for (int kq = 0; kq < TK; kq += 16) {
            float af[4][TI], bf[4][TJ];
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++) {
                const int ka = kq + 4 * s4 + (lane >> 4);
#pragma unroll
                for (int i = 0; i < TI; i++)
                    af[s4][i] = at[ka][wr + i * 16 + (lane & 15)];
#pragma unroll
                for (int j = 0; j < TJ; j++)
                    bf[s4][j] = bs[ka][wc + j * 16 + (lane & 15)];
            }
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < TJ; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            af[s4][i], bf[s4][j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    };
    for (int k0 = 0; k0 < k; k0 += D * TK) {
#pragma unroll
        for (int j = 0; j < D; j++)
            if (k0 + j * TK < k) // workgroup-uniform
                slice(k0 + j * TK, ra[j], rb[j]);
    }
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = row0 + wr + i * 16 + 4 * (lane >> 4) + v;
                const int col = col0 + wc + j * 16 + (lane & 15);
                c[size_t(r) * n + col] = acc[i][j][v];
            }
}

// The k-split kernel: one 32 x 32 tile of C per workgroup of KW waves, wave
// w taking the k range [w k / KW, (w + 1) k / KW) for the whole tile (2 x 2
// MFMA tiles, four independent accumulators). Operands go from global
// memory (L2) straight to registers through a DEPTH-deep ring of 16-wide k
// chunks; no LDS staging or barrier inside the loop. In MFMA step s of a
// chunk, lane group g (lanes 16 g .. 16 g + 15) supplies k = 4 g + s of
// both operands: the k order inside a chunk is permuted identically for A
// and B, so each lane's A values are four consecutive floats (one float4
// load) and its B values four rows of one column. The KW partial tiles are
// added in LDS in wave order, so the result does not depend on timing.
constexpr int KW = 8, KDEPTH = 3;

__global__ __launch_bounds__(64 * KW) void matmul_f32_ksplit(
    const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ c, int m,
    int k, int n)
{
    __shared__ floatx4 red[KW][4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = blockIdx.y * 32, col0 = blockIdx.x * 32;
    const int li = lane & 15, g = lane >> 4;
    const int kw = k / KW, chunks = kw / 16;
    const int kb = wave * kw;
    const float *pa = a + size_t(row0 + li) * k + kb + 4 * g;
    const float *pb = b + size_t(kb + 4 * g) * n + col0 + li;
    float4 ra[KDEPTH][2];
    float rb[KDEPTH][2][4];
    auto load = [&](int slot, int q) {
#pragma unroll
        for (int i = 0; i < 2; i++)
            ra[slot][i] = *reinterpret_cast<const float4 *>(pa + size_t(16 * i) * k + 16 * q);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const float *p = pb + size_t(16 * q + s) * n;
            rb[slot][0][s] = p[0];
            rb[slot][1][s] = p[16];
        }
    };
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int d = 0; d < KDEPTH; d++)
        if (d < chunks)
            load(d, d);
    for (int q0 = 0; q0 < chunks; q0 += KDEPTH) {
#pragma unroll
        for (int d = 0; d < KDEPTH; d++) {
            if (q0 + d < chunks) { // workgroup-uniform
                float av[2][4], bv[2][4];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    av[i][0] = ra[d][i].x;
                    av[i][1] = ra[d][i].y;
                    av[i][2] = ra[d][i].z;
                    av[i][3] = ra[d][i].w;
                }
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int s = 0; s < 4; s++)
                        bv[j][s] = rb[d][j][s];
                if (q0 + d + KDEPTH < chunks)
                    load(d, q0 + d + KDEPTH); // in flight during the MFMAs below
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 0; j < 2; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                                av[i][s], bv[j][s], acc[i][j], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            red[wave][2 * i + j][lane] = acc[i][j];
    __syncthreads();
    // threads 0-255 add the KW partials of tile t = tid / 64, lane tid % 64
    if (threadIdx.x < 256) {
        const int t = threadIdx.x >> 6;
        floatx4 sum = red[0][t][lane];
#pragma unroll
        for (int w = 1; w < KW; w++)
            sum += red[w][t][lane];
        const int i = t >> 1, j = t & 1;
        // D layout: lane holds rows 4 (lane / 16) + v, column lane % 16
#pragma unroll
        for (int v = 0; v < 4; v++)
            c[size_t(row0 + 16 * i + 4 * g + v) * n + col0 + 16 * j + li] = sum[v];
    }
}

} // namespace

void launch_matmul_f32(const float *a, const float *b, float *c, int m, int k,
                       int n, hipStream_t stream)
{
    const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) |
                           reinterpret_cast<uintptr_t>(b)) & 15) == 0;
    const bool few_tiles = size_t(m / BM) * (n / BN) < 256;
    if (aligned && few_tiles && m % 32 == 0 && n % 32 == 0 && k % (16 * KW) == 0) {
        // grids of 64 x 64 tiles that would leave CUs idle: 32 x 32 tiles
        // with k split over the workgroup's waves (768^3: 17.8-18.7 us
        // against 26-27 us for the tiled kernel below with 32 x 32 tiles)
        hipLaunchKernelGGL(matmul_f32_ksplit, dim3(n / 32, m / 32), dim3(64 * KW), 0, stream,
                           a, b, c, m, k, n);
    } else if (aligned && m % BM == 0 && n % BN == 0 && k % TK == 0) {
        // 32 x 32 tiles when 64 x 64 ones would leave CUs without a tile
        if (size_t(m / BM) * (n / BN) < 256)
            hipLaunchKernelGGL((matmul_f32_tiled<32, 32, 1>), dim3(n / 32, m / 32),
                               dim3(kThreads), 0, stream, a, b, c, m, k, n);
        else
            hipLaunchKernelGGL((matmul_f32_tiled<64, 64, 1>), grid, dim3(kThreads), 0, stream,
                               a, b, c, m, k, n);
    } else {
        hipLaunchKernelGGL(matmul_f32_kernel, grid, dim3(kThreads), 0, stream,
                           a, b, c, m, k, n);
    }
    check_launch("threaded matmul");
}

} // namespace nut
