// prefill.hip — the prompt as a batch: prefill_quantized
// (src/quant_model.cpp:208-220) computes, token after token, the decode
// step of src/quant_model.cpp:158-206; this file computes the same function
// for all T prompt tokens at once, layer by layer:
//   rmsnorm rows -> Q/K/V GEMMs -> RoPE + KV-cache store -> causal attention
//   -> Wo GEMM (+ residual) -> rmsnorm rows -> gate/up GEMMs -> silu * up
//   -> W2 GEMM (+ residual)
// The quantised GEMMs dequantise each 32-weight block exactly into LDS as
// fp32 (q * fp16 scale is exact in fp32) and run v_mfma_f32_16x16x4f32, so
// every product is exact and only the summation order differs from the
// per-token path.
#include "prefill.hpp"
#include "runtime.hpp"

namespace nut {

namespace {

constexpr int kThreads = 256;
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ rows --

__global__ __launch_bounds__(kThreads) void embed_rows_kernel(
    const float *embeddings, const int *tokens, float *h, int dim)
{
    const float *e = embeddings + size_t(tokens[blockIdx.x]) * dim;
    float *out = h + size_t(blockIdx.x) * dim;
    for (int i = threadIdx.x; i < dim; i += kThreads)
        out[i] = e[i];
}

// out[t] = h[t] * (1 / sqrt(mean(h[t]^2) + 1e-5)) * w  (src/ops.cpp:111-134)
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(
    const float *h, const float *w, float *out, int dim)
{
    __shared__ float red[kThreads / kWave];
    const float *x = h + size_t(blockIdx.x) * dim;
    float sq = 0.0f;
    for (int i = threadIdx.x; i < dim; i += kThreads)
        sq = fmaf(x[i], x[i], sq);
    const float total = block_sum(sq, red, kThreads / kWave);
    const float scale = 1.0f / sqrtf(total / float(dim) + 1e-5f);
    float *o = out + size_t(blockIdx.x) * dim;
    for (int i = threadIdx.x; i < dim; i += kThreads)
        o[i] = x[i] * scale * w[i];
}

// act[t][i] = silu(g[t][i]) * u[t][i]  (src/quant_model.cpp:197-198)
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float *g,
                                                            const float *u,
                                                            float *act, size_t n)
{
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) {
        const float v = g[i];
        act[i] = v / (1.0f + expf(-v)) * u[i];
    }
}

// RoPE on q (all heads) and k (kv heads) of token t at position start + t,
// the rotation of the decode path (src/quant_model.cpp:26-37), then K and V
// rows into the cache [kv_head][max_seq][head_dim] of this layer.
__global__ __launch_bounds__(kThreads) void rope_store_kernel(
    float *q, const float *k, const float *v, const float2 *rope, float *k_cache,
    float *v_cache, int heads, int kv_heads, int hd, int max_seq, int start)
{
    const int t = blockIdx.x;
    const int pos = start + t;
    const int dim = heads * hd, kvd = kv_heads * hd;
    const float2 *cs = rope + size_t(pos) * (hd / 2);
    for (int i = threadIdx.x; i < dim / 2; i += kThreads) {
        float *p = q + size_t(t) * dim + 2 * i;
        const float2 f = cs[i % (hd / 2)];
        const float even = p[0], odd = p[1];
        p[0] = fmaf(even, f.x, -(odd * f.y));
        p[1] = fmaf(even, f.y, odd * f.x);
    }
    for (int i = threadIdx.x; i < kvd / 2; i += kThreads) {
        const float *p = k + size_t(t) * kvd + 2 * i;
        const float2 f = cs[i % (hd / 2)];
        const float even = p[0], odd = p[1];
        const int head = (2 * i) / hd, d = (2 * i) % hd;
        float *kc = k_cache + (size_t(head) * max_seq + pos) * hd + d;
        kc[0] = fmaf(even, f.x, -(odd * f.y));
        kc[1] = fmaf(even, f.y, odd * f.x);
        const float *vp = v + size_t(t) * kvd + 2 * i;
        float *vcp = v_cache + (size_t(head) * max_seq + pos) * hd + d;
        vcp[0] = vp[0];
        vcp[1] = vp[1];
    }
}

// --------------------------------------------------- quantised GEMM --

// C[t][n] (= or +=) sum_k X[t][k] W[n][k]; W quantised (block 32 along k,
// k % 32 == 0). A workgroup owns 64 tokens x 64 outputs; four waves of
// 2 x 2 MFMA tiles. Per 32-wide k slice: X (64 x 32) and the W rows' block
// (64 x 32, dequantised) go to LDS; the next slice's raw bytes are loaded
// into registers during the MFMAs.
constexpr int BM = 64, BN = 64, BK = 32;

template <int QT, bool ADD>
__global__ __launch_bounds__(kThreads) void qgemm_kernel(
    const float *__restrict__ x, int t_count, QMat w, float *__restrict__ c,
    int ldc)
{
    __shared__ float xs[BK][BM + 4]; // X slice, transposed: xs[k][t]
    __shared__ float ws[BK][BN + 4]; // W slice, dequantised: ws[k][n]
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    const int k = w.cols, n_count = w.rows;
    // X loader: rows xr, xr + 32; k columns xc .. xc + 3
    const int xr = tid >> 3, xc = (tid & 7) * 4;
    // W loader: row wn (64 rows, 4 threads each), weights 8 * wp .. + 7
    const int wn = tid >> 2, wp = tid & 3;
    const int wrow = min(n0 + wn, n_count - 1);
    constexpr int RB_DIV = QT == 1 ? 2 : 1;
    const uint8_t *wdata = w.data + size_t(wrow) * (k / RB_DIV);
    const uint16_t *wsc = w.scales + size_t(wrow) * (k / 32);
    float4 rx[2];
    uint2 rw; // 8 weights: INT4 uses rw.x only
    uint16_t rs;
    auto load = [&](int k0) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = t0 + xr + 32 * h;
            rx[h] = t < t_count
                        ? *reinterpret_cast<const float4 *>(x + size_t(t) * k + k0 + xc)
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (QT == 1) {
            rw.x = *reinterpret_cast<const uint32_t *>(wdata + k0 / 2 + 4 * wp);
            rw.y = 0;
        } else {
            rw = *reinterpret_cast<const uint2 *>(wdata + k0 + 8 * wp);
        }
        rs = wsc[k0 / 32];
    };
    auto store = [&]() {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int r = xr + 32 * h;
            xs[xc][r] = rx[h].x;
            xs[xc + 1][r] = rx[h].y;
            xs[xc + 2][r] = rx[h].z;
            xs[xc + 3][r] = rx[h].w;
        }
        const float s = half_bits_to_float(rs);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            int q;
            if (QT == 1) {
                const uint32_t nib = (rw.x >> (4 * e)) & 0xfu;
                q = int(nib) - (nib >= 8 ? 16 : 0);
            } else {
                const uint32_t word = e < 4 ? rw.x : rw.y;
                q = int(int8_t((word >> (8 * (e & 3))) & 0xffu));
            }
            ws[8 * wp + e][wn] = float(q) * s;
        }
    };
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    load(0);
    for (int k0 = 0; k0 < k; k0 += BK) {
        store();
        __syncthreads();
        if (k0 + BK < k)
            load(k0 + BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            const int ka = kk + (lane >> 4);
            float af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                af[i] = xs[ka][wr + i * 16 + (lane & 15)];
#pragma unroll
            for (int j = 0; j < 2; j++)
                bf[j] = ws[ka][wc + j * 16 + (lane & 15)];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // D layout: lane holds rows 4 * (lane / 16) + v, column lane % 16.
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = t0 + wr + i * 16 + 4 * (lane >> 4) + v;
                const int n = n0 + wc + j * 16 + (lane & 15);
                if (t < t_count && n < n_count) {
                    float *p = c + size_t(t) * ldc + n;
                    *p = ADD ? *p + acc[i][j][v] : acc[i][j][v];
                }
            }
}

// ------------------------------------------------ causal attention --

// One workgroup per (64-query tile, head): queries t0 .. t0 + 63 at
// positions start + t attend to cache positions 0 .. start + t. Key tiles
// of 64 positions stream through LDS; scores, the online softmax and the
// context accumulate in fp32. Thread (i = tid / 4, part = tid % 4) owns
// query row i: scores of keys 16 part .. 16 part + 15 of each tile and
// context columns part * HD / 4 .. (part + 1) * HD / 4 - 1.
constexpr int AQ = 64, AK = 64;

template <int HD>
__global__ __launch_bounds__(kThreads) void attention_prefill_kernel(
    const float *q, const float *k_cache, const float *v_cache, float *ctx,
    int t_count, int heads, int kv_heads, int max_seq, int start, float scale)
{
    __shared__ float qs[AQ][HD + 4];
    __shared__ float kt[HD][AK + 4]; // K tile transposed: kt[d][j]
    __shared__ float vs[AK][HD + 4];
    __shared__ float ps[AQ][AK + 4];
    const int tid = threadIdx.x;
    const int head = blockIdx.y, g = head / (heads / kv_heads);
    const int t0 = blockIdx.x * AQ;
    const int dim = heads * HD;
    const int i = tid >> 2, part = tid & 3;
    for (int e = tid; e < AQ * HD; e += kThreads) {
        const int r = e / HD, d = e % HD;
        qs[r][d] = t0 + r < t_count ? q[size_t(t0 + r) * dim + head * HD + d] : 0.0f;
    }
    const float *kg = k_cache + size_t(g) * max_seq * HD;
    const float *vg = v_cache + size_t(g) * max_seq * HD;
    const int my_pos = start + t0 + i; // position of query row i
    const int last = min(start + t0 + AQ - 1, start + t_count - 1);
    constexpr int OC = HD / 4; // context columns per thread
    float m = -INFINITY, l = 0.0f;
    float o[OC];
#pragma unroll
    for (int d = 0; d < OC; d++)
        o[d] = 0.0f;
    for (int p0 = 0; p0 <= last; p0 += AK) {
        __syncthreads(); // previous tile's readers are done
        for (int e = tid; e < AK * HD; e += kThreads) {
            const int j = e / HD, d = e % HD;
            const bool in = p0 + j <= last;
            kt[d][j] = in ? kg[size_t(p0 + j) * HD + d] : 0.0f;
            vs[j][d] = in ? vg[size_t(p0 + j) * HD + d] : 0.0f;
        }
        __syncthreads();
        float s[16];
#pragma unroll
        for (int jj = 0; jj < 16; jj++)
            s[jj] = 0.0f;
        for (int d = 0; d < HD; d++) {
            const float qd = qs[i][d];
#pragma unroll
            for (int jj = 0; jj < 16; jj += 4) {
                const float4 kk = *reinterpret_cast<const float4 *>(&kt[d][16 * part + jj]);
                s[jj] = fmaf(qd, kk.x, s[jj]);
                s[jj + 1] = fmaf(qd, kk.y, s[jj + 1]);
                s[jj + 2] = fmaf(qd, kk.z, s[jj + 2]);
                s[jj + 3] = fmaf(qd, kk.w, s[jj + 3]);
            }
        }
        float tile_max = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < 16; jj++) {
            const int pos = p0 + 16 * part + jj;
            s[jj] = pos <= my_pos ? s[jj] * scale : -INFINITY;
            tile_max = fmaxf(tile_max, s[jj]);
        }
        // the four threads of row i share max and sum (quad DPP)
        tile_max = fmaxf(tile_max, dpp<kDppQuadSwap1>(tile_max, -INFINITY));
        tile_max = fmaxf(tile_max, dpp<kDppQuadSwap2>(tile_max, -INFINITY));
        const float m_new = fmaxf(m, tile_max);
        // rows past t_count (and fully masked tiles) keep m = -inf
        const float correction = m_new == -INFINITY ? 1.0f : expf(m - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int jj = 0; jj < 16; jj++) {
            const float e = s[jj] == -INFINITY ? 0.0f : expf(s[jj] - m_new);
            ps[i][16 * part + jj] = e;
            sum += e;
        }
        sum += dpp<kDppQuadSwap1>(sum, 0.0f);
        sum += dpp<kDppQuadSwap2>(sum, 0.0f);
        l = l * correction + sum;
        m = m_new;
#pragma unroll
        for (int d = 0; d < OC; d++)
            o[d] *= correction;
        __syncthreads(); // ps complete
        for (int j = 0; j < AK; j++) {
            const float pj = ps[i][j];
#pragma unroll
            for (int d = 0; d < OC; d += 4) {
                const float4 vv = *reinterpret_cast<const float4 *>(&vs[j][OC * part + d]);
                o[d] = fmaf(pj, vv.x, o[d]);
                o[d + 1] = fmaf(pj, vv.y, o[d + 1]);
                o[d + 2] = fmaf(pj, vv.z, o[d + 2]);
                o[d + 3] = fmaf(pj, vv.w, o[d + 3]);
            }
        }
    }
    if (t0 + i < t_count) {
        const float inv = 1.0f / l;
        float *out = ctx + size_t(t0 + i) * dim + head * HD + OC * part;
#pragma unroll
        for (int d = 0; d < OC; d++)
            out[d] = o[d] * inv;
    }
}

template <int QT>
void launch_qgemm(const float *x, int t_count, const QMat &w, float *c, int ldc,
                  bool add, hipStream_t stream)
{
    const dim3 grid((w.rows + BN - 1) / BN, (t_count + BM - 1) / BM);
    if (add)
        hipLaunchKernelGGL((qgemm_kernel<QT, true>), grid, dim3(kThreads), 0,
                           stream, x, t_count, w, c, ldc);
    else
        hipLaunchKernelGGL((qgemm_kernel<QT, false>), grid, dim3(kThreads), 0,
                           stream, x, t_count, w, c, ldc);
}

} // namespace

bool prefill_gemm_supported(const DecodeShape &s, const LayerView &w)
{
    const QMat *mats[7] = {&w.query, &w.key, &w.value, &w.output,
                           &w.gate, &w.up, &w.down};
    for (const QMat *m : mats)
        if (!fast_layout(*m))
            return false;
    return s.head_dim == 64 || s.head_dim == 128;
}

void launch_embed_rows(const float *embeddings, const int *tokens, float *h,
                       int t_count, int dim, hipStream_t stream)
{
    hipLaunchKernelGGL(embed_rows_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, embeddings, tokens, h, dim);
    check_launch("prefill embed");
}

void launch_rmsnorm_rows(const float *h, const float *w, float *out,
                         int t_count, int dim, hipStream_t stream)
{
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, h, w, out, dim);
    check_launch("prefill rmsnorm");
}

void launch_qgemm_rows(const float *x, int t_count, const QMat &w, float *c,
                       int ldc, bool add, hipStream_t stream)
{
    if (w.type == 1)
        launch_qgemm<1>(x, t_count, w, c, ldc, add, stream);
    else
        launch_qgemm<0>(x, t_count, w, c, ldc, add, stream);
    check_launch("prefill gemm");
}

void launch_rope_store(float *q, const float *k, const float *v,
                       const float2 *rope, float *k_cache, float *v_cache,
                       const DecodeShape &s, int t_count, int start,
                       hipStream_t stream)
{
    hipLaunchKernelGGL(rope_store_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, q, k, v, rope, k_cache, v_cache, s.heads,
                       s.kv_heads, s.head_dim, s.max_seq, start);
    check_launch("prefill rope");
}

void launch_attention_prefill(const float *q, const float *k_cache,
                              const float *v_cache, float *ctx,
                              const DecodeShape &s, int t_count, int start,
                              hipStream_t stream)
{
    const dim3 grid((t_count + AQ - 1) / AQ, s.heads);
    if (s.head_dim == 128)
        hipLaunchKernelGGL(attention_prefill_kernel<128>, grid, dim3(kThreads), 0,
                           stream, q, k_cache, v_cache, ctx, t_count, s.heads,
                           s.kv_heads, s.max_seq, start, s.attn_scale);
    else
        hipLaunchKernelGGL(attention_prefill_kernel<64>, grid, dim3(kThreads), 0,
                           stream, q, k_cache, v_cache, ctx, t_count, s.heads,
                           s.kv_heads, s.max_seq, start, s.attn_scale);
    check_launch("prefill attention");
}

void launch_silu_mul(const float *g, const float *u, float *act, size_t n,
                     hipStream_t stream)
{
    const int blocks = int((n + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                       g, u, act, n);
    check_launch("prefill silu");
}

} // namespace nut
