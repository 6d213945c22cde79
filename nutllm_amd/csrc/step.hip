// step.hip — fast kernels of one decode step (decode_quantized_token,
// src/quant_model.cpp:158-206) for layers whose matrices use 32-wide quant
// blocks along whole rows. Per layer:
//   norm        xn = rmsnorm(h) * attention_norm          (one workgroup)
//   qkv         Q/K/V rows of xn, RoPE, K/V into the cache at *length
//   attn_split  split-K attention: 64-position chunks of one head per
//               workgroup, partial (max, sum, context) per chunk
//   attn_merge  per head: merge the chunks into the context vector
//   wo          h += Wo ctx
//   norm        xn = rmsnorm(h) * ffn_norm
//   gate_up     act = silu(Wg xn) * (Wu xn)
//   down        h += W2 act
// The matvecs stream rows like the standalone matvec: a wave owns R rows
// (an even count, so a RoPE pair stays in one wave), each lane issues its
// 16-byte chunk of every row and its x chunk together, x chunk sums are
// formed in registers, and the R row sums are reduced with DPP.
// Every kernel returns at once when the step state says the loop ended.
#include "kernels.hpp"
#include "runtime.hpp"

namespace nut {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 2;      // rows per wave
constexpr int kChunk = 64;    // positions per attention split

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load_stream(const uint8_t *p)
{
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// sum_k q_k x_k s over rows row0 .. row0 + kRows - 1 of m (rows past the end
// re-read the last row), every lane gets all sums.
template <int QT>
__device__ __forceinline__ void rows_dot(const QMat &m, int row0, const float *x,
                                         float (&out)[kRows])
{
    constexpr int CW = QT == 1 ? 32 : 16;
    constexpr float kBias = QT == 1 ? 8.0f : 128.0f;
    const int lane = threadIdx.x & (kWave - 1);
    const int row_bytes = QT == 1 ? m.cols / 2 : m.cols;
    const int chunks = row_bytes / 16;
    const int bpr = m.cols / 32;
    const uint8_t *rp[kRows];
    const uint16_t *sp[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++) {
        const int rr = min(row0 + r, m.rows - 1);
        rp[r] = m.data + size_t(rr) * row_bytes;
        sp[r] = m.scales + size_t(rr) * bpr;
    }
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++)
        acc[r] = 0.0f;
    for (int c = lane; c < chunks; c += kWave) {
        const int block = QT == 1 ? c : (c >> 1);
        uint4 w[kRows];
        float s[kRows];
#pragma unroll
        for (int r = 0; r < kRows; r++) {
            w[r] = load_stream(rp[r] + 16 * c);
            s[r] = half_bits_to_float(sp[r][block]);
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
        for (int r = 0; r < kRows; r++) {
            const float d = QT == 1 ? dot_int4_chunk(w[r], xc) : dot_int8_chunk(w[r], xc);
            acc[r] = fmaf(s[r], d - kBias * xsum, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < kRows; r++)
        out[r] = wave_total(acc[r]);
}

__device__ __forceinline__ int wave_id()
{
    return __builtin_amdgcn_readfirstlane(blockIdx.x * kWaves + threadIdx.x / kWave);
}

// xn = h * (1 / sqrt(mean(h^2) + 1e-5)) * w  (src/ops.cpp:111-134)
__global__ __launch_bounds__(1024) void norm_kernel(const float *h, const float *w,
                                                    float *xn, int dim,
                                                    const StepState *state)
{
    if (state->done)
        return;
    __shared__ float red[1024 / kWave];
    float sq = 0.0f;
    for (int i = threadIdx.x; i < dim; i += 1024)
        sq = fmaf(h[i], h[i], sq);
    const float total = block_sum(sq, red, 1024 / kWave);
    const float scale = 1.0f / sqrtf(total / float(dim) + 1e-5f);
    for (int i = threadIdx.x; i < dim; i += 1024)
        xn[i] = h[i] * scale * w[i];
}

// Q/K/V rows (concatenated: query rows, key rows, value rows), RoPE on the
// query and key pairs at position *length (src/quant_model.cpp:26-37), key
// and value rows into the layer's cache.
template <int QT>
__global__ __launch_bounds__(kThreads) void qkv_fast_kernel(
    DecodeShape s, const float *xn, QMat wq, QMat wk, QMat wv, const float2 *rope,
    const int *length, float *k_layer, float *v_layer, float *query,
    const StepState *state)
{
    if (state->done)
        return;
    const int kvd = s.kv_heads * s.head_dim;
    const int row = wave_id() * kRows;
    if (row >= s.dim + 2 * kvd)
        return;
    const int which = row < s.dim ? 0 : row < s.dim + kvd ? 1 : 2;
    const int local = which == 0 ? row : which == 1 ? row - s.dim : row - s.dim - kvd;
    float out[kRows];
    rows_dot<QT>(which == 0 ? wq : which == 1 ? wk : wv, local, xn, out);
    const int pos = *length;
    const int head = local / s.head_dim, d = local % s.head_dim;
    if (which < 2) {
        const float2 cs = rope[size_t(pos) * (s.head_dim / 2) + d / 2];
        const float even = out[0], odd = out[1];
        out[0] = fmaf(even, cs.x, -(odd * cs.y));
        out[1] = fmaf(even, cs.y, odd * cs.x);
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        float *dst = which == 0 ? query + local
                                : (which == 1 ? k_layer : v_layer) +
                                      (size_t(head) * s.max_seq + pos) * s.head_dim + d;
        dst[0] = out[0];
        dst[1] = out[1];
    }
}

// y[r] += (W x)[r]  (Wo + residual, W2 + residual)
template <int QT>
__global__ __launch_bounds__(kThreads) void residual_fast_kernel(
    QMat m, const float *x, float *y, const StepState *state)
{
    if (state->done)
        return;
    const int row = wave_id() * kRows;
    if (row >= m.rows)
        return;
    float out[kRows];
    rows_dot<QT>(m, row, x, out);
    if ((threadIdx.x & (kWave - 1)) == 0)
#pragma unroll
        for (int r = 0; r < kRows; r++)
            if (row + r < m.rows)
                y[row + r] += out[r];
}

// act[r] = silu((Wg xn)[r]) * (Wu xn)[r]  (src/quant_model.cpp:197-198)
template <int QT>
__global__ __launch_bounds__(kThreads) void gate_up_fast_kernel(
    QMat wg, QMat wu, const float *xn, float *act, const StepState *state)
{
    if (state->done)
        return;
    const int row = wave_id() * kRows;
    if (row >= wg.rows)
        return;
    float g[kRows], u[kRows];
    rows_dot<QT>(wg, row, xn, g);
    rows_dot<QT>(wu, row, xn, u);
    if ((threadIdx.x & (kWave - 1)) == 0)
#pragma unroll
        for (int r = 0; r < kRows; r++)
            if (row + r < wg.rows)
                act[row + r] = g[r] / (1.0f + expf(-g[r])) * u[r];
}

// Split-K attention (src/quant_model.cpp:68-105 for one chunk of
// positions): workgroup (head, split) covers positions
// [split * kChunk, min(n, (split + 1) * kChunk)), n = *length + 1, and
// writes (max, sum of exp, unnormalised context) for its chunk.
template <int HD>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(
    DecodeShape s, const float *query, const float *k_layer, const float *v_layer,
    const int *length, float *part, int max_splits, const StepState *state)
{
    if (state->done)
        return;
    __shared__ float qs[HD];
    __shared__ float sc[kChunk];
    __shared__ float red[kWaves];
    __shared__ float ctx_part[kThreads / (HD / 4)][HD];
    const int head = blockIdx.x, split = blockIdx.y;
    const int n = *length + 1;
    const int p0 = split * kChunk;
    if (p0 >= n)
        return; // workgroup-uniform
    const int count = min(kChunk, n - p0);
    const int kvh = head / (s.heads / s.kv_heads);
    const float *kg = k_layer + (size_t(kvh) * s.max_seq + p0) * HD;
    const float *vg = v_layer + (size_t(kvh) * s.max_seq + p0) * HD;
    for (int i = threadIdx.x; i < HD; i += kThreads)
        qs[i] = query[head * HD + i];
    __syncthreads();
    // scores: thread (p = tid / 4, quarter = tid % 4) dots a quarter row
    {
        const int p = threadIdx.x >> 2, quarter = threadIdx.x & 3;
        constexpr int Q4 = HD / 16; // float4 per quarter row
        float dot = 0.0f;
        if (p < count) {
            const float4 *kr = reinterpret_cast<const float4 *>(kg + size_t(p) * HD) +
                               quarter * Q4;
            const float4 *q4 = reinterpret_cast<const float4 *>(qs) + quarter * Q4;
#pragma unroll
            for (int j = 0; j < Q4; j++) {
                const float4 k = kr[j], q = q4[j];
                dot = fmaf(q.x, k.x, dot);
                dot = fmaf(q.y, k.y, dot);
                dot = fmaf(q.z, k.z, dot);
                dot = fmaf(q.w, k.w, dot);
            }
        }
        dot += dpp<kDppQuadSwap1>(dot, 0.0f);
        dot += dpp<kDppQuadSwap2>(dot, 0.0f);
        if (quarter == 0 && p < kChunk)
            sc[p] = p < count ? dot * s.attn_scale : -INFINITY;
    }
    __syncthreads();
    float m = -INFINITY;
    if (threadIdx.x < kWave) {
        m = wave_maximum(threadIdx.x < kChunk ? sc[threadIdx.x] : -INFINITY);
        const float e = threadIdx.x < count ? expf(sc[threadIdx.x] - m) : 0.0f;
        sc[threadIdx.x] = e;
        const float l = wave_total(e);
        if (threadIdx.x == 0) {
            red[0] = m;
            red[1] = l;
        }
    }
    __syncthreads();
    // context: thread (group = tid / (HD / 4), quad = tid % (HD / 4))
    // accumulates positions group, group + groups, ...
    constexpr int QUADS = HD / 4, GROUPS = kThreads / QUADS;
    const int quad = threadIdx.x % QUADS, group = threadIdx.x / QUADS;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int p = group; p < count; p += GROUPS) {
        const float w = sc[p];
        const float4 v = reinterpret_cast<const float4 *>(vg + size_t(p) * HD)[quad];
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
    }
    *reinterpret_cast<float4 *>(&ctx_part[group][4 * quad]) = acc;
    __syncthreads();
    float *out = part + (size_t(head) * max_splits + split) * (HD + 2);
    for (int d = threadIdx.x; d < HD; d += kThreads) {
        float sum = 0.0f;
        for (int g = 0; g < GROUPS; g++)
            sum += ctx_part[g][d];
        out[2 + d] = sum;
    }
    if (threadIdx.x == 0) {
        out[0] = red[0];
        out[1] = red[1];
    }
}

// context[head] = sum_s exp(m_s - M) o_s / sum_s exp(m_s - M) l_s
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(const float *part,
                                                        const int *length,
                                                        float *context,
                                                        int max_splits,
                                                        const StepState *state)
{
    if (state->done)
        return;
    const int head = blockIdx.x;
    const int splits = (*length + 1 + kChunk - 1) / kChunk;
    const float *p = part + size_t(head) * max_splits * (HD + 2);
    float mx = -INFINITY;
    for (int s = 0; s < splits; s++)
        mx = fmaxf(mx, p[s * (HD + 2)]);
    float l = 0.0f, o = 0.0f;
    for (int s = 0; s < splits; s++) {
        const float f = expf(p[s * (HD + 2)] - mx);
        l = fmaf(p[s * (HD + 2) + 1], f, l);
        o = fmaf(p[s * (HD + 2) + 2 + threadIdx.x], f, o);
    }
    context[head * HD + threadIdx.x] = o / l;
}

int blocks_for_rows(int rows)
{
    const int waves = (rows + kRows - 1) / kRows;
    return (waves + kWaves - 1) / kWaves;
}

template <int QT, int HD>
void launch_layer_fast_t(const DecodeShape &s, const LayerView &w,
                         const float2 *rope, const int *length, float *k_layer,
                         float *v_layer, const StepBuffers &b,
                         const StepState *state, hipStream_t stream)
{
    const int kvd = s.kv_heads * s.head_dim;
    const int max_splits = (s.max_seq + kChunk - 1) / kChunk;
    hipLaunchKernelGGL(norm_kernel, dim3(1), dim3(1024), 0, stream, b.hidden,
                       w.attention_norm, b.xn, s.dim, state);
    hipLaunchKernelGGL((qkv_fast_kernel<QT>), dim3(blocks_for_rows(s.dim + 2 * kvd)),
                       dim3(kThreads), 0, stream, s, b.xn, w.query, w.key, w.value,
                       rope, length, k_layer, v_layer, b.query, state);
    hipLaunchKernelGGL((attn_split_kernel<HD>), dim3(s.heads, max_splits),
                       dim3(kThreads), 0, stream, s, b.query, k_layer, v_layer,
                       length, b.attn_part, max_splits, state);
    hipLaunchKernelGGL((attn_merge_kernel<HD>), dim3(s.heads), dim3(HD), 0, stream,
                       b.attn_part, length, b.context, max_splits, state);
    hipLaunchKernelGGL((residual_fast_kernel<QT>), dim3(blocks_for_rows(s.dim)),
                       dim3(kThreads), 0, stream, w.output, b.context, b.hidden,
                       state);
    hipLaunchKernelGGL(norm_kernel, dim3(1), dim3(1024), 0, stream, b.hidden,
                       w.ffn_norm, b.xn, s.dim, state);
    hipLaunchKernelGGL((gate_up_fast_kernel<QT>), dim3(blocks_for_rows(s.ffn_dim)),
                       dim3(kThreads), 0, stream, w.gate, w.up, b.xn, b.act, state);
    hipLaunchKernelGGL((residual_fast_kernel<QT>), dim3(blocks_for_rows(s.dim)),
                       dim3(kThreads), 0, stream, w.down, b.act, b.hidden, state);
    check_launch("decode step");
}

} // namespace

bool step_fast_supported(const DecodeShape &s, const LayerView &w)
{
    const QMat *mats[7] = {&w.query, &w.key, &w.value, &w.output,
                           &w.gate, &w.up, &w.down};
    for (const QMat *m : mats)
        if (!fast_layout(*m) || m->type != w.query.type)
            return false;
    return (s.head_dim == 64 || s.head_dim == 128) && s.dim <= 16384 &&
           (s.dim + 2 * s.kv_heads * s.head_dim) % kRows == 0;
}

size_t step_attn_part_floats(const DecodeShape &s)
{
    const size_t splits = (size_t(s.max_seq) + kChunk - 1) / kChunk;
    return size_t(s.heads) * splits * (size_t(s.head_dim) + 2);
}

void launch_layer_fast(const DecodeShape &s, const LayerView &w,
                       const float2 *rope, const int *length, float *k_layer,
                       float *v_layer, const StepBuffers &b,
                       const StepState *state, hipStream_t stream)
{
    if (w.query.type == 1)
        s.head_dim == 128
            ? launch_layer_fast_t<1, 128>(s, w, rope, length, k_layer, v_layer, b, state, stream)
            : launch_layer_fast_t<1, 64>(s, w, rope, length, k_layer, v_layer, b, state, stream);
    else
        s.head_dim == 128
            ? launch_layer_fast_t<0, 128>(s, w, rope, length, k_layer, v_layer, b, state, stream)
            : launch_layer_fast_t<0, 64>(s, w, rope, length, k_layer, v_layer, b, state, stream);
}

} // namespace nut
