// decode.hip — one decode step of the quantised decoder on gfx950.
//
// A step is decode_quantized_token (src/quant_model.cpp:158-206); per layer
// it runs five kernels, each fusing the elementwise work around its matvec:
//   qkv        rmsnorm prologue, Q/K/V rows, RoPE epilogue, K/V cache store
//   attention  GQA softmax(q.K^T / sqrt(hd)) V over positions 0..length
//   output     ctx -> Wo rows, residual add into the hidden state
//   gate_up    rmsnorm prologue, gate and up rows, silu(gate)*up epilogue
//   down       act -> W2 rows, residual add into the hidden state
// then a finish kernel advances the device KV length. The classifier kernel
// fuses the final rmsnorm, the fp32 matvec and a per-block argmax; pick
// reduces the blocks to the first maximal index (std::max_element,
// src/generate.cpp:28-30).
//
// Every kernel first reads StepState::done, so a step enqueued after eos is
// a no-op and a whole greedy generation can be enqueued without host syncs.
#include "kernels.hpp"
#include "runtime.hpp"

#include <climits>

namespace nut {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

__device__ __forceinline__ void chunk_sums(const float *xs, float *xsum,
                                           int n, int cw)
{
    const int chunks = (n + cw - 1) / cw;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
        float s = 0.0f;
        const int end = min(n, (c + 1) * cw);
        for (int i = c * cw; i < end; i++)
            s += xs[i];
        xsum[c] = s;
    }
    __syncthreads();
}

// xs = rmsnorm(h) * w (src/ops.cpp:111-134: scale = 1/sqrt(mean(h^2) +
// 1e-5), out = h * scale * w), plus per-chunk sums when xsum is given.
__device__ __forceinline__ void stage_rmsnorm(const float *h, const float *w,
                                              float *xs, float *xsum, int n,
                                              int cw, float *red)
{
    float squares = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = h[i];
        xs[i] = v;
        squares = fmaf(v, v, squares);
    }
    const float total = block_sum(squares, red, blockDim.x / kWave);
    const float scale = 1.0f / sqrtf(total / float(n) + 1e-5f);
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        xs[i] = xs[i] * scale * w[i];
    __syncthreads();
    if (xsum != nullptr)
        chunk_sums(xs, xsum, n, cw);
}

// Two consecutive rows of m (the second may be past the end).
__device__ __forceinline__ void two_rows(const QMat &m, int row,
                                         const float *xs, const float *xsum,
                                         float (&out)[2])
{
    if (fast_layout(m)) {
        qrows_fast<2>(m, row, xs, xsum, out);
    } else {
        out[0] = qrow_generic(m, row, xs);
        out[1] = row + 1 < m.rows ? qrow_generic(m, row + 1, xs) : 0.0f;
    }
}

__global__ void embed_kernel(const float *embeddings, const int *token_ptr,
                             const StepState *state, float *hidden, int dim)
{
    if (state->done)
        return;
    const size_t token = size_t(*token_ptr);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim;
         i += gridDim.x * blockDim.x)
        hidden[i] = embeddings[token * dim + i];
}

// attention_step's projections (src/quant_model.cpp:54-66): rows of
// [Wq; Wk; Wv] in pairs; RoPE on q and k pairs (rotate_vector, lines 26-37)
// with the host-built cos/sin table; k and v go to the cache at `length`.
__global__ __launch_bounds__(kThreads) void qkv_kernel(
    DecodeShape s, const float *hidden, const float *norm, QMat wq, QMat wk,
    QMat wv, const float2 *rope, const int *length, float *k_layer,
    float *v_layer, float *query, const StepState *state)
{
    if (state->done)
        return;
    extern __shared__ float lds[];
    const int cw = chunk_weights(wq.type);
    float *xs = lds;
    float *xsum = xs + s.dim;
    float *red = xsum + (s.dim + cw - 1) / cw;
    stage_rmsnorm(hidden, norm, xs, xsum, s.dim, cw, red);
    const int pos = *length;
    const int kvd = s.kv_heads * s.head_dim;
    const int tiles = (s.dim + 2 * kvd) / 2;
    const int lane = threadIdx.x & (kWave - 1);
    for (int t = blockIdx.x * kWaves + threadIdx.x / kWave; t < tiles;
         t += gridDim.x * kWaves) {
        const int row = 2 * t;
        int which, local;
        if (row < s.dim) {
            which = 0;
            local = row;
        } else if (row < s.dim + kvd) {
            which = 1;
            local = row - s.dim;
        } else {
            which = 2;
            local = row - s.dim - kvd;
        }
        const QMat &m = which == 0 ? wq : (which == 1 ? wk : wv);
        float out[2];
        two_rows(m, local, xs, xsum, out);
        const int head = local / s.head_dim;
        const int d = local - head * s.head_dim;
        if (which < 2) {
            const float2 cs = rope[size_t(pos) * (s.head_dim / 2) + d / 2];
            const float even = out[0], odd = out[1];
            out[0] = fmaf(even, cs.x, -(odd * cs.y));
            out[1] = fmaf(even, cs.y, odd * cs.x);
        }
        if (lane == 0) {
            float *dst;
            if (which == 0)
                dst = query + local;
            else
                dst = (which == 1 ? k_layer : v_layer) +
                      (size_t(head) * s.max_seq + pos) * s.head_dim + d;
            dst[0] = out[0];
            dst[1] = out[1];
        }
    }
}

// The GQA score / softmax / context loops of attention_step
// (src/quant_model.cpp:68-105) for one query head per workgroup.
__global__ __launch_bounds__(kThreads) void attention_kernel(
    DecodeShape s, const float *query, const float *k_layer,
    const float *v_layer, const int *length, float *context,
    const StepState *state)
{
    if (state->done)
        return;
    extern __shared__ float lds[];
    const int hd = s.head_dim;
    const int head = blockIdx.x;
    const int kvh = head / (s.heads / s.kv_heads);
    const int n = *length + 1;
    float *qs = lds;
    float *part = qs + hd;          // kThreads floats
    float *red = part + kThreads;   // kWaves floats
    float *scores = red + kWaves;   // max_seq floats
    for (int i = threadIdx.x; i < hd; i += blockDim.x)
        qs[i] = query[head * hd + i];
    __syncthreads();
    const float *keys = k_layer + size_t(kvh) * s.max_seq * hd;
    const float *values = v_layer + size_t(kvh) * s.max_seq * hd;
    float local_max = -INFINITY;
    for (int p = threadIdx.x; p < n; p += blockDim.x) {
        const float4 *kr = reinterpret_cast<const float4 *>(keys + size_t(p) * hd);
        float dot = 0.0f;
        for (int d4 = 0; d4 < hd / 4; d4++) {
            const float4 k = kr[d4];
            dot = fmaf(qs[4 * d4 + 0], k.x, dot);
            dot = fmaf(qs[4 * d4 + 1], k.y, dot);
            dot = fmaf(qs[4 * d4 + 2], k.z, dot);
            dot = fmaf(qs[4 * d4 + 3], k.w, dot);
        }
        const float score = dot * s.attn_scale;
        scores[p] = score;
        local_max = fmaxf(local_max, score);
    }
    const float maximum = block_max(local_max, red, kWaves);
    float local_sum = 0.0f;
    for (int p = threadIdx.x; p < n; p += blockDim.x) {
        const float e = expf(scores[p] - maximum);
        scores[p] = e;
        local_sum += e;
    }
    const float total = block_sum(local_sum, red, kWaves);
    const int groups = blockDim.x / hd;
    const int g = threadIdx.x / hd, d = threadIdx.x - g * hd;
    float acc = 0.0f;
    if (g < groups)
        for (int p = g; p < n; p += groups)
            acc = fmaf(scores[p], values[size_t(p) * hd + d], acc);
    part[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < hd) {
        float sum = 0.0f;
        for (int gg = 0; gg < groups; gg++)
            sum += part[gg * hd + threadIdx.x];
        context[head * hd + threadIdx.x] = sum / total;
    }
}

// hidden[r] += (W x)[r]: the Wo projection + residual
// (src/quant_model.cpp:106-107,187) and W2 + residual (199-202).
__global__ __launch_bounds__(kThreads) void residual_kernel(
    QMat m, const float *x, float *hidden, const StepState *state)
{
    if (state->done)
        return;
    extern __shared__ float lds[];
    const int cw = chunk_weights(m.type);
    float *xs = lds;
    float *xsum = xs + m.cols;
    stage_x(x, xs, xsum, m.cols, cw);
    const int lane = threadIdx.x & (kWave - 1);
    const int tiles = (m.rows + 1) / 2;
    for (int t = blockIdx.x * kWaves + threadIdx.x / kWave; t < tiles;
         t += gridDim.x * kWaves) {
        float out[2];
        two_rows(m, 2 * t, xs, xsum, out);
        if (lane == 0) {
            hidden[2 * t] += out[0];
            if (2 * t + 1 < m.rows)
                hidden[2 * t + 1] += out[1];
        }
    }
}

// Feed-forward input side (src/quant_model.cpp:189-198): rmsnorm, gate and
// up rows, gate = silu(gate) * up with silu(v) = v / (1 + exp(-v)).
__global__ __launch_bounds__(kThreads) void gate_up_kernel(
    DecodeShape s, const float *hidden, const float *norm, QMat wg, QMat wu,
    float *act, const StepState *state)
{
    if (state->done)
        return;
    extern __shared__ float lds[];
    const int cw = chunk_weights(wg.type);
    float *xs = lds;
    float *xsum = xs + s.dim;
    float *red = xsum + (s.dim + cw - 1) / cw;
    stage_rmsnorm(hidden, norm, xs, xsum, s.dim, cw, red);
    const int lane = threadIdx.x & (kWave - 1);
    const int tiles = (s.ffn_dim + 1) / 2;
    for (int t = blockIdx.x * kWaves + threadIdx.x / kWave; t < tiles;
         t += gridDim.x * kWaves) {
        float g[2], u[2];
        two_rows(wg, 2 * t, xs, xsum, g);
        two_rows(wu, 2 * t, xs, xsum, u);
        if (lane == 0) {
            act[2 * t] = g[0] / (1.0f + expf(-g[0])) * u[0];
            if (2 * t + 1 < s.ffn_dim)
                act[2 * t + 1] = g[1] / (1.0f + expf(-g[1])) * u[1];
        }
    }
}

__global__ void finish_step_kernel(const StepState *state, int *length)
{
    if (!state->done)
        *length += 1;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi)
{
    return v > bv || (v == bv && i < bi);
}

// Final rmsnorm + fp32 classifier rows (src/generate.cpp:197-200,
// src/threading.cpp:183-198) and the block's first maximal logit.
__global__ __launch_bounds__(kThreads) void classifier_kernel(
    DecodeShape s, const float *hidden, const float *final_norm,
    const float *weights, float *logits, float *part_val, int *part_idx,
    const StepState *state)
{
    if (state->done)
        return;
    extern __shared__ float lds[];
    float *xs = lds;
    float *red = xs + s.dim;
    __shared__ float wave_val[kWaves];
    __shared__ int wave_idx[kWaves];
    stage_rmsnorm(hidden, final_norm, xs, nullptr, s.dim, 1, red);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    float best_v = -INFINITY;
    int best_i = INT_MAX;
    const bool vec = (s.dim & 3) == 0;
    for (int row = blockIdx.x * kWaves + wave; row < s.vocab;
         row += gridDim.x * kWaves) {
        const float *wr = weights + size_t(row) * s.dim;
        float acc = 0.0f;
        if (vec) {
            for (int c = lane; c < s.dim / 4; c += kWave) {
                const float4 v = reinterpret_cast<const float4 *>(wr)[c];
                const float *xc = xs + 4 * c;
                acc = fmaf(v.x, xc[0], acc);
                acc = fmaf(v.y, xc[1], acc);
                acc = fmaf(v.z, xc[2], acc);
                acc = fmaf(v.w, xc[3], acc);
            }
        } else {
            for (int c = lane; c < s.dim; c += kWave)
                acc = fmaf(wr[c], xs[c], acc);
        }
        acc = wave_sum(acc);
        if (logits != nullptr && lane == 0)
            logits[row] = acc;
        if (better(acc, row, best_v, best_i)) {
            best_v = acc;
            best_i = row;
        }
    }
    if (lane == 0) {
        wave_val[wave] = best_v;
        wave_idx[wave] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kWaves; w++)
            if (better(wave_val[w], wave_idx[w], best_v, best_i)) {
                best_v = wave_val[w];
                best_i = wave_idx[w];
            }
        part_val[blockIdx.x] = best_v;
        part_idx[blockIdx.x] = best_i;
    }
}

// choose_token's greedy branch and the loop's eos test
// (src/generate.cpp:24-30,200-205).
__global__ __launch_bounds__(kThreads) void pick_token_kernel(
    const float *part_val, const int *part_idx, int parts, StepState *state,
    int *tokens, int eos)
{
    if (state->done)
        return;
    __shared__ float vals[kThreads];
    __shared__ int idxs[kThreads];
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int i = threadIdx.x; i < parts; i += blockDim.x)
        if (better(part_val[i], part_idx[i], bv, bi)) {
            bv = part_val[i];
            bi = part_idx[i];
        }
    vals[threadIdx.x] = bv;
    idxs[threadIdx.x] = bi;
    __syncthreads();
    for (int stride = blockDim.x / 2; stride > 0; stride >>= 1) {
        if (threadIdx.x < stride &&
            better(vals[threadIdx.x + stride], idxs[threadIdx.x + stride],
                   vals[threadIdx.x], idxs[threadIdx.x])) {
            vals[threadIdx.x] = vals[threadIdx.x + stride];
            idxs[threadIdx.x] = idxs[threadIdx.x + stride];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        // An all-NaN row leaves INT_MAX; std::max_element would return 0.
        const int token = idxs[0] == INT_MAX ? 0 : idxs[0];
        if (token == eos) {
            state->done = 1;
        } else {
            tokens[state->count] = token;
            state->count += 1;
            state->token = token;
        }
    }
}

// The screening copy of the fp32 classifier as INT8 block-32 codes, one
// thread per (row, block): the scale s = the smallest fp16 >= max|w| / 127
// and >= 2^-14 (so no code needs clamping, |w - s q| <= s / 2, and no
// scale is subnormal), q = rint(w / s) in double. A block with a non-finite weight gets a NaN scale (its rows
// always stay candidates), an all-zero block s = 0.
__global__ __launch_bounds__(kThreads) void classifier_screen_kernel(
    const float *w, int vocab, int dim, int8_t *codes, uint16_t *scales)
{
    const int blocks = dim / 32;
    const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
    if (i >= (long long)vocab * blocks)
        return;
    float v[32];
    const float4 *src = reinterpret_cast<const float4 *>(w + i * 32);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float4 f = src[k];
        v[4 * k] = f.x;
        v[4 * k + 1] = f.y;
        v[4 * k + 2] = f.z;
        v[4 * k + 3] = f.w;
    }
    float m = 0.0f;
    bool finite = true;
#pragma unroll
    for (int k = 0; k < 32; k++) {
        finite = finite && isfinite(v[k]);
        m = fmaxf(m, fabsf(v[k]));
    }
    uint16_t bits = 0;
    double inv = 0.0;
    if (!finite) {
        bits = 0x7e00; // NaN
    } else if (m > 0.0f) {
        const double t = double(m) / 127.0;
        bits = __builtin_bit_cast(uint16_t, _Float16(float(t)));
        if (double(__builtin_bit_cast(_Float16, bits)) < t)
            bits++; // the next fp16 up (t > 0)
        // never a subnormal scale (a flush to zero would void the bound)
        bits = bits < 0x0400u ? uint16_t(0x0400u) : bits;
        // w / s as w * (1 / s) in double: off the exact quotient by far
        // less than the 2^-10 s the bound allows beyond s / 2
        inv = 1.0 / double(__builtin_bit_cast(_Float16, bits));
    }
    uint32_t packed[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const double q = fmin(127.0, fmax(-127.0, rint(double(v[4 * k + e]) * inv)));
            word |= uint32_t(uint8_t(int8_t(q))) << (8 * e);
        }
        packed[k] = word;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(codes + i * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    scales[i] = bits;
}

__global__ void set_int_kernel(int *target, int value) { *target = value; }

__global__ void reset_state_kernel(StepState *state, int token)
{
    state->token = token;
    state->done = 0;
    state->count = 0;
}

int blocks_for_tiles(int tiles)
{
    return tiles <= 0 ? 1 : (tiles + kWaves - 1) / kWaves;
}

} // namespace

void launch_embed(const DecodeShape &s, const float *embeddings,
                  const int *token_ptr, const StepState *state, float *hidden,
                  hipStream_t stream)
{
    hipLaunchKernelGGL(embed_kernel, dim3((s.dim + 255) / 256), dim3(256), 0,
                       stream, embeddings, token_ptr, state, hidden, s.dim);
    check_launch("decode: embedding");
}

void launch_attention(const DecodeShape &s, const float *query, const float *k_layer,
                      const float *v_layer, const int *length, float *context,
                      const StepState *state, hipStream_t stream)
{
    const size_t attn_lds =
        sizeof(float) * (size_t(s.head_dim) + kThreads + kWaves + s.max_seq);
    hipLaunchKernelGGL(attention_kernel, dim3(s.heads), dim3(kThreads), attn_lds, stream, s,
                       query, k_layer, v_layer, length, context, state);
    check_launch("decode: attention");
}

void launch_layer(const DecodeShape &s, const LayerView &w,
                  const float2 *rope, const int *length, float *k_layer,
                  float *v_layer, float *hidden, float *query, float *context,
                  float *act, const StepState *state, hipStream_t stream)
{
    const int cw = chunk_weights(w.query.type);
    const size_t norm_lds =
        sizeof(float) * (size_t(s.dim) + (s.dim + cw - 1) / cw + kWaves);
    const int kvd = s.kv_heads * s.head_dim;

    hipLaunchKernelGGL(qkv_kernel, dim3(blocks_for_tiles((s.dim + 2 * kvd) / 2)),
                       dim3(kThreads), norm_lds, stream, s, hidden,
                       w.attention_norm, w.query, w.key, w.value, rope, length,
                       k_layer, v_layer, query, state);
    check_launch("decode: qkv");

    const size_t attn_lds =
        sizeof(float) * (size_t(s.head_dim) + kThreads + kWaves + s.max_seq);
    hipLaunchKernelGGL(attention_kernel, dim3(s.heads), dim3(kThreads),
                       attn_lds, stream, s, query, k_layer, v_layer, length,
                       context, state);
    check_launch("decode: attention");

    hipLaunchKernelGGL(residual_kernel,
                       dim3(blocks_for_tiles((w.output.rows + 1) / 2)),
                       dim3(kThreads), matvec_q_lds_bytes(w.output), stream,
                       w.output, context, hidden, state);
    check_launch("decode: output projection");

    hipLaunchKernelGGL(gate_up_kernel,
                       dim3(blocks_for_tiles((s.ffn_dim + 1) / 2)),
                       dim3(kThreads), norm_lds, stream, s, hidden,
                       w.ffn_norm, w.gate, w.up, act, state);
    check_launch("decode: gate/up");

    hipLaunchKernelGGL(residual_kernel,
                       dim3(blocks_for_tiles((w.down.rows + 1) / 2)),
                       dim3(kThreads), matvec_q_lds_bytes(w.down), stream,
                       w.down, act, hidden, state);
    check_launch("decode: down projection");
}

void launch_finish_step(const StepState *state, int *length,
                        hipStream_t stream)
{
    hipLaunchKernelGGL(finish_step_kernel, dim3(1), dim3(1), 0, stream, state,
                       length);
    check_launch("decode: finish");
}

int classifier_blocks(const DecodeShape &s)
{
    const int blocks = (s.vocab + kWaves - 1) / kWaves;
    return blocks > 1024 ? 1024 : blocks;
}

void launch_classifier(const DecodeShape &s, const float *hidden,
                       const float *final_norm, const float *weights,
                       float *logits, float *part_val, int *part_idx,
                       const StepState *state, hipStream_t stream)
{
    const size_t lds = sizeof(float) * (size_t(s.dim) + kWaves);
    hipLaunchKernelGGL(classifier_kernel, dim3(classifier_blocks(s)),
                       dim3(kThreads), lds, stream, s, hidden, final_norm,
                       weights, logits, part_val, part_idx, state);
    check_launch("generation: classifier");
}

void launch_classifier_screen(const float *weights, int vocab, int dim, int8_t *codes,
                              uint16_t *scales, hipStream_t stream)
{
    const long long cells = (long long)vocab * (dim / 32);
    hipLaunchKernelGGL(classifier_screen_kernel, dim3(unsigned((cells + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, stream, weights, vocab, dim, codes, scales);
    check_launch("classifier screening copy");
}

void launch_set_int(int *target, int value, hipStream_t stream)
{
    hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, stream, target,
                       value);
    check_launch("device state update");
}

void launch_reset_state(StepState *state, int token, hipStream_t stream)
{
    hipLaunchKernelGGL(reset_state_kernel, dim3(1), dim3(1), 0, stream, state,
                       token);
    check_launch("device state update");
}

void launch_pick_token(const DecodeShape &s, const float *part_val,
                       const int *part_idx, int parts, StepState *state,
                       int *tokens, hipStream_t stream)
{
    hipLaunchKernelGGL(pick_token_kernel, dim3(1), dim3(kThreads), 0, stream,
                       part_val, part_idx, parts, state, tokens, s.eos);
    check_launch("generation: argmax");
}

} // namespace nut
