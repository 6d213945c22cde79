// step.hip — fast kernels of one decode step (decode_quantized_token,
// src/quant_model.cpp:158-206) for layers whose matrices use 32-wide quant
// blocks along whole rows. Five launches per layer:
//   qkv        xn = rmsnorm(h) * attention_norm folded into the Q/K/V
//              rows, RoPE, K/V into the cache at *length
//   attention  one workgroup per (KV head, split of the positions) for all
//              query heads of the group; online softmax over 32-position
//              chunks; the last workgroup of a KV head to finish merges
//              the splits into the context vectors
//   wo         h += Wo ctx
//   gate_up    act = silu(Wg xn) * (Wu xn), xn = rmsnorm(h) * ffn_norm
//   down       h += W2 act
// The matvecs stream rows: a wave owns R rows (an even count, so a RoPE
// pair stays in one wave), each lane issues its 16-byte chunk of every row
// with nontemporal loads, and the R row sums are reduced with DPP. The
// workgroup stages x (times the norm weights) once in LDS, which keeps the
// x reads of every wave off the L1; the RMSNorm scalar factors out of the
// dot: sum_k q_k s (x_k w_k) r = r * sum_k q_k s (x_k w_k) with
// r = 1 / sqrt(mean(x^2) + 1e-5) (src/ops.cpp:111-134).
// Every kernel returns at once when the step state says the loop ended.
//
// The same launches run T consecutive tokens at once (prompt chunks):
// token t = blockIdx.y (blockIdx.z for attention) sits at position
// *length + t, reads and writes row t of each activation buffer, and
// attends to positions [0, *length + t]. Decode is T = 1.
#include <algorithm>

#include "kernels.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace nut {

namespace {

constexpr int kThreads = kRowThreads;
constexpr int kWaves = kRowWaves;
constexpr int kAttnChunk = 32;    // positions per attention chunk (8 per wave)
constexpr int kAttnMaxSplits = 32;
constexpr int kDppRowRor8 = 0x128; // row_ror:8, lane i <- lane i ^ 8 in a row

__device__ __forceinline__ int wave_id(int block)
{
    return __builtin_amdgcn_readfirstlane(block * kWaves + threadIdx.x / kWave);
}

// Workgroups go to the 8 XCDs round-robin (blockIdx % 8 is the XCD).
constexpr int kXcds = 8;

// The (row block, token) of this workgroup. Decode (CHUNK false): block
// blockIdx.x, token blockIdx.y. Prompt chunks: a flat grid of
// ceil(blocks / 8) * 8 * tokens workgroups in which the chunk's tokens of
// row block b are consecutive workgroups on b's XCD, so that the weight rows
// one of them reads come from that XCD's L2 for the others. Returns false
// for the padding workgroups (block >= blocks).
template <bool CHUNK>
__device__ __forceinline__ bool chunk_cell(int blocks, int tokens, int &block, int &t)
{
    if (!CHUNK) {
        block = blockIdx.x;
        t = blockIdx.y;
        return true;
    }
    const int i = blockIdx.x, rest = i / kXcds;
    t = rest % tokens;
    block = (rest / tokens) * kXcds + i % kXcds;
    return block < blocks;
}

// Q/K/V rows of rmsnorm(h) * attention_norm (concatenated: query rows, key
// rows, value rows; R divides dim and kv_heads * head_dim), RoPE on the
// query and key pairs at position *length (src/quant_model.cpp:26-37), key
// and value rows into the layer's cache.
template <int QT, int R, bool CHUNK = false>
__global__ __launch_bounds__(kThreads) void qkv_fast_kernel(
    DecodeShape s, const float *hidden, const float *norm, QMat wq, QMat wk,
    QMat wv, const float2 *rope, const int *length, float *k_layer,
    float *v_layer, float *query, int blocks, int tokens, const StepState *state)
{
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    int block, t;
    if (state->done || !chunk_cell<CHUNK>(blocks, tokens, block, t))
        return;
    hidden += size_t(t) * s.dim;
    query += size_t(t) * s.dim;
    const int kvd = s.kv_heads * s.head_dim;
    const int row = wave_id(block) * R;
    const bool active = row < s.dim + 2 * kvd;
    const int which = row < s.dim ? 0 : row < s.dim + kvd ? 1 : 2;
    const int local = which == 0 ? row : which == 1 ? row - s.dim : row - s.dim - kvd;
    const uint8_t *rp[R];
    const uint16_t *sp[R];
    row_ptrs<QT, R>(which == 0 ? wq : which == 1 ? wk : wv, local, 0, R, rp, sp);
    float out[R];
    rows_matvec<QT, R, true, !CHUNK>(rp, sp, s.dim, hidden, norm, active, xs, red, out);
    if (!active)
        return;
    const int pos = *length + t;
    const int head = local / s.head_dim, d = local % s.head_dim;
    if (which < 2) {
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            const float2 cs = rope[size_t(pos) * (s.head_dim / 2) + (d + r) / 2];
            const float even = out[r], odd = out[r + 1];
            out[r] = fmaf(even, cs.x, -(odd * cs.y));
            out[r + 1] = fmaf(even, cs.y, odd * cs.x);
        }
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        float *dst = which == 0 ? query + local
                                : (which == 1 ? k_layer : v_layer) +
                                      (size_t(head) * s.max_seq + pos) * s.head_dim + d;
#pragma unroll
        for (int r = 0; r < R; r++)
            dst[r] = out[r];
    }
}

// y[r] += (W x)[r]  (Wo + residual, W2 + residual)
template <int QT, int R, bool CHUNK = false>
__global__ __launch_bounds__(kThreads) void residual_fast_kernel(
    QMat m, const float *x, float *y, int blocks, int tokens, const StepState *state)
{
    extern __shared__ float xs[];
    int block, t;
    if (state->done || !chunk_cell<CHUNK>(blocks, tokens, block, t))
        return;
    x += size_t(t) * m.cols;
    y += size_t(t) * m.rows;
    const int row = wave_id(block) * R;
    const uint8_t *rp[R];
    const uint16_t *sp[R];
    row_ptrs<QT, R>(m, row, 0, R, rp, sp);
    float out[R];
    rows_matvec<QT, R, false, !CHUNK>(rp, sp, m.cols, x, nullptr, row < m.rows, xs, nullptr,
                                      out);
    if (row < m.rows && (threadIdx.x & (kWave - 1)) == 0)
#pragma unroll
        for (int r = 0; r < R; r++)
            if (row + r < m.rows)
                y[row + r] += out[r];
}

// act[r] = silu((Wg xn)[r]) * (Wu xn)[r], xn = rmsnorm(h) * ffn_norm
// (src/quant_model.cpp:194-198); R rows of each matrix per wave.
template <int QT, int R, bool CHUNK = false>
__global__ __launch_bounds__(kThreads) void gate_up_fast_kernel(
    const float *hidden, const float *norm, QMat wg, QMat wu, float *act, int blocks,
    int tokens, const StepState *state)
{
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    int block, t;
    if (state->done || !chunk_cell<CHUNK>(blocks, tokens, block, t))
        return;
    hidden += size_t(t) * wg.cols;
    act += size_t(t) * wg.rows;
    const int row = wave_id(block) * R;
    const uint8_t *rp[2 * R];
    const uint16_t *sp[2 * R];
    row_ptrs<QT, 2 * R>(wg, row, 0, R, rp, sp);
    row_ptrs<QT, 2 * R>(wu, row, R, R, rp, sp);
    float gu[2 * R];
    rows_matvec<QT, 2 * R, true, !CHUNK>(rp, sp, wg.cols, hidden, norm, row < wg.rows, xs, red,
                                         gu);
    if (row < wg.rows && (threadIdx.x & (kWave - 1)) == 0)
#pragma unroll
        for (int r = 0; r < R; r++)
            if (row + r < wg.rows) {
                const float g = gu[r], u = gu[R + r];
                act[row + r] = g / (1.0f + expf(-g)) * u;
            }
}

// Sums / max over lane bits 0-2 or 3-5, in every lane.
__device__ __forceinline__ float sum_lanes_0_2(float v)
{
    v += dpp<kDppQuadSwap1>(v, 0.0f);
    v += dpp<kDppQuadSwap2>(v, 0.0f);
    return v + dpp<kDppRowHalfMirror>(v, 0.0f);
}

__device__ __forceinline__ float sum_lanes_3_5(float v)
{
    v += dpp<kDppRowRor8>(v, 0.0f);
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

__device__ __forceinline__ float max_lanes_0_2(float v)
{
    v = fmaxf(v, dpp<kDppQuadSwap1>(v, -INFINITY));
    v = fmaxf(v, dpp<kDppQuadSwap2>(v, -INFINITY));
    return fmaxf(v, dpp<kDppRowHalfMirror>(v, -INFINITY));
}

// Tagged words of the split results: (tag << 32) | value bits, stored and
// loaded at agent scope, so every XCD sees them whatever its L2 holds. A
// word read with the wrong tag is one whose store has not arrived yet; the
// merge re-reads such words at most kMergeSpin times, then takes NaN (which
// shows in the context).
constexpr int kMergeSpin = 1 << 20;

__device__ __forceinline__ void publish(uint64_t *p, float v, uint32_t tag)
{
    __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t take_word(const uint64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Attention of query heads [G row, G row + G), row = blockIdx.x, over
// positions [0, n), n = *length + 1 (src/quant_model.cpp:68-105); the G
// heads share one KV head. The n positions form 32-position chunks, dealt
// in equal runs to at most gridDim.y splits.
// Workgroup (row, split) loads up to PF chunks at once and runs an online
// softmax over each such group: lane (pl = lane % 8, part = lane / 8) of
// wave w holds position 8 w + pl of every chunk, dims
// [part * HD / 8, (part + 1) * HD / 8) of its K and V rows, and the running
// max, sum and context of each head over its positions. One split writes
// the context directly; otherwise each split publishes (max, sum,
// unnormalised context) and the workgroup that completes the count of its
// row merges them:
//   ctx = sum_s exp(m_s - M) o_s / sum_s exp(m_s - M) l_s,  M = max_s m_s.
// counts[row] counts arrivals over all launches and counts[rows + row] holds
// its value at the start of this launch (the base; rows = gridDim.x, one
// such pair of arrays per token): a workgroup whose
// ticket is base + splits - 1 is the last, and moves the base on. The base
// also tags this launch's words, so the merge needs no memory fence: it
// re-reads a word until the word carries the tag.
template <int HD, int G>
__global__ __launch_bounds__(kThreads) void attention_kernel(
    DecodeShape s, const float *query, const float *k_layer, const float *v_layer,
    const int *length, uint64_t *o_part, uint64_t *ml_part, int *counts,
    float *context, const StepState *state)
{
    if (state->done)
        return;
    constexpr int S = HD / 8;
    // chunks in flight: four while q, the context and the K/V rows fit the
    // register file
    constexpr int PF = 2 * G * S + 8 * S <= 224 ? 4 : 2;
    constexpr int OUT = (G * HD + kThreads - 1) / kThreads;
    const int row = blockIdx.x, split = blockIdx.y, t = blockIdx.z;
    const int kvh = row * G / (s.heads / s.kv_heads);
    const int n = *length + t + 1;
    // token t's query, context, counters and split results
    query += size_t(t) * s.heads * HD;
    context += size_t(t) * s.heads * HD;
    counts += 2 * t * gridDim.x;
    o_part += size_t(t) * s.heads * gridDim.y * (HD + 2);
    ml_part += size_t(t) * s.heads * gridDim.y * (HD + 2);
    const int chunks = (n + kAttnChunk - 1) / kAttnChunk;
    const int want = min(int(gridDim.y), chunks);
    const int per = (chunks + want - 1) / want;
    const int splits = (chunks + per - 1) / per;
    if (split >= splits)
        return; // workgroup-uniform
    const int c_begin = split * per, c_end = min(chunks, c_begin + per);
    const int base = splits > 1 ? __hip_atomic_load(counts + gridDim.x + row, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                                : 0;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int pl = lane & 7, part = lane >> 3, prow = wave * 8 + pl;

    __shared__ float wmax[2][kWaves][G];
    __shared__ float red[kWaves][G][HD];
    __shared__ float lred[kWaves][G];
    __shared__ float fw[kAttnMaxSplits][G];
    __shared__ int last;

    float q[G][S];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float4 *src = reinterpret_cast<const float4 *>(
            query + size_t(row * G + g) * HD + part * S);
#pragma unroll
        for (int j = 0; j < S / 4; j++) {
            const float4 v = src[j];
            q[g][4 * j] = v.x;
            q[g][4 * j + 1] = v.y;
            q[g][4 * j + 2] = v.z;
            q[g][4 * j + 3] = v.w;
        }
    }
    const float *kbase = k_layer + size_t(kvh) * s.max_seq * HD + part * S;
    const float *vbase = v_layer + size_t(kvh) * s.max_seq * HD + part * S;
    float m[G], l[G], acc[G][S];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < S; i++)
            acc[g][i] = 0.0f;
    }
    for (int c0 = c_begin, group = 0; c0 < c_end; c0 += PF, group++) {
        float kb[PF][S], vb[PF][S];
        bool valid[PF];
#pragma unroll
        for (int j = 0; j < PF; j++) {
            const int p = (c0 + j) * kAttnChunk + prow;
            valid[j] = c0 + j < c_end && p < n;
            if (valid[j]) {
                const float4 *k4 = reinterpret_cast<const float4 *>(kbase + size_t(p) * HD);
                const float4 *v4 = reinterpret_cast<const float4 *>(vbase + size_t(p) * HD);
#pragma unroll
                for (int i = 0; i < S / 4; i++) {
                    const float4 a = k4[i], b = v4[i];
                    kb[j][4 * i] = a.x, kb[j][4 * i + 1] = a.y;
                    kb[j][4 * i + 2] = a.z, kb[j][4 * i + 3] = a.w;
                    vb[j][4 * i] = b.x, vb[j][4 * i + 1] = b.y;
                    vb[j][4 * i + 2] = b.z, vb[j][4 * i + 3] = b.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < S; i++)
                    kb[j][i] = vb[j][i] = 0.0f;
            }
        }
        // scores of the group's positions, and their max per head
        float sc[PF][G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float gm = -INFINITY;
#pragma unroll
            for (int j = 0; j < PF; j++) {
                sc[j][g] = -INFINITY;
                if (c0 + j < c_end) { // workgroup-uniform
                    float d = 0.0f;
#pragma unroll
                    for (int i = 0; i < S; i++)
                        d = fmaf(q[g][i], kb[j][i], d);
                    d = sum_lanes_3_5(d);
                    sc[j][g] = valid[j] ? d * s.attn_scale : -INFINITY;
                }
                gm = fmaxf(gm, sc[j][g]);
            }
            gm = max_lanes_0_2(gm);
            if (lane == 0)
                wmax[group & 1][wave][g] = gm;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++) {
            float cm = wmax[group & 1][0][g];
#pragma unroll
            for (int w = 1; w < kWaves; w++)
                cm = fmaxf(cm, wmax[group & 1][w][g]);
            const float mn = fmaxf(m[g], cm);
            const float alpha = expf(m[g] - mn);
            m[g] = mn;
            l[g] *= alpha;
#pragma unroll
            for (int i = 0; i < S; i++)
                acc[g][i] *= alpha;
#pragma unroll
            for (int j = 0; j < PF; j++)
                if (c0 + j < c_end) { // workgroup-uniform
                    const float e = valid[j] ? expf(sc[j][g] - mn) : 0.0f;
                    l[g] += e;
#pragma unroll
                    for (int i = 0; i < S; i++)
                        acc[g][i] = fmaf(e, vb[j][i], acc[g][i]);
                }
        }
    }
    // sum the lanes' positions: within the wave, then over the waves
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int i = 0; i < S; i++)
            acc[g][i] = sum_lanes_0_2(acc[g][i]);
        l[g] = sum_lanes_0_2(l[g]);
        if (pl == 0) {
#pragma unroll
            for (int i = 0; i < S; i++)
                red[wave][g][part * S + i] = acc[g][i];
        }
        if (lane == 0)
            lred[wave][g] = l[g];
    }
    __syncthreads();
    if (splits == 1) {
        for (int t = threadIdx.x; t < G * HD; t += kThreads) {
            const int g = t / HD, d = t % HD;
            float o = 0.0f, lt = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                o += red[w][g][d];
                lt += lred[w][g];
            }
            context[size_t(row * G) * HD + t] = o / lt;
        }
        return;
    }
    const uint32_t tag = uint32_t(base);
    const size_t slot = size_t(row) * gridDim.y + split;
    for (int t = threadIdx.x; t < G * HD; t += kThreads) {
        const int g = t / HD, d = t % HD;
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++)
            o += red[w][g][d];
        publish(o_part + slot * G * HD + t, o, tag);
    }
    if (threadIdx.x < G) {
        float lt = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++)
            lt += lred[w][threadIdx.x];
        // every lane tracked every group max, so m[g] is the split's max
        float mg = m[0];
#pragma unroll
        for (int g = 1; g < G; g++)
            if (int(threadIdx.x) == g)
                mg = m[g];
        publish(ml_part + (slot * G + threadIdx.x) * 2, mg, tag);
        publish(ml_part + (slot * G + threadIdx.x) * 2 + 1, lt, tag);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int ticket = __hip_atomic_fetch_add(counts + row, 1, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        last = ticket - base == splits - 1;
        if (ticket - base == splits - 1)
            __hip_atomic_store(counts + gridDim.x + row, base + splits, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last)
        return;
    // merge: every word is requested at once. Lane sp of a 32-lane half
    // wave takes (m, l) of split sp of one head, so the weights
    // exp(m_s - M) / L come from DPP and one cross-row swap, into LDS; then
    // the context words are re-read together until all carry the tag.
    const uint64_t *ml = ml_part + size_t(row) * gridDim.y * G * 2;
    const uint64_t *op = o_part + size_t(row) * gridDim.y * G * HD;
    uint64_t a[OUT][kAttnMaxSplits];
#pragma unroll
    for (int u = 0; u < OUT; u++) {
        const int e = threadIdx.x + u * kThreads;
#pragma unroll
        for (int j = 0; j < kAttnMaxSplits; j++)
            a[u][j] = e < G * HD && j < splits ? take_word(op + size_t(j) * G * HD + e)
                                               : uint64_t(tag) << 32;
    }
    static_assert(kAttnMaxSplits == 32 && 32 * G <= kThreads, "one half wave per head");
    if (threadIdx.x < 32 * G) {
        const int g = threadIdx.x / 32, sp = threadIdx.x % 32;
        const uint64_t *p = ml + (size_t(sp) * G + g) * 2;
        uint64_t w0 = uint64_t(tag) << 32, w1 = w0;
        if (sp < splits) {
            w0 = take_word(p);
            w1 = take_word(p + 1);
        }
        for (int spin = 0; uint32_t(w0 >> 32) != tag || uint32_t(w1 >> 32) != tag; spin++) {
            if (spin >= kMergeSpin) {
                w0 = w1 = (uint64_t(tag) << 32) | __float_as_uint(__builtin_nanf(""));
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (uint32_t(w0 >> 32) != tag)
                w0 = take_word(p);
            if (uint32_t(w1 >> 32) != tag)
                w1 = take_word(p + 1);
        }
        const float mv = sp < splits ? __uint_as_float(uint32_t(w0)) : -INFINITY;
        const float lv = sp < splits ? __uint_as_float(uint32_t(w1)) : 0.0f;
        float mx = row16_max(mv);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        const float ev = sp < splits ? expf(mv - mx) : 0.0f;
        float total = row16_sum(ev * lv);
        total += __shfl_xor(total, 16);
        fw[sp][g] = ev / total;
    }
    for (int spin = 0;; spin++) {
        bool stale = false;
#pragma unroll
        for (int u = 0; u < OUT; u++)
#pragma unroll
            for (int j = 0; j < kAttnMaxSplits; j++)
                stale |= uint32_t(a[u][j] >> 32) != tag;
        if (!stale)
            break;
        if (spin >= kMergeSpin) {
#pragma unroll
            for (int u = 0; u < OUT; u++)
#pragma unroll
                for (int j = 0; j < kAttnMaxSplits; j++)
                    if (uint32_t(a[u][j] >> 32) != tag)
                        a[u][j] = (uint64_t(tag) << 32) | __float_as_uint(__builtin_nanf(""));
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < OUT; u++) {
            const int e = threadIdx.x + u * kThreads;
#pragma unroll
            for (int j = 0; j < kAttnMaxSplits; j++)
                if (uint32_t(a[u][j] >> 32) != tag)
                    a[u][j] = take_word(op + size_t(j) * G * HD + e);
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < OUT; u++) {
        const int e = threadIdx.x + u * kThreads;
        if (e < G * HD) {
            const int g = e / HD;
            float o = 0.0f;
#pragma unroll
            for (int j = 0; j < kAttnMaxSplits; j++)
                if (j < splits)
                    o = fmaf(__uint_as_float(uint32_t(a[u][j])), fw[j][g], o);
            context[size_t(row * G) * HD + e] = o;
        }
    }
}

int blocks_for_rows(int rows, int per_wave)
{
    const int waves = (rows + per_wave - 1) / per_wave;
    return (waves + kWaves - 1) / kWaves;
}

// Query heads per attention workgroup (they share the K/V rows it loads):
// up to four of head_dim 64, one of 128.
int attention_group(const DecodeShape &s)
{
    const int group = s.heads / s.kv_heads;
    if (s.head_dim != 64)
        return 1;
    return group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
}

// Splits of the attention grid: enough workgroups for the chip's 256 CUs,
// at most kAttnMaxSplits, at most one per chunk of max_seq.
int attention_splits(const DecodeShape &s)
{
    const int rows = s.heads / attention_group(s);
    const int chunks = (s.max_seq + kAttnChunk - 1) / kAttnChunk;
    const int want = (256 + rows - 1) / rows;
    return std::max(1, std::min({want, kAttnMaxSplits, chunks}));
}

template <int HD, int G>
void launch_attention(const DecodeShape &s, const float *k_layer, const float *v_layer,
                      const int *length, const StepBuffers &b, int tokens,
                      const StepState *state, hipStream_t stream)
{
    const int splits = attention_splits(s);
    uint64_t *o_part = b.attn_part;
    uint64_t *ml_part = b.attn_part + size_t(s.heads) * splits * HD;
    hipLaunchKernelGGL((attention_kernel<HD, G>), dim3(s.heads / G, splits, tokens),
                       dim3(kThreads), 0, stream, s, b.query, k_layer, v_layer, length,
                       o_part, ml_part, b.attn_count, b.context, state);
}

template <int HD>
void launch_attention_g(const DecodeShape &s, const float *k_layer, const float *v_layer,
                        const int *length, const StepBuffers &b, int tokens,
                        const StepState *state, hipStream_t stream)
{
    const int g = attention_group(s);
    if constexpr (HD == 64) {
        if (g == 4) {
            launch_attention<HD, 4>(s, k_layer, v_layer, length, b, tokens, state, stream);
            return;
        }
        if (g == 2) {
            launch_attention<HD, 2>(s, k_layer, v_layer, length, b, tokens, state, stream);
            return;
        }
    }
    launch_attention<HD, 1>(s, k_layer, v_layer, length, b, tokens, state, stream);
}

// Grid of a row kernel over `blocks` row blocks and `tokens` tokens, in the
// layout chunk_cell<CHUNK> reads.
dim3 row_grid(int blocks, int tokens, bool chunk)
{
    if (!chunk)
        return dim3(blocks, tokens);
    return dim3(((blocks + kXcds - 1) / kXcds) * kXcds * tokens);
}

// One layer on the step kernels. CHUNK: a prompt chunk of several tokens,
// whose workgroups of one row block share an XCD and read the weights
// through the caches; otherwise one token, weights streamed.
template <int QT, int HD, bool CHUNK>
void launch_layer_fast_c(const DecodeShape &s, const LayerView &w,
                         const float2 *rope, const int *length, float *k_layer,
                         float *v_layer, const StepBuffers &b, int tokens,
                         const StepState *state, hipStream_t stream)
{
    const int kvd = s.kv_heads * s.head_dim;
    const size_t x_dim = staged_x_bytes<QT>(s.dim), x_ffn = staged_x_bytes<QT>(s.ffn_dim);
    const int qkv_rows = s.dim + 2 * kvd;
    // Four rows per wave where that still gives every CU a workgroup, and
    // for prompt chunks of 6+ tokens, whose workgroups would otherwise take
    // several rounds of the chip's wave slots. TinyLlama INT4 prompts, every
    // row launch at four rows per wave against two: 15 tokens 1.987 ->
    // 1.854 ms, 8 tokens 1.296 -> 1.226, 7 tokens 1.216 -> 1.165, 6 tokens
    // 1.090 -> 1.070; but 5 tokens 0.998 -> 1.013, 4 tokens 0.893 -> 0.917,
    // 3 tokens 0.818 -> 0.850.
    const bool wide_chunk = CHUNK && tokens >= 6;
    if ((qkv_rows >= 8192 || wide_chunk) && s.dim % 4 == 0 && kvd % 4 == 0) {
        const int blocks = blocks_for_rows(qkv_rows, 4);
        hipLaunchKernelGGL((qkv_fast_kernel<QT, 4, CHUNK>), row_grid(blocks, tokens, CHUNK),
                           dim3(kThreads), x_dim, stream, s, b.hidden, w.attention_norm,
                           w.query, w.key, w.value, rope, length, k_layer, v_layer,
                           b.query, blocks, tokens, state);
    } else {
        const int blocks = blocks_for_rows(qkv_rows, 2);
        hipLaunchKernelGGL((qkv_fast_kernel<QT, 2, CHUNK>), row_grid(blocks, tokens, CHUNK),
                           dim3(kThreads), x_dim, stream, s, b.hidden, w.attention_norm,
                           w.query, w.key, w.value, rope, length, k_layer, v_layer,
                           b.query, blocks, tokens, state);
    }
    launch_attention_g<HD>(s, k_layer, v_layer, length, b, tokens, state, stream);
    // Wo and W2 + residual: four rows per wave for chunks of 6+ tokens
    const int dim_blocks = blocks_for_rows(s.dim, wide_chunk ? 4 : 2);
    auto residual = [&](const QMat &m, const float *x, size_t x_bytes) {
        if (wide_chunk)
            hipLaunchKernelGGL((residual_fast_kernel<QT, 4, CHUNK>),
                               row_grid(dim_blocks, tokens, CHUNK), dim3(kThreads), x_bytes,
                               stream, m, x, b.hidden, dim_blocks, tokens, state);
        else
            hipLaunchKernelGGL((residual_fast_kernel<QT, 2, CHUNK>),
                               row_grid(dim_blocks, tokens, CHUNK), dim3(kThreads), x_bytes,
                               stream, m, x, b.hidden, dim_blocks, tokens, state);
    };
    residual(w.output, b.context, x_dim);
    if (s.ffn_dim >= 8192 || wide_chunk) {
        const int blocks = blocks_for_rows(s.ffn_dim, 4);
        hipLaunchKernelGGL((gate_up_fast_kernel<QT, 4, CHUNK>), row_grid(blocks, tokens, CHUNK),
                           dim3(kThreads), x_dim, stream, b.hidden, w.ffn_norm, w.gate, w.up,
                           b.act, blocks, tokens, state);
    } else {
        const int blocks = blocks_for_rows(s.ffn_dim, 2);
        hipLaunchKernelGGL((gate_up_fast_kernel<QT, 2, CHUNK>), row_grid(blocks, tokens, CHUNK),
                           dim3(kThreads), x_dim, stream, b.hidden, w.ffn_norm, w.gate, w.up,
                           b.act, blocks, tokens, state);
    }
    residual(w.down, b.act, x_ffn);
    check_launch("decode step");
}

template <int QT, int HD>
void launch_layer_fast_t(const DecodeShape &s, const LayerView &w,
                         const float2 *rope, const int *length, float *k_layer,
                         float *v_layer, const StepBuffers &b, int tokens,
                         const StepState *state, hipStream_t stream)
{
    if (tokens > 1)
        launch_layer_fast_c<QT, HD, true>(s, w, rope, length, k_layer, v_layer, b, tokens,
                                          state, stream);
    else
        launch_layer_fast_c<QT, HD, false>(s, w, rope, length, k_layer, v_layer, b, tokens,
                                           state, stream);
}

} // namespace

bool step_fast_supported(const DecodeShape &s, const LayerView &w)
{
    const QMat *mats[7] = {&w.query, &w.key, &w.value, &w.output,
                           &w.gate, &w.up, &w.down};
    for (const QMat *m : mats)
        if (!fast_layout(*m) || m->type != w.query.type)
            return false;
    const int group = s.kv_heads > 0 ? s.heads / s.kv_heads : 0;
    // the staged x of every matvec fits a workgroup's 64 KB of LDS
    const int cols = std::max(s.dim, s.ffn_dim);
    const size_t staged = w.query.type == 1 ? staged_x_bytes<1>(cols) : staged_x_bytes<0>(cols);
    return (s.head_dim == 64 || s.head_dim == 128) && staged <= 65536 &&
           s.heads == group * s.kv_heads &&
           (group == 1 || group == 2 || group == 4 || group == 8) &&
           s.dim % 2 == 0 && (s.kv_heads * s.head_dim) % 2 == 0;
}

size_t step_attn_part_words(const DecodeShape &s)
{
    return size_t(kStepTokensMax) * s.heads * attention_splits(s) * (size_t(s.head_dim) + 2);
}

void launch_layer_fast(const DecodeShape &s, const LayerView &w,
                       const float2 *rope, const int *length, float *k_layer,
                       float *v_layer, const StepBuffers &b, int tokens,
                       const StepState *state, hipStream_t stream)
{
    require(tokens >= 1 && tokens <= kStepTokensMax, NUT_EINVAL,
            "decode step: token count out of range");
    if (w.query.type == 1)
        s.head_dim == 128
            ? launch_layer_fast_t<1, 128>(s, w, rope, length, k_layer, v_layer, b, tokens, state, stream)
            : launch_layer_fast_t<1, 64>(s, w, rope, length, k_layer, v_layer, b, tokens, state, stream);
    else
        s.head_dim == 128
            ? launch_layer_fast_t<0, 128>(s, w, rope, length, k_layer, v_layer, b, tokens, state, stream)
            : launch_layer_fast_t<0, 64>(s, w, rope, length, k_layer, v_layer, b, tokens, state, stream);
}

} // namespace nut
