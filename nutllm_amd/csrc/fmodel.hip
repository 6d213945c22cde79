// fmodel.hip — the fp32 model path on gfx950: decode_token and
// prefill_tokens (src/kvcache.cpp:237-284) over the device KV cache, with
// ModelWeights' [in x out] fp32 projections resident in HBM.
//
// One decode step per layer: the Q/K/V, Wo, gate/up and down projections
// are column GEMVs (y_j = sum_i x_i W[i][j], linear_threaded,
// src/threading.cpp:200-215): a workgroup takes 256 consecutive columns and
// a run of the input, reads each weight row run coalesced, and writes a
// partial sum; a small epilogue kernel adds the partials in order and
// applies what follows the projection (RoPE and the cache store for Q/K/V,
// the residual add, silu(gate) * up). RMSNorm (src/ops.cpp:111-134) is the
// GEMV's prologue: every workgroup forms x * scale * w for its run after
// summing the squares of all of x. Attention is the quantised decode step's
// kernel (decode.hip), since the cache and the arithmetic are the same.
#include "fmodel.hpp"
#include "runtime.hpp"

#include <algorithm>
#include <cmath>
#include <memory>

namespace nut {

namespace {

constexpr int kCols = 256;
// a GEMV's partial sums, per projection: splits x out floats
constexpr size_t kPartialFloats = size_t(1) << 20;

template <bool NORM>
__global__ __launch_bounds__(kCols) void colgemv_kernel(const float *x, int in,
                                                        const float *norm_w, const float *w,
                                                        int out, int run, float *partial)
{
    extern __shared__ float xs[];
    __shared__ float red[kCols / kWave];
    const int k0 = blockIdx.y * run, k1 = min(in, k0 + run);
    float scale = 1.0f;
    if (NORM) {
        float sq = 0.0f;
        for (int i = threadIdx.x; i < in; i += kCols)
            sq = fmaf(x[i], x[i], sq);
        scale = 1.0f / sqrtf(block_sum(sq, red, kCols / kWave) / float(in) + 1e-5f);
    }
    for (int k = k0 + threadIdx.x; k < k1; k += kCols)
        xs[k - k0] = NORM ? x[k] * scale * norm_w[k] : x[k];
    __syncthreads();
    const int j = blockIdx.x * kCols + threadIdx.x;
    if (j >= out)
        return;
    const float *col = w + size_t(k0) * out + j;
    float acc = 0.0f;
    for (int k = 0; k < k1 - k0; k++)
        acc = fmaf(xs[k], col[size_t(k) * out], acc);
    partial[size_t(blockIdx.y) * out + j] = acc;
}

__device__ __forceinline__ float sum_parts(const float *partial, int splits, int out, int j)
{
    float s = 0.0f;
    for (int p = 0; p < splits; p++)
        s += partial[size_t(p) * out + j];
    return s;
}

__global__ void residual_kernel(const float *partial, int splits, int out, float *h)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < out)
        h[j] += sum_parts(partial, splits, out, j);
}

__global__ void swiglu_kernel(const float *pg, int gs, const float *pu, int us, int ffn,
                              float *act)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < ffn) {
        const float g = sum_parts(pg, gs, ffn, j), u = sum_parts(pu, us, ffn, j);
        act[j] = g / (1.0f + expf(-g)) * u;
    }
}

// attention_step's projections after the matvecs (src/kvcache.cpp:84-100):
// column pairs of q, k, v; RoPE (rotate_vector, lines 48-59) on q and k with
// the host-built table; k and v stored at position *length.
__global__ void qkv_kernel(const float *pq, int qs, const float *pk, int ks, const float *pv,
                           int vs, DecodeShape s, const float2 *rope, const int *length,
                           float *query, float *k_layer, float *v_layer)
{
    const int kvd = s.kv_heads * s.head_dim;
    const int pairs = s.dim / 2 + kvd;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= pairs)
        return;
    const int pos = *length;
    int which, c;
    if (t < s.dim / 2) {
        which = 0;
        c = 2 * t;
    } else if (t < s.dim / 2 + kvd / 2) {
        which = 1;
        c = 2 * (t - s.dim / 2);
    } else {
        which = 2;
        c = 2 * (t - s.dim / 2 - kvd / 2);
    }
    const float *part = which == 0 ? pq : which == 1 ? pk : pv;
    const int splits = which == 0 ? qs : which == 1 ? ks : vs;
    const int out = which == 0 ? s.dim : kvd;
    float e = sum_parts(part, splits, out, c), o = sum_parts(part, splits, out, c + 1);
    const int head = c / s.head_dim, d = c % s.head_dim;
    if (which < 2) {
        const float2 cs = rope[size_t(pos) * (s.head_dim / 2) + d / 2];
        const float even = e, odd = o;
        e = fmaf(even, cs.x, -(odd * cs.y));
        o = fmaf(even, cs.y, odd * cs.x);
    }
    if (which == 0) {
        query[c] = e;
        query[c + 1] = o;
    } else {
        float *cache = (which == 1 ? k_layer : v_layer) +
                       (size_t(head) * s.max_seq + pos) * s.head_dim + d;
        cache[0] = e;
        cache[1] = o;
    }
}

__global__ void copy_kernel(const float *src, float *dst, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        dst[i] = src[i];
}

int blocks(int n) { return (n + 255) / 256; }

// partial <- the GEMV of x (rmsnorm'd with norm_w when given) by w
// [in x out]; returns the number of partial rows (splits).
int colgemv(const float *x, int in, const float *norm_w, const float *w, int out,
            float *partial, hipStream_t stream)
{
    const int col_blocks = (out + kCols - 1) / kCols;
    int splits = std::max(1, std::min((1024 + col_blocks - 1) / col_blocks, (in + 31) / 32));
    splits = std::max(1, std::min<int>(splits, int(kPartialFloats / size_t(out))));
    const int run = (in + splits - 1) / splits;
    splits = (in + run - 1) / run;
    const size_t lds = size_t(run) * sizeof(float);
    if (norm_w != nullptr)
        hipLaunchKernelGGL(colgemv_kernel<true>, dim3(col_blocks, splits), dim3(kCols), lds,
                           stream, x, in, norm_w, w, out, run, partial);
    else
        hipLaunchKernelGGL(colgemv_kernel<false>, dim3(col_blocks, splits), dim3(kCols), lds,
                           stream, x, in, nullptr, w, out, run, partial);
    check_launch("fp32 decode: projection");
    return splits;
}

void check_fready(const nut_fmodel &m)
{
    require(m.globals_set, NUT_EINVAL, "kv cache: model weights not uploaded");
    for (const nut_fmodel::Layer &l : m.layers)
        require(l.set, NUT_EINVAL, "kv cache: layer count mismatch");
}

// One token through every layer at position *length (device), its hidden
// state left in m.hidden; the device length advances.
void enqueue_token(nut_fmodel &m, nut_kvcache &kv, int token)
{
    const DecodeShape &s = m.shape;
    const nut_config &c = m.config;
    const int kvd = s.kv_heads * s.head_dim;
    StepState *state = m.state.as<StepState>();
    float *h = m.hidden.as<float>(), *q = m.query.as<float>(), *ctx = m.context.as<float>(),
          *act = m.act.as<float>();
    float *p0 = m.partial.as<float>(), *p1 = p0 + kPartialFloats, *p2 = p1 + kPartialFloats;
    launch_reset_state(state, token, m.stream);
    launch_embed(s, m.embeddings.as<float>(), &state->token, state, h, m.stream);
    const size_t layer_elems = kv.layer_elements();
    for (size_t l = 0; l < c.layers; l++) {
        const nut_fmodel::Layer &L = m.layers[l];
        float *kc = kv.keys.as<float>() + l * layer_elems;
        float *vc = kv.values.as<float>() + l * layer_elems;
        const float *an = L.attention_norm.as<float>(), *fn = L.ffn_norm.as<float>();
        const int qs = colgemv(h, s.dim, an, L.w[0].as<float>(), s.dim, p0, m.stream);
        const int ks = colgemv(h, s.dim, an, L.w[1].as<float>(), kvd, p1, m.stream);
        const int vs = colgemv(h, s.dim, an, L.w[2].as<float>(), kvd, p2, m.stream);
        hipLaunchKernelGGL(qkv_kernel, dim3(blocks(s.dim / 2 + kvd)), dim3(256), 0, m.stream, p0,
                           qs, p1, ks, p2, vs, s, m.rope.as<float2>(),
                           kv.device_length.as<int>(), q, kc, vc);
        check_launch("fp32 decode: rope and cache store");
        launch_attention(s, q, kc, vc, kv.device_length.as<int>(), ctx, state, m.stream);
        const int os = colgemv(ctx, s.dim, nullptr, L.w[3].as<float>(), s.dim, p0, m.stream);
        hipLaunchKernelGGL(residual_kernel, dim3(blocks(s.dim)), dim3(256), 0, m.stream, p0, os,
                           s.dim, h);
        const int gs = colgemv(h, s.dim, fn, L.w[4].as<float>(), s.ffn_dim, p1, m.stream);
        const int us = colgemv(h, s.dim, fn, L.w[5].as<float>(), s.ffn_dim, p2, m.stream);
        hipLaunchKernelGGL(swiglu_kernel, dim3(blocks(s.ffn_dim)), dim3(256), 0, m.stream, p1, gs,
                           p2, us, s.ffn_dim, act);
        const int ds = colgemv(act, s.ffn_dim, nullptr, L.w[6].as<float>(), s.dim, p0, m.stream);
        hipLaunchKernelGGL(residual_kernel, dim3(blocks(s.dim)), dim3(256), 0, m.stream, p0, ds,
                           s.dim, h);
        check_launch("fp32 decode: epilogue");
    }
    launch_finish_step(state, kv.device_length.as<int>(), m.stream);
}

void check_cache(const nut_fmodel &m, const nut_kvcache &kv)
{
    require(config_valid(m.config), NUT_EINVAL, "model config: invalid dimensions");
    require(kv_compatible(kv, m.config), NUT_EINVAL, "kv cache: model configuration mismatch");
    check_fready(m);
}

void upload_to(DeviceBuffer &b, const float *src, size_t count)
{
    b.allocate(count * sizeof(float));
    hip_check(hipMemcpy(b.get(), src, count * sizeof(float), hipMemcpyHostToDevice),
              "hipMemcpy to device");
}

} // namespace

nut_fmodel *create_fmodel(const nut_config &config, bool tied)
{
    require(config_valid(config), NUT_EINVAL, "model config: invalid dimensions");
    require(config.head_dim % 4 == 0 && config.dim <= 65536 && config.ffn_dim <= 65536 &&
                config.max_seq <= 15000 && config.vocab_size <= 0x7fffffff,
            NUT_EINVAL, "fp32 model: shape exceeds device kernel limits");
    ensure_device();
    std::unique_ptr<nut_fmodel> m(new nut_fmodel());
    m->config = config;
    m->tied = tied;
    DecodeShape &s = m->shape;
    s.dim = int(config.dim);
    s.heads = int(config.heads);
    s.kv_heads = int(config.kv_heads == 0 ? config.heads : config.kv_heads);
    s.head_dim = int(config.head_dim);
    s.ffn_dim = int(config.ffn_dim);
    s.vocab = int(config.vocab_size);
    s.max_seq = int(config.max_seq);
    s.eos = int(config.eos_token);
    s.attn_scale = 1.0f / std::sqrt(float(config.head_dim));
    m->layers.resize(config.layers);
    const std::vector<float> rope = rope_table(config);
    upload_to(m->rope, rope.data(), rope.size());
    m->hidden.allocate(config.dim * sizeof(float));
    m->query.allocate(config.dim * sizeof(float));
    m->context.allocate(config.dim * sizeof(float));
    m->act.allocate(config.ffn_dim * sizeof(float));
    m->partial.allocate(3 * kPartialFloats * sizeof(float));
    m->state.allocate(sizeof(StepState));
    m->token.allocate(sizeof(int));
    hip_check(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate");
    return m.release();
}

void set_fglobals(nut_fmodel &m, const float *embeddings, const float *final_norm,
                  const float *lm_head)
{
    require(embeddings != nullptr && final_norm != nullptr && (m.tied || lm_head != nullptr),
            NUT_EINVAL, "fp32 model: null weights");
    const size_t n = m.config.vocab_size * m.config.dim;
    upload_to(m.embeddings, embeddings, n);
    upload_to(m.final_norm, final_norm, m.config.dim);
    if (!m.tied)
        upload_to(m.lm_head, lm_head, n);
    m.globals_set = true;
}

void set_flayer(nut_fmodel &m, size_t layer, const float *const w[7],
                const float *attention_norm, const float *ffn_norm)
{
    const nut_config &c = m.config;
    require(layer < c.layers, NUT_EOUTOFRANGE, "fp32 model: layer out of range");
    require(attention_norm != nullptr && ffn_norm != nullptr, NUT_EINVAL,
            "fp32 model: null norm weights");
    const size_t kvd = (c.kv_heads == 0 ? c.heads : c.kv_heads) * c.head_dim;
    const size_t sizes[7] = {c.dim * c.dim,     c.dim * kvd,       c.dim * kvd, c.dim * c.dim,
                             c.dim * c.ffn_dim, c.dim * c.ffn_dim, c.ffn_dim * c.dim};
    nut_fmodel::Layer &L = m.layers[layer];
    for (int i = 0; i < 7; i++) {
        require(w[i] != nullptr, NUT_EINVAL, "fp32 model: null projection");
        upload_to(L.w[i], w[i], sizes[i]);
    }
    upload_to(L.attention_norm, attention_norm, c.dim);
    upload_to(L.ffn_norm, ffn_norm, c.dim);
    L.set = true;
}

void decode_token(nut_fmodel &m, nut_kvcache &kv, int token, float *hidden)
{
    check_cache(m, kv);
    require(kv.length < m.config.max_seq, NUT_ELENGTH, "kv cache: context is full");
    require(token >= 0 && size_t(token) < m.config.vocab_size, NUT_EOUTOFRANGE,
            "kv cache: token id out of range");
    kv.sync_length(m.stream);
    enqueue_token(m, kv, token);
    if (hidden != nullptr)
        hip_check(hipMemcpyAsync(hidden, m.hidden.get(), m.config.dim * sizeof(float),
                                 hipMemcpyDeviceToHost, m.stream),
                  "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    kv.length += 1;
}

void prefill_tokens(nut_fmodel &m, nut_kvcache &kv, const int *tokens, size_t count,
                    float *rows)
{
    check_cache(m, kv);
    require(tokens != nullptr && count != 0 && count <= m.config.max_seq, NUT_EINVAL,
            "kv cache: invalid prefill length");
    kv.length = 0;
    // the reference embeds every token before the first layer, so a bad id
    // fails with nothing computed (src/kvcache.cpp:247-250)
    for (size_t t = 0; t < count; t++)
        require(tokens[t] >= 0 && size_t(tokens[t]) < m.config.vocab_size, NUT_EOUTOFRANGE,
                "kv cache: token id out of range");
    DeviceBuffer out(count * m.config.dim * sizeof(float));
    launch_set_int(kv.device_length.as<int>(), 0, m.stream);
    for (size_t t = 0; t < count; t++) {
        enqueue_token(m, kv, tokens[t]);
        hipLaunchKernelGGL(copy_kernel, dim3(blocks(m.shape.dim)), dim3(256), 0, m.stream,
                           m.hidden.as<float>(), out.as<float>() + t * m.config.dim, m.shape.dim);
    }
    if (rows != nullptr)
        hip_check(hipMemcpyAsync(rows, out.get(), count * m.config.dim * sizeof(float),
                                 hipMemcpyDeviceToHost, m.stream),
                  "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    kv.length = count;
}

} // namespace nut

nut_fmodel::~nut_fmodel()
{
    if (stream != nullptr)
        (void)hipStreamDestroy(stream);
}
