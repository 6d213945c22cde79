// model.cpp — upload of QuantizedModelWeights to HBM, the device KV cache
// and the host side of the token loop (decode, prefill, logits, greedy
// generation). Validation and messages follow the reference's exceptions
// (src/quant_model.cpp:161-172,212-213; src/generate.cpp:177-181).
#include "model.hpp"
#include "noalloc.hpp"
#include "persistent.hpp"
#include "prefill.hpp"
#include "sample.hpp"
#include "host/nucleus.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <random>
#include <string>

namespace nut {

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

size_t kv_heads_of(const nut_config &c)
{
    return c.kv_heads == 0 ? c.heads : c.kv_heads;
}

DecodeShape shape_of(const nut_config &c)
{
    DecodeShape s{};
    s.dim = int(c.dim);
    s.heads = int(c.heads);
    s.kv_heads = int(kv_heads_of(c));
    s.head_dim = int(c.head_dim);
    s.ffn_dim = int(c.ffn_dim);
    s.vocab = int(c.vocab_size);
    s.max_seq = int(c.max_seq);
    s.eos = int(c.eos_token);
    s.attn_scale = 1.0f / std::sqrt(float(c.head_dim));
    return s;
}

void upload(void *dst, const void *src, size_t bytes);

} // namespace

// cos/sin of rotate_vector (src/quant_model.cpp:26-37), computed exactly as
// the reference does: double frequency 10000^(-pair/hd), double angle,
// rounded to fp32. Entry [pos][pair/2] = (cos, sin).
std::vector<float> rope_table(const nut_config &c)
{
    const size_t half = c.head_dim / 2;
    std::vector<float> table(c.max_seq * half * 2);
    for (size_t pos = 0; pos < c.max_seq; pos++)
        for (size_t i = 0; i < half; i++) {
            const double frequency =
                std::pow(10000.0, -double(2 * i) / double(c.head_dim));
            const double angle = double(pos) * frequency;
            table[(pos * half + i) * 2] = float(std::cos(angle));
            table[(pos * half + i) * 2 + 1] = float(std::sin(angle));
        }
    return table;
}

namespace {

void upload(void *dst, const void *src, size_t bytes)
{
    hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice),
              "hipMemcpy to device");
}

void check_ready(const nut_model &m, const char *who)
{
    if (!m.globals_set)
        fail(NUT_EINVAL, std::string(who) + ": model weights not uploaded");
    for (const DeviceLayer &l : m.layers)
        if (!l.set)
            fail(NUT_EINVAL, std::string(who) + ": layer count mismatch");
}

// True when every layer can run the fast step kernels.
bool fast_steps(const nut_model &m)
{
    for (const DeviceLayer &l : m.layers)
        if (!step_fast_supported(m.shape, l.view))
            return false;
    return true;
}

// The captured iteration names the model's buffers; weight uploads drop it.
void drop_graph(nut_model &m)
{
    if (m.step_graph != nullptr) {
        hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
        (void)hipGraphExecDestroy(m.step_graph);
        m.step_graph = nullptr;
    }
}

// Workspace of the fast step kernels (allocated before any capture).
void prepare_fast_steps(nut_model &m)
{
    if (m.attn_count.get() == nullptr) {
        const size_t part = step_attn_part_words(m.shape) * sizeof(uint64_t);
        const size_t count = 2 * size_t(m.shape.heads) * kStepTokensMax * sizeof(int);
        m.attn_part.allocate(part);
        m.attn_count.allocate(count);
        hip_check(hipMemsetAsync(m.attn_part.get(), 0xff, part, m.stream), "hipMemsetAsync");
        hip_check(hipMemsetAsync(m.attn_count.get(), 0, count, m.stream), "hipMemsetAsync");
    }
}

// Enqueue one decode step reading its token from token_ptr (device).
void enqueue_step(nut_model &m, nut_kvcache &kv, const int *token_ptr)
{
    const DecodeShape &s = m.shape;
    StepState *state = m.state.as<StepState>();
    launch_embed(s, m.embeddings.as<float>(), token_ptr, state,
                 m.hidden.as<float>(), m.stream);
    const size_t layer_elems = kv.layer_elements();
    if (fast_steps(m)) {
        prepare_fast_steps(m);
        const StepBuffers b{m.hidden.as<float>(), m.query.as<float>(),
                            m.context.as<float>(), m.act.as<float>(),
                            m.attn_part.as<uint64_t>(), m.attn_count.as<int>()};
        for (size_t l = 0; l < m.layers.size(); l++)
            launch_layer_fast(s, m.layers[l].view, m.rope.as<float2>(),
                              kv.device_length.as<int>(),
                              kv.keys.as<float>() + l * layer_elems,
                              kv.values.as<float>() + l * layer_elems, b, 1, state,
                              m.stream);
        launch_finish_step(state, kv.device_length.as<int>(), m.stream);
        return;
    }
    for (size_t l = 0; l < m.layers.size(); l++)
        launch_layer(s, m.layers[l].view, m.rope.as<float2>(),
                     kv.device_length.as<int>(),
                     kv.keys.as<float>() + l * layer_elems,
                     kv.values.as<float>() + l * layer_elems,
                     m.hidden.as<float>(), m.query.as<float>(),
                     m.context.as<float>(), m.act.as<float>(), state,
                     m.stream);
    launch_finish_step(state, kv.device_length.as<int>(), m.stream);
}

void sync(nut_model &m) { hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize"); }

// Tokens [0, count) (device ids in m.prompt) through the step kernels in
// chunks of up to kStepTokensMax consecutive tokens per launch: every
// weight row is streamed once per chunk instead of once per token, and the
// arithmetic of each token is the decode step's. The last token's hidden
// state lands in m.hidden; kv.device_length ends at count.
void prefill_steps(nut_model &m, nut_kvcache &kv, size_t count)
{
    const DecodeShape &s = m.shape;
    prepare_fast_steps(m);
    if (m.mt_hidden.get() == nullptr) {
        m.mt_hidden.allocate(size_t(kStepTokensMax) * s.dim * sizeof(float));
        m.mt_query.allocate(size_t(kStepTokensMax) * s.dim * sizeof(float));
        m.mt_context.allocate(size_t(kStepTokensMax) * s.dim * sizeof(float));
        m.mt_act.allocate(size_t(kStepTokensMax) * s.ffn_dim * sizeof(float));
    }
    StepState *state = m.state.as<StepState>();
    launch_reset_state(state, 0, m.stream);
    const StepBuffers b{m.mt_hidden.as<float>(), m.mt_query.as<float>(),
                        m.mt_context.as<float>(), m.mt_act.as<float>(),
                        m.attn_part.as<uint64_t>(), m.attn_count.as<int>()};
    const size_t layer_elems = kv.layer_elements();
    size_t t = 0;
    for (size_t start = 0; start < count; start += t) {
        t = std::min<size_t>(kStepTokensMax, count - start);
        launch_set_int(kv.device_length.as<int>(), int(start), m.stream);
        launch_embed_rows(m.embeddings.as<float>(), m.prompt.as<int>() + start,
                          m.mt_hidden.as<float>(), int(t), s.dim, m.stream);
        for (size_t l = 0; l < m.layers.size(); l++)
            launch_layer_fast(s, m.layers[l].view, m.rope.as<float2>(),
                              kv.device_length.as<int>(),
                              kv.keys.as<float>() + l * layer_elems,
                              kv.values.as<float>() + l * layer_elems, b, int(t), state,
                              m.stream);
    }
    hip_check(hipMemcpyAsync(m.hidden.get(), m.mt_hidden.as<float>() + (t - 1) * s.dim,
                             s.dim * sizeof(float), hipMemcpyDeviceToDevice, m.stream),
              "hipMemcpyAsync");
}

// Prompts of at least this many tokens run as a batch (GEMM prefill);
// shorter ones run as one step-kernel chunk (kStepTokensMax = 31). A chunk
// costs its row dots once per token, the batch one 64-token MFMA tile, so
// the crossover depends on the width. TinyLlama INT4 (dim 2048), batch
// against one chunk: 24 tokens 3.11 against 2.64 ms, 28 tokens 3.12
// against 2.94, 31 tokens 3.12 against 3.16. Llama-2-7B shape INT4 (dim
// 4096): one chunk 4.78 ms at 8 tokens, 8.35 at 16, 13.9 at 29; the batch
// 7.9 ms at 31.
size_t prefill_gemm_min(const DecodeShape &s)
{
    return s.dim >= 4096 ? 16 : 30;
}

// The batched prefill applies when every layer uses 32-wide blocks, the
// head size matches its attention tiles, and per-token steps are not
// forced.
bool use_prefill_gemm(const nut_model &m, size_t count)
{
    if (m.path == 1 || count < prefill_gemm_min(m.shape))
        return false;
    for (const DeviceLayer &l : m.layers)
        if (!prefill_gemm_supported(m.shape, l.view) || l.stage_scale[0] == nullptr)
            return false;
    return true;
}

// Tokens [0, count) (device ids in m.prompt) through every layer as a batch
// at positions 0 .. count - 1; K/V rows land in the cache and the last
// token's hidden state in m.hidden.
void prefill_batch(nut_model &m, nut_kvcache &kv, size_t count)
{
    const nut_config &c = m.config;
    const DecodeShape &s = m.shape;
    if (m.pf_h.get() == nullptr) {
        const size_t rows = c.max_seq;
        m.pf_h.allocate(rows * c.dim * sizeof(float));
        m.pf_x.allocate(rows * c.dim * sizeof(float));
        m.pf_act.allocate(rows * c.ffn_dim * sizeof(float));
        m.pf_q.allocate(rows * c.dim * sizeof(float));
        m.pf_ctx.allocate(rows * c.dim * sizeof(float));
        m.pf_kv.allocate(4 * prefill_kv_limb_elems(s) * sizeof(_Float16));
    }
    const int t = int(count);
    // GEMM inputs as f16 limbs (hi rows, then lo rows): the normalised x in
    // pf_x, the attention context in pf_ctx, the SwiGLU activations in pf_act
    float *h = m.pf_h.as<float>();
    _Float16 *xh = m.pf_x.as<_Float16>(), *ch = m.pf_ctx.as<_Float16>();
    _Float16 *act_h = m.pf_act.as<_Float16>();
    float *q = m.pf_q.as<float>();
    launch_embed_rows(m.embeddings.as<float>(), m.prompt.as<int>(), h, t, s.dim,
                      m.stream);
    const size_t layer_elems = kv.layer_elements();
    for (size_t l = 0; l < m.layers.size(); l++) {
        const LayerView &w = m.layers[l].view;
        const uint32_t *const *ss = m.layers[l].stage_scale;
        float *kc = kv.keys.as<float>() + l * layer_elems;
        float *vc = kv.values.as<float>() + l * layer_elems;
        const QMat *qkv_w[3] = {&w.query, &w.key, &w.value};
        const QMat *wo = &w.output, *wd = &w.down;
        launch_rmsnorm_rows(h, w.attention_norm, xh, xh + size_t(t) * s.dim, t, s.dim,
                            m.stream);
        // Q/K/V products, RoPE, the cache rows and the attention's K/V limbs
        // in one launch
        launch_qgemm_qkv(xh, xh + size_t(t) * s.dim, t, qkv_w, ss, q, m.rope.as<float2>(), kc,
                         vc, m.pf_kv.as<_Float16>(), s, m.stream);
        launch_attention_prefill(q, m.pf_kv.as<_Float16>(), ch, ch + size_t(t) * s.dim, s, t,
                                 m.stream);
        launch_qgemm_rows(ch, ch + size_t(t) * s.dim, t, &wo, ss + 3, &h, &s.dim, 1, true,
                          m.stream);
        launch_rmsnorm_rows(h, w.ffn_norm, xh, xh + size_t(t) * s.dim, t, s.dim, m.stream);
        // gate/up products and SwiGLU in one launch
        launch_qgemm_swiglu(xh, xh + size_t(t) * s.dim, t, w.gate, w.up, ss[4], ss[5],
                            act_h, act_h + size_t(t) * s.ffn_dim, m.stream);
        launch_qgemm_rows(act_h, act_h + size_t(t) * s.ffn_dim, t, &wd, ss + 6, &h, &s.dim, 1,
                          true, m.stream);
    }
    hip_check(hipMemcpyAsync(m.hidden.get(), h + size_t(t - 1) * s.dim,
                             s.dim * sizeof(float), hipMemcpyDeviceToDevice,
                             m.stream),
              "hipMemcpyAsync");
}

double now() { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); }

} // namespace

bool config_valid(const nut_config &c)
{
    const size_t kv = kv_heads_of(c);
    return c.layers != 0 && c.heads != 0 && c.dim != 0 && c.head_dim != 0 &&
           c.ffn_dim != 0 && c.vocab_size != 0 && c.max_seq != 0 &&
           c.heads <= SIZE_MAX / c.head_dim && c.heads * c.head_dim == c.dim &&
           c.head_dim % 2 == 0 && c.eos_token < c.vocab_size && kv != 0 &&
           kv <= c.heads && c.heads % kv == 0;
}

nut_model *create_model(const nut_config &config, int type, bool tied)
{
    require(config_valid(config), NUT_EINVAL, "model config: invalid dimensions");
    require(type == NUT_INT8 || type == NUT_INT4, NUT_EINVAL,
            "quantized model: unknown quant type");
    // Device-path limits: float4 head rows, LDS staging of x and scores.
    require(config.head_dim % 4 == 0 && config.head_dim <= 256 &&
                config.dim <= 15000 && config.ffn_dim <= 15000 &&
                config.max_seq <= 15000 && config.vocab_size <= 0x7fffffff,
            NUT_EINVAL, "quantized model: shape exceeds device kernel limits");
    ensure_device();
    std::unique_ptr<nut_model> m(new nut_model());
    m->config = config;
    m->type = type;
    m->tied = tied;
    m->shape = shape_of(config);
    m->layout = layer_layout(type, config.dim, config.ffn_dim,
                             kv_heads_of(config) * config.head_dim);
    m->layers.resize(config.layers);
    const size_t dim = config.dim, vocab = config.vocab_size;
    m->embeddings.allocate(vocab * dim * sizeof(float));
    m->final_norm.allocate(dim * sizeof(float));
    if (!tied)
        m->lm_head.allocate(vocab * dim * sizeof(float));
    const std::vector<float> rope = rope_table(config);
    m->rope.allocate(rope.size() * sizeof(float));
    upload(m->rope.get(), rope.data(), rope.size() * sizeof(float));
    m->hidden.allocate(dim * sizeof(float));
    m->scratch_hidden.allocate(dim * sizeof(float));
    m->query.allocate(dim * sizeof(float));
    m->context.allocate(dim * sizeof(float));
    m->act.allocate(config.ffn_dim * sizeof(float));
    m->logits.allocate(vocab * sizeof(float));
    m->part_val.allocate(1024 * sizeof(float));
    m->part_idx.allocate(1024 * sizeof(int));
    m->state.allocate(sizeof(StepState));
    m->tokens.allocate((config.max_seq + 1) * sizeof(int));
    m->prompt.allocate((config.max_seq + 1) * sizeof(int));
    hip_check(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking),
              "hipStreamCreate");
    hip_check(hipEventCreate(&m->decode_begin), "hipEventCreate");
    hip_check(hipEventCreate(&m->decode_end), "hipEventCreate");
    return m.release();
}

void set_globals(nut_model &m, const float *embeddings,
                 const float *final_norm, const float *lm_head)
{
    drop_graph(m);
    const size_t dim = m.config.dim, vocab = m.config.vocab_size;
    require(embeddings != nullptr && final_norm != nullptr &&
                (m.tied || lm_head != nullptr),
            NUT_EINVAL, "quantized model: null weights");
    upload(m.embeddings.get(), embeddings, vocab * dim * sizeof(float));
    upload(m.final_norm.get(), final_norm, dim * sizeof(float));
    if (!m.tied)
        upload(m.lm_head.get(), lm_head, vocab * dim * sizeof(float));
    m.globals_set = true;
    m.screen_ready = false;
}

void set_layer(nut_model &m, size_t layer, const nut_qmatrix *const mats[7],
               const float *attention_norm, const float *ffn_norm)
{
    drop_graph(m);
    const nut_config &c = m.config;
    require(layer < c.layers, NUT_EOUTOFRANGE, "quantized model: layer out of range");
    require(attention_norm != nullptr && ffn_norm != nullptr, NUT_EINVAL,
            "quantized model: null norm weights");
    const size_t kvd = kv_heads_of(c) * c.head_dim;
    const size_t shapes[7][2] = {{c.dim, c.dim},     {kvd, c.dim},
                                 {kvd, c.dim},       {c.dim, c.dim},
                                 {c.ffn_dim, c.dim}, {c.ffn_dim, c.dim},
                                 {c.dim, c.ffn_dim}};
    size_t offsets[7][2];
    size_t total = 0, accounted = 0;
    bool blocks32 = true;
    for (int i = 0; i < 7; i++) {
        const nut_qmatrix *q = mats[i];
        require(q != nullptr && q->data != nullptr && q->scales != nullptr,
                NUT_EINVAL, "quantized model: null projection");
        require(q->rows == shapes[i][0] && q->cols == shapes[i][1],
                NUT_EINVAL, "quantized model: projection shape mismatch");
        require(q->type == m.type, NUT_EINVAL, "quantized model: quant type mismatch");
        require(q->block_size != 0, NUT_EINVAL, "quantize: zero block size");
        const size_t data = nut_quant_data_bytes(q->rows, q->cols, q->type);
        const size_t scales = 2 * nut_quant_scale_count(q->rows, q->cols, q->block_size);
        offsets[i][0] = total;
        total = align_up(total + data);
        offsets[i][1] = total;
        total = align_up(total + scales);
        accounted += data + scales;
        blocks32 = blocks32 && q->block_size == 32;
    }
    size_t norms = total;
    total += 2 * c.dim * sizeof(float);
    DeviceLayer &dl = m.layers[layer];
    dl.storage.release();
    uint8_t *base;
    if (blocks32) {
        // Same offsets as layer_layout (checked), inside the arena.
        const LayerLayout &lay = m.layout;
        for (int i = 0; i < 7; i++)
            require(offsets[i][0] == lay.data[i] && offsets[i][1] == lay.scales[i],
                    NUT_EINVAL, "quantized model: arena layout mismatch");
        require(norms == lay.attention_norm, NUT_EINVAL,
                "quantized model: arena layout mismatch");
        if (m.arena.get() == nullptr)
            m.arena.allocate(lay.bytes * c.layers);
        base = m.arena.as<uint8_t>() + layer * lay.bytes;
    } else {
        dl.storage.allocate(total);
        base = dl.storage.as<uint8_t>();
    }
    dl.in_arena = blocks32;
    QMat views[7];
    for (int i = 0; i < 7; i++) {
        const nut_qmatrix *q = mats[i];
        upload(base + offsets[i][0], q->data, nut_quant_data_bytes(q->rows, q->cols, q->type));
        upload(base + offsets[i][1], q->scales,
               2 * nut_quant_scale_count(q->rows, q->cols, q->block_size));
        views[i] = QMat{base + offsets[i][0],
                        reinterpret_cast<const uint16_t *>(base + offsets[i][1]),
                        int(q->rows), int(q->cols), int(q->block_size), q->type};
    }
    float *norm_base = reinterpret_cast<float *>(base + norms);
    upload(norm_base, attention_norm, c.dim * sizeof(float));
    upload(norm_base + c.dim, ffn_norm, c.dim * sizeof(float));
    dl.view = LayerView{views[0], views[1], views[2], views[3], views[4],
                        views[5], views[6], norm_base, norm_base + c.dim};
    dl.stage_scales.release();
    for (int i = 0; i < 7; i++)
        dl.stage_scale[i] = nullptr;
    bool stages = true;
    size_t words = 0;
    for (int i = 0; i < 7; i++) {
        stages = stages && views[i].block_size == 32 && views[i].cols % 64 == 0;
        words += stages ? stage_scale_words(views[i]) : 0;
    }
    if (stages) {
        dl.stage_scales.allocate(words * sizeof(uint32_t));
        uint32_t *at = dl.stage_scales.as<uint32_t>();
        for (int i = 0; i < 7; i++) {
            launch_scales_by_stage(views[i], at, m.stream);
            dl.stage_scale[i] = at;
            at += stage_scale_words(views[i]);
        }
    }
    dl.storage_bytes = accounted + 2 * c.dim * sizeof(float);
    dl.set = true;
}

size_t storage_bytes(const nut_model &m)
{
    // QuantizedModelWeights::storage_bytes (src/quant_model.cpp:140-156).
    const size_t dim = m.config.dim, vocab = m.config.vocab_size;
    size_t total = vocab * dim * 4 + dim * 4 + (m.tied ? 0 : vocab * dim * 4);
    for (const DeviceLayer &l : m.layers)
        total += l.storage_bytes;
    return total;
}

nut_kvcache *create_kv(const nut_config &config)
{
    require(config_valid(config), NUT_EINVAL, "model config: invalid dimensions");
    ensure_device();
    std::unique_ptr<nut_kvcache> kv(new nut_kvcache());
    kv->config = config;
    const size_t bytes = config.layers * kv->layer_elements() * sizeof(float);
    kv->keys.allocate(bytes);
    kv->values.allocate(bytes);
    hip_check(hipMemset(kv->keys.get(), 0, bytes), "hipMemset");
    hip_check(hipMemset(kv->values.get(), 0, bytes), "hipMemset");
    kv->device_length.allocate(sizeof(int));
    hip_check(hipMemset(kv->device_length.get(), 0, sizeof(int)), "hipMemset");
    return kv.release();
}

bool kv_compatible(const nut_kvcache &kv, const nut_config &c)
{
    // KVCache::compatible (src/kvcache.cpp:187-195).
    const nut_config &k = kv.config;
    return k.layers == c.layers && k.heads == c.heads && k.dim == c.dim &&
           k.head_dim == c.head_dim && k.ffn_dim == c.ffn_dim &&
           k.vocab_size == c.vocab_size && k.max_seq == c.max_seq &&
           k.eos_token == c.eos_token && kv_heads_of(k) == kv_heads_of(c);
}

} // namespace nut

void nut_kvcache::sync_length(hipStream_t stream)
{
    nut::launch_set_int(device_length.as<int>(), int(length), stream);
}

nut_model::~nut_model()
{
    if (step_graph != nullptr)
        (void)hipGraphExecDestroy(step_graph);
    if (decode_begin != nullptr)
        (void)hipEventDestroy(decode_begin);
    if (decode_end != nullptr)
        (void)hipEventDestroy(decode_end);
    if (stream != nullptr)
        (void)hipStreamDestroy(stream);
}

namespace nut {

namespace {

// The cooperative token kernel runs when the model shape has an
// instantiation, the device can hold its grid, and every position of the
// launch fits the fused attention pass or, beyond it, the split one.
bool use_token_kernel(nut_model &m, size_t end_length)
{
    if (m.path == 1)
        return false;
    bool arena = true;
    for (const DeviceLayer &l : m.layers)
        arena = arena && l.in_arena;
    const bool ok = arena && token_kernel_supported(m.type, m.shape) &&
                    end_length <= size_t(token_kernel_long_positions(m.type, m.shape));
    if (m.path == 2 && !ok)
        fail(NUT_EINVAL, "token kernel: shape or context not supported");
    return ok;
}

// The classifier's INT8 screening copy (launch_classifier_screen) for the
// generate loop, when the vocabulary's share per workgroup fits the
// kernel's bound array; null otherwise.
void prepare_screen(nut_model &m, const uint8_t *&codes, const uint16_t *&scales)
{
    codes = nullptr;
    scales = nullptr;
    const int vocab = m.shape.vocab, dim = m.shape.dim;
    if ((vocab + kTokenGrid - 1) / kTokenGrid > kScreenRowsMax || dim % 32 != 0)
        return;
    if (!m.screen_ready) {
        if (m.classifier8.get() == nullptr) {
            m.classifier8.allocate(size_t(vocab) * dim);
            m.classifier8_scales.allocate(size_t(vocab) * (dim / 32) * sizeof(uint16_t));
        }
        launch_classifier_screen(m.output_weights(), vocab, dim, m.classifier8.as<int8_t>(),
                                 m.classifier8_scales.as<uint16_t>(), m.stream);
        m.screen_ready = true;
    }
    codes = m.classifier8.as<uint8_t>();
    scales = m.classifier8_scales.as<uint16_t>();
}

void prepare_token_kernel(nut_model &m)
{
    if (m.exchange.get() == nullptr) {
        const size_t entries = token_exchange_entries(m.shape);
        m.exchange.allocate(entries * sizeof(uint64_t));
        hip_check(hipMemset(m.exchange.get(), 0, entries * sizeof(uint64_t)), "hipMemset");
        m.token_error.allocate(sizeof(int));
    }
}

// Enqueue one launch; iteration it decodes position start + it.
void run_token_kernel(nut_model &m, nut_kvcache &kv, size_t start, size_t n_iter,
                      bool classify, const int *tokens_in, const float *hidden_in,
                      float *hidden_out)
{
    prepare_token_kernel(m);
    const DecodeShape &s = m.shape;
    const size_t kvd = size_t(s.kv_heads) * s.head_dim;
    uint64_t *x = m.exchange.as<uint64_t>();
    TokenArgs a{};
    a.weights = m.arena.as<uint8_t>();
    a.embeddings = m.embeddings.as<float>();
    a.final_norm = m.final_norm.as<float>();
    a.classifier = m.output_weights();
    if (classify)
        prepare_screen(m, a.classifier8, a.classifier8_scales);
    a.rope = m.rope.as<float2>();
    a.k_cache = kv.keys.as<float>();
    a.v_cache = kv.values.as<float>();
    a.x_qkv = x;
    a.x_hidden = x + s.dim + 2 * kvd;
    a.x_act = a.x_hidden + s.dim;
    a.x_part = a.x_act + s.ffn_dim;
    a.x_apart = a.x_part + 2 * kTokenGrid;
    a.x_ctx = a.x_apart + size_t(kTokenGrid) * (s.heads / s.kv_heads) * (s.head_dim + 2);
    a.x_scores = wide_kernel_score_entries(s) > 0 ? a.x_ctx + s.dim : nullptr;
    // beyond the fused attention pass, attention is split over the grid
    a.long_attention =
        start + n_iter > size_t(token_kernel_max_positions(m.type, s)) ? 1 : 0;
    {
        // every word of the write-once ring unset (0xffffffff) when the
        // launch starts; the ring's size does not depend on n_iter
        const bool wide = wide_kernel_positions(m.type, s) > 0;
        const size_t floats = token_once_floats(s, wide);
        if (floats * sizeof(float) > m.exchange_once.bytes()) {
            m.exchange_once.release();
            m.exchange_once.allocate(floats * sizeof(float));
        }
        hip_check(hipMemsetAsync(m.exchange_once.get(), 0xff, floats * sizeof(float), m.stream),
                  "hipMemsetAsync");
        a.x_once = m.exchange_once.as<float>();
    }
    a.hidden_in = hidden_in;
    a.hidden_out = hidden_out;
    a.tokens_in = tokens_in;
    a.tokens_out = m.tokens.as<int>();
    a.state = m.state.as<StepState>();
    a.error = m.token_error.as<int>();
    bool clear = false;
    a.tag_base = next_tag_base(m.launch_count, clear);
    if (clear)
        hip_check(hipMemsetAsync(m.exchange.get(), 0,
                                 token_exchange_entries(s) * sizeof(uint64_t), m.stream),
                  "hipMemsetAsync");
    a.fault = m.fault;
    a.layer_count = int(m.config.layers);
    a.vocab = s.vocab;
    a.max_seq = s.max_seq;
    a.eos = s.eos;
    a.start_len = int(start);
    a.n_iter = int(n_iter);
    a.classify = classify ? 1 : 0;
    a.attn_scale = s.attn_scale;
    a.timeline = m.timeline_entries > 0 ? m.timeline.as<unsigned long long>() : nullptr;
    a.timeline_wgs = m.timeline_wgs;
    a.timeline_cap = m.timeline_wgs > 0 ? int(m.timeline_entries / m.timeline_wgs) : 0;
    launch_set_int(a.error, 0, m.stream);
    launch_token_kernel(m.type, s, a, m.stream);
}

// After the stream synchronised: raise the kernel's bounded-wait failure,
// once (the flag is cleared, so later calls that run no token kernel do
// not report it again).
void check_token_error(nut_model &m)
{
    if (m.token_error.get() == nullptr)
        return;
    int error = 0;
    hip_check(hipMemcpy(&error, m.token_error.get(), sizeof error, hipMemcpyDeviceToHost),
              "hipMemcpy");
    if (error != 0) {
        const int zero = 0;
        hip_check(hipMemcpy(m.token_error.get(), &zero, sizeof zero, hipMemcpyHostToDevice),
                  "hipMemcpy");
        fail(NUT_EDEVICE, "token kernel: phase exchange timed out");
    }
}

} // namespace

void decode(nut_model &m, nut_kvcache &kv, int token, float *hidden)
{
    require(config_valid(m.config), NUT_EINVAL, "model config: invalid dimensions");
    require(kv_compatible(kv, m.config), NUT_EINVAL,
            "quantized decode: cache configuration mismatch");
    check_ready(m, "quantized decode");
    require(token >= 0 && size_t(token) < m.config.vocab_size, NUT_EOUTOFRANGE,
            "quantized decode: token out of range");
    require(kv.length < kv.config.max_seq, NUT_ELENGTH,
            "quantized decode: context is full");
    if (use_token_kernel(m, kv.length + 1)) {
        launch_set_int(m.prompt.as<int>(), token, m.stream);
        run_token_kernel(m, kv, kv.length, 1, false, m.prompt.as<int>(), nullptr,
                         m.hidden.as<float>());
    } else {
        kv.sync_length(m.stream);
        launch_reset_state(m.state.as<StepState>(), token, m.stream);
        enqueue_step(m, kv, &m.state.as<StepState>()->token);
    }
    if (hidden != nullptr)
        hip_check(hipMemcpyAsync(hidden, m.hidden.get(), m.config.dim * sizeof(float),
                                 hipMemcpyDeviceToHost, m.stream),
                  "hipMemcpyAsync");
    sync(m);
    check_token_error(m);
    kv.length += 1;
}

void decode_noalloc(nut_model &m, nut_kvcache &kv, int token, float *d_hidden)
{
    require(config_valid(m.config), NUT_EINVAL, "model config: invalid dimensions");
    require(kv_compatible(kv, m.config), NUT_EINVAL,
            "quantized decode: cache configuration mismatch");
    check_ready(m, "quantized decode");
    require(token >= 0 && size_t(token) < m.config.vocab_size, NUT_EOUTOFRANGE,
            "quantized decode: token out of range");
    require(kv.length < kv.config.max_seq, NUT_ELENGTH,
            "quantized decode: context is full");
    require(fast_steps(m), NUT_EINVAL,
            "no-alloc decode: needs 32-wide quant blocks along whole rows and head_dim "
            "64 or 128");
    const DecodeShape &s = m.shape;
    // one token's split-attention partials (0xff-filled: no word carries a
    // live tag) and arrival counters (zero), as a fresh model starts them
    const size_t part_words = step_attn_part_words(s) / kStepTokensMax;
    const size_t count_ints = 2 * size_t(s.heads);
    require(part_words * sizeof(uint64_t) + count_ints * sizeof(int) <= kNoAllocScratchBytes,
            NUT_EINVAL, "no-alloc decode: attention workspace exceeds the 2 MiB scratch");
    uint8_t *scratch = static_cast<uint8_t *>(noalloc_scratch());
    uint64_t *parts = reinterpret_cast<uint64_t *>(scratch);
    int *counts = reinterpret_cast<int *>(scratch + part_words * sizeof(uint64_t));
    launch_fill_words(reinterpret_cast<uint32_t *>(parts), 0xffffffffu, 2 * part_words,
                      m.stream);
    launch_fill_words(reinterpret_cast<uint32_t *>(counts), 0u, count_ints, m.stream);
    kv.sync_length(m.stream);
    StepState *state = m.state.as<StepState>();
    launch_reset_state(state, token, m.stream);
    launch_embed(s, m.embeddings.as<float>(), &state->token, state, m.hidden.as<float>(),
                 m.stream);
    const StepBuffers b{m.hidden.as<float>(), m.query.as<float>(), m.context.as<float>(),
                        m.act.as<float>(), parts, counts};
    const size_t layer_elems = kv.layer_elements();
    for (size_t l = 0; l < m.layers.size(); l++)
        launch_layer_fast(s, m.layers[l].view, m.rope.as<float2>(),
                          kv.device_length.as<int>(), kv.keys.as<float>() + l * layer_elems,
                          kv.values.as<float>() + l * layer_elems, b, 1, state, m.stream);
    launch_finish_step(state, kv.device_length.as<int>(), m.stream);
    if (d_hidden != nullptr)
        hip_check(hipMemcpyAsync(d_hidden, m.hidden.get(), m.config.dim * sizeof(float),
                                 hipMemcpyDeviceToDevice, m.stream),
                  "hipMemcpyAsync");
    sync(m);
    kv.length += 1;
}

void prefill(nut_model &m, nut_kvcache &kv, const int *tokens, size_t count,
             float *hidden)
{
    require(tokens != nullptr && count != 0 && count <= kv.config.max_seq,
            NUT_EINVAL, "quantized prefill: invalid prompt");
    require(config_valid(m.config), NUT_EINVAL, "model config: invalid dimensions");
    require(kv_compatible(kv, m.config), NUT_EINVAL,
            "quantized decode: cache configuration mismatch");
    check_ready(m, "quantized decode");
    kv.length = 0;
    // The reference decodes token by token, so a bad id fails only when it
    // is reached, with the valid prefix already in the cache.
    size_t valid = 0;
    while (valid < count && tokens[valid] >= 0 &&
           size_t(tokens[valid]) < m.config.vocab_size)
        valid++;
    if (valid > 0) {
        hip_check(hipMemcpyAsync(m.prompt.get(), tokens, valid * sizeof(int),
                                 hipMemcpyHostToDevice, m.stream),
                  "hipMemcpyAsync");
        if (use_prefill_gemm(m, valid)) {
            prefill_batch(m, kv, valid);
        } else if (m.path != 2 && valid > 1 && fast_steps(m)) {
            prefill_steps(m, kv, valid);
        } else if (use_token_kernel(m, valid)) {
            run_token_kernel(m, kv, 0, valid, false, m.prompt.as<int>(), nullptr,
                             m.hidden.as<float>());
        } else {
            kv.sync_length(m.stream);
            launch_reset_state(m.state.as<StepState>(), tokens[0], m.stream);
            for (size_t t = 0; t < valid; t++)
                enqueue_step(m, kv, m.prompt.as<int>() + t);
        }
        if (hidden != nullptr)
            hip_check(hipMemcpyAsync(hidden, m.hidden.get(), m.config.dim * sizeof(float),
                                     hipMemcpyDeviceToHost, m.stream),
                      "hipMemcpyAsync");
        kv.length = valid;
        // the step kernels read the length from the device; the batched and
        // token-kernel paths do not advance it themselves
        kv.sync_length(m.stream);
        sync(m);
        check_token_error(m);
    }
    require(valid == count, NUT_EOUTOFRANGE, "quantized decode: token out of range");
}

void logits(nut_model &m, const float *hidden, float *out)
{
    require(hidden != nullptr && out != nullptr, NUT_EINVAL, "logits: null pointer");
    check_ready(m, "logits");
    const size_t dim = m.config.dim;
    hip_check(hipMemcpyAsync(m.scratch_hidden.get(), hidden, dim * sizeof(float),
                             hipMemcpyHostToDevice, m.stream),
              "hipMemcpyAsync");
    launch_reset_state(m.state.as<StepState>(), 0, m.stream);
    launch_classifier(m.shape, m.scratch_hidden.as<float>(), m.final_norm.as<float>(),
                      m.output_weights(), m.logits.as<float>(), m.part_val.as<float>(),
                      m.part_idx.as<int>(), m.state.as<StepState>(), m.stream);
    hip_check(hipMemcpyAsync(out, m.logits.get(), m.config.vocab_size * sizeof(float),
                             hipMemcpyDeviceToHost, m.stream),
              "hipMemcpyAsync");
    sync(m);
}

void generate_greedy(nut_model &m, const int *prompt, size_t prompt_len,
                     size_t max_tokens, int *out, size_t *out_count,
                     nut_generation_stats *stats)
{
    require(config_valid(m.config), NUT_EINVAL, "model config: invalid dimensions");
    require(prompt != nullptr && prompt_len != 0 && prompt_len <= m.config.max_seq,
            NUT_EINVAL, "generation: invalid prompt length");
    require(out != nullptr || max_tokens == 0, NUT_EINVAL, "generation: null output");
    require(out_count != nullptr, NUT_EINVAL, "generation: null output");
    check_ready(m, "generation");
    if (!m.generation_cache)
        m.generation_cache.reset(create_kv(m.config));
    nut_kvcache &kv = *m.generation_cache;

    const double t0 = now();
    prefill(m, kv, prompt, prompt_len, nullptr);
    const double t1 = now();
    const size_t steps = std::min(max_tokens, m.config.max_seq - prompt_len);
    StepState *state = m.state.as<StepState>();
    launch_reset_state(state, 0, m.stream);
    const int parts = classifier_blocks(m.shape);
    const bool fused = steps > 0 && use_token_kernel(m, prompt_len + steps);
    hip_check(hipEventRecord(m.decode_begin, m.stream), "hipEventRecord");
    if (fused) {
        run_token_kernel(m, kv, prompt_len, steps, true, nullptr, m.hidden.as<float>(),
                         m.scratch_hidden.as<float>());
    } else {
        auto iteration = [&]() {
            launch_classifier(m.shape, m.hidden.as<float>(), m.final_norm.as<float>(),
                              m.output_weights(), nullptr, m.part_val.as<float>(),
                              m.part_idx.as<int>(), state, m.stream);
            launch_pick_token(m.shape, m.part_val.as<float>(), m.part_idx.as<int>(),
                              parts, state, m.tokens.as<int>(), m.stream);
            enqueue_step(m, kv, &state->token);
        };
        if (m.path == 1 || steps < 2) {
            for (size_t i = 0; i < steps; i++)
                iteration();
        } else {
            // Every kernel of an iteration reads its token, position and
            // stop flag from device memory, so one captured iteration is
            // replayed for every token; the cache and buffers it names are
            // the model's own (the generation cache lives as long as it).
            if (m.step_graph == nullptr) {
                if (fast_steps(m))
                    prepare_fast_steps(m);
                hipGraph_t graph = nullptr;
                hip_check(hipStreamBeginCapture(m.stream, hipStreamCaptureModeThreadLocal),
                          "hipStreamBeginCapture");
                iteration();
                hip_check(hipStreamEndCapture(m.stream, &graph), "hipStreamEndCapture");
                const hipError_t e = hipGraphInstantiate(&m.step_graph, graph, nullptr,
                                                         nullptr, 0);
                (void)hipGraphDestroy(graph);
                hip_check(e, "hipGraphInstantiate");
            }
            for (size_t i = 0; i < steps; i++)
                hip_check(hipGraphLaunch(m.step_graph, m.stream), "hipGraphLaunch");
        }
    }
    hip_check(hipEventRecord(m.decode_end, m.stream), "hipEventRecord");
    StepState host_state{};
    hip_check(hipMemcpyAsync(&host_state, state, sizeof host_state,
                             hipMemcpyDeviceToHost, m.stream),
              "hipMemcpyAsync");
    sync(m);
    const double t2 = now();
    check_token_error(m);
    float device_ms = 0.0f;
    hip_check(hipEventElapsedTime(&device_ms, m.decode_begin, m.decode_end),
              "hipEventElapsedTime");
    m.last_decode_device_ms = device_ms;
    const size_t count = size_t(host_state.count);
    if (count > 0)
        hip_check(hipMemcpy(out, m.tokens.get(), count * sizeof(int),
                            hipMemcpyDeviceToHost),
                  "hipMemcpy");
    kv.length = prompt_len + count; // every emitted token was decoded
    *out_count = count;
    if (stats != nullptr) {
        stats->prefill_tokens = prompt_len;
        stats->generated_tokens = count;
        stats->prefill_seconds = t1 - t0;
        stats->decode_seconds = t2 - t1;
    }
}

void generate_sampled(nut_model &m, const int *prompt, size_t prompt_len,
                      size_t max_tokens, float temperature, float top_p, uint32_t seed,
                      int *out, size_t *out_count, nut_generation_stats *stats)
{
    if (temperature <= 0.0f) {
        // choose_token's greedy branch (src/generate.cpp:28-30)
        generate_greedy(m, prompt, prompt_len, max_tokens, out, out_count, stats);
        return;
    }
    require(config_valid(m.config), NUT_EINVAL, "model config: invalid dimensions");
    require(prompt != nullptr && prompt_len != 0 && prompt_len <= m.config.max_seq,
            NUT_EINVAL, "generation: invalid prompt length");
    require(out != nullptr || max_tokens == 0, NUT_EINVAL, "generation: null output");
    require(out_count != nullptr, NUT_EINVAL, "generation: null output");
    check_ready(m, "generation");
    if (!m.generation_cache)
        m.generation_cache.reset(create_kv(m.config));
    nut_kvcache &kv = *m.generation_cache;
    const DecodeShape &s = m.shape;
    const int vocab = s.vocab;
    if (m.sample_ws.get() == nullptr)
        m.sample_ws.allocate(sample_workspace_bytes(vocab));

    const double t0 = now();
    prefill(m, kv, prompt, prompt_len, nullptr);
    const double t1 = now();
    // src/generate.cpp:184-207: one mt19937 per call, seeded with the seed
    std::mt19937 rng(seed);
    std::vector<float> p;
    std::vector<int> ids;
    std::vector<double> totals;
    constexpr size_t kChunk = 4096;
    size_t count = 0;
    StepState *state = m.state.as<StepState>();
    const int parts = classifier_blocks(s);
    while (count < max_tokens && kv.length < kv.config.max_seq) {
        // choose_token's checks (src/generate.cpp:34-36), at its first call
        require(std::isfinite(temperature) && top_p > 0.0f && top_p <= 1.0f, NUT_EINVAL,
                "sampling: invalid temperature or top-p");
        launch_reset_state(state, 0, m.stream);
        launch_classifier(s, m.hidden.as<float>(), m.final_norm.as<float>(), m.output_weights(),
                          m.logits.as<float>(), m.part_val.as<float>(), m.part_idx.as<int>(),
                          state, m.stream);
        float *sorted_p = nullptr, *token_p = nullptr;
        int *sorted_ids = nullptr, *bad = nullptr;
        double *block_totals = nullptr;
        const int nt = sample_sort(m.logits.as<float>(), vocab, m.part_val.as<float>(), parts,
                                   temperature, m.sample_ws.get(), &sorted_p, &sorted_ids,
                                   &token_p, &block_totals, &bad, m.stream);
        totals.resize(nt);
        int bad_host = 0;
        hip_check(hipMemcpyAsync(totals.data(), block_totals, nt * sizeof(double),
                                 hipMemcpyDeviceToHost, m.stream),
                  "hipMemcpyAsync");
        hip_check(hipMemcpyAsync(&bad_host, bad, sizeof bad_host, hipMemcpyDeviceToHost,
                                 m.stream),
                  "hipMemcpyAsync");
        sync(m);
        if (bad_host != 0)
            fail(NUT_ERUNTIME, "sampling: non-finite probability");
        double total = 0.0;
        for (double t : totals)
            total += t;
        if (!(total > 0.0))
            fail(NUT_ERUNTIME, "sampling: zero probability mass");
        // the nucleus: the sorted prefix until its mass reaches top_p of the
        // total (src/generate.cpp:63-68), read in chunks
        p.clear();
        ids.clear();
        auto sorted = [&](size_t i) {
            if (i == p.size()) {
                const size_t n = std::min(kChunk, size_t(vocab) - p.size());
                p.resize(p.size() + n);
                ids.resize(ids.size() + n);
                hip_check(hipMemcpy(p.data() + i, sorted_p + i, n * sizeof(float),
                                    hipMemcpyDeviceToHost),
                          "hipMemcpy to host");
                hip_check(hipMemcpy(ids.data() + i, sorted_ids + i, n * sizeof(int),
                                    hipMemcpyDeviceToHost),
                          "hipMemcpy to host");
            }
            return double(p[i]);
        };
        // The block sums and the reference's sum in token order round
        // differently: each is within (vocab - 1) 2^-53 of the exact sum,
        // relative to it. When a total that far off could move the cut,
        // the total is formed in token order, as the reference forms it.
        const double slack = total * double(vocab) * 0x1p-52 * 1.01;
        double nucleus = 0.0;
        bool ambiguous = false;
        size_t taken = nucleus_count(sorted, size_t(vocab), top_p, total, slack, nucleus,
                                     ambiguous);
        if (ambiguous) {
            std::vector<float> in_order(static_cast<size_t>(vocab));
            hip_check(hipMemcpy(in_order.data(), token_p, in_order.size() * sizeof(float),
                                hipMemcpyDeviceToHost),
                      "hipMemcpy to host");
            double sequential = 0.0;
            for (float q : in_order)
                sequential += q;
            taken = nucleus_count(sorted, size_t(vocab), top_p, sequential, 0.0, nucleus,
                                  ambiguous);
        }
        // the draw and the walk (src/generate.cpp:70-79)
        std::uniform_real_distribution<double> draw(0.0, nucleus);
        const double target = draw(rng);
        double cumulative = 0.0;
        int token = ids[taken - 1];
        for (size_t i = 0; i < taken; i++) {
            cumulative += p[i];
            if (target <= cumulative) {
                token = ids[i];
                break;
            }
        }
        if (size_t(token) == m.config.eos_token)
            break;
        out[count++] = token;
        decode(m, kv, token, nullptr);
    }
    const double t2 = now();
    *out_count = count;
    if (stats != nullptr) {
        stats->prefill_tokens = prompt_len;
        stats->generated_tokens = count;
        stats->prefill_seconds = t1 - t0;
        stats->decode_seconds = t2 - t1;
    }
}

} // namespace nut
