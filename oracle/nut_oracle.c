/* nut_oracle.c — CPU oracle for nutllm's quantised token loop.
 *
 * TEST INFRASTRUCTURE: the oracle for the HIP path and the "port" CPU
 * baseline. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it; the product library never does.
 *
 * Each function restates the reference function named beside it
 * (MokiMeow/nutllm, path:line). Floating-point expressions are written with
 * explicit fmaf()/fma() wherever g++ -O3 -mfma contracts the reference's
 * source, and this file is compiled with -ffp-contract=off, so rounding is
 * fixed by this text rather than by compiler flags.
 *
 * Pinning (how each part is checked against something other than itself):
 *   fp16 helpers     golden vectors from the compiled reference (crafted ties,
 *                    subnormal boundary, random), exhaustive round trip of
 *                    every positive finite half, monotonicity, zero-block KAT
 *   quantiser        byte/scale golden vectors from the compiled reference,
 *                    the f9 72 packing KAT, the storage formula, error bound
 *   matvec (both)    golden outputs from the compiled reference; e_k columns
 *                    of the dequantised matrix; fp64 brute force bound
 *   rmsnorm/rope/silu golden decode hidden states from the compiled
 *                    reference; reference hand fixtures (rmsnorm [3,4], rope
 *                    at position 1)
 *   attention        position 0 returns V0; equal keys give mean(V); GQA
 *                    head permutation; golden decode hidden states
 *   classifier/argmax golden logits and greedy ids; constructed ties
 *   generate         golden greedy ids (compiled reference) for the tiny
 *                    decoder; tiny llama2.c fixture gives {4, 5}
 */
#include "nut_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int orc_get_threads(void) { return g_threads; }

/* ---------------------------------------------------------------- fp16 -- */

/* positive_float_to_half (src/quant.cpp:23-47), restated on the fp32 bit
 * pattern: the reference rounds the 10-bit mantissa with lround (half away
 * from zero, i.e. half up for positive values) and, below 2^-14, rounds
 * value*2^24 the same way and clamps to [1, 1023] instead of carrying into
 * the smallest normal. */
int orc_float_to_half(float value, uint16_t *bits)
{
    if (!(value > 0.0f) || !isfinite(value))
        return ORC_EINVAL;
    if (value > 65504.0f)
        return ORC_ERANGE;
    uint32_t u;
    memcpy(&u, &value, sizeof u);
    const int biased = (int)(u >> 23);
    uint32_t significand = u & 0x7fffffu;
    int exponent = biased - 127;
    if (biased == 0)
        exponent = -126;
    else
        significand |= 0x800000u;
    if (exponent < -14) {
        /* value * 2^24 = significand * 2^(exponent + 1); shift >= 14. */
        const int shift = -(exponent + 1);
        uint64_t m = 0;
        if (shift < 40)
            m = ((uint64_t)significand + (1ull << (shift - 1))) >> shift;
        if (m < 1)
            m = 1;
        if (m > 1023)
            m = 1023;
        *bits = (uint16_t)m;
        return ORC_OK;
    }
    uint32_t mantissa = ((significand & 0x7fffffu) + (1u << 12)) >> 13;
    if (mantissa == 1024) {
        mantissa = 0;
        exponent++;
    }
    if (exponent > 15)
        return ORC_ERANGE;
    *bits = (uint16_t)(((uint32_t)(exponent + 15) << 10) | mantissa);
    return ORC_OK;
}

/* positive_half_to_float (src/quant.cpp:49-56). */
float orc_half_to_float(uint16_t bits)
{
    const uint32_t exponent = (bits >> 10) & 0x1f;
    const uint32_t mantissa = bits & 0x3ff;
    if (exponent == 0)
        return (float)mantissa * 0x1p-24f;
    const uint32_t u = ((exponent - 15 + 127) << 23) | (mantissa << 13);
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* ----------------------------------------------------------- quantiser -- */

static int limit_of(int type) { return type == ORC_INT8 ? 127 : 7; }

size_t orc_storage_bytes(size_t rows, size_t cols, int type,
                         size_t block_size)
{
    /* src/quant.cpp:134-145 sizes, 235-241 sum. */
    const size_t n = rows * cols;
    const size_t blocks = (n + block_size - 1) / block_size;
    const size_t data = type == ORC_INT8 ? n : (n + 1) / 2;
    return data + blocks * 2;
}

/* QuantizedMatrix::quantize (src/quant.cpp:154-197): per flattened block,
 * max |w|, scale = max/limit (2^-24 for an all-zero block) rounded through
 * fp16, q = clamp(lround(w / stored_scale), +-limit). */
int orc_quantize(const float *source, size_t rows, size_t cols, int type,
                 size_t block_size, uint8_t *data, uint16_t *scales)
{
    if (source == NULL || data == NULL || scales == NULL)
        return ORC_EINVAL;
    if (rows == 0 || cols == 0 || block_size == 0 ||
        rows > (size_t)-1 / cols)
        return ORC_EINVAL;
    if (type != ORC_INT8 && type != ORC_INT4)
        return ORC_EINVAL;
    const size_t n = rows * cols;
    const size_t blocks = (n + block_size - 1) / block_size;
    const int limit = limit_of(type);
    const size_t data_bytes = type == ORC_INT8 ? n : (n + 1) / 2;
    memset(data, 0, data_bytes);
    for (size_t b = 0; b < blocks; b++) {
        const size_t begin = b * block_size;
        const size_t end = begin + block_size < n ? begin + block_size : n;
        float maximum = 0.0f;
        for (size_t i = begin; i < end; i++) {
            if (!isfinite(source[i]))
                return ORC_EINVAL;
            const float a = fabsf(source[i]);
            if (maximum < a)
                maximum = a;
        }
        const float exact = maximum == 0.0f ? 0x1p-24f
                                            : maximum / (float)limit;
        uint16_t bits = 0;
        const int status = orc_float_to_half(exact, &bits);
        if (status != ORC_OK)
            return status;
        scales[b] = bits;
        const float stored = orc_half_to_float(bits);
        for (size_t i = begin; i < end; i++) {
            long q = lroundf(source[i] / stored);
            if (q > limit)
                q = limit;
            if (q < -limit)
                q = -limit;
            if (type == ORC_INT8) {
                data[i] = (uint8_t)((unsigned long)q & 0xffu);
            } else {
                const uint8_t nibble = (uint8_t)((unsigned long)q & 0x0fu);
                if ((i & 1) == 0)
                    data[i / 2] = (uint8_t)((data[i / 2] & 0xf0u) | nibble);
                else
                    data[i / 2] =
                        (uint8_t)((data[i / 2] & 0x0fu) | (nibble << 4));
            }
        }
    }
    return ORC_OK;
}

/* quantized_value (src/quant.cpp:199-209): two's-complement byte or
 * nibble. */
int orc_quantized_value(const orc_qmat *m, size_t index)
{
    if (m->type == ORC_INT8)
        return (int)(int8_t)m->data[index];
    const uint8_t packed = m->data[index / 2];
    const unsigned nibble = (index & 1) ? (packed >> 4) & 0xfu : packed & 0xfu;
    return nibble >= 8 ? (int)nibble - 16 : (int)nibble;
}

/* value (src/quant.cpp:217-222). */
float orc_value(const orc_qmat *m, size_t row, size_t column)
{
    const size_t index = row * m->cols + column;
    return (float)orc_quantized_value(m, index) *
           orc_half_to_float(m->scales[index / m->block_size]);
}

/* error_bound (src/quant.cpp:224-233). */
float orc_error_bound(const orc_qmat *m, size_t row, size_t column)
{
    const size_t index = row * m->cols + column;
    const float stored = orc_half_to_float(m->scales[index / m->block_size]);
    float half_rounding = stored / 2047.0f;
    if (half_rounding < 0x1p-25f)
        half_rounding = 0x1p-25f;
    const float limit = m->type == ORC_INT8 ? 127.0f : 7.0f;
    /* g++ -mfma contracts this sum as fma(stored, 0.5f, product): the
     * (limit + 0.5) * half_rounding product is rounded on its own, and
     * stored * 0.5f is exact, so the fma equals the plain sum below. */
    const float product = (limit + 0.5f) * half_rounding;
    return stored * 0.5f + product;
}

void orc_dequantize(const orc_qmat *m, float *out)
{
    for (size_t r = 0; r < m->rows; r++)
        for (size_t c = 0; c < m->cols; c++)
            out[r * m->cols + c] = orc_value(m, r, c);
}

/* -------------------------------------------------------------- matvec -- */

/* dot_int8_blocks / dot_int4_blocks (src/quant.cpp:75-129) with
 * horizontal_sum (66-73): eight fp32 lanes, lane j accumulating the row's
 * elements j, j+8, j+16, ... in index order as fma(q*scale, x, lane); the
 * lanes are then summed left to right from 0. q*scale is exact in fp32. */
static float dot_blocks_avx2_order(const orc_qmat *m, size_t row,
                                   const float *x)
{
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const size_t cols = m->cols;
    const size_t row_begin = row * cols;
    for (size_t b = 0; b < cols / 32; b++) {
        const float scale =
            orc_half_to_float(m->scales[row_begin / 32 + b]);
        for (size_t k = 0; k < 32; k++) {
            const size_t i = row_begin + b * 32 + k;
            const float v = (float)orc_quantized_value(m, i) * scale;
            lanes[k & 7] = fmaf(v, x[b * 32 + k], lanes[k & 7]);
        }
    }
    float total = 0.0f;
    for (int j = 0; j < 8; j++)
        total += lanes[j];
    return total;
}

/* Scalar path (src/quant.cpp:289-317): blocks may straddle rows; products
 * double(float(q)*scale)*double(x) are exact in double and summed in
 * index order. */
static float dot_blocks_scalar(const orc_qmat *m, size_t row, const float *x)
{
    double sum = 0.0;
    const size_t row_begin = row * m->cols;
    const size_t row_end = row_begin + m->cols;
    for (size_t i = row_begin; i < row_end; i++) {
        const float scale = orc_half_to_float(m->scales[i / m->block_size]);
        const float v = (float)orc_quantized_value(m, i) * scale;
        sum = fma((double)v, (double)x[i - row_begin], sum);
    }
    return (float)sum;
}

int orc_matvec_q(const orc_qmat *m, const float *x, float *y)
{
    if (x == NULL || y == NULL || m == NULL)
        return ORC_EINVAL;
    const int fast = m->block_size == 32 && m->cols % 32 == 0;
    const long rows = (long)m->rows;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (long r = 0; r < rows; r++)
        y[r] = fast ? dot_blocks_avx2_order(m, (size_t)r, x)
                    : dot_blocks_scalar(m, (size_t)r, x);
    return ORC_OK;
}

/* matvec_threaded (src/threading.cpp:183-198): sequential fp32 dot per row.
 * The compiled reference rounds the product before the add here (checked
 * bit-for-bit against the reference build), so no fma. */
int orc_matvec_f32(const float *w, size_t rows, size_t cols, const float *x,
                   float *y)
{
    if (w == NULL || x == NULL || y == NULL)
        return ORC_EINVAL;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (long r = 0; r < (long)rows; r++) {
        const float *row = w + (size_t)r * cols;
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            const float product = row[c] * x[c];
            sum = sum + product;
        }
        y[r] = sum;
    }
    return ORC_OK;
}

/* matmul_threaded (src/threading.cpp:163-181): i-k-j order,
 * out[j] += a[i,k]*b[k,j] contracted to fma. */
int orc_matmul(const float *a, const float *b, float *c, size_t m, size_t k,
               size_t n)
{
    if (a == NULL || b == NULL || c == NULL)
        return ORC_EINVAL;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (long i = 0; i < (long)m; i++) {
        float *out = c + (size_t)i * n;
        for (size_t j = 0; j < n; j++)
            out[j] = 0.0f;
        for (size_t p = 0; p < k; p++) {
            const float v = a[(size_t)i * k + p];
            const float *brow = b + p * n;
            for (size_t j = 0; j < n; j++)
                out[j] = fmaf(v, brow[j], out[j]);
        }
    }
    return ORC_OK;
}

/* --------------------------------------------------------- elementwise -- */

/* rmsnorm (src/ops.cpp:111-134): eight fp32 lanes of x*x over full groups
 * of 8 (g++ contracts the mul+add intrinsics to fma), lanes summed left to
 * right, fp32 tail, then out = x*scale*w. */
int orc_rmsnorm(const float *x, const float *w, float *out, size_t n,
                float eps)
{
    if (x == NULL || w == NULL || out == NULL || n == 0 || !(eps >= 0.0f) ||
        !isfinite(eps))
        return ORC_EINVAL;
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++)
            lanes[j] = fmaf(x[i + j], x[i + j], lanes[j]);
    float squares = 0.0f;
    for (int j = 0; j < 8; j++)
        squares += lanes[j];
    for (; i < n; i++)
        squares = fmaf(x[i], x[i], squares);
    const float scale = 1.0f / sqrtf(squares / (float)n + eps);
    for (size_t o = 0; o < n; o++)
        out[o] = x[o] * scale * w[o];
    return ORC_OK;
}

/* silu (src/ops.cpp:136-138). */
float orc_silu(float v) { return v / (1.0f + expf(-v)); }

/* rotate_vector (src/quant_model.cpp:26-37): double frequency and angle,
 * fp32 cos/sin, fp32 rotation with the first product of each line fused. */
void orc_rotate(float *values, size_t dims, size_t position)
{
    for (size_t pair = 0; pair < dims; pair += 2) {
        const double frequency = pow(10000.0, -(double)pair / (double)dims);
        const float c = (float)cos((double)position * frequency);
        const float s = (float)sin((double)position * frequency);
        const float even = values[pair];
        const float odd = values[pair + 1];
        values[pair] = fmaf(even, c, -(odd * s));
        values[pair + 1] = fmaf(even, s, odd * c);
    }
}

/* --------------------------------------------------------------- model -- */

static size_t kv_heads_of(const orc_config *c)
{
    return c->kv_heads == 0 ? c->heads : c->kv_heads;
}

/* ModelConfig::validate (src/attention.cpp:15-27). */
int orc_config_valid(const orc_config *c)
{
    const size_t kv = kv_heads_of(c);
    if (c->layers == 0 || c->heads == 0 || c->dim == 0 || c->head_dim == 0 ||
        c->ffn_dim == 0 || c->vocab_size == 0 || c->max_seq == 0 ||
        c->heads * c->head_dim != c->dim || c->head_dim % 2 != 0 ||
        c->eos_token >= c->vocab_size || kv == 0 || kv > c->heads ||
        c->heads % kv != 0)
        return 0;
    return 1;
}

size_t orc_kv_elements(const orc_config *c)
{
    return c->layers * kv_heads_of(c) * c->max_seq * c->head_dim;
}

/* KVCache::offset (src/kvcache.cpp:196-205). */
static size_t kv_offset(const orc_config *c, size_t layer, size_t head,
                        size_t position)
{
    return ((layer * kv_heads_of(c) + head) * c->max_seq + position) *
           c->head_dim;
}

/* attention_step (src/quant_model.cpp:45-108). */
static void attention_step(const orc_model *m, const orc_layer *w,
                           size_t layer, size_t position,
                           const float *normalized, float *keys,
                           float *values, float *output, float *query,
                           float *key, float *value, float *context,
                           float *scores)
{
    const orc_config *c = &m->config;
    const size_t kv = kv_heads_of(c), hd = c->head_dim;
    orc_matvec_q(&w->query, normalized, query);
    orc_matvec_q(&w->key, normalized, key);
    orc_matvec_q(&w->value, normalized, value);
    for (size_t h = 0; h < c->heads; h++)
        orc_rotate(query + h * hd, hd, position);
    for (size_t h = 0; h < kv; h++)
        orc_rotate(key + h * hd, hd, position);
    for (size_t h = 0; h < kv; h++) {
        const size_t dst = kv_offset(c, layer, h, position);
        memcpy(keys + dst, key + h * hd, hd * sizeof(float));
        memcpy(values + dst, value + h * hd, hd * sizeof(float));
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t group = c->heads / kv;
    for (size_t h = 0; h < c->heads; h++) {
        const size_t kvh = h / group;
        const float *q = query + h * hd;
        float maximum = -INFINITY;
        for (size_t p = 0; p <= position; p++) {
            const float *k = keys + kv_offset(c, layer, kvh, p);
            double dot = 0.0;
            for (size_t d = 0; d < hd; d++)
                dot = fma((double)q[d], (double)k[d], dot);
            scores[p] = (float)dot * scale;
            if (maximum < scores[p])
                maximum = scores[p];
        }
        double total = 0.0;
        for (size_t p = 0; p <= position; p++) {
            scores[p] = expf(scores[p] - maximum);
            total += scores[p];
        }
        for (size_t d = 0; d < hd; d++) {
            double sum = 0.0;
            for (size_t p = 0; p <= position; p++) {
                const float *v = values + kv_offset(c, layer, kvh, p);
                sum = fma((double)(scores[p] / (float)total), (double)v[d],
                          sum);
            }
            context[h * hd + d] = (float)sum;
        }
    }
    orc_matvec_q(&w->output, context, output);
}

/* decode_quantized_token (src/quant_model.cpp:158-206). */
int orc_decode(const orc_model *m, float *keys, float *values,
               size_t *length, int token, float *hidden)
{
    const orc_config *c = &m->config;
    if (!orc_config_valid(c))
        return ORC_EINVAL;
    if (token < 0 || (size_t)token >= c->vocab_size)
        return ORC_ERANGE_IDX;
    if (*length >= c->max_seq)
        return ORC_ELENGTH;
    const size_t position = *length;
    const size_t dim = c->dim, ffn = c->ffn_dim, kvd = kv_heads_of(c) * c->head_dim;
    float *buf = malloc(sizeof(float) *
                        (dim * 5 + kvd * 2 + ffn * 2 + c->max_seq));
    if (buf == NULL)
        return ORC_ELENGTH;
    float *normalized = buf, *attention = buf + dim, *query = buf + 2 * dim,
          *context = buf + 3 * dim, *ff = buf + 4 * dim,
          *key = buf + 5 * dim, *value = key + kvd, *gate = value + kvd,
          *up = gate + ffn, *scores = up + ffn;
    memcpy(hidden, m->embeddings + (size_t)token * dim, dim * sizeof(float));
    for (size_t l = 0; l < c->layers; l++) {
        const orc_layer *w = &m->layers[l];
        orc_rmsnorm(hidden, w->attention_norm, normalized, dim, 1e-5f);
        attention_step(m, w, l, position, normalized, keys, values,
                       attention, query, key, value, context, scores);
        for (size_t i = 0; i < dim; i++)
            hidden[i] += attention[i];
        orc_rmsnorm(hidden, w->ffn_norm, normalized, dim, 1e-5f);
        orc_matvec_q(&w->gate, normalized, gate);
        orc_matvec_q(&w->up, normalized, up);
        for (size_t i = 0; i < ffn; i++)
            gate[i] = orc_silu(gate[i]) * up[i];
        orc_matvec_q(&w->down, gate, ff);
        for (size_t i = 0; i < dim; i++)
            hidden[i] += ff[i];
    }
    *length = position + 1;
    free(buf);
    return ORC_OK;
}

/* prefill_quantized (src/quant_model.cpp:208-220): reset, then one decode
 * step per prompt token; returns the last hidden state. */
int orc_prefill(const orc_model *m, float *keys, float *values,
                size_t *length, const int *tokens, size_t count,
                float *hidden)
{
    if (count == 0 || count > m->config.max_seq)
        return ORC_EINVAL;
    *length = 0;
    for (size_t t = 0; t < count; t++) {
        const int status = orc_decode(m, keys, values, length, tokens[t],
                                      hidden);
        if (status != ORC_OK)
            return status;
    }
    return ORC_OK;
}

int orc_logits(const orc_model *m, const float *hidden, float *logits)
{
    const size_t dim = m->config.dim;
    float *normalized = malloc(dim * sizeof(float));
    if (normalized == NULL)
        return ORC_ELENGTH;
    orc_rmsnorm(hidden, m->final_norm, normalized, dim, 1e-5f);
    orc_matvec_f32(m->output_weights, m->config.vocab_size, dim, normalized,
                   logits);
    free(normalized);
    return ORC_OK;
}

/* std::max_element: the first index holding the maximum. */
size_t orc_argmax(const float *logits, size_t n)
{
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (logits[best] < logits[i])
            best = i;
    return best;
}

static double now_seconds(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* generate_tokens_cached(const QuantizedModelWeights&) greedy branch
 * (src/generate.cpp:174-216), with its GenerationStats timing: prefill
 * covers the prefill call; decode covers every norm+classifier+argmax and
 * every decode step, including the decode of the last emitted token. */
int orc_generate(const orc_model *m, const int *prompt, size_t prompt_len,
                 size_t max_tokens, int *out, size_t *out_count,
                 double *prefill_seconds, double *decode_seconds)
{
    const orc_config *c = &m->config;
    if (!orc_config_valid(c))
        return ORC_EINVAL;
    if (prompt_len == 0 || prompt_len > c->max_seq)
        return ORC_EINVAL;
    const size_t kv = orc_kv_elements(c);
    float *keys = calloc(kv, sizeof(float));
    float *values = calloc(kv, sizeof(float));
    float *hidden = malloc(c->dim * sizeof(float));
    float *logits = malloc(c->vocab_size * sizeof(float));
    if (!keys || !values || !hidden || !logits) {
        free(keys), free(values), free(hidden), free(logits);
        return ORC_ELENGTH;
    }
    size_t length = 0;
    const double t0 = now_seconds();
    int status = orc_prefill(m, keys, values, &length, prompt, prompt_len,
                             hidden);
    const double t1 = now_seconds();
    size_t count = 0;
    while (status == ORC_OK && count < max_tokens && length < c->max_seq) {
        orc_logits(m, hidden, logits);
        const size_t token = orc_argmax(logits, c->vocab_size);
        if (token == c->eos_token)
            break;
        out[count++] = (int)token;
        status = orc_decode(m, keys, values, &length, (int)token, hidden);
    }
    const double t2 = now_seconds();
    if (prefill_seconds)
        *prefill_seconds = t1 - t0;
    if (decode_seconds)
        *decode_seconds = t2 - t1;
    *out_count = count;
    free(keys), free(values), free(hidden), free(logits);
    return status;
}
