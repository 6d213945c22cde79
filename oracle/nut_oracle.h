/* nut_oracle.h — CPU oracle for nutllm's quantised token loop.
 *
 * TEST INFRASTRUCTURE. It checks the HIP path and is never the thing measured or
 * shipped: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product path (nutllm_amd) never links or calls it.
 *
 * Every function restates the reference algorithm it names (file:line in
 * MokiMeow/nutllm) in plain C, bit-for-bit where the reference is exact:
 * same fp16 rounding quirks, same flattened quant blocks, same AVX2 lane
 * order, same FMA contractions that g++ -O3 -mfma applies to the reference.
 */
#ifndef NUT_ORACLE_H
#define NUT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes mirror the C++ exception types the reference throws. */
enum {
    ORC_OK = 0,
    ORC_EINVAL = 1,  /* std::invalid_argument */
    ORC_ERANGE_IDX = 2, /* std::out_of_range */
    ORC_ELENGTH = 3, /* std::length_error */
    ORC_ERANGE = 4,  /* std::range_error */
};

enum { ORC_INT8 = 0, ORC_INT4 = 1 };

/* ModelConfig (include/model.hpp:8-24). kv_heads == 0 means heads. */
typedef struct {
    size_t layers, heads, dim, head_dim, ffn_dim, vocab_size, max_seq,
        eos_token, kv_heads;
} orc_config;

/* A QuantizedMatrix's storage (include/quant.hpp:40-49): flattened
 * row-major quant blocks of block_size, INT8 bytes or INT4 nibbles (even
 * flattened index in the low nibble), fp16 scale bit patterns. */
typedef struct {
    const uint8_t *data;
    const uint16_t *scales;
    size_t rows, cols, block_size;
    int type;
} orc_qmat;

/* QuantizedLayerWeights (include/quant_model.hpp:9-30). */
typedef struct {
    orc_qmat query, key, value, output, gate, up, down;
    const float *attention_norm, *ffn_norm;
} orc_layer;

/* QuantizedModelWeights (include/quant_model.hpp:32-46); output_weights is
 * lm_head, or embeddings when tied. */
typedef struct {
    orc_config config;
    const float *embeddings;
    const float *final_norm;
    const float *output_weights;
    const orc_layer *layers;
} orc_model;

/* fp16 helpers: src/quant.cpp:23-56. */
int orc_float_to_half(float value, uint16_t *bits);
float orc_half_to_float(uint16_t bits);

/* Quantiser: src/quant.cpp:134-197. data holds n (INT8) or ceil(n/2)
 * (INT4) bytes, scales ceil(n/block_size) entries. */
int orc_quantize(const float *source, size_t rows, size_t cols, int type,
                 size_t block_size, uint8_t *data, uint16_t *scales);
size_t orc_storage_bytes(size_t rows, size_t cols, int type,
                         size_t block_size);
int orc_quantized_value(const orc_qmat *m, size_t index);
float orc_value(const orc_qmat *m, size_t row, size_t column);
float orc_error_bound(const orc_qmat *m, size_t row, size_t column);
void orc_dequantize(const orc_qmat *m, float *out);

/* matvec_quantized_threaded: src/quant.cpp:262-321 (AVX2 block path when
 * block_size == 32 && cols % 32 == 0, else the double scalar path). */
int orc_matvec_q(const orc_qmat *m, const float *x, float *y);
/* matvec_threaded: src/threading.cpp:183-198 (fp32 classifier). */
int orc_matvec_f32(const float *w, size_t rows, size_t cols, const float *x,
                   float *y);
/* matmul_threaded: src/threading.cpp:163-181 (C = A.B, row-major). */
int orc_matmul(const float *a, const float *b, float *c, size_t m, size_t k,
               size_t n);

/* Elementwise ops: src/ops.cpp:111-138, src/quant_model.cpp:26-43. */
int orc_rmsnorm(const float *x, const float *w, float *out, size_t n,
                float eps);
float orc_silu(float v);
void orc_rotate(float *values, size_t dims, size_t position);

/* ModelConfig::validate (src/attention.cpp:15-27). */
int orc_config_valid(const orc_config *c);
/* KV cache geometry (src/kvcache.cpp:196-205). */
size_t orc_kv_elements(const orc_config *c);

/* decode_quantized_token (src/quant_model.cpp:158-206). keys/values hold
 * orc_kv_elements floats each, [layer][kv_head][position][head_dim]. */
int orc_decode(const orc_model *m, float *keys, float *values,
               size_t *length, int token, float *hidden);
/* prefill_quantized (src/quant_model.cpp:208-220). */
int orc_prefill(const orc_model *m, float *keys, float *values,
                size_t *length, const int *tokens, size_t count,
                float *hidden);
/* Final rmsnorm + classifier (src/generate.cpp:197-200). */
int orc_logits(const orc_model *m, const float *hidden, float *logits);
/* Greedy branch of choose_token (src/generate.cpp:24-30). */
size_t orc_argmax(const float *logits, size_t n);
/* generate_tokens_cached for quantised weights, greedy
 * (src/generate.cpp:174-216). Writes up to max_tokens ids. */
int orc_generate(const orc_model *m, const int *prompt, size_t prompt_len,
                 size_t max_tokens, int *out, size_t *out_count,
                 double *prefill_seconds, double *decode_seconds);

/* Worker threads the oracle uses for row loops (1 = scalar port). */
void orc_set_threads(int threads);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
