// prefill.hpp — batched prompt processing (the prefill GEMM path).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "kernels.hpp"

namespace nut {

// True when every projection uses the fast layout (block 32, rows of whole
// blocks) and the head size is the one the attention tiles assume.
bool prefill_gemm_supported(const DecodeShape &s, const LayerView &w);

void launch_embed_rows(const float *embeddings, const int *tokens, float *h,
                       int t_count, int dim, hipStream_t stream);
void launch_rmsnorm_rows(const float *h, const float *w, float *out,
                         int t_count, int dim, hipStream_t stream);
// c[t][n] (= or +=) sum_k x[t][k] w[n][k], t < t_count; x rows are w.cols
// floats, c rows ldc floats.
void launch_qgemm_rows(const float *x, int t_count, const QMat &w, float *c,
                       int ldc, bool add, hipStream_t stream);
// RoPE of q rows and k rows at positions start + t; k and v rows into the
// layer's cache.
void launch_rope_store(float *q, const float *k, const float *v,
                       const float2 *rope, float *k_cache, float *v_cache,
                       const DecodeShape &s, int t_count, int start,
                       hipStream_t stream);
// Causal attention of the t_count queries over cache positions
// 0 .. start + t.
void launch_attention_prefill(const float *q, const float *k_cache,
                              const float *v_cache, float *ctx,
                              const DecodeShape &s, int t_count, int start,
                              hipStream_t stream);
void launch_silu_mul(const float *g, const float *u, float *act, size_t n,
                     hipStream_t stream);

} // namespace nut
