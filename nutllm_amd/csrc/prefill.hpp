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
// GEMM inputs are written as two f16 limbs per value: hi = f16(v) and
// lo = f16(v - hi), [t][k] each.
void launch_rmsnorm_rows(const float *h, const float *w, _Float16 *out_hi,
                         _Float16 *out_lo, int t_count, int dim, hipStream_t stream);
// The prefill GEMM reads each matrix's fp16 scales stage-major: dword
// [st][row] holds the scales of blocks 2 st and 2 st + 1 of the row
// (stage_scale_words(m) dwords, built once per matrix).
size_t stage_scale_words(const QMat &m);
void launch_scales_by_stage(const QMat &m, uint32_t *dst, hipStream_t stream);
// c_i[t][n] (= or +=) sum_k x[t][k] w_i[n][k] for `count` (1 to 3)
// matrices of one type and input size, t < t_count, in one launch; x as
// limbs of w.cols values per row, c_i rows ldc_i floats.
void launch_qgemm_rows(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                       const QMat *const *w, const uint32_t *const *stage_scales,
                       float *const *c, const int *ldc, int count, bool add,
                       hipStream_t stream);
// act[t][n] = silu(gate[n] . x[t]) * (up[n] . x[t]) as limbs (act_hi,
// act_lo, gate.rows values per row): both products in one launch, each
// workgroup 64 outputs of both matrices, so neither product leaves the
// registers.
void launch_qgemm_swiglu(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                         const QMat &gate, const QMat &up, const uint32_t *st_gate,
                         const uint32_t *st_up, _Float16 *act_hi, _Float16 *act_lo,
                         hipStream_t stream);
// The batch's K and V as f16 limbs, the prefill attention's operands:
// 4 * prefill_kv_limb_elems(s) f16 (K hi, K lo, V^T hi, V^T lo).
size_t prefill_kv_limb_elems(const DecodeShape &s);
// Q/K/V products of the batch (w: query, key, value) at positions 0 ..
// t_count - 1 with RoPE applied to q and k: q rows into q ([t][heads *
// head_dim]), k and v rows into the layer's cache, and both as limbs into
// kv_limbs for launch_attention_prefill.
void launch_qgemm_qkv(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                      const QMat *const *w, const uint32_t *const *stage_scales, float *q,
                      const float2 *rope, float *k_cache, float *v_cache, _Float16 *kv_limbs,
                      const DecodeShape &s, hipStream_t stream);
// Causal attention of the t_count queries (positions 0 .. t_count - 1) over
// positions 0 .. t, K and V from kv_limbs as launch_qgemm_qkv wrote them.
void launch_attention_prefill(const float *q, const _Float16 *kv_limbs, _Float16 *ctx_hi,
                              _Float16 *ctx_lo, const DecodeShape &s, int t_count,
                              hipStream_t stream);

} // namespace nut
