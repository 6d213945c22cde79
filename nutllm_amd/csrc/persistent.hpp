// persistent.hpp — host interface of the cooperative token-loop kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace nut {

// Workgroups of the cooperative kernel (one per CU of an MI355X).
constexpr int kTokenGrid = 256;

// Arguments of one launch. The kernel runs n_iter iterations; with
// classify set, each iteration first runs the final rmsnorm + classifier +
// argmax on the current hidden state (the generate loop), otherwise it
// decodes tokens_in[it] (the prefill loop). Iteration it decodes at KV
// position start_len + it.
struct TokenArgs {
    // Weight arena: layer l at weights + l * layer_layout(...).bytes.
    const uint8_t *weights;
    const float *embeddings, *final_norm, *classifier;
    // The classifier's INT8 screening copy (launch_classifier_screen): codes
    // and block scales, or null for the plain fp32 pass over every row.
    const uint8_t *classifier8;
    const uint16_t *classifier8_scales;
    const float2 *rope;
    float *k_cache, *v_cache; // [layer][kv_head][max_seq][head_dim]
    uint64_t *x_qkv, *x_hidden, *x_act, *x_part; // tagged exchange buffers
    // The q/k/v (or the wide kernel's context), h and act exchanges in
    // write-once words (token_once_floats of them, every word kUnset =
    // 0xffffffff when the launch starts), iteration it and layer l at
    // x_once + once_slice(it, l, layer_count) * token_once_stride (the
    // kernels advance the slice index by one per step).
    float *x_once;
    // Long contexts (long_attention != 0): attention is split over the
    // workgroups; x_apart holds each workgroup's partial (m, l, o) for the
    // query heads of its KV head, x_ctx the merged context.
    uint64_t *x_apart, *x_ctx;
    int long_attention;
    // Wide shapes (wide.hip): each workgroup's partial attention scores,
    // [head][workgroup of the head][position].
    uint64_t *x_scores;
    const float *hidden_in;   // hidden state before iteration 0 (classify)
    float *hidden_out;        // hidden state after the last decode step
    const int *tokens_in;     // per-iteration tokens (prefill)
    int *tokens_out;          // emitted tokens (generate)
    StepState *state;
    int *error;               // set on a bounded-wait timeout
    unsigned tag_base;        // next_tag_base: unique since the last clear
    // Optional phase timeline (s_memrealtime ticks, 100 MHz) of workgroups
    // [0, timeline_wgs): marks_per_iteration(layers) entries per iteration,
    // timeline_cap entries per workgroup.
    unsigned long long *timeline;
    int timeline_cap, timeline_wgs;
    // Test hook (nut_model_inject_fault): 1 = workgroup 0 leaves its words
    // of the first step's h after W2 unpublished.
    int fault;
    int layer_count, vocab, max_seq, eos;
    int start_len, n_iter, classify;
    float attn_scale;
};

// Largest share of classifier rows per workgroup for which the generate
// loop screens the classifier through its INT8 copy (TokenArgs::
// classifier8); larger vocabularies take the plain fp32 pass.
constexpr int kScreenRowsMax = 1024;

// Write-once words per iteration and layer. The TinyLlama-shape kernel:
// q/k/v, the Wo partial sums of each KV head group (fused attention; split
// attention puts the merged context and h after Wo in that space), act, h
// after W2. The wide kernel (wide.hip): the context, h after Wo, act, h
// after W2.
inline size_t token_once_stride(const DecodeShape &s, bool wide)
{
    if (wide)
        return 3 * size_t(s.dim) + s.ffn_dim;
    return size_t(s.dim) * (2 + s.kv_heads) + 2 * size_t(s.kv_heads) * s.head_dim + s.ffn_dim;
}

// The write-once words form a ring of kOnceRing slices, one per (iteration,
// layer) step: step u = it * layers + l uses slice u % kOnceRing. At the
// start of phase C of step u + 2, before its take of that step's h after
// Wo, each workgroup sets the words it published in step u back to kUnset:
// it has taken the h after Wo of step u + 1, into which every workgroup
// publishes only after it has taken every exchange of step u, so no
// consumer still polls them. The take that follows retires the re-arming
// stores (its closing s_waitcnt vmcnt(0)) before the workgroup publishes
// its activation of step u + 2, and every consumer takes that activation
// before it polls a word of step u + 3, the slice's next use, so it finds
// kUnset there until the new value; the workgroup's own words of step
// u + 3 come after its re-arm in program order. tests/test_cpu_once_ring.py
// replays the protocol and shows that two slices would not do. The ring's
// size is independent of the tokens a launch decodes.
constexpr int kOnceRing = 3;

__host__ __device__ inline int once_slice(int it, int layer, int layers)
{
    return (it * layers + layer) % kOnceRing;
}

inline size_t token_once_floats(const DecodeShape &s, bool wide)
{
    return kOnceRing * token_once_stride(s, wide);
}

// Exchange tags. Every exchange word is (tag << 32) | value, and a launch
// uses the tags [base, base + 2^kTagShift) with base = count << kTagShift for
// a launch counter count in 1 .. kTagBases. A word in the buffer carries
// either tag 0 (the buffer was zeroed) or a tag of a launch since the last
// zeroing; bases are never 0 and never repeat between zeroings, so no
// consumer can find a stale word already holding the tag it waits for. When
// the counter runs out, next_tag_base asks for the buffer to be zeroed
// before the launch and restarts it at 1.
constexpr unsigned kTagShift = 20;
constexpr unsigned kTagBases = (1u << (32 - kTagShift)) - 1;

inline unsigned next_tag_base(unsigned &count, bool &clear)
{
    clear = count >= kTagBases;
    if (clear)
        count = 0;
    return (++count) << kTagShift;
}

// Tags one launch may use: per iteration one for the argmax exchange, then
// per layer at most six (q/k/v, two for split attention, h after Wo, act,
// h after W2).
inline long long token_tags_needed(long long n_iter, long long layers)
{
    return n_iter * (1 + 6 * layers) + 1;
}

// Timeline entries per iteration: iteration start, classifier input staged,
// classifier pass done (this workgroup's best row), token known, then per
// layer, for each of the phases A, B, C, D: input staged, outputs published
// (every wave past its publishes), next weights issued to LDS DMA; phase B
// also marks attention done after its input.
__host__ __device__ inline int marks_per_iteration(int layers)
{
    return 4 + 13 * layers;
}

// Longest context (positions) the kernel's fused attention phase handles
// for this shape; 0 when the shape has no instantiation.
int token_kernel_max_positions(int type, const DecodeShape &s);
// Longest context of the split-attention variant (long_attention), used
// beyond token_kernel_max_positions; 0 when the shape has no instantiation.
int token_kernel_long_positions(int type, const DecodeShape &s);

// True when the cooperative kernel has an instantiation for this shape and
// quant type and the device can hold its grid.
bool token_kernel_supported(int type, const DecodeShape &s);
// Exchange-buffer sizes (uint64 entries).
size_t token_exchange_entries(const DecodeShape &s);
void launch_token_kernel(int type, const DecodeShape &s, const TokenArgs &a,
                         hipStream_t stream);

// The kernel for wide multi-head shapes (wide.hip): its longest context (0
// when the shape and type have no instantiation), the uint64 entries of its
// score buffer (TokenArgs::x_scores; 0 for other shapes), and its launch.
int wide_kernel_positions(int type, const DecodeShape &s);
size_t wide_kernel_score_entries(const DecodeShape &s);
void launch_wide_kernel(int type, const DecodeShape &s, const TokenArgs &a,
                        hipStream_t stream);

} // namespace nut
