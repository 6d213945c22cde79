// device.hpp — device building blocks shared by the gfx950 kernels.
//
// Quantised rows are read in 16-byte "chunks": one INT4 chunk is one
// 32-weight quant block (one fp16 scale), one INT8 chunk is half a block.
// Lane l of a wave owns chunks l, l+64, l+128, ... of every row it reads, so
// a wave-wide 128-bit load covers 1 KB of consecutive row bytes.
//
// Dequantisation happens in registers. A chunk's two's-complement codes are
// flipped to offset binary (xor 0x8 per nibble / 0x80 per byte), widened
// with v_cvt_f32_ubyte*, and dotted with x; the offset is removed once per
// chunk with the precomputed chunk sum of x:
//     sum_k q_k x_k = sum_k u_k x_k - bias * sum_k x_k,  u_k = q_k + bias.
// The chunk result is then scaled by the block's fp16 scale (exact in fp32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nut {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v = fmaxf(v, __shfl_xor(v, offset));
    return v;
}

// DPP cross-lane moves (GFX9 encodings). Rows are groups of 16 lanes.
constexpr int kDppQuadSwap1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v, float fill)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(
        __float_as_int(fill), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// a0 += q_J · k0 and a1 += q_{J+1} · k1, component by component (x, y, z,
// w; a0 then a1 each time, so the rounding is that of the fmaf chain in
// this order), where q_j is the float4 q of lane j of this lane's row of 16
// lanes, read by v_fmac_f32 through a row_newbcast DPP source. Every lane
// of the row must be active. The s_nop covers a VALU write of q just
// before (DPP reads need two wait states after one).
template <int J>
__device__ __forceinline__ void fma_row_bcast2(float &a0, float &a1, float4 q, float4 k0,
                                               float4 k1)
{
    static_assert(J >= 0 && J + 1 < 16, "lanes of a 16-lane row");
    asm volatile("s_nop 1\n\t"
                 "v_fmac_f32_dpp %0, %2, %6 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %1, %2, %10 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %3, %7 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %1, %3, %11 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %4, %8 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %1, %4, %12 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %0, %5, %9 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %1, %5, %13 row_newbcast:%15 row_mask:0xf bank_mask:0xf"
                 : "+v"(a0), "+v"(a1)
                 : "v"(q.x), "v"(q.y), "v"(q.z), "v"(q.w), "v"(k0.x), "v"(k0.y), "v"(k0.z),
                   "v"(k0.w), "v"(k1.x), "v"(k1.y), "v"(k1.z), "v"(k1.w), "i"(J), "i"(J + 1));
}

// Sum over each row of 16 lanes, in every lane of the row.
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp<kDppQuadSwap1>(v, 0.0f);
    v += dpp<kDppQuadSwap2>(v, 0.0f);
    v += dpp<kDppRowHalfMirror>(v, 0.0f);
    v += dpp<kDppRowMirror>(v, 0.0f);
    return v;
}

__device__ __forceinline__ float row16_max(float v)
{
    v = fmaxf(v, dpp<kDppQuadSwap1>(v, -INFINITY));
    v = fmaxf(v, dpp<kDppQuadSwap2>(v, -INFINITY));
    v = fmaxf(v, dpp<kDppRowHalfMirror>(v, -INFINITY));
    v = fmaxf(v, dpp<kDppRowMirror>(v, -INFINITY));
    return v;
}

// Wave-wide sum / max with DPP (rows, then row broadcasts into lane 63),
// returned wave-uniform.
__device__ __forceinline__ float wave_total(float v)
{
    v = row16_sum(v);
    v += dpp<kDppRowBcast15, 0xA>(v, 0.0f);
    v += dpp<kDppRowBcast31, 0xC>(v, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_maximum(float v)
{
    v = row16_max(v);
    v = fmaxf(v, dpp<kDppRowBcast15, 0xA>(v, -INFINITY));
    v = fmaxf(v, dpp<kDppRowBcast31, 0xC>(v, -INFINITY));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over a workgroup of `waves` waves; every thread gets the total.
// `scratch` holds at least `waves` floats of LDS.
__device__ __forceinline__ float block_sum(float v, float *scratch, int waves)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0)
        scratch[wave] = v;
    __syncthreads();
    float total = 0.0f;
    for (int w = 0; w < waves; w++)
        total += scratch[w];
    return total;
}

__device__ __forceinline__ float block_max(float v, float *scratch, int waves)
{
    v = wave_max(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0)
        scratch[wave] = v;
    __syncthreads();
    float m = scratch[0];
    for (int w = 1; w < waves; w++)
        m = fmaxf(m, scratch[w]);
    return m;
}

// fp16 scale bits -> fp32 (exact for every half, subnormals included).
__device__ __forceinline__ float half_bits_to_float(uint16_t bits)
{
    return float(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ float ubyte0(uint32_t v) { return float(v & 0xffu); }
__device__ __forceinline__ float ubyte1(uint32_t v) { return float((v >> 8) & 0xffu); }
__device__ __forceinline__ float ubyte2(uint32_t v) { return float((v >> 16) & 0xffu); }
__device__ __forceinline__ float ubyte3(uint32_t v) { return float(v >> 24); }

// Keeps v opaque to known-bits folding, so byte conversions of a masked
// word stay single v_cvt_f32_ubyte{0..3} instead of a bit-field extract
// per nibble. Emits no instruction.
__device__ __forceinline__ uint32_t opaque(uint32_t v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// sum_k u_k x[k] over one INT4 chunk (32 weights, offset-binary codes).
// Byte b of word j holds weights 8j+2b (low nibble) and 8j+2b+1 (high).
// High nibbles are converted in place (16 u) and their accumulator scaled
// by 1/16 once; power-of-two scaling commutes with rounding, so the result
// equals accumulating u x.
__device__ __forceinline__ float dot_int4_chunk(uint4 w, const float *x)
{
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t lo = opaque((words[j] ^ 0x88888888u) & 0x0f0f0f0fu);
        const uint32_t hi = opaque((words[j] ^ 0x88888888u) & 0xf0f0f0f0u);
        const float *xs = x + 8 * j;
        a0 = fmaf(ubyte0(lo), xs[0], a0);
        a1 = fmaf(ubyte0(hi), xs[1], a1);
        a0 = fmaf(ubyte1(lo), xs[2], a0);
        a1 = fmaf(ubyte1(hi), xs[3], a1);
        a0 = fmaf(ubyte2(lo), xs[4], a0);
        a1 = fmaf(ubyte2(hi), xs[5], a1);
        a0 = fmaf(ubyte3(lo), xs[6], a0);
        a1 = fmaf(ubyte3(hi), xs[7], a1);
    }
    return fmaf(a1, 0.0625f, a0);
}

// sum_k u_k x[k] over one INT8 chunk (16 weights, offset-binary codes).
__device__ __forceinline__ float dot_int8_chunk(uint4 w, const float *x)
{
    const uint32_t words[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u,
                               w.z ^ 0x80808080u, w.w ^ 0x80808080u};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float *xs = x + 4 * j;
        a0 = fmaf(ubyte0(words[j]), xs[0], a0);
        a1 = fmaf(ubyte1(words[j]), xs[1], a1);
        a0 = fmaf(ubyte2(words[j]), xs[2], a0);
        a1 = fmaf(ubyte3(words[j]), xs[3], a1);
    }
    return a0 + a1;
}

// A quantised matrix in HBM: reference layout, data verbatim.
struct QMat {
    const uint8_t *data;
    const uint16_t *scales;
    int rows, cols, block_size, type; // type: 0 INT8, 1 INT4
};

__host__ __device__ __forceinline__ bool fast_layout(const QMat &m)
{
    return m.block_size == 32 && (m.cols & 31) == 0;
}

// Weights per 16-byte chunk.
__host__ __device__ __forceinline__ int chunk_weights(int type)
{
    return type == 1 ? 32 : 16;
}

// Stage x[0..n) into LDS with per-chunk sums (chunk of `cw` weights). Must
// be called by the whole workgroup; ends with a barrier.
__device__ __forceinline__ void stage_x(const float *x, float *xs,
                                        float *xsum, int n, int cw)
{
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        xs[i] = x[i];
    __syncthreads();
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

// Dot products of R consecutive fast-layout rows row0..row0+R-1 with the
// staged x; rows past the end re-read the last row (callers drop them).
// Every lane of the wave returns all R sums.
template <int R>
__device__ __forceinline__ void qrows_fast(const QMat &m, int row0,
                                           const float *xs,
                                           const float *xsum, float (&out)[R])
{
    const int lane = threadIdx.x & (kWave - 1);
    const bool int4 = m.type == 1;
    const int row_bytes = int4 ? m.cols / 2 : m.cols;
    const int chunks = row_bytes / 16;
    const int blocks_per_row = m.cols / 32;
    const float bias = int4 ? 8.0f : 128.0f;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++)
        acc[r] = 0.0f;
    for (int c = lane; c < chunks; c += kWave) {
        uint4 w[R];
        float s[R];
        const int block = int4 ? c : (c >> 1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int rr = min(row0 + r, m.rows - 1);
            const uint8_t *row = m.data + size_t(rr) * row_bytes;
            w[r] = *reinterpret_cast<const uint4 *>(row + 16 * c);
            s[r] = half_bits_to_float(
                m.scales[size_t(rr) * blocks_per_row + block]);
        }
        const float *xc = xs + c * (int4 ? 32 : 16);
        const float xc_sum = xsum[c];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = int4 ? dot_int4_chunk(w[r], xc)
                                 : dot_int8_chunk(w[r], xc);
            acc[r] = fmaf(s[r], d - bias * xc_sum, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
        out[r] = wave_sum(acc[r]);
}

// Any layout (blocks may straddle rows, any block size): one row per call,
// lanes stride over the row's weights. Every lane returns the sum.
__device__ __forceinline__ float qrow_generic(const QMat &m, int row,
                                              const float *xs)
{
    const int lane = threadIdx.x & (kWave - 1);
    const size_t base = size_t(row) * m.cols;
    float acc = 0.0f;
    for (int c = lane; c < m.cols; c += kWave) {
        const size_t i = base + c;
        int q;
        if (m.type == 1) {
            const uint32_t byte = m.data[i >> 1];
            const uint32_t nib = (i & 1) ? (byte >> 4) & 0xfu : byte & 0xfu;
            q = int(nib) - (nib >= 8 ? 16 : 0);
        } else {
            q = int(int8_t(m.data[i]));
        }
        const float scale = half_bits_to_float(m.scales[i / m.block_size]);
        acc = fmaf(float(q) * scale, xs[c], acc);
    }
    return wave_sum(acc);
}

} // namespace nut
