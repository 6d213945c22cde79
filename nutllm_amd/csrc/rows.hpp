// rows.hpp — the decode matvec's row dot with x staged in LDS, shared by
// the step kernels and the standalone quantised matvec (matvec_quantized,
// src/quant.cpp:257-321, for 32-wide blocks along whole rows).
//
// A workgroup of kRowThreads threads stages x (times the RMSNorm weights
// when asked) once in LDS; each wave streams R rows with nontemporal
// 16-byte loads (one INT4 block or half an INT8 block per chunk), dots them
// with the staged x chunk, subtracts the offset-binary bias through the x
// chunk sum, and reduces the R row sums with DPP.
#pragma once

#include "device.hpp"

namespace nut {

constexpr int kRowThreads = 256;
constexpr int kRowWaves = kRowThreads / kWave;

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load_stream(const uint8_t *p)
{
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A weight chunk: nontemporal (STREAM, every byte read once) or through the
// caches (rows that other workgroups of the XCD read again).
template <bool STREAM>
__device__ __forceinline__ uint4 load_chunk(const uint8_t *p)
{
    if (STREAM)
        return load_stream(p);
    return *reinterpret_cast<const uint4 *>(p);
}

// Pointers of rows row0 .. row0 + n - 1 of m (rows past the end re-read the
// last row) into slots base .. base + n - 1.
template <int QT, int R>
__device__ __forceinline__ void row_ptrs(const QMat &m, int row0, int base, int n,
                                         const uint8_t *(&rp)[R],
                                         const uint16_t *(&sp)[R])
{
    const int row_bytes = QT == 1 ? m.cols / 2 : m.cols;
    const int bpr = m.cols / 32;
#pragma unroll
    for (int r = 0; r < R; r++)
        if (r >= base && r < base + n) {
            const int rr = min(row0 + r - base, m.rows - 1);
            rp[r] = m.data + size_t(rr) * row_bytes;
            sp[r] = m.scales + size_t(rr) * bpr;
        }
}

// Weights per 16-byte chunk, and floats per chunk of the staged x (padded
// by 4 so that the 16-byte reads of 8 consecutive lanes, one chunk apart,
// fall in distinct LDS banks).
template <int QT> constexpr int chunk_cw() { return QT == 1 ? 32 : 16; }
template <int QT> constexpr int chunk_xs() { return chunk_cw<QT>() + 4; }

// LDS bytes of the staged x of a matvec with `cols` columns.
template <int QT> inline size_t staged_x_bytes(int cols)
{
    return size_t(cols / chunk_cw<QT>()) * chunk_xs<QT>() * sizeof(float);
}

// out[r] = sum_k q_k s x'_k over row r of R rows (pointers rp / sp, `cols`
// columns), x'_k = x_k * nw_k when NORM, then times the RMS factor of x;
// every lane gets all sums. Every wave of the workgroup calls it (`active`
// false for waves without rows): the workgroup stages x' once into LDS (xs,
// staged_x_bytes) and reduces sum x^2 in red[kRowWaves]; each wave issues its
// first weight chunks before the staging, so they load meanwhile. STREAM:
// the weight loads' cache policy (load_chunk).
template <int QT, int R, bool NORM, bool STREAM = true>
__device__ __forceinline__ void rows_matvec(const uint8_t *const (&rp)[R],
                                            const uint16_t *const (&sp)[R], int cols,
                                            const float *x, const float *nw, bool active,
                                            float *xs, float *red, float (&out)[R])
{
    constexpr int CW = chunk_cw<QT>(), XS = chunk_xs<QT>();
    constexpr float kBias = QT == 1 ? 8.0f : 128.0f;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int chunks = cols / CW;
    uint4 w0[R];
    float s0[R];
    const bool first = active && lane < chunks;
    if (first) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            w0[r] = load_chunk<STREAM>(rp[r] + 16 * lane);
            s0[r] = half_bits_to_float(sp[r][QT == 1 ? lane : lane >> 1]);
        }
    }
    float sq = 0.0f;
    for (int i = threadIdx.x * 4; i < cols; i += kRowThreads * 4) {
        float4 v = *reinterpret_cast<const float4 *>(x + i);
        if (NORM) {
            const float4 g = *reinterpret_cast<const float4 *>(nw + i);
            sq = fmaf(v.x, v.x, sq);
            sq = fmaf(v.y, v.y, sq);
            sq = fmaf(v.z, v.z, sq);
            sq = fmaf(v.w, v.w, sq);
            v.x *= g.x;
            v.y *= g.y;
            v.z *= g.z;
            v.w *= g.w;
        }
        *reinterpret_cast<float4 *>(xs + (i / CW) * XS + i % CW) = v;
    }
    if (NORM) {
        sq = wave_total(sq);
        if (lane == 0)
            red[wave] = sq;
    }
    __syncthreads();
    float scale = 1.0f;
    if (NORM) {
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < kRowWaves; w++)
            total += red[w];
        scale = 1.0f / sqrtf(total / float(cols) + 1e-5f);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++)
        acc[r] = 0.0f;
    auto chunk = [&](int c, const uint4 (&w)[R], const float (&s)[R]) {
        float xc[CW];
        const float4 *x4 = reinterpret_cast<const float4 *>(xs + c * XS);
#pragma unroll
        for (int q = 0; q < CW / 4; q++) {
            const float4 v = x4[q];
            xc[4 * q] = v.x;
            xc[4 * q + 1] = v.y;
            xc[4 * q + 2] = v.z;
            xc[4 * q + 3] = v.w;
        }
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < CW; i++)
            xsum += xc[i];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = QT == 1 ? dot_int4_chunk(w[r], xc) : dot_int8_chunk(w[r], xc);
            acc[r] = fmaf(s[r], d - kBias * xsum, acc[r]);
        }
    };
    if (first)
        chunk(lane, w0, s0);
    if (active)
        for (int c = lane + kWave; c < chunks; c += kWave) {
            uint4 w[R];
            float s[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                w[r] = load_chunk<STREAM>(rp[r] + 16 * c);
                s[r] = half_bits_to_float(sp[r][QT == 1 ? c : c >> 1]);
            }
            chunk(c, w, s);
        }
#pragma unroll
    for (int r = 0; r < R; r++)
        out[r] = wave_total(acc[r]) * scale;
}

} // namespace nut
