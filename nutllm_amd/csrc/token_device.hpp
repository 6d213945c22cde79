// token_device.hpp — device helpers shared by the cooperative token
// kernels (persistent.hip, wide.hip): tagged exchange words, LDS DMA, x as
// integer digits, and the quantised row dots. Included by HIP sources only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.hpp"
#include "persistent.hpp"

namespace nut {
namespace {

constexpr int kGrid = kTokenGrid;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kSpinLimit = 200000;

constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }

// v as a value the compiler cannot see through: expressions derived from it
// are formed where they are used instead of being hoisted out of enclosing
// loops and kept live in registers.
__device__ __forceinline__ int opaque_lane_value(int v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// ------------------------------------------------------------ exchange --

__device__ __forceinline__ uint64_t load_coherent(const uint64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_coherent(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void put(uint64_t *p, float v, unsigned tag)
{
    __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Write-once words: an exchange that owns its words alone within a step of
// a launch (TokenArgs::x_once: a ring of slices, persistent.hpp) publishes
// plain 32-bit values into words that hold kUnset (set by the host before
// the launch, or re-armed by their producer once every consumer has read
// them). Each word goes from kUnset to its value once per use, so the value
// is its own flag at half the bytes of a tagged word, and a 64-bit poll of
// two words needs no atomicity across them. kUnset is a NaN that put_once
// never writes: it publishes every NaN as the canonical one.
constexpr uint32_t kUnset = 0xffffffffu;

__device__ __forceinline__ void put_once(float *p, float v)
{
    store_coherent(p, v != v ? __uint_as_float(0x7fc00000u) : v);
}

// Re-arming (the ring of write-once slices, persistent.hpp: kOnceRing):
// wave w sets the n <= kWave words at p back to kUnset. The next take's
// closing s_waitcnt vmcnt(0) retires the stores.
__device__ __forceinline__ void rearm_words(float *p, int n, int w)
{
    if (__builtin_amdgcn_readfirstlane(threadIdx.x / kWave) == w) {
        const int lane = threadIdx.x & (kWave - 1);
        if (lane < n)
            store_coherent(p + lane, __uint_as_float(kUnset));
    }
}

__device__ __forceinline__ bool unset_pair(uint64_t w)
{
    return uint32_t(w) == kUnset || uint32_t(w >> 32) == kUnset;
}

__device__ __forceinline__ bool failed(const int *error)
{
    return __hip_atomic_load(error, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// The error flag as seen by thread 0, made uniform over the workgroup so
// every thread takes the same branch.
__device__ __forceinline__ bool wg_failed(const int *error, int *slot)
{
    __syncthreads();
    if (threadIdx.x == 0)
        *slot = failed(error) ? 1 : 0;
    __syncthreads();
    return *slot != 0;
}

__device__ __forceinline__ int wave_index()
{
    return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

// --------------------------------------------------------------- LDS DMA --

// Copy `bytes` (a multiple of 16) from global memory to LDS without
// registers: 1 KB per wave instruction, lane i moving bytes [16i, 16i+16) of
// its kilobyte; instructions are spread over the workgroup's waves.
// Completion: s_waitcnt vmcnt(0) in every wave, then a workgroup barrier.
// The loads carry the non-temporal cache policy (nt, bit 1 of the
// instruction's cache-policy field): each weight byte is read once per token,
// and streaming it leaves the memory-side cache to the fp32 classifier, whose
// rows then partly hit there on the next token (classifier pass 50 -> 44 us
// for the TinyLlama shape).
constexpr int kStreamPolicy = 2;

template <int POLICY = kStreamPolicy>
__device__ __forceinline__ void dma(void *lds_dst, const void *src, int bytes)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int n = (bytes + 1023) >> 10;
    for (int i = wave_index(); i < n; i += kWaves) {
        const int off = (i << 10) + (lane << 4);
        if (off < bytes)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(
                    static_cast<const char *>(src) + off),
                (__attribute__((address_space(3))) void *)(
                    static_cast<char *>(lds_dst) + (i << 10)),
                16, 0, POLICY);
    }
}

__device__ __forceinline__ void dma_wait()
{
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// sc1 (bit 4 of the cache-policy field): the load is coherent at agent
// scope, as the relaxed agent-scope atomic loads of the exchange are
// (gfx950 compiles those to `global_load ... sc1`). K/V cache rows that
// another workgroup stored earlier in the same launch are staged with it:
// those rows were written with agent-scope stores (sc1) from CUs on other
// XCDs, and a load without sc1 may be served by a line that its own XCD's
// L2 or its CU's L1 held before the write. The stores are retired by the
// writer's s_waitcnt vmcnt(0) before its next publish, and the reader issues
// the staging only after it has seen a later publish of that writer, so an
// agent-coherent load returns the stored row.
constexpr int kAgentCoherent = 16;

// Rows [0, n) of 64-float rows at src into LDS rows of 68 floats (16 data
// granules + 1 spare): LDS granule j holds row j / 17, granule j % 17.
// POLICY is the loads' cache policy, which for K/V cache rows includes
// kAgentCoherent: alone where every workgroup of a KV head group stages the
// same rows, with kStreamPolicy where each row is staged by one workgroup
// once per token.
template <int POLICY>
__device__ __forceinline__ void dma_padded_rows(float *lds_dst,
                                                const float *src, int n)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int instrs = (n * 17 + kWave - 1) / kWave;
    for (int i = wave_index(); i < instrs; i += kWaves) {
        const int j = i * kWave + lane;
        const int row = j / 17, g = j - row * 17;
        if (row < n && g < 16)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(
                    src + row * 64 + g * 4),
                (__attribute__((address_space(3))) void *)(
                    reinterpret_cast<char *>(lds_dst) + i * 1024),
                16, 0, POLICY);
    }
}

// --------------------------------------------------------- x staging --

// Element i of x lives at swz(i): quads of each 32-element block are
// rotated by the block index, so lane b reading quad q of block b hits a
// different 16-byte bank group than lanes b+1..b+7.
__device__ __forceinline__ int swz(int i)
{
    const int b = i >> 5, q = (i >> 2) & 7;
    return (b << 5) | (((q + b) & 7) << 2) | (i & 3);
}

// Workgroup sum of per-thread values; every thread gets the total.
__device__ __forceinline__ float wg_sum(float v, float *red)
{
    v = wave_total(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++)
        total += red[w];
    return total;
}

// Block sums of x (swizzled), for the offset-binary float dots.
__device__ void block_sums(const float *xs, float *xsum, int n)
{
    for (int b = threadIdx.x; b < n / 32; b += kThreads) {
        const float4 *base = reinterpret_cast<const float4 *>(xs + (b << 5));
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++)
            s += (base[q].x + base[q].y) + (base[q].z + base[q].w);
        xsum[b] = s;
    }
    __syncthreads();
}

// x of a dim-sized phase as integer digits for the dot instructions. Per
// 32-element block b with m = max |x_k|: X_k = rint(x_k * kLimbRange / m),
// so x_k = xsc[b] * X_k to 2^-23.7 m, and X_k is written as signed digits,
// six of 4 bits (INT4 rows, v_dot8_i32_i4) or three of 8 bits (INT8 rows,
// v_dot4_i32_i8): X_k = sum_d digit_d 16^d (or 256^d). The digits come from
// the offset form: for INT4, X + 0x888888 has hex digits e_d in 0..15 and
// digit_d = e_d - 8, which as a 4-bit two's-complement field is e_d ^ 8, so
// (X + 0x888888) ^ 0x888888 holds the six digits as nibbles (|X| <= 7e6
// keeps X + 0x888888 in 0..2^24); INT8 likewise with 0x808080. Block b's
// kLimbWords words at xl + kLimbStride * b: INT4 word 4 d + j holds digit d
// of elements 8 j .. 8 j + 7 (nibble t = element 8 j + t, the weights'
// nibble order); INT8 word 8 d + j digit d of elements 4 j .. 4 j + 3. A
// NaN or infinity in a block makes xsc[b] NaN.
constexpr float kLimbRange = 7.0e6f;
constexpr int kLimbWords = 24;
constexpr int kLimbStride = 28; // words; lanes b .. b + 15 hit distinct banks

// Digits of quartet q (elements 4 q .. 4 q + 3) of block b, from the lane
// holding it; the block's eight quartets sit in lanes 8 k .. 8 k + 7 of one
// wave (DPP reduces the block maximum), all lanes of the wave take part.
template <int QT>
__device__ __forceinline__ void quartet_digits(float4 v, int b, int q, uint32_t *xl,
                                               float *xsc)
{
    float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    float poison = ((v.x + v.y) + (v.z + v.w)) * 0.0f; // NaN for NaN or inf
    mx = fmaxf(mx, dpp<kDppQuadSwap1>(mx, 0.0f));
    mx = fmaxf(mx, dpp<kDppQuadSwap2>(mx, 0.0f));
    mx = fmaxf(mx, dpp<kDppRowHalfMirror>(mx, 0.0f));
    poison += dpp<kDppQuadSwap1>(poison, 0.0f);
    poison += dpp<kDppQuadSwap2>(poison, 0.0f);
    poison += dpp<kDppRowHalfMirror>(poison, 0.0f);
    // r within an ulp of kLimbRange / mx: x_k = xsc X_k holds to 2^-23
    const float r = mx > 0.0f ? kLimbRange * __builtin_amdgcn_rcpf(mx) : 0.0f;
    if (q == 0)
        xsc[b] = mx * (1.0f / kLimbRange) + poison;
    // X + offset in one FMA (exact below 2^24 up to its rounding) and one
    // conversion: v_cvt_rpi_i32_f32 is floor(v + 0.5)
    constexpr uint32_t kOff = QT == 1 ? 0x888888u : 0x808080u;
    const float xv[4] = {v.x, v.y, v.z, v.w};
    uint32_t y[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int c;
        asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(c) : "v"(fmaf(xv[k], r, float(kOff))));
        y[k] = uint32_t(c) ^ kOff;
    }
    // P[i] = byte i of y[0..3], one per byte
    const uint32_t a01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);
    const uint32_t a23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
    const uint32_t c01 = __builtin_amdgcn_perm(y[1], y[0], 0x0c0c0602u);
    const uint32_t c23 = __builtin_amdgcn_perm(y[3], y[2], 0x0c0c0602u);
    const uint32_t P[3] = {__builtin_amdgcn_perm(a23, a01, 0x05040100u),
                           __builtin_amdgcn_perm(a23, a01, 0x07060302u),
                           __builtin_amdgcn_perm(c23, c01, 0x05040100u)};
    uint32_t *blk = xl + kLimbStride * b;
    if (QT == 1) {
        // digit 2 i is the low nibble of byte i, 2 i + 1 the high one; the
        // quartet is nibbles 4 (q & 1) .. 4 (q & 1) + 3 of word (d, q >> 1)
        uint16_t *half = reinterpret_cast<uint16_t *>(blk + (q >> 1)) + (q & 1);
#pragma unroll
        for (int i = 0; i < 3; i++) {
#pragma unroll
            for (int hi = 0; hi < 2; hi++) {
                const uint32_t n = (hi ? P[i] >> 4 : P[i]) & 0x0f0f0f0fu;
                const uint32_t m = n | (n >> 4); // nibble pairs in bytes 0, 2
                half[2 * 4 * (2 * i + hi)] =
                    uint16_t(__builtin_amdgcn_perm(0u, m, 0x0c0c0200u));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 3; i++)
            blk[8 * i + q] = P[i];
    }
}

// This thread's elements i = threadIdx.x + kThreads * u of an N-vector in
// global memory, in registers; loads issued together (no dependent waits).
template <int N> struct Slice {
    static constexpr int PER = cdiv(N, kThreads);
    float v[PER];
    __device__ __forceinline__ void load(const float *src)
    {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = threadIdx.x + u * kThreads;
            v[u] = i < N ? src[i] : 0.0f;
        }
    }
    // dst[i] = v, returns this thread's sum of squares.
    __device__ __forceinline__ float store(float *dst) const
    {
        float sq = 0.0f;
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = threadIdx.x + u * kThreads;
            if (i < N) {
                dst[i] = v[u];
                sq = fmaf(v[u], v[u], sq);
            }
        }
        return sq;
    }
};

// Digits (quartet_digits) of x = src * scale * w for a dim of 4 kThreads:
// thread t takes elements 4 t .. 4 t + 3, w holding its four weights.
// Ends with a barrier.
template <int QT, int N>
__device__ void stage_x(const float *src, float4 w, float scale, uint32_t *xl,
                        float *xsc)
{
    static_assert(N == 4 * kThreads, "one quartet per thread");
    const float4 h = reinterpret_cast<const float4 *>(src)[threadIdx.x];
    const float4 x = make_float4(h.x * scale * w.x, h.y * scale * w.y, h.z * scale * w.z,
                                 h.w * scale * w.w);
    quartet_digits<QT>(x, threadIdx.x >> 3, threadIdx.x & 7, xl, xsc);
    __syncthreads();
}

__device__ __forceinline__ float rms_scale(float squares, int n)
{
    return 1.0f / sqrtf(squares / float(n) + 1e-5f);
}

// dst[map(i)] = value of src[i] once tagged, i < N; returns this thread's
// sum of squares. The first poll waits DELAY ticks (10 ns) of the real-time
// clock. A thread's loads are issued together, and every round
// re-issues all of its still-stale loads together, so a late producer costs
// one coherent round trip per round rather than one per element. Bounded:
// gives up once any wait failed. Waits for this wave's outstanding DMA, then
// a barrier.
template <int N, bool SWIZZLE, bool FRESH = false, int DELAY = 0>
__device__ float take(const uint64_t *src, float *dst, unsigned tag,
                      int *error)
{
    constexpr int PER = cdiv(N, kThreads);
    const unsigned tid = FRESH ? unsigned(opaque_lane_value(threadIdx.x)) : threadIdx.x;
    if (DELAY > 0) {
        const unsigned long long until = __builtin_amdgcn_s_memrealtime() + DELAY;
        while (__builtin_amdgcn_s_memrealtime() < until)
            __builtin_amdgcn_s_sleep(1);
    }
    uint64_t v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + u * kThreads;
        v[u] = i < N ? load_coherent(src + i) : uint64_t(tag) << 32;
    }
    for (int spins = 0;; spins++) {
        bool stale = false;
#pragma unroll
        for (int u = 0; u < PER; u++)
            stale |= unsigned(v[u] >> 32) != tag;
        if (!stale)
            break;
        if ((spins & 63) == 63 && failed(error))
            break;
        if (spins > kSpinLimit) {
            __hip_atomic_store(error, 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < PER; u++)
            if (unsigned(v[u] >> 32) != tag)
                v[u] = load_coherent(src + tid + u * kThreads);
    }
    float squares = 0.0f;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + u * kThreads;
        if (i < N) {
            const float f = __uint_as_float(unsigned(v[u]));
            dst[SWIZZLE ? swz(i) : i] = f;
            squares = fmaf(f, f, squares);
        }
    }
    dma_wait();
    return squares;
}

// take for write-once words: dst[map(i)] = src[i] once set, i < N (even,
// src 8-byte aligned). Thread t polls the word pairs t, t + kThreads, ...
// as 64-bit loads, re-issuing every pair that still holds kUnset; returns
// this thread's sum of squares. Same delay, bound, FRESH and closing DMA
// wait and barrier as take.
template <int N, bool SWIZZLE, int DELAY = 0, bool FRESH = false>
__device__ float take_once(const float *src, float *dst, int *error)
{
    static_assert(N % 2 == 0, "whole word pairs");
    constexpr int PAIRS = N / 2;
    constexpr int PER = cdiv(PAIRS, kThreads);
    const unsigned tid = FRESH ? unsigned(opaque_lane_value(threadIdx.x)) : threadIdx.x;
    const uint64_t *src2 = reinterpret_cast<const uint64_t *>(src);
    if (DELAY > 0) {
        const unsigned long long until = __builtin_amdgcn_s_memrealtime() + DELAY;
        while (__builtin_amdgcn_s_memrealtime() < until)
            __builtin_amdgcn_s_sleep(1);
    }
    uint64_t v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + u * kThreads;
        v[u] = i < PAIRS ? load_coherent(src2 + i) : 0;
    }
    for (int spins = 0;; spins++) {
        bool stale = false;
#pragma unroll
        for (int u = 0; u < PER; u++)
            stale |= unset_pair(v[u]);
        if (!stale)
            break;
        if ((spins & 63) == 63 && failed(error))
            break;
        if (spins > kSpinLimit) {
            __hip_atomic_store(error, 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < PER; u++)
            if (unset_pair(v[u]))
                v[u] = load_coherent(src2 + tid + u * kThreads);
    }
    float squares = 0.0f;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + u * kThreads;
        if (i < PAIRS) {
            const float lo = __uint_as_float(uint32_t(v[u]));
            const float hi = __uint_as_float(uint32_t(v[u] >> 32));
            // 2i and 2i + 1 share a quad, so they stay adjacent under swz
            *reinterpret_cast<float2 *>(dst + (SWIZZLE ? swz(2 * i) : 2 * i)) =
                make_float2(lo, hi);
            squares = fmaf(lo, lo, squares);
            squares = fmaf(hi, hi, squares);
        }
    }
    dma_wait();
    return squares;
}

// take_once of PARTS partial sums of an N-vector (part k at src + k N) onto
// dst: dst[i] += (p_0[i] + p_1[i]) + ... in part order, the same arithmetic
// in every workgroup; returns this thread's sum of squares of the new dst.
template <int N, int PARTS, int DELAY = 0>
__device__ float take_once_sum(const float *src, float *dst, int *error)
{
    static_assert(N % 2 == 0, "whole word pairs");
    constexpr int PAIRS = N / 2;
    constexpr int PER = cdiv(PAIRS, kThreads);
    const uint64_t *src2 = reinterpret_cast<const uint64_t *>(src);
    if (DELAY > 0) {
        const unsigned long long until = __builtin_amdgcn_s_memrealtime() + DELAY;
        while (__builtin_amdgcn_s_memrealtime() < until)
            __builtin_amdgcn_s_sleep(1);
    }
    uint64_t v[PER][PARTS];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + u * kThreads;
#pragma unroll
        for (int k = 0; k < PARTS; k++)
            v[u][k] = i < PAIRS ? load_coherent(src2 + k * PAIRS + i) : 0;
    }
    for (int spins = 0;; spins++) {
        bool stale = false;
#pragma unroll
        for (int u = 0; u < PER; u++)
#pragma unroll
            for (int k = 0; k < PARTS; k++)
                stale |= unset_pair(v[u][k]);
        if (!stale)
            break;
        if ((spins & 63) == 63 && failed(error))
            break;
        if (spins > kSpinLimit) {
            __hip_atomic_store(error, 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < PER; u++)
#pragma unroll
            for (int k = 0; k < PARTS; k++)
                if (unset_pair(v[u][k]))
                    v[u][k] = load_coherent(src2 + k * PAIRS + threadIdx.x + u * kThreads);
    }
    float squares = 0.0f;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + u * kThreads;
        if (i < PAIRS) {
            float lo = __uint_as_float(uint32_t(v[u][0]));
            float hi = __uint_as_float(uint32_t(v[u][0] >> 32));
#pragma unroll
            for (int k = 1; k < PARTS; k++) {
                lo += __uint_as_float(uint32_t(v[u][k]));
                hi += __uint_as_float(uint32_t(v[u][k] >> 32));
            }
            float2 *h = reinterpret_cast<float2 *>(dst + 2 * i);
            const float2 old = *h;
            lo += old.x;
            hi += old.y;
            *h = make_float2(lo, hi);
            squares = fmaf(lo, lo, squares);
            squares = fmaf(hi, hi, squares);
        }
    }
    dma_wait();
    return squares;
}

// ------------------------------------------------------ quantised rows --

// sum_k u_k x_k over one INT4 block (u = q + 8, offset binary). The high
// nibbles are converted in place (16 u), and their accumulator is scaled by
// 1/16 once: power-of-two scaling commutes with rounding, so the result is
// the same as accumulating u x.
__device__ __forceinline__ float dot_block_int4(const uint4 &w,
                                                const float4 (&x)[8])
{
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t lo = opaque((words[j] ^ 0x88888888u) & 0x0f0f0f0fu);
        const uint32_t hi = opaque((words[j] ^ 0x88888888u) & 0xf0f0f0f0u);
        const float4 xa = x[2 * j], xb = x[2 * j + 1];
        a0 = fmaf(ubyte0(lo), xa.x, a0);
        a1 = fmaf(ubyte0(hi), xa.y, a1);
        a0 = fmaf(ubyte1(lo), xa.z, a0);
        a1 = fmaf(ubyte1(hi), xa.w, a1);
        a0 = fmaf(ubyte2(lo), xb.x, a0);
        a1 = fmaf(ubyte2(hi), xb.y, a1);
        a0 = fmaf(ubyte3(lo), xb.z, a0);
        a1 = fmaf(ubyte3(hi), xb.w, a1);
    }
    return fmaf(a1, 0.0625f, a0);
}

__device__ __forceinline__ float dot_block_int8(const uint4 &w0,
                                                const uint4 &w1,
                                                const float4 (&x)[8])
{
    const uint32_t words[8] = {w0.x ^ 0x80808080u, w0.y ^ 0x80808080u,
                               w0.z ^ 0x80808080u, w0.w ^ 0x80808080u,
                               w1.x ^ 0x80808080u, w1.y ^ 0x80808080u,
                               w1.z ^ 0x80808080u, w1.w ^ 0x80808080u};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        a0 = fmaf(ubyte0(words[j]), x[j].x, a0);
        a1 = fmaf(ubyte1(words[j]), x[j].y, a1);
        a0 = fmaf(ubyte2(words[j]), x[j].z, a0);
        a1 = fmaf(ubyte3(words[j]), x[j].w, a1);
    }
    return a0 + a1;
}

// Wave dot product of a staged row with x (swizzled floats in LDS, block
// sums xsum): per block, offset-binary codes against x minus the bias times
// the block sum, times the block's fp16 scale. Used where x is ffn-sized:
// staging its digits would cost more than the float dot.
template <int QT, int CPL>
__device__ __forceinline__ float row_dot_floats(const uint8_t *row,
                                                const uint16_t *scales,
                                                const float *xs,
                                                const float *xsum, int blocks)
{
    const int lane = threadIdx.x & (kWave - 1);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int b = lane + kWave * j;
        if (b < blocks) {
            float4 xq[8];
            const float4 *base = reinterpret_cast<const float4 *>(xs + (b << 5));
#pragma unroll
            for (int q = 0; q < 8; q++)
                xq[q] = base[(q + b) & 7];
            float d;
            if (QT == 1) {
                d = dot_block_int4(reinterpret_cast<const uint4 *>(row)[b], xq) -
                    8.0f * xsum[b];
            } else {
                const uint4 *p = reinterpret_cast<const uint4 *>(row) + 2 * b;
                d = dot_block_int8(p[0], p[1], xq) - 128.0f * xsum[b];
            }
            acc += half_bits_to_float(scales[b]) * d;
        }
    }
    return wave_total(acc);
}

// One block of a staged row (its two's-complement codes as stored) dotted
// with the block's digits, exactly in integers per digit: every digit sum
// is at most 32 * 7 * 8 (INT4) or 32 * 127 * 128 (INT8) in magnitude, and
// the weighted sums below stay inside int32; the one or two conversions to
// float round once each.
template <int QT>
__device__ __forceinline__ float dot_words_digits(const uint4 *w, const uint4 (&d)[6])
{
    if (QT == 1) {
        const uint32_t ws[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
        int acc[6];
#pragma unroll
        for (int i = 0; i < 6; i++) {
            const uint32_t ds[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
            acc[i] = 0;
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i] = __builtin_amdgcn_sdot8(int(ws[j]), int(ds[j]), acc[i], false);
        }
        const int lo = acc[0] + acc[1] * 16 + acc[2] * 256;
        const int hi = acc[3] + acc[4] * 16 + acc[5] * 256;
        return fmaf(float(hi), 4096.0f, float(lo));
    } else {
        const uint32_t ws[8] = {w[0].x, w[0].y, w[0].z, w[0].w,
                                w[1].x, w[1].y, w[1].z, w[1].w};
        int acc[3];
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const uint32_t ds[8] = {d[2 * i].x, d[2 * i].y, d[2 * i].z, d[2 * i].w,
                                    d[2 * i + 1].x, d[2 * i + 1].y, d[2 * i + 1].z,
                                    d[2 * i + 1].w};
            acc[i] = 0;
#pragma unroll
            for (int j = 0; j < 8; j++)
                acc[i] = __builtin_amdgcn_sdot4(int(ws[j]), int(ds[j]), acc[i], false);
        }
        const int lo = acc[0] + acc[1] * 256;
        return fmaf(float(acc[2]), 65536.0f, float(lo));
    }
}

// As dot_words_digits for block b of a staged row.
template <int QT>
__device__ __forceinline__ float dot_block_digits(const uint8_t *row, int b,
                                                  const uint4 (&d)[6])
{
    const uint4 *p = reinterpret_cast<const uint4 *>(row) + (QT == 1 ? b : 2 * b);
    uint4 w[2];
    w[0] = p[0];
    if (QT != 1)
        w[1] = p[1];
    return dot_words_digits<QT>(w, d);
}

__device__ __forceinline__ void load_digits(const uint32_t *xl, int b, uint4 (&d)[6])
{
    const uint4 *p = reinterpret_cast<const uint4 *>(xl + kLimbStride * b);
#pragma unroll
    for (int i = 0; i < 6; i++)
        d[i] = p[i];
}

// x of one phase held in registers as digits, lane's blocks b = lane + 64 j.
template <int CPL> struct XDigits {
    uint4 d[CPL][6];
    float sc[CPL];
};

template <int CPL>
__device__ __forceinline__ void load_x(XDigits<CPL> &x, const uint32_t *xl,
                                       const float *xsc, int blocks)
{
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int b = lane + kWave * j;
        if (b < blocks) {
            load_digits(xl, b, x.d[j]);
            x.sc[j] = xsc[b];
        }
    }
}

// Wave dot product of a staged row with x in registers; all lanes get it.
// Block b contributes (its fp16 scale) * xsc[b] * (integer block dot).
template <int QT, int CPL>
__device__ __forceinline__ float row_dot(const uint8_t *row,
                                         const uint16_t *scales,
                                         const XDigits<CPL> &x, int blocks)
{
    const int lane = threadIdx.x & (kWave - 1);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int b = lane + kWave * j;
        if (b < blocks)
            acc = fmaf(half_bits_to_float(scales[b]) * x.sc[j],
                       dot_block_digits<QT>(row, b, x.d[j]), acc);
    }
    return wave_total(acc);
}

// As row_dot, reading the digits from LDS (rows swept once per wave).
template <int QT, int CPL>
__device__ __forceinline__ float row_dot_lds(const uint8_t *row,
                                             const uint16_t *scales,
                                             const uint32_t *xl,
                                             const float *xsc, int blocks)
{
    const int lane = threadIdx.x & (kWave - 1);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int b = lane + kWave * j;
        if (b < blocks) {
            uint4 d[6];
            load_digits(xl, b, d);
            acc = fmaf(half_bits_to_float(scales[b]) * xsc[b],
                       dot_block_digits<QT>(row, b, d), acc);
        }
    }
    return wave_total(acc);
}

// Units [begin, end) of `units` owned by this workgroup.
__device__ __forceinline__ void wg_share(int units, int &begin, int &end)
{
    begin = int((long long)units * blockIdx.x / kGrid);
    end = int((long long)units * (blockIdx.x + 1) / kGrid);
}

// ------------------------------------------------------- classifier --

// The fp32 classifier rows of this workgroup (its wg_share of the vocab,
// split over the waves) against x (xs, DIM floats in plain order): the
// wave's best (value, row), the first row on ties (src/generate.cpp:24-30).
template <int DIM, bool FRESH = false>
__device__ __forceinline__ void classifier_best(const float *cls, const float *xs, int vocab,
                                                float &best_v, int &best_i)
{
    const int lane = FRESH ? opaque_lane_value(threadIdx.x & (kWave - 1))
                           : int(threadIdx.x & (kWave - 1));
    const int wave = wave_index();
    constexpr int C4 = DIM / 4 / kWave; // float4 per lane per row
    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
    int rb, re;
    {
        int wb, we;
        wg_share(vocab, wb, we);
        rb = wb + (we - wb) * wave / kWaves;
        re = wb + (we - wb) * (wave + 1) / kWaves;
    }
    best_v = -INFINITY;
    best_i = 0x7fffffff;
    for (int row = rb; row < re; row += 2) {
        const bool two = row + 1 < re;
        const float4 *w0 = reinterpret_cast<const float4 *>(cls + size_t(row) * DIM);
        const float4 *w1 = reinterpret_cast<const float4 *>(cls + size_t(two ? row + 1 : row) * DIM);
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j0 = 0; j0 < C4; j0 += 4) {
            float4 v0[4], v1[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v0[j] = w0[lane + kWave * (j0 + j)];
                v1[j] = w1[lane + kWave * (j0 + j)];
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 x = x4[lane + kWave * (j0 + j)];
                s0 = fmaf(v0[j].x, x.x, s0);
                s0 = fmaf(v0[j].y, x.y, s0);
                s0 = fmaf(v0[j].z, x.z, s0);
                s0 = fmaf(v0[j].w, x.w, s0);
                s1 = fmaf(v1[j].x, x.x, s1);
                s1 = fmaf(v1[j].y, x.y, s1);
                s1 = fmaf(v1[j].z, x.z, s1);
                s1 = fmaf(v1[j].w, x.w, s1);
            }
        }
        s0 = wave_total(s0);
        s1 = wave_total(s1);
        if (s0 > best_v) {
            best_v = s0;
            best_i = row;
        }
        if (two && s1 > best_v) {
            best_v = s1;
            best_i = row + 1;
        }
    }
}

// The fp32 logits of NR classifier rows against x (xs, DIM floats in plain
// order), in every lane: every row's loads are issued before any row's dot,
// so NR rows cost one memory round trip. Per row the arithmetic is
// classifier_best's (lane l: float4 chunks l, l + 64, ... in order, one
// fmaf chain, then the wave sum), so both give the same value for a row.
template <int DIM, bool FRESH, int NR>
__device__ __forceinline__ void classifier_rows(const float *cls, const float *xs,
                                                const int (&row)[NR], float (&out)[NR])
{
    const int lane = FRESH ? opaque_lane_value(threadIdx.x & (kWave - 1))
                           : int(threadIdx.x & (kWave - 1));
    constexpr int C4 = DIM / 4 / kWave;
    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
    float4 v[NR][C4];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const float4 *w = reinterpret_cast<const float4 *>(cls + size_t(row[r]) * DIM);
#pragma unroll
        for (int j = 0; j < C4; j++)
            v[r][j] = w[lane + kWave * j];
    }
    float s[NR];
#pragma unroll
    for (int r = 0; r < NR; r++)
        s[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < C4; j++) {
        const float4 x = x4[lane + kWave * j];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            s[r] = fmaf(v[r][j].x, x.x, s[r]);
            s[r] = fmaf(v[r][j].y, x.y, s[r]);
            s[r] = fmaf(v[r][j].z, x.z, s[r]);
            s[r] = fmaf(v[r][j].w, x.w, s[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++)
        out[r] = wave_total(s[r]);
}

// Rows of the workgroup's classifier share one screened argmax can track:
// an upper bound per row in LDS.
__host__ __device__ constexpr int screened_rows(int vocab)
{
    return (vocab + kGrid - 1) / kGrid;
}

// The screened argmax's input: INT8 digits of x (quartet_digits<0>) in xl
// and xsc, and xl1[b] = sum of |x_k| over block b, for a DIM-vector x in
// LDS. Ends with a barrier.
template <int DIM>
__device__ void screen_x_digits(const float *x, uint32_t *xl, float *xsc, float *xl1)
{
    static_assert(DIM % (4 * kThreads) == 0, "whole quartets per thread");
#pragma unroll
    for (int u = 0; u < DIM / (4 * kThreads); u++) {
        const int t = threadIdx.x + kThreads * u; // quartet t of x
        const float4 v = reinterpret_cast<const float4 *>(x)[t];
        float l1 = (fabsf(v.x) + fabsf(v.y)) + (fabsf(v.z) + fabsf(v.w));
        l1 += dpp<kDppQuadSwap1>(l1, 0.0f);
        l1 += dpp<kDppQuadSwap2>(l1, 0.0f);
        l1 += dpp<kDppRowHalfMirror>(l1, 0.0f);
        if ((t & 7) == 0)
            xl1[t >> 3] = l1;
        quartet_digits<0>(v, t >> 3, t & 7, xl, xsc);
    }
    __syncthreads();
}

// Bound factor of the screened argmax for rows of n weights:
// |s_j - a_j| <= kappa(n) T_j with T_j = sum_b s_jb ||x_b||_1 (s_jb the
// block scales of the INT8 copy, x_b the input's blocks). Terms: the copy's
// rounding, |w - s q| <= s / 2 (the scale rounded up, so no code clamps;
// 2^-10 more for the fp32 quotient); the fp32 rounding of the exact logit,
// gamma_n sum |w_k x_k| <= gamma_n 127 T_j (|w_k| <= 127 s_jb); the digits
// of x, |x_k - xsc X_k| <= 3 xsc_b with xsc_b <= ||x_b||_1 / 7e6, and the
// fp32 sum over blocks (0.0025 covers both); 1 % over all for the fp32
// rounding of T_j and of the block sums of |x|.
__host__ __device__ constexpr float screen_kappa(int n)
{
    return float(1.01 * (0.5 * (1.0 + 1.0 / 1024) + 127.0 * (n * 0x1p-24 / (1.0 - n * 0x1p-24)) +
                         0.0025));
}

// This workgroup's share of the classifier (wg_share of the vocab, split
// over the waves as classifier_best) screened through an INT8 block-32 copy:
// the wave's best (value, row) of the fp32 logits, first row on ties, equal
// to classifier_best's. The copy holds row j as codes q (c8, DIM bytes per
// row) and fp16 block scales s_jb rounded up from max|w| / 127 (c8s). Its
// logit a_j = sum_b s_jb xsc_b (integer block dot of q and the digits of
// x) satisfies |s_j - a_j| <= E_j = screen_kappa(DIM) T_j, s_j the fp32
// logit (classifier_rows), widened by the fp32 rounding of a_j +- E_j. With
// L = max_j (a_j - E_j) over the workgroup's rows and k the row attaining
// it, every row with a_j + E_j < L has s_j <= a_j + E_j < L <= s_k, so only
// the other rows (the candidates, k among them) need their fp32 logits:
// the workgroup reads 2,176 bytes per row instead of 8,192, and a few fp32
// rows. A NaN or infinity anywhere makes the rows concerned candidates.
// xs: x (DIM floats, plain order); xl, xsc, xl1: screen_x_digits of x;
// upper: LDS, screened_rows(vocab) floats; red: LDS, kWaves floats. Ends
// without a barrier: red is read until every wave has passed the candidate
// step. ROWS: rows whose loads a wave issues together (measured: 1 to 4 the
// same for dim 2048; 1 is 6 us per token faster than 4 for dim 4096). CAND:
// candidate rows whose fp32 loads a wave issues together. The candidates
// of one workgroup number 4 at the median but up to two dozen (TinyLlama
// INT4 bench model), and the argmax exchange waits for the workgroup with
// the most, so their rows go in batches of CAND per wave.
template <int DIM, bool FRESH = false, int ROWS = 4, int CAND = 1>
__device__ void classifier_screened(const float *cls, const uint8_t *c8, const uint16_t *c8s,
                                    const float *xs, const uint32_t *xl, const float *xsc,
                                    const float *xl1, int vocab, float *upper, float *red,
                                    float &best_v, int &best_i)
{
    const int lane = FRESH ? opaque_lane_value(threadIdx.x & (kWave - 1))
                           : int(threadIdx.x & (kWave - 1));
    const int wave = wave_index();
    constexpr int BLK = DIM / 32, CPL = BLK / kWave; // blocks per lane
    static_assert(BLK % kWave == 0, "whole blocks per lane");
    int wb, we, rb, re;
    wg_share(vocab, wb, we);
    rb = wb + (we - wb) * wave / kWaves;
    re = wb + (we - wb) * (wave + 1) / kWaves;
    XDigits<CPL> x;
    load_x(x, xl, xsc, BLK);
    float l1[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++)
        l1[j] = xl1[lane + kWave * j];
    constexpr float kappa = screen_kappa(DIM);

    // a_j and T_j of the INT8 copy, ROWS rows at a time; E_j, the lower
    // bounds' max
    float lmax = -INFINITY;
    for (int row = rb; row < re; row += ROWS) {
        uint4 w[ROWS][CPL][2];
        uint16_t sc[ROWS][CPL];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int rr = min(row + r, re - 1);
            const uint4 *p = reinterpret_cast<const uint4 *>(c8 + size_t(rr) * DIM);
#pragma unroll
            for (int j = 0; j < CPL; j++) {
                const int b = lane + kWave * j;
                w[r][j][0] = p[2 * b];
                w[r][j][1] = p[2 * b + 1];
                sc[r][j] = c8s[size_t(rr) * BLK + b];
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            float ap = 0.0f, tp = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; j++) {
                const float s = half_bits_to_float(sc[r][j]);
                ap = fmaf(s * x.sc[j], dot_words_digits<0>(w[r][j], x.d[j]), ap);
                tp = fmaf(s, l1[j], tp);
            }
            if (row + r < re) {
                const float a = wave_total(ap);
                const float t = wave_total(tp);
                // the bound, widened by the rounding of a +- e and floored
                // below the smallest normal scale a logit can carry
                const float e = fmaf(fabsf(a), 0x1p-22f, kappa * t) + 0x1p-120f;
                lmax = fmaxf(lmax, a - e);
                if (lane == 0)
                    upper[row + r - wb] = a + e;
            }
        }
    }
    if (lane == 0)
        red[wave] = lmax;
    __syncthreads();
    float bound = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; w++)
        bound = fmaxf(bound, red[w]);

    // candidates in row order, the c-th to wave c % kWaves; exact logits,
    // CAND rows of a wave at a time (a short last batch repeats its first
    // row, whose duplicate logit changes nothing)
    best_v = -INFINITY;
    best_i = 0x7fffffff;
    int seen = 0, held = 0;
    int rows[CAND];
#pragma unroll
    for (int r = 0; r < CAND; r++)
        rows[r] = wb;
    auto flush = [&]() {
        float v[CAND];
        classifier_rows<DIM, FRESH, CAND>(cls, xs, rows, v);
#pragma unroll
        for (int r = 0; r < CAND; r++)
            if (v[r] > best_v || (v[r] == best_v && rows[r] < best_i)) {
                best_v = v[r];
                best_i = rows[r];
            }
    };
    for (int base = 0; base < we - wb; base += kWave) {
        const int i = base + lane;
        const bool cand = i < we - wb && !(upper[i] < bound);
        unsigned long long mask = __ballot(cand);
        while (mask != 0) {
            const int bit = __builtin_ctzll(mask);
            mask &= mask - 1;
            if (seen % kWaves == wave) {
                const int row = wb + base + bit;
#pragma unroll
                for (int r = 0; r < CAND; r++)
                    if (r == held)
                        rows[r] = row;
                if (held == 0) {
#pragma unroll
                    for (int r = 1; r < CAND; r++)
                        rows[r] = row;
                }
                if (++held == CAND) {
                    flush();
                    held = 0;
                }
            }
            seen++;
        }
    }
    if (held > 0)
        flush();
}

// First-index argmax over the grid from every wave's best (value, row), in
// two calls: argmax_publish puts the workgroup's best as two tagged words
// in x_part (value, then index at x_part + kGrid) and ends on a barrier, so
// that the stores leave before any DMA the caller issues next (the grid
// waits for the last workgroup's publish); argmax_take reduces all kGrid
// partials to the same row in every workgroup. red, misc: LDS, kWaves + 1
// entries each. failed: the error flag (a bounded wait timed out), read
// with the first poll of the partials instead of in a round trip of its
// own, the same value in every thread of the workgroup.
__device__ __forceinline__ void argmax_publish(uint64_t *x_part, float best_v, int best_i,
                                               float *red, int *misc, unsigned tag)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = wave_index();
    if (lane == 0) {
        red[wave] = best_v;
        misc[wave] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = red[0];
        int bi = misc[0];
        for (int w = 1; w < kWaves; w++)
            if (red[w] > bv || (red[w] == bv && misc[w] < bi)) {
                bv = red[w];
                bi = misc[w];
            }
        // the block's best (value, index) as two tagged words
        put(x_part + blockIdx.x, bv, tag);
        put(x_part + kGrid + blockIdx.x, __int_as_float(bi), tag);
    }
    __syncthreads(); // red and misc are read again by argmax_take
}

__device__ __forceinline__ int argmax_take(const uint64_t *x_part, float *red, int *misc,
                                           unsigned tag, int *error, bool &failed_wait)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = wave_index();
    // every workgroup reduces all partials to the same token
    float pv = -INFINITY;
    int pi = 0x7fffffff;
    int err = 0;
    if (threadIdx.x == kGrid)
        err = failed(error) ? 1 : 0;
    if (threadIdx.x < kGrid) {
        // both words of a partial polled together, so the pair costs one
        // round trip once its producer has published
        uint64_t v = load_coherent(x_part + threadIdx.x);
        uint64_t i = load_coherent(x_part + kGrid + threadIdx.x);
        for (int spins = 0; unsigned(v >> 32) != tag || unsigned(i >> 32) != tag; spins++) {
            if ((spins & 63) == 63 && failed(error))
                break;
            if (spins > kSpinLimit) {
                __hip_atomic_store(error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (unsigned(v >> 32) != tag)
                v = load_coherent(x_part + threadIdx.x);
            if (unsigned(i >> 32) != tag)
                i = load_coherent(x_part + kGrid + threadIdx.x);
        }
        pv = __uint_as_float(unsigned(v));
        pi = int(unsigned(i));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(pv, off);
        const int oi = __shfl_xor(pi, off);
        if (ov > pv || (ov == pv && oi < pi)) {
            pv = ov;
            pi = oi;
        }
    }
    __syncthreads();
    if (lane == 0) {
        red[wave] = pv;
        misc[wave] = pi;
    }
    if (threadIdx.x == kGrid)
        misc[kWaves] = err;
    __syncthreads();
    float bv = red[0];
    int bi = misc[0];
    for (int w = 1; w < kWaves; w++)
        if (red[w] > bv || (red[w] == bv && misc[w] < bi)) {
            bv = red[w];
            bi = misc[w];
        }
    failed_wait = misc[kWaves] != 0;
    return bi;
}

} // namespace
} // namespace nut
