// prefill.hip — the prompt as a batch: prefill_quantized
// (src/quant_model.cpp:208-220) computes, token after token, the decode
// step of src/quant_model.cpp:158-206; this file computes the same function
// for all T prompt tokens at once, layer by layer, in six launches:
//   rmsnorm rows -> Q/K/V GEMM (epilogue: RoPE, q, the KV-cache rows and
//   the attention's K/V limbs) -> causal attention -> Wo GEMM (+ residual)
//   -> rmsnorm rows -> gate/up GEMM (epilogue: silu(gate) * up as limbs)
//   -> W2 GEMM (+ residual)
// The quantised GEMMs run on f16 MFMA with the weight codes exact in f16,
// the activations split into two f16 limbs and the block scales applied
// in fp32 per 32-wide block; attention runs on f16 MFMA with its operands
// as f16 limbs, three products per term. The hidden state stays within
// about 1e-5 of the per-token path (fp32 throughout).
#include "prefill.hpp"
#include "runtime.hpp"

#include <type_traits>

namespace nut {

namespace {

constexpr int kThreads = 256;
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ rows --

__global__ __launch_bounds__(kThreads) void embed_rows_kernel(
    const float *embeddings, const int *tokens, float *h, int dim)
{
    const float *e = embeddings + size_t(tokens[blockIdx.x]) * dim;
    float *out = h + size_t(blockIdx.x) * dim;
    for (int i = threadIdx.x; i < dim; i += kThreads)
        out[i] = e[i];
}

// out[t] = h[t] * (1 / sqrt(mean(h[t]^2) + 1e-5)) * w  (src/ops.cpp:111-134)
// An activation the GEMMs read as two f16 limbs: hi = f16(v), lo =
// f16(v - hi), so hi + lo carries v to about 2^-22 relative.
// v as an fp32 value in a register, opaque to the optimiser: otherwise the
// multiply that produced v may be folded into either conversion (fma_mix
// from the unrounded product) but not the other, and hi + lo then misses v
// by an f16 ulp where the two roundings part (measured: rel-L2 5e-5 on the
// K/V rows of a batched prefill instead of 5e-7).
__device__ __forceinline__ float settle(float v)
{
    asm("" : "+v"(v));
    return v;
}

__device__ __forceinline__ void put_limbs(_Float16 *hi, _Float16 *lo, size_t i, float v)
{
    v = settle(v);
    const _Float16 a = (_Float16)v;
    hi[i] = a;
    lo[i] = (_Float16)(v - (float)a);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// put_limbs of four consecutive values, i a multiple of 4: one 8-byte store
// per limb.
__device__ __forceinline__ void put_limbs4(_Float16 *hi, _Float16 *lo, size_t i, float4 v)
{
    v = make_float4(settle(v.x), settle(v.y), settle(v.z), settle(v.w));
    half4v a, b;
    a.x = (_Float16)v.x;
    a.y = (_Float16)v.y;
    a.z = (_Float16)v.z;
    a.w = (_Float16)v.w;
    b.x = (_Float16)(v.x - (float)a.x);
    b.y = (_Float16)(v.y - (float)a.y);
    b.z = (_Float16)(v.z - (float)a.z);
    b.w = (_Float16)(v.w - (float)a.w);
    *reinterpret_cast<half4v *>(hi + i) = a;
    *reinterpret_cast<half4v *>(lo + i) = b;
}

// put_limbs of two consecutive values, i even: one 4-byte store per limb.
__device__ __forceinline__ void put_limbs2(_Float16 *hi, _Float16 *lo, size_t i, float2 v)
{
    v = make_float2(settle(v.x), settle(v.y));
    half2v a, b;
    a.x = (_Float16)v.x;
    a.y = (_Float16)v.y;
    b.x = (_Float16)(v.x - (float)a.x);
    b.y = (_Float16)(v.y - (float)a.y);
    *reinterpret_cast<half2v *>(hi + i) = a;
    *reinterpret_cast<half2v *>(lo + i) = b;
}

// float4s of a row each thread keeps in registers between the sum of
// squares and the scaling: rows up to 4,096 wide are read from memory once
// (wider rows read their remainder twice).
constexpr int kRowVecs = 4;

// One workgroup per token row; dim % 4 == 0.
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(
    const float *h, const float *w, _Float16 *out_hi, _Float16 *out_lo, int dim)
{
    __shared__ float red[kThreads / kWave];
    const float4 *x = reinterpret_cast<const float4 *>(h + size_t(blockIdx.x) * dim);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    const int n4 = dim / 4;
    float4 v[kRowVecs];
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < kRowVecs; j++) {
        const int i = threadIdx.x + kThreads * j;
        v[j] = i < n4 ? x[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < kRowVecs; j++) {
        sq = fmaf(v[j].x, v[j].x, sq);
        sq = fmaf(v[j].y, v[j].y, sq);
        sq = fmaf(v[j].z, v[j].z, sq);
        sq = fmaf(v[j].w, v[j].w, sq);
    }
    for (int i = threadIdx.x + kThreads * kRowVecs; i < n4; i += kThreads) {
        const float4 u = x[i];
        sq = fmaf(u.x, u.x, sq);
        sq = fmaf(u.y, u.y, sq);
        sq = fmaf(u.z, u.z, sq);
        sq = fmaf(u.w, u.w, sq);
    }
    const float total = block_sum(sq, red, kThreads / kWave);
    const float scale = 1.0f / sqrtf(total / float(dim) + 1e-5f);
    const size_t row = size_t(blockIdx.x) * dim;
    auto put = [&](int i, float4 u) {
        const float4 g = w4[i];
        put_limbs4(out_hi, out_lo, row + 4 * size_t(i),
                   make_float4(u.x * scale * g.x, u.y * scale * g.y, u.z * scale * g.z,
                               u.w * scale * g.w));
    };
#pragma unroll
    for (int j = 0; j < kRowVecs; j++) {
        const int i = threadIdx.x + kThreads * j;
        if (i < n4)
            put(i, v[j]);
    }
    for (int i = threadIdx.x + kThreads * kRowVecs; i < n4; i += kThreads)
        put(i, x[i]);
}

// ------------------------------------- quantised GEMM on f16 MFMA --

// C[t][n] (= or +=) sum_k X[t][k] W[n][k], W quantised (block 32 along k,
// k % 32 == 0), on v_mfma_f32_16x16x32_f16, whose K = 32 is one quant
// block:
//   * W codes q (INT4 -8..7, INT8 -128..127) are exact in f16;
//   * X arrives as two f16 limbs, hi = f16(x) and lo = f16(x - hi), so
//     hi + lo carries x to about 2^-22 relative (f16 subnormals aside),
//     written by the kernel that produces X (put_limbs);
//   * every product of two f16 values is exact in the fp32 accumulator;
//   * per block, D = A_hi B + A_lo B, then acc += s_n D with the block's
//     fp16 scale s_n (one column n per lane in the D layout).
// A workgroup owns 64 tokens x 128 outputs; its four compute waves each
// multiply all 64 tokens by 32 outputs, and the operands of each 64-wide k
// stage reach LDS by DMA into a three-slot ring (qgemm_f16_kernel below).
// Lane layout (measured): A[i][k] in lane i % 16 + 16 g holding
// k = 8 g .. 8 g + 7; B[k][n] likewise with n = lane % 16; D[i][n] in
// lane n + 16 (i / 4), element i % 4.
constexpr int FM_ROWS = 64, FN = 128, FK = 32;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Two quantisation codes as two f16 (exact): an offset-binary code u sits
// in the low byte of an f16 whose high byte is 0x64, which is the value
// 1024 + u; subtracting 1024 + bias gives the code. `pair` holds such a
// word for two codes.
__device__ __forceinline__ uint32_t codes_from_pair(uint32_t pair, float bias)
{
    const half2v v = __builtin_bit_cast(half2v, pair) -
                     half2v{(_Float16)(1024.0f + bias), (_Float16)(1024.0f + bias)};
    return __builtin_bit_cast(uint32_t, v);
}

// Stage-major scales: dword [st][row] = the fp16 scales of blocks 2 st and
// 2 st + 1 of row `row` (the dword at row * stages + st of the row-major
// scales).
__global__ __launch_bounds__(kThreads) void scales_by_stage_kernel(const uint32_t *src,
                                                                  uint32_t *dst, int rows,
                                                                  int stages)
{
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= size_t(rows) * stages)
        return;
    const int st = int(i / rows), row = int(i % rows);
    dst[i] = src[size_t(row) * stages + st];
}

// Up to three matrices sharing X and k (Q/K/V, or gate/up) in one launch:
// column tiles of FN outputs are numbered across the segments in order.
struct GemmSegs {
    QMat w[3];
    const uint32_t *st[3]; // stage-major scales (launch_scales_by_stage)
    float *c[3];
    int ldc[3];
    int tiles[3];
    int count;
    // SwiGLU launches: w[0] gate, w[1] up; silu(gate) * up as limbs
    _Float16 *act_hi, *act_lo;
    int act_ld;
    // Q/K/V launches (segments q, k, v): RoPE table [pos][hd / 2] (cos,
    // sin); the layer's cache [kv_head][max_seq][hd]; the batch's K and V
    // as f16 limbs, K [kv_head][t_pad][hd], V transposed [kv_head][hd][t_pad]
    const float2 *rope;
    float *k_cache, *v_cache;
    _Float16 *k_hi, *k_lo, *vt_hi, *vt_lo;
    int hd, max_seq, t_pad;
};

// What a GEMM launch does with its products: store, add to C (residual),
// silu(gate) * up as limbs, or RoPE + K/V cache and limb stores.
enum Epilogue { kEpiStore = 0, kEpiAdd = 1, kEpiSwiglu = 2, kEpiQkv = 3 };

// Source row of tile row r (0 .. 127) and its matrix (0 or 1): row n0 + r
// of the segment's matrix; for a SwiGLU tile, gate and up rows alternate in
// groups of 16 (tile rows 32 v .. 32 v + 15 are gate rows n0 + 16 v + i,
// tile rows 32 v + 16 .. 32 v + 31 the up rows of the same outputs), so
// that a wave's two 16-row MFMA tiles hold gate and up of one output
// column in the same lane.
template <bool SWIGLU>
__device__ __forceinline__ int tile_row_source(int r, int n0, int &mat)
{
    if (SWIGLU) {
        mat = (r >> 4) & 1;
        return n0 + 16 * (r >> 5) + (r & 15);
    }
    mat = 0;
    return n0 + r;
}

// ------------------------------------------------------ quantised GEMM --

// C[t][n] (+)= sum_k x[t][k] q[n][k] s[n][k / 32] for a 64-token x 128-row
// tile per workgroup, one 64-wide k stage (two quant blocks) per step.
// Operands reach LDS by DMA (global_load_lds_dwordx4) into a ring of
// kStages stages, so one stage loads while one is multiplied and no
// register holds them in flight. Per stage: x_hi and x_lo (64 rows x 128 B
// each, whole 128-byte lines; the eight 16-byte granules of a row
// XOR-swizzled by row & 7 so that the A-fragment reads of 8 consecutive rows
// hit distinct banks), the weight bytes (128 rows x 64 B for INT8, x 32 B
// for INT4; granules swizzled by (row >> 1) & 3 and (row >> 2) & 1) and the
// dword of each row's scales holding the stage's two fp16 scales. A stage
// costs the L2 one request per x row and limb, one per weight row and one
// per scale dword: the L2 request rate, not its bandwidth, bounded the
// 32-wide version.
// Wave w multiplies all 64 tokens by rows [32 w, 32 w + 32): 4 x 2 tiles
// of v_mfma_f32_16x16x32_f16 per block, A = x limbs (hi and lo, two MFMAs
// per tile), B = the codes, dequantised exactly into f16 from the wave's
// own rows; then acc += s_n * D per tile and block. Lane layouts (checked
// on the device): A[i][k]: lane i % 16 + 16 g holds k = 8 g .. 8 g + 7;
// B[k][n]: lane n % 16 + 16 g the same k; D[i][n]: lane n + 16 (i / 4),
// element i % 4.
constexpr int kStages = 3;
constexpr int kDmaPerWave = 7; // DMA instructions per wave per stage
constexpr int FS = 2 * FK;     // k per stage

template <int QT> struct GemmSlot {
    uint4 xh[FM_ROWS * 8];
    uint4 xl[FM_ROWS * 8];
    uint4 w[QT == 1 ? 2 * FN : 4 * FN];
    uint32_t sc[FN];
};

// LDS address (byte offset) of a generic pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return uint32_t(reinterpret_cast<uintptr_t>(
        (const __attribute__((address_space(3))) char *)(p)));
}

// LDS DMA of 16 (or 4) bytes per lane to LDS byte address m0 + 16 (or 4) *
// lane, written as asm: the compiler then neither tracks the DMA (it would
// wait for all of it before any LDS read, as it cannot tell the ring slots
// apart) nor moves memory operations across it. m0 is wave-uniform (an
// SGPR), formed once per kernel: recomputing it from a pointer at every
// issue cost each wave-stage about 20 VALU and 30 SALU instructions.
__device__ __forceinline__ void dma16(const void *src, uint32_t m0)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(m0)
                 : "memory", "m0");
}

__device__ __forceinline__ void dma4(const void *src, uint32_t m0)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(src), "s"(m0)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(n) then s_barrier, as one compiler-level memory fence
// (no workgroup fence: that would wait for every DMA in flight).
template <int N> __device__ __forceinline__ void wait_dma_barrier()
{
    static_assert(N == 7, "the ring keeps one stage (seven DMA per wave) in flight");
    asm volatile("s_waitcnt vmcnt(7)\n\ts_barrier" ::: "memory");
}

// Eight codes (k = 8 g .. 8 g + 7 of one row) as f16: INT8 from 8 bytes,
// INT4 from 4 bytes (even k in the low nibble).
template <int QT>
__device__ __forceinline__ half8 codes8(uint2 raw)
{
    uint32_t out[4];
    if (QT == 1) {
        const uint32_t t = raw.x ^ 0x88888888u, s4 = t >> 4;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t sel = 0x0c000c00u | uint32_t(4 + b) << 16 | uint32_t(b);
            out[b] = codes_from_pair((__builtin_amdgcn_perm(s4, t, sel) & 0x000f000fu) |
                                         0x64006400u,
                                     8.0f);
        }
    } else {
        const uint32_t words[2] = {raw.x, raw.y};
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t t = words[j] ^ 0x80808080u;
            out[2 * j] = codes_from_pair(__builtin_amdgcn_perm(0x64646464u, t, 0x04010400u), 128.0f);
            out[2 * j + 1] =
                codes_from_pair(__builtin_amdgcn_perm(0x64646464u, t, 0x04030402u), 128.0f);
        }
    }
    return __builtin_bit_cast(half8, make_uint4(out[0], out[1], out[2], out[3]));
}

// The loader wave of qgemm_f16_kernel<QT, EPI, true>: it issues every DMA
// instruction of a stage (x_hi and x_lo rows 8 i .. 8 i + 7, i < 8; the
// weight rows, 16 (INT8) or 32 (INT4) per instruction; the scale dwords of
// rows 64 i + lane, i < 2) into the three-slot ring, and meets the compute
// waves at one barrier per stage, once stage s has landed (stage s + 1
// stays in flight), after which stage s + 2 goes into the slot of s - 1.
template <int QT, bool SWIGLU>
__device__ __forceinline__ void qgemm_loader(const _Float16 *x_hi, const _Float16 *x_lo,
                                             int t_count, const QMat &w, const QMat &w_up,
                                             const uint32_t *st, const uint32_t *st_up,
                                             int t0, int n0, GemmSlot<QT> *const (&slot)[kStages])
{
    constexpr int NW = QT == 1 ? 4 : 8; // weight instructions per stage
    constexpr int D = 16 + NW + 2;      // DMA instructions per stage
    constexpr int W_ROWS = QT == 1 ? 32 : 16;
    constexpr int W_STEP = QT == 1 ? FS / 2 : FS;
    const int lane = threadIdx.x & (kWave - 1);
    const int k = w.cols, n_count = w.rows, stages = k / FS;
    const size_t row_bytes = QT == 1 ? size_t(k) / 2 : size_t(k);
    size_t xoff[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int row = 8 * i + (lane >> 3);
        const int cg = (lane & 7) ^ (row & 7);
        xoff[i] = size_t(min(t0 + row, t_count - 1)) * k + 8 * cg;
    }
    const char *wsrc[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) {
        const int row = W_ROWS * i + (QT == 1 ? lane >> 1 : lane >> 2);
        const int cg = QT == 1 ? (lane & 1) ^ ((row >> 2) & 1) : (lane & 3) ^ ((row >> 1) & 3);
        int mat;
        const int src = tile_row_source<SWIGLU>(row, n0, mat);
        wsrc[i] = reinterpret_cast<const char *>(mat ? w_up.data : w.data) +
                  size_t(min(src, n_count - 1)) * row_bytes + 16 * cg;
    }
    const uint32_t *ssrc[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        int mat;
        const int src = tile_row_source<SWIGLU>(kWave * i + lane, n0, mat);
        ssrc[i] = (mat ? st_up : st) + min(src, n_count - 1);
    }
    uint32_t mb[kStages];
#pragma unroll
    for (int r = 0; r < kStages; r++)
        mb[r] = __builtin_amdgcn_readfirstlane(lds_addr(slot[r]));
    auto issue = [&](int r, int s) {
        s = min(s, stages - 1); // past the end: reload the last stage
        const size_t xs = size_t(s) * FS, ws = size_t(s) * W_STEP;
#pragma unroll
        for (int i = 0; i < 8; i++)
            dma16(x_hi + xoff[i] + xs, mb[r] + offsetof(GemmSlot<QT>, xh) + 1024 * i);
#pragma unroll
        for (int i = 0; i < 8; i++)
            dma16(x_lo + xoff[i] + xs, mb[r] + offsetof(GemmSlot<QT>, xl) + 1024 * i);
#pragma unroll
        for (int i = 0; i < NW; i++)
            dma16(wsrc[i] + ws, mb[r] + offsetof(GemmSlot<QT>, w) + 1024 * i);
#pragma unroll
        for (int i = 0; i < 2; i++)
            dma4(ssrc[i] + size_t(s) * n_count, mb[r] + offsetof(GemmSlot<QT>, sc) + 256 * i);
    };
    issue(0, 0);
    issue(1, 1);
    for (int s0 = 0; s0 < stages; s0 += kStages) {
#pragma unroll
        for (int r = 0; r < kStages; r++) {
            if (s0 + r < stages) {
                asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(D) : "memory");
                issue((r + 2) % kStages, s0 + r + 2);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // no DMA outlives the workgroup
}

// LOADER: a fifth wave issues all of a stage's DMA (qgemm_loader) and the
// four compute waves issue none. For grids of at most one workgroup per CU
// (the 7B shape's Wo and W2 at 512 tokens: 256 workgroups), where no second
// workgroup runs while a wave stalls on its own DMA issue: Wo 58.0 ->
// 53.1 us, W2 144-147 -> 130-134 us (alternated on one box). With two
// workgroups per CU it is slower (TinyLlama gate/up at 2,048 tokens: 256 ->
// 292 us).
// EPI (Epilogue): kEpiSwiglu tiles hold gate and up rows of 64 outputs
// (tile_row_source) and write silu(gate) * up as limbs (act_hi, act_lo)
// instead of the two products; kEpiQkv rotates q and k (RoPE), stores q,
// puts k and v rows into the cache and their limbs into the attention's
// K / V operands (zeros for the padding positions t_count .. t_pad - 1).
template <int QT, int EPI, bool LOADER>
__global__ __launch_bounds__(LOADER ? kThreads + kWave : kThreads) void qgemm_f16_kernel(
    const _Float16 *__restrict__ x_hi, const _Float16 *__restrict__ x_lo, int t_count,
    GemmSegs segs)
{
    constexpr bool SWIGLU = EPI == kEpiSwiglu, ADD = EPI == kEpiAdd;
    __shared__ GemmSlot<QT> slot[kStages];
    __shared__ uint32_t junk[kWave];
    int seg = 0, tile = blockIdx.x;
    while (seg + 1 < segs.count && tile >= segs.tiles[seg])
        tile -= segs.tiles[seg++]; // workgroup-uniform
    const QMat w = segs.w[seg];
    float *__restrict__ c = segs.c[seg];
    const int ldc = segs.ldc[seg];
    // the wave index as a scalar, so that every LDS address derived from it
    // stays in SGPRs
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    // first output of the tile (SWIGLU: 64 outputs, 128 rows)
    const int t0 = blockIdx.y * FM_ROWS, n0 = tile * (SWIGLU ? FN / 2 : FN);
    const int k = w.cols, n_count = w.rows, stages = k / FS;
    const size_t row_bytes = QT == 1 ? size_t(k) / 2 : size_t(k);
    const QMat &w_up = segs.w[SWIGLU ? 1 : 0];
    const uint32_t *const st_up = segs.st[SWIGLU ? 1 : 0];
    if constexpr (LOADER) {
        if (wave == kThreads / kWave) {
            GemmSlot<QT> *const slots[kStages] = {&slot[0], &slot[1], &slot[2]};
            qgemm_loader<QT, SWIGLU>(x_hi, x_lo, t_count, w, w_up, segs.st[seg], st_up, t0, n0,
                                     slots);
            return;
        }
    }

    // The wave's seven DMA instructions of a stage (every wave issues
    // seven, so one vmcnt value covers every wave): x_hi and x_lo
    // instructions 2 wave and 2 wave + 1 (8 rows each: row 8 i + lane / 8,
    // granule lane % 8); INT8 weight instructions 2 wave and 2 wave + 1
    // (16 rows each) and, for waves 0-1, the scale instructions; INT4:
    // waves 0-1 the four weight instructions (32 rows each), waves 2-3 the
    // two scale instructions; fillers into `junk` make up the seven. Source
    // pointers are at stage 0.
    // x rows of instructions 2 wave and 2 wave + 1
    auto x_src = [&](const _Float16 *x, int i) {
        const int row = 8 * i + (lane >> 3);
        const int cg = (lane & 7) ^ (row & 7);
        return reinterpret_cast<const char *>(x + size_t(min(t0 + row, t_count - 1)) * k +
                                              8 * cg);
    };
    const int xi0 = 2 * wave, xi1 = 2 * wave + 1;
    const char *const xh0 = x_src(x_hi, xi0), *const xh1 = x_src(x_hi, xi1);
    const char *const xl0 = x_src(x_lo, xi0), *const xl1 = x_src(x_lo, xi1);
    // weight rows: INT8 16 per instruction (instructions 2 wave, 2 wave + 1),
    // INT4 32 per instruction (waves 0-1 only)
    constexpr int W_ROWS = QT == 1 ? 32 : 16;
    auto w_src = [&](int i) {
        const int row = W_ROWS * i + (QT == 1 ? lane >> 1 : lane >> 2);
        const int cg = QT == 1 ? (lane & 1) ^ ((row >> 2) & 1) : (lane & 3) ^ ((row >> 1) & 3);
        int mat;
        const int src = tile_row_source<SWIGLU>(row, n0, mat);
        return reinterpret_cast<const char *>(mat ? w_up.data : w.data) +
               size_t(min(src, n_count - 1)) * row_bytes + 16 * cg;
    };
    const char *const w0 = w_src(xi0), *const w1 = w_src(xi1);
    // scale dwords of rows 64 si + lane (stage-major: consecutive rows are
    // consecutive dwords): INT8 waves 0-1, INT4 waves 2-3
    const bool scales = QT == 1 ? wave >= 2 : wave < 2; // wave-uniform
    const int si = QT == 1 ? wave - 2 : wave;
    int s_mat;
    const int s_row = tile_row_source<SWIGLU>(kWave * max(si, 0) + lane, n0, s_mat);
    const char *const s0 = reinterpret_cast<const char *>(
        (s_mat ? st_up : segs.st[seg]) + min(s_row, n_count - 1));
    const size_t s_step = size_t(n_count) * 4; // bytes per stage
    const char *const filler = reinterpret_cast<const char *>(x_hi);
    constexpr int W_STEP = QT == 1 ? FS / 2 : FS; // weight bytes per row and stage
    // LDS destinations (m0 values) of the wave's DMA, per ring slot
    struct SlotM0 {
        uint32_t xh0, xh1, xl0, xl1, w0, w1, sc;
    };
    auto slot_m0 = [&](GemmSlot<QT> &sl) {
        SlotM0 m;
        m.xh0 = __builtin_amdgcn_readfirstlane(lds_addr(&sl.xh[kWave * xi0]));
        m.xh1 = __builtin_amdgcn_readfirstlane(lds_addr(&sl.xh[kWave * xi1]));
        m.xl0 = __builtin_amdgcn_readfirstlane(lds_addr(&sl.xl[kWave * xi0]));
        m.xl1 = __builtin_amdgcn_readfirstlane(lds_addr(&sl.xl[kWave * xi1]));
        // INT4 weight instructions exist in waves 0-1 only (xi1 <= 3)
        const bool w_here = QT == 0 || !scales;
        m.w0 = w_here ? __builtin_amdgcn_readfirstlane(lds_addr(&sl.w[kWave * xi0])) : 0u;
        m.w1 = w_here ? __builtin_amdgcn_readfirstlane(lds_addr(&sl.w[kWave * xi1])) : 0u;
        m.sc = scales ? __builtin_amdgcn_readfirstlane(lds_addr(&sl.sc[kWave * si])) : 0u;
        return m;
    };
    const SlotM0 m_slot[kStages] = {slot_m0(slot[0]), slot_m0(slot[1]), slot_m0(slot[2])};
    const uint32_t m_junk = __builtin_amdgcn_readfirstlane(lds_addr(&junk[0]));
    auto issue = [&](int slot, int st) {
        const SlotM0 &m = m_slot[slot];
        st = min(st, stages - 1); // past the end: reload the last stage
        const size_t xs = size_t(st) * (FS * 2), ws = size_t(st) * W_STEP;
        dma16(xh0 + xs, m.xh0);
        dma16(xh1 + xs, m.xh1);
        dma16(xl0 + xs, m.xl0);
        dma16(xl1 + xs, m.xl1);
        if (QT == 0) {
            dma16(w0 + ws, m.w0);
            dma16(w1 + ws, m.w1);
            if (scales)
                dma4(s0 + size_t(st) * s_step, m.sc);
            else
                dma4(filler, m_junk);
        } else {
            if (scales) {
                dma4(s0 + size_t(st) * s_step, m.sc);
                dma4(filler, m_junk);
            } else {
                dma16(w0 + ws, m.w0);
                dma16(w1 + ws, m.w1);
            }
            dma4(filler, m_junk);
        }
    };

    // acc += s D per block; the second block's D of a stage waits in pend
    // (with its scales in psc) and is added at the start of the next stage,
    // under that stage's LDS reads instead of after the stage's last MFMA.
    // The order of the additions into acc is unchanged.
    floatx4 acc[4][2], pend[4][2];
    float psc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            pend[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    auto add_pending = [&]() {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    acc[i][j][v] = fmaf(psc[j], pend[i][j][v], acc[i][j][v]);
    };
    const int g = lane >> 4, li = lane & 15;
    const int n_lane = 32 * wave + li;
    // Fragment byte offsets in a slot (the swizzles depend on li only):
    // A of row 16 i + li, block b: granule (4 b + g) ^ (li & 7) of the row;
    // B of row n_lane + 16 j, block b.
    auto a_off = [&](int b) { return 128 * li + 16 * ((4 * b + g) ^ (li & 7)); };
    auto b_off = [&](int b) {
        return QT == 1 ? 32 * n_lane + 16 * (b ^ ((li >> 2) & 1)) + 4 * g
                       : 64 * n_lane + 16 * ((2 * b + (g >> 1)) ^ ((li >> 1) & 3)) + 8 * (g & 1);
    };
    auto stage_mma = [&](const GemmSlot<QT> &sl) {
        const char *xh = reinterpret_cast<const char *>(sl.xh);
        const char *xl = reinterpret_cast<const char *>(sl.xl);
        const char *wb = reinterpret_cast<const char *>(sl.w);
        uint4 xa[2][4], xb[2][4];
        uint2 raw[2][2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xa[b][i] = *reinterpret_cast<const uint4 *>(xh + 2048 * i + a_off(b));
                xb[b][i] = *reinterpret_cast<const uint4 *>(xl + 2048 * i + a_off(b));
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const char *p = wb + b_off(b) + (QT == 1 ? 512 : 1024) * j;
                raw[b][j] = QT == 1 ? make_uint2(*reinterpret_cast<const uint32_t *>(p), 0u)
                                    : *reinterpret_cast<const uint2 *>(p);
            }
        }
        uint32_t sw[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
            sw[j] = sl.sc[n_lane + 16 * j];
        add_pending(); // the previous stage's second block
#pragma unroll
        for (int b = 0; b < 2; b++) {
            half8 bq[2];
            float sc[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                bq[j] = codes8<QT>(raw[b][j]);
                sc[j] = half_bits_to_float(uint16_t(sw[j] >> (16 * b)));
            }
            // all eight x_hi products first, then the x_lo products into
            // them, so no MFMA waits for the one just before it
            floatx4 d[4][2];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    d[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8, xa[b][i]), bq[j],
                        floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    d[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8, xb[b][i]), bq[j], d[i][j], 0, 0, 0);
            if (b == 1) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        pend[i][j] = d[i][j];
                psc[0] = sc[0];
                psc[1] = sc[1];
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            acc[i][j][v] = fmaf(sc[j], d[i][j][v], acc[i][j][v]);
            }
        }
    };
    // Stage s lives in slot s % 3. Step s: stage s landed in every wave
    // (stage s + 1 stays in flight), and every wave is done with stage
    // s - 1, whose slot takes stage s + 2.
    // With LOADER the compute waves only meet the loader at the barrier.
    auto step = [&](GemmSlot<QT> &cur, int free_slot, int st) {
        if constexpr (LOADER) {
            asm volatile("s_barrier" ::: "memory");
        } else {
            wait_dma_barrier<kDmaPerWave>();
            issue(free_slot, st + 2);
        }
        stage_mma(cur);
    };
    if constexpr (!LOADER) {
        issue(0, 0);
        issue(1, 1);
    }
    for (int st = 0; st < stages; st += kStages) {
#pragma unroll
        for (int r = 0; r < kStages; r++)
            if (st + r < stages) // workgroup-uniform
                step(slot[r], (r + 2) % kStages, st + r);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // no DMA outlives the workgroup
    add_pending();
    if constexpr (SWIGLU) {
        // acc[i][0]: gate, acc[i][1]: up of output n0 + 16 wave + li
        // (silu as the decode step: src/quant_model.cpp:197-200)
        const int n = n0 + 16 * wave + li;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = t0 + 16 * i + 4 * g + v;
                if (t < t_count && n < n_count) {
                    const float gv = acc[i][0][v];
                    put_limbs(segs.act_hi, segs.act_lo, size_t(t) * segs.act_ld + n,
                              gv / (1.0f + expf(-gv)) * acc[i][1][v]);
                }
            }
        return;
    }
    if constexpr (EPI == kEpiQkv) {
        // seg 0: q, 1: k, 2: v (workgroup-uniform); a tile never straddles
        // a head (hd is 64 or 128). The pair (d even, d + 1) sits in lanes
        // li, li ^ 1 of one 16-lane row: the even lane takes its partner's
        // value by DPP, rotates the pair as the decode step does
        // (src/quant_model.cpp:26-37, the host's RoPE table at position t)
        // and stores both values.
        const int hd = segs.hd;
        const bool even = (li & 1) == 0;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + 32 * wave + 16 * j + li;
            const int head = n / hd, d = n % hd;
            const bool col = even && n < n_count;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float re[4], ro[4];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    re[v] = acc[i][j][v];
                    ro[v] = dpp<kDppQuadSwap1>(re[v], 0.0f); // lane li ^ 1
                }
                const int tb = t0 + 16 * i + 4 * g;
                if (!col)
                    continue;
                if (seg < 2) {
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const float2 f =
                            segs.rope[size_t(min(tb + v, t_count - 1)) * (hd / 2) + d / 2];
                        const float e = re[v], o = ro[v];
                        re[v] = fmaf(e, f.x, -(o * f.y));
                        ro[v] = fmaf(e, f.y, o * f.x);
                    }
                }
                if (seg == 0) {
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        if (tb + v < t_count)
                            *reinterpret_cast<float2 *>(c + size_t(tb + v) * ldc + n) =
                                make_float2(re[v], ro[v]);
                    continue;
                }
                float *cache = seg == 1 ? segs.k_cache : segs.v_cache;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    if (tb + v < t_count) {
                        *reinterpret_cast<float2 *>(
                            cache + (size_t(head) * segs.max_seq + tb + v) * hd + d) =
                            make_float2(re[v], ro[v]);
                    } else {
                        re[v] = 0.0f; // padding positions: exact zeros
                        ro[v] = 0.0f;
                    }
                }
                if (seg == 1) {
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        put_limbs2(segs.k_hi, segs.k_lo,
                                   (size_t(head) * segs.t_pad + tb + v) * hd + d,
                                   make_float2(re[v], ro[v]));
                } else {
                    const size_t at = (size_t(head) * hd + d) * segs.t_pad + tb;
                    put_limbs4(segs.vt_hi, segs.vt_lo, at,
                               make_float4(re[0], re[1], re[2], re[3]));
                    put_limbs4(segs.vt_hi, segs.vt_lo, at + segs.t_pad,
                               make_float4(ro[0], ro[1], ro[2], ro[3]));
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = t0 + 16 * i + 4 * g + v;
                const int n = n0 + 32 * wave + 16 * j + li;
                if (t < t_count && n < n_count) {
                    float *p = c + size_t(t) * ldc + n;
                    *p = ADD ? *p + acc[i][j][v] : acc[i][j][v];
                }
            }
}

template <int QT, int EPI>
void launch_qgemm_form(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                       const GemmSegs &segs, hipStream_t stream)
{
    int tiles = 0;
    for (int i = 0; i < segs.count; i++)
        tiles += segs.tiles[i];
    const dim3 grid(tiles, (t_count + FM_ROWS - 1) / FM_ROWS);
    // at most one workgroup per CU (MI355X: 256 CUs): the loader-wave form
    if (size_t(grid.x) * grid.y <= 256)
        hipLaunchKernelGGL((qgemm_f16_kernel<QT, EPI, true>), grid,
                           dim3(kThreads + kWave), 0, stream, x_hi, x_lo, t_count, segs);
    else
        hipLaunchKernelGGL((qgemm_f16_kernel<QT, EPI, false>), grid, dim3(kThreads), 0,
                           stream, x_hi, x_lo, t_count, segs);
}

template <int QT>
void launch_qgemm(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                  const GemmSegs &segs, bool add, hipStream_t stream)
{
    if (add)
        launch_qgemm_form<QT, kEpiAdd>(x_hi, x_lo, t_count, segs, stream);
    else
        launch_qgemm_form<QT, kEpiStore>(x_hi, x_lo, t_count, segs, stream);
}

// Causal attention of a prompt batch: queries t0 .. t0 + 63 at positions
// t attend to cache positions 0 .. t, in 64-key tiles.
constexpr int AQ = 64, AK = 64;

// Positions of the K/V limb buffers: max_seq rounded up to whole key tiles.
int kv_limb_rows(const DecodeShape &s) { return (s.max_seq + AK - 1) / AK * AK; }

// On v_mfma_f32_16x16x32_f16 with operands as f16 limbs: every product a b
// is a_hi b_hi + a_hi b_lo + a_lo b_hi (three MFMAs; the dropped a_lo b_lo
// is below 2^-22 of a b), so S and P V carry fp32-level precision at the
// f16 matrix rate. One workgroup per (head, 64-query tile); wave w owns
// queries 16 w .. 16 w + 15 and holds their Q limbs in registers. Per
// 64-key tile (K limbs [key][d] and V limbs [d][key] in LDS): S = Q K^T,
// the online softmax on S in registers (a query row lives in one 16-lane
// DPP row), P as limbs through LDS into the A layout, then O += P V. Lane
// layouts (checked on the device): A[i][k]: lane i % 16 + 16 g holds k =
// 8 g .. 8 g + 7; B[k][n]: lane n % 16 + 16 g the same k; D[i][n]: lane
// n + 16 (i / 4), element i % 4.
// HEADS query heads of one KV head per workgroup (4 waves each, 64 query
// rows), sharing each K/V tile they stage.
template <int HD, int HEADS>
__global__ __launch_bounds__(64 * 4 * HEADS) void attention_prefill_f16(
    const float *q, const _Float16 *k_hi, const _Float16 *k_lo, const _Float16 *vt_hi,
    const _Float16 *vt_lo, _Float16 *ctx_hi, _Float16 *ctx_lo, int t_count, int t_pad,
    int heads, int kv_heads, float scale)
{
    constexpr int NT = 64 * 4 * HEADS;                     // threads
    constexpr int KP = HD + 8, VP = AK + 8, PP = AK + 8; // rows padded by 16 bytes
    constexpr int KB = HD / 32;                            // 32-wide k blocks of a head
    // K / V^T tiles: at head_dim 128, and for two heads per workgroup, two
    // buffers filled by DMA (tile k + 1 in flight while tile k is
    // multiplied; 161,792 and 110,592 bytes of LDS with P); the one-head
    // head_dim-64 form keeps one buffer filled from registers (below).
    // Measured against the register forms: 512 tokens at head_dim 128
    // 43.8 -> 31.0 us per layer, 2,048 tokens with head pairs 111.5 ->
    // 105.1 us (one workgroup per CU instead of two).
    constexpr bool DMA = HD == 128 || HEADS == 2;
    constexpr int NB = DMA ? 2 : 1;
    __shared__ __attribute__((aligned(16))) _Float16 ksh[NB][AK][KP], ksl[NB][AK][KP];
    __shared__ __attribute__((aligned(16))) _Float16 vsh[NB][HD][VP], vsl[NB][HD][VP];
    __shared__ __attribute__((aligned(16))) _Float16 psh[4 * HEADS][16][PP], psl[4 * HEADS][16][PP];
    const int tid = threadIdx.x, lane = tid & 63, wave_all = tid >> 6, wave = wave_all & 3;
    const int li = lane & 15, lg = lane >> 4;
    // heads vary fastest and the longest query tiles (the most key tiles
    // under the causal mask) are dispatched first
    const int head = blockIdx.x * HEADS + (wave_all >> 2), g = head / (heads / kv_heads);
    const int t0 = (gridDim.y - 1 - blockIdx.y) * AQ;
    const int dim = heads * HD;
    // Q limbs of this wave's rows: A[i = li][k = 32 kb + 8 lg + j]
    half8 qh[KB], ql[KB];
    {
        const int t = t0 + 16 * wave + li;
        const float *qr = q + size_t(min(t, t_count - 1)) * dim + head * HD;
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float x = t < t_count ? qr[32 * kb + 8 * lg + j] : 0.0f;
                const _Float16 hi = (_Float16)x;
                qh[kb][j] = hi;
                ql[kb][j] = (_Float16)(x - (float)hi);
            }
    }
    const _Float16 *kgh = k_hi + size_t(g) * t_pad * HD, *kgl = k_lo + size_t(g) * t_pad * HD;
    const _Float16 *vgh = vt_hi + size_t(g) * HD * t_pad, *vgl = vt_lo + size_t(g) * HD * t_pad;
    const int last = min(t0 + AQ - 1, t_count - 1);
    // softmax in base 2: scores scaled by scale * log2(e), weights
    // exp2(s - m) with the hardware exp2 (about 1 ulp)
    const float scale2 = scale * 1.4426950408889634f;
    // rows of this lane: r = 4 lg + v (v < 4) of the wave's 16
    int qpos[4];
#pragma unroll
    for (int v = 0; v < 4; v++)
        qpos[v] = t0 + 16 * wave + 4 * lg + v;
    float m[4], l[4];
    floatx4 o[HD / 16];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        m[v] = -INFINITY;
        l[v] = 0.0f;
    }
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++)
        o[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma3 = [](const half8 &ah, const half8 &al, const half8 &bh, const half8 &bl,
                   floatx4 acc) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc, 0, 0, 0);
    };
    // The K tile rows p0 .. p0 + 63 and the V^T tile [d][p0 ..] in 16-byte
    // pieces, PIECES per thread and array. Without DMA the next tile's
    // pieces are loaded into registers while the current tile is multiplied
    // and written to LDS at the start of the next iteration (2,048 tokens
    // with head pairs: 118.7 -> 115.0 us per layer; at head_dim 128 it cost
    // more than it hid, 43.1 -> 53.0 us, for 64 more VGPRs).
    constexpr bool PREFETCH = !DMA;
    constexpr int PIECES = AK * HD / 8 / NT;
    static_assert(PIECES * NT == AK * HD / 8, "whole pieces per thread");
    uint4 nkh[PIECES], nkl[PIECES], nvh[PIECES], nvl[PIECES];
    auto load_tile = [&](int p0) {
#pragma unroll
        for (int r = 0; r < PIECES; r++) {
            const int e = tid + NT * r;
            const int j = e / (HD / 8), c8 = e % (HD / 8);
            const size_t at = size_t(p0 + j) * HD + 8 * c8;
            nkh[r] = *reinterpret_cast<const uint4 *>(kgh + at);
            nkl[r] = *reinterpret_cast<const uint4 *>(kgl + at);
            const int d = e / (AK / 8), v8 = e % (AK / 8);
            const size_t av = size_t(d) * t_pad + p0 + 8 * v8;
            nvh[r] = *reinterpret_cast<const uint4 *>(vgh + av);
            nvl[r] = *reinterpret_cast<const uint4 *>(vgl + av);
        }
    };
    // DMA of the tile at keys p0 into buffer b: wave 0 the K hi rows, 1 K
    // lo, 2 V^T hi, 3 V^T lo (the first head's waves). An instruction fills
    // 1 KB of LDS, 16 bytes a lane, in the padded layout: a K row is HD / 8
    // + 1 slots of 16 bytes (the data, then the pad, which takes a copy of
    // the row's last slot), a V^T row 9 (8 data + pad); at head_dim 128,
    // 64 x 17 and 128 x 9 slots are 17 and 18 instructions, at head_dim 64
    // nine each.
    auto dma_tile = [&](int b, int p0) {
        if (wave_all >= 4) // the second head's waves issue none
            return;
        const int limb = wave & 1;
        if (wave < 2) {
            const _Float16 *src = (limb ? kgl : kgh) + size_t(p0) * HD;
            const uint32_t base = lds_addr(limb ? &ksl[b][0][0] : &ksh[b][0][0]);
#pragma unroll
            for (int i = 0; i < AK * (KP / 8) / kWave; i++) {
                const int sl = kWave * i + lane, j = sl / (KP / 8);
                const int c = min(sl % (KP / 8), HD / 8 - 1);
                dma16(src + j * HD + 8 * c, __builtin_amdgcn_readfirstlane(base + 1024 * i));
            }
        } else {
            const _Float16 *src = (limb ? vgl : vgh) + p0;
            const uint32_t base = lds_addr(limb ? &vsl[b][0][0] : &vsh[b][0][0]);
#pragma unroll
            for (int i = 0; i < HD * (VP / 8) / kWave; i++) {
                const int sl = kWave * i + lane, d = sl / (VP / 8);
                const int c = min(sl % (VP / 8), AK / 8 - 1);
                dma16(src + size_t(d) * t_pad + 8 * c,
                      __builtin_amdgcn_readfirstlane(base + 1024 * i));
            }
        }
    };
    static_assert(!DMA || (AK * (KP / 8) % kWave == 0 && HD * (VP / 8) % kWave == 0),
                  "whole DMA instructions per array");
    if constexpr (PREFETCH)
        load_tile(0);
    else
        dma_tile(0, 0);
    int b = 0; // the buffer of the current tile
    for (int p0 = 0; p0 <= last; p0 += AK) {
        if constexpr (DMA) {
            // this wave's DMA of the tile has landed, and after the barrier
            // every wave's has and every wave is done with the other buffer
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
            if (p0 + AK <= last) // workgroup-uniform
                dma_tile(b ^ 1, p0 + AK);
        } else {
            __syncthreads(); // previous tile's readers are done
#pragma unroll
            for (int r = 0; r < PIECES; r++) {
                const int e = tid + NT * r;
                const int j = e / (HD / 8), c8 = e % (HD / 8);
                *reinterpret_cast<uint4 *>(&ksh[0][j][8 * c8]) = nkh[r];
                *reinterpret_cast<uint4 *>(&ksl[0][j][8 * c8]) = nkl[r];
                const int d = e / (AK / 8), v8 = e % (AK / 8);
                *reinterpret_cast<uint4 *>(&vsh[0][d][8 * v8]) = nvh[r];
                *reinterpret_cast<uint4 *>(&vsl[0][d][8 * v8]) = nvl[r];
            }
            __syncthreads();
            if (p0 + AK <= last) // workgroup-uniform
                load_tile(p0 + AK);
            // keep the loads ahead of the tile's MFMAs
            __builtin_amdgcn_sched_barrier(0);
        }
        // S tiles: keys 16 nt + li, rows 4 lg + v
        floatx4 sc[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++)
            sc[nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const half8 bh = *reinterpret_cast<const half8 *>(&ksh[b][16 * nt + li][32 * kb + 8 * lg]);
                const half8 bl = *reinterpret_cast<const half8 *>(&ksl[b][16 * nt + li][32 * kb + 8 * lg]);
                sc[nt] = mma3(qh[kb], ql[kb], bh, bl, sc[nt]);
            }
        float corr[4];
        // Only the diagonal tile (p0 == t0) needs the causal mask: every key
        // of an earlier tile precedes every query of this one, so its
        // scores and running maxima are finite (m = -inf before the first
        // tile gives corr = 2^-inf = 0).
        auto softmax = [&](auto masked) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float tmax = -INFINITY;
#pragma unroll
                for (int nt = 0; nt < 4; nt++) {
                    const int kpos = p0 + 16 * nt + li;
                    const float x = !masked || kpos <= qpos[v] ? sc[nt][v] * scale2 : -INFINITY;
                    sc[nt][v] = x;
                    tmax = fmaxf(tmax, x);
                }
                tmax = row16_max(tmax);
                const float mn = fmaxf(m[v], tmax);
                // rows past t_count (and fully masked tiles) keep m = -inf
                corr[v] = masked && mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[v] - mn);
                float sum = 0.0f;
#pragma unroll
                for (int nt = 0; nt < 4; nt++) {
                    const float e = masked && sc[nt][v] == -INFINITY
                                        ? 0.0f
                                        : __builtin_amdgcn_exp2f(sc[nt][v] - mn);
                    const _Float16 hi = (_Float16)e;
                    psh[wave_all][4 * lg + v][16 * nt + li] = hi;
                    psl[wave_all][4 * lg + v][16 * nt + li] = (_Float16)(e - (float)hi);
                    sum += e;
                }
                l[v] = l[v] * corr[v] + row16_sum(sum);
                m[v] = mn;
            }
        };
        if (p0 == t0) // workgroup-uniform
            softmax(std::true_type{});
        else
            softmax(std::false_type{});
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                o[dt][v] *= corr[v];
        // P rows of this wave are written and read by this wave only (LDS
        // runs a wave's accesses in order; the fences keep the compiler's)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int kb = 0; kb < AK / 32; kb++) {
            const half8 ah = *reinterpret_cast<const half8 *>(&psh[wave_all][li][32 * kb + 8 * lg]);
            const half8 al = *reinterpret_cast<const half8 *>(&psl[wave_all][li][32 * kb + 8 * lg]);
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++) {
                const half8 bh = *reinterpret_cast<const half8 *>(&vsh[b][16 * dt + li][32 * kb + 8 * lg]);
                const half8 bl = *reinterpret_cast<const half8 *>(&vsl[b][16 * dt + li][32 * kb + 8 * lg]);
                o[dt] = mma3(ah, al, bh, bl, o[dt]);
            }
        }
        if constexpr (DMA)
            b ^= 1;
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int t = t0 + 16 * wave + 4 * lg + v;
        if (t < t_count) {
            const float inv = 1.0f / l[v];
            const size_t row = size_t(t) * dim + head * HD;
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++)
                put_limbs(ctx_hi, ctx_lo, row + 16 * dt + li, o[dt][v] * inv);
        }
    }
}

} // namespace

bool prefill_gemm_supported(const DecodeShape &s, const LayerView &w)
{
    const QMat *mats[7] = {&w.query, &w.key, &w.value, &w.output,
                           &w.gate, &w.up, &w.down};
    // whole blocks per row, and an even block count (a row's scales are
    // DMA'd as dwords)
    for (const QMat *m : mats)
        if (!fast_layout(*m) || m->cols % 64 != 0)
            return false;
    return s.head_dim == 64 || s.head_dim == 128;
}

void launch_embed_rows(const float *embeddings, const int *tokens, float *h,
                       int t_count, int dim, hipStream_t stream)
{
    hipLaunchKernelGGL(embed_rows_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, embeddings, tokens, h, dim);
    check_launch("prefill embed");
}

void launch_rmsnorm_rows(const float *h, const float *w, _Float16 *out_hi,
                         _Float16 *out_lo, int t_count, int dim, hipStream_t stream)
{
    require(dim % 4 == 0, NUT_EINVAL, "prefill rmsnorm: dim must be a multiple of 4");
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, h, w, out_hi, out_lo, dim);
    check_launch("prefill rmsnorm");
}

size_t stage_scale_words(const QMat &m)
{
    return size_t(m.rows) * size_t(m.cols / FS);
}

void launch_scales_by_stage(const QMat &m, uint32_t *dst, hipStream_t stream)
{
    require(m.block_size == 32 && m.cols % FS == 0, NUT_EINVAL,
            "prefill gemm: stage scales need 32-wide blocks in whole 64-wide stages");
    const size_t n = stage_scale_words(m);
    hipLaunchKernelGGL(scales_by_stage_kernel, dim3(unsigned((n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, stream,
                       reinterpret_cast<const uint32_t *>(m.scales), dst, m.rows,
                       m.cols / FS);
    check_launch("prefill stage scales");
}

void launch_qgemm_rows(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                       const QMat *const *w, const uint32_t *const *stage_scales,
                       float *const *c, const int *ldc, int count, bool add,
                       hipStream_t stream)
{
    require(count >= 1 && count <= 3, NUT_EINVAL, "prefill gemm: 1 to 3 matrices");
    GemmSegs segs{};
    segs.count = count;
    for (int i = 0; i < count; i++) {
        require(w[i]->type == w[0]->type && w[i]->cols == w[0]->cols, NUT_EINVAL,
                "prefill gemm: matrices differ in type or input size");
        require(w[i]->cols % FS == 0 && stage_scales[i] != nullptr, NUT_EINVAL,
                "prefill gemm: rows of whole 64-wide stages with stage-major scales");
        segs.w[i] = *w[i];
        segs.st[i] = stage_scales[i];
        segs.c[i] = c[i];
        segs.ldc[i] = ldc[i];
        segs.tiles[i] = (w[i]->rows + FN - 1) / FN;
    }
    if (w[0]->type == 1)
        launch_qgemm<1>(x_hi, x_lo, t_count, segs, add, stream);
    else
        launch_qgemm<0>(x_hi, x_lo, t_count, segs, add, stream);
    check_launch("prefill gemm");
}

void launch_qgemm_swiglu(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                         const QMat &gate, const QMat &up, const uint32_t *st_gate,
                         const uint32_t *st_up, _Float16 *act_hi, _Float16 *act_lo,
                         hipStream_t stream)
{
    require(gate.type == up.type && gate.cols == up.cols && gate.rows == up.rows, NUT_EINVAL,
            "prefill gemm: gate and up differ in type or shape");
    require(gate.cols % FS == 0 && st_gate != nullptr && st_up != nullptr, NUT_EINVAL,
            "prefill gemm: rows of whole 64-wide stages with stage-major scales");
    GemmSegs segs{};
    segs.count = 1;
    segs.w[0] = gate;
    segs.w[1] = up;
    segs.st[0] = st_gate;
    segs.st[1] = st_up;
    segs.tiles[0] = (gate.rows + FN / 2 - 1) / (FN / 2);
    segs.act_hi = act_hi;
    segs.act_lo = act_lo;
    segs.act_ld = gate.rows;
    if (gate.type == 1)
        launch_qgemm_form<1, kEpiSwiglu>(x_hi, x_lo, t_count, segs, stream);
    else
        launch_qgemm_form<0, kEpiSwiglu>(x_hi, x_lo, t_count, segs, stream);
    check_launch("prefill gemm swiglu");
}

size_t prefill_kv_limb_elems(const DecodeShape &s)
{
    return size_t(s.kv_heads) * kv_limb_rows(s) * s.head_dim;
}

void launch_qgemm_qkv(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                      const QMat *const *w, const uint32_t *const *stage_scales, float *q,
                      const float2 *rope, float *k_cache, float *v_cache, _Float16 *kv_limbs,
                      const DecodeShape &s, hipStream_t stream)
{
    const int kvd = s.kv_heads * s.head_dim;
    require(s.head_dim == 64 || s.head_dim == 128, NUT_EINVAL,
            "prefill gemm: head_dim must be 64 or 128");
    require(w[0]->rows == s.heads * s.head_dim && w[1]->rows == kvd && w[2]->rows == kvd,
            NUT_EINVAL, "prefill gemm: q/k/v rows do not match the shape");
    const int t_pad = (t_count + AK - 1) / AK * AK;
    require(t_pad <= kv_limb_rows(s) && t_count <= s.max_seq, NUT_EINVAL,
            "prefill gemm: prompt too long");
    GemmSegs segs{};
    segs.count = 3;
    for (int i = 0; i < 3; i++) {
        require(w[i]->type == w[0]->type && w[i]->cols == w[0]->cols, NUT_EINVAL,
                "prefill gemm: matrices differ in type or input size");
        require(w[i]->cols % FS == 0 && stage_scales[i] != nullptr, NUT_EINVAL,
                "prefill gemm: rows of whole 64-wide stages with stage-major scales");
        segs.w[i] = *w[i];
        segs.st[i] = stage_scales[i];
        segs.tiles[i] = (w[i]->rows + FN - 1) / FN;
    }
    segs.c[0] = q;
    segs.ldc[0] = s.heads * s.head_dim;
    const size_t n = size_t(s.kv_heads) * t_pad * s.head_dim;
    segs.rope = rope;
    segs.k_cache = k_cache;
    segs.v_cache = v_cache;
    segs.k_hi = kv_limbs;
    segs.k_lo = kv_limbs + n;
    segs.vt_hi = kv_limbs + 2 * n;
    segs.vt_lo = kv_limbs + 3 * n;
    segs.hd = s.head_dim;
    segs.max_seq = s.max_seq;
    segs.t_pad = t_pad;
    if (w[0]->type == 1)
        launch_qgemm_form<1, kEpiQkv>(x_hi, x_lo, t_count, segs, stream);
    else
        launch_qgemm_form<0, kEpiQkv>(x_hi, x_lo, t_count, segs, stream);
    check_launch("prefill gemm qkv");
}

void launch_attention_prefill(const float *q, const _Float16 *kv_limbs, _Float16 *ctx_hi,
                              _Float16 *ctx_lo, const DecodeShape &s, int t_count,
                              hipStream_t stream)
{
    const int t_pad = (t_count + AK - 1) / AK * AK;
    require(t_pad <= kv_limb_rows(s), NUT_EINVAL, "prefill attention: prompt too long");
    const size_t n = size_t(s.kv_heads) * t_pad * s.head_dim;
    const _Float16 *k_hi = kv_limbs, *k_lo = k_hi + n, *vt_hi = k_lo + n, *vt_lo = vt_hi + n;
    const dim3 grid(s.heads, t_pad / AQ);
    // head_dim 64: two query heads per workgroup when they share a KV head
    const bool pair = (s.heads / s.kv_heads) % 2 == 0;
    const dim3 pair_grid(s.heads / 2, t_pad / AQ);
    if (s.head_dim == 128)
        hipLaunchKernelGGL((attention_prefill_f16<128, 1>), grid, dim3(256), 0, stream, q,
                           k_hi, k_lo, vt_hi, vt_lo, ctx_hi, ctx_lo, t_count, t_pad,
                           s.heads, s.kv_heads, s.attn_scale);
    else if (pair)
        hipLaunchKernelGGL((attention_prefill_f16<64, 2>), pair_grid, dim3(512), 0, stream, q,
                           k_hi, k_lo, vt_hi, vt_lo, ctx_hi, ctx_lo, t_count, t_pad,
                           s.heads, s.kv_heads, s.attn_scale);
    else
        hipLaunchKernelGGL((attention_prefill_f16<64, 1>), grid, dim3(256), 0, stream, q,
                           k_hi, k_lo, vt_hi, vt_lo, ctx_hi, ctx_lo, t_count, t_pad,
                           s.heads, s.kv_heads, s.attn_scale);
    check_launch("prefill attention");
}

} // namespace nut
