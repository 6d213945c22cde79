// prefill.hip — the prompt as a batch: prefill_quantized
// (src/quant_model.cpp:208-220) computes, token after token, the decode
// step of src/quant_model.cpp:158-206; this file computes the same function
// for all T prompt tokens at once, layer by layer:
//   rmsnorm rows -> Q/K/V GEMMs -> RoPE + KV-cache store -> causal attention
//   -> Wo GEMM (+ residual) -> rmsnorm rows -> gate/up GEMMs -> silu * up
//   -> W2 GEMM (+ residual)
// The quantised GEMMs run on f16 MFMA with the weight codes exact in f16,
// the activations split into two f16 limbs and the block scales applied
// in fp32 per 32-wide block; attention runs on fp32 MFMA. The hidden state
// stays within about 1e-5 of the per-token path (fp32 throughout).
#include "prefill.hpp"
#include "runtime.hpp"

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
__device__ __forceinline__ void put_limbs(_Float16 *hi, _Float16 *lo, size_t i, float v)
{
    const _Float16 a = (_Float16)v;
    hi[i] = a;
    lo[i] = (_Float16)(v - (float)a);
}

__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(
    const float *h, const float *w, _Float16 *out_hi, _Float16 *out_lo, int dim)
{
    __shared__ float red[kThreads / kWave];
    const float *x = h + size_t(blockIdx.x) * dim;
    float sq = 0.0f;
    for (int i = threadIdx.x; i < dim; i += kThreads)
        sq = fmaf(x[i], x[i], sq);
    const float total = block_sum(sq, red, kThreads / kWave);
    const float scale = 1.0f / sqrtf(total / float(dim) + 1e-5f);
    const size_t row = size_t(blockIdx.x) * dim;
    for (int i = threadIdx.x; i < dim; i += kThreads)
        put_limbs(out_hi, out_lo, row + i, x[i] * scale * w[i]);
}

// act[t][i] = silu(g[t][i]) * u[t][i]  (src/quant_model.cpp:197-198)
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float *g,
                                                            const float *u,
                                                            _Float16 *act_hi,
                                                            _Float16 *act_lo, size_t n)
{
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) {
        const float v = g[i];
        put_limbs(act_hi, act_lo, i, v / (1.0f + expf(-v)) * u[i]);
    }
}

// RoPE on q (all heads) and k (kv heads) of token t at position start + t,
// the rotation of the decode path (src/quant_model.cpp:26-37), then K and V
// rows into the cache [kv_head][max_seq][head_dim] of this layer.
__global__ __launch_bounds__(kThreads) void rope_store_kernel(
    float *q, const float *k, const float *v, const float2 *rope, float *k_cache,
    float *v_cache, int heads, int kv_heads, int hd, int max_seq, int start)
{
    const int t = blockIdx.x;
    const int pos = start + t;
    const int dim = heads * hd, kvd = kv_heads * hd;
    const float2 *cs = rope + size_t(pos) * (hd / 2);
    for (int i = threadIdx.x; i < dim / 2; i += kThreads) {
        float *p = q + size_t(t) * dim + 2 * i;
        const float2 f = cs[i % (hd / 2)];
        const float even = p[0], odd = p[1];
        p[0] = fmaf(even, f.x, -(odd * f.y));
        p[1] = fmaf(even, f.y, odd * f.x);
    }
    for (int i = threadIdx.x; i < kvd / 2; i += kThreads) {
        const float *p = k + size_t(t) * kvd + 2 * i;
        const float2 f = cs[i % (hd / 2)];
        const float even = p[0], odd = p[1];
        const int head = (2 * i) / hd, d = (2 * i) % hd;
        float *kc = k_cache + (size_t(head) * max_seq + pos) * hd + d;
        kc[0] = fmaf(even, f.x, -(odd * f.y));
        kc[1] = fmaf(even, f.y, odd * f.x);
        const float *vp = v + size_t(t) * kvd + 2 * i;
        float *vcp = v_cache + (size_t(head) * max_seq + pos) * hd + d;
        vcp[0] = vp[0];
        vcp[1] = vp[1];
    }
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
// A workgroup owns FM tokens x 128 outputs; four waves of (FM / 32) x 4
// MFMA tiles. Per 32-wide k slice the limbs of X and the W
// codes go to LDS (double-buffered) while the next three slices load into
// registers. Lane layout (measured): A[i][k] in lane i % 16 + 16 g
// holding k = 8 g .. 8 g + 7; B[k][n] likewise with n = lane % 16;
// D[i][n] in lane n + 16 (i / 4), element i % 4.
constexpr int FN = 128, FK = 32;
constexpr int FROW = FK + 8; // f16 per LDS row (16-byte pad)

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Up to three matrices sharing X and k (Q/K/V, or gate/up) in one launch:
// column tiles of FN outputs are numbered across the segments in order.
struct GemmSegs {
    QMat w[3];
    float *c[3];
    int ldc[3];
    int tiles[3];
    int count;
};

template <int QT, bool ADD, int FM>
__global__ __launch_bounds__(kThreads) void qgemm_f16_kernel(
    const _Float16 *__restrict__ x_hi, const _Float16 *__restrict__ x_lo, int t_count,
    GemmSegs segs)
{
    constexpr int MT = FM / 32; // 16-row MFMA tiles per wave (waves 2 x 2)
    __shared__ __attribute__((aligned(16))) _Float16 xh[2][FM][FROW];
    __shared__ __attribute__((aligned(16))) _Float16 xl[2][FM][FROW];
    __shared__ __attribute__((aligned(16))) _Float16 wq[2][FN][FROW];
    __shared__ float wsc[2][FN];
    int seg = 0, tile = blockIdx.x;
    while (seg + 1 < segs.count && tile >= segs.tiles[seg])
        tile -= segs.tiles[seg++]; // workgroup-uniform
    const QMat w = segs.w[seg];
    float *__restrict__ c = segs.c[seg];
    const int ldc = segs.ldc[seg];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.y * FM, n0 = tile * FN;
    const int wm = (wave >> 1) * (FM / 2), wn = (wave & 1) * 64;
    const int k = w.cols, n_count = w.rows, blocks = k / FK;
    // W loader: row r = tid / 2, 16 consecutive k from 16 h; X loader: the
    // same for rows r < FM (FM = 64: the upper half of the threads idle)
    const int r = tid >> 1, h = tid & 1;
    const bool xload = r < FM;
    const int xrow = t0 + r;
    const size_t xoff = size_t(min(xrow, t_count - 1)) * k + 16 * h;
    const _Float16 *xph = x_hi + xoff, *xpl = x_lo + xoff;
    const int wrow = min(n0 + r, n_count - 1);
    constexpr int RB_DIV = QT == 1 ? 2 : 1;
    const uint8_t *wp = w.data + size_t(wrow) * (k / RB_DIV) + (QT == 1 ? 8 : 16) * h;
    const uint16_t *sp = w.scales + size_t(wrow) * blocks;
    // One k slice in registers: X limbs, W bytes (INT4 uses .x, .y), scale.
    struct Slice {
        half8 xh[2], xl[2];
        uint4 w;
        uint16_t s;
    };
    auto load = [&](Slice &sl, int kb) {
        if (xload) {
            const half8 *sh = reinterpret_cast<const half8 *>(xph + kb * FK);
            const half8 *sx = reinterpret_cast<const half8 *>(xpl + kb * FK);
            const half8 zero = {};
#pragma unroll
            for (int j = 0; j < 2; j++) {
                sl.xh[j] = xrow < t_count ? sh[j] : zero;
                sl.xl[j] = xrow < t_count ? sx[j] : zero;
            }
        }
        if (QT == 1) {
            const uint2 v = *reinterpret_cast<const uint2 *>(wp + kb * (FK / 2));
            sl.w = make_uint4(v.x, v.y, 0u, 0u);
        } else {
            sl.w = *reinterpret_cast<const uint4 *>(wp + kb * FK);
        }
        if (h == 0)
            sl.s = sp[kb];
    };
    auto stage = [&](const Slice &sl, int buf) {
        if (xload) {
            *reinterpret_cast<half8 *>(&xh[buf][r][16 * h]) = sl.xh[0];
            *reinterpret_cast<half8 *>(&xh[buf][r][16 * h + 8]) = sl.xh[1];
            *reinterpret_cast<half8 *>(&xl[buf][r][16 * h]) = sl.xl[0];
            *reinterpret_cast<half8 *>(&xl[buf][r][16 * h + 8]) = sl.xl[1];
        }
        half8 q[2];
        const uint32_t words[4] = {sl.w.x, sl.w.y, sl.w.z, sl.w.w};
#pragma unroll
        for (int e = 0; e < 16; e++) {
            int code;
            if (QT == 1) {
                const uint32_t nib = (words[e >> 3] >> (4 * (e & 7))) & 0xfu;
                code = int(nib) - (nib >= 8 ? 16 : 0);
            } else {
                code = int(int8_t((words[e >> 2] >> (8 * (e & 3))) & 0xffu));
            }
            q[e >> 3][e & 7] = (_Float16)code;
        }
        *reinterpret_cast<half8 *>(&wq[buf][r][16 * h]) = q[0];
        *reinterpret_cast<half8 *>(&wq[buf][r][16 * h + 8]) = q[1];
        if (h == 0)
            wsc[buf][r] = half_bits_to_float(sl.s);
    };
    floatx4 acc[MT][4];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const int g = lane >> 4, li = lane & 15;
    auto compute = [&](int buf) {
        half8 ah[MT], al[MT], b[4];
        float sc[4];
#pragma unroll
        for (int i = 0; i < MT; i++) {
            ah[i] = *reinterpret_cast<const half8 *>(&xh[buf][wm + 16 * i + li][8 * g]);
            al[i] = *reinterpret_cast<const half8 *>(&xl[buf][wm + 16 * i + li][8 * g]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            b[j] = *reinterpret_cast<const half8 *>(&wq[buf][wn + 16 * j + li][8 * g]);
            sc[j] = wsc[buf][wn + 16 * j + li];
        }
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    ah[i], b[j], floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], d, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++)
                    acc[i][j][v] = fmaf(sc[j], d[v], acc[i][j][v]);
            }
    };
    // Slices kb .. kb + 2 are in flight in three register sets (slice s in
    // set s % 3) while slice kb is multiplied from LDS buffer kb % 2.
    Slice s0, s1, s2;
    load(s0, 0);
    if (1 < blocks)
        load(s1, 1);
    if (2 < blocks)
        load(s2, 2);
    stage(s0, 0);
    __syncthreads();
    auto step = [&](int kb, Slice &next, Slice &done) {
        compute(kb & 1);
        if (kb + 1 < blocks)
            stage(next, (kb + 1) & 1);
        if (kb + 3 < blocks)
            load(done, kb + 3);
        __syncthreads();
    };
    for (int kb = 0; kb < blocks; kb += 3) {
        step(kb, s1, s0);
        if (kb + 1 < blocks)
            step(kb + 1, s2, s1);
        if (kb + 2 < blocks)
            step(kb + 2, s0, s2);
    }
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = t0 + wm + 16 * i + 4 * g + v;
                const int n = n0 + wn + 16 * j + li;
                if (t < t_count && n < n_count) {
                    float *p = c + size_t(t) * ldc + n;
                    *p = ADD ? *p + acc[i][j][v] : acc[i][j][v];
                }
            }
}

// Causal attention of a prompt batch: queries t0 .. t0 + 63 at positions
// start + t attend to cache positions 0 .. start + t, in 64-key tiles.
constexpr int AQ = 64, AK = 64;

// On v_mfma_f32_16x16x4f32 (fp32 operands, as the reference's
// arithmetic): one workgroup per (head, 64-query tile);
// wave w owns queries 16 w .. 16 w + 15. Per 64-key tile (K and V in LDS):
// S = Q K^T as 4 x (HD / 4) MFMAs with Q in registers, the online softmax
// on S in registers (a query row lives in one 16-lane DPP row), P through
// LDS into the A layout, then O += P V as (HD / 16) x 16 MFMAs. Lane
// layouts of the 16x16x4 MFMA: A[i][k] in lane i + 16 k, B[k][n] in lane
// n + 16 k, D[i][n] in lane n + 16 (i / 4), element i % 4.
template <int HD>
__global__ __launch_bounds__(kThreads) void attention_prefill_mfma(
    const float *q, const float *k_cache, const float *v_cache, _Float16 *ctx_hi,
    _Float16 *ctx_lo, int t_count, int heads, int kv_heads, int max_seq, int start,
    float scale)
{
    constexpr int KP = HD + 4, VP = HD + 16, PP = AK + 4;
    __shared__ float ks[AK][KP];
    __shared__ float vs[AK][VP];
    __shared__ float ps[4][16][PP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // heads vary fastest and the longest query tiles (the most key tiles
    // under the causal mask) are dispatched first
    const int head = blockIdx.x, g = head / (heads / kv_heads);
    const int t0 = (gridDim.y - 1 - blockIdx.y) * AQ;
    const int dim = heads * HD;
    // Q fragments of this wave's rows: A[i = li][k = 4 s + lg]
    float qa[HD / 4];
    {
        const int t = t0 + 16 * wave + li;
        const float *qr = q + size_t(min(t, t_count - 1)) * dim + head * HD;
#pragma unroll
        for (int st = 0; st < HD / 4; st++)
            qa[st] = t < t_count ? qr[4 * st + lg] : 0.0f;
    }
    const float *kg = k_cache + size_t(g) * max_seq * HD;
    const float *vg = v_cache + size_t(g) * max_seq * HD;
    const int last = min(start + t0 + AQ - 1, start + t_count - 1);
    // rows of this lane: r = 4 lg + v (v < 4) of the wave's 16
    int qpos[4];
#pragma unroll
    for (int v = 0; v < 4; v++)
        qpos[v] = start + t0 + 16 * wave + 4 * lg + v;
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
    for (int p0 = 0; p0 <= last; p0 += AK) {
        __syncthreads(); // previous tile's readers are done
        for (int e = tid; e < AK * HD / 4; e += kThreads) {
            const int j = e / (HD / 4), d4 = e % (HD / 4);
            const bool in = p0 + j <= last;
            const float4 kv = in ? reinterpret_cast<const float4 *>(kg + size_t(p0 + j) * HD)[d4]
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 vv = in ? reinterpret_cast<const float4 *>(vg + size_t(p0 + j) * HD)[d4]
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            *reinterpret_cast<float4 *>(&ks[j][4 * d4]) = kv;
            *reinterpret_cast<float4 *>(&vs[j][4 * d4]) = vv;
        }
        __syncthreads();
        // S tiles: keys 16 nt + li, rows 4 lg + v
        floatx4 sc[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            sc[nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < HD / 4; st++)
                sc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    qa[st], ks[16 * nt + li][4 * st + lg], sc[nt], 0, 0, 0);
        }
        float corr[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float tmax = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const int kpos = p0 + 16 * nt + li;
                const float x = kpos <= qpos[v] ? sc[nt][v] * scale : -INFINITY;
                sc[nt][v] = x;
                tmax = fmaxf(tmax, x);
            }
            tmax = row16_max(tmax);
            const float mn = fmaxf(m[v], tmax);
            // rows past t_count (and fully masked tiles) keep m = -inf
            corr[v] = mn == -INFINITY ? 1.0f : expf(m[v] - mn);
            float sum = 0.0f;
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const float e = sc[nt][v] == -INFINITY ? 0.0f : expf(sc[nt][v] - mn);
                ps[wave][4 * lg + v][16 * nt + li] = e;
                sum += e;
            }
            l[v] = l[v] * corr[v] + row16_sum(sum);
            m[v] = mn;
        }
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                o[dt][v] *= corr[v];
        // ps rows of this wave are written by this wave only
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): LDS writes done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int st = 0; st < AK / 4; st++) {
            const float pa = ps[wave][li][4 * st + lg];
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++)
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    pa, vs[4 * st + lg][16 * dt + li], o[dt], 0, 0, 0);
        }
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

template <int QT, bool ADD, int FM>
void launch_qgemm_fm(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                     const GemmSegs &segs, hipStream_t stream)
{
    int tiles = 0;
    for (int i = 0; i < segs.count; i++)
        tiles += segs.tiles[i];
    hipLaunchKernelGGL((qgemm_f16_kernel<QT, ADD, FM>), dim3(tiles, (t_count + FM - 1) / FM),
                       dim3(kThreads), 0, stream, x_hi, x_lo, t_count, segs);
}

// 64-token tiles: with three slices in flight the 128-token tile needs
// more than 256 registers and runs one wave per SIMD, which measured slower
// on every prefill shape.
template <int QT>
void launch_qgemm(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                  const GemmSegs &segs, bool add, hipStream_t stream)
{
    if (add)
        launch_qgemm_fm<QT, true, 64>(x_hi, x_lo, t_count, segs, stream);
    else
        launch_qgemm_fm<QT, false, 64>(x_hi, x_lo, t_count, segs, stream);
}

} // namespace

bool prefill_gemm_supported(const DecodeShape &s, const LayerView &w)
{
    const QMat *mats[7] = {&w.query, &w.key, &w.value, &w.output,
                           &w.gate, &w.up, &w.down};
    for (const QMat *m : mats)
        if (!fast_layout(*m))
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
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, h, w, out_hi, out_lo, dim);
    check_launch("prefill rmsnorm");
}

void launch_qgemm_rows(const _Float16 *x_hi, const _Float16 *x_lo, int t_count,
                       const QMat *const *w, float *const *c, const int *ldc, int count,
                       bool add, hipStream_t stream)
{
    require(count >= 1 && count <= 3, NUT_EINVAL, "prefill gemm: 1 to 3 matrices");
    GemmSegs segs{};
    segs.count = count;
    for (int i = 0; i < count; i++) {
        require(w[i]->type == w[0]->type && w[i]->cols == w[0]->cols, NUT_EINVAL,
                "prefill gemm: matrices differ in type or input size");
        segs.w[i] = *w[i];
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

void launch_rope_store(float *q, const float *k, const float *v,
                       const float2 *rope, float *k_cache, float *v_cache,
                       const DecodeShape &s, int t_count, int start,
                       hipStream_t stream)
{
    hipLaunchKernelGGL(rope_store_kernel, dim3(t_count), dim3(kThreads), 0,
                       stream, q, k, v, rope, k_cache, v_cache, s.heads,
                       s.kv_heads, s.head_dim, s.max_seq, start);
    check_launch("prefill rope");
}

void launch_attention_prefill(const float *q, const float *k_cache,
                              const float *v_cache, _Float16 *ctx_hi, _Float16 *ctx_lo,
                              const DecodeShape &s, int t_count, int start,
                              hipStream_t stream)
{
    const dim3 grid(s.heads, (t_count + AQ - 1) / AQ);
    if (s.head_dim == 128)
        hipLaunchKernelGGL(attention_prefill_mfma<128>, grid, dim3(kThreads), 0,
                           stream, q, k_cache, v_cache, ctx_hi, ctx_lo, t_count, s.heads,
                           s.kv_heads, s.max_seq, start, s.attn_scale);
    else
        hipLaunchKernelGGL(attention_prefill_mfma<64>, grid, dim3(kThreads), 0,
                           stream, q, k_cache, v_cache, ctx_hi, ctx_lo, t_count, s.heads,
                           s.kv_heads, s.max_seq, start, s.attn_scale);
    check_launch("prefill attention");
}

void launch_silu_mul(const float *g, const float *u, _Float16 *act_hi,
                     _Float16 *act_lo, size_t n, hipStream_t stream)
{
    const int blocks = int((n + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                       g, u, act_hi, act_lo, n);
    check_launch("prefill silu");
}

} // namespace nut
