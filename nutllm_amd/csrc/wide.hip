// wide.hip — the quantised token loop for wide multi-head shapes
// (Llama-2-7B: dim 4096, 32 heads of 128 each with its own K/V head, ffn
// 11008) as one cooperative kernel of 256 x 512 threads.
//
// The phases are those of persistent.hip (A q/k/v, B attention + Wo,
// C gate/up, D W2; when generating, the final rmsnorm + classifier +
// first-index argmax first, src/generate.cpp:195-207), with two changes
// for shapes whose weight rows per workgroup (about 440 KB per layer here)
// fit neither LDS nor the register file:
//
// * Each phase's rows are prefetched partly into LDS (LDS DMA, cooperative
//   over the workgroup) and partly into registers (buffer loads, each wave
//   its own rows), issued right after a publish and before the next wait:
//   HBM streams while the exchange completes, and no publish queues behind
//   the bulk loads in the CU's memory pipeline (measured: moving the
//   gate/up rows under attention's exchanges, or any bulk under a compute
//   phase, makes the layer slower, as the issuing waves stall until the
//   CU's queue drains and the exchanges' stores and polls wait behind it).
// * Attention is split by head dims. Head h belongs to the eight
//   workgroups b with b % 32 == h (one XCD under round-robin dispatch);
//   workgroup j = b / 32 of the group computes dims [16 j, 16 j + 16) of
//   head h's q, k and v in phase A (so RoPE pairs and the K/V cache stores
//   stay local), then partial scores over those dims at every position,
//   published as tagged words. Every workgroup of the group sums the
//   eight partials in the same order, so all agree on the softmax, and
//   computes its sixteen context dims from the same dims of the V rows.
//   Per layer this makes five exchanges: partial scores (inside the
//   group), the context, h after Wo, the activation, h after W2.
//
// Each workgroup reads only its own slice of the K/V cache, which it also
// wrote, so the cache needs no cross-CU coherence inside a launch. Every
// wait is bounded as in persistent.hip.
//
// Values derived from the lane index or from kernel arguments pass through
// opaque_lane_value / fresh where they are used: otherwise the compiler
// hoists them out of the token and layer loops and keeps hundreds of them
// live across every phase.
#include "persistent.hpp"
#include "runtime.hpp"
#include "token_device.hpp"

namespace nut {

namespace {

template <int QT_, int DIM_, int FFN_, int HEADS_, int HD_, int NMAX_>
struct Wide {
    static constexpr int QT = QT_, DIM = DIM_, FFN = FFN_, HEADS = HEADS_, HD = HD_;
    static constexpr int NMAX = NMAX_;      // longest context
    static constexpr int GW = kGrid / HEADS; // workgroups per head
    static constexpr int SLICE = HD / GW;    // head dims per workgroup
    static constexpr int BLK_DIM = DIM / 32, BLK_FFN = FFN / 32;
    static constexpr int CPL_DIM = cdiv(BLK_DIM, kWave); // blocks per lane
    static constexpr int CPL_FFN = cdiv(BLK_FFN, kWave);
    static constexpr int RB_DIM = QT == 1 ? DIM / 2 : DIM; // bytes of a row
    static constexpr int RB_FFN = QT == 1 ? FFN / 2 : FFN;
    static constexpr int SB_DIM = 2 * BLK_DIM, SB_FFN = 2 * BLK_FFN; // scale bytes
    static constexpr int ROWS = DIM / kGrid;  // Wo and W2 rows per workgroup
    static constexpr int GU = FFN / kGrid;    // gate/up pairs per workgroup
    static constexpr int GU_LDS = 27;         // ... of them staged in LDS
    static constexpr int NLDS = cdiv(GU_LDS, kWaves);      // per wave (at most)
    static constexpr int NREG = (GU - GU_LDS) / kWaves;    // in registers
    static constexpr int PPT = NMAX / kThreads;     // positions per thread
    static constexpr int XQ = DIM / (4 * kThreads); // quartets of x per thread
    // LDS staging bytes: the slice's q, k and v rows (A), the gate/up pairs
    // of LDS (C)
    static constexpr int ST_A_BYTES = 3 * SLICE * (RB_DIM + SB_DIM);
    static constexpr int ST_GU_BYTES = 2 * GU_LDS * (RB_DIM + SB_DIM);
    static constexpr LayerLayout LAY = layer_layout(QT, DIM, FFN, DIM);
    static_assert(HEADS * GW == kGrid && HD % GW == 0 && SLICE == 2 * kWaves,
                  "sixteen head dims per workgroup: one q, k and v pair per wave");
    static_assert(DIM % kGrid == 0 && ROWS == 2 * kWaves, "one Wo / W2 row pair per wave");
    static_assert(FFN % kGrid == 0, "gate/up pairs split evenly over workgroups");
    static_assert(SLICE <= kWave && ROWS <= kWave && GU <= kWave,
                  "a workgroup's words of each exchange re-armed by one wave");
    static_assert((GU - GU_LDS) % kWaves == 0, "gate/up pairs in registers split evenly over waves");
    static_assert(DIM % (4 * kThreads) == 0 && NMAX % kThreads == 0,
                  "whole quartets and positions per thread");
    static_assert(DIM % 32 == 0 && FFN % 32 == 0 && BLK_DIM % kWave == 0, "block-aligned rows");
    static_assert(RB_DIM % 16 == 0 && RB_FFN % 16 == 0 && SB_DIM % 16 == 0 && SB_FFN % 16 == 0,
                  "16-byte DMA granules");
};

// LDS, in bytes. Phases with a dim-sized input hold its digits (XD) and
// the input itself (H); the gate/up rows staged during phase B sit at
// ST_GU until phase C has used them; phase D holds the activation as floats
// over XD, H and the start of ST_GU (ACT); phase A's q/k/v rows are staged
// at ST_A, clear of XD and H. The classifier's normalised x sits at ST_GU,
// its block sums of |x| and the screened argmax's row bounds after it.
template <class G> struct WideLds {
    static constexpr int XD = 0;
    static constexpr int H = XD + kLimbStride * G::BLK_DIM * 4;
    static constexpr int ST_GU = H + G::DIM * 4;
    static constexpr int ACT = 0;
    static constexpr int ST_A = ACT + G::FFN * 4;
    static constexpr int END = cmax(ST_GU + G::ST_GU_BYTES, ST_A + G::ST_A_BYTES);
    static constexpr int XSC = END;                // per block: digit scale, or sum
    static constexpr int QS = XSC + G::BLK_FFN * 4; // q, new k, new v: this slice
    static constexpr int KS = QS + G::SLICE * 4;
    static constexpr int VS = KS + G::SLICE * 4;
    static constexpr int CTX = VS + G::SLICE * 4;  // context partials [kWaves][SLICE]
    static constexpr int RED = CTX + kWaves * G::SLICE * 4;
    static constexpr int MISC = RED + 2 * kWaves * 4; // 16 ints
    static constexpr size_t BYTES = MISC + 16 * 4;
    static_assert(H % 16 == 0 && ST_GU % 16 == 0 && ST_A % 16 == 0 && XSC % 16 == 0,
                  "16-byte aligned regions");
    static_assert(ST_A >= H + G::DIM * 4, "q/k staging clear of the digits and h");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
    static_assert(G::ST_GU_BYTES >= (G::DIM + G::BLK_DIM + kScreenRowsMax) * 4,
                  "the classifier's x, its block sums and the row bounds at ST_GU");
};

typedef int i32x4 __attribute__((ext_vector_type(4)));

// First-poll delays (10 ns ticks of the real-time clock) of the two
// attention exchanges that no weight DMA precedes: the partial scores of a
// head group and the context. Polling right after the own publish floods
// the memory system with coherent reads of words most producers have not
// written yet. Measured on the Llama-2-7B shape (128 tokens at KV 512-639):
// none 1,639 us per token; scores 300 ns + context 600 ns 1,627; 1.2 +
// 2.4 us 1,596-1,597; 1.8 + 2.4 us 1,605; 2.4 + 2.4 us 1,623; 1.2 + 3.6 us
// 1,631. Re-swept with write-once words and the ring (two runs each, one
// box): scores 0.9 / 1.2 / 1.5 us 1,555.3-1,556.0 / 1,548.7-1,549.3 /
// 1,551.7-1,553.5; context 0.8 / 1.2 / 1.6 / 2.0 / 2.4 / 2.8 us
// 1,552.8-1,553.4 / 1,551.3-1,552.4 / 1,548.9-1,549.8 / 1,545.9-1,547.6 /
// 1,547.8-1,549.3 / 1,559.3-1,559.4 (2.0 kept). The other three exchanges
// (h into A, h after Wo, act) wait behind their phase's weight DMA
// already; 600 ns more on all three cost 9 us. Alone, two runs each: act
// none / 300 / 600 / 900 ns 1,549.8-1,550.9 / 1,553.3-1,554.3 /
// 1,559.5-1,560.8 / 1,562.3-1,563.0; h after Wo 300 / 600 ns
// 1,549.8-1,552.6 / 1,558.3-1,558.5 (none kept on both).
constexpr int kWidePollDelayScores = 120;
constexpr int kWidePollDelayContext = 200;
// The classifier's input (the last layer's h after W2): 600 ns as in the
// TinyLlama-shape kernel (1,548.8 against 1,549.7 us per token with none).
constexpr int kWidePollDelayClassifier = 60;

// Cache policy of the weight loads: non-temporal (nt, bit 1), as each
// weight byte is read once per token and the memory-side cache is left to
// the classifier.
constexpr int kWeightPolicy = 2;

// p (a global-memory pointer) as an opaque wave-uniform value: addresses
// derived from it are formed where they are used. It stays a global
// pointer, so accesses through it remain global (not flat) instructions.
template <class T>
__device__ __forceinline__ T *fresh(T *p)
{
    auto g = (__attribute__((address_space(1))) T *)p;
    asm volatile("" : "+s"(g));
    return (T *)g;
}

// LDS address (byte offset) of a generic pointer into shared memory.
__device__ __forceinline__ uint32_t lds_offset(const void *p)
{
    return uint32_t(reinterpret_cast<uintptr_t>(
        (const __attribute__((address_space(3))) char *)(p)));
}

// As dma (1 KB per wave instruction, lane i moving bytes [16 i, 16 i + 16)
// of its kilobyte, instructions spread over the waves; non-temporal), with
// the instruction written as asm: the compiler then does not track the
// copy, and so does not make every later LDS read wait for all of it (it
// cannot tell the staging regions apart). Completion: s_waitcnt vmcnt(0)
// in every wave, then a workgroup barrier (the next take).
__device__ __forceinline__ void dma_untracked(void *lds_dst, const void *src, int bytes)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int n = (bytes + 1023) >> 10;
    for (int i = wave_index(); i < n; i += kWaves) {
        const int off = (i << 10) + (lane << 4);
        const uint32_t m0 =
            __builtin_amdgcn_readfirstlane(lds_offset(static_cast<char *>(lds_dst) + (i << 10)));
        if (off < bytes)
            asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                         :
                         : "v"(static_cast<const char *>(src) + off), "s"(m0)
                         : "memory", "m0");
    }
}

// Buffer resource over one layer's weights: rows are then addressed by a
// wave-uniform byte offset and the lane's offset (one VGPR shared by every
// row), so no per-row 64-bit addresses are formed.
template <class G>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t layer_rsrc(const uint8_t *weights, int layer)
{
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(fresh(weights) + size_t(layer) * G::LAY.bytes), 0,
        int(G::LAY.bytes), 0x00020000);
}

// A lane's share of one quantised row: blocks b = lane + 64 j (j < CPL),
// their codes (16 bytes INT4, 32 bytes INT8) and fp16 scale bits.
template <int QT, int CPL> struct RowRegs {
    static constexpr int V = QT == 1 ? 1 : 2;
    uint4 w[CPL][2];
    uint16_t s[CPL];

    // The row whose codes start at byte `data` and scales at byte `scales`
    // of the layer (both wave-uniform). Every lane loads all CPL blocks
    // without a branch, so the loads issue back to back: blocks past the
    // row's end read the bytes after it (never used; beyond the layer the
    // buffer bound makes them zero).
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t layer, uint32_t data,
                                         uint32_t scales)
    {
        const int lane = opaque_lane_value(threadIdx.x & (kWave - 1));
#pragma unroll
        for (int j = 0; j < CPL; j++) {
#pragma unroll
            for (int v = 0; v < V; v++) {
                const i32x4 t = __builtin_amdgcn_raw_buffer_load_b128(
                    layer, 16 * (V * lane + v), data + 16 * V * kWave * j, kWeightPolicy);
                w[j][v] = make_uint4(t.x, t.y, t.z, t.w);
            }
            s[j] = uint16_t(__builtin_amdgcn_raw_buffer_load_b16(
                layer, 2 * lane, scales + 2 * kWave * j, kWeightPolicy));
        }
    }

    // The same share of a row staged in LDS (codes at row, scales at sc).
    __device__ __forceinline__ void read(const uint8_t *row, const uint16_t *sc)
    {
        const int lane = opaque_lane_value(threadIdx.x & (kWave - 1));
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int b = lane + kWave * j;
#pragma unroll
            for (int v = 0; v < V; v++)
                w[j][v] = reinterpret_cast<const uint4 *>(row)[V * b + v];
            s[j] = sc[b];
        }
    }
};

// Wave dot products of rows [0, count) with x (digits in LDS, per-block
// scales xsc), one block column at a time, so only one block's digits are
// in registers; each lane sums its blocks in the order j = 0, 1, ... as
// row_dot does. All lanes get out[i], i < count.
template <int QT, int CPL, int R>
__device__ __forceinline__ void rows_dot(const RowRegs<QT, CPL> (&rows)[R], int count,
                                         const uint32_t *xl, const float *xsc,
                                         float (&out)[R])
{
    const int lane = opaque_lane_value(threadIdx.x & (kWave - 1));
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++)
        acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int b = lane + kWave * j;
        uint4 d[6];
        load_digits(xl, b, d);
        const float sx = xsc[b];
#pragma unroll
        for (int i = 0; i < R; i++)
            if (i < count)
                acc[i] = fmaf(half_bits_to_float(rows[i].s[j]) * sx,
                              dot_words_digits<QT>(rows[i].w[j], d), acc[i]);
    }
#pragma unroll
    for (int i = 0; i < R; i++)
        out[i] = i < count ? wave_total(acc[i]) : 0.0f;
}

// As rows_dot for rows staged in LDS: row i's codes at base + code[i] and
// its fp16 scales at base + scale[i] (byte offsets); only one block's
// digits and one row's codes are in registers at a time.
template <int QT, int CPL, int R>
__device__ __forceinline__ void lds_rows_dot(const uint8_t *base, const int (&code)[R],
                                             const int (&scale)[R], int count,
                                             const uint32_t *xl, const float *xsc,
                                             float (&out)[R])
{
    const int lane = opaque_lane_value(threadIdx.x & (kWave - 1));
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++)
        acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int b = lane + kWave * j;
        uint4 d[6];
        load_digits(xl, b, d);
        const float sx = xsc[b];
#pragma unroll
        for (int i = 0; i < R; i++)
            if (i < count) {
                const uint4 *row = reinterpret_cast<const uint4 *>(base + code[i]);
                uint4 w[2];
                w[0] = row[(QT == 1 ? 1 : 2) * b];
                if (QT != 1)
                    w[1] = row[2 * b + 1];
                const uint16_t sc = reinterpret_cast<const uint16_t *>(base + scale[i])[b];
                acc[i] = fmaf(half_bits_to_float(sc) * sx, dot_words_digits<QT>(w, d), acc[i]);
            }
    }
#pragma unroll
    for (int i = 0; i < R; i++)
        out[i] = i < count ? wave_total(acc[i]) : 0.0f;
}

// Wave dot product of one row with x as swizzled floats in LDS and its
// block sums (ffn-sized x), as row_dot_floats, with the row in registers.
template <int QT, int CPL>
__device__ __forceinline__ float regs_dot_floats(const RowRegs<QT, CPL> &r, const float *xs,
                                                 const float *xsum, int blocks)
{
    const int lane = opaque_lane_value(threadIdx.x & (kWave - 1));
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
            const float d = QT == 1 ? dot_block_int4(r.w[j][0], xq) - 8.0f * xsum[b]
                                    : dot_block_int8(r.w[j][0], r.w[j][1], xq) -
                                          128.0f * xsum[b];
            acc += half_bits_to_float(r.s[j]) * d;
        }
    }
    return wave_total(acc);
}

// This workgroup's dims [SLICE part, +SLICE) of K or V rows at positions
// p = threadIdx.x + kThreads u (u < PPT) of one head, whose rows
// [0, max_seq) start at head_rows; no branch, so the loads issue back to
// back. Positions past max_seq read zero (buffer bound); rows at or past
// the current position are stale and never used.
template <class G>
__device__ __forceinline__ void load_kv_rows(float4 (&r)[G::PPT][4], const float *head_rows,
                                             int max_seq, int part)
{
    const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(head_rows), 0, max_seq * G::HD * int(sizeof(float)), 0x00020000);
    const int tid = opaque_lane_value(threadIdx.x);
#pragma unroll
    for (int u = 0; u < G::PPT; u++) {
        const int at = ((tid + kThreads * u) * G::HD + G::SLICE * part) * int(sizeof(float));
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const i32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rows, at + 16 * d, 0, 0);
            r[u][d] = make_float4(__int_as_float(t.x), __int_as_float(t.y),
                                  __int_as_float(t.z), __int_as_float(t.w));
        }
    }
}

// Digits of x = src * scale * w for quartets Q = threadIdx.x + kThreads u
// (u < XQ; w holds this thread's weights, loaded ahead). Ends with a
// barrier.
template <int QT, int XQ>
__device__ void stage_quartets(const float *src, const float4 (&w)[XQ], float scale,
                               uint32_t *xl, float *xsc)
{
    const int tid = opaque_lane_value(threadIdx.x);
#pragma unroll
    for (int u = 0; u < XQ; u++) {
        const int q = tid + kThreads * u;
        const float4 h = reinterpret_cast<const float4 *>(src)[q];
        const float4 x = make_float4(h.x * scale * w[u].x, h.y * scale * w[u].y,
                                     h.z * scale * w[u].z, h.w * scale * w[u].w);
        quartet_digits<QT>(x, q >> 3, q & 7, xl, xsc);
    }
    __syncthreads();
}

// This thread's norm weights for stage_quartets.
template <int XQ>
__device__ __forceinline__ void load_quartets(float4 (&w)[XQ], const float4 *src)
{
    const int tid = opaque_lane_value(threadIdx.x);
#pragma unroll
    for (int u = 0; u < XQ; u++)
        w[u] = src[tid + kThreads * u];
}

// Workgroup maximum of per-thread values; every thread gets it.
__device__ __forceinline__ float wg_max(float v, float *red)
{
    v = wave_maximum(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; w++)
        m = fmaxf(m, red[w]);
    return m;
}

template <class G, bool CLASSIFY>
__global__ __launch_bounds__(kThreads, 1) void wide_kernel(TokenArgs a)
{
    extern __shared__ float4 lds4[];
    uint8_t *lds = reinterpret_cast<uint8_t *>(lds4);
    using L = WideLds<G>;
    float *hbuf = reinterpret_cast<float *>(lds + L::H);
    uint32_t *xl = reinterpret_cast<uint32_t *>(lds + L::XD);
    float *act = reinterpret_cast<float *>(lds + L::ACT);
    float *xsc = reinterpret_cast<float *>(lds + L::XSC);
    float *qs = reinterpret_cast<float *>(lds + L::QS);
    float *ks = reinterpret_cast<float *>(lds + L::KS);
    float *vs = reinterpret_cast<float *>(lds + L::VS);
    float *ctxp = reinterpret_cast<float *>(lds + L::CTX);
    float *red = reinterpret_cast<float *>(lds + L::RED);
    int *misc = reinterpret_cast<int *>(lds + L::MISC);
    uint8_t *st_gu = lds + L::ST_GU, *st_a = lds + L::ST_A;
    float *xcls = reinterpret_cast<float *>(st_gu); // the classifier's x

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = wave_index();
    const int head = blockIdx.x % G::HEADS; // this workgroup's head
    const int part = blockIdx.x / G::HEADS; // and its dims [SLICE part, +SLICE)
    const int row0 = G::ROWS * blockIdx.x;  // its Wo / W2 rows, and h entries
    const int gu0 = G::GU * blockIdx.x;     // its gate/up pairs
    // first row of this workgroup's slice in the q, k and v matrices
    const int qkv0 = head * G::HD + G::SLICE * part;
    // wave w's Wo and W2 rows
    const int ra = row0 + wave, rb = row0 + kWaves + wave;
    // wave w's gate/up pairs: w, w + 8, ... below GU_LDS (LDS), then
    // GU_LDS + w + 8 i, i < NREG (registers)
    const int n_lds = (G::GU_LDS - wave + kWaves - 1) / kWaves;
    unsigned tag = a.tag_base;
    int *error = a.error;
    const size_t kv_layer = size_t(G::HEADS) * a.max_seq * G::HD;
    const int marks = marks_per_iteration(a.layer_count);
    auto mark = [&](int it, int k) {
        if (a.timeline != nullptr && int(blockIdx.x) < a.timeline_wgs && threadIdx.x == 0) {
            const int i = it * marks + k;
            if (i < a.timeline_cap)
                a.timeline[size_t(blockIdx.x) * a.timeline_cap + i] =
                    __builtin_amdgcn_s_memrealtime();
        }
    };
    // byte offsets of row `row` of matrix m inside a layer
    auto wdata = [&](int m, int row, int rb_) { return uint32_t(G::LAY.data[m] + size_t(row) * rb_); };
    auto wscales = [&](int m, int row, int sb) {
        return uint32_t(G::LAY.scales[m] + size_t(row) * sb);
    };
    auto layer_base = [&](int layer) { return fresh(a.weights) + size_t(layer) * G::LAY.bytes; };
    // rows [lo, lo + n) of matrix m into LDS: codes at `codes`, scales at
    // `scales` (LDS DMA; complete after the next take)
    auto stage = [&](uint8_t *codes, uint8_t *scales, int rb_, int sb, int layer, int m, int lo,
                     int n) {
        const uint8_t *base = layer_base(layer);
        dma_untracked(codes, base + G::LAY.data[m] + size_t(lo) * rb_, n * rb_);
        dma_untracked(scales, base + G::LAY.scales[m] + size_t(lo) * sb, n * sb);
    };
    auto norm = [&](int layer, bool ffn) {
        return reinterpret_cast<const float4 *>(layer_base(layer) +
                                                (ffn ? G::LAY.ffn_norm : G::LAY.attention_norm));
    };

    // Phase A's inputs, issued after the previous layer's publish (layer
    // 0: with the token) and before the wait for h: the slice's q, k and v
    // rows (LDS, ST_A: codes of the q, k, v rows, then their scales), this
    // thread's K rows of the cached positions and its attention-norm
    // quartets (registers).
    float4 kr[G::PPT][4];
    float4 nw[G::XQ];
    auto issue_a = [&](int layer) {
        uint8_t *sc = st_a + 3 * G::SLICE * G::RB_DIM;
#pragma unroll
        for (int m = 0; m < 3; m++)
            stage(st_a + m * G::SLICE * G::RB_DIM, sc + m * G::SLICE * G::SB_DIM, G::RB_DIM,
                  G::SB_DIM, layer, m, qkv0, G::SLICE);
        load_kv_rows<G>(kr,
                        fresh(a.k_cache) + layer * kv_layer + size_t(head) * a.max_seq * G::HD,
                        a.max_seq, part);
        load_quartets(nw, norm(layer, false));
    };

    // Write-once exchange words of iteration it, layer l: the context, h
    // after Wo, act, h after W2 (the partial scores stay tagged).
    constexpr int X_WO = G::DIM, X_ACT = 2 * G::DIM, X_DN = 2 * G::DIM + G::FFN;
    constexpr int X_STRIDE = X_DN + G::DIM;
    // the ring slice of the current (iteration, layer) step, advanced by one
    // per step (once_slice(it, layer, layer_count)); this step's words and
    // the previous step's
    int slice = 0;
    auto once = [&](int part) { return fresh(a.x_once) + size_t(slice) * X_STRIDE + part; };
    // the words of two steps back, which phase C re-arms
    auto once_back2 = [&](int part) {
        return fresh(a.x_once) + size_t(slice >= 2 ? slice - 2 : slice + kOnceRing - 2) * X_STRIDE +
               part;
    };

    int count = 0, done = 0, last_token = 0;
    // Tag of the hidden state the next classifier reads; 0 = hidden_in.
    unsigned hidden_tag = 0;
    // The same hidden state's write-once words.
    const float *hidden_once = nullptr;

    for (int it = 0; it < a.n_iter && !done; it++) {
        int token;
        const int pos = a.start_len + it;
        // RoPE factors of this wave's q/k pair at this position
        const float2 cs =
            fresh(a.rope)[size_t(pos) * (G::HD / 2) + (G::SLICE * part + 2 * wave) / 2];
        mark(it, 0);
        if (CLASSIFY) {
            // ---------------- final rmsnorm + classifier + argmax ----
            Slice<G::DIM> fw;
            fw.load(fresh(a.final_norm));
            float sq;
            if (hidden_tag == 0) {
                Slice<G::DIM> h;
                h.load(fresh(a.hidden_in));
                sq = h.store(hbuf);
                __syncthreads();
            } else {
                sq = take_once<G::DIM, false, kWidePollDelayClassifier, true>(hidden_once, hbuf,
                                                                              error);
            }
            const float scale = rms_scale(wg_sum(sq, red), G::DIM);
#pragma unroll
            for (int u = 0; u < Slice<G::DIM>::PER; u++) {
                const int i = threadIdx.x + u * kThreads;
                if (i < G::DIM)
                    xcls[i] = hbuf[i] * scale * fw.v[u];
            }
            __syncthreads();
            mark(it, 1);
            float best_v;
            int best_i;
            if (a.classifier8 != nullptr) {
                // digits in XD / XSC, block sums of |x| and row bounds at
                // ST_GU after x
                float *xl1 = xcls + G::DIM, *upper = xl1 + G::BLK_DIM;
                screen_x_digits<G::DIM>(xcls, xl, xsc, xl1);
                classifier_screened<G::DIM, true, 1, 2>(fresh(a.classifier), fresh(a.classifier8),
                                                  fresh(a.classifier8_scales), xcls, xl, xsc,
                                                  xl1, a.vocab, upper, red, best_v, best_i);
            } else {
                classifier_best<G::DIM, true>(fresh(a.classifier), xcls, a.vocab, best_v,
                                              best_i);
            }
            // every wave is past its reads of x before the q/k rows land
            __syncthreads();
            mark(it, 2);
            // the partial leaves first; layer 0's inputs then stream during
            // the argmax exchange
            argmax_publish(fresh(a.x_part), best_v, best_i, red, misc, tag);
            issue_a(0);
            bool failed_wait = false;
            const int bi = argmax_take(fresh(a.x_part), red, misc, tag, error, failed_wait);
            tag++;
            token = (bi >= 0 && bi < a.vocab) ? bi : 0;
            if (failed_wait)
                break;
            if (token == a.eos) {
                done = 1;
                break;
            }
            if (blockIdx.x == 0 && threadIdx.x == 0)
                a.tokens_out[count] = token;
            count++;
        } else {
            token = a.tokens_in[it];
            issue_a(0);
        }
        last_token = token;
        mark(it, 3);

        for (int l = 0; l < a.layer_count; l++) {
            const bool last = l + 1 == a.layer_count;
            const size_t head_rows = l * kv_layer + size_t(head) * a.max_seq * G::HD;

            // ------------------------------------- phase A: q/k/v slice --
            // (layer 0's inputs were issued with the token)
            if (l > 0)
                issue_a(l);
            float sq;
            if (l == 0) {
                Slice<G::DIM> e;
                e.load(fresh(a.embeddings) + size_t(token) * G::DIM);
                sq = e.store(hbuf);
                dma_wait();
            } else {
                sq = take_once<G::DIM, false, 0, true>(hidden_once, hbuf, error);
            }
            // this wave's residual inputs
            float res0 = hbuf[ra], res1 = hbuf[rb];
            stage_quartets<G::QT, G::XQ>(hbuf, nw, rms_scale(wg_sum(sq, red), G::DIM), xl, xsc);
            mark(it, 4 + 13 * l);
            {
                // wave w: q, k and v rows 2 w, 2 w + 1 of the slice
                int code[6], scale[6];
#pragma unroll
                for (int i = 0; i < 6; i++) {
                    const int r = (i >> 1) * G::SLICE + 2 * wave + (i & 1); // staged row
                    code[i] = r * G::RB_DIM;
                    scale[i] = 3 * G::SLICE * G::RB_DIM + r * G::SB_DIM;
                }
                float e[6];
                lds_rows_dot<G::QT, G::CPL_DIM>(st_a, code, scale, 6, xl, xsc, e);
                if (lane == 0) {
                    const int dd = 2 * wave;
                    const size_t at = head_rows + size_t(pos) * G::HD + G::SLICE * part + dd;
                    float qk[4];
#pragma unroll
                    for (int which = 0; which < 2; which++) {
                        const float even = e[2 * which], odd = e[2 * which + 1];
                        qk[2 * which] = fmaf(even, cs.x, -(odd * cs.y));
                        qk[2 * which + 1] = fmaf(even, cs.y, odd * cs.x);
                    }
                    qs[dd] = qk[0];
                    qs[dd + 1] = qk[1];
                    ks[dd] = qk[2];
                    ks[dd + 1] = qk[3];
                    vs[dd] = e[4];
                    vs[dd + 1] = e[5];
                    float *kc = fresh(a.k_cache) + at;
                    float *vc = fresh(a.v_cache) + at;
                    kc[0] = qk[2];
                    kc[1] = qk[3];
                    vc[0] = e[4];
                    vc[1] = e[5];
                }
            }
            // q/k/v of the slice are in LDS, and the q/k staging is free
            __syncthreads();
            mark(it, 5 + 13 * l);

            // ------------------------------ phase B: attention over dims --
            // V rows and this wave's Wo rows (registers) stream during the
            // score exchange
            float4 vr[G::PPT][4];
            load_kv_rows<G>(vr, fresh(a.v_cache) + head_rows, a.max_seq, part);
            RowRegs<G::QT, G::CPL_DIM> wo[2];
            wo[0].load(layer_rsrc<G>(a.weights, l), wdata(3, ra, G::RB_DIM),
                       wscales(3, ra, G::SB_DIM));
            wo[1].load(layer_rsrc<G>(a.weights, l), wdata(3, rb, G::RB_DIM),
                       wscales(3, rb, G::SB_DIM));
            const int n = pos + 1;
            uint64_t *xsc_g = fresh(a.x_scores) + size_t(head) * G::GW * G::NMAX;
            {
                float4 q[4];
#pragma unroll
                for (int d = 0; d < 4; d++)
                    q[d] = reinterpret_cast<const float4 *>(qs)[d];
#pragma unroll
                for (int u = 0; u < G::PPT; u++) {
                    const int p = threadIdx.x + kThreads * u;
                    if (p < n) {
                        float4 k[4];
#pragma unroll
                        for (int d = 0; d < 4; d++)
                            k[d] = p < pos ? kr[u][d] : reinterpret_cast<const float4 *>(ks)[d];
                        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                        for (int d = 0; d < 4; d += 2) {
                            a0 = fmaf(q[d].x, k[d].x, a0);
                            a1 = fmaf(q[d + 1].x, k[d + 1].x, a1);
                            a0 = fmaf(q[d].y, k[d].y, a0);
                            a1 = fmaf(q[d + 1].y, k[d + 1].y, a1);
                            a0 = fmaf(q[d].z, k[d].z, a0);
                            a1 = fmaf(q[d + 1].z, k[d + 1].z, a1);
                            a0 = fmaf(q[d].w, k[d].w, a0);
                            a1 = fmaf(q[d + 1].w, k[d + 1].w, a1);
                        }
                        put(xsc_g + size_t(part) * G::NMAX + p, a0 + a1, tag);
                    }
                }
            }
            mark(it, 6 + 13 * l);
            // scores: the group's partials summed in a fixed order
            float s[G::PPT];
            {
                uint64_t v[G::PPT][G::GW];
                const int tid = opaque_lane_value(threadIdx.x);
                {
                    const unsigned long long until =
                        __builtin_amdgcn_s_memrealtime() + kWidePollDelayScores;
                    while (__builtin_amdgcn_s_memrealtime() < until)
                        __builtin_amdgcn_s_sleep(1);
                }
#pragma unroll
                for (int u = 0; u < G::PPT; u++) {
                    const int p = tid + kThreads * u;
#pragma unroll
                    for (int g = 0; g < G::GW; g++)
                        v[u][g] = p < n ? load_coherent(xsc_g + size_t(g) * G::NMAX + p)
                                        : uint64_t(tag) << 32;
                }
                for (int spins = 0;; spins++) {
                    bool stale = false;
#pragma unroll
                    for (int u = 0; u < G::PPT; u++)
#pragma unroll
                        for (int g = 0; g < G::GW; g++)
                            stale |= unsigned(v[u][g] >> 32) != tag;
                    if (!stale)
                        break;
                    if ((spins & 63) == 63 && failed(error))
                        break;
                    if (spins > kSpinLimit) {
                        __hip_atomic_store(error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
#pragma unroll
                    for (int u = 0; u < G::PPT; u++)
#pragma unroll
                        for (int g = 0; g < G::GW; g++)
                            if (unsigned(v[u][g] >> 32) != tag)
                                v[u][g] = load_coherent(xsc_g + size_t(g) * G::NMAX + tid +
                                                        kThreads * u);
                }
#pragma unroll
                for (int u = 0; u < G::PPT; u++) {
                    float t = 0.0f;
#pragma unroll
                    for (int g = 0; g < G::GW; g++)
                        t += __uint_as_float(unsigned(v[u][g]));
                    s[u] = tid + kThreads * u < n ? t * a.attn_scale : -INFINITY;
                }
            }
            tag++;
            float mx = s[0];
#pragma unroll
            for (int u = 1; u < G::PPT; u++)
                mx = fmaxf(mx, s[u]);
            mx = wg_max(mx, red);
            float total = 0.0f;
            float c[G::SLICE];
#pragma unroll
            for (int d = 0; d < G::SLICE; d++)
                c[d] = 0.0f;
#pragma unroll
            for (int u = 0; u < G::PPT; u++) {
                const int p = threadIdx.x + kThreads * u;
                if (p < n) {
                    const float e = expf(s[u] - mx);
                    total += e;
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const float4 v =
                            p < pos ? vr[u][d] : reinterpret_cast<const float4 *>(vs)[d];
                        c[4 * d] = fmaf(e, v.x, c[4 * d]);
                        c[4 * d + 1] = fmaf(e, v.y, c[4 * d + 1]);
                        c[4 * d + 2] = fmaf(e, v.z, c[4 * d + 2]);
                        c[4 * d + 3] = fmaf(e, v.w, c[4 * d + 3]);
                    }
                }
            }
            total = wg_sum(total, red + kWaves);
#pragma unroll
            for (int d = 0; d < G::SLICE; d++) {
                const float t = wave_total(c[d]);
                if (lane == d)
                    ctxp[wave * G::SLICE + d] = t;
            }
            __syncthreads();
            if (threadIdx.x < G::SLICE) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; w++)
                    t += ctxp[w * G::SLICE + threadIdx.x];
                put_once(once(0) + qkv0 + threadIdx.x, t / total);
            }
            tag++;
            mark(it, 7 + 13 * l);

            // ------------------------------------ Wo rows + residual --
            take_once<G::DIM, false, kWidePollDelayContext, true>(once(0), hbuf, error);
            {
                float4 ones[G::XQ];
#pragma unroll
                for (int u = 0; u < G::XQ; u++)
                    ones[u] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
                stage_quartets<G::QT, G::XQ>(hbuf, ones, 1.0f, xl, xsc);
            }
            mark(it, 8 + 13 * l);
            {
                float y[2];
                rows_dot(wo, 2, xl, xsc, y);
                res0 += y[0];
                res1 += y[1];
                if (lane == 0) {
                    put_once(once(X_WO) + ra, res0);
                    put_once(once(X_WO) + rb, res1);
                }
            }
            tag++;
            mark(it, 9 + 13 * l);

            // ------------------------------------------ phase C: gate/up --
            // The gate/up pairs of LDS (ST_GU: gate codes, up codes, then
            // their scales) and this wave's pairs in registers, issued after
            // the publish of h and before its wait.
            {
                uint8_t *sc = st_gu + 2 * G::GU_LDS * G::RB_DIM;
                stage(st_gu, sc, G::RB_DIM, G::SB_DIM, l, 4, gu0, G::GU_LDS);
                stage(st_gu + G::GU_LDS * G::RB_DIM, sc + G::GU_LDS * G::SB_DIM, G::RB_DIM,
                      G::SB_DIM, l, 5, gu0, G::GU_LDS);
            }
            RowRegs<G::QT, G::CPL_DIM> wr[2 * G::NREG];
#pragma unroll
            for (int i = 0; i < G::NREG; i++) {
                const int r = gu0 + G::GU_LDS + wave + kWaves * i;
                wr[2 * i].load(layer_rsrc<G>(a.weights, l), wdata(4, r, G::RB_DIM),
                               wscales(4, r, G::SB_DIM));
                wr[2 * i + 1].load(layer_rsrc<G>(a.weights, l), wdata(5, r, G::RB_DIM),
                                   wscales(5, r, G::SB_DIM));
            }
            load_quartets(nw, norm(l, true));
            // Every workgroup has taken the previous step's h after Wo, so
            // every word of the step before it has been read: this
            // workgroup's words of that step go back to kUnset for the
            // slice's next use (this take retires the stores).
            if (it * a.layer_count + l >= 2) {
                rearm_words(once_back2(0) + qkv0, G::SLICE, 0);
                rearm_words(once_back2(X_WO) + row0, G::ROWS, 1);
                rearm_words(once_back2(X_ACT) + gu0, G::GU, 2);
                rearm_words(once_back2(X_DN) + row0, G::ROWS, 3);
            }
            sq = take_once<G::DIM, false, 0, true>(once(X_WO), hbuf, error);
            stage_quartets<G::QT, G::XQ>(hbuf, nw, rms_scale(wg_sum(sq, red), G::DIM), xl, xsc);
            mark(it, 10 + 13 * l);
            {
                float y[2 * G::NREG];
                rows_dot(wr, 2 * G::NREG, xl, xsc, y);
#pragma unroll
                for (int i = 0; i < G::NREG; i++)
                    if (lane == 0) {
                        const float g = y[2 * i], u = y[2 * i + 1];
                        put_once(once(X_ACT) + gu0 + G::GU_LDS + wave + kWaves * i,
                                 g / (1.0f + expf(-g)) * u);
                    }
            }
            {
                int code[2 * G::NLDS], scale[2 * G::NLDS];
#pragma unroll
                for (int i = 0; i < G::NLDS; i++) {
                    const int p = wave + kWaves * i; // staged pair
                    code[2 * i] = p * G::RB_DIM;
                    code[2 * i + 1] = (G::GU_LDS + p) * G::RB_DIM;
                    scale[2 * i] = 2 * G::GU_LDS * G::RB_DIM + p * G::SB_DIM;
                    scale[2 * i + 1] = 2 * G::GU_LDS * G::RB_DIM + (G::GU_LDS + p) * G::SB_DIM;
                }
                float y[2 * G::NLDS];
                lds_rows_dot<G::QT, G::CPL_DIM>(st_gu, code, scale, 2 * n_lds, xl, xsc, y);
#pragma unroll
                for (int i = 0; i < G::NLDS; i++)
                    if (i < n_lds && lane == 0) {
                        const float g = y[2 * i], u = y[2 * i + 1];
                        put_once(once(X_ACT) + gu0 + wave + kWaves * i,
                                 g / (1.0f + expf(-g)) * u);
                    }
            }
            tag++;
            // every wave is past its reads of the gate/up staging, which the
            // activation overwrites
            __syncthreads();
            mark(it, 11 + 13 * l);

            // --------------------------------------------- phase D: down --
            // this wave's W2 rows stream while the activation is exchanged
            RowRegs<G::QT, G::CPL_FFN> wd[2];
            wd[0].load(layer_rsrc<G>(a.weights, l), wdata(6, ra, G::RB_FFN),
                       wscales(6, ra, G::SB_FFN));
            wd[1].load(layer_rsrc<G>(a.weights, l), wdata(6, rb, G::RB_FFN),
                       wscales(6, rb, G::SB_FFN));
            take_once<G::FFN, true, 0, true>(once(X_ACT), act, error);
            block_sums(act, xsc, G::FFN);
            mark(it, 12 + 13 * l);
            res0 += regs_dot_floats(wd[0], act, xsc, G::BLK_FFN);
            res1 += regs_dot_floats(wd[1], act, xsc, G::BLK_FFN);
            if (lane == 0) {
                put_once(once(X_DN) + ra, res0);
                put_once(once(X_DN) + rb, res1);
                if (last && it + 1 == a.n_iter) {
                    a.hidden_out[ra] = res0;
                    a.hidden_out[rb] = res1;
                }
            }
            hidden_tag = tag;
            hidden_once = once(X_DN);
            slice = slice + 1 == kOnceRing ? 0 : slice + 1;
            tag++;
            mark(it, 13 + 13 * l);
            // every wave is past its reads of the activation, which the next
            // take overwrites
            __syncthreads();
            mark(it, 14 + 13 * l);
            mark(it, 16 + 13 * l);
        }
        // The generate loop learns of a failed wait in the next argmax
        // exchange (every wait gives up once the flag is set, so the grid
        // drains either way); the prefill loop checks here.
        if (!CLASSIFY && wg_failed(error, misc + 8))
            break;
    }
    // hidden_out after an early stop (eos): the state the loop ended with
    if (done && hidden_tag != 0) {
        take_once<G::DIM, false, 0, true>(hidden_once, hbuf, error);
        for (int i = threadIdx.x; i < G::DIM; i += kThreads)
            if (blockIdx.x == 0)
                a.hidden_out[i] = hbuf[i];
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.state->count = count;
        a.state->done = done;
        a.state->token = last_token;
    }
}

// Llama-2-7B: dim 4096, 32 heads of 128 (MHA), ffn 11008, INT4 rows,
// contexts up to 1024 positions.
using Llama7bInt4 = Wide<1, 4096, 11008, 32, 128, 1024>;

template <class G>
bool wide_shape_is(const DecodeShape &s)
{
    return s.dim == G::DIM && s.ffn_dim == G::FFN && s.heads == G::HEADS &&
           s.kv_heads == G::HEADS && s.head_dim == G::HD;
}

template <class G, bool CLASSIFY>
void wide_launch_as(const TokenArgs &args, hipStream_t stream)
{
    const auto kernel = wide_kernel<G, CLASSIFY>;
    hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  int(WideLds<G>::BYTES)),
              "hipFuncSetAttribute");
    int per_cu = 0;
    hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                  &per_cu, reinterpret_cast<const void *>(kernel), kThreads,
                  WideLds<G>::BYTES),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    int device = 0, cus = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
              "hipDeviceGetAttribute");
    require(per_cu >= 1 && cus >= kGrid, NUT_EDEVICE,
            "token kernel: grid does not fit the device");
    require(args.start_len >= 0 && args.start_len + args.n_iter <= G::NMAX &&
                args.start_len + args.n_iter <= args.max_seq,
            NUT_EINVAL, "token kernel: context exceeds the attention pass");
    require(token_tags_needed(args.n_iter, args.layer_count) <= (1ll << kTagShift), NUT_EINVAL,
            "token kernel: launch exceeds its exchange tag range");
    require(args.x_once != nullptr, NUT_EINVAL,
            "token kernel: the wide kernel needs its write-once exchange words");
    require(args.x_scores != nullptr, NUT_EINVAL,
            "token kernel: head-dim attention needs its score buffer");
    TokenArgs a = args;
    void *params[] = {&a};
    hip_check(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(kernel), dim3(kGrid),
                                         dim3(kThreads), params, WideLds<G>::BYTES, stream),
              "token kernel launch");
}

} // namespace

int wide_kernel_positions(int type, const DecodeShape &s)
{
    if (type == Llama7bInt4::QT && wide_shape_is<Llama7bInt4>(s))
        return Llama7bInt4::NMAX;
    return 0;
}

size_t wide_kernel_score_entries(const DecodeShape &s)
{
    if (wide_shape_is<Llama7bInt4>(s))
        return size_t(Llama7bInt4::HEADS) * Llama7bInt4::GW * Llama7bInt4::NMAX;
    return 0;
}

void launch_wide_kernel(int type, const DecodeShape &s, const TokenArgs &a, hipStream_t stream)
{
    require(wide_kernel_positions(type, s) > 0, NUT_EINVAL, "token kernel: unsupported shape");
    if (a.classify)
        wide_launch_as<Llama7bInt4, true>(a, stream);
    else
        wide_launch_as<Llama7bInt4, false>(a, stream);
}

} // namespace nut
