// persistent.hip — the quantised token loop as one cooperative kernel.
//
// One workgroup per CU (256 x 512 threads) runs every phase of every token:
//   A  rmsnorm(h) -> Q/K/V rows, RoPE, K/V cache store
//   B  GQA attention over positions 0..pos for all heads, then Wo rows and
//      the residual add
//   C  rmsnorm(h) -> gate/up rows, silu(gate) * up
//   D  W2 rows and the residual add
// and, when generating, the final rmsnorm + fp32 classifier + first-index
// argmax (src/generate.cpp:195-207) before each decode step.
//
// Phases exchange activations through HBM in words written with agent-scope
// (sc1) stores; a consumer polls the words it needs until they hold the
// producing phase's output, so the flag is the data itself and no cache-wide
// writeback or invalidate is needed. Every exchange of a (token, layer) step
// has write-once 32-bit words of its own (unset until written) in a ring of
// three step slices, each re-armed by its producers once every consumer has
// read it; split attention's per-position partials and the argmax reuse
// their words with 64-bit (value, tag) words.
//
// Latency hiding: before a workgroup waits for a phase's input, it starts
// LDS DMA (global_load_lds_dwordx4) of that phase's weight rows — and, for
// attention, of the K/V rows of earlier positions — so HBM streams during
// the wait and nothing is held in registers across it.
//
// Every wait is bounded: on timeout the kernel raises an error flag that all
// waits observe, and every workgroup runs to the end.
#include "persistent.hpp"
#include "runtime.hpp"
#include "token_device.hpp"


namespace nut {

namespace {

// Wait before each exchange's first poll, in 10 ns ticks of s_memrealtime.
// A workgroup that polls right after its own publish re-reads words most
// producers have not written yet, and 256 workgroups doing so flood the
// memory system with coherent reads that slow every producer's publish and
// every consumer's later rounds. Measured per exchange (TinyLlama INT4, 16
// tokens: 423 us per token with no delays, 388 with the first set; INT8 at
// KV 2048-2175, split attention: 602 -> 514): into phases A (h after W2) and
// D (act) 450 ns, into B (q/k/v) and C (h after Wo), which follow a larger
// weight DMA that already delays their polls, 150 ns; with split attention
// 600 and 300 ns, and 900 ns for its partials and merged context. Re-swept
// for the fused attention once the attention scores and the classifier
// had become faster: A 300, B 50, C 150, D 600 ns (361.2 -> 357.7 us per
// token, two alternating runs each on one box). Other points of the
// sweep: A 150, B 0 366.9 against 360.2 for the first set; A 450, B 0,
// D 600 359.0 and A 300, B 0, D 900 361.7 against 358.5 for A 300, B 0,
// D 600.
// Split attention's partials and merged context, swept on INT8 at KV
// 2048-2175 (two runs each, one box): 900 ns both 479.2 us per token;
// 600 / 600 490.1, 300 / 300 526.5, 600 / 300 518.3, 300 / 600 500.6,
// 1,200 / 1,200 491.5, 1,500 / 1,500 508.1, 1,200 / 900 487.9, 900 / 1,200
// 484.7. The classifier's input (the last layer's h after W2), swept on
// TinyLlama INT4 once the generate loop no longer read the error flag in
// a round trip of its own before it (three runs each): none 345.6 us per
// token, 300 ns 344.0, 600 ns 344.0. Once phases A and C published after
// a barrier (two runs each, one box): B 0, 50, 150 ns 340.3-340.8,
// 340.2-340.2, 339.4-339.7 us per token (150 ns kept); A 150, 300,
// 450 ns 339.6-340.5, 340.2, 343.9-344.2; then D (three runs each) 600,
// 750, 900, 1,050 ns 338.4-339.4, 336.1-336.8, 338.6-340.4, 345.9-348.2
// (750 ns kept; the act exchange 1.62 -> 1.49 us), C 50, 300 ns no
// better than 150; with split attention D 450, 900 ns no better than 600,
// and A 450 / 750, B 150 / 450, C 150 / 450 ns all within 0.5 us of
// 469.5-469.8 us per token (INT8 at KV 2048-2175). The classifier's input
// then (three runs each): 300, 600, 900 ns 335.8-336.5, 337.1-338.1,
// 336.1-337.1 us per token (300 ns kept).
template <bool LONG> struct PollDelay {
    static constexpr int A = LONG ? 60 : 30, B = LONG ? 30 : 15;
    static constexpr int C = LONG ? 30 : 15, D = LONG ? 60 : 75;
    static constexpr int PARTIALS = 90, CONTEXT = 90;
    static constexpr int CLASSIFIER = 30;
};

template <int QT_, int DIM_, int FFN_, int HEADS_, int KVH_, int HD_, int NP_>
struct Geo {
    static constexpr int QT = QT_, DIM = DIM_, FFN = FFN_, HEADS = HEADS_;
    static constexpr int KVH = KVH_, HD = HD_;
    static constexpr int NP = NP_; // positions of the fused attention
    static constexpr int KVD = KVH * HD, GROUP = HEADS / KVH;
    static constexpr int HPW = HEADS / kWaves; // attention heads per wave
    static constexpr int BLK_DIM = DIM / 32, BLK_FFN = FFN / 32;
    static constexpr int CPL_DIM = cdiv(BLK_DIM, kWave); // blocks per lane
    static constexpr int CPL_FFN = cdiv(BLK_FFN, kWave);
    // bytes of one quantised row (data, fp16 scales) for input dim / ffn
    static constexpr int RB_DIM = QT == 1 ? DIM / 2 : DIM;
    static constexpr int RB_FFN = QT == 1 ? FFN / 2 : FFN;
    static constexpr int SB_DIM = 2 * BLK_DIM, SB_FFN = 2 * BLK_FFN;
    // rows one workgroup owns in each phase (upper bounds)
    static constexpr int ROWS_QKV = 2 * cdiv((DIM + 2 * KVD) / 2, kGrid);
    static constexpr int ROWS_WO = cdiv(DIM, kGrid);
    static constexpr int ROWS_GU = 2 * cdiv(FFN, kGrid);
    static constexpr int ROWS_DN = cdiv(DIM, kGrid);
    // LDS staging: region 1 holds, in turn, K/V rows and the QKV, gate/up
    // and down weight rows; region 2 the Wo rows (live across attention)
    // K/V staging rows padded to KROW floats (one spare 16-byte granule)
    // so lanes reading the same column of consecutive rows hit distinct
    // LDS banks
    static constexpr int KROW = HD + 4;
    static constexpr int KV_BYTES = 2 * KVH * NP * KROW * 4;
    static constexpr int W_QKV = ROWS_QKV * (RB_DIM + SB_DIM);
    static constexpr int W_GU = ROWS_GU * (RB_DIM + SB_DIM);
    static constexpr int W_DN = ROWS_DN * (RB_FFN + SB_FFN);
    static constexpr int W_WO = ROWS_WO * (RB_DIM + SB_DIM);
    // Fused attention by KV head group: group g (KV head g) owns the q rows
    // of its GROUP query heads, then its k and v rows (GR rows), over the
    // WGS_G workgroups of the group, GR_WG rows each; and the Wo partial
    // sums over its GQ context columns, WO_WG rows per workgroup (WO_SEG
    // bytes and WO_BLK blocks of each row).
    static constexpr int GQ = GROUP * HD, GR = GQ + 2 * HD;
    static constexpr int WGS_G = kGrid / KVH;
    static constexpr int GR_WG = GR / WGS_G, WO_WG = DIM / WGS_G;
    static constexpr int WO_SEG = RB_DIM / KVH, WO_BLK = BLK_DIM / KVH;
    static constexpr int W_WO_G = WO_WG * (WO_SEG + 2 * WO_BLK);
    // region 1 holds, in turn, the K/V staging (packed by the live position
    // count) and the QKV, gate/up and W2 rows of a phase
    static constexpr int R1 = cmax(cmax(KV_BYTES, W_QKV), cmax(W_GU, W_DN));
    static constexpr int R2 = cmax(W_WO, W_WO_G);
    // Split attention for long contexts: workgroup b takes KV head
    // b / SPLITS and the b % SPLITS-th run of at most PMAX positions.
    static constexpr int SPLITS = kGrid / KVH;
    static constexpr int PMAX = 64;
    static_assert(SPLITS == kWave, "one merge lane per split");
    static_assert(2 * PMAX * KROW * 4 <= R1 && GROUP * PMAX <= kWaves * HPW * NP,
                  "split attention staging");
    static_assert(GROUP == 2 * HPW && kGrid == HEADS * (HD / 8),
                  "split attention: two waves per KV head, eight context values per merger");
    // weight arena layout of one layer
    static constexpr LayerLayout LAY = layer_layout(QT, DIM, FFN, KVD);
    static_assert(DIM % 32 == 0 && FFN % 32 == 0, "block-aligned rows");
    static_assert(RB_FFN % 16 == 0 && SB_FFN % 16 == 0 && SB_DIM % 16 == 0,
                  "16-byte DMA granules");
    static_assert(HEADS % kWaves == 0, "heads split over waves");
    static_assert(HD == 64 && HPW * (HD / 4) == kWave && GROUP % HPW == 0,
                  "attention: 16 lanes per head row, a wave's heads share a kv head");
    static_assert((DIM + 2 * KVD) % 2 == 0 && KVD % 2 == 0, "row pairs");
    static_assert(KVH == 4 && GR % WGS_G == 0 && GR_WG % 2 == 0 && GR_WG <= ROWS_QKV &&
                      GR_WG / 2 <= kWaves && GQ % HD == 0,
                  "fused attention: a KV head's q/k/v row pairs over two XCDs' workgroups");
    static_assert(GROUP == kWaves && HD == kWave && NP <= kWave && GQ / 4 <= kThreads,
                  "fused attention: a wave per query head, a lane per dim and per position");
    static_assert(DIM % WGS_G == 0 && WO_BLK == 16 && WO_WG == 4 * kWaves && WO_SEG % 16 == 0,
                  "fused attention Wo: four rows of 16 blocks per wave");
    static_assert(GR_WG <= kWave && WO_WG <= kWave && ROWS_GU / 2 <= kWave &&
                      ROWS_DN <= kWave && ROWS_WO <= kWave && HD / 8 == kWaves,
                  "a workgroup's words of each exchange re-armed by one wave");
};

// ------------------------------------------------- split attention --

// dst[i] = value of *addr(i) once tagged, i < N; as take (a first-poll
// delay of DELAY ticks, batched re-polls, bounded), for words scattered over
// an exchange buffer. Ends with a barrier.
template <int N, int DELAY, class Addr>
__device__ void take_words(Addr addr, float *dst, unsigned tag, int *error)
{
    constexpr int PER = cdiv(N, kThreads);
    if (DELAY > 0) {
        const unsigned long long until = __builtin_amdgcn_s_memrealtime() + DELAY;
        while (__builtin_amdgcn_s_memrealtime() < until)
            __builtin_amdgcn_s_sleep(1);
    }
    uint64_t v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + u * kThreads;
        v[u] = i < N ? load_coherent(addr(i)) : uint64_t(tag) << 32;
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
            __hip_atomic_store(error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < PER; u++)
            if (unsigned(v[u] >> 32) != tag)
                v[u] = load_coherent(addr(threadIdx.x + u * kThreads));
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + u * kThreads;
        if (i < N)
            dst[i] = __uint_as_float(unsigned(v[u]));
    }
    __syncthreads();
}

// Attention of a long context split over the grid (src/quant_model.cpp:
// 45-108 computes the same softmax over all positions at once). Workgroup
// b owns KV head ag = b / SPLITS and its cnt positions [ap0, ap1) (K and V
// rows staged at kst / vst, q of the group's heads at qkv): wave w
// computes, for query head w of the KV head's group, the run's maximum
// score m, l = sum exp(s_p - m) and
// o = sum exp(s_p - m) V_p, published with `tag` as x_apart words
// [b][head][o 0..HD-1, m, l]. Then workgroup b merges context values
// 8 (b % 8) .. +7 of head b / 8 over its KV head's SPLITS runs (wave w
// value w, lane sp run sp): M = max m, context = sum e^(m - M) o / sum
// e^(m - M) l, published as write-once words at ctx_out. mb: LDS,
// SPLITS * 10 floats.
template <class G>
__device__ void split_attention(int cnt, int ag, const float *kst, const float *vst,
                                const float *qkv, float *scores, float *mb,
                                const TokenArgs &a, float *ctx_out, unsigned tag, int *error)
{
    static_assert(G::GROUP == kWaves && G::PMAX == kWave && G::HD == kWave,
                  "split attention: a wave per query head, a lane per position and per dim");
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    {
        // wave w: query head w of the group; lane p: position p's score,
        // then lane d: context dim d
        const float4 *q4 = reinterpret_cast<const float4 *>(qkv + wave * G::HD);
        float sv = -INFINITY;
        if (lane < cnt) {
            const float4 *k4 = reinterpret_cast<const float4 *>(kst + lane * G::KROW);
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int d4 = 0; d4 < 16; d4 += 2) {
                const float4 k0 = k4[d4], q0 = q4[d4];
                const float4 k1 = k4[d4 + 1], q1 = q4[d4 + 1];
                a0 = fmaf(q0.x, k0.x, a0);
                a1 = fmaf(q1.x, k1.x, a1);
                a0 = fmaf(q0.y, k0.y, a0);
                a1 = fmaf(q1.y, k1.y, a1);
                a0 = fmaf(q0.z, k0.z, a0);
                a1 = fmaf(q1.z, k1.z, a1);
                a0 = fmaf(q0.w, k0.w, a0);
                a1 = fmaf(q1.w, k1.w, a1);
            }
            sv = (a0 + a1) * a.attn_scale;
        }
        const float m = wave_maximum(sv);
        const float e = lane < cnt ? expf(sv - m) : 0.0f;
        const float total = wave_total(e);
        float *sc = scores + wave * G::PMAX;
        sc[lane] = e;
        // the wave's weights, written by every lane, before any lane reads
        // them (LDS runs one wave's accesses in order; the fences keep the
        // compiler's order)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float o = 0.0f;
#pragma unroll 8
        for (int p = 0; p < cnt; p++)
            o = fmaf(sc[p], vst[p * G::KROW + lane], o);
        uint64_t *dst = a.x_apart + size_t(blockIdx.x * G::GROUP + wave) * (G::HD + 2);
        put(dst + lane, o, tag);
        if (lane == 0) {
            put(dst + G::HD, m, tag);
            put(dst + G::HD + 1, total, tag);
        }
    }
    const int mh = blockIdx.x >> 3, md0 = (blockIdx.x & 7) * 8;
    const int mg = mh / G::GROUP, mhl = mh % G::GROUP;
    take_words<G::SPLITS * 10, PollDelay<true>::PARTIALS>(
        [&](int i) {
            const int sp = i / 10, j = i - sp * 10;
            return a.x_apart + size_t((mg * G::SPLITS + sp) * G::GROUP + mhl) * (G::HD + 2) +
                   (j < 8 ? md0 + j : G::HD + j - 8);
        },
        mb, tag, error);
    {
        // wave w merges context value md0 + w
        const float pm = mb[lane * 10 + 8], pl = mb[lane * 10 + 9];
        const float mx = wave_maximum(pm);
        const float w = pm == -INFINITY ? 0.0f : expf(pm - mx);
        const float total = wave_total(w * pl);
        const float c = wave_total(w * mb[lane * 10 + wave]);
        if (lane == 0)
            put_once(ctx_out + mh * G::HD + md0 + wave, c / total);
    }
}

// LDS DMA of `rows` segments of `seg` bytes (a multiple of 16), row r at
// src + r * stride, packed in LDS (segment r at lds_dst + r * seg); issued
// as dma() is, with the same completion.
template <int POLICY = kStreamPolicy>
__device__ __forceinline__ void dma_segments(uint8_t *lds_dst, const uint8_t *src, int rows,
                                             int seg, int stride)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int per = seg >> 4; // granules per segment
    const int instrs = (rows * per + kWave - 1) / kWave;
    for (int i = wave_index(); i < instrs; i += kWaves) {
        const int k = i * kWave + lane, row = k / per, g = k - row * per;
        if (row < rows)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(src + size_t(row) * stride +
                                                                 g * 16),
                (__attribute__((address_space(3))) void *)(lds_dst + i * 1024), 16, 0,
                POLICY);
    }
}

// ------------------------------------------------------------- kernel --

template <class G> struct Lds {
    static constexpr int XN = cmax(G::FFN, G::DIM);
    static constexpr int H = 0;                      // raw h [DIM]
    static constexpr int X = H + G::DIM;             // swizzled x, then its digits
    static constexpr int XSC = X + XN; // per block: digit scale, or sum (ffn)
    static constexpr int QKV = XSC + XN / 32;        // q, k, v staging
    static constexpr int SCORES = QKV + G::DIM + 2 * G::KVD;
    static constexpr int R1 = cdiv(SCORES + kWaves * G::HPW * G::NP, 4) * 4;
    static constexpr int R2 = R1 + G::R1 / 4;
    static constexpr int RED = R2 + G::R2 / 4;
    static constexpr int MISC = RED + 2 * kWaves; // 16 ints
    static constexpr int TOTAL = MISC + 16;
    static constexpr size_t BYTES = size_t(TOTAL) * sizeof(float);
    static_assert(BYTES <= 160 * 1024, "LDS budget");
    static_assert(kWaves * G::HPW * G::NP >= kScreenRowsMax,
                  "the screened classifier's upper bounds fit the scores region");
    static_assert(kWaves * G::HPW * G::NP >= G::ROWS_GU &&
                      kWaves * G::HPW * G::NP >= G::GR_WG,
                  "phase A's q/k/v and phase C's gate and up results fit the scores region");
    static_assert(G::R1 >= 4 * G::DIM && G::DIM + 2 * G::KVD >= G::DIM / 32,
                  "the classifier's x in region 1, its block sums of |x| over q/k/v");
};

// CLASSIFY: the generate loop (classifier + argmax first in every
// iteration); otherwise the prefill loop over a.tokens_in. Two kernels, so
// profiles tell the launches apart.
template <class G, bool CLASSIFY, bool LONG>
__global__ __launch_bounds__(kThreads, 1) void token_kernel(TokenArgs a)
{
    extern __shared__ float4 lds4[];
    float *lds = reinterpret_cast<float *>(lds4);
    using L = Lds<G>;
    float *h_raw = lds + L::H, *xs = lds + L::X, *xsc = lds + L::XSC;
    uint32_t *xl = reinterpret_cast<uint32_t *>(xs); // x's digits (dim-sized phases)
    float *qkv = lds + L::QKV, *scores = lds + L::SCORES, *red = lds + L::RED;
    uint8_t *r1 = reinterpret_cast<uint8_t *>(lds + L::R1);
    uint8_t *r2 = reinterpret_cast<uint8_t *>(lds + L::R2);
    // K/V staging of an n-position step: K [KVH][n][KROW], then V
    float *kst = lds + L::R1;
    int *misc = reinterpret_cast<int *>(lds + L::MISC);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = wave_index();
    unsigned tag = a.tag_base;
    int *error = a.error;
    const size_t kv_layer = size_t(G::KVH) * a.max_seq * G::HD;
    const int marks = marks_per_iteration(a.layer_count);
    // Phase timeline: recorded workgroups stamp entry k of iteration `it`.
    auto mark = [&](int it, int k) {
        if (a.timeline != nullptr && int(blockIdx.x) < a.timeline_wgs &&
            threadIdx.x == 0) {
            const int i = it * marks + k;
            if (i < a.timeline_cap)
                a.timeline[size_t(blockIdx.x) * a.timeline_cap + i] =
                    __builtin_amdgcn_s_memrealtime();
        }
    };

    int wo_b, wo_e, gu_b, gu_e, dn_b, dn_e;
    wg_share(G::DIM, wo_b, wo_e);
    wg_share(G::FFN, gu_b, gu_e); // (gate, up) pairs
    wg_share(G::DIM, dn_b, dn_e);
    // KV head group grp of this workgroup and its index gj in the group:
    // with the fused attention the group's workgroups sit on XCDs 2 grp and
    // 2 grp + 1 under round-robin dispatch; with split attention group g is
    // workgroups 64 g .. 64 g + 63, whose attention units are KV head g.
    const int grp = LONG ? int(blockIdx.x) / G::WGS_G : (blockIdx.x & 7) >> 1;
    const int gj = LONG ? int(blockIdx.x) % G::WGS_G
                        : ((blockIdx.x >> 3) << 1) | (blockIdx.x & 1);

    // Weight staging of each phase (region and slot layout). Weights are
    // addressed from the arena base alone, so staging issues no loads.
    auto wdata = [&](int layer, int m) {
        return a.weights + size_t(layer) * G::LAY.bytes + G::LAY.data[m];
    };
    auto wscales = [&](int layer, int m) {
        return reinterpret_cast<const uint16_t *>(
            a.weights + size_t(layer) * G::LAY.bytes + G::LAY.scales[m]);
    };
    auto stage = [&](uint8_t *region, int rows, int rb, int sb, int layer,
                     int m, int lo, int hi, int first) {
        if (hi <= lo)
            return;
        dma(region + first * rb, wdata(layer, m) + size_t(lo) * rb,
            (hi - lo) * rb);
        dma(region + rows * rb + first * sb,
            reinterpret_cast<const uint8_t *>(wscales(layer, m)) +
                size_t(lo) * sb,
            (hi - lo) * sb);
    };
    // The group's rows [lo, hi) are q rows of its heads, then its k and v
    // rows.
    auto stage_qkv_group = [&](int layer) {
        const int lo = gj * G::GR_WG, hi = lo + G::GR_WG;
        const int kb = G::GQ, vb = G::GQ + G::HD;
        stage(r1, G::ROWS_QKV, G::RB_DIM, G::SB_DIM, layer, 0, grp * G::GQ + lo,
              grp * G::GQ + min(hi, kb), 0);
        stage(r1, G::ROWS_QKV, G::RB_DIM, G::SB_DIM, layer, 1, grp * G::HD + max(lo, kb) - kb,
              grp * G::HD + min(hi, vb) - kb, max(lo, kb) - lo);
        stage(r1, G::ROWS_QKV, G::RB_DIM, G::SB_DIM, layer, 2, grp * G::HD + max(lo, vb) - vb,
              grp * G::HD + hi - vb, max(lo, vb) - lo);
    };
    auto stage_qkv = [&](int layer) { stage_qkv_group(layer); };
    auto stage_wo = [&](int layer) {
        if constexpr (LONG) {
            stage(r2, G::ROWS_WO, G::RB_DIM, G::SB_DIM, layer, 3, wo_b, wo_e, 0);
        } else {
            // the group's columns of rows [gj WO_WG, +WO_WG), then their scales
            const size_t row0 = size_t(gj) * G::WO_WG;
            dma_segments(r2, wdata(layer, 3) + row0 * G::RB_DIM + grp * G::WO_SEG, G::WO_WG,
                         G::WO_SEG, G::RB_DIM);
            dma_segments(r2 + G::WO_WG * G::WO_SEG,
                         reinterpret_cast<const uint8_t *>(wscales(layer, 3)) +
                             row0 * G::SB_DIM + grp * 2 * G::WO_BLK,
                         G::WO_WG, 2 * G::WO_BLK, G::SB_DIM);
        }
    };
    auto stage_gu = [&](int layer) {
        stage(r1, G::ROWS_GU, G::RB_DIM, G::SB_DIM, layer, 4, gu_b, gu_e, 0);
        stage(r1, G::ROWS_GU, G::RB_DIM, G::SB_DIM, layer, 5, gu_b, gu_e,
              G::ROWS_GU / 2);
    };
    auto stage_down = [&](int layer) {
        stage(r1, G::ROWS_DN, G::RB_FFN, G::SB_FFN, layer, 6, dn_b, dn_e, 0);
    };
    auto norm = [&](int layer, bool ffn) {
        return reinterpret_cast<const float *>(
            a.weights + size_t(layer) * G::LAY.bytes +
            (ffn ? G::LAY.ffn_norm : G::LAY.attention_norm));
    };
    auto slot = [&](int rows, int rb, int sb, int s, const uint8_t *&d,
                    const uint16_t *&sc, const uint8_t *region) {
        d = region + s * rb;
        sc = reinterpret_cast<const uint16_t *>(region + rows * rb + s * sb);
    };

    // Each layer's exchanges in write-once words of their own: q/k/v by
    // group (group g's GR rows at g GR), then with the fused attention the
    // Wo partial sums of group g at ON_WO + g DIM, with split attention the
    // merged context at ON_WO and h after Wo at ON_WO + DIM; act at ON_GU,
    // h after W2 at ON_DN. Split attention's partials stay tagged words.
    constexpr int ON_WO = G::DIM + 2 * G::KVD, ON_GU = ON_WO + G::KVH * G::DIM;
    constexpr int ON_DN = ON_GU + G::FFN;
    constexpr int ONCE = ON_DN + G::DIM;
    // the ring slice of the current (iteration, layer) step, advanced by one
    // per step (once_slice(it, layer, layer_count))
    int slice = 0;

    int count = 0, done = 0, last_token = 0;
    // Write-once words of the hidden state the next classifier reads; null
    // = hidden_in.
    const float *hidden_once = nullptr;
    // Each phase's weight rows (and attention's K/V rows) are issued just
    // before the wait for its input. Measured: issuing them a phase earlier
    // puts the bulk reads inside other workgroups' exchange waits or under
    // a compute phase, and both slow the token down.

    for (int it = 0; it < a.n_iter && !done; it++) {
        int token;
        mark(it, 0);
        if (CLASSIFY) {
            // ---------------- final rmsnorm + classifier + argmax ----
            const float *wcls = a.classifier;
            Slice<G::DIM> nw;
            nw.load(a.final_norm);
            float sq;
            if (hidden_once == nullptr) {
                Slice<G::DIM> h;
                h.load(a.hidden_in);
                sq = h.store(h_raw);
                __syncthreads();
            } else {
                sq = take_once<G::DIM, false, PollDelay<LONG>::CLASSIFIER>(hidden_once, h_raw,
                                                                          error);
            }
            const float scale = rms_scale(wg_sum(sq, red), G::DIM);
            // x in plain layout (lane needs x[4c..4c+3], c = lane + 64 j) in
            // region 1, free until layer 0's rows are staged; its digits
            // for the screened argmax in xl / xsc, its block sums of |x|
            // over the q/k/v staging, the row bounds over the scores
            float *xcls = reinterpret_cast<float *>(r1);
#pragma unroll
            for (int u = 0; u < Slice<G::DIM>::PER; u++) {
                const int i = threadIdx.x + u * kThreads;
                if (i < G::DIM)
                    xcls[i] = h_raw[i] * scale * nw.v[u];
            }
            __syncthreads();
            mark(it, 1);
            float best_v;
            int best_i;
            if (a.classifier8 != nullptr) {
                screen_x_digits<G::DIM>(xcls, xl, xsc, qkv);
                classifier_screened<G::DIM, false, 4, 3>(wcls, a.classifier8, a.classifier8_scales,
                                                         xcls, xl,
                                            xsc, qkv, a.vocab, scores, red, best_v, best_i);
            } else {
                classifier_best<G::DIM>(wcls, xcls, a.vocab, best_v, best_i);
            }
            __syncthreads();
            mark(it, 2);
            // The partial leaves before layer 0's QKV rows are issued (the
            // grid waits for the last workgroup's publish); the rows stream
            // into LDS during the argmax exchange.
            argmax_publish(a.x_part, best_v, best_i, red, misc, tag);
            stage_qkv(0);
            bool failed_wait = false;
            const int bi = argmax_take(a.x_part, red, misc, tag, error, failed_wait);
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
            stage_qkv(0);
        }
        last_token = token;
        const int pos = a.start_len + it;
        mark(it, 3);

        for (int l = 0; l < a.layer_count; l++) {
            float *kc = a.k_cache + l * kv_layer;
            float *vc = a.v_cache + l * kv_layer;
            // this step's write-once words, and the previous step's
            float *xo = a.x_once + size_t(slice) * ONCE;
            float *xp = a.x_once + size_t(slice == 0 ? kOnceRing - 1 : slice - 1) * ONCE;

            // ---------------------------------------------- phase A: qkv --
            // RoPE factors of this wave's first pair, read before the wait.
            // Pair `pair` of this workgroup: its first row's index in the
            // exchange, which matrix (q, k, v), its dim d and its KV head.
            const int npairs = G::GR_WG / 2;
            auto qkv_row = [&](int pair, int &xrow, int &which, int &d, int &kvh) {
                const int lr = gj * G::GR_WG + 2 * pair;
                which = lr < G::GQ ? 0 : lr < G::GQ + G::HD ? 1 : 2;
                d = lr % G::HD;
                kvh = grp;
                xrow = grp * G::GR + lr;
            };
            // (thread p < npairs publishes pair p)
            float2 rope_cs = make_float2(1.0f, 0.0f);
            if (threadIdx.x < npairs) {
                int xrow, which, d, kvh;
                qkv_row(threadIdx.x, xrow, which, d, kvh);
                if (which < 2)
                    rope_cs = a.rope[size_t(pos) * (G::HD / 2) + d / 2];
            }
            // this thread's quartet of the norm weights (stage_x)
            float4 nw4 = reinterpret_cast<const float4 *>(norm(l, false))[threadIdx.x];
            float sq;
            if (l == 0) {
                Slice<G::DIM> e;
                e.load(a.embeddings + size_t(token) * G::DIM);
                sq = e.store(h_raw);
                dma_wait();
            } else {
                sq = take_once<G::DIM, false, PollDelay<LONG>::A>(xp + ON_DN, h_raw,
                                                                   error);
            }
            stage_x<G::QT, G::DIM>(h_raw, nw4, rms_scale(wg_sum(sq, red), G::DIM), xl, xsc);
            mark(it, 4 + 13 * l);
            {
                // the workgroup's rows one at a time over the waves (10 rows:
                // at most three on a SIMD, where whole pairs put four on one),
                // each result into the scores region (free until attention)
                XDigits<G::CPL_DIM> x;
                load_x(x, xl, xsc, G::BLK_DIM);
                for (int r = wave; r < 2 * npairs; r += kWaves) {
                    const uint8_t *d;
                    const uint16_t *sc;
                    slot(G::ROWS_QKV, G::RB_DIM, G::SB_DIM, r, d, sc, r1);
                    const float y = row_dot<G::QT>(d, sc, x, G::BLK_DIM);
                    if (lane == 0)
                        scores[r] = y;
                }
            }
            __syncthreads();
            // pair p: RoPE (q and k rows), the exchange words, the cache row
            if (threadIdx.x < npairs) {
                const int pair = threadIdx.x;
                int row, which, d, head;
                qkv_row(pair, row, which, d, head);
                float e0 = scores[2 * pair], e1 = scores[2 * pair + 1];
                if (which < 2) {
                    const float even = e0, odd = e1;
                    e0 = fmaf(even, rope_cs.x, -(odd * rope_cs.y));
                    e1 = fmaf(even, rope_cs.y, odd * rope_cs.x);
                }
                put_once(xo + row, e0);
                put_once(xo + row + 1, e1);
                if (which > 0) {
                    float *cache = (which == 1 ? kc : vc) +
                                   (size_t(head) * a.max_seq + pos) * G::HD + d;
                    store_coherent(cache, e0);
                    store_coherent(cache + 1, e1);
                }
            }
            tag++;
            // K/V rows of earlier positions stream into LDS while the q/k/v
            // exchange completes (every wave is past its reads of region 1
            // and of the scores region's row results).
            __syncthreads();
            mark(it, 5 + 13 * l);
            const int n = pos + 1;
            // LONG: this workgroup's attention unit is KV head ag over
            // positions [ap0, ap1), K rows at kst and V rows at vst
            const int ag = blockIdx.x / G::SPLITS;
            const int per = cdiv(n, G::SPLITS);
            const int ap0 = min(n, int(blockIdx.x % G::SPLITS) * per);
            const int ap1 = min(n, ap0 + per);
            // fused: the group's KV head only, K rows [n][KROW] then V rows
            float *vst = LONG ? kst + G::PMAX * G::KROW : kst + n * G::KROW;
            // Rows before pos only: they were stored by earlier launches or
            // by other workgroups in earlier iterations of this one, hence
            // the agent-coherent loads; row pos comes from the exchange.
            if (LONG) {
                const int hist = max(0, min(ap1, pos) - ap0); // rows already cached
                if (hist > 0) {
                    const size_t row0 = size_t(ag) * a.max_seq + ap0;
                    dma_padded_rows<kStreamPolicy | kAgentCoherent>(kst, kc + row0 * G::HD, hist);
                    dma_padded_rows<kStreamPolicy | kAgentCoherent>(vst, vc + row0 * G::HD, hist);
                }
            } else if (pos > 0) {
                dma_padded_rows<kAgentCoherent>(kst, kc + size_t(grp) * a.max_seq * G::HD, pos);
                dma_padded_rows<kAgentCoherent>(vst, vc + size_t(grp) * a.max_seq * G::HD, pos);
            }
            stage_wo(l);
            mark(it, 6 + 13 * l);

            // ---------------------------- phase B: attention + Wo + residual --
            // (take also completes the phase-A K/V stores of this wave before
            // anything later is published)
            take_once<G::GR, false, PollDelay<LONG>::B>(xo + grp * G::GR, qkv, error);
            if (LONG) {
                // the new position's K/V row, when it falls in this unit
                if (pos >= ap0 && pos < ap1)
                    for (int i = threadIdx.x; i < 2 * G::HD; i += kThreads) {
                        const int which = i >= G::HD, d = i - which * G::HD;
                        (which ? vst : kst)[(pos - ap0) * G::KROW + d] =
                            qkv[G::GQ + which * G::HD + d];
                    }
            } else {
                // qkv holds the group's q rows, then its k and v rows
                for (int i = threadIdx.x; i < 2 * G::HD; i += kThreads) {
                    const int which = i >= G::HD, d = i - which * G::HD;
                    (which ? vst : kst)[pos * G::KROW + d] = qkv[G::GQ + i];
                }
            }

            __syncthreads();
            mark(it, 7 + 13 * l);
            if constexpr (LONG) {
                split_attention<G>(ap1 - ap0, ag, kst, vst, qkv, scores, xs, a, xo + ON_WO,
                                   tag, error);
                tag++;
                // the whole context, as digits for the Wo rows
                take_once<G::DIM, false, PollDelay<true>::CONTEXT>(xo + ON_WO, qkv, error);
                quartet_digits<G::QT>(reinterpret_cast<const float4 *>(qkv)[threadIdx.x],
                                      threadIdx.x >> 3, threadIdx.x & 7, xl, xsc);
            } else {
                // Wave w: query head w of the group. Lane p scores position
                // p, its K row from LDS and q's dims 4j..4j+3 from lane j of
                // its 16-lane row by DPP broadcast (every lane runs the dot,
                // lanes past n on the last row); then lane d sums context dim
                // d over the positions, their weights by readlane.
                const float4 qv = reinterpret_cast<const float4 *>(qkv + wave * G::HD)[lane & 15];
                const float4 *k4 =
                    reinterpret_cast<const float4 *>(kst + min(lane, n - 1) * G::KROW);
                float a0 = 0.0f, a1 = 0.0f;
                fma_row_bcast2<0>(a0, a1, qv, k4[0], k4[1]);
                fma_row_bcast2<2>(a0, a1, qv, k4[2], k4[3]);
                fma_row_bcast2<4>(a0, a1, qv, k4[4], k4[5]);
                fma_row_bcast2<6>(a0, a1, qv, k4[6], k4[7]);
                fma_row_bcast2<8>(a0, a1, qv, k4[8], k4[9]);
                fma_row_bcast2<10>(a0, a1, qv, k4[10], k4[11]);
                fma_row_bcast2<12>(a0, a1, qv, k4[12], k4[13]);
                fma_row_bcast2<14>(a0, a1, qv, k4[14], k4[15]);
                const float sc = lane < n ? (a0 + a1) * a.attn_scale : -INFINITY;
                const float m = wave_maximum(sc);
                const float e = lane < n ? expf(sc - m) : 0.0f;
                const float total = wave_total(e);
                const float *vcol = vst + lane;
                auto weight = [&](int q) {
                    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), q));
                };
                float c0 = 0.0f, c1 = 0.0f;
                int p = 0;
                for (; p + 8 <= n; p += 8) {
                    float v[8];
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        v[j] = vcol[(p + j) * G::KROW];
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        c0 = fmaf(weight(p + j), v[j], c0);
                        c1 = fmaf(weight(p + j + 1), v[j + 1], c1);
                    }
                }
                for (; p < n; p++)
                    c0 = fmaf(weight(p), vcol[p * G::KROW], c0);
                // the group's context (GQ values) over the scores region
                scores[wave * G::HD + lane] = (c0 + c1) * (1.0f / total);
                __syncthreads();
                // as digits, one quartet per thread of the first GQ / 4
                if (threadIdx.x < G::GQ / 4)
                    quartet_digits<G::QT>(reinterpret_cast<const float4 *>(scores)[threadIdx.x],
                                          threadIdx.x >> 3, threadIdx.x & 7, xl, xsc);
            }
            __syncthreads();
            mark(it, 8 + 13 * l);
            if constexpr (LONG) {
                for (int r = wave; r < wo_e - wo_b; r += kWaves) {
                    const uint8_t *d;
                    const uint16_t *s;
                    slot(G::ROWS_WO, G::RB_DIM, G::SB_DIM, r, d, s, r2);
                    const float y = row_dot_lds<G::QT, G::CPL_DIM>(d, s, xl, xsc, G::BLK_DIM);
                    if (lane == 0)
                        put_once(xo + ON_WO + G::DIM + wo_b + r, h_raw[wo_b + r] + y);
                }
            } else {
                // Wo partial sums over the group's context columns: wave w
                // takes rows 4 w .. 4 w + 3 of this workgroup's, a row of 16
                // lanes each, lane b one block; the residual is added by the
                // consumers
                const int r = 4 * wave + (lane >> 4), b = lane & 15;
                const uint8_t *d = r2 + r * G::WO_SEG;
                const uint16_t *s = reinterpret_cast<const uint16_t *>(
                    r2 + G::WO_WG * G::WO_SEG + r * 2 * G::WO_BLK);
                uint4 dg[6];
                load_digits(xl, b, dg);
                const float y = row16_sum(half_bits_to_float(s[b]) * xsc[b] *
                                          dot_block_digits<G::QT>(d, b, dg));
                if (b == 0)
                    put_once(xo + ON_WO + grp * G::DIM + gj * G::WO_WG + r, y);
            }
            tag++;
            // every wave is past attention (region 1) and past its reads of
            // h_raw, which phase C's take overwrites
            __syncthreads();
            mark(it, 9 + 13 * l);
            stage_gu(l);
            mark(it, 10 + 13 * l);

            // ------------------------------------------ phase C: gate/up --
            nw4 = reinterpret_cast<const float4 *>(norm(l, true))[threadIdx.x];
            // Every workgroup has taken the previous step's h after Wo, so
            // every word of the step before it has been read: this
            // workgroup's words of that step go back to kUnset for the
            // slice's next use (this take retires the stores).
            if (it * a.layer_count + l >= 2) {
                float *xr = a.x_once + size_t(slice >= 2 ? slice - 2 : slice + kOnceRing - 2) * ONCE;
                rearm_words(xr + grp * G::GR + gj * G::GR_WG, G::GR_WG, 0);
                if constexpr (LONG) {
                    // merged context values, then h after Wo
                    rearm_words(xr + ON_WO + (blockIdx.x >> 3) * G::HD + (blockIdx.x & 7) * 8, 8,
                                1);
                    rearm_words(xr + ON_WO + G::DIM + wo_b, wo_e - wo_b, 4);
                } else {
                    rearm_words(xr + ON_WO + grp * G::DIM + gj * G::WO_WG, G::WO_WG, 1);
                }
                rearm_words(xr + ON_GU + gu_b, gu_e - gu_b, 2);
                rearm_words(xr + ON_DN + dn_b, dn_e - dn_b, 3);
            }
            if constexpr (LONG)
                sq = take_once<G::DIM, false, PollDelay<LONG>::C>(xo + ON_WO + G::DIM,
                                                                  h_raw, error);
            else
                sq = take_once_sum<G::DIM, G::KVH, PollDelay<LONG>::C>(xo + ON_WO, h_raw,
                                                                      error);
            stage_x<G::QT, G::DIM>(h_raw, nw4, rms_scale(wg_sum(sq, red), G::DIM), xl, xsc);
            mark(it, 11 + 13 * l);
            {
                // the workgroup's gate rows, then its up rows, one at a time
                // over the waves: 2 np rows spread evenly over the CU's four
                // SIMDs (whole pairs were not: 6, 6, 5, 5 of 22), each result
                // into the scores region (free until the next attention);
                // silu(gate) * up after the barrier
                XDigits<G::CPL_DIM> x;
                load_x(x, xl, xsc, G::BLK_DIM);
                const int np = gu_e - gu_b;
                for (int r = wave; r < 2 * np; r += kWaves) {
                    const uint8_t *d;
                    const uint16_t *sc;
                    slot(G::ROWS_GU, G::RB_DIM, G::SB_DIM, r < np ? r : G::ROWS_GU / 2 + r - np,
                         d, sc, r1);
                    const float y = row_dot<G::QT>(d, sc, x, G::BLK_DIM);
                    if (lane == 0)
                        scores[r] = y;
                }
            }
            // every wave is past its reads of region 1 (the down rows go
            // there next) and its gate / up results are in LDS
            __syncthreads();
            if (threadIdx.x < gu_e - gu_b) {
                const float g = scores[threadIdx.x], u = scores[gu_e - gu_b + threadIdx.x];
                put_once(xo + ON_GU + gu_b + threadIdx.x, g / (1.0f + expf(-g)) * u);
            }
            tag++;
            mark(it, 12 + 13 * l);
            stage_down(l);
            mark(it, 13 + 13 * l);

            // --------------------------------------------- phase D: down --
            take_once<G::FFN, true, PollDelay<LONG>::D>(xo + ON_GU, xs, error);
            block_sums(xs, xsc, G::FFN);
            mark(it, 14 + 13 * l);
            {
                const bool last = l + 1 == a.layer_count;
                for (int r = wave; r < dn_e - dn_b; r += kWaves) {
                    const uint8_t *d;
                    const uint16_t *s;
                    slot(G::ROWS_DN, G::RB_FFN, G::SB_FFN, r, d, s, r1);
                    const float y = row_dot_floats<G::QT, G::CPL_FFN>(d, s, xs, xsc, G::BLK_FFN);
                    if (lane == 0) {
                        const float v = h_raw[dn_b + r] + y;
                        if (!(a.fault == 1 && blockIdx.x == 0 && it == 0 && l == 0))
                            put_once(xo + ON_DN + dn_b + r, v);
                        if (last && it + 1 == a.n_iter)
                            a.hidden_out[dn_b + r] = v;
                    }
                }
                __syncthreads();
                mark(it, 15 + 13 * l);
                if (!last)
                    stage_qkv(l + 1);
            }
            hidden_once = xo + ON_DN;
            slice = slice + 1 == kOnceRing ? 0 : slice + 1;
            tag++;
            mark(it, 16 + 13 * l);
        }
        // The generate loop learns of a failed wait in the next argmax
        // exchange (every wait gives up once the flag is set, so the grid
        // drains either way); the prefill loop checks here.
        if (!CLASSIFY && wg_failed(error, misc + 8))
            break;
    }
    // hidden_out after an early stop (eos): the state the loop ended with
    if (done && hidden_once != nullptr) {
        take_once<G::DIM, false>(hidden_once, h_raw, error);
        for (int i = threadIdx.x; i < G::DIM; i += kThreads)
            if (blockIdx.x == 0)
                a.hidden_out[i] = h_raw[i];
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.state->count = count;
        a.state->done = done;
        a.state->token = last_token;
    }
}

using TinyLlamaInt4 = Geo<1, 2048, 5632, 32, 4, 64, 48>;
using TinyLlamaInt8 = Geo<0, 2048, 5632, 32, 4, 64, 44>;

template <class G>
bool shape_is(const DecodeShape &s, int type)
{
    return type == G::QT && s.dim == G::DIM && s.ffn_dim == G::FFN &&
           s.heads == G::HEADS && s.kv_heads == G::KVH && s.head_dim == G::HD;
}

int device_cus()
{
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    int cus = 0;
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                                    device),
              "hipDeviceGetAttribute");
    return cus;
}

template <class G, bool CLASSIFY, bool LONG>
void launch_as(const TokenArgs &args, hipStream_t stream)
{
    const auto kernel = token_kernel<G, CLASSIFY, LONG>;
    hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  int(Lds<G>::BYTES)),
              "hipFuncSetAttribute");
    int per_cu = 0;
    hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                  &per_cu, reinterpret_cast<const void *>(kernel), kThreads,
                  Lds<G>::BYTES),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    require(per_cu >= 1 && device_cus() >= kGrid, NUT_EDEVICE,
            "token kernel: grid does not fit the device");
    require(args.start_len + args.n_iter <= (LONG ? G::SPLITS * G::PMAX : G::NP), NUT_EINVAL,
            "token kernel: context exceeds the attention pass");
    require(token_tags_needed(args.n_iter, args.layer_count) <= (1ll << kTagShift), NUT_EINVAL,
            "token kernel: launch exceeds its exchange tag range");
    require(!LONG || args.x_apart != nullptr, NUT_EINVAL,
            "token kernel: split attention needs its exchange buffers");
    require(args.x_once != nullptr, NUT_EINVAL,
            "token kernel: the launch needs its write-once exchange words");
    static_assert(Lds<G>::BYTES > 0 && G::DIM % 2 == 0 && G::KVD % 2 == 0 && G::FFN % 2 == 0,
                  "write-once words are polled in pairs");
    TokenArgs a = args;
    void *params[] = {&a};
    hip_check(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(kernel),
                                         dim3(kGrid), dim3(kThreads), params,
                                         Lds<G>::BYTES, stream),
              "token kernel launch");
}

template <class G>
void launch(const TokenArgs &args, hipStream_t stream)
{
    if (args.long_attention) {
        if (args.classify)
            launch_as<G, true, true>(args, stream);
        else
            launch_as<G, false, true>(args, stream);
    } else {
        if (args.classify)
            launch_as<G, true, false>(args, stream);
        else
            launch_as<G, false, false>(args, stream);
    }
}

} // namespace

bool token_kernel_supported(int type, const DecodeShape &s)
{
    if (!(shape_is<TinyLlamaInt4>(s, type) || shape_is<TinyLlamaInt8>(s, type) ||
          wide_kernel_positions(type, s) > 0))
        return false;
    return device_cus() >= kGrid;
}

int token_kernel_max_positions(int type, const DecodeShape &s)
{
    if (shape_is<TinyLlamaInt4>(s, type))
        return TinyLlamaInt4::NP;
    if (shape_is<TinyLlamaInt8>(s, type))
        return TinyLlamaInt8::NP;
    return wide_kernel_positions(type, s);
}

int token_kernel_long_positions(int type, const DecodeShape &s)
{
    if (shape_is<TinyLlamaInt4>(s, type))
        return TinyLlamaInt4::SPLITS * TinyLlamaInt4::PMAX;
    if (shape_is<TinyLlamaInt8>(s, type))
        return TinyLlamaInt8::SPLITS * TinyLlamaInt8::PMAX;
    return wide_kernel_positions(type, s);
}

size_t token_exchange_entries(const DecodeShape &s)
{
    const size_t kvd = size_t(s.kv_heads) * s.head_dim;
    const size_t group = s.heads / (s.kv_heads == 0 ? s.heads : s.kv_heads);
    // q/k/v, h, act, classifier partials; split attention partials, context;
    // the wide kernel's partial scores
    return (s.dim + 2 * kvd) + s.dim + s.ffn_dim + 2 * kGrid +
           size_t(kGrid) * group * (s.head_dim + 2) + s.dim + wide_kernel_score_entries(s);
}

void launch_token_kernel(int type, const DecodeShape &s, const TokenArgs &a,
                         hipStream_t stream)
{
    if (shape_is<TinyLlamaInt4>(s, type))
        launch<TinyLlamaInt4>(a, stream);
    else if (shape_is<TinyLlamaInt8>(s, type))
        launch<TinyLlamaInt8>(a, stream);
    else if (wide_kernel_positions(type, s) > 0)
        launch_wide_kernel(type, s, a, stream);
    else
        fail(NUT_EINVAL, "token kernel: unsupported shape");
}

} // namespace nut
