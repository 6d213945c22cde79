// sample.hip — device side of choose_token's temperature / top-p branch
// (src/generate.cpp:31-72). The device forms the softmax numerators from
// the classifier's logits, their block totals, and the (p, token) pairs in
// the reference's sort order (p descending, then token ascending); the host
// then walks the sorted prefix with the reference's sequential nucleus sum
// and draws with its own std::mt19937 (see model.cpp: generate_sampled).
#include "sample.hpp"
#include "runtime.hpp"

#include <rocprim/device/device_radix_sort.hpp>

namespace nut {

namespace {

constexpr int kThreads = 256;
constexpr int kBlocks = 128;

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

struct Layout {
    size_t keys, ids, keys_out, ids_out, totals, bad, temp, temp_bytes, total;
};

Layout layout_of(int vocab)
{
    Layout l{};
    const size_t n = size_t(vocab);
    size_t temp_bytes = 0;
    hip_check(rocprim::radix_sort_pairs_desc(nullptr, temp_bytes, static_cast<uint32_t *>(nullptr),
                                             static_cast<uint32_t *>(nullptr),
                                             static_cast<int *>(nullptr),
                                             static_cast<int *>(nullptr), unsigned(n), 0, 32),
              "rocprim radix sort size");
    size_t at = 0;
    l.keys = at;
    at = align256(at + n * 4);
    l.ids = at;
    at = align256(at + n * 4);
    l.keys_out = at;
    at = align256(at + n * 4);
    l.ids_out = at;
    at = align256(at + n * 4);
    l.totals = at;
    at = align256(at + kBlocks * sizeof(double));
    l.bad = at;
    at = align256(at + sizeof(int));
    l.temp = at;
    l.temp_bytes = temp_bytes;
    l.total = align256(at + temp_bytes);
    return l;
}

// The largest logit, from the classifier's per-block maxima.
__device__ float max_of_parts(const float *part_val, int parts, float *red)
{
    float m = -INFINITY;
    for (int i = threadIdx.x; i < parts; i += blockDim.x)
        m = fmaxf(m, part_val[i]);
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s)
            red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    return red[0];
}

// p_t = exp((logit_t - max) / temperature). The argument is formed in fp32
// as the reference forms it; the exponential is taken in double and rounded
// once to float, which is the correctly rounded float value except when the
// double result lies within one double ulp of a float rounding boundary.
__global__ __launch_bounds__(kThreads) void numerators_kernel(
    const float *logits, int vocab, const float *part_val, int parts, float temperature,
    uint32_t *keys, int *ids, double *totals, int *bad)
{
    __shared__ float red[kThreads];
    __shared__ double dred[kThreads];
    const float maximum = max_of_parts(part_val, parts, red);
    double local = 0.0;
    bool finite = true;
    for (int t = blockIdx.x * kThreads + threadIdx.x; t < vocab; t += kBlocks * kThreads) {
        const float arg = (logits[t] - maximum) / temperature;
        const float p = float(exp(double(arg)));
        finite = finite && isfinite(p);
        keys[t] = __float_as_uint(p);
        ids[t] = t;
        local += double(p);
    }
    if (!finite)
        __hip_atomic_store(bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    dred[threadIdx.x] = local;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s)
            dred[threadIdx.x] += dred[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        totals[blockIdx.x] = dred[0];
}

__global__ void clear_flag_kernel(int *flag) { *flag = 0; }

} // namespace

size_t sample_workspace_bytes(int vocab) { return layout_of(vocab).total; }

int sample_sort(const float *logits, int vocab, const float *part_val, int parts,
                float temperature, void *workspace, float **sorted_p, int **sorted_ids,
                float **token_p, double **totals, int **bad, hipStream_t stream)
{
    const Layout l = layout_of(vocab);
    char *base = static_cast<char *>(workspace);
    uint32_t *keys = reinterpret_cast<uint32_t *>(base + l.keys);
    uint32_t *keys_out = reinterpret_cast<uint32_t *>(base + l.keys_out);
    int *ids = reinterpret_cast<int *>(base + l.ids);
    int *ids_out = reinterpret_cast<int *>(base + l.ids_out);
    double *tot = reinterpret_cast<double *>(base + l.totals);
    int *flag = reinterpret_cast<int *>(base + l.bad);
    hipLaunchKernelGGL(clear_flag_kernel, dim3(1), dim3(1), 0, stream, flag);
    hipLaunchKernelGGL(numerators_kernel, dim3(kBlocks), dim3(kThreads), 0, stream, logits,
                       vocab, part_val, parts, temperature, keys, ids, tot, flag);
    check_launch("sampling: numerators");
    // p >= 0, so its float bits order as its values; the radix sort is
    // stable, so equal p keep ascending token order
    size_t temp_bytes = l.temp_bytes;
    hip_check(rocprim::radix_sort_pairs_desc(base + l.temp, temp_bytes, keys, keys_out, ids,
                                             ids_out, unsigned(vocab), 0, 32, stream),
              "sampling: radix sort");
    *sorted_p = reinterpret_cast<float *>(keys_out);
    *sorted_ids = ids_out;
    // the sort reads its input keys and leaves them as they were
    *token_p = reinterpret_cast<float *>(keys);
    *totals = tot;
    *bad = flag;
    return kBlocks;
}

} // namespace nut
