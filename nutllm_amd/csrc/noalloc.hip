// noalloc.hip — the device memory of nut_decode_noalloc. The workspace
// that nut_decode allocates (split-attention partials and arrival counters
// of the step kernels) is a file-scope device array here, so the entry
// point calls no allocator: for callers that cannot allocate (code under
// graph capture, serving loops, harnesses that forbid it). Each device
// holds its own copy of the array until the process ends; host code never
// passes the array's name to a kernel, only the address hipGetSymbolAddress
// returned for the current device.
#include "noalloc.hpp"
#include "runtime.hpp"
#include "status.hpp"

#include <mutex>

namespace nut {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices] = {};

__global__ void fill_words_kernel(uint32_t *p, uint32_t value, size_t words)
{
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
         i += size_t(gridDim.x) * blockDim.x)
        p[i] = value;
}

} // namespace

void *noalloc_scratch()
{
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    require(device >= 0 && device < kMaxDevices, NUT_EDEVICE,
            "no-alloc decode: device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_lock);
    if (g_scratch_ptr[device] == nullptr) {
        void *ptr = nullptr;
        hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress");
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}

void launch_fill_words(uint32_t *p, uint32_t value, size_t words, hipStream_t stream)
{
    if (words == 0)
        return;
    const size_t blocks = std::min<size_t>((words + 255) / 256, 1024);
    hipLaunchKernelGGL(fill_words_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, p,
                       value, words);
    check_launch("no-alloc decode: scratch fill");
}

} // namespace nut
