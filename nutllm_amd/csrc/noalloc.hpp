// noalloc.hpp — workspace of the allocation-free decode entry point.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nut {

// Size of the per-device scratch array behind nut_decode_noalloc: the step
// kernels' split-attention partials and arrival counters of one token.
constexpr size_t kNoAllocScratchBytes = size_t(2) << 20;

// This device's address of the scratch array, looked up once per device
// (hipGetSymbolAddress with the device current) and kept; allocates
// nothing.
void *noalloc_scratch();

// p[0, words) = value, as a kernel on the stream (no memset node).
void launch_fill_words(uint32_t *p, uint32_t value, size_t words,
                       hipStream_t stream);

} // namespace nut
