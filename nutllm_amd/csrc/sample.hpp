// sample.hpp — device side of temperature / top-p sampling.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nut {

// Workspace of sample_sort for a vocabulary of `vocab` tokens: keys and
// ids in and out, block totals, a flag, and rocPRIM's temporary storage.
size_t sample_workspace_bytes(int vocab);

// Softmax numerators of choose_token (src/generate.cpp:45-54) over logits
// [vocab]: p_t = exp((logit_t - max) / temperature), max the largest logit
// (from the classifier's per-block maxima part_val[0, parts)). Writes the
// (p, t) pairs sorted by p descending, ties by ascending t (the order of
// the reference's std::sort comparator, lines 56-61) to sorted_p /
// sorted_ids, p in token order to token_p, one double partial sum of p per
// block to totals (block order), and 1 to *bad when a p is not finite.
// Returns the number of totals. workspace holds sample_workspace_bytes(vocab).
int sample_sort(const float *logits, int vocab, const float *part_val, int parts,
                float temperature, void *workspace, float **sorted_p, int **sorted_ids,
                float **token_p, double **totals, int **bad, hipStream_t stream);

} // namespace nut
