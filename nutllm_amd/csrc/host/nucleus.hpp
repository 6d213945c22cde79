// nucleus.hpp — the nucleus cut of choose_token's top-p branch
// (src/generate.cpp:63-68), host code shared by the sampled generate loop
// (model.cpp) and the host tests.
#pragma once

#include <stddef.h>

namespace nut {

// How many of the sorted p (descending) the reference's loop takes for
// top_p and the total mass, and whether that count could differ for any
// total within `slack` of `total` (the reference sums the total
// sequentially in token order, the device by blocks; the two differ by at
// most slack). `next(i)` yields the i-th sorted p, i = 0, 1, ... in turn;
// `nucleus` gets the sum of the p taken, in the loop's order.
template <class Next>
size_t nucleus_count(Next next, size_t vocab, float top_p, double total, double slack,
                     double &nucleus, bool &ambiguous)
{
    const double cutoff = top_p * total;
    const double margin = double(top_p) * slack;
    nucleus = 0.0;
    size_t taken = 0;
    double before = 0.0;
    do {
        before = nucleus;
        nucleus += next(taken);
        taken++;
    } while (taken < vocab && nucleus < cutoff);
    // a cutoff lower by up to margin could stop one step earlier, a higher
    // one could go on
    ambiguous = (taken > 1 && before >= cutoff - margin) ||
                (taken < vocab && nucleus < cutoff + margin);
    return taken;
}

} // namespace nut
