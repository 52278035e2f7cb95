// The power-of-two row scale of the f16 operand rows of the batched
// products: e = ceil(log2(max |v|)) - 14 puts a row's largest magnitude at or
// below 2^14, so no value overflows f16 or drops into its subnormals; a row
// with a zero, infinite or NaN maximum keeps scale 1. Both 2^e and 2^-e stay
// normal floats.
#pragma once

#include <hip/hip_runtime.h>

namespace hyq {

__device__ __forceinline__ int f16_row_exponent(float m)
{
    int e = 0;
    if (m > 0.f && m < INFINITY) {
        int ex;
        const float fr = frexpf(m, &ex); // m = fr * 2^ex, fr in [0.5, 1)
        e = (fr == 0.5f ? ex - 1 : ex) - 14;
        e = max(-110, min(114, e));
    }
    return e;
}

} // namespace hyq
