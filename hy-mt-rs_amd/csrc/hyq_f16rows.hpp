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

// The token row of workgroup b when the rows are written in an MFMA
// fragment order whose 128-byte lines hold 16 bytes of each of 8
// consecutive rows (r / 8 equal), and workgroup b runs on XCD b % 8: with row
// 8 (8 (j / 8) + b % 8) + j % 8, j = b / 8, the 8 rows of a line run on one
// XCD, whose L2 merges their pieces into whole lines, instead of on eight.
// A bijection of [0, 64 n) onto itself.
__device__ __forceinline__ int frag_row(int b)
{
    const int j = b >> 3;
    return 8 * (8 * (j >> 3) + (b & 7)) + (j & 7);
}

} // namespace hyq
