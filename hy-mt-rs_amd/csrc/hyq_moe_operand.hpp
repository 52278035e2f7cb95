// Row operands of the Q4_K register-operand expert kernels (hyq_moe_q4k.hip):
// one f16 row of activations (a token row of x for gate/up, a pair's SiLU
// row for down) laid out in the MFMA lane order those kernels copy into LDS,
// so that a 16-token chunk's operand is gathered column by column from the
// rows of its tokens.
//
// Row layout for a row of K = 256 nbk values x, scaled by 2^-e with
// e = f16_row_exponent(max |x|) (a zero, infinite or NaN maximum keeps
// e = 0):
//   op[b][t][g] (16 bytes, superblock b, MFMA step t = 0..7, lane group
//     g = 0..3): the halves x(a), x(a+2), x(a+1), x(a+3), x(a+32), x(a+34),
//     x(a+33), x(a+35) with a = 256 b + 64 ((t < 4 ? 0 : 2) + g / 2)
//     + 16 (g & 1) + 4 (t & 3);
//   hs[b][g] (8 bytes): f16(X / 16) of the four 16-value sums the lane group
//     covers, X_p = sum over t of the step's (x(a) + x(a+1)) + (x(a+2) +
//     x(a+3)) (p = 0, 2) or of the same four at a + 32 (p = 1, 3), for t =
//     0..3 (p = 0, 1) and t = 4..7 (p = 2, 3), each added in t order;
//   sc = 2^e.
// Chunk column col of a superblock's step t is then op[b][t][g] of that
// column's row in lane 16 g + col (the kernels' LDS order).
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_f16rows.hpp"
#include "hyq_wave.hpp"

namespace hyq {

constexpr int MOE_OP_U4_PER_SB = 32; // op uint4 per superblock of a row
constexpr int MOE_OP_U2_PER_SB = 4;  // hs uint2 per superblock of a row

// Largest |x| of a row of n floats read by one wave (x 16-byte aligned,
// n a multiple of 4): infinity when the row holds a NaN.
__device__ __forceinline__ float wave_row_absmax(const float *x, int n)
{
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const int lane = threadIdx.x & 63, n4 = n / 4;
    float m = 0.f;
    // eight float4 loads in flight per pass (clamped in bounds, past the end
    // masked to zero), so that the row costs one memory round trip per 2048
    // values rather than one per float4
    for (int i0 = 0; i0 < n4; i0 += 512) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x4[min(i0 + lane + 64 * j, n4 - 1)];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (i0 + lane + 64 * j >= n4) v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)),
                               fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
            if (v[j].x != v[j].x || v[j].y != v[j].y || v[j].z != v[j].z || v[j].w != v[j].w)
                m = INFINITY;
        }
    }
    return wave::max64(m);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi)
{
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Item (b, g, half) of a row (`half` = which four steps): the four op
// entries of steps 4 half .. 4 half + 3 and half of hs[b][g], from values
// v(i) = the row's value i (any callable) times inv.
template <class V>
__device__ __forceinline__ void row_operand_item(const V &v, float inv, int b, int g, int half,
                                                 uint4 *op, uint32_t *hs)
{
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int tq = 0; tq < 4; ++tq) {
        const int tt = 4 * half + tq;
        const int a = 256 * b + 64 * (2 * half + (g >> 1)) + 16 * (g & 1) + 4 * tq;
        const float l0 = v(a) * inv, l1 = v(a + 1) * inv, l2 = v(a + 2) * inv, l3 = v(a + 3) * inv;
        const float h0 = v(a + 32) * inv, h1 = v(a + 33) * inv, h2 = v(a + 34) * inv,
                    h3 = v(a + 35) * inv;
        op[MOE_OP_U4_PER_SB * b + 4 * tt + g] =
            make_uint4(pack_f16x2(l0, l2), pack_f16x2(l1, l3), pack_f16x2(h0, h2), pack_f16x2(h1, h3));
        s0 += (l0 + l1) + (l2 + l3);
        s1 += (h0 + h1) + (h2 + h3);
    }
    // hs[b][g] as two dwords: (X_0, X_1) from half 0, (X_2, X_3) from half 1
    hs[2 * (MOE_OP_U2_PER_SB * b + g) + half] = pack_f16x2(s0 * 0.0625f, s1 * 0.0625f);
}

// One wave forms the operand of row x [K] (K a multiple of 256, x 16-byte
// aligned): its scale sc, op and hs (2 K and K / 8 bytes).
__device__ __forceinline__ void wave_row_operand(const float *x, int K, uint4 *op, uint2 *hs,
                                                 float *sc)
{
    const int lane = threadIdx.x & 63;
    const int e = f16_row_exponent(wave_row_absmax(x, K));
    const float inv = ldexpf(1.0f, -e);
    if (lane == 0) *sc = ldexpf(1.0f, e);
    auto val = [&](int i) { return x[i]; };
    uint32_t *hs32 = reinterpret_cast<uint32_t *>(hs);
    for (int it = lane; it < 8 * (K / 256); it += 64)
        row_operand_item(val, inv, it >> 3, (it >> 1) & 3, it & 1, op, hs32);
}

} // namespace hyq
