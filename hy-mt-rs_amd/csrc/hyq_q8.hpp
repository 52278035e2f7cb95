// Q8 activation quantizer as a device function (Q8::quantize_into,
// src/quant.rs:904-922, with max_abs_neon :869-892 and quantize_group_neon
// :965-991): one 256-value group per 256-thread workgroup, one value per
// thread.
//
// max = max|x| over the group's whole 16-value steps by FMAX (a NaN there
// makes it NaN), then folded with the tail's |x| by f32::max (a NaN operand
// yields the other one); scale = max/127 and inverse = 127/max (IEEE
// divisions), or 0/0 unless max > 0 (an all-zero group, or a NaN maximum:
// every code of such a group is 0); q = saturate_i8(round_half_even(x *
// inverse)) over whole 16-value steps and clamp(round_half_away(x *
// inverse), -127, 127) over a group's tail, as the NEON body and its scalar
// tail do. It also writes the integer sums of q over 16-, 32- and 256-value
// spans that the GEMV kernels use to fold code offsets (exact integers, so
// their order is free).
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

namespace hyq {

__device__ __forceinline__ int q8_sat_rne(float v)
{
    if (v != v) return 0;
    float r = __builtin_rintf(v);
    r = fminf(fmaxf(r, -128.f), 127.f);
    return (int)r;
}

__device__ __forceinline__ int q8_tail_round(float v)
{
    if (v != v) return 0;
    float r = roundf(v);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return (int)r;
}

// All 256 threads of the workgroup must call it. v: this thread's value (0
// beyond len); g: group index; base = 256*g; len: values in this group.
__device__ __forceinline__ void q8_quantize_group(float v, int g, int len, int8_t *__restrict__ q,
                                                  float *__restrict__ s,
                                                  int32_t *__restrict__ sum16,
                                                  int32_t *__restrict__ sum32,
                                                  int32_t *__restrict__ sum256)
{
    __shared__ float wmax[4], wtail[4];
    __shared__ int wsum[4];
    const int t = threadIdx.x;
    const int base = g * 256;
    const int vec = len / 16 * 16;
    // the body's maximum propagates NaN, the tail's ignores it
    const float mb = wave::nmax64(t < vec ? fabsf(v) : 0.f);
    const float mt = wave::max64(t >= vec && t < len ? fabsf(v) : 0.f);
    if ((t & 63) == 0) {
        wmax[t >> 6] = mb;
        wtail[t >> 6] = mt;
    }
    __syncthreads();
    const float m = fmaxf(wave::nmax(wave::nmax(wmax[0], wmax[1]), wave::nmax(wmax[2], wmax[3])),
                          fmaxf(fmaxf(wtail[0], wtail[1]), fmaxf(wtail[2], wtail[3])));

    float scale = 0.f, inverse = 0.f;
    if (m > 0.f) {
        scale = m / 127.f;
        inverse = 127.f / m;
    }
    int qi = 0;
    if (t < vec) qi = q8_sat_rne(v * inverse);
    else if (t < len) qi = q8_tail_round(v * inverse);
    if (t < len) q[base + t] = (int8_t)qi;
    if (t == 0) s[g] = scale;

    // one value per lane: 16-value sums over rows, 32-value over row pairs
    const int a16 = wave::sum16(qi);
    if ((t & 15) == 0 && t < len) sum16[(base + t) >> 4] = a16;
    const int h0 = wave::lane(a16, 0) + wave::lane(a16, 16);
    const int h1 = wave::lane(a16, 32) + wave::lane(a16, 48);
    if ((t & 31) == 0 && t < len) sum32[(base + t) >> 5] = (t & 32) ? h1 : h0;
    const int a = h0 + h1;
    if ((t & 63) == 0) wsum[t >> 6] = a;
    __syncthreads();
    if (t == 0) sum256[g] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

} // namespace hyq
