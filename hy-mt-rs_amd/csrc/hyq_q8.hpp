// Q8 activation quantizer as a device function (Q8::quantize_into,
// src/quant.rs:904-922, with max_abs_neon :869-892 and quantize_group_neon
// :965-991): one 256-value group per 256-thread workgroup, one value per
// thread.
//
// scale = max/127 and inverse = 127/max (IEEE divisions, or 0/0 for an
// all-zero group); q = saturate_i8(round_half_even(x * inverse)) over whole
// 16-value steps and clamp(round_half_away(x * inverse), -127, 127) over a
// group's tail, as the NEON body and its scalar tail do. It also writes the
// integer sums of q over 16-, 32- and 256-value spans that the GEMV kernels
// use to fold code offsets (exact integers, so their order is free).
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
    __shared__ float wmax[4];
    __shared__ int wsum[4];
    const int t = threadIdx.x;
    const int base = g * 256;
    float m = wave::max64(fabsf(v));
    if ((t & 63) == 0) wmax[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));

    float scale = 0.f, inverse = 0.f;
    if (m > 0.f) {
        scale = m / 127.f;
        inverse = 127.f / m;
    }
    const int vec = len / 16 * 16;
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
