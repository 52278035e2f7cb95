// Cross-lane reductions of a 64-wide gfx950 wave with DPP row operations and
// readlane instead of LDS-routed shuffles (ds_bpermute): a DPP operand is a
// VALU source modifier, so each step costs one VALU instruction rather than
// an LDS round trip.
//
//   quad_perm [1,0,3,2] / [2,3,0,1]   lane i <-> i^1 / i^2 inside each quad
//   row_half_mirror                   lane i <-> 7-i inside each 8-lane half
//   row_mirror                        lane i <-> 15-i inside each 16-lane row
// After the four steps every lane of a 16-lane row holds that row's value;
// the four rows are combined from lanes 0, 16, 32, 48 by readlane, in that
// order, so the result is uniform and formed in a fixed order.
#pragma once

#include <hip/hip_runtime.h>

namespace hyq {
namespace wave {

constexpr int DPP_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;
constexpr int DPP_ROR4 = 0x124; // row_ror:4, lane i of a row reads lane (i - 4) mod 16
constexpr int DPP_ROR8 = 0x128; // row_ror:8

template <int CTRL> __device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL> __device__ __forceinline__ int dpp(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Sums / maxima over aligned groups of 4, 8 and 16 lanes (every lane of the
// group receives the result).
template <class T> __device__ __forceinline__ T sum4(T v)
{
    v += dpp<DPP_XOR1>(v);
    return v + dpp<DPP_XOR2>(v);
}
template <class T> __device__ __forceinline__ T sum8(T v)
{
    v = sum4(v);
    return v + dpp<DPP_HALF_MIRROR>(v);
}
template <class T> __device__ __forceinline__ T sum16(T v)
{
    v = sum8(v);
    return v + dpp<DPP_MIRROR>(v);
}
__device__ __forceinline__ float max16(float v)
{
    v = fmaxf(v, dpp<DPP_XOR1>(v));
    v = fmaxf(v, dpp<DPP_XOR2>(v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    return fmaxf(v, dpp<DPP_MIRROR>(v));
}

// NaN-propagating maxima (IEEE 754-2019 maximum, v_maximum3_f32): NaN when
// any operand is NaN, as NEON's FMAX / FMAXV are, which form the Q8
// quantizer's group maximum in the reference (src/quant.rs:869-892). fmaxf
// (IEEE maxNum) returns the other operand instead.
__device__ __forceinline__ float nmax(float a, float b)
{
    return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float nmax16(float v)
{
    v = nmax(v, dpp<DPP_XOR1>(v));
    v = nmax(v, dpp<DPP_XOR2>(v));
    v = nmax(v, dpp<DPP_HALF_MIRROR>(v));
    return nmax(v, dpp<DPP_MIRROR>(v));
}

template <class T> __device__ __forceinline__ T lane(T v, int l)
{
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Whole-wave sum and maximum (uniform result).
__device__ __forceinline__ float sum64(float v)
{
    v = sum16(v);
    return (lane(v, 0) + lane(v, 16)) + (lane(v, 32) + lane(v, 48));
}
__device__ __forceinline__ int sum64(int v)
{
    v = sum16(v);
    return (lane(v, 0) + lane(v, 16)) + (lane(v, 32) + lane(v, 48));
}
__device__ __forceinline__ float max64(float v)
{
    v = max16(v);
    return fmaxf(fmaxf(lane(v, 0), lane(v, 16)), fmaxf(lane(v, 32), lane(v, 48)));
}
__device__ __forceinline__ float nmax64(float v)
{
    v = nmax16(v);
    return nmax(nmax(lane(v, 0), lane(v, 16)), nmax(lane(v, 32), lane(v, 48)));
}

// v_permlane16_swap / v_permlane32_swap of v with itself. swap16: `even`
// holds each 32-lane half's even 16-lane row in both of its rows, `odd` its
// odd row; swap32: `lo` holds lanes 0..31 in both halves, `hi` lanes 32..63.
// The second operand is an opaque copy (empty asm) because the compiler
// folds a swap of a value with itself to that value.
__device__ __forceinline__ void swap16(int v, int &even, int &odd)
{
    int u = v;
    asm volatile("" : "+v"(u));
    const auto r = __builtin_amdgcn_permlane16_swap(v, u, false, false);
    even = r[0];
    odd = r[1];
}
__device__ __forceinline__ void swap32(int v, int &lo, int &hi)
{
    int u = v;
    asm volatile("" : "+v"(u));
    const auto r = __builtin_amdgcn_permlane32_swap(v, u, false, false);
    lo = r[0];
    hi = r[1];
}
// Sums / maxima over lanes i and i ^ 16 (sum_rows2), i and i ^ 32 (sum_halves)
__device__ __forceinline__ float sum_rows2(float v)
{
    int e, o;
    swap16(__builtin_bit_cast(int, v), e, o);
    return __builtin_bit_cast(float, e) + __builtin_bit_cast(float, o);
}
__device__ __forceinline__ int sum_rows2(int v)
{
    int e, o;
    swap16(v, e, o);
    return e + o;
}
__device__ __forceinline__ float max_rows2(float v)
{
    int e, o;
    swap16(__builtin_bit_cast(int, v), e, o);
    return fmaxf(__builtin_bit_cast(float, e), __builtin_bit_cast(float, o));
}
__device__ __forceinline__ float nmax_rows2(float v)
{
    int e, o;
    swap16(__builtin_bit_cast(int, v), e, o);
    return nmax(__builtin_bit_cast(float, e), __builtin_bit_cast(float, o));
}
__device__ __forceinline__ float sum_halves(float v)
{
    int l, h;
    swap32(__builtin_bit_cast(int, v), l, h);
    return __builtin_bit_cast(float, l) + __builtin_bit_cast(float, h);
}
__device__ __forceinline__ float max_halves(float v)
{
    int l, h;
    swap32(__builtin_bit_cast(int, v), l, h);
    return fmaxf(__builtin_bit_cast(float, l), __builtin_bit_cast(float, h));
}

} // namespace wave
} // namespace hyq
