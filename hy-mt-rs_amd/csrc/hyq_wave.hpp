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

} // namespace wave
} // namespace hyq
