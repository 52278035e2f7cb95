// Batch-1 int8 GEMV (Weight::gemv_q8_fast and friends, src/quant.rs:346-651)
// for gfx950.
//
// Work split: 8 lanes ("sub-lanes") share a row and split its 256-weight
// groups (group g goes to sub-lane g % 8); a wave holds 8 such row-sets and
// each row-set owns NR consecutive rows. The Q8 activations of the whole row
// are staged once per workgroup into LDS (one 272-byte slot per group, 16
// bytes of padding so that the 8 sub-lanes of a row-set read 8 different
// bank windows while the 8 row-sets broadcast), then each lane copies its
// group's 64 dwords into registers and reuses them for its NR rows. The
// partial sums of a row are combined over the 8 sub-lanes with xor shuffles.
//
// HBM traffic per launch is the weight planes once (equal to the GGUF byte
// count), the Q8 vector once per workgroup from L2 and one f32 per row.
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_groups.hpp"
#include "hyq_q8.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

constexpr int SLOT_INTS = 68; // 256 bytes of a group + 16 bytes of padding

__device__ __forceinline__ float silu_mul(float g, float u)
{
    // silu(g) * u with silu(g) = g / (1 + exp(-g)) (src/quant.rs:573-574)
    float silu = g / (1.0f + expf(-g));
    return silu * u;
}

__device__ __forceinline__ float reduce8(float v) { return wave::sum8(v); }

// The f32 input stage: the workgroup's waves take 256-value groups in turn
// (group g = wave + 4i; lane l holds values 4l..4l+3) and write the Q8 row to
// the LDS slots, the group scales and the 16/32/256-value integer sums to
// the LDS arrays, as Q8::quantize_into (src/quant.rs:904-922) and
// q8_quantize_group do. With a norm vector the values are rms_norm_into's
// x * (1/sqrt(mean(x^2) + eps)) * w (src/model.rs:825-829); the sum of
// squares is formed per group by a fixed DPP/readlane tree (hyq_wave.hpp)
// and then over the groups in ascending order. Rows of up to 4 * STAGE_REG groups are loaded with all
// loads in flight at once; longer rows take a loop.
constexpr int STAGE_REG = 8;

__device__ __forceinline__ float4 scale_by(float4 v, float scale, float4 w)
{
    return make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z,
                       v.w * scale * w.w);
}

__device__ __forceinline__ void quantize_group4(float4 v, int g, int lane, int *slots, float *sc,
                                                int *s256, int *s16, int *s32)
{
    const float m = wave::max64(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    float s = 0.f, inv = 0.f;
    if (m > 0.f) {
        s = m / 127.f;
        inv = 127.f / m;
    }
    const int q0 = q8_sat_rne(v.x * inv), q1 = q8_sat_rne(v.y * inv);
    const int q2 = q8_sat_rne(v.z * inv), q3 = q8_sat_rne(v.w * inv);
    slots[g * SLOT_INTS + lane] =
        (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((q3 & 0xff) << 24);
    // integer sums over 16, 32 and 256 values (4, 8 and 64 lanes): exact
    const int t4 = wave::sum4((q0 + q1) + (q2 + q3));
    if ((lane & 3) == 0) s16[g * 16 + (lane >> 2)] = t4;
    const int t8 = t4 + wave::dpp<wave::DPP_HALF_MIRROR>(t4);
    if ((lane & 7) == 0) s32[g * 8 + (lane >> 3)] = t8;
    const int t16 = t8 + wave::dpp<wave::DPP_MIRROR>(t8);
    const int t256 = (wave::lane(t16, 0) + wave::lane(t16, 16)) +
                     (wave::lane(t16, 32) + wave::lane(t16, 48));
    if (lane == 0) {
        s256[g] = t256;
        sc[g] = s;
    }
}

__device__ __forceinline__ float group_ss(float4 v)
{
    return wave::sum64((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
}

// Register path (rows of at most 4 * STAGE_REG groups): the loads are
// issued by stage_load before the weights' (loads complete in issue order,
// so the stage then waits for its own data only) and consumed by stage_regs.
template <int IN>
__device__ __forceinline__ void stage_load(const GemvArgs &a, float4 (&v)[STAGE_REG],
                                           float4 (&w)[STAGE_REG])
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.xin);
    const float4 *n4 = reinterpret_cast<const float4 *>(a.norm);
#pragma unroll
    for (int i = 0; i < STAGE_REG; ++i)
        if (wave + 4 * i < a.groups) {
            v[i] = x4[(wave + 4 * i) * 64 + lane];
            if (IN == 2) w[i] = n4[(wave + 4 * i) * 64 + lane];
        }
}

__device__ __forceinline__ float finish_norm(const float *gss, int groups, float eps)
{
    __syncthreads();
    float ss = 0.f;
    for (int g = 0; g < groups; ++g) ss += gss[g];
    return 1.0f / sqrtf(ss / (float)(groups * 256) + eps);
}

template <int IN>
__device__ __forceinline__ void stage_regs(const GemvArgs &a, const float4 (&v)[STAGE_REG],
                                           const float4 (&w)[STAGE_REG], int *slots, float *sc,
                                           int *s256, int *s16, int *s32, float *gss)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int groups = a.groups;
    float scale = 1.f;
    if (IN == 2) {
#pragma unroll
        for (int i = 0; i < STAGE_REG; ++i)
            if (wave + 4 * i < groups) {
                const float s = group_ss(v[i]);
                if (lane == 0) gss[wave + 4 * i] = s;
            }
        scale = finish_norm(gss, groups, a.eps);
    }
#pragma unroll
    for (int i = 0; i < STAGE_REG; ++i)
        if (wave + 4 * i < groups)
            quantize_group4(IN == 2 ? scale_by(v[i], scale, w[i]) : v[i], wave + 4 * i, lane,
                            slots, sc, s256, s16, s32);
}

// Longer rows: a loop over the groups (loads at the top of each iteration).
template <int IN>
__device__ __forceinline__ void stage_loop(const GemvArgs &a, int *slots, float *sc, int *s256,
                                           int *s16, int *s32, float *gss)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int groups = a.groups;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.xin);
    const float4 *n4 = reinterpret_cast<const float4 *>(a.norm);
    float scale = 1.f;
    if (IN == 2) {
        for (int g = wave; g < groups; g += 4) {
            const float s = group_ss(x4[g * 64 + lane]);
            if (lane == 0) gss[g] = s;
        }
        scale = finish_norm(gss, groups, a.eps);
    }
    for (int g = wave; g < groups; g += 4) {
        const float4 v = x4[g * 64 + lane];
        quantize_group4(IN == 2 ? scale_by(v, scale, n4[g * 64 + lane]) : v, g, lane, slots, sc,
                        s256, s16, s32);
    }
}

// Q8 input rows (no input stage) of up to Q8_REG int4 per thread are read
// into registers before the weights' loads are issued, then copied to LDS.
constexpr int Q8_REG = 8;
// (a clang vector type: an array of HIP's int4 struct is not promoted to
// registers here)
typedef int i32x4 __attribute__((ext_vector_type(4)));

template <int F, int NR, int MODE, int IN, int P>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a)
{
    using G = typename GroupOf<F>::T;
    extern __shared__ int lds[];

    const int groups = a.groups;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane & 7;
    const int rset = lane >> 3;
    const int nwaves = blockDim.x >> 6;
    const int row0 = ((blockIdx.x * nwaves + wave) * 8 + rset) * NR;

    // Resolve each row of this lane to (segment, local row).
    int seg[NR], lrow[NR];
    bool valid[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int r = row0 + i;
        valid[i] = r < a.rows_total;
        int s = 0;
        if (MODE == GEMV_MULTI) {
            if (a.nseg > 1 && r >= a.seg[1].row_start) s = 1;
            if (a.nseg > 2 && r >= a.seg[2].row_start) s = 2;
        }
        seg[i] = s;
        lrow[i] = r - a.seg[s].row_start;
    }
    // rows past the end load row 0 of their segment (in bounds, unused), so
    // that every weight load is issued unconditionally
    int lrowc[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) lrowc[i] = valid[i] ? lrow[i] : 0;

    typename G::Data d[NR];
    typename G::Data d2[MODE == GEMV_SILU ? NR : 1];
    auto load_group = [&](int g) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const WView &w = MODE == GEMV_MULTI ? a.seg[seg[i]].w : a.seg[0].w;
            G::load(d[i], w, lrowc[i], g);
            if (MODE == GEMV_SILU) G::load(d2[i], a.seg[1].w, lrowc[i], g);
        }
    };
    // The activation row's loads are issued first, then the weights' (which
    // do not depend on the activations), so both latencies overlap and the
    // input stage waits for its own loads only. The weight loads are issued
    // unconditionally (group and row indices clamped into bounds), so the
    // compiler can count them and wait for the activations alone: a plain
    // GEMV with one row per lane and P = ceil(groups / 8) <= 4 issues all P
    // of its groups at once; otherwise the first group is preloaded and the
    // others load at the top of their iteration.
    float4 sv[STAGE_REG], sw[STAGE_REG];
    i32x4 qv[Q8_REG];
    const bool stage_reg = IN != 0 && groups <= 4 * STAGE_REG;
    const bool q8_reg = IN == 0 && groups * 16 <= Q8_REG * (int)blockDim.x;
    if (IN != 0 && stage_reg) stage_load<IN>(a, sv, sw);
    if (IN == 0 && q8_reg) {
        // clamped into bounds; the copy to LDS keeps the in-range ones
        const i32x4 *src = reinterpret_cast<const i32x4 *>(a.x.q);
#pragma unroll
        for (int j = 0; j < Q8_REG; ++j)
            qv[j] = src[min((int)threadIdx.x + j * (int)blockDim.x, groups * 16 - 1)];
    }
    static_assert(P == 0 || (NR == 1 && MODE == GEMV_PLAIN), "preload: plain, one row per lane");
    typename G::Data dp[P > 0 ? P : 1];
    if (P > 0) {
#pragma unroll
        for (int u = 0; u < P; ++u) G::load(dp[u], a.seg[0].w, lrowc[0], min(sub + 8 * u, groups - 1));
    } else {
        load_group(min(sub, groups - 1));
    }
    Q8View xq = a.x;
    if (IN == 0) {
        const int4 *src = reinterpret_cast<const int4 *>(a.x.q);
        int4 *dst = reinterpret_cast<int4 *>(lds);
        if (q8_reg) {
#pragma unroll
            for (int j = 0; j < Q8_REG; ++j) {
                const int i = threadIdx.x + j * (int)blockDim.x;
                if (i < groups * 16)
                    reinterpret_cast<i32x4 *>(dst)[(i >> 4) * (SLOT_INTS / 4) + (i & 15)] = qv[j];
            }
        } else {
            for (int i = threadIdx.x; i < groups * 16; i += blockDim.x)
                dst[(i >> 4) * (SLOT_INTS / 4) + (i & 15)] = src[i];
        }
    } else {
        float *sc = reinterpret_cast<float *>(lds + groups * SLOT_INTS);
        int *s256 = reinterpret_cast<int *>(sc + groups);
        int *s16 = s256 + groups;
        int *s32 = s16 + groups * 16;
        float *gss = reinterpret_cast<float *>(s32 + groups * 8);
        if (stage_reg) stage_regs<IN>(a, sv, sw, lds, sc, s256, s16, s32, gss);
        else stage_loop<IN>(a, lds, sc, s256, s16, s32, gss);
        xq.s = sc;
        xq.sum256 = s256;
        xq.sum16 = s16;
        xq.sum32 = s32;
    }
    __syncthreads();

    float acc[NR];
    float acc2[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = acc2[i] = 0.f;

    auto stage_act = [&](int g, int (&act)[64]) {
        const int4 *s4 = reinterpret_cast<const int4 *>(lds + g * SLOT_INTS);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int4 v = s4[j];
            act[4 * j] = v.x;
            act[4 * j + 1] = v.y;
            act[4 * j + 2] = v.z;
            act[4 * j + 3] = v.w;
        }
    };
    if (P > 0) {
#pragma unroll
        for (int u = 0; u < P; ++u) {
            const int g = sub + 8 * u;
            if (g >= groups || !valid[0]) continue;
            int act[64];
            stage_act(g, act);
            acc[0] += G::template dot<false>(dp[u], act, xq, g, nullptr);
        }
    } else {
        for (int g = sub; g < groups; g += 8) {
            int act[64];
            stage_act(g, act);
            if (g != sub) load_group(g);
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                if (!valid[i]) continue;
                if (MODE == GEMV_ISUMS) {
                    int32_t *out = a.isums + ((size_t)lrow[i] * groups + g) * G::ISUMS;
                    acc[i] += G::template dot<true>(d[i], act, xq, g, out);
                } else {
                    acc[i] += G::template dot<false>(d[i], act, xq, g, nullptr);
                    if (MODE == GEMV_SILU)
                        acc2[i] += G::template dot<false>(d2[i], act, xq, g, nullptr);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const float v = reduce8(acc[i]);
        const float v2 = MODE == GEMV_SILU ? reduce8(acc2[i]) : 0.f;
        if (sub != 0 || !valid[i] || MODE == GEMV_ISUMS) continue;
        if (MODE == GEMV_SILU) {
            a.seg[0].y[lrow[i]] = silu_mul(v, v2);
        } else if (MODE == GEMV_MULTI) {
            a.seg[seg[i]].y[lrow[i]] = v;
        } else {
            a.seg[0].y[lrow[i]] = a.residual ? a.residual[lrow[i]] + v : v;
        }
    }
}

template <int F, int MODE, int IN>
int launch_nr(int nr, int pre, const GemvArgs &a, dim3 grid, dim3 block, size_t lds,
              hipStream_t st)
{
    if constexpr (MODE == GEMV_PLAIN) {
        if (nr == 1) switch (pre) {
        case 1: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 1>), grid, block, lds, st, a); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 2>), grid, block, lds, st, a); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 3>), grid, block, lds, st, a); break;
        case 4: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 4>), grid, block, lds, st, a); break;
        default: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0>), grid, block, lds, st, a); break;
        }
        if (nr == 1) return (int)hipGetLastError();
    }
    switch (nr) {
    case 1: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0>), grid, block, lds, st, a); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<F, 2, MODE, IN, 0>), grid, block, lds, st, a); break;
    default: hipLaunchKernelGGL((gemv_kernel<F, 4, MODE, IN, 0>), grid, block, lds, st, a); break;
    }
    return (int)hipGetLastError();
}

template <int F, int IN>
int launch_in(int mode, int nr, int pre, const GemvArgs &a, dim3 grid, dim3 block, size_t lds,
              hipStream_t st)
{
    switch (mode) {
    case GEMV_PLAIN: return launch_nr<F, GEMV_PLAIN, IN>(nr, pre, a, grid, block, lds, st);
    case GEMV_SILU: return launch_nr<F, GEMV_SILU, IN>(nr, 0, a, grid, block, lds, st);
    case GEMV_MULTI: return launch_nr<F, GEMV_MULTI, IN>(nr, 0, a, grid, block, lds, st);
    default:
        if (IN != 0) return (int)hipErrorInvalidValue;
        return launch_nr<F, GEMV_ISUMS, 0>(1, 0, a, grid, block, lds, st);
    }
}

} // namespace

// Rows per lane and waves per workgroup: the largest tiles that still give
// at least ~2 workgroups per CU (256 CUs), so that small matrices spread over
// the whole chip and large ones amortise the activation staging.
template <int F> int launch_gemv_format(int mode, const GemvArgs &a, void *stream)
{
    const int rows = a.rows_total;
    int nr = 1, waves = 1;
    if (mode != GEMV_ISUMS) {
        const bool heavy = F == Q6_K || F == Q8_0 || F == Q4_K || mode == GEMV_SILU;
        if (rows >= 8 * 4 * 4 * 1024 && !heavy) nr = 4;
        else if (rows >= 8 * 2 * 4 * 1024) nr = 2;
        if (rows >= 8 * nr * 4 * 512) waves = 4;
        else if (rows >= 8 * nr * 2 * 512) waves = 2;
    }
    // With an f32 input stage every workgroup quantizes the whole input row,
    // so fewer, wider workgroups (4 waves) share that work.
    if (a.xin) waves = 4;
    const int rows_per_block = 8 * nr * waves;
    dim3 grid((rows + rows_per_block - 1) / rows_per_block), block(64 * waves);
    // slots, then (input stage) scales, 256/16/32-value sums and group sums of squares
    const size_t lds = (size_t)a.groups * SLOT_INTS * 4 +
                       (a.xin ? (size_t)a.groups * (4 + 4 + 64 + 32 + 4) : 0);
    // groups per lane preloaded by the plain one-row-per-lane kernel
    const int pre = a.groups <= 32 ? (a.groups + 7) / 8 : 0;
    hipStream_t st = (hipStream_t)stream;
    if (!a.xin) return launch_in<F, 0>(mode, nr, pre, a, grid, block, lds, st);
    if (!a.norm) return launch_in<F, 1>(mode, nr, pre, a, grid, block, lds, st);
    return launch_in<F, 2>(mode, nr, pre, a, grid, block, lds, st);
}

} // namespace hyq
