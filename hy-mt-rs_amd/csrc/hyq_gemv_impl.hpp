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
// sum over each 32-lane half of the wave
__device__ __forceinline__ float sum32(float v)
{
    v = wave::sum16(v);
    return v + __shfl_xor(v, 16);
}

// The f32 input stage, as Q8::quantize_into (src/quant.rs:904-922) and
// q8_quantize_group do, writing the Q8 row to the LDS slots and the group
// scales and 16/32/256-value integer sums to the LDS arrays. Each 32-lane
// half wave quantizes one 256-value group (lane c holds values 8c..8c+7),
// so a 256-thread workgroup takes 8 groups per pass: the group maximum and
// sums are reduced over a 16-lane row by DPP and across the half wave's two
// rows by v_permlane16_swap, with no readlane or LDS round trip, and the
// divisions are branch-free. With a norm vector the values are
// rms_norm_into's x * (w * (1/sqrt(mean(x^2) + eps))) (src/model.rs:785-815);
// the sum of squares is formed per group by a fixed tree and then over the
// groups in ascending order. Rows of up to 8 * STAGE_PASSES groups are loaded
// with all loads in flight at once (before the weights'); longer rows take a
// loop.
constexpr int STAGE_PASSES = 4;

struct StageRegs {
    float4 x[STAGE_PASSES][2];
    float4 w[STAGE_PASSES][2];
    float4 pt[GEMV_MAX_PARTS][2]; // partial rows of pass 0 (rows of <= 8 groups)
};

__device__ __forceinline__ float4 add4(float4 v, float4 p)
{
    return make_float4(v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w);
}

__device__ __forceinline__ float sum_rows(float v) { return wave::sum_rows2(v); }
__device__ __forceinline__ int sum_rows(int v) { return wave::sum_rows2(v); }

__device__ __forceinline__ float sq8(const float4 &a, const float4 &b)
{
    return ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) +
           ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
}

// rms_norm_into's aarch64 arm over whole 16-value steps (src/model.rs:809):
// x * (w * scale)
__device__ __forceinline__ float4 scale_by(float4 v, float scale, float4 w)
{
    return make_float4(v.x * (w.x * scale), v.y * (w.y * scale), v.z * (w.z * scale),
                       v.w * (w.w * scale));
}

__device__ __forceinline__ uint32_t pack4(int q0, int q1, int q2, int q3)
{
    return (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
           ((uint32_t)(q3 & 0xff) << 24);
}

// Group g's 8 values of this lane (c = lane of the half wave); xt (the
// trace hook, workgroup 0 only) receives the values.
__device__ __forceinline__ void quantize_half(float4 a, float4 b, int g, int c, int *slots,
                                              float *sc, int *s256, int *s16, int *s32,
                                              float *xt)
{
    if (xt) {
        reinterpret_cast<float4 *>(xt + g * 256 + 8 * c)[0] = a;
        reinterpret_cast<float4 *>(xt + g * 256 + 8 * c)[1] = b;
    }
    // the group maximum propagates NaN (max_abs_neon's FMAX): a NaN in the
    // group gives scale 0 and zero codes
    using wave::nmax;
    const float la = nmax(nmax(fabsf(a.x), fabsf(a.y)), nmax(fabsf(a.z), fabsf(a.w)));
    const float lb = nmax(nmax(fabsf(b.x), fabsf(b.y)), nmax(fabsf(b.z), fabsf(b.w)));
    const float m = wave::nmax_rows2(wave::nmax16(nmax(la, lb)));
    const bool pos = m > 0.f;
    const float md = pos ? m : 1.f;
    const float s = pos ? md / 127.f : 0.f;
    const float inv = pos ? 127.f / md : 0.f;
    const int q0 = q8_sat_rne(a.x * inv), q1 = q8_sat_rne(a.y * inv);
    const int q2 = q8_sat_rne(a.z * inv), q3 = q8_sat_rne(a.w * inv);
    const int q4 = q8_sat_rne(b.x * inv), q5 = q8_sat_rne(b.y * inv);
    const int q6 = q8_sat_rne(b.z * inv), q7 = q8_sat_rne(b.w * inv);
    *reinterpret_cast<uint2 *>(slots + g * SLOT_INTS + 2 * c) =
        make_uint2(pack4(q0, q1, q2, q3), pack4(q4, q5, q6, q7));
    // integer sums over 16, 32 and 256 values (2, 4 and 32 lanes): exact
    const int t8 = ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7));
    const int t16 = t8 + wave::dpp<wave::DPP_XOR1>(t8);
    if ((c & 1) == 0) s16[g * 16 + (c >> 1)] = t16;
    const int t32 = t16 + wave::dpp<wave::DPP_XOR2>(t16);
    if ((c & 3) == 0) s32[g * 8 + (c >> 2)] = t32;
    int t = t32 + wave::dpp<wave::DPP_HALF_MIRROR>(t32);
    t = sum_rows(t + wave::dpp<wave::DPP_MIRROR>(t));
    if (c == 0) {
        s256[g] = t;
        sc[g] = s;
    }
}

__device__ __forceinline__ float finish_norm(const float *gss, int groups, float eps)
{
    __syncthreads();
    float ss = 0.f;
    for (int g = 0; g < groups; ++g) ss += gss[g];
    return 1.0f / sqrtf(ss / (float)(groups * 256) + eps);
}

// Register path: the loads are issued by stage_load before the weights'
// (loads complete in issue order, so the stage then waits for its own data
// only) and consumed by stage_regs.
template <int IN>
__device__ __forceinline__ void stage_load(const GemvArgs &a, const float *xin, const float *norm,
                                           StageRegs &r)
{
    const int hw = threadIdx.x >> 5, c = threadIdx.x & 31;
    const float4 *x4 = reinterpret_cast<const float4 *>(xin);
    const float4 *n4 = reinterpret_cast<const float4 *>(norm);
#pragma unroll
    for (int p = 0; p < STAGE_PASSES; ++p) {
        const int g = 8 * p + hw;
        if (g < a.groups) {
            r.x[p][0] = x4[g * 64 + 2 * c];
            r.x[p][1] = x4[g * 64 + 2 * c + 1];
            if (IN == 2) {
                r.w[p][0] = n4[g * 64 + 2 * c];
                r.w[p][1] = n4[g * 64 + 2 * c + 1];
            }
        }
    }
    if (a.nsparts > 0 && hw < a.groups) {
#pragma unroll
        for (int k = 0; k < GEMV_MAX_PARTS; ++k)
            if (k < a.nsparts) {
                const float4 *p4 =
                    reinterpret_cast<const float4 *>(a.sparts + (size_t)k * a.parts_stride);
                r.pt[k][0] = p4[hw * 64 + 2 * c];
                r.pt[k][1] = p4[hw * 64 + 2 * c + 1];
            }
    }
}

template <int IN>
__device__ __forceinline__ void stage_regs(const GemvArgs &a, StageRegs &r, int *slots,
                                           float *sc, int *s256, int *s16, int *s32, float *gss,
                                           float *xt)
{
    const int hw = threadIdx.x >> 5, c = threadIdx.x & 31;
    const int groups = a.groups;
    if (a.nsparts > 0 && hw < groups) {
#pragma unroll
        for (int k = 0; k < GEMV_MAX_PARTS; ++k)
            if (k < a.nsparts) {
                r.x[0][0] = add4(r.x[0][0], r.pt[k][0]);
                r.x[0][1] = add4(r.x[0][1], r.pt[k][1]);
            }
    }
    float scale = 1.f;
    if (IN == 2) {
#pragma unroll
        for (int p = 0; p < STAGE_PASSES; ++p) {
            const int g = 8 * p + hw;
            if (g < groups) {
                const float ss = sum_rows(wave::sum16(sq8(r.x[p][0], r.x[p][1])));
                if (c == 0) gss[g] = ss;
            }
        }
        scale = finish_norm(gss, groups, a.eps);
    }
#pragma unroll
    for (int p = 0; p < STAGE_PASSES; ++p) {
        const int g = 8 * p + hw;
        if (g < groups) {
            if (IN == 2)
                quantize_half(scale_by(r.x[p][0], scale, r.w[p][0]),
                              scale_by(r.x[p][1], scale, r.w[p][1]), g, c, slots, sc, s256, s16,
                              s32, xt);
            else
                quantize_half(r.x[p][0], r.x[p][1], g, c, slots, sc, s256, s16, s32, xt);
        }
    }
}

// IN 3: IN 2 whose partial rows span two passes (rows of 9-16 groups: a
// 4096-wide QKV input after a K-split down projection), so that they stay in
// registers instead of taking the loop below; its own instantiation, so
// the other stages keep their registers and code.
constexpr int STAGE3_PASSES = 2;
struct StageRegs3 {
    float4 x[STAGE3_PASSES][2];
    float4 w[STAGE3_PASSES][2];
    float4 pt[GEMV_MAX_PARTS][STAGE3_PASSES][2];
};

__device__ __forceinline__ void stage_load3(const GemvArgs &a, const float *xin, const float *norm,
                                            StageRegs3 &r)
{
    const int hw = threadIdx.x >> 5, c = threadIdx.x & 31;
    const float4 *x4 = reinterpret_cast<const float4 *>(xin);
    const float4 *n4 = reinterpret_cast<const float4 *>(norm);
#pragma unroll
    for (int p = 0; p < STAGE3_PASSES; ++p) {
        const int g = 8 * p + hw;
        if (g < a.groups) {
            r.x[p][0] = x4[g * 64 + 2 * c];
            r.x[p][1] = x4[g * 64 + 2 * c + 1];
            r.w[p][0] = n4[g * 64 + 2 * c];
            r.w[p][1] = n4[g * 64 + 2 * c + 1];
#pragma unroll
            for (int k = 0; k < GEMV_MAX_PARTS; ++k)
                if (k < a.nsparts) {
                    const float4 *p4 =
                        reinterpret_cast<const float4 *>(a.sparts + (size_t)k * a.parts_stride);
                    r.pt[k][p][0] = p4[g * 64 + 2 * c];
                    r.pt[k][p][1] = p4[g * 64 + 2 * c + 1];
                }
        }
    }
}

__device__ __forceinline__ void stage_regs3(const GemvArgs &a, StageRegs3 &r, int *slots,
                                            float *sc, int *s256, int *s16, int *s32, float *gss,
                                            float *xt)
{
    const int hw = threadIdx.x >> 5, c = threadIdx.x & 31;
    const int groups = a.groups;
#pragma unroll
    for (int p = 0; p < STAGE3_PASSES; ++p) {
        const int g = 8 * p + hw;
        if (g < groups) {
#pragma unroll
            for (int k = 0; k < GEMV_MAX_PARTS; ++k)
                if (k < a.nsparts) {
                    r.x[p][0] = add4(r.x[p][0], r.pt[k][p][0]);
                    r.x[p][1] = add4(r.x[p][1], r.pt[k][p][1]);
                }
            const float ss = sum_rows(wave::sum16(sq8(r.x[p][0], r.x[p][1])));
            if (c == 0) gss[g] = ss;
        }
    }
    const float scale = finish_norm(gss, groups, a.eps);
#pragma unroll
    for (int p = 0; p < STAGE3_PASSES; ++p) {
        const int g = 8 * p + hw;
        if (g < groups)
            quantize_half(scale_by(r.x[p][0], scale, r.w[p][0]),
                          scale_by(r.x[p][1], scale, r.w[p][1]), g, c, slots, sc, s256, s16, s32,
                          xt);
    }
}

// Longer rows: a loop over the passes (loads at the top of each).
template <int IN>
__device__ __forceinline__ void stage_loop(const GemvArgs &a, const float *xin, const float *norm,
                                           int *slots, float *sc, int *s256, int *s16, int *s32,
                                           float *gss, float *xt)
{
    const int hw = threadIdx.x >> 5, c = threadIdx.x & 31;
    const int groups = a.groups;
    const float4 *x4 = reinterpret_cast<const float4 *>(xin);
    const float4 *n4 = reinterpret_cast<const float4 *>(norm);
    // the input pair of lane c of group g, with the partial rows added
    auto input = [&](int g, float4 &va, float4 &vb) {
        va = x4[g * 64 + 2 * c];
        vb = x4[g * 64 + 2 * c + 1];
        for (int k = 0; k < a.nsparts; ++k) {
            const float4 *p4 = reinterpret_cast<const float4 *>(a.sparts + (size_t)k * a.parts_stride);
            va = add4(va, p4[g * 64 + 2 * c]);
            vb = add4(vb, p4[g * 64 + 2 * c + 1]);
        }
    };
    float scale = 1.f;
    if (IN == 2) {
        for (int g = hw; g < groups; g += 8) {
            float4 va, vb;
            input(g, va, vb);
            const float ss = sum_rows(wave::sum16(sq8(va, vb)));
            if (c == 0) gss[g] = ss;
        }
        scale = finish_norm(gss, groups, a.eps);
    }
    for (int g = hw; g < groups; g += 8) {
        float4 va, vb;
        input(g, va, vb);
        if (IN == 2) {
            va = scale_by(va, scale, n4[g * 64 + 2 * c]);
            vb = scale_by(vb, scale, n4[g * 64 + 2 * c + 1]);
        }
        quantize_half(va, vb, g, c, slots, sc, s256, s16, s32, xt);
    }
}

// Q8 input rows (no input stage) of up to Q8_REG int4 per thread are read
// into registers before the weights' loads are issued, then copied to LDS;
// the row's scales and the integer sums a group's dot reads are loaded by
// each lane from global memory into registers just before the group's
// weights (one row per lane with Q8 input).
constexpr int Q8_REG = 8;
// (a clang vector type: an array of HIP's int4 struct is not promoted to
// registers here)
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Half-group mode (HALF_GEMV<F, NR, MODE, IN>): 16 lanes share a row and
// each 256-weight group goes to two of them (lane 2i + h takes half h of
// group i + 8k), so a workgroup covers 16 rows with half the per-lane work;
// the two halves' integer sums meet by DPP before the group's one float
// product, which keeps the result bit-identical to the full-group mode.
constexpr int HALF_MAX_WORKGROUPS = 256;
template <int F, int NR, int MODE, int IN>
constexpr bool HALF_GEMV = HasHalf<F>::value && IN != 0 && NR == 1 && MODE != GEMV_ISUMS;

// SLOT: the expert-slot forms of an MoE layer (GemvArgs::slot_expert), a
// separate instantiation so that the other kernels carry none of it.
template <int F, int NR, int MODE, int IN, int P, bool H, int SL = 0, bool SLOT = false>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a)
{
    static_assert(!H || HALF_GEMV<F, NR, MODE, IN>, "half-group mode: see HALF_GEMV");
    static_assert(!SLOT || (NR == 1 && !H && SL == 0 && P == 0 &&
                            (MODE == GEMV_SILU || MODE == GEMV_PLAIN)),
                  "expert slots: one row per lane, gate/up or plain");
    static_assert(SL == 0 || ((SL == 64 || SL == 32 || SL == 16) && !H && NR == 1 &&
                              (MODE == GEMV_PLAIN || (MODE == GEMV_SILU && SL == 16))),
                  "wide rows: 16, 32 or 64 lanes per row (16 for gate/up), one row per lane");
    using G = typename GroupOf<F>::T;
    using Dt = typename GemvData<G, H>::T;
    constexpr int SUBL = SL ? SL : H ? 16 : 8; // lanes per row
    constexpr int GSTEP = H ? 8 : SUBL;        // groups a row-set takes per step
    extern __shared__ int lds[];

    const int groups = a.groups;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane & (SUBL - 1);
    const int gi = H ? sub >> 1 : sub; // first group of this lane
    const int hh = H ? sub & 1 : 0;    // half of the group (half-group mode)
    const int rset = lane / SUBL;
    const int nwaves = blockDim.x >> 6;
    const int row0 = ((blockIdx.x * nwaves + wave) * (64 / SUBL) + rset) * NR;
    // K slice of this workgroup row (kslices > 1: plain mode, f32 input
    // without norm or partial rows): groups [gbase, gbase + groups); or the
    // expert slot of this workgroup row (slot form: whole rows)
    const int gbase = SLOT ? 0 : blockIdx.y * groups;
    const float *xin =
        a.xin + (SLOT ? (size_t)blockIdx.y * a.slot_xin_stride : (size_t)gbase * 256);
    // the slot's expert, first of all loads: the weight addresses need it
    int slot_e = 0;
    if (SLOT && a.nslots) slot_e = min(max(a.slot_expert[blockIdx.y], 0), a.slot_experts - 1);

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
    // the weight rows the loads read (an expert's rows in a stack)
    int wrow[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        wrow[i] = lrowc[i];
        if constexpr (SLOT) {
            if (a.nslots) {
                wrow[i] = slot_e * a.rows_total + lrowc[i];
            } else {
                const int slot = lrowc[i] / a.slot_rows;
                const int e = min(max(a.slot_expert[slot], 0), a.slot_experts - 1);
                wrow[i] = e * a.slot_rows + (lrowc[i] - slot * a.slot_rows);
            }
        }
    }

    auto load = [&](Dt &D, const WView &w, int row, int g) {
        if constexpr (H) G::load_half(D, w, row, gbase + g, hh);
        else G::load(D, w, row, gbase + g);
    };
    // The Q8 words a group's dot reads besides the activations: from LDS
    // where an input stage puts them, read at their use (Q8At); with Q8
    // input from global memory into registers (G::Meta), loaded just before
    // the group's weights so that their latency overlaps the weights'
    // instead of following it.
    static_assert(IN != 0 || NR == 1, "Q8 input: one row per lane");
    using Mt = typename G::Meta;
    constexpr bool META_PRE = IN == 0;
    Dt d[NR];
    Dt d2[MODE == GEMV_SILU ? NR : 1];
    auto load_group = [&](int g) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const WView &w = MODE == GEMV_MULTI ? a.seg[seg[i]].w : a.seg[0].w;
            load(d[i], w, wrow[i], g);
            if (MODE == GEMV_SILU) load(d2[i], a.seg[1].w, wrow[i], g);
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
    StageRegs sr;
    StageRegs3 sr3;
    // int4 loads per thread: a preloading kernel covers at most GSTEP * P
    // groups (16 int4 each) with 64 threads (256 in the 32- and 64-lane
    // forms), so it issues no more than those need (the surplus would re-read
    // the clamped last int4); other block sizes take the loop below
    constexpr int QW = SL >= 32 ? 4 : 1;
    constexpr int NQ = P > 0 && GSTEP * P / (4 * QW) < Q8_REG ? GSTEP * P / (4 * QW) : Q8_REG;
    i32x4 qv[NQ];
    const bool stage_reg =
        IN == 3 ? groups <= 8 * STAGE3_PASSES
                : IN != 0 && groups <= 8 * STAGE_PASSES && (a.nsparts == 0 || groups <= 8);
    const bool q8_reg = IN == 0 && groups * 16 <= NQ * (int)blockDim.x;
    if constexpr (IN == 3) {
        if (stage_reg) stage_load3(a, xin, a.norm, sr3);
    } else if (IN != 0 && stage_reg) {
        stage_load<IN>(a, xin, a.norm, sr);
    }
    if (IN == 0 && q8_reg) {
        // clamped into bounds; the copy to LDS keeps the in-range ones
        const i32x4 *src = reinterpret_cast<const i32x4 *>(a.x.q);
#pragma unroll
        for (int j = 0; j < NQ; ++j)
            qv[j] = src[min((int)threadIdx.x + j * (int)blockDim.x, groups * 16 - 1)];
    }
    static_assert(P == 0 || (NR == 1 && MODE == GEMV_PLAIN), "preload: plain, one row per lane");
    Dt dp[P > 0 ? P : 1];
    Mt mp[P > 0 ? P : 1];
    Mt md; // the current group's (P == 0)
    if (P > 0) {
#pragma unroll
        for (int u = 0; u < P; ++u) {
            const int gu = min(gi + GSTEP * u, groups - 1);
            if constexpr (META_PRE) mp[u] = G::meta(a.x, gu);
            load(dp[u], a.seg[0].w, wrow[0], gu);
        }
    } else {
        if constexpr (META_PRE) md = G::meta(a.x, min(gi, groups - 1));
        load_group(min(gi, groups - 1));
    }
    // the plain epilogue's residual and partial rows, loaded now (after the
    // weights', so that nothing waits for them) rather than at the end
    float res[GEMV_MAX_PARTS + 1][NR];
    if (MODE == GEMV_PLAIN && (a.residual || a.nrparts)) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            res[0][i] = a.residual ? a.residual[lrowc[i]] : 0.f;
#pragma unroll
            for (int k = 0; k < GEMV_MAX_PARTS; ++k)
                if (k < a.nrparts) res[k + 1][i] = a.rparts[(size_t)k * a.parts_stride + lrowc[i]];
        }
    }
    Q8View xq = a.x;
    // (input stage) scales, then 256/16/32-value sums after the slots
    float *sc = reinterpret_cast<float *>(lds + groups * SLOT_INTS);
    int *s256 = reinterpret_cast<int *>(sc + groups);
    int *s16 = s256 + groups;
    int *s32 = s16 + groups * 16;
    if (IN != 0) {
        xq.s = sc;
        xq.sum256 = s256;
        xq.sum16 = s16;
        xq.sum32 = s32;
    }
    if (IN == 0) {
        const int4 *src = reinterpret_cast<const int4 *>(a.x.q);
        int4 *dst = reinterpret_cast<int4 *>(lds);
        if (q8_reg) {
#pragma unroll
            for (int j = 0; j < NQ; ++j) {
                const int i = threadIdx.x + j * (int)blockDim.x;
                if (i < groups * 16)
                    reinterpret_cast<i32x4 *>(dst)[(i >> 4) * (SLOT_INTS / 4) + (i & 15)] = qv[j];
            }
        } else {
            for (int i = threadIdx.x; i < groups * 16; i += blockDim.x)
                dst[(i >> 4) * (SLOT_INTS / 4) + (i & 15)] = src[i];
        }
    } else {
        float *gss = reinterpret_cast<float *>(s32 + groups * 8);
        // (test hook) workgroup 0 of the slice or slot records its values
        float *xt = a.q8t_x && blockIdx.x == 0
                        ? a.q8t_x + (size_t)(SLOT ? (int)blockIdx.y * groups : gbase) * 256
                        : nullptr;
        if constexpr (IN == 3) {
            if (stage_reg) stage_regs3(a, sr3, lds, sc, s256, s16, s32, gss, xt);
            else stage_loop<2>(a, xin, a.norm, lds, sc, s256, s16, s32, gss, xt);
        } else {
            if (stage_reg) stage_regs<IN>(a, sr, lds, sc, s256, s16, s32, gss, xt);
            else stage_loop<IN>(a, xin, a.norm, lds, sc, s256, s16, s32, gss, xt);
        }
    }
    __syncthreads();
    if constexpr (IN != 0) {
        // (test hook) the codes and scales this stage formed, as they sit in
        // LDS, from workgroup 0 of the slice or slot
        if (a.q8t_codes && blockIdx.x == 0) {
            const int gb = SLOT ? (int)blockIdx.y * groups : gbase;
            int *codes = reinterpret_cast<int *>(a.q8t_codes) + (size_t)gb * 64;
            for (int i = threadIdx.x; i < groups * 64; i += blockDim.x)
                codes[i] = lds[(i >> 6) * SLOT_INTS + (i & 63)];
            for (int g = threadIdx.x; g < groups; g += blockDim.x) a.q8t_scales[gb + g] = sc[g];
        }
    }

    float acc[NR];
    float acc2[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = acc2[i] = 0.f;

    // the lane's activation dwords of group g: the whole slot (64), or half
    // hh of it (32) in half-group mode
    constexpr int NACT = H ? 32 : 64;
    auto stage_act = [&](int g, int (&act)[NACT]) {
        const int4 *s4 = reinterpret_cast<const int4 *>(lds + g * SLOT_INTS + hh * 32);
#pragma unroll
        for (int j = 0; j < NACT / 4; ++j) {
            const int4 v = s4[j];
            act[4 * j] = v.x;
            act[4 * j + 1] = v.y;
            act[4 * j + 2] = v.z;
            act[4 * j + 3] = v.w;
        }
    };
    // acc plus group g's contribution of one matrix row. Half-group mode:
    // the two halves' integer sums meet by DPP and lane hh == 0 accumulates
    // the group (as the full-group mode of the same format does, one fused
    // multiply-add per group), lane hh == 1 keeps zero.
    auto accum = [&](float acc, const Dt &D, const auto &m, const int (&act)[NACT],
                     int g) -> float {
        if constexpr (H) {
            int is = G::isum_half(D, act, xq, g, hh);
            is += wave::dpp<wave::DPP_XOR1>(is);
            const float r = G::finish_acc(acc, is, D.d, xq, g);
            return hh ? acc : r;
        } else if constexpr (HasHalf<F>::value) {
            return G::dot_acc(acc, D, act, m);
        } else {
            return acc + G::template dot<false>(D, act, m, nullptr);
        }
    };
    // group g's Q8 words: the preloaded ones, or an accessor of the LDS copy
    auto meta_of = [&](const Mt &pre, int g) {
        if constexpr (META_PRE) return pre;
        else return Q8At{xq, g};
    };
    if constexpr (P > 0) {
#pragma unroll
        for (int u = 0; u < P; ++u) {
            const int g = gi + GSTEP * u;
            // (uniform over each pair of half lanes, so the DPP partner is live)
            if (g >= groups || !valid[0]) continue;
            int act[NACT];
            stage_act(g, act);
            acc[0] = accum(acc[0], dp[u], meta_of(mp[u], g), act, g);
        }
    } else if constexpr (NR == 1 && MODE != GEMV_SILU) {
        // The lane's next group is in flight while the current one is used:
        // two register sets, the loop unrolled by two; the load past the
        // lane's last group re-reads group groups - 1 (in bounds, unused).
        Dt e[NR];
        Dt e2[MODE == GEMV_SILU ? NR : 1];
        Mt me;
        auto load_into = [&](Dt *dd, Dt *dd2, Mt &mm, int g) {
            if constexpr (META_PRE) mm = G::meta(a.x, g);
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const WView &w = MODE == GEMV_MULTI ? a.seg[seg[i]].w : a.seg[0].w;
                load(dd[i], w, wrow[i], g);
                if (MODE == GEMV_SILU) load(dd2[i], a.seg[1].w, wrow[i], g);
            }
        };
        auto step = [&](const Dt *dc, const Dt *dc2, const Mt &mm, int g) {
            int act[NACT];
            stage_act(g, act);
            const auto m = meta_of(mm, g);
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                if (!valid[i]) continue;
                if constexpr (MODE == GEMV_ISUMS && !H) {
                    int32_t *out = a.isums + ((size_t)lrow[i] * groups + g) * G::ISUMS;
                    acc[i] += G::template dot<true>(dc[i], act, m, out);
                } else {
                    acc[i] = accum(acc[i], dc[i], m, act, g);
                    if (MODE == GEMV_SILU) acc2[i] = accum(acc2[i], dc2[i], m, act, g);
                }
            }
        };
        int g = gi;
        for (; g + GSTEP < groups; g += 2 * GSTEP) {
            load_into(e, e2, me, g + GSTEP);
            step(d, d2, md, g);
            load_into(d, d2, md, min(g + 2 * GSTEP, groups - 1));
            step(e, e2, me, g + GSTEP);
        }
        if (g < groups) step(d, d2, md, g);
    } else {
        for (int g = gi; g < groups; g += GSTEP) {
            int act[NACT];
            stage_act(g, act);
            if (g != gi) {
                if constexpr (META_PRE) md = G::meta(a.x, g);
                load_group(g);
            }
            const auto m = meta_of(md, g);
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                if (!valid[i]) continue;
                if constexpr (MODE == GEMV_ISUMS && !H) {
                    int32_t *out = a.isums + ((size_t)lrow[i] * groups + g) * G::ISUMS;
                    acc[i] += G::template dot<true>(d[i], act, m, out);
                } else {
                    acc[i] = accum(acc[i], d[i], m, act, g);
                    if (MODE == GEMV_SILU) acc2[i] = accum(acc2[i], d2[i], m, act, g);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const float v = (H || SUBL == 16) ? wave::sum16(acc[i])
                        : SUBL == 64              ? wave::sum64(acc[i])
                        : SUBL == 32              ? sum32(acc[i])
                                                  : reduce8(acc[i]);
        const float v2 =
            MODE == GEMV_SILU ? ((H || SUBL == 16) ? wave::sum16(acc2[i]) : reduce8(acc2[i])) : 0.f;
        if (sub != 0 || !valid[i] || MODE == GEMV_ISUMS) continue;
        if (MODE == GEMV_SILU) {
            a.seg[0].y[lrow[i]] = silu_mul(v, v2);
        } else if (MODE == GEMV_MULTI) {
            a.seg[seg[i]].y[lrow[i]] = v;
        } else {
            if (a.kslices > 1 || (SLOT && a.nslots)) {
                a.seg[0].y[(size_t)blockIdx.y * a.rows_total + lrow[i]] = v;
            } else {
                float r = res[0][i];
#pragma unroll
                for (int k = 0; k < GEMV_MAX_PARTS; ++k)
                    if (k < a.nrparts) r += res[k + 1][i];
                a.seg[0].y[lrow[i]] = a.residual || a.nrparts ? r + v : v;
            }
        }
    }
}

template <int F, int MODE, int IN, bool H>
int launch_nr(int nr, int pre, const GemvArgs &a, dim3 grid, dim3 block, size_t lds,
              hipStream_t st)
{
    if constexpr (H) {
        // half-group kernels: one row per lane (preloads in plain mode)
        if constexpr (MODE == GEMV_PLAIN) {
            switch (pre) {
            case 1: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 1, true>), grid, block, lds, st, a); break;
            case 2: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 2, true>), grid, block, lds, st, a); break;
            case 3: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 3, true>), grid, block, lds, st, a); break;
            case 4: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 4, true>), grid, block, lds, st, a); break;
            default: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0, true>), grid, block, lds, st, a); break;
            }
        } else {
            hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0, true>), grid, block, lds, st, a);
        }
        return (int)hipGetLastError();
    } else {
        if constexpr (MODE == GEMV_PLAIN) {
            if (nr == 1) switch (pre) {
            case 1: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 1, false>), grid, block, lds, st, a); break;
            case 2: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 2, false>), grid, block, lds, st, a); break;
            case 3: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 3, false>), grid, block, lds, st, a); break;
            case 4: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 4, false>), grid, block, lds, st, a); break;
            default: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0, false>), grid, block, lds, st, a); break;
            }
            if (nr == 1) return (int)hipGetLastError();
        }
        if constexpr (IN == 2) {
            switch (nr) {
            case 1: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0, false>), grid, block, lds, st, a); break;
            case 2: hipLaunchKernelGGL((gemv_kernel<F, 2, MODE, IN, 0, false>), grid, block, lds, st, a); break;
            default: hipLaunchKernelGGL((gemv_kernel<F, 4, MODE, IN, 0, false>), grid, block, lds, st, a); break;
            }
        } else {
            // (several rows per lane only under an RMSNorm stage)
            if (nr != 1) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL((gemv_kernel<F, 1, MODE, IN, 0, false>), grid, block, lds, st, a);
        }
        return (int)hipGetLastError();
    }
}

template <int F, int IN, bool H>
int launch_in(int mode, int nr, int pre, const GemvArgs &a, dim3 grid, dim3 block, size_t lds,
              hipStream_t st)
{
    switch (mode) {
    case GEMV_PLAIN: return launch_nr<F, GEMV_PLAIN, IN, H>(nr, pre, a, grid, block, lds, st);
    case GEMV_SILU: return launch_nr<F, GEMV_SILU, IN, H>(nr, 0, a, grid, block, lds, st);
    case GEMV_MULTI: return launch_nr<F, GEMV_MULTI, IN, H>(nr, 0, a, grid, block, lds, st);
    default:
        if (IN != 0 || H) return (int)hipErrorInvalidValue;
        return launch_nr<F, GEMV_ISUMS, 0, false>(1, 0, a, grid, block, lds, st);
    }
}

} // namespace

// Rows per lane and waves per workgroup: the largest tiles that still give
// at least ~2 workgroups per CU (256 CUs), so that small matrices spread over
// the whole chip and large ones amortise the activation staging.
template <int F> int launch_gemv_format(int mode, const GemvArgs &a, void *stream)
{
    const int rows = a.rows_total;
    // One row per lane, measured fastest with Q8 input or a plain f32 stage
    // at every size (e.g. vocabulary-sized rows against two per lane: Q6_K
    // [120818 x 2048] 42.3 -> 33.5 us with Q8 input, 40.4 -> 34.0 us from an
    // f32 row; Q2_0C [131072 x 2048] 18.8 -> 13.1 us, against four). An
    // RMSNorm stage costs each workgroup more, so there matrices of 64Ki
    // rows and more take two (four for the lighter formats) rows per lane
    // (the decode step's lm_head: ~5 us per token faster than with one).
    int nr = 1;
    if (mode != GEMV_ISUMS && a.norm) {
        const bool heavy = F == Q6_K || F == Q8_0 || F == Q4_K || mode == GEMV_SILU;
        if (rows >= 8 * 4 * 4 * 1024 && !heavy) nr = 4;
        else if (rows >= 8 * 2 * 4 * 1024) nr = 2;
    }
    // Q8 input: single-wave workgroups (measured fastest, 7B shapes of
    // 6144-28672 rows). An f32 input stage is repeated by every workgroup,
    // so fewer, wider workgroups (4 waves) share that work.
    int waves = a.xin ? 4 : 1;
    const int ks = a.nslots > 0 ? a.nslots : a.kslices > 1 ? a.kslices : 1;
    // wide rows (32 lanes per row, two rows per wave): a plain GEMV of at
    // least 32 groups per row whose 8-lane row-sets would leave most SIMDs
    // without a wave; chosen from the shape alone, for the Q8 and the f32
    // input alike, so that both launches sum in the same order
    const bool wide = mode == GEMV_PLAIN && nr == 1 && ks == 1 && a.norm == nullptr &&
                      a.groups >= 32 && rows < 8 * 2048;
    // 16 lanes per row (four rows per wave), on the same terms, for 16-31
    // groups per row on fewer than 4096 rows, where 8-lane row-sets give
    // under two workgroups per CU and three or four groups per lane; at any
    // row count for Q6_K and STQ1_0, whose dots are the heaviest per byte
    // ([32000 x 4096] Q6_K 25.0 -> 20.0 us, [28672 x 4096] STQ1_0 9.17 ->
    // 9.04 us; Q4_K [6144 x 4096] measured 3 % slower so)
    const bool w16 = mode == GEMV_PLAIN && nr == 1 && ks == 1 && a.norm == nullptr &&
                     a.groups >= 16 && a.groups < 32 &&
                     (rows < 4096 || F == Q6_K || F == STQ1_0);
    // 64 lanes per row (one group each, one row per wave, 4-wave workgroups)
    // for the long rows of the two formats with the heaviest dots: the 7B
    // down [4096 x 14336] Q6_K 13.9 -> 11.9 us, STQ1_0 6.5 -> 6.4 us (Q4_K
    // and Q8_0 measured 4-5 % slower so)
    const bool w64 = wide && a.groups > 32 && a.groups <= 64 && (F == Q6_K || F == STQ1_0);
    // half-group mode (Q2_0C, f32 stage, one row per lane; 4 rows per wave)
    // when its workgroups (twice the full-group count) still fit the 256 CUs
    // one each: a CU holding two would be the launch's tail
    const int half_wgs = (rows + 4 * waves - 1) / (4 * waves) * ks;
    const bool half = HasHalf<F>::value && a.xin && nr == 1 && mode != GEMV_ISUMS && !wide &&
                      !w16 && half_wgs <= HALF_MAX_WORKGROUPS;
    if (wide) waves = 4;
    // gate/up from Q8 input, 9-16 groups per row: 16 lanes per row, so that
    // each lane's one group of both matrices is loaded before the activations
    // are staged (with 8 lanes the second group loads after the first's dots);
    // for the formats with the heaviest dots ([2 x 14336 x 4096] Q4_K 14.7 ->
    // 14.5 us, STQ1_0 9.8 -> 9.4 us; Q2_0C 8.1 -> 8.5 us, and under an
    // RMSNorm stage the 7B decode step 1.77 -> 1.82 ms per token, so not
    // there)
    const bool s16 = mode == GEMV_SILU && !a.xin && nr == 1 && ks == 1 && a.groups > 8 &&
                     a.groups <= 16 && (F == Q4_K || F == STQ1_0 || F == Q6_K);
    const int rows_per_block = (w64 ? 1 : wide ? 2 : w16 || half || s16 ? 4 : 8) * nr * waves;
    // a K split is a plain GEMV of an f32 row without norm, residual or
    // partial-row inputs (each slice writes its own partial row)
    if ((ks > 1 || a.nslots) &&
        (mode != GEMV_PLAIN || !a.xin || a.norm || a.residual || a.nsparts || a.nrparts))
        return (int)hipErrorInvalidValue;
    if (a.slot_expert && (a.slot_experts <= 0 || (!a.nslots && a.slot_rows <= 0)))
        return (int)hipErrorInvalidValue;
    if (a.nslots && (a.kslices > 1 || !a.slot_expert)) return (int)hipErrorInvalidValue;
    if (a.nsparts > GEMV_MAX_PARTS || a.nrparts > GEMV_MAX_PARTS) return (int)hipErrorInvalidValue;
    if (a.slot_expert) {
        // expert slots: one row per lane; gate/up from Q8 input (row form)
        // or a plain product of f32 rows quantized in the launch (slot form)
        const int wv = a.xin ? 4 : (rows >= 8 * 4 * 512 ? 4 : rows >= 8 * 2 * 512 ? 2 : 1);
        const dim3 sgrid((rows + 8 * wv - 1) / (8 * wv), ks), sblock(64 * wv);
        const size_t slds = (size_t)a.groups * SLOT_INTS * 4 +
                            (size_t)a.groups * (4 + 4 + 64 + 32) +
                            (a.xin ? (size_t)a.groups * 4 : 0);
        hipStream_t sst = (hipStream_t)stream;
        if (mode == GEMV_SILU && !a.xin && !a.nslots)
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_SILU, 0, 0, false, 0, true>), sgrid,
                               sblock, slds, sst, a);
        else if (mode == GEMV_PLAIN && a.xin && !a.norm && a.nslots)
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 1, 0, false, 0, true>), sgrid,
                               sblock, slds, sst, a);
        else
            return (int)hipErrorInvalidValue;
        return (int)hipGetLastError();
    }
    dim3 grid((rows + rows_per_block - 1) / rows_per_block, ks), block(64 * waves);
    // slots, then (input stage) scales, 256/16/32-value sums and group sums of squares
    const size_t lds = (size_t)a.groups * SLOT_INTS * 4 + (size_t)a.groups * (4 + 4 + 64 + 32) +
                       (a.xin ? (size_t)a.groups * 4 : 0);
    // groups per lane preloaded by the plain one-row-per-lane kernel
    const int pre = a.groups <= 32 ? (a.groups + 7) / 8 : 0;
    hipStream_t st = (hipStream_t)stream;
    if (w64) {
        if (!a.xin)
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 0, 1, false, 64>), grid, block, lds, st, a);
        else
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 1, 1, false, 64>), grid, block, lds, st, a);
        return (int)hipGetLastError();
    }
    if (wide) {
        // rows of at most 64 groups: both of a lane's groups preloaded
        // before the input stage (the same sums in the same order)
        if (a.groups <= 64) {
            if (!a.xin)
                hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 0, 2, false, 32>), grid, block, lds, st, a);
            else
                hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 1, 2, false, 32>), grid, block, lds, st, a);
        } else if (!a.xin) {
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 0, 0, false, 32>), grid, block, lds, st, a);
        } else {
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 1, 0, false, 32>), grid, block, lds, st, a);
        }
        return (int)hipGetLastError();
    }
    if (s16) {
        hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_SILU, 0, 0, false, 16>), grid, block, lds, st, a);
        return (int)hipGetLastError();
    }
    if (w16) {
        // one or two groups per lane, all preloaded
        if (a.groups <= 16) {
            if (!a.xin)
                hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 0, 1, false, 16>), grid, block, lds, st, a);
            else
                hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 1, 1, false, 16>), grid, block, lds, st, a);
        } else if (!a.xin) {
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 0, 2, false, 16>), grid, block, lds, st, a);
        } else {
            hipLaunchKernelGGL((gemv_kernel<F, 1, GEMV_PLAIN, 1, 2, false, 16>), grid, block, lds, st, a);
        }
        return (int)hipGetLastError();
    }
    if (!a.xin) return launch_in<F, 0, false>(mode, nr, pre, a, grid, block, lds, st);
    // the fused QKV launch with an RMSNorm stage over 9-16 groups that adds
    // partial rows: IN 3 keeps them in registers for both passes
    const bool two_pass_parts =
        mode == GEMV_MULTI && nr == 1 && a.nsparts > 0 && a.groups > 8 && a.groups <= 16;
    if constexpr (HasHalf<F>::value) {
        if (half) {
            if (!a.norm) return launch_in<F, 1, true>(mode, nr, pre, a, grid, block, lds, st);
            if (two_pass_parts)
                return launch_nr<F, GEMV_MULTI, 3, true>(1, 0, a, grid, block, lds, st);
            return launch_in<F, 2, true>(mode, nr, pre, a, grid, block, lds, st);
        }
    }
    if (!a.norm) return launch_in<F, 1, false>(mode, nr, pre, a, grid, block, lds, st);
    if (two_pass_parts) return launch_nr<F, GEMV_MULTI, 3, false>(1, 0, a, grid, block, lds, st);
    return launch_in<F, 2, false>(mode, nr, pre, a, grid, block, lds, st);
}

} // namespace hyq
