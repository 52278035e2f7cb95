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
#include <hip/hip_runtime.h>

#include "hyq_groups.hpp"

namespace hyq {

namespace {

constexpr int SLOT_INTS = 68; // 256 bytes of a group + 16 bytes of padding

__device__ __forceinline__ float silu_mul(float g, float u)
{
    // silu(g) * u with silu(g) = g / (1 + exp(-g)) (src/quant.rs:573-574)
    float silu = g / (1.0f + expf(-g));
    return silu * u;
}

__device__ __forceinline__ float reduce8(float v)
{
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    return v;
}

template <int F, int NR, int MODE>
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

    typename G::Data d[NR];
    typename G::Data d2[MODE == GEMV_SILU ? NR : 1];
    auto load_group = [&](int g) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            if (!valid[i]) continue;
            const WView &w = MODE == GEMV_MULTI ? a.seg[seg[i]].w : a.seg[0].w;
            G::load(d[i], w, lrow[i], g);
            if (MODE == GEMV_SILU) G::load(d2[i], a.seg[1].w, lrow[i], g);
        }
    };
    // The first group's weights do not depend on the activations: put their
    // loads in flight before staging the Q8 row, so both latencies overlap.
    if (sub < groups) load_group(sub);
    {
        const int4 *src = reinterpret_cast<const int4 *>(a.x.q);
        int4 *dst = reinterpret_cast<int4 *>(lds);
        for (int i = threadIdx.x; i < groups * 16; i += blockDim.x)
            dst[(i >> 4) * (SLOT_INTS / 4) + (i & 15)] = src[i];
    }
    __syncthreads();

    float acc[NR];
    float acc2[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = acc2[i] = 0.f;

    for (int g = sub; g < groups; g += 8) {
        int act[64];
        {
            const int4 *s4 = reinterpret_cast<const int4 *>(lds + g * SLOT_INTS);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int4 v = s4[j];
                act[4 * j] = v.x;
                act[4 * j + 1] = v.y;
                act[4 * j + 2] = v.z;
                act[4 * j + 3] = v.w;
            }
        }
        if (g != sub) load_group(g);
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            if (!valid[i]) continue;
            if (MODE == GEMV_ISUMS) {
                int32_t *out = a.isums + ((size_t)lrow[i] * groups + g) * G::ISUMS;
                acc[i] += G::template dot<true>(d[i], act, a.x, g, out);
            } else {
                acc[i] += G::template dot<false>(d[i], act, a.x, g, nullptr);
                if (MODE == GEMV_SILU)
                    acc2[i] += G::template dot<false>(d2[i], act, a.x, g, nullptr);
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

template <int F, int MODE>
int launch_nr(int nr, const GemvArgs &a, dim3 grid, dim3 block, size_t lds, hipStream_t st)
{
    switch (nr) {
    case 1: hipLaunchKernelGGL((gemv_kernel<F, 1, MODE>), grid, block, lds, st, a); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<F, 2, MODE>), grid, block, lds, st, a); break;
    default: hipLaunchKernelGGL((gemv_kernel<F, 4, MODE>), grid, block, lds, st, a); break;
    }
    return (int)hipGetLastError();
}

template <int F>
int launch_fmt(int mode, int nr, const GemvArgs &a, dim3 grid, dim3 block, size_t lds,
               hipStream_t st)
{
    switch (mode) {
    case GEMV_PLAIN: return launch_nr<F, GEMV_PLAIN>(nr, a, grid, block, lds, st);
    case GEMV_SILU: return launch_nr<F, GEMV_SILU>(nr, a, grid, block, lds, st);
    case GEMV_MULTI: return launch_nr<F, GEMV_MULTI>(nr, a, grid, block, lds, st);
    default: return launch_nr<F, GEMV_ISUMS>(1, a, grid, block, lds, st);
    }
}

} // namespace

int isums_per_group(int fmt)
{
    switch (fmt) {
    case Q2_0C: return GroupQ2C::ISUMS;
    case STQ1_0: return GroupSTQ::ISUMS;
    case Q4_K: return GroupQ4K::ISUMS;
    case Q6_K: return GroupQ6K::ISUMS;
    case Q8_0: return GroupQ80::ISUMS;
    default: return -1;
    }
}

// Rows per lane and waves per workgroup: the largest tiles that still give
// at least ~2 workgroups per CU (256 CUs), so that small matrices spread over
// the whole chip and large ones amortise the activation staging.
int launch_gemv(int fmt, int mode, const GemvArgs &a, void *stream)
{
    const int rows = a.rows_total;
    int nr = 1, waves = 1;
    if (mode != GEMV_ISUMS) {
        const bool heavy = fmt == Q6_K || fmt == Q8_0 || fmt == Q4_K || mode == GEMV_SILU;
        if (rows >= 8 * 4 * 4 * 1024 && !heavy) nr = 4;
        else if (rows >= 8 * 2 * 4 * 1024) nr = 2;
        if (rows >= 8 * nr * 4 * 512) waves = 4;
        else if (rows >= 8 * nr * 2 * 512) waves = 2;
    }
    const int rows_per_block = 8 * nr * waves;
    dim3 grid((rows + rows_per_block - 1) / rows_per_block), block(64 * waves);
    const size_t lds = (size_t)a.groups * SLOT_INTS * 4;
    hipStream_t st = (hipStream_t)stream;
    switch (fmt) {
    case Q2_0C: return launch_fmt<Q2_0C>(mode, nr, a, grid, block, lds, st);
    case STQ1_0: return launch_fmt<STQ1_0>(mode, nr, a, grid, block, lds, st);
    case Q4_K: return launch_fmt<Q4_K>(mode, nr, a, grid, block, lds, st);
    case Q6_K: return launch_fmt<Q6_K>(mode, nr, a, grid, block, lds, st);
    case Q8_0: return launch_fmt<Q8_0>(mode, nr, a, grid, block, lds, st);
    default: return (int)hipErrorInvalidValue;
    }
}

} // namespace hyq
