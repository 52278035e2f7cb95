// Batched products on gfx950 with the f16-MFMA tile engine of hyq_tile.hpp:
//   gemm_f16      Weight::matmul at batch >= 2 (src/quant.rs:272-344):
//                 Y[batch, rows] = X[batch, cols] W^T;
//   moe_*         Moe::forward's expert loop (src/model.rs:699-725): token
//                 rows grouped by expert, each expert's DenseFfn as a
//                 gate/up GEMM with the SiLU product in its epilogue and a
//                 down GEMM, then the routed sum in ascending expert order.
//
// Activations are rounded to f16 once (to_f16 / the gate-up epilogue) and
// read by the tiles as f16. Tile order is XCD-aware: workgroups are
// dispatched round-robin over the 8 XCDs, so workgroup b runs on XCD b % 8;
// tile (b % 8) * per + b / 8 gives each XCD a contiguous range of tiles, and
// the tiles sharing one weight row block land on the same XCD and its L2.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hyq_f16rows.hpp"
#include "hyq_few_q80.hpp"
#include "hyq_moe_operand.hpp"
#include "hyq_tile.hpp"
#include "hyq_wave.hpp"

#pragma clang fp contract(off)

namespace hyq {

namespace {

using namespace tile;

__device__ __forceinline__ int xcd_tile(int total)
{
    const int per = (total + 7) / 8;
    return (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
}

// One workgroup per row: xh[r][k] = f16(v[k] * 2^-e) and rscale[r] = 2^e,
// where v = x[src] (or, with `norm`, its RMSNorm v[k] = x[k] * (norm[k] * s)
// over whole 16-value steps and x[k] * s * norm[k] over a tail, s = 1 /
// sqrt(mean(x^2) + eps), the aarch64 arm of src/model.rs:832-870) and
// e = ceil(log2(max_k |v[k]|)) - 14 puts the row's largest magnitude at or
// below 2^14, so no value overflows f16 or drops into its subnormals; the
// power-of-two scale is exact and the GEMM epilogues multiply it back.
// src = r, or ptok[order[r]] when order is given; rows r >= *count (when
// count is given) are left alone. A row with a zero, infinite or NaN maximum
// keeps scale 1 (and its infinities / NaNs propagate).
//
// R > 0 (rows of at most 1024 R values): thread t holds float4s t + 256 j,
// j < R, of the row (and of the norm vector) in registers, all their loads
// issued at once (clamped into the row) before the first is used, so a row
// costs one memory latency instead of one per float4 of a thread, and the
// passes (sum of squares, maximum, conversion) read the registers. R = 0
// loops over the row in global memory (any length). Every value is formed
// by the same operations in the same order either way.
template <int R>
__global__ __launch_bounds__(256) void rows_to_f16_kernel(const float *__restrict__ x, int K,
                                                          int nrows,
                                                          const int *__restrict__ order,
                                                          const int *__restrict__ ptok,
                                                          const int *__restrict__ count,
                                                          const float *__restrict__ norm,
                                                          float eps,
                                                          _Float16 *__restrict__ xh,
                                                          float *__restrict__ rscale,
                                                          bool frag)
{
    __shared__ float wred[4];
    const int r = frag ? frag_row((int)blockIdx.x) : (int)blockIdx.x;
    if (r >= nrows || (count && r >= *count)) return;
    const size_t src = order ? (size_t)ptok[order[r]] : (size_t)r;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + src * K);
    const float4 *n4p = reinterpret_cast<const float4 *>(norm);
    const int t = threadIdx.x, n4 = K / 4;
    constexpr int NJ = R > 0 ? R : 1;
    float4 xv[NJ], wv[NJ];
    if constexpr (R > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) xv[j] = x4[min(t + 256 * j, n4 - 1)];
        if (norm) {
#pragma unroll
            for (int j = 0; j < R; ++j) wv[j] = n4p[min(t + 256 * j, n4 - 1)];
        }
    }
    // float4 i = t + 256 j of the row, before the norm
    auto raw = [&](int j, int i) { return R > 0 ? xv[j] : x4[i]; };
    // The passes below visit i = t + 256 j for j = 0, 1, ... while i < n4:
    // unrolled over the registers for R > 0, a loop for R = 0.
    auto each = [&](auto &&f) {
        if constexpr (R > 0) {
#pragma unroll
            for (int j = 0; j < R; ++j)
                if (t + 256 * j < n4) f(j, t + 256 * j);
        } else {
            for (int i = t; i < n4; i += 256) f(0, i);
        }
    };
    float s = 1.f;
    if (norm) {
        float ss = 0.f;
        each([&](int j, int i) {
            const float4 v = raw(j, i);
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        });
        ss = wave::sum64(ss);
        if ((t & 63) == 0) wred[t >> 6] = ss;
        __syncthreads();
        ss = (wred[0] + wred[1]) + (wred[2] + wred[3]);
        __syncthreads();
        s = 1.0f / sqrtf(ss / (float)K + eps);
    }
    auto value = [&](int j, int i) {
        float4 v = raw(j, i);
        if (norm) {
            const float4 w = R > 0 ? wv[j] : n4p[i];
            if (4 * i < (K & ~15))
                v = make_float4(v.x * (w.x * s), v.y * (w.y * s), v.z * (w.z * s),
                                v.w * (w.w * s));
            else
                v = make_float4(v.x * s * w.x, v.y * s * w.y, v.z * s * w.z, v.w * s * w.w);
        }
        return v;
    };
    float m = 0.f;
    each([&](int j, int i) {
        const float4 v = value(j, i);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w) m = INFINITY;
    });
    m = wave::max64(m);
    if ((t & 63) == 0) wred[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
    const int e = f16_row_exponent(m);
    const float inv = ldexpf(1.0f, -e);
    if (t == 0) rscale[r] = ldexpf(1.0f, e);
    // (fragment order: values 4i .. 4i + 3 stay together, k % 8 being 0 or 4)
    _Float16 *o = frag ? xh + (size_t)(r / 32) * 32 * K + (size_t)(r % 32) * 8 : xh + (size_t)r * K;
    each([&](int j, int i) {
        const float4 v = value(j, i);
        const half2v a = __builtin_convertvector((float2v){v.x * inv, v.y * inv}, half2v);
        const half2v b = __builtin_convertvector((float2v){v.z * inv, v.w * inv}, half2v);
        const int k = 4 * i;
        _Float16 *q = frag ? o + (size_t)(k / 16) * 512 + 256 * ((k / 8) & 1) + (k & 4) : o + k;
        *reinterpret_cast<half2v *>(q) = a;
        *reinterpret_cast<half2v *>(q + 2) = b;
    });
}

// rows_to_f16_kernel for rows of K values: the register form with the fewest
// registers that holds the row, else the loop. In fragment order the grid
// is the rows rounded up to 64 (see frag_row).
void launch_rows_to_f16(int rows, int K, hipStream_t st, const float *x, const int *order,
                        const int *ptok, const int *count, const float *norm, float eps,
                        _Float16 *xh, float *rscale, bool frag)
{
    const int need = K < 4 ? 1 << 30 : (K + 1023) / 1024;
    const dim3 grid(frag ? (rows + 63) / 64 * 64 : rows);
#define HYQ_ROWS_F16(RR)                                                                       \
    hipLaunchKernelGGL(rows_to_f16_kernel<RR>, grid, dim3(256), 0, st, x, K, rows, order, ptok, \
                       count, norm, eps, xh, rscale, frag)
    if (need <= 2) HYQ_ROWS_F16(2);
    else if (need <= 4) HYQ_ROWS_F16(4);
    else if (need <= 6) HYQ_ROWS_F16(6);
    else if (need <= 8) HYQ_ROWS_F16(8);
    else if (need <= 12) HYQ_ROWS_F16(12);
    else if (need <= 16) HYQ_ROWS_F16(16);
    else HYQ_ROWS_F16(0);
#undef HYQ_ROWS_F16
}

// Y[n][m] = (X[n] . W[m]) * rscale[n], plus residual[n][m] when given (the
// residual add of src/model.rs:595, 601 after the product is rounded; it
// may alias y: each element is read and then written by one thread). The
// row space is up to three weights sharing the activation rows (Q, K and V
// in one launch); a tile's BM rows lie in one of them (its row count is a
// multiple of BM, or it is the last). With kslices > 1 (one weight) grid.y
// splits K: slice z writes its scaled partial product to
// part[z][n][m] and gemm_reduce_kernel adds the slices in order. NW waves
// per workgroup: tiles of BM rows by 32 NW tokens, the same arithmetic per
// element for NW = 4 and 8 (the 256-token tiles of a plain product run as
// gemm_f16_pc_kernel, the same arithmetic again).
template <int F, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void gemm_f16_kernel(
    GemmSegs g, int K, const _Float16 *__restrict__ xh, const float *__restrict__ rscale, int N,
    int mtiles, int ntiles, int kslices, float *__restrict__ part)
{
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<NW>()];
    const int T = xcd_tile(mtiles * ntiles);
    if (T >= mtiles * ntiles) return;
    int mt = T / ntiles, sg = 0;
    while (sg + 1 < g.nseg && mt >= g.s[sg].tiles) mt -= g.s[sg++].tiles;
    const GemmSeg &S = g.s[sg];
    const int M = S.rows;
    const int m0 = mt * BM, n0 = (T % ntiles) * (32 * NW);
    const int wave = threadIdx.x >> 6, wm = wave / (NW / 2), wn = wave % (NW / 2);

    f32x16 acc[2][2];
    zero_acc(acc);
    auto wsrc = [&](int lrow, WView &v, int &row) {
        v = S.w;
        row = m0 + lrow < M ? m0 + lrow : -1;
    };
    auto xrow = [&](int r) -> const _Float16 * {
        return n0 + r < N ? xh + (size_t)(n0 + r) * K : nullptr;
    };
    auto arow = [&](int i) { return wm * 64 + 32 * i; };
    const int kslice = K / kslices;
    k_loop<F, 2, NW>(wsrc, xrow, arow, kslice, wn, lds, acc, blockIdx.y * kslice);

    float *y = kslices > 1 ? part + (size_t)blockIdx.y * N * M : S.y;
    const float *residual = kslices > 1 ? nullptr : S.residual;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + acc_col(wn, j);
            if (n >= N) continue;
            float *yr = y + (size_t)n * M;
            const float *rr = residual ? residual + (size_t)n * M : nullptr;
            const float sc = rscale[n];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int m = m0 + arow(i) + acc_row_in_block(4 * g4);
                if (m + 3 < M && (M & 3) == 0) {
                    float4 v = make_float4(acc[i][j][4 * g4] * sc, acc[i][j][4 * g4 + 1] * sc,
                                           acc[i][j][4 * g4 + 2] * sc, acc[i][j][4 * g4 + 3] * sc);
                    if (rr) {
                        const float4 a = *reinterpret_cast<const float4 *>(rr + m);
                        v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
                    }
                    *reinterpret_cast<float4 *>(yr + m) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e < M) {
                            const float v = acc[i][j][4 * g4 + e] * sc;
                            yr[m + e] = rr ? rr[m + e] + v : v;
                        }
                }
            }
        }
}

// gemm_f16_kernel's 256-token tiles in the producer/consumer form of the
// K loop (k_loop_pc): the same grid, the same tile order and bit-identical
// results; waves 4-7 hold the sums and write them. (The fused gate/up keeps
// the 8-wave k_loop: its SiLU epilogue on four waves instead of eight made
// the 1.8B prefill 2.4 % slower.)
template <int F>
__global__ __launch_bounds__(PC_THREADS, 1) void gemm_f16_pc_kernel(
    GemmSegs g, int K, const _Float16 *__restrict__ xh, const float *__restrict__ rscale, int N,
    int mtiles, int ntiles, int kslices, float *__restrict__ part)
{
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<8>()];
    const int T = xcd_tile(mtiles * ntiles);
    if (T >= mtiles * ntiles) return;
    int mt = T / ntiles, sg = 0;
    while (sg + 1 < g.nseg && mt >= g.s[sg].tiles) mt -= g.s[sg++].tiles;
    const GemmSeg &S = g.s[sg];
    const int M = S.rows;
    const int m0 = mt * BM, n0 = (T % ntiles) * 256;

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    auto wsrc = [&](int lrow, WView &v, int &row) {
        v = S.w;
        row = m0 + lrow < M ? m0 + lrow : -1;
    };
    auto xrow = [&](int r) -> const _Float16 * {
        return n0 + r < N ? xh + (size_t)(n0 + r) * K : nullptr;
    };
    const int c = (threadIdx.x >> 6) & 3, wm = c >> 1, wn = c & 1;
    auto arow = [&](int i) { return wm * 64 + 32 * i; };
    const int kslice = K / kslices;
    k_loop_pc<F>(wsrc, xrow, arow, kslice, lds, acc, blockIdx.y * kslice);
    if (threadIdx.x < 256) return; // the producers

    float *y = kslices > 1 ? part + (size_t)blockIdx.y * N * M : S.y;
    const float *residual = kslices > 1 ? nullptr : S.residual;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 128 + 32 * j + (threadIdx.x & 31);
            if (n >= N) continue;
            float *yr = y + (size_t)n * M;
            const float *rr = residual ? residual + (size_t)n * M : nullptr;
            const float sc = rscale[n];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int m = m0 + wm * 64 + 32 * i + acc_row_in_block(4 * g4);
                if (m + 3 < M && (M & 3) == 0) {
                    float4 v = make_float4(acc[i][j][4 * g4] * sc, acc[i][j][4 * g4 + 1] * sc,
                                           acc[i][j][4 * g4 + 2] * sc, acc[i][j][4 * g4 + 3] * sc);
                    if (rr) {
                        const float4 a = *reinterpret_cast<const float4 *>(rr + m);
                        v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
                    }
                    *reinterpret_cast<float4 *>(yr + m) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e < M) {
                            const float v = acc[i][j][4 * g4 + e] * sc;
                            yr[m + e] = rr ? rr[m + e] + v : v;
                        }
                }
            }
        }
}

// The 256-token tiles with the activations, in fragment order
// (launch_to_f16 with frag), straight into the consumers' registers
// (k_loop_pcx): the tile order of gemm_f16_pc_kernel over tiles of 32 NI
// weight rows (128, or 96 where that fills more of the CUs), bit-identical
// results; consumer wave 4 + c writes tokens 64 c ...
template <int F, int NI>
__global__ __launch_bounds__(PC_THREADS, 1) void gemm_f16_pcx_kernel(
    GemmSegs g, int K, const _Float16 *__restrict__ xh, const float *__restrict__ rscale, int N,
    int mtiles, int ntiles, int kslices, float *__restrict__ part)
{
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * TILE_HALVES];
    const int T = xcd_tile(mtiles * ntiles);
    if (T >= mtiles * ntiles) return;
    int mt = T / ntiles, sg = 0;
    while (sg + 1 < g.nseg && mt >= g.s[sg].tiles) mt -= g.s[sg++].tiles;
    const GemmSeg &S = g.s[sg];
    const int M = S.rows;
    const int m0 = mt * (32 * NI), n0 = (T % ntiles) * 256;

    f32x16 acc[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    auto wsrc = [&](int lrow, WView &v, int &row) {
        v = S.w;
        row = m0 + lrow < M ? m0 + lrow : -1;
    };
    // the fragment-order run of the 32-token block holding tile token r
    // (clamped into the batch's blocks)
    auto xsrc = [&](int r) -> const _Float16 * {
        return xh + (size_t)min((n0 + r) / 32, (N - 1) / 32) * 32 * K;
    };
    const int kslice = K / kslices;
    k_loop_pcx<F, NI>(wsrc, xsrc, kslice, lds, acc, blockIdx.y * kslice);
    if (threadIdx.x < 256) return; // the producers
    const int c = (threadIdx.x >> 6) & 3;

    float *y = kslices > 1 ? part + (size_t)blockIdx.y * N * M : S.y;
    const float *residual = kslices > 1 ? nullptr : S.residual;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + 64 * c + 32 * j + (threadIdx.x & 31);
            if (n >= N) continue;
            float *yr = y + (size_t)n * M;
            const float *rr = residual ? residual + (size_t)n * M : nullptr;
            const float sc = rscale[n];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int m = m0 + 32 * i + acc_row_in_block(4 * g4);
                if (m + 3 < M && (M & 3) == 0) {
                    float4 v = make_float4(acc[i][j][4 * g4] * sc, acc[i][j][4 * g4 + 1] * sc,
                                           acc[i][j][4 * g4 + 2] * sc, acc[i][j][4 * g4 + 3] * sc);
                    if (rr) {
                        const float4 a = *reinterpret_cast<const float4 *>(rr + m);
                        v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
                    }
                    *reinterpret_cast<float4 *>(yr + m) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e < M) {
                            const float v = acc[i][j][4 * g4 + e] * sc;
                            yr[m + e] = rr ? rr[m + e] + v : v;
                        }
                }
            }
        }
}

// y = residual + (((part[0] + part[1]) + part[2]) + ...) over `count`
// floats (float4 lanes; count a multiple of 4): the K slices of a split GEMM
// added in slice order, then the residual, as the unsplit epilogue adds it.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float4 *__restrict__ part,
                                                          int kslices, size_t count4,
                                                          const float4 *residual, float4 *y)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count4) return;
    float4 v = part[i];
    for (int z = 1; z < kslices; ++z) {
        const float4 p = part[(size_t)z * count4 + i];
        v = make_float4(v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w);
    }
    if (residual) {
        const float4 r = residual[i];
        v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
    }
    y[i] = v;
}

// ---------------------------------------------------------------------------
// MoE planning: one workgroup groups the routed (token, expert) pairs.
//   order[q]   pair at position q of the expert-grouped sequence (experts
//              ascending; inside an expert, pairs in input order - the order
//              in which Moe::forward pushes assignments, src/model.rs:694-697)
//   eoff[e]    first position of expert e (eoff[E] = valid pairs)
//   tiles[i]   (expert, chunk) of every chunk of a non-empty expert: BN tokens
//              for the LDS-tiled kernels, 16 for the Q4_K register kernels
//   toff/tlist for each token, its positions q in ascending expert order
//              (the order the scatter-add visits them, src/model.rs:700-722)
// Pairs whose token or expert is out of range are dropped.
// ---------------------------------------------------------------------------
constexpr int PLAN_MAX = 4096; // experts and tokens per call

// Exclusive scan of cnt[0..n) in LDS into off[0..n] (global), 256 threads:
// each thread sums a contiguous range, the range sums are scanned within each
// wave by shuffles and across the four waves through lsum[0..3].
__device__ void block_exclusive_scan(const int *cnt, int n, int *off, int *lsum)
{
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (n + 255) / 256;
    const int lo = t * per, hi = min(n, lo + per);
    int s = 0;
    for (int i = lo; i < hi; ++i) s += cnt[i];
    int v = s; // inclusive scan over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d);
        if (lane >= d) v += u;
    }
    if (lane == 63) lsum[w] = v;
    __syncthreads();
    int wb = 0;
    for (int j = 0; j < w; ++j) wb += lsum[j];
    int run = wb + v - s;
    for (int i = lo; i < hi; ++i) {
        off[i] = run;
        run += cnt[i];
    }
    if (t == 255) off[n] = wb + v;
    __syncthreads();
}

// Stable counting sort: for i in [0, n), rank[i] = number of j < i with
// key(j) == key(i), plus the running count of key(i) from earlier chunks;
// cnt[k] ends as the total count of key k. key < 0 = skipped.
template <class KeyFn>
__device__ void stable_rank(const KeyFn &key, int n, int *cnt, int nkeys, int *rank, int *lkey)
{
    const int t = threadIdx.x;
    for (int i = t; i < nkeys; i += 256) cnt[i] = 0;
    __syncthreads();
    for (int base = 0; base < n; base += 256) {
        const int i = base + t;
        const int k = i < n ? key(i) : -1;
        lkey[t] = k;
        __syncthreads();
        if (k >= 0) {
            // keys of the earlier threads, four per LDS read, four reads in flight
            const int4 *l4 = reinterpret_cast<const int4 *>(lkey);
            int r = 0;
#pragma unroll 4
            for (int j = 0; j < (t >> 2); ++j) {
                const int4 v = l4[j];
                r += (v.x == k) + (v.y == k) + (v.z == k) + (v.w == k);
            }
            for (int j = t & ~3; j < t; ++j) r += lkey[j] == k;
            rank[i] = cnt[k] + r;
        }
        __syncthreads();
        if (k >= 0) atomicAdd(&cnt[k], 1);
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void moe_plan_kernel(const int *__restrict__ ptok,
                                                       const int *__restrict__ pexp, int P, int T,
                                                       int E, int *eoff, int *order, int *rank,
                                                       int *toff, int *tlist, int *tiles,
                                                       int *ntiles, int chunk)
{
    __shared__ int cnt[PLAN_MAX];
    __shared__ __attribute__((aligned(16))) int lkey[256];
    __shared__ int lsum[256];
    const int t = threadIdx.x;
    auto ekey = [&](int p) {
        const int tok = ptok[p], e = pexp[p];
        return (tok >= 0 && tok < T && e >= 0 && e < E) ? e : -1;
    };
    // group pairs by expert (stable)
    stable_rank(ekey, P, cnt, E, rank, lkey);
    block_exclusive_scan(cnt, E, eoff, lsum);
    for (int p = t; p < P; p += 256) {
        const int e = ekey(p);
        if (e >= 0) order[eoff[e] + rank[p]] = p;
    }
    // chunk-token chunks of every expert
    for (int e = t; e < E; e += 256) cnt[e] = (cnt[e] + chunk - 1) / chunk;
    __syncthreads();
    block_exclusive_scan(cnt, E, rank, lsum); // rank[0..E] reused as chunk offsets
    for (int e = t; e < E; e += 256)
        for (int c = 0; c < cnt[e]; ++c) {
            tiles[2 * (rank[e] + c)] = e;
            tiles[2 * (rank[e] + c) + 1] = c;
        }
    if (t == 0) *ntiles = rank[E];
    __syncthreads();
    // for each token, its positions in ascending expert order
    const int nv = eoff[E];
    auto tkey = [&](int q) { return ptok[order[q]]; };
    stable_rank(tkey, nv, cnt, T, rank, lkey);
    block_exclusive_scan(cnt, T, toff, lsum);
    for (int q = t; q < nv; q += 256) tlist[toff[tkey(q)] + rank[q]] = q;
}

// The plan for up to PLAN_SMALL pairs (and at most PLAN_SMALL tokens and
// experts) with every intermediate in LDS: the same outputs as
// moe_plan_kernel, without its global round trips between the steps.
constexpr int PLAN_SMALL = 2048;

__device__ void lds_exclusive_scan(const int *cnt, int n, int *off, int *lsum)
{
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (n + 255) / 256;
    const int lo = t * per, hi = min(n, lo + per);
    int s = 0;
    for (int i = lo; i < hi; ++i) s += cnt[i];
    int v = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d);
        if (lane >= d) v += u;
    }
    if (lane == 63) lsum[w] = v;
    __syncthreads();
    int wb = 0;
    for (int j = 0; j < w; ++j) wb += lsum[j];
    int run = wb + v - s;
    for (int i = lo; i < hi; ++i) {
        off[i] = run;
        run += cnt[i];
    }
    if (t == 255) off[n] = wb + v;
    __syncthreads();
}

// rank[i] = number of j < i with key[j] == key[i] (key < 0 skipped), cnt[k]
// = count of key k; all arrays in LDS, key 16-byte aligned and padded with
// -1 to a multiple of 4.
__device__ void lds_stable_rank(const int *key, int n, int *cnt, int nkeys, int *rank)
{
    const int t = threadIdx.x;
    for (int k = t; k < nkeys; k += 256) cnt[k] = 0;
    __syncthreads();
    for (int base = 0; base < n; base += 256) {
        const int i = base + t;
        const int k = i < n ? key[i] : -1;
        if (k >= 0) {
            const int4 *l4 = reinterpret_cast<const int4 *>(key + base);
            int r = 0;
#pragma unroll 4
            for (int j = 0; j < (t >> 2); ++j) {
                const int4 v = l4[j];
                r += (v.x == k) + (v.y == k) + (v.z == k) + (v.w == k);
            }
            for (int j = t & ~3; j < t; ++j) r += key[base + j] == k;
            rank[i] = cnt[k] + r;
        }
        __syncthreads();
        if (k >= 0) atomicAdd(&cnt[k], 1);
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void moe_plan_small_kernel(
    const int *__restrict__ ptok, const int *__restrict__ pexp, int P, int T, int E, int *eoff,
    int *order, int *toff, int *tlist, int *tiles, int *ntiles, int chunk)
{
    __shared__ int cnt[PLAN_SMALL];
    __shared__ int off[PLAN_SMALL + 1];
    __shared__ __attribute__((aligned(16))) int key[PLAN_SMALL + 4];
    __shared__ int tok[PLAN_SMALL];
    __shared__ int ord[PLAN_SMALL];
    __shared__ int rank[PLAN_SMALL + 1];
    __shared__ int lsum[4];
    const int t = threadIdx.x;
    const int P4 = (P + 3) & ~3;
    for (int p = t; p < P4; p += 256) {
        int e = -1, tk = -1;
        if (p < P) {
            tk = ptok[p];
            e = pexp[p];
            if (!(tk >= 0 && tk < T && e >= 0 && e < E)) e = -1;
        }
        key[p] = e;
        tok[p] = tk;
    }
    __syncthreads();
    // group pairs by expert (stable)
    lds_stable_rank(key, P, cnt, E, rank);
    lds_exclusive_scan(cnt, E, off, lsum);
    for (int e = t; e <= E; e += 256) eoff[e] = off[e];
    for (int p = t; p < P; p += 256)
        if (key[p] >= 0) ord[off[key[p]] + rank[p]] = p;
    __syncthreads();
    const int nv = off[E];
    for (int q = t; q < nv; q += 256) order[q] = ord[q];
    // chunk-token chunks of every expert
    for (int e = t; e < E; e += 256) cnt[e] = (off[e + 1] - off[e] + chunk - 1) / chunk;
    __syncthreads();
    lds_exclusive_scan(cnt, E, rank, lsum); // rank[0..E]: chunk offsets
    for (int e = t; e < E; e += 256)
        for (int c = 0; c < cnt[e]; ++c) {
            tiles[2 * (rank[e] + c)] = e;
            tiles[2 * (rank[e] + c) + 1] = c;
        }
    if (t == 0) *ntiles = rank[E];
    __syncthreads();
    // for each token, its positions in ascending expert order
    const int nv4 = (nv + 3) & ~3;
    for (int q = t; q < nv4; q += 256) key[q] = q < nv ? tok[ord[q]] : -1;
    __syncthreads();
    lds_stable_rank(key, nv, cnt, T, rank);
    lds_exclusive_scan(cnt, T, off, lsum);
    for (int k = t; k <= T; k += 256) toff[k] = off[k];
    for (int q = t; q < nv; q += 256) tlist[off[key[q]] + rank[q]] = q;
}

// The plan for up to PLAN_FAST pairs, tokens and experts, with at most
// PLAN_FAST_TAB (batch, key) cells per grouping, on 1024 threads: the same
// outputs as moe_plan_small_kernel. A grouping's stable rank comes from
// bit masks instead of pairwise compares: in batch b (64 consecutive
// elements, one wave) every lane sets its bit in the mask of (b, its key)
// with one LDS atomic OR, so the bits below its own give its rank among the
// batch's equal keys and the mask's population the key's batch count; a
// per-key prefix over the batches and a scan over the keys then place
// element i at off[key] + (its key's count in earlier batches) + (its rank
// in its batch).
constexpr int PLAN_FAST = 1024;
constexpr int PLAN_FAST_TAB = 4096;

// Exclusive scan of v[0..n) in place (n <= 1024 * 4), v[n] = the total; all
// 1024 threads.
__device__ void lds_scan_1024(int *v, int n, int *lsum)
{
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (n + 1023) / 1024, lo = min(n, t * per), hi = min(n, lo + per);
    int s = 0;
    for (int i = lo; i < hi; ++i) s += v[i];
    int x = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(x, d);
        if (lane >= d) x += u;
    }
    if (lane == 63) lsum[w] = x;
    __syncthreads();
    int run = x - s;
    for (int j = 0; j < w; ++j) run += lsum[j];
    for (int i = lo; i < hi; ++i) {
        const int c = v[i];
        v[i] = run;
        run += c;
    }
    if (t == 1023) v[n] = run;
    __syncthreads();
}

// Stable grouping of key[0..n) (key < 0: not grouped) into nkeys groups:
// off[0..nkeys] = the exclusive scan of the group sizes, and element i goes
// to off[key[i]] + tab[(i / 64) nkeys + key[i]] + rk[i]. Needs
// ceil(n / 64) nkeys <= PLAN_FAST_TAB; all 1024 threads.
__device__ void lds_group_1024(const int *key, int n, int nkeys, unsigned long long *tab,
                               int *rk, int *off, int *lsum)
{
    const int t = threadIdx.x, lane = t & 63, nb = (n + 63) / 64;
    for (int i = t; i < nb * nkeys; i += 1024) tab[i] = 0;
    __syncthreads();
    const unsigned long long below = (1ull << lane) - 1;
    for (int b = t >> 6; b < nb; b += 16) {
        const int i = 64 * b + lane;
        const int k = i < n ? key[i] : -1;
        if (k >= 0) {
            unsigned long long *m = tab + b * nkeys + k;
            atomicOr(m, 1ull << lane);
            // one wave's LDS operations complete in order, and the batch is
            // this wave's alone: the read sees the bit of every lane of it
            rk[i] = __popcll(*m & below);
        }
    }
    __syncthreads();
    for (int k = t; k < nkeys; k += 1024) {
        unsigned long long s = 0;
        for (int b = 0; b < nb; ++b) {
            const unsigned long long c = __popcll(tab[b * nkeys + k]);
            tab[b * nkeys + k] = s;
            s += c;
        }
        off[k] = (int)s;
    }
    __syncthreads();
    lds_scan_1024(off, nkeys, lsum);
}

__host__ __device__ inline bool plan_fast_fits(int P, int T, int E)
{
    const long nb = (P + 63) / 64;
    return P <= PLAN_FAST && T <= PLAN_FAST && E <= PLAN_FAST && nb * E <= PLAN_FAST_TAB &&
           nb * T <= PLAN_FAST_TAB;
}

// Workgroups 0 and 1 make the plan, each grouping the pairs by expert: 0
// writes eoff, order and the tiles, 1 the per-token lists (toff, tlist). With
// x given (the Q4_K register-operand kernels), workgroups 2, 3, ... also form
// the row operand of each token row of x [T, K] (wave_row_operand: xop, xhs,
// xsc), one wave per row, and the plan also writes, per chunk column (ti, col), the pair position it takes
// (cpos: the chunk's last pair for columns past its pairs) and that pair's
// token (ctok). With xf given, a second wave per row writes the row's f16
// fragments for a few-token Q8_0 product (hyq_few_q80.hpp; zeros for the rows
// past T of the last 16-row chunk), scaled by the same 2^-e (its own
// maximum of the row): xsc is then that product's row scale too.
__global__ __launch_bounds__(1024) void moe_plan_fast_kernel(
    const int *__restrict__ ptok, const int *__restrict__ pexp, int P, int T, int E, int *eoff,
    int *order, int *toff, int *tlist, int *tiles, int *ntiles, int chunk,
    const float *__restrict__ x, int K, uint4 *__restrict__ xop, uint2 *__restrict__ xhs,
    float *__restrict__ xsc, int *__restrict__ cpos, int *__restrict__ ctok,
    _Float16 *__restrict__ xf)
{
    const int t = threadIdx.x;
    if (blockIdx.x > 1) {
        // one wave per row, or with xf two: the row operand and the fragments
        const int w = t >> 6;
        const int r = (xf ? 8 * (blockIdx.x - 2) + (w >> 1) : 16 * (blockIdx.x - 2) + w);
        if (!xf || !(w & 1)) {
            if (r < T)
                wave_row_operand(x + (size_t)r * K, K, xop + (size_t)r * (K / 8),
                                 xhs + (size_t)r * (K / 64), xsc + r);
            return;
        }
        const float *xr = r < T ? x + (size_t)r * K : nullptr;
        const int e = xr ? f16_row_exponent(wave_row_absmax(xr, K)) : 0;
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        for (int p = t & 63; p < K / 8; p += 64)
            few::fragment_piece(x4, ldexpf(1.0f, -e), r, p, K, xf);
        return;
    }
    __shared__ int key[PLAN_FAST];
    __shared__ int tok[PLAN_FAST];
    __shared__ int rk[PLAN_FAST + 1];
    __shared__ int ord[PLAN_FAST];
    __shared__ unsigned long long tab[PLAN_FAST_TAB];
    __shared__ int off[PLAN_FAST + 1];
    __shared__ int lsum[16];
    // tile -> expert: at most P / chunk + min(E, P) tiles for chunk >= 16
    __shared__ int tle[PLAN_FAST + PLAN_FAST / 16 + 1];
    // workgroup 1 forms the per-token lists; both group the pairs by expert
    const bool tokens_wg = blockIdx.x == 1;
    for (int p = t; p < P; p += 1024) {
        const int tk = ptok[p], e = pexp[p];
        key[p] = tk >= 0 && tk < T && e >= 0 && e < E ? e : -1;
        tok[p] = tk;
    }
    __syncthreads();
    // group pairs by expert (stable)
    lds_group_1024(key, P, E, tab, rk, off, lsum);
    if (!tokens_wg)
        for (int e = t; e <= E; e += 1024) eoff[e] = off[e];
    for (int p = t; p < P; p += 1024) {
        const int e = key[p];
        if (e >= 0) ord[off[e] + (int)tab[(p >> 6) * E + e] + rk[p]] = p;
    }
    __syncthreads();
    const int nv = off[E];
    if (!tokens_wg) {
        for (int q = t; q < nv; q += 1024) order[q] = ord[q];
        // chunk-token chunks of every expert (counts in rk, scanned)
        for (int e = t; e < E; e += 1024) rk[e] = (off[e + 1] - off[e] + chunk - 1) / chunk;
        __syncthreads();
        lds_scan_1024(rk, E, lsum);
        for (int e = t; e < E; e += 1024)
            for (int c = 0; c < rk[e + 1] - rk[e]; ++c) {
                tiles[2 * (rk[e] + c)] = e;
                tiles[2 * (rk[e] + c) + 1] = c;
                tle[rk[e] + c] = e;
            }
        const int nt = rk[E];
        if (t == 0) *ntiles = nt;
        if (cpos) {
            __syncthreads();
            // each chunk column's pair position (the chunk's last pair past
            // its pairs) and token, one column per thread
            for (int i = t; i < nt * chunk; i += 1024) {
                const int ti = i / chunk, col = i - ti * chunk, e = tle[ti];
                const int nb = off[e] + (ti - rk[e]) * chunk, last = min(chunk, off[e + 1] - nb) - 1;
                const int q = nb + min(col, last);
                cpos[i] = q;
                ctok[i] = tok[ord[q]];
            }
        }
        return;
    }
    // for each token, its positions in ascending expert order
    for (int q = t; q < nv; q += 1024) key[q] = tok[ord[q]];
    __syncthreads();
    lds_group_1024(key, nv, T, tab, rk, off, lsum);
    for (int k = t; k <= T; k += 1024) toff[k] = off[k];
    for (int q = t; q < nv; q += 1024) {
        const int k = key[q];
        tlist[off[k] + (int)tab[(q >> 6) * T + k] + rk[q]] = q;
    }
}

__device__ __forceinline__ float silu_mul(float g, float u)
{
    // (g / (1 + exp(-g))) * u, DenseFfn::forward (src/model.rs:680-682)
    return (g / (1.0f + expf(-g))) * u;
}

// Gate and up of one expert chunk: LDS rows 0..63 dequantize gate rows
// m0..m0+63 and rows 64..127 the same rows of up; wave (wm, wn) holds gate
// rows 32*wm.. in acc[0] and the matching up rows in acc[1], so the SiLU
// product pairs registers one to one. H[q][m] = silu(g) * u in f32, with g
// and u scaled back by the token row's activation scale.
template <int F>
__global__ __launch_bounds__(256, 2) void moe_gate_up_kernel(
    WView gate, WView up, int mid, int K, const int *__restrict__ eoff,
    const int *__restrict__ tiles, const int *__restrict__ ntiles,
    const _Float16 *__restrict__ xg, const float *__restrict__ xscale, float *__restrict__ H,
    int mtiles, int max_tiles)
{
    __shared__ __attribute__((aligned(16))) _Float16 lds[4 * TILE_HALVES];
    const int T = xcd_tile(mtiles * max_tiles);
    if (T >= mtiles * max_tiles) return;
    const int ti = T / mtiles, mt = T % mtiles;
    if (ti >= *ntiles) return;
    const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
    const int nb = eoff[e] + c * BN;
    const int cnt = min(BN, eoff[e + 1] - nb);
    const int m0 = mt * 64;
    const int wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;

    f32x16 acc[2][2];
    zero_acc(acc);
    auto wsrc = [&](int lrow, WView &v, int &row) {
        const int m = m0 + (lrow & 63);
        v = lrow < 64 ? gate : up;
        row = m < mid ? e * mid + m : -1;
    };
    auto xrow = [&](int r) -> const _Float16 * {
        return r < cnt ? xg + (size_t)(nb + r) * K : nullptr;
    };
    auto arow = [&](int i) { return 64 * i + 32 * wm; };
    if (cnt <= 32) k_loop<F, 1>(wsrc, xrow, arow, K, wn, lds, acc);
    else k_loop<F, 2>(wsrc, xrow, arow, K, wn, lds, acc);

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = acc_col(wn, j);
        if (r >= cnt) continue;
        float *hr = H + (size_t)(nb + r) * mid;
        const float sc = xscale[nb + r];
#pragma unroll
        for (int e4 = 0; e4 < 16; ++e4) {
            const int m = m0 + 32 * wm + acc_row_in_block(e4);
            if (m < mid) hr[m] = silu_mul(acc[0][j][e4] * sc, acc[1][j][e4] * sc);
        }
    }
}

// Gate and up of a dense FFN at batch N (DenseFfn::forward, src/model.rs:
// 679-683): the tile pairs gate rows m0..m0+63 with the same rows of up, as
// moe_gate_up_kernel does, and writes H[n][m] = silu(g) * u in f32 (NW waves,
// 32 NW tokens per tile, as gemm_f16_kernel).
template <int F, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void gemm_gate_up_kernel(
    WView gate, WView up, int mid, int K, const _Float16 *__restrict__ xh,
    const float *__restrict__ rscale, int N, float *__restrict__ H, int mtiles, int ntiles)
{
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<NW>()];
    const int T = xcd_tile(mtiles * ntiles);
    if (T >= mtiles * ntiles) return;
    const int m0 = (T / ntiles) * 64, n0 = (T % ntiles) * (32 * NW);
    const int wave = threadIdx.x >> 6, wm = wave / (NW / 2), wn = wave % (NW / 2);

    f32x16 acc[2][2];
    zero_acc(acc);
    auto wsrc = [&](int lrow, WView &v, int &row) {
        const int m = m0 + (lrow & 63);
        v = lrow < 64 ? gate : up;
        row = m < mid ? m : -1;
    };
    auto xrow = [&](int r) -> const _Float16 * {
        return n0 + r < N ? xh + (size_t)(n0 + r) * K : nullptr;
    };
    auto arow = [&](int i) { return 64 * i + 32 * wm; };
    k_loop<F, 2, NW>(wsrc, xrow, arow, K, wn, lds, acc);

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + acc_col(wn, j);
        if (n >= N) continue;
        float *hr = H + (size_t)n * mid;
        const float sc = rscale[n];
#pragma unroll
        for (int e4 = 0; e4 < 16; ++e4) {
            const int m = m0 + 32 * wm + acc_row_in_block(e4);
            if (m < mid) hr[m] = silu_mul(acc[0][j][e4] * sc, acc[1][j][e4] * sc);
        }
    }
}

// Down of one expert chunk: outp[q][m] = down_e[m] . H[q] (H in f16 with its
// row scale).
template <int F>
__global__ __launch_bounds__(256, 2) void moe_down_kernel(
    WView down, int hidden, int K, const int *__restrict__ eoff, const int *__restrict__ tiles,
    const int *__restrict__ ntiles, const _Float16 *__restrict__ H,
    const float *__restrict__ hscale, float *__restrict__ outp, int mtiles, int max_tiles)
{
    __shared__ __attribute__((aligned(16))) _Float16 lds[4 * TILE_HALVES];
    const int T = xcd_tile(mtiles * max_tiles);
    if (T >= mtiles * max_tiles) return;
    const int ti = T / mtiles, mt = T % mtiles;
    if (ti >= *ntiles) return;
    const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
    const int nb = eoff[e] + c * BN;
    const int cnt = min(BN, eoff[e + 1] - nb);
    const int m0 = mt * BM;
    const int wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;

    f32x16 acc[2][2];
    zero_acc(acc);
    auto wsrc = [&](int lrow, WView &v, int &row) {
        v = down;
        row = m0 + lrow < hidden ? e * hidden + m0 + lrow : -1;
    };
    auto xrow = [&](int r) -> const _Float16 * {
        return r < cnt ? H + (size_t)(nb + r) * K : nullptr;
    };
    auto arow = [&](int i) { return wm * 64 + 32 * i; };
    if (cnt <= 32) k_loop<F, 1>(wsrc, xrow, arow, K, wn, lds, acc);
    else k_loop<F, 2>(wsrc, xrow, arow, K, wn, lds, acc);

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = acc_col(wn, j);
            if (r >= cnt) continue;
            float *orow = outp + (size_t)(nb + r) * hidden;
            const float sc = hscale[nb + r];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int m = m0 + arow(i) + acc_row_in_block(4 * g);
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4)
                    if (m + e4 < hidden) orow[m + e4] = acc[i][j][4 * g + e4] * sc;
            }
        }
}

// out[t][i] += w * value[i] per routed pair of token t, experts ascending
// (src/model.rs:715-722), as separate rounded products and sums.
__global__ __launch_bounds__(256) void moe_combine_kernel(float *__restrict__ out, int hidden,
                                                          const int *__restrict__ toff,
                                                          const int *__restrict__ tlist,
                                                          const int *__restrict__ order,
                                                          const float *__restrict__ pw,
                                                          const float *__restrict__ outp)
{
    const int t = blockIdx.y;
    const int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= hidden) return;
    float acc = out[(size_t)t * hidden + col];
    for (int i = toff[t]; i < toff[t + 1]; ++i) {
        const int q = tlist[i];
        acc = acc + pw[order[q]] * outp[(size_t)q * hidden + col];
    }
    out[(size_t)t * hidden + col] = acc;
}

} // namespace

int launch_to_f16(const float *x, int rows, int K, _Float16 *xh, float *rscale, void *stream,
                  bool frag)
{
    if (!frag) return launch_norm_to_f16(x, rows, K, nullptr, 0.f, xh, rscale, stream);
    if (rows <= 0) return 0;
    if (K % 16) return (int)hipErrorInvalidValue;
    launch_rows_to_f16(rows, K, (hipStream_t)stream, x, nullptr, nullptr, nullptr, nullptr, 0.f,
                       xh, rscale, true);
    return (int)hipGetLastError();
}

int launch_norm_to_f16(const float *x, int rows, int K, const float *norm, float eps,
                       _Float16 *xh, float *rscale, void *stream)
{
    if (rows <= 0) return 0;
    if (K % 4) return (int)hipErrorInvalidValue;
    launch_rows_to_f16(rows, K, (hipStream_t)stream, x, nullptr, nullptr, nullptr, norm, eps, xh,
                       rscale, false);
    return (int)hipGetLastError();
}

// Waves per dense GEMM workgroup: 8 (256-token tiles, each dequantized
// weight slice feeding twice the MFMAs) when the batch exceeds one 128-token
// tile and the 8-wave grid (`tiles` row tiles x K slices, times the 256-token
// tiles) still gives at least 3/4 of the 256 CUs a workgroup; else 4 (two
// workgroups per CU). Measured: Q4_K [14336 x 4096] x 512 tokens 120 -> 100
// us, while grids of 64-96 workgroups ran 6-13 % slower with 8 waves. Both
// forms give every element the same result, so the choice is free.
int gemm_waves(int batch, int tiles)
{
    return batch > BN && (size_t)tiles * ((batch + 255) / 256) >= 192 ? 8 : 4;
}

int launch_gate_up_f16(int fmt, WView gate, WView up, int cols, const _Float16 *xh,
                       const float *rscale, int batch, float *h, void *stream)
{
    if (cols % BK) return (int)hipErrorInvalidValue;
    const int mid = gate.rows;
    const int mtiles = (mid + 63) / 64;
    const int nw = gemm_waves(batch, mtiles), bn = 32 * nw;
    const int ntiles = (batch + bn - 1) / bn;
    const int per = (mtiles * ntiles + 7) / 8;
    dim3 grid(8 * per), block(64 * nw);
    hipStream_t st = (hipStream_t)stream;
#define HYQ_GU(F)                                                                              \
    case F:                                                                                    \
        if (nw == 8)                                                                           \
            hipLaunchKernelGGL((gemm_gate_up_kernel<F, 8>), grid, block, 0, st, gate, up, mid,  \
                               cols, xh, rscale, batch, h, mtiles, ntiles);                    \
        else                                                                                   \
            hipLaunchKernelGGL((gemm_gate_up_kernel<F, 4>), grid, block, 0, st, gate, up, mid,  \
                               cols, xh, rscale, batch, h, mtiles, ntiles);                    \
        break;
    switch (fmt) {
        HYQ_GU(Q4_K)
        HYQ_GU(Q6_K)
        HYQ_GU(Q8_0)
        HYQ_GU(Q2_0C)
        HYQ_GU(STQ1_0)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_GU
    return (int)hipGetLastError();
}

// K slices for a one-weight GEMM of few row tiles, whose tiles would leave
// CUs idle: up to 4 slices for at most 32 row tiles, 2 for at most 64 - the
// largest count that cuts K into whole numbers of the format's blocks (and
// 64-column steps) of at least 1024 columns. It depends on the weight's
// shape only, so a token row's result does not depend on how many rows
// share the launch.
int gemm_kslices(int fmt, int M, int K)
{
    const int unit = std::max(BK, block_len(fmt));
    const int mtiles = (M + BM - 1) / BM;
    const int kmax = mtiles <= 32 ? 4 : mtiles <= 64 ? 2 : 1;
    if (K % unit || M % 4) return 1;
    for (int k = kmax; k > 1; --k)
        if ((K / unit) % k == 0 && K / k >= 1024) return k;
    return 1;
}

size_t gemm_split_floats(int fmt, int M, int N, int K)
{
    const int k = gemm_kslices(fmt, M, K);
    return k > 1 ? (size_t)k * N * M : 0;
}

// K slices of Weight::matmul's batched product (hyq_matmul_d). Above one
// token tile (BN rows) it is gemm_kslices, a rule on the weight's shape only.
// A batch of at most BN token rows is one token tile, so the grid is the row
// tiles times the slices: the largest count up to 8 that keeps that grid
// within the 256 CUs and cuts K into whole blocks (and 64-column steps) of at
// least 256 columns, never fewer than gemm_kslices gives. A [2048 x 2048]
// weight at 64 tokens (the MoE shared projection) runs as 8 slices on 128
// workgroups instead of 2 slices on 32. Token rows of batches on the same
// side of BN get identical results.
int matmul_kslices(int fmt, int M, int K, int batch)
{
    const int base = gemm_kslices(fmt, M, K);
    if (batch > BN || K % BK || M % 4) return base;
    const int unit = std::max(BK, block_len(fmt));
    if (K % unit) return base;
    const int mtiles = (M + BM - 1) / BM;
    for (int k = 8; k > base; --k)
        if (mtiles * k <= 256 && (K / unit) % k == 0 && K / k >= 256) return k;
    return base;
}

bool gemm_frag_operand(int fmt, int rows, int cols, int batch, int kslices)
{
    (void)fmt;
    (void)cols;
    const int mtiles = (rows + BM - 1) / BM;
    return gemm_waves(batch, mtiles * (kslices > 1 ? kslices : 1)) == 8;
}

int launch_gemm_f16(int fmt, WView w, int cols, const _Float16 *xh, const float *rscale,
                    int batch, float *y, const float *residual, void *stream, float *part,
                    size_t part_floats, int kslices, bool xfrag)
{
    GemmSegs g{};
    g.nseg = 1;
    g.s[0].w = w;
    g.s[0].y = y;
    g.s[0].residual = residual;
    g.s[0].rows = w.rows;
    const int ks = kslices > 0 ? kslices : gemm_kslices(fmt, w.rows, cols);
    if (ks > 1 && part && part_floats >= (size_t)ks * batch * w.rows) {
        int rc = launch_gemm_f16_segs(fmt, g, cols, xh, rscale, batch, stream, ks, part, xfrag);
        if (rc) return rc;
        const size_t count4 = (size_t)batch * w.rows / 4;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((count4 + 255) / 256)), dim3(256),
                           0, (hipStream_t)stream, reinterpret_cast<const float4 *>(part), ks,
                           count4, reinterpret_cast<const float4 *>(residual),
                           reinterpret_cast<float4 *>(y));
        return (int)hipGetLastError();
    }
    return launch_gemm_f16_segs(fmt, g, cols, xh, rscale, batch, stream, 1, nullptr, xfrag);
}

int launch_gemm_f16_segs(int fmt, GemmSegs g, int cols, const _Float16 *xh, const float *rscale,
                         int batch, void *stream, int kslices, float *part, bool xfrag)
{
    if (cols % BK || g.nseg < 1 || g.nseg > 3) return (int)hipErrorInvalidValue;
    if (kslices < 1 || (kslices > 1 && (g.nseg != 1 || !part || cols % kslices)))
        return (int)hipErrorInvalidValue;
    int mtiles = 0;
    for (int i = 0; i < g.nseg; ++i) {
        if (i + 1 < g.nseg && g.s[i].rows % BM) return (int)hipErrorInvalidValue;
        g.s[i].tiles = (g.s[i].rows + BM - 1) / BM;
        mtiles += g.s[i].tiles;
    }
    const int nw = gemm_waves(batch, mtiles * kslices), bn = 32 * nw;
    // fragment-order activations: only the 256-token tiles of one weight
    if (xfrag && (nw != 8 || g.nseg != 1 || cols % 16)) return (int)hipErrorInvalidValue;
    const int ntiles = (batch + bn - 1) / bn;
    // The fragment-order kernel takes 96-row tiles where they need fewer
    // rounds of workgroups over the 256 CUs per row of a tile (rounds x tile
    // rows): a [6144 x 4096] product in two K slices at 512 tokens runs as
    // 64 x 2 x 2 = 256 workgroups of 96 rows instead of 192 of 128.
    bool rows96 = false;
    if (xfrag) {
        const int m96 = (g.s[0].rows + 95) / 96;
        auto rounds = [&](int mt) { return (mt * ntiles * kslices + 255) / 256; };
        if (rounds(m96) * 96 < rounds(mtiles) * BM) {
            rows96 = true;
            mtiles = g.s[0].tiles = m96;
        }
    }
    const int per = (mtiles * ntiles + 7) / 8;
    dim3 grid(8 * per, kslices), block(64 * nw);
    hipStream_t st = (hipStream_t)stream;
#define HYQ_GEMM(F)                                                                            \
    case F:                                                                                    \
        if (xfrag && rows96)                                                                   \
            hipLaunchKernelGGL((gemm_f16_pcx_kernel<F, 3>), grid, block, 0, st, g, cols, xh,    \
                               rscale, batch, mtiles, ntiles, kslices, part);                  \
        else if (xfrag)                                                                        \
            hipLaunchKernelGGL((gemm_f16_pcx_kernel<F, 4>), grid, block, 0, st, g, cols, xh,    \
                               rscale, batch, mtiles, ntiles, kslices, part);                  \
        else if (nw == 8)                                                                      \
            hipLaunchKernelGGL((gemm_f16_pc_kernel<F>), grid, block, 0, st, g, cols, xh,        \
                               rscale, batch, mtiles, ntiles, kslices, part);                  \
        else                                                                                   \
            hipLaunchKernelGGL((gemm_f16_kernel<F, 4>), grid, block, 0, st, g, cols, xh, rscale, \
                               batch, mtiles, ntiles, kslices, part);                          \
        break;
    switch (fmt) {
        HYQ_GEMM(Q4_K)
        HYQ_GEMM(Q6_K)
        HYQ_GEMM(Q8_0)
        HYQ_GEMM(Q2_0C)
        HYQ_GEMM(STQ1_0)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_GEMM
    return (int)hipGetLastError();
}

MoeLayout moe_layout(int tokens, int npairs, int experts, int hidden, int mid)
{
    MoeLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    const int few = moe_q4k_chunk();
    L.max_tiles = npairs / BN + (experts < npairs ? experts : npairs) + 1;
    L.max_tiles_few = npairs / few + (experts < npairs ? experts : npairs) + 1;
    L.eoff = take(4 * ((size_t)experts + 1));
    L.order = take(4 * (size_t)npairs);
    L.rank = take(4 * ((size_t)npairs + experts + tokens + 1));
    L.toff = take(4 * ((size_t)tokens + 1));
    L.tlist = take(4 * (size_t)npairs);
    L.tiles = take(8 * (size_t)L.max_tiles_few);
    L.ntiles = take(4);
    L.xg = take(2 * (size_t)npairs * hidden);
    L.xscale = take(4 * (size_t)npairs);
    L.h32 = take(4 * (size_t)npairs * mid);
    L.h = take(2 * (size_t)npairs * mid);
    L.hscale = take(4 * (size_t)npairs);
    L.outp = take(4 * (size_t)npairs * hidden);
    const size_t cols = (size_t)L.max_tiles_few * few; // chunk columns of the Q4_K kernels
    L.xop = take(2 * (size_t)tokens * hidden);
    L.xhs = take((size_t)tokens * hidden / 8);
    L.xsc = take(4 * (size_t)tokens);
    L.hop = take(2 * (size_t)npairs * mid);
    L.hhs = take((size_t)npairs * mid / 8);
    L.hsc = take(4 * (size_t)npairs);
    L.cpos = take(4 * cols);
    L.ctok = take(4 * cols);
    L.gpart = take(4 * 2 * (size_t)npairs * mid);
    L.upart = take(4 * 2 * (size_t)npairs * mid);
    // f16 fragments of the token rows for a fused Q8_0 shared projection
    L.xf = take(tokens <= FEW_Q80_MAX_TOKENS ? few_q80_operand_bytes(hidden, tokens) : 0);
    L.bytes = off;
    return L;
}

int moe_plan_max() { return PLAN_MAX; }

namespace {

// Register-operand Q4_K kernels while the pairs average at most one
// 16-token chunk per expert (weight-bound); the LDS-tiled GEMM otherwise.
bool few_path(int fmt_gu, int fmt_down, const WView &gate, const WView &up, const WView &down,
              int hidden, int mid, int npairs, int experts)
{
    return fmt_gu == Q4_K && fmt_down == Q4_K && moe_q4k_fits(hidden, mid) && gate.p2 && up.p2 &&
           down.p2 && npairs <= moe_q4k_chunk() * experts;
}

} // namespace

bool moe_fuses_shared(int fmt_gu, int fmt_down, WView gate, WView up, WView down, int hidden,
                      int mid, int tokens, int npairs, int experts)
{
    return npairs > 0 && tokens >= 2 && few_path(fmt_gu, fmt_down, gate, up, down, hidden, mid, npairs, experts) &&
           plan_fast_fits(npairs, tokens, experts) && few_q80_fits(hidden, hidden, tokens);
}

int launch_moe(int fmt_gu, int fmt_down, WView gate, WView up, WView down, int hidden, int mid,
               const float *x, int tokens, const int *ptok, const int *pexp, const float *pw,
               int npairs, int experts, uint8_t *scratch, const MoeLayout &L, float *out,
               void *stream, const WView *shared)
{
    if (hidden % BK || mid % BK || hidden % 4 || tokens > PLAN_MAX || experts > PLAN_MAX)
        return (int)hipErrorInvalidValue;
    if (shared && (shared->rows != hidden ||
                   !moe_fuses_shared(fmt_gu, fmt_down, gate, up, down, hidden, mid, tokens,
                                     npairs, experts)))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    int *eoff = (int *)(scratch + L.eoff), *order = (int *)(scratch + L.order);
    int *rank = (int *)(scratch + L.rank), *toff = (int *)(scratch + L.toff);
    int *tlist = (int *)(scratch + L.tlist), *tiles = (int *)(scratch + L.tiles);
    int *ntiles = (int *)(scratch + L.ntiles);
    _Float16 *xg = (_Float16 *)(scratch + L.xg), *H = (_Float16 *)(scratch + L.h);
    float *xscale = (float *)(scratch + L.xscale), *hscale = (float *)(scratch + L.hscale);
    float *h32 = (float *)(scratch + L.h32), *outp = (float *)(scratch + L.outp);
    if (npairs == 0) return 0;

    const bool few = few_path(fmt_gu, fmt_down, gate, up, down, hidden, mid, npairs, experts);
    // (the few-token kernels take the token rows' largest magnitudes from the
    // plan's launch)
    const bool fast = plan_fast_fits(npairs, tokens, experts);
    uint4 *xop = (uint4 *)(scratch + L.xop);
    uint2 *xhs = (uint2 *)(scratch + L.xhs);
    float *xsc = (float *)(scratch + L.xsc);
    int *cpos = (int *)(scratch + L.cpos), *ctok = (int *)(scratch + L.ctok);
    _Float16 *xf = shared ? (_Float16 *)(scratch + L.xf) : nullptr;
    if (fast)
        hipLaunchKernelGGL(moe_plan_fast_kernel,
                           dim3(few ? 2 + (xf ? 2 : 1) * ((tokens + 15) / 16) : 2),
                           dim3(1024), 0, st, ptok, pexp, npairs, tokens, experts, eoff, order,
                           toff, tlist, tiles, ntiles, few ? moe_q4k_chunk() : BN,
                           few ? x : nullptr, hidden, xop, xhs, xsc, few ? cpos : nullptr,
                           ctok, xf);
    else if (npairs <= PLAN_SMALL && tokens <= PLAN_SMALL && experts <= PLAN_SMALL)
        hipLaunchKernelGGL(moe_plan_small_kernel, dim3(1), dim3(256), 0, st, ptok, pexp, npairs,
                           tokens, experts, eoff, order, toff, tlist, tiles, ntiles,
                           few ? moe_q4k_chunk() : BN);
    else
        hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(256), 0, st, ptok, pexp, npairs, tokens,
                           experts, eoff, order, rank, toff, tlist, tiles, ntiles,
                           few ? moe_q4k_chunk() : BN);
    if (few) {
        int rc = launch_moe_q4k(gate, up, down, hidden, mid, x, tokens, ptok, eoff, eoff + experts,
                                order, tiles, ntiles, L.max_tiles_few, npairs, fast, xop, xhs,
                                xsc, cpos, ctok, (float *)(scratch + L.gpart),
                                (float *)(scratch + L.upart), (uint4 *)(scratch + L.hop),
                                (uint2 *)(scratch + L.hhs), (float *)(scratch + L.hsc), outp,
                                stream, shared, xf, out);
        if (rc) return rc;
        hipLaunchKernelGGL(moe_combine_kernel, dim3((hidden + 255) / 256, tokens), dim3(256), 0,
                           st, out, hidden, toff, tlist, order, pw, outp);
        return (int)hipGetLastError();
    }
    launch_rows_to_f16(npairs, hidden, st, x, order, ptok, eoff + experts, nullptr, 0.f, xg,
                       xscale, false);
    {
        const int mtiles = (mid + 63) / 64;
        const int per = (mtiles * L.max_tiles + 7) / 8;
        dim3 grid(8 * per), block(256);
#define HYQ_MOE_GU(F)                                                                          \
    case F:                                                                                    \
        hipLaunchKernelGGL(moe_gate_up_kernel<F>, grid, block, 0, st, gate, up, mid, hidden,   \
                           eoff, tiles, ntiles, xg, xscale, h32, mtiles, L.max_tiles);         \
        break;
        switch (fmt_gu) {
            HYQ_MOE_GU(Q4_K)
            HYQ_MOE_GU(Q6_K)
            HYQ_MOE_GU(Q8_0)
            HYQ_MOE_GU(Q2_0C)
            HYQ_MOE_GU(STQ1_0)
        default: return (int)hipErrorInvalidValue;
        }
#undef HYQ_MOE_GU
    }
    launch_rows_to_f16(npairs, mid, st, h32, nullptr, nullptr, eoff + experts, nullptr, 0.f, H,
                       hscale, false);
    {
        const int mtiles = (hidden + BM - 1) / BM;
        const int per = (mtiles * L.max_tiles + 7) / 8;
        dim3 grid(8 * per), block(256);
#define HYQ_MOE_DN(F)                                                                          \
    case F:                                                                                    \
        hipLaunchKernelGGL(moe_down_kernel<F>, grid, block, 0, st, down, hidden, mid, eoff,     \
                           tiles, ntiles, H, hscale, outp, mtiles, L.max_tiles);               \
        break;
        switch (fmt_down) {
            HYQ_MOE_DN(Q4_K)
            HYQ_MOE_DN(Q6_K)
            HYQ_MOE_DN(Q8_0)
            HYQ_MOE_DN(Q2_0C)
            HYQ_MOE_DN(STQ1_0)
        default: return (int)hipErrorInvalidValue;
        }
#undef HYQ_MOE_DN
    }
    hipLaunchKernelGGL(moe_combine_kernel, dim3((hidden + 255) / 256, tokens), dim3(256), 0, st,
                       out, hidden, toff, tlist, order, pw, outp);
    return (int)hipGetLastError();
}

} // namespace hyq
