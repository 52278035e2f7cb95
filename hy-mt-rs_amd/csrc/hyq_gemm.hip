// Batched matmul (Weight::matmul batch >= 2, src/quant.rs:272-344) for
// gfx950: Y[batch, rows] = X[batch, cols] W^T with weight tiles dequantized
// to f16 in LDS and v_mfma_f32_32x32x16_f16 accumulating in f32 (the tile
// engine is in hyq_tile.hpp).
//
// Tile order is XCD-aware: workgroups are dispatched round-robin over the 8
// XCDs, so workgroup b runs on XCD b % 8; tile index (b % 8) * per + b / 8
// gives each XCD a contiguous range of tiles, and the BN-token tiles of one
// weight row block land on the same XCD and share its L2.
#include <hip/hip_runtime.h>

#include "hyq_tile.hpp"

namespace hyq {

namespace {

using namespace tile;

template <int F>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(WView w, int M, int K,
                                                          const float *__restrict__ x, int N,
                                                          float *__restrict__ y, int mtiles,
                                                          int ntiles)
{
    __shared__ __attribute__((aligned(16))) _Float16 Ws[BM * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Xs[BN * LDK];
    const int total = mtiles * ntiles;
    const int per = (total + 7) / 8;
    const int T = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (T >= total) return;
    const int m0 = (T / ntiles) * BM, n0 = (T % ntiles) * BN;
    const int t = threadIdx.x, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int drow = t >> 1, dh = t & 1;
    const bool row_ok = m0 + drow < M;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    auto xrow = [&](int r) -> const float * {
        const int n = n0 + r;
        return n < N ? x + (size_t)n * K : nullptr;
    };
    for (int k0 = 0; k0 < K; k0 += BK) {
        float4 xv[8];
        load_x(xrow, k0, xv);
        if (row_ok) Deq<F>::run(w, m0 + drow, k0, dh, Ws + drow * LDK);
        else zero_half(Ws + drow * LDK, dh);
        store_x(Xs, xv);
        __syncthreads();
        mma_step(Ws, Xs, wm, wn, acc);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + acc_col(wn, j);
            if (n >= N) continue;
            float *yr = y + (size_t)n * M;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int m = m0 + acc_row(wm, i, 4 * g);
                if (m + 3 < M && (M & 3) == 0) {
                    *reinterpret_cast<float4 *>(yr + m) =
                        make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                    acc[i][j][4 * g + 3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e < M) yr[m + e] = acc[i][j][4 * g + e];
                }
            }
        }
}

} // namespace

int launch_gemm_f16(int fmt, WView w, int cols, const float *x, int batch, float *y,
                    void *stream)
{
    if (cols % BK) return (int)hipErrorInvalidValue;
    const int M = w.rows;
    const int mtiles = (M + BM - 1) / BM, ntiles = (batch + BN - 1) / BN;
    const int total = mtiles * ntiles;
    const int per = (total + 7) / 8;
    dim3 grid(8 * per), block(256);
    hipStream_t st = (hipStream_t)stream;
#define HYQ_GEMM(F)                                                                            \
    case F:                                                                                    \
        hipLaunchKernelGGL(gemm_f16_kernel<F>, grid, block, 0, st, w, M, cols, x, batch, y,     \
                           mtiles, ntiles);                                                    \
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

} // namespace hyq
