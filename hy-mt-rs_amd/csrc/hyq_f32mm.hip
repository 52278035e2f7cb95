// Weight::matmul by decoded rows (src/quant.rs:225-237 at batch 1,
// :272-343 at batch >= 2): every row decoded to f32 exactly as the decoder
// does it (an f16 widens without rounding; a Q8_0 value is d * q) and dotted
// with the f32 activations in f32. This serves the F32 and F16 weights (the
// HyV3 router, src/model.rs:223-226, is required F32, and a GGUF file may
// carry either in place of a quantized tensor) and Q8_0 matrices whose width
// is a whole number of 32-value blocks but not of the int8 GEMV's 256-value
// groups or the GEMM's 64-column slices.
//
// Batch 1 is a GEMV, HBM-bound: one wave per row (four rows per 256-thread
// workgroup), each lane streaming 4-value slices of the row with the
// matching float4 of x, four independent fused multiply-adds, then a wave
// reduction. The gate/up form computes silu(g) * u of two rows in the same
// wave. Batch >= 2 is a register-tiled f32 GEMM (64 rows x 64 tokens per
// workgroup, K in steps of 16 through LDS, 4 x 4 outputs per thread).
#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

// Value access to one decoded row r of a weight view: elem(k) and, for k a
// multiple of 4, load4(k) (the four values k..k+3, one Q8_0 block).
template <int F> struct Raw;
template <> struct Raw<F32> {
    __device__ static float elem(const WView &w, int cols, int r, int k)
    {
        return reinterpret_cast<const float *>(w.p0)[(size_t)r * cols + k];
    }
    __device__ static float4 load4(const WView &w, int cols, int r, int k)
    {
        return *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(w.p0) +
                                                 (size_t)r * cols + k);
    }
};
template <> struct Raw<F16> {
    __device__ static float elem(const WView &w, int cols, int r, int k)
    {
        return (float)reinterpret_cast<const _Float16 *>(w.p0)[(size_t)r * cols + k];
    }
    __device__ static float4 load4(const WView &w, int cols, int r, int k)
    {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 v = *reinterpret_cast<const h4 *>(reinterpret_cast<const _Float16 *>(w.p0) +
                                                   (size_t)r * cols + k);
        return make_float4((float)v.x, (float)v.y, (float)v.z, (float)v.w);
    }
};
// Q8_0 planes: 32 int8 per block, then the blocks' f16 scales
// (decode: d * q, src/quant.rs:2413-2418)
template <> struct Raw<Q8_0> {
    __device__ static float scale(const WView &w, size_t b)
    {
        return (float)reinterpret_cast<const _Float16 *>(w.p1)[b];
    }
    __device__ static float elem(const WView &w, int cols, int r, int k)
    {
        const size_t b = (size_t)r * (cols >> 5) + (k >> 5);
        return scale(w, b) * (float)reinterpret_cast<const int8_t *>(w.p0)[b * 32 + (k & 31)];
    }
    __device__ static float4 load4(const WView &w, int cols, int r, int k)
    {
        const size_t b = (size_t)r * (cols >> 5) + (k >> 5);
        const float d = scale(w, b);
        const uint32_t q = *reinterpret_cast<const uint32_t *>(w.p0 + b * 32 + (k & 31));
        return make_float4(d * (float)(int8_t)(q & 0xff), d * (float)(int8_t)((q >> 8) & 0xff),
                           d * (float)(int8_t)((q >> 16) & 0xff), d * (float)(int8_t)(q >> 24));
    }
};

// The dot of weight row r with x over a wave: lane l takes the 4-value
// slices l, l + 64, ... (VEC: cols % 4 == 0 and x 16-byte aligned), or the
// single values l, l + 64, ... otherwise.
template <int F, bool VEC>
__device__ __forceinline__ float row_dot(const WView &w, int r, const float *x, int cols,
                                         int lane)
{
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if constexpr (VEC) {
        const int n4 = cols >> 2;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (int c = lane; c < n4; c += 64) {
            const float4 wv = Raw<F>::load4(w, cols, r, 4 * c);
            const float4 xv = x4[c];
            a0 = fmaf(wv.x, xv.x, a0);
            a1 = fmaf(wv.y, xv.y, a1);
            a2 = fmaf(wv.z, xv.z, a2);
            a3 = fmaf(wv.w, xv.w, a3);
        }
    } else {
        for (int c = lane; c < cols; c += 64) a0 = fmaf(Raw<F>::elem(w, cols, r, c), x[c], a0);
    }
    return wave::sum64((a0 + a1) + (a2 + a3));
}

template <int F, bool VEC, bool SILU>
__global__ __launch_bounds__(256) void f32_gemv_kernel(WView w, WView u, int cols,
                                                       const float *__restrict__ x,
                                                       float *__restrict__ y)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= w.rows) return;
    const float g = row_dot<F, VEC>(w, row, x, cols, lane);
    if constexpr (SILU) {
        const float v = row_dot<F, VEC>(u, row, x, cols, lane);
        // silu(g) * u, silu(g) = g / (1 + exp(-g)) (src/model.rs:681)
        if (lane == 0) y[row] = (g / (1.0f + expf(-g))) * v;
    } else {
        if (lane == 0) y[row] = g;
    }
}

constexpr int MM_T = 64; // rows and tokens per workgroup
constexpr int MM_K = 16; // K step through LDS

// y[b][r] = sum_k w[r][k] * x[b][k] for a 64-row x 64-token tile; thread
// (tx, ty) = (t % 16, t / 16) owns rows 4ty.. and tokens 4tx..; every output
// sums its K terms in ascending order with one fused multiply-add each.
template <int F>
__global__ __launch_bounds__(256) void f32_gemm_kernel(WView w, int cols,
                                                       const float *__restrict__ x, int batch,
                                                       float *__restrict__ y)
{
    __shared__ float Ws[MM_K][MM_T + 4];
    __shared__ float Xs[MM_K][MM_T + 4];
    const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
    const int r0 = blockIdx.x * MM_T, b0 = blockIdx.y * MM_T;
    const int rows = w.rows;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    // loader roles: 4 elements each of the W and X tiles; element e = t + 256 i
    // is (row e / 16, k e % 16), so 16 consecutive threads read 16
    // consecutive columns of one row
    for (int k0 = 0; k0 < cols; k0 += MM_K) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = t + 256 * i, rr = e >> 4, kk = e & 15;
            const int k = k0 + kk;
            const int r = r0 + rr, b = b0 + rr;
            Ws[kk][rr] = r < rows && k < cols ? Raw<F>::elem(w, cols, r, k) : 0.f;
            Xs[kk][rr] = b < batch && k < cols ? x[(size_t)b * cols + k] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < MM_K; ++kk) {
            const float4 wv = *reinterpret_cast<const float4 *>(&Ws[kk][4 * ty]);
            const float4 xv = *reinterpret_cast<const float4 *>(&Xs[kk][4 * tx]);
            const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
            const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(wa[i], xa[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = b0 + 4 * tx + j;
        if (b >= batch) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 4 * ty + i;
            if (r < rows) y[(size_t)b * rows + r] = acc[i][j];
        }
    }
}

template <int F>
int gemv_f(WView w, const WView *u, int cols, const float *x, float *y, hipStream_t st)
{
    const dim3 grid((w.rows + 3) / 4), block(256);
    const bool vec = cols % 4 == 0 && (uintptr_t)x % 16 == 0;
    if (u) {
        if (vec) hipLaunchKernelGGL((f32_gemv_kernel<F, true, true>), grid, block, 0, st, w, *u, cols, x, y);
        else hipLaunchKernelGGL((f32_gemv_kernel<F, false, true>), grid, block, 0, st, w, *u, cols, x, y);
    } else {
        if (vec) hipLaunchKernelGGL((f32_gemv_kernel<F, true, false>), grid, block, 0, st, w, w, cols, x, y);
        else hipLaunchKernelGGL((f32_gemv_kernel<F, false, false>), grid, block, 0, st, w, w, cols, x, y);
    }
    return (int)hipGetLastError();
}

} // namespace

int launch_f32_gemv(int fmt, WView w, const WView *up, int cols, const float *x, float *y,
                    void *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (w.rows <= 0) return 0;
    if (fmt == F32) return gemv_f<F32>(w, up, cols, x, y, st);
    if (fmt == F16) return gemv_f<F16>(w, up, cols, x, y, st);
    if (fmt == Q8_0) return gemv_f<Q8_0>(w, up, cols, x, y, st);
    return (int)hipErrorInvalidValue;
}

int launch_f32_gemm(int fmt, WView w, int cols, const float *x, int batch, float *y,
                    void *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (w.rows <= 0 || batch <= 0) return 0;
    const dim3 grid((w.rows + MM_T - 1) / MM_T, (batch + MM_T - 1) / MM_T), block(256);
    if (fmt == F32)
        hipLaunchKernelGGL(f32_gemm_kernel<F32>, grid, block, 0, st, w, cols, x, batch, y);
    else if (fmt == F16)
        hipLaunchKernelGGL(f32_gemm_kernel<F16>, grid, block, 0, st, w, cols, x, batch, y);
    else if (fmt == Q8_0)
        hipLaunchKernelGGL(f32_gemm_kernel<Q8_0>, grid, block, 0, st, w, cols, x, batch, y);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

} // namespace hyq
