// Few-token products of Q8_0 weights: Weight::matmul at batch 2..128
// (src/quant.rs:272-344) on the f16-MFMA path, as one launch with no LDS
// stage and no K split across workgroups. There the product is bound by
// streaming the weight once, not by the matrix cores, so the weights go from
// HBM straight into MFMA operands in registers (the tile: hyq_few_q80.hpp).
#include <hip/hip_runtime.h>

#include "hyq_f16rows.hpp"
#include "hyq_few_q80.hpp"
#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

#pragma clang fp contract(off)

namespace hyq {

namespace {

// One workgroup per token row n of the chunks (n < nrows = chunks * 16;
// workgroup b takes row frag_row(b), so a line's 8 tokens share an XCD): its f16
// values (x[n] scaled by 2^-e, e from the row's largest magnitude as
// launch_to_f16 forms it; zeros for n >= N) into the fragment layout, and
// rscale[n] = 2^e.
__global__ __launch_bounds__(256) void few_rows_kernel(const float *__restrict__ x, int K, int N,
                                                       int nrows, _Float16 *__restrict__ xf,
                                                       float *__restrict__ rscale)
{
    __shared__ float wred[4];
    const int n = frag_row((int)blockIdx.x), t = (int)threadIdx.x, nb = K / 32;
    if (n >= nrows) return;
    const bool live = n < N;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)(live ? n : 0) * K);
    float m = 0.f;
    if (live)
        for (int i = t; i < K / 4; i += 256) {
            const float4 v = x4[i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            if (v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w) m = INFINITY;
        }
    m = wave::max64(m);
    if ((t & 63) == 0) wred[t >> 6] = m;
    __syncthreads();
    const int e = f16_row_exponent(fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3])));
    const float inv = ldexpf(1.0f, -e);
    if (t == 0 && live) rscale[n] = ldexpf(1.0f, e);
    for (int p = t; p < 4 * nb; p += 256) few::fragment_piece(live ? x4 : nullptr, inv, n, p, K, xf);
}

__global__ __launch_bounds__(64 * few::WAVES) void few_q80_kernel(WView w, int K,
                                                                  const _Float16 *__restrict__ xh,
                                                                  const float *__restrict__ rscale,
                                                                  int N, float *__restrict__ y,
                                                                  int cgroups)
{
    __shared__ few::Red red;
    few::q80_tile((int)blockIdx.x, w, K, xh, rscale, N, y, cgroups, red);
}

} // namespace

bool few_q80_fits(int rows, int cols, int batch)
{
    return batch >= 1 && batch <= FEW_Q80_MAX_TOKENS && cols % 256 == 0 && rows >= 1;
}

size_t few_q80_operand_bytes(int cols, int batch)
{
    return (size_t)((batch + few::CHUNK - 1) / few::CHUNK) * few::CHUNK * cols * 2;
}

int launch_few_q80(WView w, int cols, const float *x, _Float16 *xh, float *rscale, int batch,
                   float *y, void *stream)
{
    if (!few_q80_fits(w.rows, cols, batch)) return (int)hipErrorInvalidValue;
    const int nrows = (batch + few::CHUNK - 1) / few::CHUNK * few::CHUNK;
    // rows n < nrows, on workgroups frag_row^-1(n): a line's 8 tokens on one XCD
    hipLaunchKernelGGL(few_rows_kernel, dim3((nrows + 63) / 64 * 64), dim3(256), 0,
                       (hipStream_t)stream, x, cols, batch, nrows, xh, rscale);
    int cgroups = 0;
    const int tiles = few::q80_tiles(w.rows, batch, &cgroups);
    hipLaunchKernelGGL(few_q80_kernel, dim3(tiles), dim3(64 * few::WAVES), 0,
                       (hipStream_t)stream, w, cols, xh, rscale, batch, y, cgroups);
    return (int)hipGetLastError();
}

} // namespace hyq
