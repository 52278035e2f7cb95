// Q8 activation quantizer kernel (Q8::quantize_into, src/quant.rs:904-922)
// for gfx950; the arithmetic lives in hyq_q8.hpp.
#include <hip/hip_runtime.h>

#include "hyq_q8.hpp"

namespace hyq {

namespace {

__global__ __launch_bounds__(256) void quantize_q8_kernel(const float *__restrict__ x, int n,
                                                          int8_t *__restrict__ q,
                                                          float *__restrict__ s,
                                                          int32_t *__restrict__ sum16,
                                                          int32_t *__restrict__ sum32,
                                                          int32_t *__restrict__ sum256)
{
    const int g = blockIdx.x;
    const int len = min(256, n - g * 256);
    const int t = threadIdx.x;
    const float v = t < len ? x[g * 256 + t] : 0.f;
    q8_quantize_group(v, g, len, q, s, sum16, sum32, sum256);
}

} // namespace

int launch_quantize_q8(const float *x, int n, int8_t *q, float *s, int32_t *sum16,
                       int32_t *sum32, int32_t *sum256, void *stream)
{
    if (n <= 0) return 0;
    dim3 grid((n + 255) / 256), block(256);
    hipLaunchKernelGGL(quantize_q8_kernel, grid, block, 0, (hipStream_t)stream, x, n, q, s,
                       sum16, sum32, sum256);
    return (int)hipGetLastError();
}

} // namespace hyq
