// A read-only HBM stream: the practical ceiling that the HBM-bound GEMVs are
// compared with (measurement aid; no counterpart in the reference). Every
// thread reads 16-byte words in a grid-stride loop with four loads in
// flight, the workgroup reduces what it read and one word per workgroup is
// written, so the traffic is the buffer read once.
#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

__global__ __launch_bounds__(256) void hbm_read_kernel(const float4 *__restrict__ p, size_t n4,
                                                       float *__restrict__ sink)
{
    __shared__ float part[4];
    const size_t stride = (size_t)gridDim.x * 256;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        const float4 u = p[i], v = p[i + stride], w = p[i + 2 * stride], z = p[i + 3 * stride];
        a0 += (u.x + u.y) + (u.z + u.w);
        a1 += (v.x + v.y) + (v.z + v.w);
        a2 += (w.x + w.y) + (w.z + w.w);
        a3 += (z.x + z.y) + (z.z + z.w);
    }
    for (; i < n4; i += stride) {
        const float4 u = p[i];
        a0 += (u.x + u.y) + (u.z + u.w);
    }
    const float s = wave::sum64((a0 + a1) + (a2 + a3));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

} // namespace

int launch_hbm_read(const void *buf, size_t bytes, int workgroups, float *sink, void *stream)
{
    if (workgroups <= 0 || bytes < 16) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(hbm_read_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const float4 *)buf, bytes / 16, sink);
    return (int)hipGetLastError();
}

} // namespace hyq
