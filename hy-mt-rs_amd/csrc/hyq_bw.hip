// Measurement aids (no counterpart in the reference): a read-only HBM stream,
// the practical ceiling that the HBM-bound GEMVs are compared with (every
// thread reads 16-byte words in a grid-stride loop with eight loads in
// flight, the workgroup reduces what it read and one word per workgroup is
// written, so the traffic is the buffer read once), and an MFMA stream, the
// practical ceiling of the f16 matrix cores under sustained load that the
// batched products are compared with.
#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

// Non-temporal loads: a read-only stream of whole 1 KiB wave rows measures
// ~6.9 TB/s with them and ~6.0 TB/s without on MI355X.
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void hbm_read_kernel(const f32x4 *__restrict__ p, size_t n4,
                                                       float *__restrict__ sink)
{
    constexpr int U = 8; // loads in flight per thread
    __shared__ float part[4];
    const size_t stride = (size_t)gridDim.x * 256;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    float acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = 0.f;
    for (; i + (U - 1) * stride < n4; i += U * stride) {
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    for (; i < n4; i += stride) {
        const f32x4 v = p[i];
        acc[0] += (v.x + v.y) + (v.z + v.w);
    }
    float a = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) a += acc[u];
    const float s = wave::sum64(a);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// Each wave issues `iters` rounds of four independent
// v_mfma_f32_32x32x16_f16 (32768 flop each) on register operands, then
// writes one sum per thread so that nothing is eliminated.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_stream_kernel(int iters, float *__restrict__ sink)
{
    const int t = threadIdx.x;
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (float)(t + i));
        b[i] = (_Float16)(0.002f * (float)(t - i));
    }
    f32x16 acc[4] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[j][e];
    sink[(size_t)blockIdx.x * 256 + t] = s;
}

} // namespace

int launch_mfma_stream(int workgroups, int iters, float *sink, void *stream)
{
    if (workgroups <= 0 || iters <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(mfma_stream_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       iters, sink);
    return (int)hipGetLastError();
}

int launch_hbm_read(const void *buf, size_t bytes, int workgroups, float *sink, void *stream)
{
    if (workgroups <= 0 || bytes < 16) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(hbm_read_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const f32x4 *)buf, bytes / 16, sink);
    return (int)hipGetLastError();
}

} // namespace hyq
