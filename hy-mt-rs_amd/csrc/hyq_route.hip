// route (src/model.rs:728-767) on the device, and the MoE output's combine
// into the hidden row (src/model.rs:699-722, :512).
//
// route: one wave per token. Lane l holds experts l, l + 64, ... (up to
// ROUTE_MAX_EXPERTS): their stable sigmoid and the selection key
// sigmoid + bias. An expert's rank is the number of experts whose key is
// larger under the IEEE total order, or equal with a smaller index - the
// reference's sort_unstable_by(total_cmp, then index), which is a total order
// with unique ranks. The `used` lowest ranks are chosen; their sigmoids are
// summed in rank order (the reference sums the sorted, truncated list), the
// sum floored at f16's smallest normal when normalising, and each weight is
// sigmoid / sum * scale. The chosen experts are written in ascending expert
// order - the order Moe::forward visits them (:700) - as slot lists
// [tokens][used] and, optionally, as (token, expert, weight) pairs.
//
// combine: hidden[t] + (shared[t] + w_0 e_0[t] + ...) in that order (the
// shared expert's output seeds the sum, each expert adds weight * value,
// then the hidden row adds the sum), with every product and sum rounded
// once, as the reference computes it. rms_rows: the f32 RMSNorm of token
// rows that the router and the MoE products of a prefill pass read.
#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

constexpr int ROUTE_MAX_EXPERTS = 1024;
constexpr int ROUTE_PER_LANE = ROUTE_MAX_EXPERTS / 64;

__device__ __forceinline__ float stable_sigmoid(float x)
{
    if (x >= 0.f) return 1.f / (1.f + expf(-x));
    const float e = expf(x);
    return e / (1.f + e);
}

// f32::total_cmp's key: the bits as a signed integer with the magnitude
// bits of negative values flipped, so that integer order is IEEE totalOrder.
__device__ __forceinline__ int total_key(float f)
{
    int i = __float_as_int(f);
    return i ^ (int)((unsigned)(i >> 31) >> 1);
}

__global__ __launch_bounds__(64) void route_kernel(const float *__restrict__ logits,
                                                   const float *__restrict__ bias, int experts,
                                                   int used, int normalize, float scale,
                                                   int *__restrict__ slot_expert,
                                                   float *__restrict__ slot_weight,
                                                   int *__restrict__ pair_token)
{
    const int t = blockIdx.x, lane = threadIdx.x;
    logits += (size_t)t * experts;
    const int per = (experts + 63) / 64;
    float sig[ROUTE_PER_LANE];
    int key[ROUTE_PER_LANE];
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; ++j) {
        const int e = lane + 64 * j;
        sig[j] = 0.f;
        key[j] = 0;
        if (j < per && e < experts) {
            sig[j] = stable_sigmoid(logits[e]);
            key[j] = total_key(sig[j] + bias[e]);
        }
    }
    // ranks: experts before e in the sorted order
    int rank[ROUTE_PER_LANE];
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; ++j) rank[j] = 0;
    for (int f = 0; f < experts; ++f) {
        const int jf = f >> 6, lf = f & 63;
        int kf = 0;
#pragma unroll
        for (int j = 0; j < ROUTE_PER_LANE; ++j)
            if (j == jf) kf = __shfl(key[j], lf, 64);
#pragma unroll
        for (int j = 0; j < ROUTE_PER_LANE; ++j) {
            const int e = lane + 64 * j;
            if (kf > key[j] || (kf == key[j] && f < e)) ++rank[j];
        }
    }
    // sum of the chosen sigmoids in rank order
    float sum = 1.f;
    if (normalize) {
        sum = -0.0f;
        for (int r = 0; r < used; ++r) {
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < ROUTE_PER_LANE; ++j) {
                const int e = lane + 64 * j;
                const bool hit = j < per && e < experts && rank[j] == r;
                const unsigned long long m = __ballot(hit);
                if (m) v = __shfl(sig[j], __ffsll((long long)m) - 1, 64);
            }
            sum += v;
        }
        sum = fmaxf(sum, 6.103515625e-05f); // half::f16::MIN_POSITIVE
    }
    // chosen experts in ascending index: slot = chosen experts before e
    int before = 0;
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; ++j) {
        const int e = lane + 64 * j;
        const bool chosen = j < per && e < experts && rank[j] < used;
        const unsigned long long m = __ballot(chosen);
        const int slot = before + __popcll(m & ((1ull << lane) - 1ull));
        if (chosen) {
            const size_t o = (size_t)t * used + slot;
            slot_expert[o] = e;
            slot_weight[o] = sig[j] / sum * scale;
            if (pair_token) pair_token[o] = t;
        }
        before += __popcll(m);
    }
}

// out[t][i] = residual[t][i] + (((shared[t][i] + w_0 * ex[t][0][i]) +
// w_1 * ex[t][1][i]) + ...) over `used` expert rows (ex may be null: used 0;
// without a residual, the sum alone); trace, if set, gets a copy. out may
// alias residual.
__global__ __launch_bounds__(256) void ffn_combine_kernel(const float *residual,
                                                          const float *__restrict__ shared,
                                                          const float *__restrict__ ex,
                                                          const float *__restrict__ w, int used,
                                                          int H, float *out,
                                                          float *__restrict__ trace)
{
    const int i = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (i >= H) return;
    const size_t row = (size_t)t * H;
    float acc = shared[row + i];
    for (int s = 0; s < used; ++s)
        acc = __fadd_rn(acc, __fmul_rn(w[(size_t)t * used + s],
                                       ex[((size_t)t * used + s) * H + i]));
    const float h = residual ? __fadd_rn(residual[row + i], acc) : acc;
    out[row + i] = h;
    if (trace) trace[row + i] = h;
}

// rms_norm_into of n rows (src/model.rs:785-830): y = x * (w * scale) over
// whole 16-value steps and x * scale * w over a tail (the aarch64 arm), scale
// = 1/sqrt(mean(x^2) + eps), one workgroup per row.
__global__ __launch_bounds__(256) void rms_rows_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ w, int H,
                                                       float eps, float *__restrict__ y)
{
    __shared__ float part[4];
    const int t = threadIdx.x;
    x += (size_t)blockIdx.x * H;
    y += (size_t)blockIdx.x * H;
    float ss = 0.f;
    for (int i = t; i < H; i += 256) ss += x[i] * x[i];
    ss = wave::sum64(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf(ss / (float)H + eps);
    const int body = H & ~15;
    for (int i = t; i < H; i += 256) y[i] = i < body ? x[i] * (w[i] * scale) : x[i] * scale * w[i];
}

} // namespace

int route_max_experts() { return ROUTE_MAX_EXPERTS; }

int launch_route(const float *logits, const float *bias, int tokens, int experts, int used,
                 bool normalize, float scale, int *slot_expert, float *slot_weight,
                 int *pair_token, void *stream)
{
    if (tokens <= 0) return 0;
    if (experts <= 0 || experts > ROUTE_MAX_EXPERTS || used <= 0 || used > experts)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(route_kernel, dim3(tokens), dim3(64), 0, (hipStream_t)stream, logits,
                       bias, experts, used, (int)normalize, scale, slot_expert, slot_weight,
                       pair_token);
    return (int)hipGetLastError();
}

int launch_ffn_combine(const float *residual, const float *shared, const float *ex,
                       const float *w, int used, int H, int tokens, float *out, float *trace,
                       void *stream)
{
    if (tokens <= 0) return 0;
    hipLaunchKernelGGL(ffn_combine_kernel, dim3((H + 255) / 256, tokens), dim3(256), 0,
                       (hipStream_t)stream, residual, shared, ex, w, used, H, out, trace);
    return (int)hipGetLastError();
}

int launch_rms_rows(const float *x, const float *w, int rows, int H, float eps, float *y,
                    void *stream)
{
    if (rows <= 0) return 0;
    hipLaunchKernelGGL(rms_rows_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, w, H,
                       eps, y);
    return (int)hipGetLastError();
}

} // namespace hyq
