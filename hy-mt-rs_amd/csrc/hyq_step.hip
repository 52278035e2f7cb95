// Device-resident glue of the batch-1 decode step of the dense graph
// (Model::forward_into, src/model.rs:374-546) around the int8 GEMVs:
//   embed_row        embedding.row_into(token)              (src/model.rs:376)
//   rms_norm_q8      rms_norm_into + Q8::quantize_into      (:396-416, :785-830)
//   rope_norm_kv     rope_with_cache, per-head rms_norm of q and k (dense
//                    order: RoPE first), KvCache::append    (:425-452, :874-917)
//   attention        attention_into for one query token    (:949-1035)
//   argmax           greedy sampling                        (src/generation.rs:281-290)
// The current position and token live in device memory, so a whole step can
// be captured once in a HIP graph and replayed without host work.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hyq_decode.hpp"
#include "hyq_q8.hpp"
#include "hyq_step.hpp"

namespace hyq {

namespace {

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// ---- embedding row (Weight::row_into with a device-resident token id) ----
template <int F>
__global__ __launch_bounds__(256) void embed_kernel(WView w, int cols, const int *__restrict__ token,
                                                    float *__restrict__ out)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= cols) return;
    const size_t row = (size_t)*token;
    const size_t blk = row * (size_t)w.nb + i / block_len(F);
    out[i] = dec::decode_plane_value<F>(w, blk, i % block_len(F));
}

// ---- rms_norm_into fused with the Q8 quantizer ----
// One workgroup per 256-value group; each recomputes sum(x^2) over the whole
// row (n <= 64 Ki values, read from L2) so that no cross-workgroup sync is
// needed. y = x * scale * w with scale = 1 / sqrt(mean(x^2) + eps), the x86
// arm's operation order (src/model.rs:825-829).
__global__ __launch_bounds__(256) void rms_norm_q8_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ w, int n,
                                                          float eps, float *__restrict__ y,
                                                          int8_t *q, float *s, int32_t *s16,
                                                          int32_t *s32, int32_t *s256)
{
    __shared__ float part[4];
    const int t = threadIdx.x;
    float ss = 0.f;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        // all of this thread's float4 loads in flight together
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const int n4 = n / 4;
        int i = t;
        for (; i + 768 < n4; i += 1024) {
            const float4 a = x4[i], b = x4[i + 256], c = x4[i + 512], d = x4[i + 768];
            ss += (a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w) +
                  (b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w) +
                  (c.x * c.x + c.y * c.y + c.z * c.z + c.w * c.w) +
                  (d.x * d.x + d.y * d.y + d.z * d.z + d.w * d.w);
        }
        for (; i < n4; i += 256) {
            const float4 a = x4[i];
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
        for (int j = n4 * 4 + t; j < n; j += 256) ss += x[j] * x[j];
    } else {
        for (int i = t; i < n; i += 256) ss += x[i] * x[i];
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float variance = ss / (float)n;
    const float scale = 1.0f / sqrtf(variance + eps);
    const int g = blockIdx.x;
    const int len = min(256, n - g * 256);
    float v = 0.f;
    if (t < len) {
        const int i = g * 256 + t;
        v = x[i] * scale * w[i];
        if (y) y[i] = v;
    }
    q8_quantize_group(v, g, len, q, s, s16, s32, s256);
}

// ---- RoPE + per-head Q/K RMSNorm + KV append ----
// Workgroups [0, heads) rotate and normalise the query heads in place,
// [heads, heads+kv) the key heads into kcache[pos], [heads+kv, heads+2kv)
// copy the value heads into vcache[pos]. Lane j owns the NeoX pair
// (j, j + dim/2) (docs/reference.md:79), so dim/2 lanes per head.
__global__ void rope_norm_kv_kernel(float *__restrict__ q, const float *__restrict__ k,
                                    const float *__restrict__ v, const float *__restrict__ qn,
                                    const float *__restrict__ kn,
                                    const float *__restrict__ freq, const int *__restrict__ pos_p,
                                    int heads, int kvh, int dim, float eps,
                                    float *__restrict__ kcache, float *__restrict__ vcache)
{
    const int b = blockIdx.x;
    const int j = threadIdx.x;
    const int half = dim / 2;
    const int pos = *pos_p;
    const size_t kvw = (size_t)kvh * dim;
    if (b >= heads + kvh) {
        const int h = b - heads - kvh;
        float *dst = vcache + (size_t)pos * kvw + (size_t)h * dim;
        dst[j] = v[h * dim + j];
        dst[j + half] = v[h * dim + j + half];
        return;
    }
    const bool is_q = b < heads;
    const int h = is_q ? b : b - heads;
    const float *src = is_q ? q + (size_t)h * dim : k + (size_t)h * dim;
    const float a = src[j], c2 = src[j + half];
    const float ang = (float)pos * freq[j];
    const float cs = cosf(ang), sn = sinf(ang);
    const float r0 = a * cs - c2 * sn;
    const float r1 = a * sn + c2 * cs;
    // rms_norm over the head (src/model.rs:832-870): scale = 1/sqrt(mean + eps)
    __shared__ float part[4];
    float ss = wave_sum(r0 * r0 + r1 * r1);
    if ((j & 63) == 0) part[j >> 6] = ss;
    __syncthreads();
    ss = 0.f;
    for (int i = 0; i < (half + 63) / 64; ++i) ss += part[i];
    const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    const float *nw = is_q ? qn : kn;
    const float o0 = r0 * scale * nw[j];
    const float o1 = r1 * scale * nw[j + half];
    if (is_q) {
        q[(size_t)h * dim + j] = o0;
        q[(size_t)h * dim + j + half] = o1;
    } else {
        float *dst = kcache + (size_t)pos * kvw + (size_t)h * dim;
        dst[j] = o0;
        dst[j + half] = o1;
    }
}

// ---- attention over positions 0..=pos, split into ATT_CHUNK-position slices ----
// Grid (splits, kv_heads); wave w of a workgroup serves query head
// kvh*rep + hh0 + w for hh0 = 0, 4, ... (rep = heads/kv_heads). The slice's K
// and V rows are fetched with all loads in flight at once (4 float4 of each
// per thread), then staged in LDS (K rows padded to 129 floats). Two lanes
// share one position's 128-wide dot; the wave then forms the slice's max,
// exp-sum and exp-weighted V sum; attn_combine merges the slices.
constexpr int ATT_CHUNK = 32;
constexpr int ATT_D = 128;

__global__ __launch_bounds__(256) void attn_partial_kernel(
    const float *__restrict__ q, const float *__restrict__ kcache,
    const float *__restrict__ vcache, const int *__restrict__ pos_p, int heads, int kvh,
    float scale, float *__restrict__ part, int splits)
{
    constexpr int D = ATT_D;
    __shared__ float Ks[ATT_CHUNK][D + 1];
    __shared__ float4 Vs[ATT_CHUNK][D / 4];
    __shared__ float Qs[4][D];
    const int split = blockIdx.x, kh = blockIdx.y;
    const int visible = *pos_p + 1;
    const int p0 = split * ATT_CHUNK;
    const int n = min(ATT_CHUNK, visible - p0);
    const int rep = heads / kvh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const size_t kvw = (size_t)kvh * D;
    if (n <= 0) {
        for (int i = t; i < rep; i += 256) {
            float *o = part + ((size_t)(kh * rep + i) * splits + split) * (D + 2);
            o[0] = -INFINITY;
            o[1] = 0.f;
        }
        return;
    }
    float4 kr[4], vr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = t + 256 * j; // float4 index in the 32 x 128 slice
        const int p = idx >> 5, d4 = idx & 31;
        if (p < n) {
            const size_t off = (size_t)(p0 + p) * kvw + (size_t)kh * D + 4 * d4;
            kr[j] = *reinterpret_cast<const float4 *>(kcache + off);
            vr[j] = *reinterpret_cast<const float4 *>(vcache + off);
        } else {
            kr[j] = vr[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = t + 256 * j;
        const int p = idx >> 5, d4 = idx & 31;
        Ks[p][4 * d4] = kr[j].x;
        Ks[p][4 * d4 + 1] = kr[j].y;
        Ks[p][4 * d4 + 2] = kr[j].z;
        Ks[p][4 * d4 + 3] = kr[j].w;
        Vs[p][d4] = vr[j];
    }
    const int p = lane & 31, hf = lane >> 5;
    for (int hh0 = 0; hh0 < rep; hh0 += 4) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = t + 256 * j, hq = i / D;
            if (hh0 + hq < rep) Qs[hq][i % D] = q[(size_t)(kh * rep + hh0 + hq) * D + i % D];
        }
        __syncthreads();
        const int hh = hh0 + wave;
        if (hh < rep) {
            const int h = kh * rep + hh;
            float dot = 0.f;
#pragma unroll 16
            for (int d = 0; d < 64; ++d) dot += Qs[wave][hf * 64 + d] * Ks[p][hf * 64 + d];
            dot += __shfl_xor(dot, 32, 64);
            const float sc = p < n ? dot * scale : -INFINITY;
            const float m = wave_max(sc);
            const float e = p < n ? expf(sc - m) : 0.f;
            const float sum = wave_sum(e) * 0.5f; // each position is held by two lanes
            // lanes 0..31 own output dims 4*lane .. 4*lane+3 of V rows
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int pp = 0; pp < n; ++pp) {
                const float ep = __shfl(e, pp, 64);
                const float4 vv = Vs[pp][lane & 31];
                a.x += ep * vv.x;
                a.y += ep * vv.y;
                a.z += ep * vv.z;
                a.w += ep * vv.w;
            }
            float *o = part + ((size_t)h * splits + split) * (D + 2);
            if (lane == 0) {
                o[0] = m;
                o[1] = sum;
            }
            if (lane < 32) {
                o[2 + 4 * lane] = a.x;
                o[3 + 4 * lane] = a.y;
                o[4 + 4 * lane] = a.z;
                o[5 + 4 * lane] = a.w;
            }
        }
        __syncthreads();
    }
}

// Merges the slices of two heads per workgroup (256 output values = one Q8
// group) and quantizes the attended vector for the output projection. The
// per-slice maxima and sums are staged in LDS (dynamic: 6 floats per slice),
// then every output value sums its slices with independent loads.
__global__ __launch_bounds__(256) void attn_combine_q8_kernel(
    const float *__restrict__ part, int heads, int splits, float *__restrict__ out, int8_t *q,
    float *s, int32_t *s16, int32_t *s32, int32_t *s256)
{
    constexpr int D = ATT_D;
    extern __shared__ float st[]; // m[2][S], sum[2][S], w[2][S]
    __shared__ float den[2];
    float *sm = st, *ssum = st + 2 * splits, *sw = st + 4 * splits;
    const int t = threadIdx.x;
    const int g = blockIdx.x;
    for (int i = t; i < 2 * splits; i += 256) {
        const int hl = i / splits, sp = i % splits, h = 2 * g + hl;
        float m = -INFINITY, sum = 0.f;
        if (h < heads) {
            const float *o = part + ((size_t)h * splits + sp) * (D + 2);
            m = o[0];
            sum = o[1];
        }
        sm[i] = m;
        ssum[i] = sum;
    }
    __syncthreads();
    // Slices that hold positions have sum >= 1 and form a prefix; the
    // accumulators of the others were never written and are not read.
    __shared__ float Mh[2];
    __shared__ int nvalid;
    if (t < 2) {
        float M = -INFINITY;
        int nv = 0;
        for (int sp = 0; sp < splits; ++sp)
            if (ssum[t * splits + sp] > 0.f) {
                M = fmaxf(M, sm[t * splits + sp]);
                nv = sp + 1;
            }
        Mh[t] = M;
        if (t == 0) nvalid = nv;
    }
    __syncthreads();
    for (int i = t; i < 2 * splits; i += 256)
        sw[i] = ssum[i] > 0.f ? expf(sm[i] - Mh[i / splits]) : 0.f;
    __syncthreads();
    if (t < 2) {
        float dsum = 0.f;
        for (int sp = 0; sp < splits; ++sp) dsum += sw[t * splits + sp] * ssum[t * splits + sp];
        den[t] = dsum;
    }
    __syncthreads();
    const int hl = t / D, d = t % D, h = 2 * g + hl;
    float v = 0.f;
    if (h < heads) {
        const float *ph = part + (size_t)h * splits * (D + 2) + 2 + d;
        const float *w = sw + hl * splits;
        float n0 = 0.f, n1 = 0.f, n2 = 0.f, n3 = 0.f;
        const int nv = nvalid;
        int sp = 0;
        for (; sp + 4 <= nv; sp += 4) {
            n0 += w[sp] * ph[(size_t)sp * (D + 2)];
            n1 += w[sp + 1] * ph[(size_t)(sp + 1) * (D + 2)];
            n2 += w[sp + 2] * ph[(size_t)(sp + 2) * (D + 2)];
            n3 += w[sp + 3] * ph[(size_t)(sp + 3) * (D + 2)];
        }
        for (; sp < nv; ++sp) n0 += w[sp] * ph[(size_t)sp * (D + 2)];
        v = ((n0 + n1) + (n2 + n3)) / den[hl];
        if (out) out[h * D + d] = v;
    }
    const int len = min(256, heads * D - g * 256);
    if (q) q8_quantize_group(v, g, len, q, s, s16, s32, s256);
}

// ---- greedy argmax: first maximum wins ----
// Pass 1: each workgroup reduces a slice to (value, index); pass 2: one
// workgroup reduces the partials and stores the token (and optionally
// advances the step state).
__device__ __forceinline__ void better(float &v, int &i, float ov, int oi)
{
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ x, int n,
                                                             float *__restrict__ pv,
                                                             int *__restrict__ pi)
{
    __shared__ float sv[4];
    __shared__ int si[4];
    const int t = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = blockIdx.x * 256 + t; i < n; i += gridDim.x * 256) better(v, idx, x[i], i);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    if ((t & 63) == 0) {
        sv[t >> 6] = v;
        si[t >> 6] = idx;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 4; ++w) better(v, idx, sv[w], si[w]);
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float *__restrict__ pv,
                                                          const int *__restrict__ pi, int np,
                                                          int *__restrict__ token,
                                                          StepState *st, int *history)
{
    const int t = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = t; i < np; i += 64) better(v, idx, pv[i], pi[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    if (t == 0) {
        *token = idx;
        if (st) {
            if (history && st->step < st->history_cap) history[st->step] = idx;
            st->step += 1;
            st->pos += 1;
        }
    }
}

} // namespace

int launch_embed_row(int fmt, WView w, int cols, const int *token, float *out, void *stream)
{
    dim3 grid((cols + 255) / 256), block(256);
    hipStream_t st = (hipStream_t)stream;
#define HYQ_EMB(F)                                                                             \
    case F: hipLaunchKernelGGL(embed_kernel<F>, grid, block, 0, st, w, cols, token, out); break;
    switch (fmt) {
        HYQ_EMB(Q2_0C)
        HYQ_EMB(STQ1_0)
        HYQ_EMB(Q4_K)
        HYQ_EMB(Q6_K)
        HYQ_EMB(Q8_0)
        HYQ_EMB(F32)
        HYQ_EMB(F16)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_EMB
    return (int)hipGetLastError();
}

int launch_rms_norm_q8(const float *x, const float *w, int n, float eps, float *y, int8_t *q,
                       float *s, int32_t *s16, int32_t *s32, int32_t *s256, void *stream)
{
    hipLaunchKernelGGL(rms_norm_q8_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, x, w, n, eps, y, q, s, s16, s32, s256);
    return (int)hipGetLastError();
}

int launch_rope_norm_kv(float *q, const float *k, const float *v, const float *qn,
                        const float *kn, const float *freq, const int *pos, int heads, int kvh,
                        int dim, float eps, float *kcache, float *vcache, void *stream)
{
    hipLaunchKernelGGL(rope_norm_kv_kernel, dim3(heads + 2 * kvh), dim3(dim / 2), 0,
                       (hipStream_t)stream, q, k, v, qn, kn, freq, pos, heads, kvh, dim, eps,
                       kcache, vcache);
    return (int)hipGetLastError();
}

int attention_splits(int context) { return (context + ATT_CHUNK - 1) / ATT_CHUNK; }

int launch_attention(const float *q, const float *kcache, const float *vcache, const int *pos,
                     int context, int heads, int kvh, float *part, float *out, int8_t *qq,
                     float *s, int32_t *s16, int32_t *s32, int32_t *s256, void *stream)
{
    const int splits = attention_splits(context);
    const float scale = 1.0f / sqrtf(128.0f);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(attn_partial_kernel, dim3(splits, kvh), dim3(256), 0, st, q, kcache,
                       vcache, pos, heads, kvh, scale, part, splits);
    hipLaunchKernelGGL(attn_combine_q8_kernel, dim3((heads * 128 + 255) / 256), dim3(256),
                       (size_t)splits * 6 * sizeof(float), st, part, heads, splits, out, qq, s,
                       s16, s32, s256);
    return (int)hipGetLastError();
}

int argmax_partials(int n) { return std::min(64, (n + 4095) / 4096 > 0 ? (n + 4095) / 4096 : 1); }

int launch_argmax(const float *x, int n, float *pv, int *pi, int *token, StepState *st,
                  int *history, void *stream)
{
    const int np = argmax_partials(n);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(np), dim3(256), 0, s, x, n, pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, s, pv, pi, np, token, st,
                       history);
    return (int)hipGetLastError();
}

} // namespace hyq
