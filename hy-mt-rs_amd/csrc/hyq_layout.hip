// GGUF blocks <-> device planes, and the bit-exact block decoders
// (decode_unchecked, src/quant.rs:2405-2486) on gfx950.
//
// The decoders must reproduce the reference's f32 bit patterns, so this file
// is compiled without floating-point contraction: `d1 * q - m1` stays a
// rounded product followed by a rounded difference, as in the Rust source.
#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"

#pragma clang fp contract(off)

namespace hyq {

namespace {

__device__ __forceinline__ float h2f_bytes(const uint8_t *p)
{
    uint16_t b = (uint16_t)(p[0] | (p[1] << 8));
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// STQ_CODEBOOK (src/quant.rs:1081-1084), ggml-derived (MIT).
__constant__ uint8_t kStqCodebook[32] = {
    0xa9, 0x89, 0x29, 0x09, 0xa6, 0x86, 0x26, 0x06, 0x9a, 0x92, 0x1a, 0x12, 0x6a, 0x62, 0x4a, 0x42,
    0x01, 0x21, 0x81, 0xa1, 0x04, 0x24, 0x84, 0xa4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68,
};

// ---------------------------------------------------------------------------
// Repack: one thread per GGUF block; linear block i lands at i * plane_bytes
// in every plane (both orders are row-major over (row, block)).
// ---------------------------------------------------------------------------
template <int F>
__global__ void repack_kernel(const uint8_t *__restrict__ gguf, size_t nblocks,
                              uint8_t *__restrict__ p0, uint8_t *__restrict__ p1,
                              uint8_t *__restrict__ p2)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t *b = gguf + i * block_bytes(F);
    if (F == Q2_0C) {
        p1[2 * i] = b[0];
        p1[2 * i + 1] = b[1];
        const uint8_t *codes = b + 2;
        uint8_t *o = p0 + i * 128;
        for (int u = 0; u < 8; ++u)
            for (int m = 0; m < 4; ++m)
                for (int t = 0; t < 4; ++t) {
                    int v = 0;
                    for (int k = 0; k < 4; ++k)
                        v |= ((codes[u * 16 + 4 * k + m] >> (2 * t)) & 3) << (2 * k);
                    o[u * 16 + 4 * m + t] = (uint8_t)v;
                }
    } else if (F == STQ1_0) {
        uint8_t *o = p0 + i * 32;
        for (int c = 0; c < 4; ++c)
            for (int h = 0; h < 2; ++h)
                for (int t = 0; t < 4; ++t) {
                    const int lo = 16 * c + 8 * h + t, hi = lo + 4;
                    const int nlo = (b[lo >> 1] >> (4 * (lo & 1))) & 15;
                    const int nhi = (b[hi >> 1] >> (4 * (hi & 1))) & 15;
                    o[8 * c + 4 * h + t] = (uint8_t)(nlo | (nhi << 4));
                }
        for (int j = 0; j < 2; ++j) {
            uint32_t S = 0;
            for (int q = 0; q < 8; ++q)
                for (int t = 0; t < 4; ++t) {
                    const int g = 16 * (2 * j + q / 4) + 4 * (q % 4) + t;
                    const uint32_t sg = (b[32 + (g >> 3)] >> (g & 7)) & 1;
                    S |= sg << (q + 8 * t);
                }
            for (int k = 0; k < 4; ++k) p1[i * 8 + 4 * j + k] = (uint8_t)(S >> (8 * k));
        }
        p2[2 * i] = b[40];
        p2[2 * i + 1] = b[41];
    } else if (F == Q4_K) {
        for (int k = 0; k < 16; ++k) p1[i * 16 + k] = b[k];
        for (int k = 0; k < 128; ++k) p0[i * 128 + k] = b[16 + k];
    } else if (F == Q6_K) {
        for (int k = 0; k < 192; ++k) p0[i * 192 + k] = b[k];
        for (int k = 0; k < 16; ++k) p1[i * 16 + k] = b[192 + k];
        p2[2 * i] = b[208];
        p2[2 * i + 1] = b[209];
    } else if (F == Q8_0) {
        for (int k = 0; k < 32; ++k) p0[i * 32 + k] = b[2 + k];
        p1[2 * i] = b[0];
        p1[2 * i + 1] = b[1];
    } else {
        for (int k = 0; k < block_bytes(F); ++k) p0[i * block_bytes(F) + k] = b[k];
    }
}

// Q4_K sub-block scale and min (src/quant.rs:2441-2451).
__device__ __forceinline__ void q4k_scale_min(const uint8_t *scales, int j, int &s, int &m)
{
    if (j < 4) {
        s = scales[j] & 63;
        m = scales[j + 4] & 63;
    } else {
        s = (scales[j + 4] & 15) | ((scales[j - 4] >> 6) << 4);
        m = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------
// Decode of output value j (0 <= j < block_len) of one block, from the GGUF
// block bytes. Mirrors decode_unchecked's arithmetic exactly.
// ---------------------------------------------------------------------------
template <int F>
__device__ __forceinline__ float decode_gguf_value(const uint8_t *b, int j)
{
    if (F == Q8_0) {
        const float d = h2f_bytes(b);
        return d * (float)(int8_t)b[2 + j];
    } else if (F == Q2_0C) {
        const float d = h2f_bytes(b);
        const int c = (b[2 + j / 4] >> (2 * (j % 4))) & 3;
        return (float)(2 * c - 3) * d;
    } else if (F == STQ1_0) {
        const float d = h2f_bytes(b + 40);
        const int c = j / 64, p = (j % 64) / 16, g = 16 * c + j % 16;
        const int code = (b[g >> 1] >> (4 * (g % 2))) & 15;
        const int sign = (b[32 + (g >> 3)] >> (g & 7)) & 1;
        const int e = kStqCodebook[(sign << 4) | code];
        return (float)(((e >> (2 * p)) & 3) - 1) * d;
    } else if (F == Q4_K) {
        const float d = h2f_bytes(b), dmin = h2f_bytes(b + 2);
        const int group = j / 64, hi = (j % 64) / 32, l = j % 32;
        int s, m;
        q4k_scale_min(b + 4, group * 2 + hi, s, m);
        const float d1 = d * (float)s, m1 = dmin * (float)m;
        const int q = b[16 + group * 32 + l];
        return d1 * (float)(hi ? q >> 4 : q & 15) - m1;
    } else if (F == Q6_K) {
        const float d = h2f_bytes(b + 208);
        const int chunk = j / 128, rem = j % 128, p = rem / 32, hf = (rem % 32) / 16, i = rem % 16;
        const float s = d * (float)(int8_t)b[192 + chunk * 8 + 2 * p + hf];
        const int qv = b[chunk * 64 + hf * 16 + (p & 1) * 32 + i];
        const int hv = b[128 + chunk * 32 + hf * 16 + i];
        const int q = ((qv >> ((p >> 1) * 4)) & 15) | (((hv >> (2 * p)) & 3) << 4);
        return s * (float)(q - 32);
    } else if (F == F16) {
        return h2f_bytes(b);
    } else {
        float v;
        __builtin_memcpy(&v, b, 4);
        return v;
    }
}

template <int F>
__global__ void decode_gguf_kernel(const uint8_t *__restrict__ bytes, size_t nblocks,
                                   float *__restrict__ out)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nblocks * (size_t)block_len(F)) return;
    const size_t blk = idx / block_len(F);
    const int j = (int)(idx % block_len(F));
    out[idx] = decode_gguf_value<F>(bytes + blk * block_bytes(F), j);
}

// ---------------------------------------------------------------------------
// Decode from the device planes (embedding rows, to_vec, prefill fallback).
// ---------------------------------------------------------------------------
template <int F>
__device__ __forceinline__ float decode_plane_value(const WView &w, size_t blk, int j)
{
    if (F == Q8_0) {
        const float d = h2f_bytes(w.p1 + 2 * blk);
        return d * (float)(int8_t)w.p0[blk * 32 + j];
    } else if (F == Q2_0C) {
        const float d = h2f_bytes(w.p1 + 2 * blk);
        const int u = j / 64, wi = j % 64, k = wi / 16, m = (wi % 16) / 4, t = wi % 4;
        const int c = (w.p0[blk * 128 + u * 16 + 4 * m + t] >> (2 * k)) & 3;
        return (float)(2 * c - 3) * d;
    } else if (F == STQ1_0) {
        const float d = h2f_bytes(w.p2 + 2 * blk);
        const int c = j / 64, p = (j % 64) / 16, gg = j % 16;
        const int h = gg / 8, r8 = gg % 8, t = r8 % 4, hi = r8 / 4;
        const int code = (w.p0[blk * 32 + 8 * c + 4 * h + t] >> (4 * hi)) & 15;
        const int qi = gg / 4, tq = gg % 4, q = (c % 2) * 4 + qi;
        const uint8_t *sp = w.p1 + blk * 8 + 4 * (c / 2);
        const uint32_t S = sp[0] | (sp[1] << 8) | (sp[2] << 16) | ((uint32_t)sp[3] << 24);
        const int sign = (S >> (q + 8 * tq)) & 1;
        const int e = kStqCodebook[(sign << 4) | code];
        return (float)(((e >> (2 * p)) & 3) - 1) * d;
    } else if (F == Q4_K) {
        const uint8_t *meta = w.p1 + blk * 16;
        const float d = h2f_bytes(meta), dmin = h2f_bytes(meta + 2);
        const int group = j / 64, hi = (j % 64) / 32, l = j % 32;
        int s, m;
        q4k_scale_min(meta + 4, group * 2 + hi, s, m);
        const float d1 = d * (float)s, m1 = dmin * (float)m;
        const int q = w.p0[blk * 128 + group * 32 + l];
        return d1 * (float)(hi ? q >> 4 : q & 15) - m1;
    } else if (F == Q6_K) {
        const float d = h2f_bytes(w.p2 + 2 * blk);
        const int chunk = j / 128, rem = j % 128, p = rem / 32, hf = (rem % 32) / 16, i = rem % 16;
        const float s = d * (float)(int8_t)w.p1[blk * 16 + chunk * 8 + 2 * p + hf];
        const uint8_t *x = w.p0 + blk * 192;
        const int qv = x[chunk * 64 + hf * 16 + (p & 1) * 32 + i];
        const int hv = x[128 + chunk * 32 + hf * 16 + i];
        const int q = ((qv >> ((p >> 1) * 4)) & 15) | (((hv >> (2 * p)) & 3) << 4);
        return s * (float)(q - 32);
    } else if (F == F16) {
        return h2f_bytes(w.p0 + 2 * blk);
    } else {
        float v;
        __builtin_memcpy(&v, w.p0 + 4 * blk, 4);
        return v;
    }
}

template <int F>
__global__ void dequant_rows_kernel(WView w, int row0, int nrows, int cols,
                                    float *__restrict__ out)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)nrows * cols) return;
    const size_t r = row0 + idx / cols;
    const int i = (int)(idx % cols);
    const size_t blk = r * (size_t)w.nb + i / block_len(F);
    out[idx] = decode_plane_value<F>(w, blk, i % block_len(F));
}

} // namespace

int launch_repack(int fmt, const uint8_t *gguf, size_t nblocks, int, uint8_t *p0, uint8_t *p1,
                  uint8_t *p2, void *stream)
{
    if (nblocks == 0) return 0;
    dim3 block(256), grid((unsigned)((nblocks + 255) / 256));
    hipStream_t st = (hipStream_t)stream;
#define HYQ_REPACK(F)                                                                          \
    case F: hipLaunchKernelGGL(repack_kernel<F>, grid, block, 0, st, gguf, nblocks, p0, p1, p2); \
        break;
    switch (fmt) {
        HYQ_REPACK(Q2_0C)
        HYQ_REPACK(STQ1_0)
        HYQ_REPACK(Q4_K)
        HYQ_REPACK(Q6_K)
        HYQ_REPACK(Q8_0)
        HYQ_REPACK(F32)
        HYQ_REPACK(F16)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_REPACK
    return (int)hipGetLastError();
}

int launch_decode_gguf(int fmt, const uint8_t *bytes, size_t nblocks, float *out, void *stream)
{
    const size_t n = nblocks * (size_t)block_len(fmt);
    if (n == 0) return 0;
    dim3 block(256), grid((unsigned)((n + 255) / 256));
    hipStream_t st = (hipStream_t)stream;
#define HYQ_DEC(F)                                                                             \
    case F: hipLaunchKernelGGL(decode_gguf_kernel<F>, grid, block, 0, st, bytes, nblocks, out); \
        break;
    switch (fmt) {
        HYQ_DEC(Q2_0C)
        HYQ_DEC(STQ1_0)
        HYQ_DEC(Q4_K)
        HYQ_DEC(Q6_K)
        HYQ_DEC(Q8_0)
        HYQ_DEC(F32)
        HYQ_DEC(F16)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_DEC
    return (int)hipGetLastError();
}

int launch_dequant_rows(int fmt, WView w, int row0, int nrows, int cols, float *out,
                        void *stream)
{
    const size_t n = (size_t)nrows * cols;
    if (n == 0) return 0;
    dim3 block(256), grid((unsigned)((n + 255) / 256));
    hipStream_t st = (hipStream_t)stream;
#define HYQ_DQ(F)                                                                              \
    case F:                                                                                    \
        hipLaunchKernelGGL(dequant_rows_kernel<F>, grid, block, 0, st, w, row0, nrows, cols,   \
                           out);                                                               \
        break;
    switch (fmt) {
        HYQ_DQ(Q2_0C)
        HYQ_DQ(STQ1_0)
        HYQ_DQ(Q4_K)
        HYQ_DQ(Q6_K)
        HYQ_DQ(Q8_0)
        HYQ_DQ(F32)
        HYQ_DQ(F16)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_DQ
    return (int)hipGetLastError();
}

} // namespace hyq
