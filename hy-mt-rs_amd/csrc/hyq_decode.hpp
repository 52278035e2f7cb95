// Bit-exact block decoders (decode_unchecked, src/quant.rs:2405-2486) as
// device functions, from GGUF block bytes and from the device planes.
// Floating-point contraction is off for every file that includes this
// header: `d1 * q - m1` must stay a rounded product and a rounded difference,
// as in the Rust source, to reproduce the reference's f32 bit patterns.
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"

#pragma clang fp contract(off)

namespace hyq {
namespace dec {

__device__ __forceinline__ float h2f_bytes(const uint8_t *p)
{
    uint16_t b = (uint16_t)(p[0] | (p[1] << 8));
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// STQ_CODEBOOK (src/quant.rs:1081-1084), ggml-derived (MIT; notice in THIRD_PARTY_NOTICES.md).
static __constant__ uint8_t kStqCodebook[32] = {
    0xa9, 0x89, 0x29, 0x09, 0xa6, 0x86, 0x26, 0x06, 0x9a, 0x92, 0x1a, 0x12, 0x6a, 0x62, 0x4a, 0x42,
    0x01, 0x21, 0x81, 0xa1, 0x04, 0x24, 0x84, 0xa4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68,
};

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

} // namespace dec
} // namespace hyq
