// Building blocks of the f16-MFMA GEMMs on gfx950 (batched matmul,
// Weight::matmul batch >= 2, src/quant.rs:272-344, and the MoE expert
// products, src/model.rs:699-725).
//
// A workgroup of 256 threads (4 waves) owns a BM x BN tile of the product
// Y^T = W X^T (BM weight rows by BN tokens) and walks K in BK = 64 steps:
//   1. every thread dequantizes 32 weights of one row (row t/2, half t%2) of
//      the 64-column slice from the device planes into LDS as f16, with the
//      reference decoder's f32 arithmetic (decode_unchecked,
//      src/quant.rs:2405-2486) followed by one f32->f16 rounding;
//   2. the X slice (f32 activations) is converted to f16 into LDS;
//   3. each wave multiplies its 64 x 64 sub-tile with 2 x 2
//      v_mfma_f32_32x32x16_f16 blocks per 16-wide k step, accumulating in f32.
// LDS rows are padded to 72 halves (144 bytes), so the 16-byte fragment reads
// of 8 consecutive rows fall on 8 distinct 4-bank windows.
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_decode.hpp"

namespace hyq {
namespace tile {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    _Float16 h;
    uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t dw, int i) { return (dw >> (8 * i)) & 0xffu; }

// 16 halves (32 bytes) to an LDS address aligned to 16 bytes.
__device__ __forceinline__ void store16(_Float16 *dst, const _Float16 (&v)[16])
{
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = v[i];
        b[i] = v[8 + i];
    }
    *reinterpret_cast<half8 *>(dst) = a;
    *reinterpret_cast<half8 *>(dst + 8) = b;
}

// ---------------------------------------------------------------------------
// Dequantization of 32 weights of `row`, columns [k0, k0 + 64) half h, to
// dst (the LDS row, indexed by the column offset inside the 64-slice).
// Which 32 of the 64 columns a thread writes depends on the format; the two
// halves of a row always cover all 64.
// ---------------------------------------------------------------------------
template <int F> struct Deq;

// Q4_K (decode_unchecked, src/quant.rs:2437-2461): byte l of a 64-weight
// chunk holds weight l (low nibble, sub-block 2c) and 32 + l (high nibble,
// sub-block 2c+1); value = (d*s_j)*q - (dmin*m_j). Half h takes bytes
// 16h..16h+15, i.e. columns 16h.. and 32+16h...
template <> struct Deq<Q4_K> {
    __device__ __forceinline__ static void run(const WView &w, int row, int k0, int h,
                                               _Float16 *dst)
    {
        const size_t blk = (size_t)row * w.nb + (k0 >> 8);
        const int c = (k0 >> 6) & 3;
        const uint4 qv = *reinterpret_cast<const uint4 *>(w.p0 + blk * 128 + 32 * c + 16 * h);
        const uint4 meta = *reinterpret_cast<const uint4 *>(w.p1 + blk * 16);
        const float d = h2f(meta.x & 0xffffu), dmin = h2f(meta.x >> 16);
        // scales[12] = meta.y, meta.z, meta.w (little endian)
        auto sc = [&](int j) -> int {
            const uint32_t dw = j < 4 ? meta.y : j < 8 ? meta.z : meta.w;
            return (int)byte_of(dw, j & 3);
        };
        int s0, m0, s1, m1;
        {
            const int j0 = 2 * c, j1 = 2 * c + 1;
            if (j0 < 4) {
                s0 = sc(j0) & 63;
                m0 = sc(j0 + 4) & 63;
            } else {
                s0 = (sc(j0 + 4) & 15) | ((sc(j0 - 4) >> 6) << 4);
                m0 = (sc(j0 + 4) >> 4) | ((sc(j0) >> 6) << 4);
            }
            if (j1 < 4) {
                s1 = sc(j1) & 63;
                m1 = sc(j1 + 4) & 63;
            } else {
                s1 = (sc(j1 + 4) & 15) | ((sc(j1 - 4) >> 6) << 4);
                m1 = (sc(j1 + 4) >> 4) | ((sc(j1) >> 6) << 4);
            }
        }
        const float d1a = d * (float)s0, m1a = dmin * (float)m0;
        const float d1b = d * (float)s1, m1b = dmin * (float)m1;
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
        _Float16 lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t b = byte_of(q[i >> 2], i & 3);
            lo[i] = (_Float16)(d1a * (float)(b & 15u) - m1a);
            hi[i] = (_Float16)(d1b * (float)(b >> 4) - m1b);
        }
        store16(dst + 16 * h, lo);
        store16(dst + 32 + 16 * h, hi);
    }
};

// Q6_K (src/quant.rs:2462-2483): in a 128-weight chunk, weight p*32+hf*16+i
// has low bits from ql[(p&1)*32 + hf*16 + i] (nibble p>>1) and high bits
// from qh[hf*16 + i] (bits 2p); value = (d*sc[2p+hf]) * (q - 32). A 64-slice
// holds planes p0, p0+1 (p0 even); half h takes plane p0 + h.
template <> struct Deq<Q6_K> {
    __device__ __forceinline__ static void run(const WView &w, int row, int k0, int h,
                                               _Float16 *dst)
    {
        const size_t blk = (size_t)row * w.nb + (k0 >> 8);
        const int kb = k0 & 255, chunk = kb >> 7;
        const int p = 2 * ((kb >> 6) & 1) + h;
        const uint8_t *base = w.p0 + blk * 192;
        const uint4 l0 = *reinterpret_cast<const uint4 *>(base + chunk * 64 + 32 * h);
        const uint4 l1 = *reinterpret_cast<const uint4 *>(base + chunk * 64 + 32 * h + 16);
        const uint4 g0 = *reinterpret_cast<const uint4 *>(base + 128 + chunk * 32);
        const uint4 g1 = *reinterpret_cast<const uint4 *>(base + 128 + chunk * 32 + 16);
        const uint16_t scp = *reinterpret_cast<const uint16_t *>(w.p1 + blk * 16 + chunk * 8 + 2 * p);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(w.p2 + blk * 2));
        const float s0 = d * (float)(int8_t)(scp & 0xff), s1 = d * (float)(int8_t)(scp >> 8);
        const uint32_t ql[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
        const uint32_t qh[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const int lsh = (p >> 1) * 4, hsh = 2 * p;
        _Float16 v0[16], v1[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t a0 = byte_of(ql[i >> 2], i & 3), a1 = byte_of(ql[4 + (i >> 2)], i & 3);
            const uint32_t b0 = byte_of(qh[i >> 2], i & 3), b1 = byte_of(qh[4 + (i >> 2)], i & 3);
            const int q0 = (int)(((a0 >> lsh) & 15u) | (((b0 >> hsh) & 3u) << 4));
            const int q1 = (int)(((a1 >> lsh) & 15u) | (((b1 >> hsh) & 3u) << 4));
            v0[i] = (_Float16)(s0 * (float)(q0 - 32));
            v1[i] = (_Float16)(s1 * (float)(q1 - 32));
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// Q8_0 (src/quant.rs:2409-2414): value = d * q; half h takes the 32-block h.
template <> struct Deq<Q8_0> {
    __device__ __forceinline__ static void run(const WView &w, int row, int k0, int h,
                                               _Float16 *dst)
    {
        const size_t blk = (size_t)row * w.nb + (k0 >> 5) + h;
        const uint4 a = *reinterpret_cast<const uint4 *>(w.p0 + blk * 32);
        const uint4 b = *reinterpret_cast<const uint4 *>(w.p0 + blk * 32 + 16);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(w.p1 + blk * 2));
        const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        _Float16 v0[16], v1[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            v0[i] = (_Float16)(d * (float)(int8_t)byte_of(q[i >> 2], i & 3));
            v1[i] = (_Float16)(d * (float)(int8_t)byte_of(q[4 + (i >> 2)], i & 3));
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// Q2_0C (src/quant.rs:2415-2422): value = (2c - 3) * d. The device plane
// keeps a 64-weight unit in 16 bytes with weight 16k+i in bits 2k of byte i;
// half h takes k = 2h and 2h+1 (columns 32h..32h+31).
template <> struct Deq<Q2_0C> {
    __device__ __forceinline__ static void run(const WView &w, int row, int k0, int h,
                                               _Float16 *dst)
    {
        const size_t blk = (size_t)row * w.nb + (k0 >> 9);
        const int u = (k0 >> 6) & 7;
        const uint4 cv = *reinterpret_cast<const uint4 *>(w.p0 + blk * 128 + u * 16);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(w.p1 + blk * 2));
        const uint32_t cw[4] = {cv.x, cv.y, cv.z, cv.w};
        _Float16 v0[16], v1[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t b = byte_of(cw[i >> 2], i & 3);
            const int c0 = (int)((b >> (4 * h)) & 3u), c1 = (int)((b >> (4 * h + 2)) & 3u);
            v0[i] = (_Float16)((float)(2 * c0 - 3) * d);
            v1[i] = (_Float16)((float)(2 * c1 - 3) * d);
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// STQ1_0 (src/quant.rs:1086-1123, 2423-2430): 64-weight chunk c holds 16
// groups; digit p of group gg is column p*16 + gg, value (digit - 1) * d with
// the digit read from the codebook entry of (sign << 4 | nibble). Half h
// takes digits 2h and 2h+1. Device planes as in hyq_internal.hpp.
template <> struct Deq<STQ1_0> {
    __device__ __forceinline__ static void run(const WView &w, int row, int k0, int h,
                                               _Float16 *dst)
    {
        const size_t blk = (size_t)row * w.nb + (k0 >> 8);
        const int c = (k0 >> 6) & 3;
        const uint2 nv = *reinterpret_cast<const uint2 *>(w.p0 + blk * 32 + 8 * c);
        const uint32_t S = *reinterpret_cast<const uint32_t *>(w.p1 + blk * 8 + 4 * (c >> 1));
        const float d = h2f(*reinterpret_cast<const uint16_t *>(w.p2 + blk * 2));
        const uint32_t nb[2] = {nv.x, nv.y};
        _Float16 v0[16], v1[16];
#pragma unroll
        for (int gg = 0; gg < 16; ++gg) {
            const int hh = gg >> 3, r8 = gg & 7, t = r8 & 3, hi = r8 >> 2;
            const int code = (int)((byte_of(nb[hh], t) >> (4 * hi)) & 15u);
            const int q = (c & 1) * 4 + (gg >> 2), tq = gg & 3;
            const int sign = (int)((S >> (q + 8 * tq)) & 1u);
            const int e = dec::kStqCodebook[(sign << 4) | code];
            v0[gg] = (_Float16)((float)(((e >> (4 * h)) & 3) - 1) * d);
            v1[gg] = (_Float16)((float)(((e >> (4 * h + 2)) & 3) - 1) * d);
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// Zeros for rows past the end of the weight (each half clears its 32 columns).
__device__ __forceinline__ void zero_half(_Float16 *dst, int h)
{
    const half8 z = {};
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<half8 *>(dst + 32 * h + 8 * i) = z;
}

// ---------------------------------------------------------------------------
// X slice: BN rows (tokens) x 64 columns of f32 -> f16 in LDS. Row r of the
// tile reads src_row(r) (nullptr = zero row). 2048 float4 per slice, 8 per
// thread, 16 consecutive threads per 256-byte row segment.
// ---------------------------------------------------------------------------
template <class RowFn>
__device__ __forceinline__ void load_x(const RowFn &src_row, int k0, float4 (&v)[8])
{
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = t + 256 * i, r = f >> 4, c4 = f & 15;
        const float *p = src_row(r);
        v[i] = p ? *reinterpret_cast<const float4 *>(p + k0 + 4 * c4)
                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

__device__ __forceinline__ void store_x(_Float16 *Xs, const float4 (&v)[8])
{
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = t + 256 * i, r = f >> 4, c4 = f & 15;
        half4 hv = {(_Float16)v[i].x, (_Float16)v[i].y, (_Float16)v[i].z, (_Float16)v[i].w};
        *reinterpret_cast<half4 *>(Xs + r * LDK + 4 * c4) = hv;
    }
}

// One 64-deep step of the wave's 64 x 64 sub-tile: acc[bi][bj] covers weight
// rows wm*64 + 32*bi .. and tokens wn*64 + 32*bj ...
__device__ __forceinline__ void mma_step(const _Float16 *Ws, const _Float16 *Xs, int wm, int wn,
                                         f32x16 (&acc)[2][2])
{
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, kq = 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
        half8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[i] = *reinterpret_cast<const half8 *>(Ws + (wm * 64 + 32 * i + r) * LDK + kk + kq);
            b[i] = *reinterpret_cast<const half8 *>(Xs + (wn * 64 + 32 * i + r) * LDK + kk + kq);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// Element (weight row, token) of accumulator register e of block (i, j):
// v_mfma 32x32 output layout, row = 8*(e/4) + 4*(lane/32) + e%4, col = lane%32.
__device__ __forceinline__ int acc_row(int wm, int i, int e)
{
    const int lane = threadIdx.x & 63;
    return wm * 64 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
__device__ __forceinline__ int acc_col(int wn, int j)
{
    const int lane = threadIdx.x & 63;
    return wn * 64 + 32 * j + (lane & 31);
}

} // namespace tile
} // namespace hyq
