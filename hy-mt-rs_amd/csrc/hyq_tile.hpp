// Building blocks of the f16-MFMA GEMMs on gfx950 (batched matmul,
// Weight::matmul batch >= 2, src/quant.rs:272-344, and the MoE expert
// products, src/model.rs:699-725).
//
// A workgroup of 256 threads (4 waves) owns BM = 128 LDS weight rows by
// BN = 128 tokens and walks K in BK = 64 steps:
//   1. every thread fetches the packed bytes of 32 weights of one LDS row
//      (row t/2, half t%2) of the next 64-column slice, and 4 x 16 bytes of
//      the f16 activation slice, into registers (Raw / XRaw);
//   2. after the current slice's MFMAs it dequantizes them into the other
//      LDS buffer with the reference decoder's f32 arithmetic
//      (decode_unchecked, src/quant.rs:2405-2486) and one f32->f16 rounding;
//   3. each wave multiplies a 64 x 64 (weight rows x tokens) sub-tile with
//      2 x 2 v_mfma_f32_32x32x16_f16 blocks per 16-wide k step, in f32.
// Two LDS buffers let one barrier per step separate writers from readers.
// LDS rows are padded to 72 halves (144 bytes), so the 16-byte fragment
// reads of 8 consecutive rows fall on 8 distinct 4-bank windows.
// The wide form (NW = 8 waves, 512 threads) takes 256 tokens: waves 0-3
// dequantize the weight slice as above, all eight fetch the activations and
// each multiplies its own 64 x 64 sub-tile, so a dequantized weight feeds
// twice the MFMAs. Every output element sees the same operands in the same
// k order in both forms, so their results are bit-identical.
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_decode.hpp"
#include "hyq_groups.hpp"

namespace hyq {
namespace tile {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;
constexpr int TILE_HALVES = BM * LDK; // one LDS operand buffer (BM == BN)

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    _Float16 h;
    uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t dw, int i) { return (dw >> (8 * i)) & 0xffu; }

// 16 f32 values rounded to f16 (round to nearest even), stored as 32 bytes
// at a 16-byte aligned LDS address.
__device__ __forceinline__ void store16(_Float16 *dst, const float (&v)[16])
{
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v p = __builtin_convertvector((float2v){v[2 * i], v[2 * i + 1]}, half2v);
        const half2v q = __builtin_convertvector((float2v){v[8 + 2 * i], v[9 + 2 * i]}, half2v);
        a[2 * i] = p[0];
        a[2 * i + 1] = p[1];
        b[2 * i] = q[0];
        b[2 * i + 1] = q[1];
    }
    *reinterpret_cast<half8 *>(dst) = a;
    *reinterpret_cast<half8 *>(dst + 8) = b;
}

// ---------------------------------------------------------------------------
// Per-format dequantization of 32 weights of one row, columns [k0, k0 + 64)
// half h, to dst (the LDS row, indexed by column offset inside the slice).
// Which 32 columns a half writes depends on the format; the two halves of a
// row always cover all 64. load() only issues global loads from the row's
// plane bases (RowPtr, computed once per thread); convert() does the
// arithmetic from registers.
//
// Every value is formed as one fma whose exact result is the decoder's
// exact value, so the f32 result is bit-identical to decode_unchecked
// (src/quant.rs:2405-2486), then rounded once to f16: the packed codes are
// widened with v_cvt_f32_ubyteN (byte n of a dword to f32) and offsets are
// folded into the fma's addend (q - 32 as s*q + (-32 s), int8 q as
// d*(q + 128) + (-128 d), 2c - 3 as 2d*c + (-3d)). The products in those
// addends and multipliers are exact in f32 (at most 24 significant bits).
// ---------------------------------------------------------------------------
struct RowPtr {
    const uint8_t *p0, *p1, *p2;
};

__device__ __forceinline__ RowPtr row_ptr(const WView &w, int F_p0, int F_p1, int F_p2, int row)
{
    const size_t b = (size_t)row * w.nb;
    return RowPtr{w.p0 + b * F_p0, w.p1 + b * F_p1, w.p2 + b * F_p2};
}

// byte i of x as f32 (v_cvt_f32_ubyte{i})
__device__ __forceinline__ float ub(uint32_t x, int i) { return (float)((x >> (8 * i)) & 0xffu); }

template <int F> struct Deq;

// Q4_K (decode_unchecked, src/quant.rs:2437-2461): byte l of a 64-weight
// chunk holds weight l (low nibble, sub-block 2c) and 32 + l (high nibble,
// sub-block 2c+1); value = (d*s_j)*q - (dmin*m_j). Half h takes bytes
// 16h..16h+15, i.e. columns 16h.. and 32+16h...
template <> struct Deq<Q4_K> {
    struct Raw {
        uint4 q, meta;
    };
    __device__ __forceinline__ static RowPtr rows(const WView &w, int row)
    {
        return row_ptr(w, 128, 16, 0, row);
    }
    __device__ __forceinline__ static void load(Raw &r, const RowPtr &p, int k0, int h)
    {
        const int blk = k0 >> 8, c = (k0 >> 6) & 3;
        r.q = *reinterpret_cast<const uint4 *>(p.p0 + blk * 128 + 32 * c + 16 * h);
        r.meta = *reinterpret_cast<const uint4 *>(p.p1 + blk * 16);
    }
    __device__ __forceinline__ static void scale_min(const uint4 &meta, int j, int &s, int &m)
    {
        auto sc = [&](int i) -> int {
            const uint32_t dw = i < 4 ? meta.y : i < 8 ? meta.z : meta.w;
            return (int)byte_of(dw, i & 3);
        };
        if (j < 4) {
            s = sc(j) & 63;
            m = sc(j + 4) & 63;
        } else {
            s = (sc(j + 4) & 15) | ((sc(j - 4) >> 6) << 4);
            m = (sc(j + 4) >> 4) | ((sc(j) >> 6) << 4);
        }
    }
    __device__ __forceinline__ static void convert(const Raw &r, int u, int h, _Float16 *dst)
    {
        const int c = u;
        const float d = h2f(r.meta.x & 0xffffu), dmin = h2f(r.meta.x >> 16);
        int s0, m0, s1, m1;
        scale_min(r.meta, 2 * c, s0, m0);
        scale_min(r.meta, 2 * c + 1, s1, m1);
        const float d1a = d * (float)s0, nm1a = -(dmin * (float)m0);
        const float d1b = d * (float)s1, nm1b = -(dmin * (float)m1);
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float lo[16], hi[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t l = q[w] & 0x0F0F0F0Fu, u = (q[w] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[4 * w + i] = __builtin_fmaf(d1a, ub(l, i), nm1a);
                hi[4 * w + i] = __builtin_fmaf(d1b, ub(u, i), nm1b);
            }
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
    struct Raw {
        uint4 l0, l1, g0, g1;
        uint32_t sc, d;
    };
    __device__ __forceinline__ static RowPtr rows(const WView &w, int row)
    {
        return row_ptr(w, 192, 16, 2, row);
    }
    __device__ __forceinline__ static void load(Raw &r, const RowPtr &p, int k0, int h)
    {
        const int blk = k0 >> 8, kb = k0 & 255, chunk = kb >> 7;
        const int pl = 2 * ((kb >> 6) & 1) + h;
        const uint8_t *base = p.p0 + blk * 192;
        r.l0 = *reinterpret_cast<const uint4 *>(base + chunk * 64 + 32 * h);
        r.l1 = *reinterpret_cast<const uint4 *>(base + chunk * 64 + 32 * h + 16);
        r.g0 = *reinterpret_cast<const uint4 *>(base + 128 + chunk * 32);
        r.g1 = *reinterpret_cast<const uint4 *>(base + 128 + chunk * 32 + 16);
        r.sc = *reinterpret_cast<const uint16_t *>(p.p1 + blk * 16 + chunk * 8 + 2 * pl);
        r.d = *reinterpret_cast<const uint16_t *>(p.p2 + blk * 2);
    }
    __device__ __forceinline__ static void convert(const Raw &r, int u, int h, _Float16 *dst)
    {
        const int pl = 2 * (u & 1) + h;
        const float d = h2f(r.d);
        const float s0 = d * (float)(int8_t)(r.sc & 0xff), s1 = d * (float)(int8_t)(r.sc >> 8);
        const float o0 = -32.f * s0, o1 = -32.f * s1;
        const uint32_t ql[8] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w, r.l1.x, r.l1.y, r.l1.z, r.l1.w};
        const uint32_t qh[8] = {r.g0.x, r.g0.y, r.g0.z, r.g0.w, r.g1.x, r.g1.y, r.g1.z, r.g1.w};
        const int lsh = (pl >> 1) * 4, hsh = 2 * pl;
        float v0[16], v1[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t qa = ((ql[w] >> lsh) & 0x0F0F0F0Fu) | (((qh[w] >> hsh) & 0x03030303u) << 4);
            const uint32_t qb =
                ((ql[4 + w] >> lsh) & 0x0F0F0F0Fu) | (((qh[4 + w] >> hsh) & 0x03030303u) << 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v0[4 * w + i] = __builtin_fmaf(s0, ub(qa, i), o0);
                v1[4 * w + i] = __builtin_fmaf(s1, ub(qb, i), o1);
            }
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// Q8_0 (src/quant.rs:2409-2414): value = d * q; half h takes the 32-block h.
template <> struct Deq<Q8_0> {
    struct Raw {
        uint4 a, b;
        uint32_t d;
    };
    __device__ __forceinline__ static RowPtr rows(const WView &w, int row)
    {
        return row_ptr(w, 32, 2, 0, row);
    }
    __device__ __forceinline__ static void load(Raw &r, const RowPtr &p, int k0, int h)
    {
        const int blk = (k0 >> 5) + h;
        r.a = *reinterpret_cast<const uint4 *>(p.p0 + blk * 32);
        r.b = *reinterpret_cast<const uint4 *>(p.p0 + blk * 32 + 16);
        r.d = *reinterpret_cast<const uint16_t *>(p.p1 + blk * 2);
    }
    __device__ __forceinline__ static void convert(const Raw &r, int, int h, _Float16 *dst)
    {
        const float d = h2f(r.d), o = -128.f * d;
        const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        float v0[16], v1[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t qa = q[w] ^ 0x80808080u, qb = q[4 + w] ^ 0x80808080u; // q + 128
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v0[4 * w + i] = __builtin_fmaf(d, ub(qa, i), o);
                v1[4 * w + i] = __builtin_fmaf(d, ub(qb, i), o);
            }
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// Q2_0C (src/quant.rs:2415-2422): value = (2c - 3) * d. The device plane
// keeps a 64-weight unit in 16 bytes with weight 16k+i in bits 2k of byte i;
// half h takes k = 2h and 2h+1 (columns 32h..32h+31).
template <> struct Deq<Q2_0C> {
    struct Raw {
        uint4 c;
        uint32_t d;
    };
    __device__ __forceinline__ static RowPtr rows(const WView &w, int row)
    {
        return row_ptr(w, 128, 2, 0, row);
    }
    __device__ __forceinline__ static void load(Raw &r, const RowPtr &p, int k0, int)
    {
        const int blk = k0 >> 9, u = (k0 >> 6) & 7;
        r.c = *reinterpret_cast<const uint4 *>(p.p0 + blk * 128 + u * 16);
        r.d = *reinterpret_cast<const uint16_t *>(p.p1 + blk * 2);
    }
    __device__ __forceinline__ static void convert(const Raw &r, int, int h, _Float16 *dst)
    {
        const float d = h2f(r.d), d2 = 2.f * d, o = -3.f * d;
        const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        float v0[16], v1[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t x0 = (cw[w] >> (4 * h)) & 0x03030303u;
            const uint32_t x1 = (cw[w] >> (4 * h + 2)) & 0x03030303u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v0[4 * w + i] = __builtin_fmaf(d2, ub(x0, i), o);
                v1[4 * w + i] = __builtin_fmaf(d2, ub(x1, i), o);
            }
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// STQ1_0 (src/quant.rs:1086-1123, 2423-2430): 64-weight chunk c holds 16
// groups; digit p of group gg is column p*16 + gg, value (digit - 1) * d with
// the digit read from the codebook entry of (sign << 4 | nibble). Half h
// takes digits 2h and 2h+1. Device planes as in hyq_internal.hpp: groups
// 4j..4j+3 have their nibbles in bytes of dword j/2 (high nibbles for odd j)
// and their signs at bits (c%2)*4 + j + 8t of the chunk pair's sign dword.
template <> struct Deq<STQ1_0> {
    struct Raw {
        uint2 nib;
        uint32_t s, d;
    };
    __device__ __forceinline__ static RowPtr rows(const WView &w, int row)
    {
        return row_ptr(w, 32, 8, 2, row);
    }
    __device__ __forceinline__ static void load(Raw &r, const RowPtr &p, int k0, int)
    {
        const int blk = k0 >> 8, c = (k0 >> 6) & 3;
        r.nib = *reinterpret_cast<const uint2 *>(p.p0 + blk * 32 + 8 * c);
        r.s = *reinterpret_cast<const uint32_t *>(p.p1 + blk * 8 + 4 * (c >> 1));
        r.d = *reinterpret_cast<const uint16_t *>(p.p2 + blk * 2);
    }
    __device__ __forceinline__ static void convert(const Raw &r, int u, int h, _Float16 *dst)
    {
        const int c = u;
        const float d = h2f(r.d), o = -d;
        const uint32_t nb[2] = {r.nib.x, r.nib.y};
        float v0[16], v1[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t nibs = (nb[j >> 1] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
            const uint32_t sb = ((r.s >> ((c & 1) * 4 + j)) & 0x01010101u) << 4;
            const uint32_t e = GroupSTQ::lut(nibs | sb);
            const uint32_t da = (e >> (4 * h)) & 0x03030303u;
            const uint32_t db = (e >> (4 * h + 2)) & 0x03030303u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v0[4 * j + i] = __builtin_fmaf(d, ub(da, i), o);
                v1[4 * j + i] = __builtin_fmaf(d, ub(db, i), o);
            }
        }
        store16(dst + 32 * h, v0);
        store16(dst + 32 * h + 16, v1);
    }
};

// Zeros for LDS rows past the end of the weight (each half clears 32 columns).
__device__ __forceinline__ void zero_half(_Float16 *dst, int h)
{
    const half8 z = {};
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<half8 *>(dst + 32 * h + 8 * i) = z;
}

// ---------------------------------------------------------------------------
// Activation slice: BN rows (tokens) x 64 f16 columns, 16 bytes per thread
// per load: index f = t + 256 i -> row f/8 = t/8 + 32 i, columns 8*(t%8)...
// xp[i] is the thread's row pointer for load i (offset by its 8 columns),
// nullptr for rows past the end (zeros).
// ---------------------------------------------------------------------------
struct XRaw {
    uint4 v[4];
};

__device__ __forceinline__ void load_x(XRaw &x, const _Float16 *const (&xp)[4], int k0)
{
#pragma unroll
    for (int i = 0; i < 4; ++i)
        x.v[i] = xp[i] ? *reinterpret_cast<const uint4 *>(xp[i] + k0) : make_uint4(0, 0, 0, 0);
}

// NW waves: load i of thread t covers token row t / 8 + 8 NW i.
template <int NW = 4> __device__ __forceinline__ void store_x(_Float16 *Xs, const XRaw &x)
{
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint4 *>(Xs + ((t >> 3) + 8 * NW * i) * LDK + 8 * (t & 7)) = x.v[i];
}

// LDS halves of one operand buffer (weights, then activations) and of the
// two buffers a k_loop of NW waves uses.
template <int NW> constexpr int buf_halves() { return TILE_HALVES + 32 * NW * LDK; }
template <int NW> constexpr int lds_halves() { return 2 * buf_halves<NW>(); }

// One 64-deep step: acc[i][j] accumulates LDS weight rows arow(i) + lane%32
// against tokens wn*64 + 32*j + lane%32, for the wave's first J token
// blocks (the others hold no token of the tile).
template <int J, class ARow>
__device__ __forceinline__ void mma_step(const _Float16 *Ws, const _Float16 *Xs, const ARow &arow,
                                         int wn, f32x16 (&acc)[2][2])
{
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, kq = 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
        half8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[i] = *reinterpret_cast<const half8 *>(Ws + (arow(i) + r) * LDK + kk + kq);
            if (i < J)
                b[i] = *reinterpret_cast<const half8 *>(Xs + (wn * 64 + 32 * i + r) * LDK + kk +
                                                        kq);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < J; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// v_mfma 32x32 output layout: register e of a block holds row
// 8*(e/4) + 4*(lane/32) + e%4 and column lane%32 of the block.
__device__ __forceinline__ int acc_row_in_block(int e)
{
    return 8 * (e >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (e & 3);
}
__device__ __forceinline__ int acc_col(int wn, int j)
{
    return wn * 64 + 32 * j + (threadIdx.x & 31);
}

__device__ __forceinline__ void zero_acc(f32x16 (&acc)[2][2])
{
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
}

// ---------------------------------------------------------------------------
// The K loop shared by every GEMM kernel. wsrc(lrow, view, row) sets the
// weight view and row that LDS row lrow dequantizes (row < 0: zeros);
// xrow(r) gives the f16 activation row of token r of the tile (nullptr =
// zeros); arow(i) the first LDS weight row of the wave's block i. lds holds
// lds_halves<NW>() halves: buffer b at lds + b * buf_halves<NW>(), weights
// then activations. The loop covers columns [kbase, kbase + K) (a K slice
// when kbase > 0; both multiples of the format's block). JM = 1 is the
// variant for tiles of at most 32 tokens (MoE experts): only the first token
// block holds tokens, so the waves with wn = 1 skip their MFMAs and the
// others run one token block.
// ---------------------------------------------------------------------------
template <int F, int JM = 2, int NW = 4, class WSrc, class XRow, class ARow>
__device__ __forceinline__ void k_loop(const WSrc &wsrc, const XRow &xrow, const ARow &arow,
                                       int K, int wn, _Float16 *lds, f32x16 (&acc)[2][2],
                                       int kbase = 0)
{
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    using D = Deq<F>;
    constexpr int BUF = buf_halves<NW>();
    const int t = threadIdx.x;
    // the first 256 threads dequantize the weight slice (a wave-uniform test)
    const bool wthr = NW == 4 || t < 256;
    const int lrow = (t & 255) >> 1, h = t & 1;
    WView wv{};
    int row = -1;
    wsrc(lrow, wv, row);
    const RowPtr rp = D::rows(wv, row < 0 ? 0 : row);
    const _Float16 *xp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const _Float16 *p = xrow((t >> 3) + 8 * NW * i);
        xp[i] = p ? p + 8 * (t & 7) : nullptr;
    }
    typename D::Raw raw;
    XRaw xr;
    auto fetch = [&](int k0) {
        if (wthr && row >= 0) D::load(raw, rp, kbase + k0, h);
        load_x(xr, xp, kbase + k0);
    };
    auto put = [&](int k0, int b) {
        _Float16 *Ws = lds + b * BUF;
        if (wthr) {
            if (row >= 0) D::convert(raw, ((kbase + k0) >> 6) & 3, h, Ws + lrow * LDK);
            else zero_half(Ws + lrow * LDK, h);
        }
        store_x<NW>(Ws + TILE_HALVES, xr);
    };
    const int steps = K / BK;
    const bool mma = JM == 2 || __builtin_amdgcn_readfirstlane(wn) == 0;
    fetch(0);
    put(0, 0);
    if (steps > 1) fetch(BK);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int cur = s & 1;
        const _Float16 *Ws = lds + cur * BUF;
        if (mma) mma_step<JM>(Ws, Ws + TILE_HALVES, arow, wn, acc);
        if (s + 1 < steps) {
            put((s + 1) * BK, cur ^ 1);
            if (s + 2 < steps) fetch((s + 2) * BK);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Producer/consumer form of k_loop for 512 threads (tiles of BM weight rows by
// 256 tokens): waves 0-3 (one per SIMD) fetch and dequantize the weight slice
// as k_loop's first 256 threads do; waves 4-7 (the other wave of each SIMD)
// multiply, each 2 blocks of 32 weight rows (LDS rows arow(0), arow(1) ..
// + 31, a function of the wave) by 128 tokens, wave 4 + c taking tokens
// 128 (c % 2): 2 weight and 4 token fragments per 16-deep step feed 8
// MFMAs (0.75 KB of LDS reads per MFMA against k_loop's 1 KB); all eight
// copy the activation slice as k_loop does (four 16-byte pieces each). Every output
// element sees the same operands in the same k order as in k_loop, so the
// results are bit-identical. acc[i][j]: weight block i, token block j.
// ---------------------------------------------------------------------------
constexpr int PC_THREADS = 512;

template <class ARow>
__device__ __forceinline__ void mma_step_pc(const _Float16 *Ws, const _Float16 *Xs,
                                            const ARow &arow, int wn, f32x16 (&acc)[2][4])
{
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, kq = 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
        half8 a[2], b[4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            a[i] = *reinterpret_cast<const half8 *>(Ws + (arow(i) + r) * LDK + kk + kq);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            b[j] = *reinterpret_cast<const half8 *>(Xs + (wn * 128 + 32 * j + r) * LDK + kk + kq);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

template <int F, class WSrc, class XRow, class ARow>
__device__ __forceinline__ void k_loop_pc(const WSrc &wsrc, const XRow &xrow, const ARow &arow,
                                          int K, _Float16 *lds, f32x16 (&acc)[2][4],
                                          int kbase = 0)
{
    using D = Deq<F>;
    constexpr int BUF = buf_halves<8>();
    const int t = threadIdx.x;
    // waves 0-3 produce, waves 4-7 consume (a wave-uniform test); both copy
    // activation rows: thread t the four rows (t % 256) / 8 + 32 i + 128 (t / 256)
    const bool prod = __builtin_amdgcn_readfirstlane(t) < 256;
    const int lrow = (t & 255) >> 1, h = t & 1;
    const int wn = (t >> 6) & 1;
    WView wv{};
    int row = -1;
    if (prod) wsrc(lrow, wv, row);
    const _Float16 *xp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const _Float16 *p = xrow(((t & 255) >> 3) + 32 * i + 128 * (t >> 8));
        xp[i] = p ? p + 8 * (t & 7) : nullptr;
    }
    const RowPtr rp = D::rows(wv, row < 0 ? 0 : row);
    typename D::Raw raw;
    uint4 xr[4];
    auto fetch_x = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            xr[i] = xp[i] ? *reinterpret_cast<const uint4 *>(xp[i] + kbase + k0)
                          : make_uint4(0, 0, 0, 0);
    };
    auto put_x = [&](int b) {
        _Float16 *Xs = lds + b * BUF + TILE_HALVES;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4 *>(
                Xs + (((t & 255) >> 3) + 32 * i + 128 * (t >> 8)) * LDK + 8 * (t & 7)) = xr[i];
    };
    auto fetch_w = [&](int k0) {
        if (row >= 0) D::load(raw, rp, kbase + k0, h);
    };
    auto put_w = [&](int k0, int b) {
        _Float16 *Ws = lds + b * BUF;
        if (row >= 0) D::convert(raw, ((kbase + k0) >> 6) & 3, h, Ws + lrow * LDK);
        else zero_half(Ws + lrow * LDK, h);
    };
    // Two loops, one per role, each passing the same 1 + steps barriers (a
    // barrier counts waves, whichever instruction they reach it at), so that
    // neither role keeps the other's registers live: the producers' staged
    // weights, the consumers' 128 accumulators.
    const int steps = K / BK;
    if (prod) {
        fetch_w(0);
        fetch_x(0);
        put_w(0, 0);
        put_x(0);
        if (steps > 1) {
            fetch_w(BK);
            fetch_x(BK);
        }
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            if (s + 1 < steps) {
                put_w((s + 1) * BK, (s & 1) ^ 1);
                put_x((s & 1) ^ 1);
                if (s + 2 < steps) {
                    fetch_w((s + 2) * BK);
                    fetch_x((s + 2) * BK);
                }
            }
            __syncthreads();
        }
    } else {
        fetch_x(0);
        put_x(0);
        if (steps > 1) fetch_x(BK);
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            const _Float16 *Ws = lds + (s & 1) * BUF;
            mma_step_pc(Ws, Ws + TILE_HALVES, arow, wn, acc);
            if (s + 1 < steps) {
                put_x((s & 1) ^ 1);
                if (s + 2 < steps) fetch_x((s + 2) * BK);
            }
            __syncthreads();
        }
    }
}

// The producer/consumer loop with the activations, in fragment order
// (launch_to_f16 with frag), taken straight into the consumers' registers (no
// LDS copy): consumer wave 4 + c owns tokens 64 c .. 64 c + 63 of the tile
// against all 32 NI weight rows (NI weight and 2 token fragments per 16-deep
// step feed 2 NI MFMAs), loading its token fragments one step ahead into a
// two-set register ring, each a contiguous KiB (lane l: 8 consecutive k of
// token 32 j + l % 32); LDS holds only the dequantized weights. NI = 4 is
// the 128-row tile; NI = 3 a 96-row tile (producer threads of rows 96-127
// idle), for grids that 128-row tiles would leave short of the CUs.
// xsrc(r): the fragment-order run of the 32-token block of tile token r
// (clamped into the batch: tokens past it produce sums nobody writes). Same
// operands, same k order per element as k_loop: bit-identical results.
// acc[i][j]: weight block i, token block j.
template <int F, int NI, class WSrc, class XSrc>
__device__ __forceinline__ void k_loop_pcx(const WSrc &wsrc, const XSrc &xsrc, int K,
                                           _Float16 *lds, f32x16 (&acc)[NI][2], int kbase = 0)
{
    static_assert(NI == 3 || NI == 4, "96- or 128-row tiles");
    using D = Deq<F>;
    const int t = threadIdx.x;
    const bool prod = __builtin_amdgcn_readfirstlane(t) < 256;
    const int steps = K / BK;
    if (prod) {
        const int lrow = t >> 1, h = t & 1;
        const bool used = lrow < 32 * NI;
        WView wv{};
        int row = -1;
        if (used) wsrc(lrow, wv, row);
        const RowPtr rp = D::rows(wv, row < 0 ? 0 : row);
        typename D::Raw raw;
        auto fetch = [&](int k0) {
            if (row >= 0) D::load(raw, rp, kbase + k0, h);
        };
        auto put = [&](int k0, int b) {
            _Float16 *Ws = lds + b * TILE_HALVES + lrow * LDK;
            if (row >= 0) D::convert(raw, ((kbase + k0) >> 6) & 3, h, Ws);
            else if (used) zero_half(Ws, h);
        };
        fetch(0);
        put(0, 0);
        if (steps > 1) fetch(BK);
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            if (s + 1 < steps) {
                put((s + 1) * BK, (s & 1) ^ 1);
                if (s + 2 < steps) fetch((s + 2) * BK);
            }
            __syncthreads();
        }
        return;
    }
    const int lane = t & 63, c = (t >> 6) & 3;
    const int r = lane & 31, kq = 8 * (lane >> 5);
    // lane l's 8 halves of 16-deep step b in the block's fragment-order run
    const _Float16 *xb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) xb[j] = xsrc(64 * c + 32 * j) + (size_t)(kbase / 16) * 512 + lane * 8;
    half8 B0[4][2], B1[4][2];
    auto loadB = [&](half8 (&b)[4][2], int k0) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[kk][j] = *reinterpret_cast<const half8 *>(xb[j] + (size_t)(k0 / 16 + kk) * 512);
    };
    auto mma = [&](const _Float16 *Ws, const half8 (&b)[4][2]) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            half8 a[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i)
                a[i] = *reinterpret_cast<const half8 *>(Ws + (32 * i + r) * LDK + 16 * kk + kq);
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[kk][j], acc[i][j], 0, 0, 0);
        }
    };
    loadB(B0, 0);
    __syncthreads();
    for (int s = 0; s < steps; s += 2) {
        if (s + 1 < steps) loadB(B1, (s + 1) * BK);
        mma(lds, B0);
        __syncthreads();
        if (s + 1 < steps) {
            if (s + 2 < steps) loadB(B0, (s + 2) * BK);
            mma(lds + TILE_HALVES, B1);
            __syncthreads();
        }
    }
}

} // namespace tile
} // namespace hyq
