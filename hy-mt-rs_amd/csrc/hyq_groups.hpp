// Per-format group kernels of the int8 GEMV on gfx950.
//
// One lane owns one 256-weight group of one row at a time: it loads the
// group's planes with 16-byte loads, expands the codes to int8 bytes in
// registers and accumulates v_dot4_i32_i8 products against 64 dwords of Q8
// activations held in registers. Code offsets (Q2_0C's 2c-3, STQ's code-1,
// Q6_K's q-32, Q4_K's mins) are folded into one multiply by a precomputed
// activation sum instead of being applied per weight.
//
// Each `dot` returns the group's f32 contribution and, when EMIT is set,
// writes the group's integer block sums in the granularity the reference's
// SDOT kernels accumulate them (see hyq.h, hyq_gemv_isums_d). The Q8 words a
// group's dot reads besides the codes (the group scale and the integer sums
// the format folds its offsets with) come through an accessor object: a
// format's `Meta`, loaded into registers by `meta` (so that a kernel can
// issue those loads with the group's weights), or a `Q8At`, which reads
// them where they lie at the dot (the LDS copies of an input stage).
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"

namespace hyq {

__device__ __forceinline__ float h2f(uint16_t b)
{
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ int sdot4(uint32_t a, int b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

// A group's loaded words are passed through an empty volatile asm at the
// top of `dot`, so that no arithmetic on them (f16 scale conversion, scale
// unpacking) is hoisted to the load: a load issued under a condition would
// otherwise be followed at once by its conversion, and the wave would wait
// there for that load and every load issued before it instead of letting
// them complete behind the input stage.
__device__ __forceinline__ void hold(uint32_t &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void hold(uint4 &v)
{
    hold(v.x);
    hold(v.y);
    hold(v.z);
    hold(v.w);
}
__device__ __forceinline__ void hold(uint2 &v)
{
    hold(v.x);
    hold(v.y);
}
__device__ __forceinline__ void hold(uint16_t &v)
{
    uint32_t t = v;
    hold(t);
    v = (uint16_t)t;
}

// ---------------------------------------------------------------------------
// Q2_0C: 512-weight blocks, two 256-weight groups (halves) per block.
// isum_half = sum (2c-3) q = 2 sum c q - 3 sum q   (src/quant.rs:1891-1951)
// contribution = f32(isum) * (d * s_g)             (src/quant.rs:1896,1922)
// ---------------------------------------------------------------------------
// The Q8 integer sums a format's dot reads (QSUMS: a mask of these).
constexpr int Q8_SUM256 = 1, Q8_SUM16 = 2, Q8_SUM32 = 4;

// Group g's Q8 words, read at each use.
struct Q8At {
    Q8View x;
    int g;
    __device__ __forceinline__ float scale() const { return x.s[g]; }
    __device__ __forceinline__ int sum256() const { return x.sum256[g]; }
    __device__ __forceinline__ int sum16(int k) const { return x.sum16[16 * g + k]; }
    __device__ __forceinline__ int sum32(int j) const { return x.sum32[8 * g + j]; }
};

struct GroupQ2C {
    // sum c q over U 16-byte code units: byte b of unit dword m holds codes
    // k = 0..3 (bits 2k, 2k + 1) of weights 64 u + 16 k + 4 m + b. The codes
    // are dotted at their place values (code k as 4^k c for k < 3, and k = 3
    // via one shift as 16 c, so every byte stays below 64) into three
    // accumulators, each an exact multiple of its place value.
    template <int U>
    __device__ __forceinline__ static int code_dot(const uint4 *w, const int *act)
    {
        int r0 = 0, r1 = 0, r23 = 0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t c[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                r0 = sdot4(c[m] & 0x03030303u, act[16 * u + m], r0);
                r1 = sdot4(c[m] & 0x0C0C0C0Cu, act[16 * u + 4 + m], r1);
                r23 = sdot4(c[m] & 0x30303030u, act[16 * u + 8 + m], r23);
                r23 = sdot4((c[m] >> 2) & 0x30303030u, act[16 * u + 12 + m], r23);
            }
        }
        return (r0 + (r1 >> 2)) + (r23 >> 4);
    }
    static constexpr int ISUMS = 1;
    static constexpr int QSUMS = Q8_SUM256 | Q8_SUM32; // full / half-group dots
    struct Meta {
        float s;
        int s256;
        __device__ __forceinline__ float scale() const { return s; }
        __device__ __forceinline__ int sum256() const { return s256; }
    };
    __device__ __forceinline__ static Meta meta(const Q8View &x, int g)
    {
        return Meta{x.s[g], x.sum256[g]};
    }
    struct Data {
        uint4 w[4];
        uint16_t d;
        __device__ __forceinline__ void hold_all()
        {
#pragma unroll
            for (int u = 0; u < 4; ++u) hold(w[u]);
            hold(d);
        }
    };
    __device__ __forceinline__ static void load(Data &D, const WView &w, int row, int g)
    {
        size_t blk = (size_t)row * w.nb + (g >> 1);
        const uint4 *p = reinterpret_cast<const uint4 *>(w.p0 + blk * 128 + (g & 1) * 64);
#pragma unroll
        for (int u = 0; u < 4; ++u) D.w[u] = p[u];
        D.d = reinterpret_cast<const uint16_t *>(w.p1)[blk];
    }
    template <bool EMIT, class M>
    __device__ __forceinline__ static float dot(const Data &Din, const int *act, const M &x,
                                                int32_t *out)
    {
        Data D = Din;
        D.hold_all();
        const int raw = code_dot<4>(D.w, act);
        int isum = 2 * raw - 3 * x.sum256();
        if (EMIT) out[0] = isum;
        return (float)isum * (h2f(D.d) * x.scale());
    }

    // Half of a group (weights 128h .. 128h + 127: code units 2h, 2h + 1) for
    // the GEMV that gives each 256-weight group to two lanes. A half's
    // integer sum 2 sum(c q) - 3 sum(q) over its 128 values adds exactly to
    // the group's, so the two halves' sums are added (as integers) before
    // the one float product of `finish`, which is the whole group's.
    struct Half {
        uint4 w[2];
        uint16_t d;
        __device__ __forceinline__ void hold_all()
        {
            hold(w[0]);
            hold(w[1]);
            hold(d);
        }
    };
    __device__ __forceinline__ static void load_half(Half &D, const WView &w, int row, int g,
                                                     int h)
    {
        size_t blk = (size_t)row * w.nb + (g >> 1);
        const uint4 *p = reinterpret_cast<const uint4 *>(w.p0 + blk * 128 + (g & 1) * 64);
        D.w[0] = p[2 * h];
        D.w[1] = p[2 * h + 1];
        D.d = reinterpret_cast<const uint16_t *>(w.p1)[blk];
    }
    // act: the half's 32 activation dwords (values 128h .. 128h + 127)
    __device__ __forceinline__ static int isum_half(const Half &Din, const int *act,
                                                    const Q8View &x, int g, int h)
    {
        Half D = Din;
        D.hold_all();
        const int raw = code_dot<2>(D.w, act);
        const int *s32 = x.sum32 + g * 8 + 4 * h;
        return 2 * raw - 3 * ((s32[0] + s32[1]) + (s32[2] + s32[3]));
    }
    // acc + f32(isum) * (d * s_g) as one fused multiply-add, the form both
    // GEMV modes accumulate groups in
    __device__ __forceinline__ static float finish_acc(float acc, int isum, uint16_t d,
                                                       const Q8View &x, int g)
    {
        return fmaf(h2f(d) * x.s[g], (float)isum, acc);
    }
    template <class M>
    __device__ __forceinline__ static float dot_acc(float acc, const Data &Din, const int *act,
                                                    const M &x)
    {
        Data D = Din;
        D.hold_all();
        const int raw = code_dot<4>(D.w, act);
        return fmaf(h2f(D.d) * x.scale(), (float)(2 * raw - 3 * x.sum256()), acc);
    }
};

// ---------------------------------------------------------------------------
// STQ1_0: 256-weight blocks of 64 groups of 4 ternary digits (codebook).
// isum_block = sum digit q = sum code q - sum q      (src/quant.rs:1511-1556)
// contribution = f32(isum) * (d * s_g)               (src/quant.rs:1512,1555)
// ---------------------------------------------------------------------------
struct GroupSTQ {
    static constexpr int ISUMS = 1;
    static constexpr int QSUMS = Q8_SUM256;
    struct Meta {
        float s;
        int s256;
        __device__ __forceinline__ float scale() const { return s; }
        __device__ __forceinline__ int sum256() const { return s256; }
    };
    __device__ __forceinline__ static Meta meta(const Q8View &x, int g)
    {
        return Meta{x.s[g], x.sum256[g]};
    }
    struct Data {
        uint4 nib[2];
        uint2 sgn;
        uint16_t d;
        __device__ __forceinline__ void hold_all()
        {
            hold(nib[0]);
            hold(nib[1]);
            hold(sgn);
            hold(d);
        }
    };
    __device__ __forceinline__ static void load(Data &D, const WView &w, int row, int g)
    {
        size_t blk = (size_t)row * w.nb + g;
        const uint4 *p = reinterpret_cast<const uint4 *>(w.p0 + blk * 32);
        D.nib[0] = p[0];
        D.nib[1] = p[1];
        D.sgn = reinterpret_cast<const uint2 *>(w.p1)[blk];
        D.d = reinterpret_cast<const uint16_t *>(w.p2)[blk];
    }
    // 0xFF in each byte whose bit 7 is set, else 0x00: v_perm_b32 selectors
    // 8, 9, 10, 11 replicate bit 7 of bytes 1, 3, 5, 7 of {first, second};
    // with second = v << 8 those are v's bytes 0, 2 and first's 1, 3.
    __device__ __forceinline__ static uint32_t byte_mask(uint32_t v)
    {
        return __builtin_amdgcn_perm(v, v << 8, 0x0B090A08u);
    }
    // Codebook bytes of four groups: nibbles nb (one per byte, 0..15) and a
    // per-byte sign mask ms. STQ_CODEBOOK (src/quant.rs:1081-1084) holds 2-bit
    // digit codes (0..2, digit = code - 1); each of its sign-1 entries is the
    // sign-0 entry of the same nibble with every code c replaced by 2 - c
    // (the digits negated), i.e. the byte 0xAA - e, so only the 16 sign-0
    // entries are looked up (packed 4 per dword, little endian; v_perm_b32
    // selects bytes 0-3 from its second operand and 4-7 from its first) and
    // the sign picks e or 0xAA - e per byte (no borrows: every code is <= 2).
    __device__ __forceinline__ static uint32_t codes(uint32_t nb, uint32_t ms)
    {
        return codes_sel(nb & 0x07070707u, byte_mask(nb << 4), ms);
    }
    // The same from the nibbles' low three bits (sel, one per byte) and the
    // 0xFF / 0x00 byte mask of their bit 3 (m3).
    __device__ __forceinline__ static uint32_t codes_sel(uint32_t sel, uint32_t m3, uint32_t ms)
    {
        constexpr uint32_t CB0 = 0x092989a9u, CB1 = 0x062686a6u, CB2 = 0x121a929au,
                           CB3 = 0x424a626au;
        const uint32_t r0 = __builtin_amdgcn_perm(CB1, CB0, sel);
        const uint32_t r1 = __builtin_amdgcn_perm(CB3, CB2, sel);
        const uint32_t e = (r1 & m3) | (r0 & ~m3);
        const uint32_t en = 0xAAAAAAAAu - e;
        return (en & ms) | (e & ~ms);
    }
    // The codebook bytes of the four groups of nibble dword dw (its low
    // nibbles, or with hi its high ones) with sign bit q of each byte of S:
    // the low three bits select from the sign-0 entries 0-7 and 8-15 (two
    // v_perm_b32), and each of the two remaining choices (bit 3: the upper
    // entries; the sign: 0xAA - e) is a v_perm_b32 between two candidate
    // dwords whose selector is kb = 0x03020100 plus 4 in every byte whose bit
    // is set (byte b of the first source or of the second).
    __device__ __forceinline__ static uint32_t codes_perm(uint32_t dw, int hi, uint32_t S, int q,
                                                          uint32_t kb)
    {
        constexpr uint32_t CB0 = 0x092989a9u, CB1 = 0x062686a6u, CB2 = 0x121a929au,
                           CB3 = 0x424a626au;
        const uint32_t sel = hi ? (dw >> 4) & 0x07070707u : dw & 0x07070707u;
        const uint32_t s3 = ((hi ? dw >> 5 : dw >> 1) & 0x04040404u) | kb;
        const uint32_t ss = ((q >= 2 ? S >> (q - 2) : S << (2 - q)) & 0x04040404u) | kb;
        const uint32_t r0 = __builtin_amdgcn_perm(CB1, CB0, sel);
        const uint32_t r1 = __builtin_amdgcn_perm(CB3, CB2, sel);
        const uint32_t e = __builtin_amdgcn_perm(r1, r0, s3);
        return __builtin_amdgcn_perm(0xAAAAAAAAu - e, e, ss);
    }
    // 5-bit index bytes (sign<<4 | nibble) -> codebook bytes, four at a time.
    __device__ __forceinline__ static uint32_t lut(uint32_t idx)
    {
        return codes(idx & 0x0F0F0F0Fu, byte_mask(idx << 3));
    }
    template <bool EMIT, class M>
    __device__ __forceinline__ static float dot(const Data &Din, const int *act, const M &x,
                                                int32_t *out)
    {
        Data D = Din;
        D.hold_all();
        const uint32_t nib[8] = {D.nib[0].x, D.nib[0].y, D.nib[0].z, D.nib[0].w,
                                 D.nib[1].x, D.nib[1].y, D.nib[1].z, D.nib[1].w};
        const uint32_t sg[2] = {D.sgn.x, D.sgn.y};
        // The four 2-bit codes of each codebook byte are dotted at their
        // place values (code p as 4^p code, bytes at most 48, for p = 3 via
        // one shift: 16 code) into four accumulators, each then an exact
        // multiple of its place value.
        int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
        // (the byte-select base in a register, so that each selector is one
        // v_and_or_b32)
        uint32_t kb = 0x03020100u;
        asm volatile("" : "+v"(kb));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int qi = 0; qi < 4; ++qi) {
                const uint32_t dw = nib[2 * c + (qi >> 1)];
                const int q = (c & 1) * 4 + qi; // quad index inside the sign dword
                const uint32_t e = codes_perm(dw, qi & 1, sg[c >> 1], q, kb);
                const int *a = act + 16 * c + qi;
                r0 = sdot4(e & 0x03030303u, a[0], r0);
                r1 = sdot4(e & 0x0C0C0C0Cu, a[4], r1);
                r2 = sdot4(e & 0x30303030u, a[8], r2);
                r3 = sdot4((e >> 2) & 0x30303030u, a[12], r3);
            }
        }
        const int raw = (r0 + (r1 >> 2)) + ((r2 + r3) >> 4);
        int isum = raw - x.sum256();
        if (EMIT) out[0] = isum;
        return (float)isum * (h2f(D.d) * x.scale());
    }
};

// ---------------------------------------------------------------------------
// Q4_K: 256-weight superblocks, 8 sub-blocks of 32 with 6-bit scale s_j and
// min m_j (src/quant.rs:2437-2461). Integer form (no reference int path):
//   A = sum_j s_j * sum(q * a),  B = sum_j m_j * sum(a)
//   contribution = s_g * (d * f32(A) - dmin * f32(B))
// which equals the decoder's d*s_j*q - dmin*m_j dotted with the Q8 values.
// ---------------------------------------------------------------------------
struct GroupQ4K {
    static constexpr int ISUMS = 2;
    static constexpr int QSUMS = Q8_SUM32;
    struct Meta {
        float s;
        int s32[8];
        __device__ __forceinline__ float scale() const { return s; }
        __device__ __forceinline__ int sum32(int j) const { return s32[j]; }
    };
    __device__ __forceinline__ static Meta meta(const Q8View &x, int g)
    {
        Meta m;
        m.s = x.s[g];
#pragma unroll
        for (int j = 0; j < 8; ++j) m.s32[j] = x.sum32[8 * g + j];
        return m;
    }
    struct Data {
        uint4 qs[8];
        uint4 meta;
        __device__ __forceinline__ void hold_all()
        {
#pragma unroll
            for (int i = 0; i < 8; ++i) hold(qs[i]);
            hold(meta);
        }
    };
    __device__ __forceinline__ static void load(Data &D, const WView &w, int row, int g)
    {
        size_t blk = (size_t)row * w.nb + g;
        const uint4 *p = reinterpret_cast<const uint4 *>(w.p0 + blk * 128);
#pragma unroll
        for (int i = 0; i < 8; ++i) D.qs[i] = p[i];
        D.meta = reinterpret_cast<const uint4 *>(w.p1)[blk];
    }
    template <bool EMIT, class M>
    __device__ __forceinline__ static float dot(const Data &Din, const int *act, const M &x,
                                                int32_t *out)
    {
        Data D = Din;
        D.hold_all();
        uint32_t q[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            q[4 * i] = D.qs[i].x;
            q[4 * i + 1] = D.qs[i].y;
            q[4 * i + 2] = D.qs[i].z;
            q[4 * i + 3] = D.qs[i].w;
        }
        const uint32_t m0 = D.meta.x, m1 = D.meta.y, m2 = D.meta.z, m3 = D.meta.w;
        const uint8_t sc[12] = {
            (uint8_t)m1,         (uint8_t)(m1 >> 8),  (uint8_t)(m1 >> 16), (uint8_t)(m1 >> 24),
            (uint8_t)m2,         (uint8_t)(m2 >> 8),  (uint8_t)(m2 >> 16), (uint8_t)(m2 >> 24),
            (uint8_t)m3,         (uint8_t)(m3 >> 8),  (uint8_t)(m3 >> 16), (uint8_t)(m3 >> 24)};
        int A = 0, B = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int s, m;
            if (j < 4) {
                s = sc[j] & 63;
                m = sc[j + 4] & 63;
            } else {
                s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
                m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
            }
            const int grp = j >> 1, hi = j & 1;
            int qx = 0;
#pragma unroll
            for (int i4 = 0; i4 < 8; ++i4) {
                const uint32_t dw = q[8 * grp + i4];
                const uint32_t nb = hi ? (dw >> 4) & 0x0F0F0F0Fu : dw & 0x0F0F0F0Fu;
                qx = sdot4(nb, act[16 * grp + 8 * hi + i4], qx);
            }
            A += s * qx;
            B += m * x.sum32(j);
        }
        if (EMIT) {
            out[0] = A;
            out[1] = B;
        }
        const float d = h2f((uint16_t)m0), dmin = h2f((uint16_t)(m0 >> 16));
        return x.scale() * (d * (float)A - dmin * (float)B);
    }
};

// ---------------------------------------------------------------------------
// Q6_K: 256-weight blocks, 16 planes of 16 weights with int8 sub-scales.
// isum_plane = sum (q6 - 32) a = sum q6 a - 32 sum a  (src/quant.rs:2257-2330)
// contribution = sum_k f32(isum_k) * ((d * s_g) * sc_k)   (src/quant.rs:2258,2281)
// ---------------------------------------------------------------------------
struct GroupQ6K {
    static constexpr int ISUMS = 16;
    static constexpr int QSUMS = Q8_SUM16;
    struct Meta {
        float s;
        int s16[16];
        __device__ __forceinline__ float scale() const { return s; }
        __device__ __forceinline__ int sum16(int k) const { return s16[k]; }
    };
    __device__ __forceinline__ static Meta meta(const Q8View &x, int g)
    {
        Meta m;
        m.s = x.s[g];
#pragma unroll
        for (int k = 0; k < 16; ++k) m.s16[k] = x.sum16[16 * g + k];
        return m;
    }
    struct Data {
        uint4 q[12];
        uint4 sc;
        uint16_t d;
        __device__ __forceinline__ void hold_all()
        {
#pragma unroll
            for (int i = 0; i < 12; ++i) hold(q[i]);
            hold(sc);
            hold(d);
        }
    };
    __device__ __forceinline__ static void load(Data &D, const WView &w, int row, int g)
    {
        size_t blk = (size_t)row * w.nb + g;
        const uint4 *p = reinterpret_cast<const uint4 *>(w.p0 + blk * 192);
#pragma unroll
        for (int i = 0; i < 12; ++i) D.q[i] = p[i];
        D.sc = reinterpret_cast<const uint4 *>(w.p1)[blk];
        D.d = reinterpret_cast<const uint16_t *>(w.p2)[blk];
    }
    template <bool EMIT, class M>
    __device__ __forceinline__ static float dot(const Data &Din, const int *act, const M &x,
                                                int32_t *out)
    {
        Data D = Din;
        D.hold_all();
        uint32_t v[48];
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            v[4 * i] = D.q[i].x;
            v[4 * i + 1] = D.q[i].y;
            v[4 * i + 2] = D.q[i].z;
            v[4 * i + 3] = D.q[i].w;
        }
        const uint32_t *ql = v;      // 32 dwords
        const uint32_t *qh = v + 32; // 16 dwords
        const uint32_t scw[4] = {D.sc.x, D.sc.y, D.sc.z, D.sc.w};
        const float dd = h2f(D.d) * x.scale();
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const uint32_t L0 = ql[16 * c + 4 * h + i4];
                    const uint32_t L1 = ql[16 * c + 8 + 4 * h + i4];
                    const uint32_t H = qh[8 * c + 4 * h + i4];
                    const uint32_t q0 = (L0 & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
                    const uint32_t q1 = (L1 & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
                    const uint32_t q2 = ((L0 >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
                    const uint32_t q3 = ((L1 >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
                    r0 = sdot4(q0, act[32 * c + 0 + 4 * h + i4], r0);
                    r1 = sdot4(q1, act[32 * c + 8 + 4 * h + i4], r1);
                    r2 = sdot4(q2, act[32 * c + 16 + 4 * h + i4], r2);
                    r3 = sdot4(q3, act[32 * c + 24 + 4 * h + i4], r3);
                }
                const int rr[4] = {r0, r1, r2, r3};
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int k = 8 * c + 2 * p + h; // plane = sub-scale index
                    const int isum = rr[p] - 32 * x.sum16(k);
                    if (EMIT) out[k] = isum;
                    const int8_t s8 = (int8_t)(scw[k >> 2] >> (8 * (k & 3)));
                    acc += (float)isum * (dd * (float)s8);
                }
            }
        }
        return acc;
    }
};

// ---------------------------------------------------------------------------
// Q8_0: 32-weight blocks, eight per 256-weight group (no reference int path):
// isum_b = sum qw q;  contribution = sum_b f32(isum_b) * (d_b * s_g)
// ---------------------------------------------------------------------------
struct GroupQ80 {
    static constexpr int ISUMS = 8;
    static constexpr int QSUMS = 0;
    struct Meta {
        float s;
        __device__ __forceinline__ float scale() const { return s; }
    };
    __device__ __forceinline__ static Meta meta(const Q8View &x, int g) { return Meta{x.s[g]}; }
    struct Data {
        uint4 q[16];
        uint4 d;
        __device__ __forceinline__ void hold_all()
        {
#pragma unroll
            for (int i = 0; i < 16; ++i) hold(q[i]);
            hold(d);
        }
    };
    __device__ __forceinline__ static void load(Data &D, const WView &w, int row, int g)
    {
        size_t blk = (size_t)row * w.nb + 8 * g;
        const uint4 *p = reinterpret_cast<const uint4 *>(w.p0 + blk * 32);
#pragma unroll
        for (int i = 0; i < 16; ++i) D.q[i] = p[i];
        D.d = *reinterpret_cast<const uint4 *>(w.p1 + blk * 2);
    }
    template <bool EMIT, class M>
    __device__ __forceinline__ static float dot(const Data &Din, const int *act, const M &x,
                                                int32_t *out)
    {
        Data D = Din;
        D.hold_all();
        const uint32_t dw[4] = {D.d.x, D.d.y, D.d.z, D.d.w};
        const float sg = x.scale();
        float acc = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint4 a = D.q[2 * b], c = D.q[2 * b + 1];
            int r = 0;
            r = sdot4(a.x, act[8 * b + 0], r);
            r = sdot4(a.y, act[8 * b + 1], r);
            r = sdot4(a.z, act[8 * b + 2], r);
            r = sdot4(a.w, act[8 * b + 3], r);
            r = sdot4(c.x, act[8 * b + 4], r);
            r = sdot4(c.y, act[8 * b + 5], r);
            r = sdot4(c.z, act[8 * b + 6], r);
            r = sdot4(c.w, act[8 * b + 7], r);
            if (EMIT) out[b] = r;
            const float d = h2f((uint16_t)(dw[b >> 1] >> (16 * (b & 1))));
            acc += (float)r * (d * sg);
        }
        return acc;
    }
};

template <int F> struct GroupOf;
// Formats whose GEMV can give each group to two lanes (GroupX::Half).
template <int F> struct HasHalf { static constexpr bool value = false; };
template <> struct HasHalf<Q2_0C> { static constexpr bool value = true; };
template <class G, bool H> struct GemvData { using T = typename G::Data; };
template <class G> struct GemvData<G, true> { using T = typename G::Half; };
template <> struct GroupOf<Q2_0C> { using T = GroupQ2C; };
template <> struct GroupOf<STQ1_0> { using T = GroupSTQ; };
template <> struct GroupOf<Q4_K> { using T = GroupQ4K; };
template <> struct GroupOf<Q6_K> { using T = GroupQ6K; };
template <> struct GroupOf<Q8_0> { using T = GroupQ80; };

} // namespace hyq
