// Few-token MoE expert products for Q4_K experts: Moe::forward's expert loop
// (src/model.rs:699-725), each expert's DenseFfn::forward (src/model.rs:
// 673-684) at batch = the expert's token count, when the routed pairs average
// at most 16 tokens per expert. There the products are bound by reading the
// expert weights, so the weights go from HBM straight into MFMA operands in
// registers: no LDS stage, no barrier, every wave independent.
//
// Arithmetic. A Q4_K weight is (d*sc_s)*q - dmin*m_s (decode_unchecked,
// src/quant.rs:2437-2461). Per 256-weight superblock and 16x16 (rows x tokens)
// tile a wave forms
//   P = sum_k (sc_s(k) * q_k) * x_k      on v_mfma_f32_16x16x32_f16 (8 steps)
//   M = sum_s (16 m_s) * (X_s / 16)      on v_mfma_f32_16x16x16_f16 (1 step)
// where X_s sums the activations of 32-weight sub-block s (in two 16-weight
// halves, one per lane group); sc*q <= 945 and 16 m <= 1008 are integers
// exact in f16, and f16 products are exact in the f32 accumulation. The
// accumulator then takes d*P - dmin*M in f32. The weights thus enter exactly;
// the activations enter as f16 with a power-of-two scale per token column (as
// in the LDS-tiled GEMM), the half-sums X / 16 as f16.
//
// Weight operand. Lane l holds weight row l % 16 of the tile; with g = l / 16
// it loads qs bytes 16g..16g+15 (chunk g/2 of the superblock, sub-blocks
// g & ~1, (g & ~1) + 1) and 64+16g..64+16g+15 (chunk 2 + g/2), so each load
// instruction reads the first or second 64 bytes of 16 rows. MFMA step t
// takes dword t of the pair: its bytes b0..b3 hold chunk weights o+0..3 (low
// nibbles) and 32+o+0..3 (high nibbles). (w & 0x000F000F) | 0x64006400 is the
// f16 pair (1024 + q(b0), 1024 + q(b2)), and one v_pk_fma_f16 with
// (sc, -1024 sc) leaves (sc q(b0), sc q(b2)) exactly; (w & 0x00F000F0) |
// 0x64006400 = (1024 + 16 q'(b0), ...) takes (sc'/16, -64 sc'); w >> 8 gives
// b1 and b3 the same way.
//
// Activation operand (chunk_q4k_kernel). Per 16-token chunk, superblock b and
// step t, 64 lanes x 16 bytes in lane order (lane = 16 g + column), so one
// load instruction reads 1 KiB of consecutive bytes. Lane (g, col)'s 8 halves
// for step t are x(a), x(a+2), x(a+1), x(a+3), x(a+32), x(a+34), x(a+33),
// x(a+35) of token col with a = 256 b + 64 c + o, c = g/2 (+ 2 for t >= 4),
// o = 16 (g & 1) + 4 (t & 3): the A and B lanes of an MFMA pair the same k.
// The activations are the MFMA's A operand, the weights its B operand: output
// lane l holds tokens 4 (l / 16) + i, i = 0..3, of weight row l % 16, the row
// whose d and dmin the lane loaded.
#include <hip/hip_runtime.h>

#include "hyq_f16rows.hpp"
#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

#pragma clang fp contract(off)

namespace hyq {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int CHUNK = 16; // tokens per expert chunk (one MFMA column block)

__device__ __forceinline__ float half_bits(uint32_t b)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ float silu_mul(float g, float u)
{
    // (g / (1 + exp(-g))) * u, DenseFfn::forward (src/model.rs:680-682)
    return (g / (1.0f + expf(-g))) * u;
}

// One row tile's superblock: the lane's two 16-byte qs pieces and the
// 16-byte header (d | dmin << 16, scales[12]).
struct WRaw {
    uint4 q0, q1, meta;
};
// One token column's superblock operand: 8 MFMA steps and the four half-sums.
struct XRaw {
    uint4 v[8];
    uint2 m;
};

__device__ __forceinline__ uint32_t dword(const uint4 &v, int i)
{
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ h2 pair_bits(uint32_t b) { return __builtin_bit_cast(h2, b); }

__device__ __forceinline__ _Float16 f16i(uint32_t v, float scale)
{
    return (_Float16)(scale * (float)v);
}

// acc += d * P - dmin * M for one superblock of one row tile. `magic` holds
// 0x64006400 in a VGPR, so each nibble pair is one v_and_or_b32 (whose mask
// then takes the one scalar operand gfx9's VOP3 allows). The activations are
// the MFMA's A operand and the weights its B operand, so output lane l holds
// tokens 4 (l / 16) + i of weight row l % 16: the lane's own row, whose d and
// dmin it loaded.
__device__ __forceinline__ void superblock(const WRaw &w, const XRaw &x, int g, uint32_t magic,
                                           f4 &acc)
{
    // 6-bit scales and mins (get_scale_min_k4) of sub-blocks 2c, 2c+1 (low
    // form: low six bits of scales[s], scales[s+4]) and 2c+4, 2c+5 (high form:
    // a nibble of scales[s+4] with the top two bits of scales[s-4] /
    // scales[s]), c = g / 2, as bytes 0 and 1 of each word; then as f16 pairs
    // through the same 1024 + v trick (v <= 63 is exact).
    const int sh = 16 * (g >> 1);
    const uint32_t Y = w.meta.y >> sh, Z = w.meta.z >> sh, W = w.meta.w >> sh;
    const uint32_t sl = Y & 0x3f3fu, ml = Z & 0x3f3fu;
    const uint32_t sh4 = (W & 0x0f0fu) | ((Y >> 2) & 0x3030u);
    const uint32_t mh4 = ((W >> 4) & 0x0f0fu) | ((Z >> 2) & 0x3030u);
    const h2 k1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    auto pair16 = [&](uint32_t v) { // bytes 0, 1 of v as an exact f16 pair
        return pair_bits(__builtin_amdgcn_perm(0u, v, 0x0c010c00u) | magic) + k1024;
    };
    const h2 lo_mul = {(_Float16)1.f, (_Float16)0.0625f}, lo_add = {(_Float16)-1024.f, (_Float16)-64.f};
    h2 K1[2], K2[2]; // (sc_a, sc_b / 16) and (-1024 sc_a, -64 sc_b) of each sub-block pair
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const h2 sc = pair16(p == 0 ? sl : sh4);
        K1[p] = sc * lo_mul;
        K2[p] = sc * lo_add;
    }
    f4 P = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int p = t >> 2;
        const uint32_t q = dword(p == 0 ? w.q0 : w.q1, t & 3), q8 = q >> 8;
        const h2 S0 = {K1[p].x, K1[p].x}, B0 = {K2[p].x, K2[p].x};
        const h2 S1 = {K1[p].y, K1[p].y}, B1 = {K2[p].y, K2[p].y};
        const h2 a0 = __builtin_elementwise_fma(pair_bits((q & 0x000F000Fu) | magic), S0, B0);
        const h2 a1 = __builtin_elementwise_fma(pair_bits((q8 & 0x000F000Fu) | magic), S0, B0);
        const h2 a2 = __builtin_elementwise_fma(pair_bits((q & 0x00F000F0u) | magic), S1, B1);
        const h2 a3 = __builtin_elementwise_fma(pair_bits((q8 & 0x00F000F0u) | magic), S1, B1);
        const h8 Wt = {a0.x, a0.y, a1.x, a1.y, a2.x, a2.y, a3.x, a3.y};
        P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, x.v[t]), Wt, P, 0, 0, 0);
    }
    const h2 k16 = {(_Float16)16.f, (_Float16)16.f};
    const h2 m0 = pair16(ml) * k16, m1 = pair16(mh4) * k16;
    const h4 Am = {m0.x, m0.y, m1.x, m1.y};
    const f4 M = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, x.m), Am,
                                                       f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    const float d = half_bits(w.meta.x & 0xffffu), dmin = half_bits(w.meta.x >> 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc[i] = __builtin_fmaf(d, P[i], acc[i]);
        acc[i] = __builtin_fmaf(-dmin, M[i], acc[i]);
    }
}

// One superblock of a chunk's activation operand in LDS: 8 MFMA steps x 64
// lanes x 16 bytes, and 64 lanes x 8 bytes of half-sums.
struct XLds {
    uint4 v[8 * 64];
    uint2 m[64];
};

// R row tiles (rows[r] = the tile's first weight row, 16 rows each, of
// matrices w[r]) against one chunk's activation operand (xc, xmc at the
// chunk) over K: acc[r]. Called by all 256 threads of the workgroup (it holds
// barriers); the four waves share the activation operand, which the
// workgroup stages through LDS one superblock ahead (xs[2]), while each wave
// streams its weights one superblock ahead in two register sets. Loads
// return in issue order, so each iteration issues the activation loads of
// superblock b+1 before the weight prefetch of b+1: the compute of b waits
// for neither, and the LDS store at the end of b waits only for the former.
// sched_barrier keeps the compiler from moving loads across those points.
// Every load is unconditional (the last prefetch re-reads superblock nbk-1,
// an L2 hit).
template <int R>
__device__ __forceinline__ void tile_rows(const WView *w, const int *rows, int K,
                                          const _Float16 *xc, const _Float16 *xmc, XLds *xs,
                                          f4 *acc)
{
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, rr = lane & 15;
    const int nbk = K / 256;
    const uint8_t *qp[R], *mp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t blk = (size_t)(rows[r] + rr) * w[r].nb;
        qp[r] = w[r].p0 + blk * 128 + 16 * g;
        mp[r] = w[r].p1 + blk * 16;
        acc[r] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const uint4 *xv = reinterpret_cast<const uint4 *>(xc);
    const uint2 *xm = reinterpret_cast<const uint2 *>(xmc);
    WRaw wa[R], wb[R];
    uint4 s0, s1;
    uint2 sm = make_uint2(0, 0);
    auto stage = [&](int b) { // global -> registers: this thread's share of superblock b
        s0 = xv[512 * b + tid];
        s1 = xv[512 * b + 256 + tid];
        if (tid < 64) sm = xm[64 * b + tid];
    };
    auto store = [&](int b) { // registers -> LDS buffer b & 1
        XLds &d = xs[b & 1];
        d.v[tid] = s0;
        d.v[256 + tid] = s1;
        if (tid < 64) d.m[tid] = sm;
    };
    auto loadw = [&](WRaw *wr, int b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wr[r].q0 = *reinterpret_cast<const uint4 *>(qp[r] + b * 128);
            wr[r].q1 = *reinterpret_cast<const uint4 *>(qp[r] + b * 128 + 64);
            wr[r].meta = *reinterpret_cast<const uint4 *>(mp[r] + b * 16);
        }
    };
    auto compute = [&](const WRaw *wr, int b) {
        const XLds &d = xs[b & 1];
        XRaw xr;
#pragma unroll
        for (int t = 0; t < 8; ++t) xr.v[t] = d.v[64 * t + lane];
        xr.m = d.m[lane];
#pragma unroll
        for (int r = 0; r < R; ++r) superblock(wr[r], xr, g, magic, acc[r]);
    };
    // one iteration: stage b+1, prefetch weights of b+1 into wn, compute b
    // from wc, publish b+1
    auto iter = [&](WRaw *wc, WRaw *wn, int b) {
        const int nx = min(b + 1, nbk - 1);
        stage(nx);
        loadw(wn, nx);
        __builtin_amdgcn_sched_barrier(0);
        compute(wc, b);
        __builtin_amdgcn_sched_barrier(0);
        store(b + 1);
        __syncthreads();
    };
    stage(0);
    loadw(wa, 0);
    store(0);
    __syncthreads();
    int b = 0;
    for (; b + 2 <= nbk; b += 2) {
        iter(wa, wb, b);
        iter(wb, wa, b + 1);
    }
    if (b < nbk) iter(wa, wb, b);
}

// Workgroup order. Workgroups are dispatched round-robin over the 8 XCDs
// (workgroup b runs on XCD b % 8), and every workgroup of a chunk reads the
// chunk's whole activation operand, so a chunk's workgroups share one XCD
// and its L2: chunk ti runs on XCD ti % 8, as workgroups b = 8 k + ti % 8
// with k = mgroups (ti / 8) + mg. The chunk count is known only on the
// device: the grid covers the largest count, and on every XCD the
// workgroups past it come last and exit.
__device__ __forceinline__ bool chunk_tile(int mgroups, int max_tiles, const int *ntiles, int &ti,
                                           int &mg)
{
    const int xcd = (int)(blockIdx.x % 8), k = (int)(blockIdx.x / 8);
    ti = xcd + 8 * (k / mgroups);
    mg = k % mgroups;
    return ti < max_tiles && ti < *ntiles;
}

inline int chunk_grid(int mgroups, int max_tiles) { return 8 * mgroups * ((max_tiles + 7) / 8); }

//
// Gate and up of one 16-token chunk of an expert: wave w of the workgroup
// takes mid rows m0 = 64 mg + 16 w of gate and of up; H[q][m] = silu(g) * u
// for the chunk's pair positions q, in f32, and hmax[q] = the largest |H[q]|
// as float bits (atomic max; NaN bits order above infinity).
__global__ __launch_bounds__(256) void moe_q4k_gate_up_kernel(
    WView gate, WView up, int mid, int K, const int *__restrict__ eoff,
    const int *__restrict__ tiles, const int *__restrict__ ntiles,
    const _Float16 *__restrict__ xc, const _Float16 *__restrict__ xmc,
    const float *__restrict__ xsc, float *__restrict__ H, uint32_t *__restrict__ hmax,
    int mgroups, int max_tiles)
{
    int ti, mg;
    if (!chunk_tile(mgroups, max_tiles, ntiles, ti, mg)) return;
    const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
    const int nb = eoff[e] + c * CHUNK, cnt = min(CHUNK, eoff[e + 1] - nb);
    const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
    const int m0 = 64 * mg + 16 * (threadIdx.x >> 6);
    __shared__ XLds xs[2];
    const WView w[2] = {gate, up};
    const int rows[2] = {e * mid + m0, e * mid + m0};
    f4 acc[2];
    tile_rows<2>(w, rows, K, xc + (size_t)ti * CHUNK * K, xmc + (size_t)ti * K, xs, acc);
    // lane (g, rr): tokens 4g+i of mid row m0 + rr
    const int rr = col;
    float *hbase = H + (size_t)nb * mid + m0 + rr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = 4 * g + i;
        uint32_t mb = 0;
        if (tok < cnt) {
            const float s = xsc[ti * CHUNK + tok];
            const float h = silu_mul(acc[0][i] * s, acc[1][i] * s);
            hbase[(size_t)tok * mid] = h;
            mb = __float_as_uint(fabsf(h));
        }
        // the 16 lanes of a lane group hold the wave's 16 rows of this token
        mb = max(mb, (uint32_t)__shfl_xor((int)mb, 1));
        mb = max(mb, (uint32_t)__shfl_xor((int)mb, 2));
        mb = max(mb, (uint32_t)__shfl_xor((int)mb, 4));
        mb = max(mb, (uint32_t)__shfl_xor((int)mb, 8));
        if (rr == 0 && tok < cnt) atomicMax(hmax + nb + tok, mb);
    }
}

// Down of one 16-token chunk: wave w takes hidden rows m0 = 128 mg + 32 w ..
// m0 + 31 (two row tiles); outp[q][m] = down_e[m] . H[q].
__global__ __launch_bounds__(256) void moe_q4k_down_kernel(
    WView down, int hidden, int K, const int *__restrict__ eoff, const int *__restrict__ tiles,
    const int *__restrict__ ntiles, const _Float16 *__restrict__ hc,
    const _Float16 *__restrict__ hmc, const float *__restrict__ hsc, float *__restrict__ outp,
    int mgroups, int max_tiles)
{
    int ti, mg;
    if (!chunk_tile(mgroups, max_tiles, ntiles, ti, mg)) return;
    const int m0 = 128 * mg + 32 * (threadIdx.x >> 6); // hidden % 128 == 0: all rows exist
    const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
    const int nb = eoff[e] + c * CHUNK, cnt = min(CHUNK, eoff[e + 1] - nb);
    const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
    __shared__ XLds xs[2];
    const WView w[2] = {down, down};
    const int rows[2] = {e * hidden + m0, e * hidden + m0 + 16};
    f4 acc[2];
    tile_rows<2>(w, rows, K, hc + (size_t)ti * CHUNK * K, hmc + (size_t)ti * K, xs, acc);
    // lane (g, rr): tokens 4g+i of hidden rows m0 + 16r + rr
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = 4 * g + i;
        if (tok >= cnt) continue;
        const float s = hsc[ti * CHUNK + tok];
        float *orow = outp + (size_t)(nb + tok) * hidden + m0 + col;
#pragma unroll
        for (int r = 0; r < 2; ++r) orow[16 * r] = acc[r][i] * s;
    }
}

// rmax[r] = the largest |x[r][k]| of row r of x [rows, K] (infinity when the
// row holds a NaN), one workgroup per row.
__global__ __launch_bounds__(256) void row_max_kernel(const float *__restrict__ x, int K,
                                                      float *__restrict__ rmax)
{
    __shared__ float wred[4];
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)blockIdx.x * K);
    const int t = threadIdx.x;
    float m = 0.f;
    for (int i = t; i < K / 4; i += 256) {
        const float4 v = x4[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w) m = INFINITY;
    }
    m = wave::max64(m);
    if ((t & 63) == 0) wred[t >> 6] = m;
    __syncthreads();
    if (t == 0) rmax[blockIdx.x] = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
}

// Workgroup (ti, b), 64 lanes, ti < *ntiles: superblock b of the activation
// operand of chunk ti (layout at the top of this file). Column col < cnt is
// row src = ptok[order[q]] of x (order given) or row q (order null), q the
// chunk's pair position, scaled by 2^-e with e = f16_row_exponent(rmax[src])
// (a zero, infinite or NaN maximum keeps scale 1); xsc[ti][col] = 2^e. xmc
// holds per lane f16(X / 16) of the four 16-element half-sums its lane group
// covers (f32 sums in a fixed order). Columns >= cnt are zero with scale 1.
// Workgroups (ti, 0) also clear hzero[q] of the chunk's positions (when
// given), ahead of the atomic maxima of the gate/up epilogue.
__global__ __launch_bounds__(64) void chunk_q4k_kernel(
    const float *__restrict__ x, int K, const float *__restrict__ rmax,
    const int *__restrict__ tiles, const int *__restrict__ ntiles, const int *__restrict__ eoff,
    const int *__restrict__ order, const int *__restrict__ ptok, _Float16 *__restrict__ xc,
    _Float16 *__restrict__ xmc, float *__restrict__ xsc, uint32_t *__restrict__ hzero)
{
    const int ti = blockIdx.x, b = blockIdx.y;
    if (ti >= *ntiles) return;
    const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
    const int nb = eoff[e] + c * CHUNK, cnt = min(CHUNK, eoff[e + 1] - nb);
    const int lane = threadIdx.x, col = lane & 15, g = lane >> 4;
    const bool live = col < cnt;
    const int src = live ? (order ? ptok[order[nb + col]] : nb + col) : 0;
    const int ex = live ? f16_row_exponent(rmax[src]) : 0;
    const float inv = ldexpf(1.0f, -ex);
    if (b == 0 && g == 0) {
        xsc[ti * CHUNK + col] = ldexpf(1.0f, ex);
        if (hzero && live) hzero[nb + col] = 0u;
    }
    auto pk = [](float p, float q) {
        const h2 v = {(_Float16)p, (_Float16)q};
        return __builtin_bit_cast(uint32_t, v);
    };
    const float4 *r4 = reinterpret_cast<const float4 *>(x + (size_t)src * K);
    uint4 *dst = reinterpret_cast<uint4 *>(xc + (size_t)ti * CHUNK * K) + 8 * b * 64 + lane;
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
        uint4 o = make_uint4(0, 0, 0, 0);
        if (live) {
            const int a = 256 * b + 64 * ((tt < 4 ? 0 : 2) + (g >> 1)) + 16 * (g & 1) + 4 * (tt & 3);
            const float4 lo = r4[a / 4], hi = r4[a / 4 + 8];
            const float l0 = lo.x * inv, l1 = lo.y * inv, l2 = lo.z * inv, l3 = lo.w * inv;
            const float h0 = hi.x * inv, h1 = hi.y * inv, h2v = hi.z * inv, h3 = hi.w * inv;
            o = make_uint4(pk(l0, l2), pk(l1, l3), pk(h0, h2v), pk(h1, h3));
            const int p = tt < 4 ? 0 : 2;
            ps[p] += (l0 + l1) + (l2 + l3);
            ps[p + 1] += (h0 + h1) + (h2v + h3);
        }
        dst[tt * 64] = o;
    }
    reinterpret_cast<uint2 *>(xmc + (size_t)ti * K)[64 * b + lane] =
        make_uint2(pk(ps[0] * 0.0625f, ps[1] * 0.0625f), pk(ps[2] * 0.0625f, ps[3] * 0.0625f));
}

} // namespace

int launch_moe_q4k(WView gate, WView up, WView down, int hidden, int mid, const float *x,
                   int tokens, const int *ptok, const int *eoff, const int *order,
                   const int *tiles, const int *ntiles, int max_tiles, float *tmax,
                   _Float16 *xc, _Float16 *xmc, float *xsc, float *h32, uint32_t *hmax,
                   _Float16 *hc, _Float16 *hmc, float *hsc, float *outp, void *stream)
{
    if (hidden % 256 || mid % 256) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(row_max_kernel, dim3(tokens), dim3(256), 0, st, x, hidden, tmax);
    hipLaunchKernelGGL(chunk_q4k_kernel, dim3(max_tiles, hidden / 256), dim3(64), 0, st, x, hidden,
                       tmax, tiles, ntiles, eoff, order, ptok, xc, xmc, xsc, hmax);
    {
        const int mgroups = mid / 64;
        hipLaunchKernelGGL(moe_q4k_gate_up_kernel, dim3(chunk_grid(mgroups, max_tiles)), dim3(256), 0, st, gate,
                           up, mid, hidden, eoff, tiles, ntiles, xc, xmc, xsc, h32, hmax, mgroups,
                           max_tiles);
    }
    hipLaunchKernelGGL(chunk_q4k_kernel, dim3(max_tiles, mid / 256), dim3(64), 0, st, h32, mid,
                       reinterpret_cast<const float *>(hmax), tiles, ntiles, eoff, nullptr,
                       nullptr, hc, hmc, hsc, nullptr);
    {
        const int mgroups = hidden / 128;
        hipLaunchKernelGGL(moe_q4k_down_kernel, dim3(chunk_grid(mgroups, max_tiles)), dim3(256), 0, st, down,
                           hidden, mid, eoff, tiles, ntiles, hc, hmc, hsc, outp, mgroups,
                           max_tiles);
    }
    return (int)hipGetLastError();
}

int moe_q4k_chunk() { return CHUNK; }

} // namespace hyq
