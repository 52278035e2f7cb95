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
// Activation operand. Per 16-token chunk, superblock b and step t, 64
// lanes x 16 bytes in lane order (lane = 16 g + column) in LDS. Lane (g,
// col)'s 8 halves for step t are x(a), x(a+2), x(a+1), x(a+3), x(a+32),
// x(a+34), x(a+33), x(a+35) of token col with a = 256 b + 64 c + o, c = g/2
// (+ 2 for t >= 4), o = 16 (g & 1) + 4 (t & 3): the A and B lanes of an MFMA
// pair the same k. Each column's pieces come from its row's operand
// (hyq_moe_operand.hpp: a token row of x, formed in the plan's launch, or a
// pair's SiLU row, formed by silu_rows_kernel), gathered while the operand
// is copied into LDS. The activations are the MFMA's A operand, the weights
// its B operand: output lane l holds tokens 4 (l / 16) + i, i = 0..3, of
// weight row l % 16, the row whose d and dmin the lane loaded.
#include <hip/hip_runtime.h>

#include "hyq_f16rows.hpp"
#include "hyq_few_q80.hpp"
#include "hyq_internal.hpp"
#include "hyq_moe_operand.hpp"
#include "hyq_wave.hpp"

#pragma clang fp contract(off)

namespace hyq {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int CHUNK = 16; // tokens per expert chunk (one MFMA column block)
constexpr int MOE_Q4K_MAX_K = 4096;  // largest K (hidden or mid)
constexpr int MOE_Q4K_MAX_KL = 2048; // largest K slice of one workgroup: 34 KL bytes of LDS

// K slices of the gate/up product: two when its superblocks split evenly
// (the tiles then number twice the workgroups, which evens out the last
// round of workgroups on the CUs), else one. The down product (fewer,
// shorter rows) measured faster unsplit.
__host__ __device__ inline int moe_kslices(int K) { return (K / 256) % 2 == 0 ? 2 : 1; }

// s_waitcnt lgkmcnt(0), leaving the other counters alone.
#define HYQ_LGKM0() __builtin_amdgcn_s_waitcnt(0xc07f)

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

// Work units. A unit is one 16-token chunk ti of an expert, one K slice kh
// and one group mg of 64 weight rows (wave w of the workgroup takes rows
// 16 w .. 16 w + 15 of the group, of each matrix it streams):
// u = (ti ks + kh) mgroups + mg, so the units that share one activation
// operand (ti, kh) are consecutive. The grid is a fixed count of
// workgroups, a multiple of 8 sized to be resident at once, and the unit
// count U = *ntiles ks mgroups is known only on the device. Workgroup b
// runs on XCD b % 8 (round-robin dispatch): XCD x takes the units
// [x U / 8, (x + 1) U / 8) and its j-th of W workgroups the j-th of W even
// shares of them. Every workgroup thus gets the same number of units to
// within one (no last round of a few workgroups on an idle chip), and a
// chunk's units stay on one or two XCDs, whose L2 holds its operand.
__device__ __forceinline__ void unit_range(int U, int &u0, int &u1)
{
    const int per = (int)gridDim.x / 8, x = (int)(blockIdx.x % 8), j = (int)(blockIdx.x / 8);
    const int ux0 = (int)((long)U * x / 8), n = (int)((long)U * (x + 1) / 8) - ux0;
    u0 = ux0 + (int)((long)n * j / per);
    u1 = ux0 + (int)((long)n * (j + 1) / per);
}

// The workgroup's units [u0, u1) against R matrices (all 256 threads). Per
// run of units that share an activation operand, the chunk's operand slice
// (16 K halves in MFMA lane order and the K / 4 half-sums, gathered from the
// columns' row operands) is copied into LDS once (xl), and each wave then streams its weights through NS register
// sets, NS - 1 superblocks ahead of the compute, across the run's row
// groups: stream position p is superblock p % nbk of the run's group
// p / nbk. The loop holds no barrier and no other global load, so the
// compiler's in-order load count waits for exactly the set being used. The
// first NS - 1 weight loads are issued after the activation loads and
// before their LDS stores, so their latency overlaps the copy; past the
// run's last superblock the weight loads read an L2-hot dummy (the thread's
// column row operand), so every step issues the same loads.
//
// run(ti, kh, mg, qp, mp, gq, gm, xrow, mrow) sets, for the run's first
// group mg, the lane's row pointers of each matrix at the slice start (qs
// and header planes) and the byte steps from one group to the next, the row
// operand (op and hs, hyq_moe_operand.hpp) of chunk column threadIdx.x % 16,
// and loads what flush needs; flush(gj, acc) takes the sums of the run's
// group gj when its last superblock is done (acc then restarts from zero).
template <int R, int NS, class Run, class Flush>
__device__ __forceinline__ void stream_units(int u0, int u1, int mgroups, int ks, int nbk,
                                             uint4 *xl, Run run, Flush flush)
{
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4;
    const int K = 256 * nbk; // the slice
    uint2 *xlm = reinterpret_cast<uint2 *>(xl + 2 * K);
    for (int u = u0; u < u1;) {
        const int blk = u / mgroups, nr = min(u1, (blk + 1) * mgroups) - u;
        const int ti = blk / ks, kh = blk - ti * ks;
        const uint8_t *qp[R], *mp[R];
        size_t gq[R], gm[R];
        const uint4 *xrow;
        const uint2 *mrow;
        run(ti, kh, u - blk * mgroups, qp, mp, gq, gm, xrow, mrow);
        const uint8_t *dummy = reinterpret_cast<const uint8_t *>(xrow); // >= 512 bytes, L2-hot
        WRaw ring[NS][R];
        int lg = 0, ls = 0; // the next stream position to load: group, superblock
        auto loadw = [&](WRaw *wr) {
            const bool in = lg < nr;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t *q = in ? qp[r] + lg * gq[r] + ls * 128 : dummy;
                const uint8_t *m = in ? mp[r] + lg * gm[r] + ls * 256 : dummy;
                wr[r].q0 = *reinterpret_cast<const uint4 *>(q);
                wr[r].q1 = *reinterpret_cast<const uint4 *>(q + 64);
                wr[r].meta = *reinterpret_cast<const uint4 *>(m);
            }
            if (++ls == nbk) {
                ls = 0;
                ++lg;
            }
        };
        // the slice's operand: 2K uint4 of steps and K/4 uint2 of half-sums
        // (K <= MOE_Q4K_MAX_KL: at most 16 and 2 per thread), element i of
        // either in LDS lane order (column i % 16, the thread's own),
        // gathered from the column's row operand; indices past the end are
        // clamped to the last element of the thread's column, so every load
        // and store is issued unconditionally and a duplicate rewrites its
        // element with its own value
        // (the thread index made opaque per run, so that the copy's 2 x 16
        // clamped indices are not hoisted out of the loop and held in
        // registers through the stream)
        int t = tid;
        asm volatile("" : "+v"(t));
        const int last4 = 2 * K - 16 + (t & 15), last2 = K / 4 - 16 + (t & 15);
        // (staged in clang vectors: HIP's uint4 struct copies stay in scratch)
        typedef unsigned u4v __attribute__((ext_vector_type(4)));
        typedef unsigned u2v __attribute__((ext_vector_type(2)));
        const u4v *xs4 = reinterpret_cast<const u4v *>(xrow) + MOE_OP_U4_PER_SB * kh * nbk;
        const u2v *ms2 = reinterpret_cast<const u2v *>(mrow) + MOE_OP_U2_PER_SB * kh * nbk;
        u4v tv[MOE_Q4K_MAX_KL / 128];
        u2v tm[MOE_Q4K_MAX_KL / 1024];
#pragma unroll
        for (int j = 0; j < MOE_Q4K_MAX_KL / 128; ++j) {
            // LDS element i = 512 superblock + 64 step + 16 g + col
            const int i = min(t + 256 * j, last4);
            tv[j] = xs4[MOE_OP_U4_PER_SB * (i >> 9) + 4 * ((i >> 6) & 7) + ((i >> 4) & 3)];
        }
#pragma unroll
        for (int j = 0; j < MOE_Q4K_MAX_KL / 1024; ++j) {
            // LDS element i = 64 superblock + 16 g + col
            const int i = min(t + 256 * j, last2);
            tm[j] = ms2[MOE_OP_U2_PER_SB * (i >> 6) + ((i >> 4) & 3)];
        }
#pragma unroll
        for (int k = 0; k < NS - 1; ++k) loadw(ring[k]);
        // every wave is done reading the previous run's operand (its LDS
        // reads have returned: lgkmcnt 0) before any wave overwrites it
        HYQ_LGKM0();
        asm volatile("s_barrier" ::: "memory");
        // (stores unconditional too, so that no load sinks into a branch:
        // the clamped duplicates rewrite the last element with its own value)
#pragma unroll
        for (int j = 0; j < MOE_Q4K_MAX_KL / 128; ++j)
            reinterpret_cast<u4v *>(xl)[min(t + 256 * j, last4)] = tv[j];
#pragma unroll
        for (int j = 0; j < MOE_Q4K_MAX_KL / 1024; ++j)
            reinterpret_cast<u2v *>(xlm)[min(t + 256 * j, last2)] = tm[j];
        HYQ_LGKM0();
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        f4 acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = f4{0.f, 0.f, 0.f, 0.f};
        int cg = 0, cs = 0; // the stream position being computed
        auto step = [&](WRaw *wc, WRaw *wn) {
            loadw(wn);
            __builtin_amdgcn_sched_barrier(0);
            XRaw xr;
#pragma unroll
            for (int t = 0; t < 8; ++t) xr.v[t] = xl[512 * cs + 64 * t + lane];
            xr.m = xlm[64 * cs + lane];
#pragma unroll
            for (int r = 0; r < R; ++r) superblock(wc[r], xr, g, magic, acc[r]);
            __builtin_amdgcn_sched_barrier(0);
            if (++cs == nbk) {
                flush(cg, acc);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = f4{0.f, 0.f, 0.f, 0.f};
                cs = 0;
                ++cg;
            }
        };
        const int np = nr * nbk;
        int p = 0;
        for (; p + NS <= np; p += NS) {
#pragma unroll
            for (int k = 0; k < NS; ++k) step(ring[k], ring[(k + NS - 1) % NS]);
        }
#pragma unroll
        for (int k = 0; k < NS - 1; ++k)
            if (p + k < np) step(ring[k], ring[(k + NS - 1) % NS]);
        u += nr;
    }
}

inline int unit_grid(int cus) { return 8 * ((2 * cus + 7) / 8); } // two workgroups per CU

// Gate and up of the units: wave w takes mid rows 64 mg + 16 w .. + 15 of
// gate and of up for one chunk and K slice; chunk column col reads the row
// operand of token ctok[ti][col] (xop, xhs); the slice's sums, scaled back
// by the token's scale xsc, go to gpart / upart[slice][q][m] for the
// chunk's pair positions q.
__global__ __launch_bounds__(256, 2) void moe_q4k_gate_up_kernel(
    WView gate, WView up, int mid, int K, const int *__restrict__ eoff,
    const int *__restrict__ tiles, const int *__restrict__ ntiles,
    const int *__restrict__ ctok, const uint4 *__restrict__ xop, const uint2 *__restrict__ xhs,
    const float *__restrict__ xsc, float *__restrict__ gpart, float *__restrict__ upart,
    size_t part_stride, int mgroups)
{
    const int ks = moe_kslices(K), nbk = K / 256 / ks;
    int u0, u1;
    unit_range(*ntiles * ks * mgroups, u0, u1);
    const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15, w16 = 16 * (threadIdx.x >> 6);
    extern __shared__ uint4 xl[];
    int nb = 0, cnt = 0, kh = 0, mg0 = 0;
    float s[4];
    auto run = [&](int ti, int kh_, int mg, const uint8_t **qp, const uint8_t **mp, size_t *gq,
                   size_t *gm, const uint4 *&xrow, const uint2 *&mrow) {
        const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
        const int tok = ctok[ti * CHUNK + col];
        xrow = xop + (size_t)tok * (K / 8);
        mrow = xhs + (size_t)tok * (K / 64);
        nb = eoff[e] + c * CHUNK;
        cnt = min(CHUNK, eoff[e + 1] - nb);
        kh = kh_;
        mg0 = mg;
        const int row = e * mid + 64 * mg + w16 + col;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const WView &W = r ? up : gate;
            const size_t blk = (size_t)row * W.nb + kh * nbk;
            qp[r] = W.p0 + blk * 128 + 16 * g;
            mp[r] = W.p2 + (((size_t)(row >> 4) * W.nb + kh * nbk) * 16 + col) * 16;
            gq[r] = (size_t)64 * W.nb * 128;
            gm[r] = (size_t)4 * W.nb * 256;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = xsc[ctok[ti * CHUNK + 4 * g + i]];
    };
    // lane (g, col): tokens 4g+i of mid row 64 (mg0 + gj) + 16 w + col
    auto flush = [&](int gj, const f4 *acc) {
        const size_t base = kh * part_stride + (size_t)nb * mid + 64 * (mg0 + gj) + w16 + col;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * g + i;
            if (tok >= cnt) continue;
            gpart[base + (size_t)tok * mid] = acc[0][i] * s[i];
            upart[base + (size_t)tok * mid] = acc[1][i] * s[i];
        }
    };
    stream_units<2, 4>(u0, u1, mgroups, ks, nbk, xl, run, flush);
}

// The SiLU rows of the pairs: h[m] = silu(g) * u with g, u the sums of the
// K slices' partial rows (in slice order), formed as pair q's row operand
// (hop, hhs, hsc: hyq_moe_operand.hpp, scaled by the row's largest |h|,
// infinity when it holds a NaN); one workgroup per valid pair position q.
// The first `stiles` workgroups take the tiles of a few-token Q8_0 product
// y = x W^T (hyq_few_q80.hpp: the shared projection that seeds the routed
// sum, its fragments xf and row scales xsc formed in the plan's launch),
// which needs nothing the SiLU rows make. They come first so that they are
// dispatched while the SiLU rows are: their registers hold one workgroup
// per CU, and the SiLU rows fill the other CUs.
template <int RS>
__global__ __launch_bounds__(64 * few::WAVES) void silu_rows_kernel(
    const float *__restrict__ gpart, const float *__restrict__ upart, int ks, size_t part_stride,
    int mid, const int *__restrict__ valid, uint4 *__restrict__ hop, uint2 *__restrict__ hhs,
    float *__restrict__ hsc, int stiles, WView shared, int K, const _Float16 *__restrict__ xf,
    const float *__restrict__ xsc, int T, float *__restrict__ y, int cgroups)
{
    constexpr int NT = 64 * few::WAVES;
    union Lds {
        struct {
            float hl[MOE_Q4K_MAX_K];
            float wred[few::WAVES];
        } s;
        few::Red red;
    };
    __shared__ __align__(16) Lds lds;
    if ((int)blockIdx.x < stiles) {
        few::q80_tile((int)blockIdx.x, shared, K, xf, xsc, T, y, cgroups, lds.red);
        return;
    }
    const int q = blockIdx.x - stiles;
    if (q >= *valid) return;
    const int t = threadIdx.x;
    const size_t row = (size_t)q * mid;
    float *hl = lds.s.hl;
    // values t + NT j, j < RS (mid <= NT RS): every load issued (clamped
    // into the row) before the first is used
    float gv[RS], uv[RS], g2[RS], u2[RS];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const size_t i = row + min(t + NT * j, mid - 1);
        gv[j] = gpart[i];
        uv[j] = upart[i];
    }
    if (ks > 1) {
#pragma unroll
        for (int j = 0; j < RS; ++j) {
            const size_t i = part_stride + row + min(t + NT * j, mid - 1);
            g2[j] = gpart[i];
            u2[j] = upart[i];
        }
    }
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const int i = t + NT * j;
        if (i >= mid) break;
        float g = gv[j], u = uv[j];
        if (ks > 1) {
            g = g + g2[j];
            u = u + u2[j];
        }
        const float v = silu_mul(g, u);
        hl[i] = v;
        m = fmaxf(m, fabsf(v));
        if (v != v) m = INFINITY;
    }
    m = wave::max64(m);
    if ((t & 63) == 0) lds.s.wred[t >> 6] = m;
    __syncthreads();
    float mm = lds.s.wred[0];
#pragma unroll
    for (int w = 1; w < few::WAVES; ++w) mm = fmaxf(mm, lds.s.wred[w]);
    const int e = f16_row_exponent(mm);
    const float inv = ldexpf(1.0f, -e);
    if (t == 0) hsc[q] = ldexpf(1.0f, e);
    auto val = [&](int i) { return hl[i]; };
    uint4 *op = hop + (size_t)q * (mid / 8);
    uint32_t *hs = reinterpret_cast<uint32_t *>(hhs + (size_t)q * (mid / 64));
    for (int it = t; it < 8 * (mid / 256); it += NT)
        row_operand_item(val, inv, it >> 3, (it >> 1) & 3, it & 1, op, hs);
}

// Down of the units (one K slice): wave w takes hidden rows 64 mg + 16 w ..
// + 15 for one chunk; the sums down_e[m] . H[q], scaled back, go to outp.
// One matrix per wave, so eight register sets (seven superblocks ahead)
// keep as many bytes in flight as gate/up's four sets of two matrices.
__global__ __launch_bounds__(256, 2) void moe_q4k_down_kernel(
    WView down, int hidden, int K, const int *__restrict__ eoff, const int *__restrict__ tiles,
    const int *__restrict__ ntiles, const int *__restrict__ cpos, const uint4 *__restrict__ hop,
    const uint2 *__restrict__ hhs, const float *__restrict__ hsc, float *__restrict__ outp,
    int mgroups)
{
    const int nbk = K / 256;
    int u0, u1;
    unit_range(*ntiles * mgroups, u0, u1);
    const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15, w16 = 16 * (threadIdx.x >> 6);
    extern __shared__ uint4 xl[];
    int nb = 0, cnt = 0, mg0 = 0;
    float s[4];
    auto run = [&](int ti, int, int mg, const uint8_t **qp, const uint8_t **mp, size_t *gq,
                   size_t *gm, const uint4 *&xrow, const uint2 *&mrow) {
        const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
        const int q = cpos[ti * CHUNK + col];
        xrow = hop + (size_t)q * (K / 8);
        mrow = hhs + (size_t)q * (K / 64);
        nb = eoff[e] + c * CHUNK;
        cnt = min(CHUNK, eoff[e + 1] - nb);
        mg0 = mg;
        const int row = e * hidden + 64 * mg + w16 + col;
        const size_t blk = (size_t)row * down.nb;
        qp[0] = down.p0 + blk * 128 + 16 * g;
        mp[0] = down.p2 + ((size_t)(row >> 4) * down.nb * 16 + col) * 16;
        gq[0] = (size_t)64 * down.nb * 128;
        gm[0] = (size_t)4 * down.nb * 256;
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = hsc[cpos[ti * CHUNK + 4 * g + i]];
    };
    // lane (g, col): tokens 4g+i of hidden row 64 (mg0 + gj) + 16 w + col
    auto flush = [&](int gj, const f4 *acc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * g + i;
            if (tok >= cnt) continue;
            outp[(size_t)(nb + tok) * hidden + 64 * (mg0 + gj) + w16 + col] = acc[0][i] * s[i];
        }
    };
    stream_units<1, 8>(u0, u1, mgroups, 1, nbk, xl, run, flush);
}

// The row operands of the token rows of x [T, K] (wave_row_operand), one
// wave per row, when the plan's launch did not form them.
__global__ __launch_bounds__(256) void row_operand_kernel(const float *__restrict__ x, int T,
                                                          int K, uint4 *__restrict__ xop,
                                                          uint2 *__restrict__ xhs,
                                                          float *__restrict__ xsc)
{
    const int r = 4 * blockIdx.x + (threadIdx.x >> 6);
    if (r >= T) return;
    wave_row_operand(x + (size_t)r * K, K, xop + (size_t)r * (K / 8), xhs + (size_t)r * (K / 64),
                     xsc + r);
}

// Per chunk column (ti, col), ti < *ntiles: the pair position the column
// takes (the chunk's last pair for columns past its pairs) and its token.
__global__ __launch_bounds__(256) void chunk_cols_kernel(const int *__restrict__ tiles,
                                                         const int *__restrict__ ntiles,
                                                         const int *__restrict__ eoff,
                                                         const int *__restrict__ order,
                                                         const int *__restrict__ ptok,
                                                         int max_tiles, int *__restrict__ cpos,
                                                         int *__restrict__ ctok)
{
    const int idx = blockIdx.x * 256 + threadIdx.x, ti = idx / CHUNK, col = idx % CHUNK;
    if (ti >= max_tiles || ti >= *ntiles) return;
    const int e = tiles[2 * ti], c = tiles[2 * ti + 1];
    const int nb = eoff[e] + c * CHUNK, last = min(CHUNK, eoff[e + 1] - nb) - 1;
    const int q = nb + min(col, last);
    cpos[idx] = q;
    ctok[idx] = ptok[order[q]];
}

} // namespace

int launch_moe_q4k(WView gate, WView up, WView down, int hidden, int mid, const float *x,
                   int tokens, const int *ptok, const int *eoff, const int *valid,
                   const int *order, const int *tiles, const int *ntiles, int max_tiles,
                   int npairs, bool have_ops, uint4 *xop, uint2 *xhs, float *xsc, int *cpos,
                   int *ctok, float *gpart, float *upart, uint4 *hop, uint2 *hhs, float *hsc,
                   float *outp, void *stream, const WView *shared,
                   const _Float16 *xf, float *y)
{
    if (!moe_q4k_fits(hidden, mid)) return (int)hipErrorInvalidValue;
    if (shared && (!have_ops || !xf || !few_q80_fits(shared->rows, hidden, tokens)))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const size_t gstride = (size_t)npairs * mid;
    if (!have_ops) {
        hipLaunchKernelGGL(row_operand_kernel, dim3((tokens + 3) / 4), dim3(256), 0, st, x, tokens,
                           hidden, xop, xhs, xsc);
        hipLaunchKernelGGL(chunk_cols_kernel, dim3((max_tiles * CHUNK + 255) / 256), dim3(256), 0,
                           st, tiles, ntiles, eoff, order, ptok, max_tiles, cpos, ctok);
    }
    int dev = 0, cus = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess)
        err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return (int)err;
    if (cus <= 0) return (int)hipErrorInvalidDevice;
    const dim3 grid(unit_grid(cus));
    hipLaunchKernelGGL(moe_q4k_gate_up_kernel, grid, dim3(256),
                       (size_t)34 * (hidden / moe_kslices(hidden)), st, gate, up, mid, hidden,
                       eoff, tiles, ntiles, ctok, xop, xhs, xsc, gpart, upart, gstride, mid / 64);
    int cgroups = 0;
    const int stiles = shared ? few::q80_tiles(shared->rows, tokens, &cgroups) : 0;
    // the SiLU rows' widths: mid <= MOE_Q4K_MAX_KL (moe_q4k_fits)
    static_assert(MOE_Q4K_MAX_KL <= 4 * 64 * few::WAVES, "four values per SiLU-row thread");
    auto silu = mid <= 3 * 64 * few::WAVES ? silu_rows_kernel<3> : silu_rows_kernel<4>;
    hipLaunchKernelGGL(silu, dim3(npairs + stiles), dim3(64 * few::WAVES), 0, st, gpart, upart,
                       moe_kslices(hidden), gstride, mid, valid, hop, hhs, hsc, stiles,
                       shared ? *shared : WView{}, hidden, xf, xsc, tokens, y, cgroups);
    hipLaunchKernelGGL(moe_q4k_down_kernel, grid, dim3(256), (size_t)34 * mid, st, down, hidden,
                       mid, eoff, tiles, ntiles, cpos, hop, hhs, hsc, outp, hidden / 64);
    return (int)hipGetLastError();
}

bool moe_q4k_fits(int hidden, int mid)
{
    return hidden % 256 == 0 && mid % 256 == 0 && hidden <= MOE_Q4K_MAX_K &&
           mid <= MOE_Q4K_MAX_K && hidden / moe_kslices(hidden) <= MOE_Q4K_MAX_KL &&
           mid <= MOE_Q4K_MAX_KL && hidden % 128 == 0;
}

int moe_q4k_chunk() { return CHUNK; }

} // namespace hyq
