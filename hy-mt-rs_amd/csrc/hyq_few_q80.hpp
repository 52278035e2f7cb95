// One workgroup tile of the few-token Q8_0 product (Weight::matmul at batch
// 2..128, src/quant.rs:272-344, on the f16-MFMA path), shared by its own
// launch (few_q80_kernel, hyq_gemm_few.hip) and by the MoE SiLU-rows launch,
// which runs a Q8_0 shared projection's tiles beside the SiLU rows
// (hyq_moe_q4k.hip).
//
// Arithmetic. A Q8_0 block is d * q with q int8 (src/quant.rs:2409-2414).
// Per 32-column block and 16 x 16 (tokens x rows) tile a wave forms
//   P = sum_k q_k * x_k     on one v_mfma_f32_16x16x32_f16
// with q exact in f16 (the byte q + 128 under the f16 exponent of 1024 is
// 1152 + q, and one packed subtraction of 1152 leaves q), x the f16
// activation rows with their power-of-two row scale, and the accumulator
// takes acc += d * P in f32 per block. The weights thus enter exactly and
// only the activations are rounded.
//
// Operands. MFMA lane l = 16 g + c holds, of a block, columns 8 g .. 8 g + 7:
// as the A operand token c of the 16-token chunk, as the B operand weight row
// c of the wave's 16 rows (8 contiguous code bytes). The activations are laid
// out in that lane order, [chunk][block][lane][8 halves] (few_fragment_piece),
// so each A operand is one 1 KiB load. Output lane l holds tokens 4 g + i,
// i = 0..3, of row c. Every token's result depends on its own row only, so
// any batch of at most 128 tokens gives each row the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include "hyq_internal.hpp"

#pragma clang fp contract(off)

namespace hyq {
namespace few {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int CHUNK = 16; // tokens per MFMA column block
constexpr int SET = 8;    // blocks per register set (256 columns)
constexpr int CHUNKS = 4; // chunks a workgroup multiplies against one weight load
constexpr int WAVES = 8;  // waves per workgroup, each a share of K

// The waves' partial sums, met in LDS.
struct Red {
    f4 v[WAVES - 1][CHUNKS][64];
};

__device__ __forceinline__ float half_bits(uint32_t b)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// 8 int8 codes (bytes of lo, then of hi) as 8 exact f16 values in order.
__device__ __forceinline__ h8 codes_f16(uint32_t lo, uint32_t hi)
{
    const uint32_t a = lo ^ 0x80808080u, b = hi ^ 0x80808080u; // q + 128
    // bytes {q + 128, 0x64} per half: the f16 value 1024 + q + 128
    const h2 p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u));
    const h2 p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u));
    const h2 p2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u));
    const h2 p3 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u));
    const h2 off = {(_Float16)-1152.f, (_Float16)-1152.f};
    const h2 q0 = p0 + off, q1 = p1 + off, q2 = p2 + off, q3 = p3 + off;
    return h8{q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
}

// Piece p (block b = p / 4, lane group g = p % 4: columns 32 b + 8 g .. + 7)
// of token row n of x [.., K] (16-byte aligned) into the fragment layout xf,
// scaled by inv (zeros when x4 is null: the rows past the batch in its last
// chunk).
__device__ __forceinline__ void fragment_piece(const float4 *x4, float inv, int n, int p, int K,
                                               _Float16 *xf)
{
    const int b = p >> 2, g = p & 3, nb = K / 32, ck = n / CHUNK, c = n % CHUNK;
    h8 o = {};
    if (x4) {
        const float4 lo = x4[8 * b + 2 * g], hi = x4[8 * b + 2 * g + 1];
        o = h8{(_Float16)(lo.x * inv), (_Float16)(lo.y * inv), (_Float16)(lo.z * inv),
               (_Float16)(lo.w * inv), (_Float16)(hi.x * inv), (_Float16)(hi.y * inv),
               (_Float16)(hi.z * inv), (_Float16)(hi.w * inv)};
    }
    *reinterpret_cast<h8 *>(xf + (((size_t)ck * nb + b) * 64 + 16 * g + c) * 8) = o;
}

// Tile `tile` (all WAVES * 64 threads): 16 weight rows against up to CHUNKS
// 16-token chunks (the chunk group tile % cgroups), the waves splitting K:
// wave w takes the 256-column sets [w S / 8, (w + 1) S / 8) of the
// S = K / 256, one set at a time with all of the set's loads in flight (the
// codes, the scales and every chunk's activations), each weight operand
// feeding one MFMA per chunk. The waves' partial sums meet through LDS in
// wave order; y[n][row] = sum * rscale[n] for the tokens n < N.
__device__ __forceinline__ void q80_tile(int tile, WView w, int K, const _Float16 *__restrict__ xh,
                                         const float *__restrict__ rscale, int N,
                                         float *__restrict__ y, int cgroups, Red &red)
{
    const int rg = tile / cgroups, cgp = tile % cgroups;
    const int M = w.rows, nb = K / 32, nsets = nb / SET;
    const int wave = (int)(threadIdx.x >> 6), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int row = rg * 16 + c;
    const int n0 = cgp * CHUNKS * CHUNK;
    const int sb = wave * nsets / WAVES, se = (wave + 1) * nsets / WAVES;
    // rows and tokens past the end read the last ones (in bounds, unused)
    const int rowc = min(row, M - 1);
    const uint8_t *wq = w.p0 + (size_t)rowc * nb * 32 + 8 * g;
    const uint4 *wd = reinterpret_cast<const uint4 *>(w.p1 + (size_t)rowc * nb * 2);
    // chunk k's fragments (chunks past the batch read the last one, unused)
    const int nck = (N + CHUNK - 1) / CHUNK;
    const _Float16 *xa[CHUNKS];
#pragma unroll
    for (int k = 0; k < CHUNKS; ++k)
        xa[k] = xh + ((size_t)min(n0 / CHUNK + k, nck - 1) * nb * 64 + lane) * 8;
    f4 acc[CHUNKS];
#pragma unroll
    for (int k = 0; k < CHUNKS; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
    for (int s = sb; s < se; ++s) {
        uint2 q[SET];
        h8 x[CHUNKS][SET];
#pragma unroll
        for (int j = 0; j < SET; ++j)
            q[j] = *reinterpret_cast<const uint2 *>(wq + (size_t)(SET * s + j) * 32);
        const uint4 d4 = wd[s];
#pragma unroll
        for (int k = 0; k < CHUNKS; ++k)
#pragma unroll
            for (int j = 0; j < SET; ++j)
                x[k][j] = *reinterpret_cast<const h8 *>(xa[k] + (size_t)(SET * s + j) * 512);
        // (all of the set's loads issued before the compute that waits for them)
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t dw[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int j = 0; j < SET; ++j) {
            const h8 wj = codes_f16(q[j].x, q[j].y);
            const float d = half_bits(dw[j >> 1] >> (16 * (j & 1)));
#pragma unroll
            for (int k = 0; k < CHUNKS; ++k) {
                const f4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[k][j], wj,
                                                                     f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[k][i] = __builtin_fmaf(d, P[i], acc[k][i]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (wave > 0)
#pragma unroll
        for (int k = 0; k < CHUNKS; ++k) red.v[wave - 1][k][lane] = acc[k];
    __syncthreads();
    if (wave > 0 || row >= M) return;
#pragma unroll
    for (int k = 0; k < CHUNKS; ++k) {
        f4 v = acc[k];
#pragma unroll
        for (int u = 0; u < WAVES - 1; ++u) {
            const f4 r = red.v[u][k][lane];
            for (int i = 0; i < 4; ++i) v[i] = v[i] + r[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + CHUNK * k + 4 * g + i;
            if (n < N) y[(size_t)n * M + row] = v[i] * rscale[n];
        }
    }
}

// Tiles of a product of `rows` weight rows at batch N (rows / 16 rounded up,
// times the chunk groups).
inline int q80_tiles(int rows, int N, int *cgroups)
{
    *cgroups = (N + CHUNKS * CHUNK - 1) / (CHUNKS * CHUNK);
    return (rows + 15) / 16 * *cgroups;
}

} // namespace few
} // namespace hyq
