// Few-token products of Q8_0 weights: Weight::matmul at batch 2..128
// (src/quant.rs:272-344) on the f16-MFMA path, as one launch with no LDS
// stage and no K split. There the product is bound by streaming the weight
// once, not by the matrix cores, so the weights go from HBM straight into
// MFMA operands in registers.
//
// Arithmetic. A Q8_0 block is d * q with q int8 (src/quant.rs:2409-2414).
// Per 32-column block and 16 x 16 (tokens x rows) tile a wave forms
//   P = sum_k q_k * x_k     on one v_mfma_f32_16x16x32_f16
// with q exact in f16 (the byte q + 128 under the f16 exponent of 1024 is
// 1152 + q, and one packed subtraction of 1152 leaves q), x the f16
// activation rows with their power-of-two row scale (launch_to_f16), and the
// accumulator takes acc += d * P in f32 per block. The weights thus enter
// exactly and only the activations are rounded.
//
// Operands. MFMA lane l = 16 g + c holds, of a block, columns 8 g .. 8 g + 7:
// as the A operand token c of the 16-token chunk, as the B operand weight row
// c of the wave's 16 rows (8 contiguous code bytes). The activations are laid
// out by few_rows_kernel in that lane order, [chunk][block][lane][8 halves],
// so each A operand is one 1 KiB load. Output lane l holds tokens 4 g + i,
// i = 0..3, of row c. Every token's result depends on its own row only, so
// any batch of at most 128 tokens gives each row the same bits.
#include <hip/hip_runtime.h>

#include "hyq_f16rows.hpp"
#include "hyq_internal.hpp"
#include "hyq_wave.hpp"

#pragma clang fp contract(off)

namespace hyq {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int FEW_CHUNK = 16;  // tokens per MFMA column block
constexpr int FEW_SET = 8;     // blocks per register set (256 columns)

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

// One workgroup per token row n of the chunks (n < chunks * 16): its f16
// values (x[n] scaled by 2^-e, e from the row's largest magnitude as
// launch_to_f16 forms it; zeros for n >= N) into the fragment layout, and
// rscale[n] = 2^e.
__global__ __launch_bounds__(256) void few_rows_kernel(const float *__restrict__ x, int K, int N,
                                                       _Float16 *__restrict__ xf,
                                                       float *__restrict__ rscale)
{
    __shared__ float wred[4];
    const int n = (int)blockIdx.x, t = (int)threadIdx.x, nb = K / 32;
    const int ck = n / FEW_CHUNK, c = n % FEW_CHUNK;
    const bool live = n < N;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)(live ? n : 0) * K);
    float m = 0.f;
    if (live)
        for (int i = t; i < K / 4; i += 256) {
            const float4 v = x4[i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            if (v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w) m = INFINITY;
        }
    m = wave::max64(m);
    if ((t & 63) == 0) wred[t >> 6] = m;
    __syncthreads();
    const int e = f16_row_exponent(fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3])));
    const float inv = ldexpf(1.0f, -e);
    if (t == 0 && live) rscale[n] = ldexpf(1.0f, e);
    // piece (block b, lane group g): columns 32 b + 8 g .. + 7
    for (int p = t; p < 4 * nb; p += 256) {
        const int b = p >> 2, g = p & 3;
        h8 o = {};
        if (live) {
            const float4 lo = x4[8 * b + 2 * g], hi = x4[8 * b + 2 * g + 1];
            o = h8{(_Float16)(lo.x * inv), (_Float16)(lo.y * inv), (_Float16)(lo.z * inv),
                   (_Float16)(lo.w * inv), (_Float16)(hi.x * inv), (_Float16)(hi.y * inv),
                   (_Float16)(hi.z * inv), (_Float16)(hi.w * inv)};
        }
        *reinterpret_cast<h8 *>(xf + (((size_t)ck * nb + b) * 64 + 16 * g + c) * 8) = o;
    }
}

constexpr int FEW_CHUNKS = 4;  // chunks a workgroup multiplies against one weight load
constexpr int FEW_WAVES = 8;   // waves per workgroup, each a share of K

// Workgroup b: 16 weight rows against up to FEW_CHUNKS 16-token chunks (the
// chunk group b % cgroups), its FEW_WAVES waves splitting K: wave w takes the
// 256-column sets [w S / 8, (w + 1) S / 8) of the S = K / 256, one set at a
// time with all of the set's loads in flight (the codes, the scales and every
// chunk's activations), each weight operand feeding one MFMA per chunk. The
// waves' partial sums meet through LDS in wave order.
__global__ __launch_bounds__(64 * FEW_WAVES) void few_q80_kernel(WView w, int K,
                                                                 const _Float16 *__restrict__ xh,
                                                                 const float *__restrict__ rscale,
                                                                 int N, float *__restrict__ y,
                                                                 int cgroups)
{
    __shared__ f4 red[FEW_WAVES - 1][FEW_CHUNKS][64];
    const int rg = (int)blockIdx.x / cgroups, cgp = (int)blockIdx.x % cgroups;
    const int M = w.rows, nb = K / 32, nsets = nb / FEW_SET;
    const int wave = (int)(threadIdx.x >> 6), lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int row = rg * 16 + c;
    const int n0 = cgp * FEW_CHUNKS * FEW_CHUNK;
    const int sb = wave * nsets / FEW_WAVES, se = (wave + 1) * nsets / FEW_WAVES;
    // rows and tokens past the end read the last ones (in bounds, unused)
    const int rowc = min(row, M - 1);
    const uint8_t *wq = w.p0 + (size_t)rowc * nb * 32 + 8 * g;
    const uint4 *wd = reinterpret_cast<const uint4 *>(w.p1 + (size_t)rowc * nb * 2);
    // chunk k's fragments (chunks past the batch read the last one, unused)
    const int nck = (N + FEW_CHUNK - 1) / FEW_CHUNK;
    const _Float16 *xa[FEW_CHUNKS];
#pragma unroll
    for (int k = 0; k < FEW_CHUNKS; ++k)
        xa[k] = xh + ((size_t)min(n0 / FEW_CHUNK + k, nck - 1) * nb * 64 + lane) * 8;
    f4 acc[FEW_CHUNKS];
#pragma unroll
    for (int k = 0; k < FEW_CHUNKS; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
    for (int s = sb; s < se; ++s) {
        uint2 q[FEW_SET];
        h8 x[FEW_CHUNKS][FEW_SET];
#pragma unroll
        for (int j = 0; j < FEW_SET; ++j)
            q[j] = *reinterpret_cast<const uint2 *>(wq + (size_t)(FEW_SET * s + j) * 32);
        const uint4 d4 = wd[s];
#pragma unroll
        for (int k = 0; k < FEW_CHUNKS; ++k)
#pragma unroll
            for (int j = 0; j < FEW_SET; ++j)
                x[k][j] = *reinterpret_cast<const h8 *>(xa[k] + (size_t)(FEW_SET * s + j) * 512);
        // (all of the set's loads issued before the compute that waits for them)
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t dw[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int j = 0; j < FEW_SET; ++j) {
            const h8 wj = codes_f16(q[j].x, q[j].y);
            const float d = half_bits(dw[j >> 1] >> (16 * (j & 1)));
#pragma unroll
            for (int k = 0; k < FEW_CHUNKS; ++k) {
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
        for (int k = 0; k < FEW_CHUNKS; ++k) red[wave - 1][k][lane] = acc[k];
    __syncthreads();
    if (wave > 0 || row >= M) return;
#pragma unroll
    for (int k = 0; k < FEW_CHUNKS; ++k) {
        f4 v = acc[k];
#pragma unroll
        for (int u = 0; u < FEW_WAVES - 1; ++u) {
            const f4 r = red[u][k][lane];
            for (int i = 0; i < 4; ++i) v[i] = v[i] + r[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + FEW_CHUNK * k + 4 * g + i;
            if (n < N) y[(size_t)n * M + row] = v[i] * rscale[n];
        }
    }
}

} // namespace

bool few_q80_fits(int rows, int cols, int batch)
{
    return batch >= 1 && batch <= FEW_Q80_MAX_TOKENS && cols % 256 == 0 && rows >= 1;
}

size_t few_q80_operand_bytes(int cols, int batch)
{
    return (size_t)((batch + FEW_CHUNK - 1) / FEW_CHUNK) * FEW_CHUNK * cols * 2;
}

int launch_few_q80(WView w, int cols, const float *x, _Float16 *xh, float *rscale, int batch,
                   float *y, void *stream)
{
    if (!few_q80_fits(w.rows, cols, batch)) return (int)hipErrorInvalidValue;
    const int nrows = (batch + FEW_CHUNK - 1) / FEW_CHUNK * FEW_CHUNK;
    hipLaunchKernelGGL(few_rows_kernel, dim3(nrows), dim3(256), 0, (hipStream_t)stream, x, cols,
                       batch, xh, rscale);
    const int rgroups = (w.rows + 15) / 16;
    const int cgroups = (batch + FEW_CHUNKS * FEW_CHUNK - 1) / (FEW_CHUNKS * FEW_CHUNK);
    hipLaunchKernelGGL(few_q80_kernel, dim3(rgroups * cgroups), dim3(64 * FEW_WAVES), 0,
                       (hipStream_t)stream, w, cols, xh, rscale, batch, y, cgroups);
    return (int)hipGetLastError();
}

} // namespace hyq
