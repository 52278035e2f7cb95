// GGUF blocks <-> device planes, and the bit-exact block decoders
// (decode_unchecked, src/quant.rs:2405-2486) on gfx950.
//
// The decoders must reproduce the reference's f32 bit patterns, so this file
// is compiled without floating-point contraction: `d1 * q - m1` stays a
// rounded product followed by a rounded difference, as in the Rust source.
#include <hip/hip_runtime.h>

#include "hyq_decode.hpp"

namespace hyq {

namespace {

using namespace dec;


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

// Q4_K headers in 16-row tiles: the 16-byte header of (row r, block b) of a
// weight of `rows` rows (a multiple of 16) and nb blocks per row goes from
// hdr[r nb + b] to tiles[((r / 16) nb + b) 16 + r % 16], so the headers of
// one block of 16 consecutive rows are 256 contiguous bytes.
__global__ void tile_headers_kernel(const uint4 *__restrict__ hdr, size_t rows, int nb,
                                    uint4 *__restrict__ tiles)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * (size_t)nb) return;
    const size_t t = i / (16 * (size_t)nb), rem = i % (16 * (size_t)nb);
    const int b = (int)(rem / 16), rr = (int)(rem % 16);
    tiles[i] = hdr[(t * 16 + rr) * nb + b];
}

} // namespace

int launch_tile_headers(const uint8_t *hdr, size_t rows, int nb, uint8_t *tiles, void *stream)
{
    const size_t n = rows * (size_t)nb;
    if (n == 0) return 0;
    if (rows % 16) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(tile_headers_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, reinterpret_cast<const uint4 *>(hdr), rows, nb,
                       reinterpret_cast<uint4 *>(tiles));
    return (int)hipGetLastError();
}

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
