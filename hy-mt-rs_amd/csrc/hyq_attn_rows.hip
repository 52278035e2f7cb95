// Causal attention of a prefill chunk's query rows on the matrix cores
// (attention / attention_into at batch n, src/model.rs:949-1037: the query
// row of token t at position pos + t sees cache rows 0..=pos + t).
//
// Grid (splits, token blocks, kv heads), 256 threads (4 waves). A workgroup
// takes the query rows of one KV head for a block of tokens - 128 rows,
// row r = token (r / rep) of the block, query head r % rep of the group - and
// one split of `span` cache positions, walked in 32-position tiles; the
// split's (max, exp-sum, exp-weighted V sum) per query row goes to the same
// partials layout as the one-token kernel, [n][heads][splits][PART_STRIDE],
// and attn_merge_kernel forms the rows.
//
// Each wave owns 32 query rows and computes transposed products with
// v_mfma_f32_32x32x16_f16, so that a lane holds one query row (column
// lane % 32) and 16 of its positions or dims:
//   S^T [32 pos x 32 rows]  = K_tile [32 x 128] . Q^T
//   O^T [128 dims x 32 rows] += V_tile^T [128 x 32] . P^T
// The online softmax is then per lane, the two lanes of a row joined by one
// permlane32 swap. Every f32 operand x is split into f16 parts hi = f16(x),
// lo = f16(x - hi), and each product sums hi.hi + lo.hi + hi.lo in f32
// (the lo.lo term is below 2^-22 relative): scores and weighted sums keep
// close to f32 accuracy. Values must lie within the f16 range (|x| < 65504).
#include <hip/hip_runtime.h>

#include "hyq_f16rows.hpp"
#include "hyq_step.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int FA_ROWS = 128;   // query rows per workgroup (32 per wave)
constexpr int FA_TILE = 32;    // cache positions per tile
constexpr int FA_KP = ATT_D + 8; // K tile row pitch (halves)
constexpr int FA_VP = FA_TILE + 8; // V^T tile row pitch (halves)

__device__ __forceinline__ f32x16 mfma(const half8 &a, const half8 &b, const f32x16 &c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// x = hi + lo with hi = f16(x), lo = f16(x - hi)
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

__device__ __forceinline__ int fbits(float v) { return __builtin_bit_cast(int, v); }
__device__ __forceinline__ float bitsf(int v) { return __builtin_bit_cast(float, v); }

__global__ __launch_bounds__(256, 2) void attn_rows_kernel(
    const float *__restrict__ q, const float *__restrict__ kcache,
    const float *__restrict__ vcache, const int *__restrict__ pos_p, int n, int heads, int kvh,
    float scale, float *__restrict__ part, int splits, int span, int context)
{
    __shared__ __align__(16) _Float16 Khi[FA_TILE][FA_KP];
    __shared__ __align__(16) _Float16 Klo[FA_TILE][FA_KP];
    __shared__ __align__(16) _Float16 Vhi[ATT_D][FA_VP];
    __shared__ __align__(16) _Float16 Vlo[ATT_D][FA_VP];

    const int rep = heads / kvh;
    const int tpw = FA_ROWS / rep; // tokens per workgroup
    const int split = blockIdx.x, kh = blockIdx.z;
    const int tb = gridDim.y - 1 - blockIdx.y; // the longest rows first
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int h = lane >> 5;                   // lane half
    const int pos0 = *pos_p;
    const size_t kvw = (size_t)kvh * ATT_D;

    // the workgroup's last token and the positions its split covers
    const int tok0 = tb * tpw;
    const int tok_last = min(n, tok0 + tpw) - 1;
    const int p_begin = split * span;
    const int p_end = min(min(p_begin + span, context), pos0 + tok_last + 1);
    if (p_begin >= p_end) return; // no row of the block sees this split

    // this lane's query row
    const int r = 32 * wave + (lane & 31);
    const int tl = r / rep;
    const int token = tok0 + tl;
    const bool row_ok = r < tpw * rep && token < n;
    const int head = kh * rep + r % rep;
    const int qpos = pos0 + (row_ok ? token : 0); // sees positions <= qpos
    // the wave's last visible position (uniform): tiles past it are skipped
    const int wave_last = pos0 + min(n - 1, tok0 + (32 * wave + 31) / rep);

    half8 qhi[ATT_D / 16], qlo[ATT_D / 16];
    {
        const float *qr = q + ((size_t)(row_ok ? token : 0) * heads + head) * ATT_D + 8 * h;
#pragma unroll
        for (int kk = 0; kk < ATT_D / 16; ++kk) {
            const float4 a = *reinterpret_cast<const float4 *>(qr + 16 * kk);
            const float4 b = *reinterpret_cast<const float4 *>(qr + 16 * kk + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                _Float16 hi, lo;
                split_f16(row_ok ? v[i] : 0.f, hi, lo);
                qhi[kk][i] = hi;
                qlo[kk][i] = lo;
            }
        }
    }

    // tile loads: thread t fetches float4 d4 of rows {2pp, 2pp+1, 2pp+16, 2pp+17}
    const int d4 = t & 31, pp = t >> 5;
    float4 kr[4], vr[4];
    auto load_tile = [&](int p0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 2 * pp + (j & 1) + 16 * (j >> 1);
            const int p = p0 + row;
            const bool ok = p < p_end;
            const size_t off = (size_t)(ok ? p : p_begin) * kvw + (size_t)kh * ATT_D + 4 * d4;
            const float4 kv = *reinterpret_cast<const float4 *>(kcache + off);
            const float4 vv = *reinterpret_cast<const float4 *>(vcache + off);
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            kr[j] = ok ? kv : z;
            vr[j] = ok ? vv : z;
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 2 * pp + (j & 1) + 16 * (j >> 1);
            const float kv[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
            half4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                _Float16 a, b;
                split_f16(kv[i], a, b);
                hi[i] = a;
                lo[i] = b;
            }
            *reinterpret_cast<half4 *>(&Khi[row][4 * d4]) = hi;
            *reinterpret_cast<half4 *>(&Klo[row][4 * d4]) = lo;
        }
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
            const int row = 2 * pp + 16 * jp;
            const float4 a = vr[2 * jp], b = vr[2 * jp + 1];
            const float va[4] = {a.x, a.y, a.z, a.w}, vb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                half2 hi, lo;
                _Float16 x, y;
                split_f16(va[i], x, y);
                hi[0] = x;
                lo[0] = y;
                split_f16(vb[i], x, y);
                hi[1] = x;
                lo[1] = y;
                *reinterpret_cast<half2 *>(&Vhi[4 * d4 + i][row]) = hi;
                *reinterpret_cast<half2 *>(&Vlo[4 * d4 + i][row]) = lo;
            }
        }
    };

    f32x16 acc[ATT_D / 32];
#pragma unroll
    for (int j = 0; j < ATT_D / 32; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    load_tile(p_begin);
    for (int p0 = p_begin; p0 < p_end; p0 += FA_TILE) {
        __syncthreads(); // the previous tile's readers are done
        store_tile();
        if (p0 + FA_TILE < p_end) load_tile(p0 + FA_TILE);
        __syncthreads();
        if (p0 > wave_last) continue; // every row of this wave is before the tile

        // S^T = K Q^T: lane holds row (lane % 32) at positions 8g + 4h + (e & 3)
        f32x16 s;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
        for (int kk = 0; kk < ATT_D / 16; ++kk) {
            const half8 ahi = *reinterpret_cast<const half8 *>(&Khi[lane & 31][16 * kk + 8 * h]);
            const half8 alo = *reinterpret_cast<const half8 *>(&Klo[lane & 31][16 * kk + 8 * h]);
            s = mfma(ahi, qhi[kk], s);
            s = mfma(alo, qhi[kk], s);
            s = mfma(ahi, qlo[kk], s);
        }
        // scale, causal mask, online softmax (one row per lane pair)
        float tmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int p = p0 + 8 * (e >> 2) + 4 * h + (e & 3);
            const float v = (row_ok && p <= qpos && p < p_end) ? s[e] * scale : -INFINITY;
            s[e] = v;
            tmax = fmaxf(tmax, v);
        }
        tmax = wave::max_halves(tmax);
        const float m_new = fmaxf(m_run, tmax);
        const bool any = m_new != -INFINITY;
        const float corr = any ? expf(m_run - m_new) : 1.f;
        float rs = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float pe = (any && s[e] != -INFINITY) ? expf(s[e] - m_new) : 0.f;
            s[e] = pe;
            rs += pe;
        }
        rs = wave::sum_halves(rs);
        l_run = l_run * corr + rs;
        m_run = m_new;
#pragma unroll
        for (int j = 0; j < ATT_D / 32; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][e] *= corr;

        // P^T operands: positions 16kk + 8h + (0..7) of this lane's row,
        // half from the partner lane (lane ^ 32)
#pragma unroll
        for (int kk = 0; kk < FA_TILE / 16; ++kk) {
            float pv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const auto sw = __builtin_amdgcn_permlane32_swap(fbits(s[8 * kk + i]),
                                                                 fbits(s[8 * kk + 4 + i]),
                                                                 false, false);
                pv[i] = bitsf(sw[0]);
                pv[4 + i] = bitsf(sw[1]);
            }
            half8 phi, plo;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                _Float16 a, b;
                split_f16(pv[i], a, b);
                phi[i] = a;
                plo[i] = b;
            }
#pragma unroll
            for (int j = 0; j < ATT_D / 32; ++j) {
                const int d = 32 * j + (lane & 31);
                const half8 vhi = *reinterpret_cast<const half8 *>(&Vhi[d][16 * kk + 8 * h]);
                const half8 vlo = *reinterpret_cast<const half8 *>(&Vlo[d][16 * kk + 8 * h]);
                acc[j] = mfma(vhi, phi, acc[j]);
                acc[j] = mfma(vlo, phi, acc[j]);
                acc[j] = mfma(vhi, plo, acc[j]);
            }
        }
    }

    if (!row_ok) return;
    float *o = part + (((size_t)token * heads + head) * splits + split) * PART_STRIDE;
    if (h == 0) {
        o[0] = m_run;
        o[1] = l_run;
    }
    // acc[j][e]: dim 32j + 8(e / 4) + 4h + (e % 4)
#pragma unroll
    for (int j = 0; j < ATT_D / 32; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<float4 *>(o + 4 + 32 * j + 8 * g + 4 * h) =
                make_float4(acc[j][4 * g], acc[j][4 * g + 1], acc[j][4 * g + 2],
                            acc[j][4 * g + 3]);
}

// Merge of one token row's split partials over all heads (grid: the n
// tokens, 256 threads), reading only the splits the token sees (splits
// 0 .. (pos + chunk) / chunk - 1): per head M = max_s m_s, w_s =
// exp(m_s - M), row = (sum_s w_s acc_s) / (sum_s w_s l_s), sums in split
// order. It writes the f32 row to out (if given) and/or the row as f16 with
// its power-of-two scale (xh, rscale: the attention-output GEMM's operand,
// rows_to_f16_kernel's rounding). Dynamic LDS: the row (heads * 128 floats)
// and the per-(head, split) weights (heads * splits floats, twice).
__global__ __launch_bounds__(256) void merge_rows_kernel(const float *__restrict__ part,
                                                         int splits, int chunk, int heads,
                                                         const int *__restrict__ pos_p,
                                                         float *__restrict__ out,
                                                         _Float16 *__restrict__ xh,
                                                         float *__restrict__ rscale)
{
    extern __shared__ float ms[];
    const int tq = blockIdx.x, t = threadIdx.x;
    const int W = heads * ATT_D;
    float *row = ms;                 // [heads * 128]
    float *wt = ms + W;              // [heads][splits]: exp(m_s - M)
    float *den = wt + heads * splits; // [heads]
    const int nact = min((*pos_p + tq + chunk) / chunk, splits);
    const float *pt = part + (size_t)tq * heads * splits * PART_STRIDE;
    for (int h = t; h < heads; h += 256) {
        const float *ph = pt + (size_t)h * splits * PART_STRIDE;
        float M = -INFINITY;
        for (int sp = 0; sp < nact; ++sp) M = fmaxf(M, ph[(size_t)sp * PART_STRIDE]);
        float d = 0.f;
        for (int sp = 0; sp < nact; ++sp) {
            const float w = expf(ph[(size_t)sp * PART_STRIDE] - M);
            wt[h * splits + sp] = w;
            d += w * ph[(size_t)sp * PART_STRIDE + 1];
        }
        den[h] = d;
    }
    __syncthreads();
    float mx = 0.f;
    for (int i = t; i < W; i += 256) {
        const int h = i / ATT_D, dd = i % ATT_D;
        const float *ph = pt + (size_t)h * splits * PART_STRIDE + 4 + dd;
        float num = 0.f;
#pragma unroll 4
        for (int sp = 0; sp < nact; ++sp) num += wt[h * splits + sp] * ph[(size_t)sp * PART_STRIDE];
        const float v = num / den[h];
        row[i] = v;
        if (out) out[(size_t)tq * W + i] = v;
        mx = fmaxf(mx, fabsf(v));
        if (v != v) mx = INFINITY;
    }
    if (!xh) return;
    __shared__ float red[4];
    mx = wave::max64(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int e = f16_row_exponent(mx);
    const float inv = ldexpf(1.0f, -e);
    if (t == 0) rscale[tq] = ldexpf(1.0f, e);
    for (int i = t; i < W; i += 256) xh[(size_t)tq * W + i] = (_Float16)(row[i] * inv);
}

} // namespace

size_t merge_rows_lds(int heads, int splits)
{
    return ((size_t)heads * ATT_D + (size_t)heads * splits + heads) * 4;
}

int launch_attention_rows_f16(const float *q, const float *kcache, const float *vcache,
                              const int *pos, int n, int context, int heads, int kvh,
                              float *part, float *out, _Float16 *xh, float *rscale,
                              void *stream)
{
    if (n <= 0) return 0;
    const int rep = heads / kvh;
    if (rep < 1 || rep > ATT_MAX_REP) return (int)hipErrorInvalidValue;
    const int splits = prefill_attention_splits(context), span = prefill_attention_chunk(context);
    const size_t lds = merge_rows_lds(heads, splits);
    if (lds > 64 * 1024) return (int)hipErrorInvalidValue;
    const int tpw = FA_ROWS / rep;
    const float scale = 1.0f / sqrtf(128.0f);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(attn_rows_kernel, dim3(splits, (n + tpw - 1) / tpw, kvh), dim3(256), 0, st,
                       q, kcache, vcache, pos, n, heads, kvh, scale, part, splits, span, context);
    hipLaunchKernelGGL(merge_rows_kernel, dim3(n), dim3(256), lds, st, part, splits, span, heads,
                       pos, out, xh, rscale);
    return (int)hipGetLastError();
}

int launch_attention_rows(const float *q, const float *kcache, const float *vcache,
                          const int *pos, int n, int context, int heads, int kvh, float *part,
                          float *out, void *stream)
{
    if (n <= 0) return 0;
    const int splits = prefill_attention_splits(context);
    if (merge_rows_lds(heads, splits) <= 64 * 1024)
        return launch_attention_rows_f16(q, kcache, vcache, pos, n, context, heads, kvh, part,
                                         out, nullptr, nullptr, stream);
    // rows too wide for the one-workgroup-per-token merge: per-head merge
    const int rep = heads / kvh;
    if (rep < 1 || rep > ATT_MAX_REP) return (int)hipErrorInvalidValue;
    const int span = prefill_attention_chunk(context);
    const int tpw = FA_ROWS / rep;
    const float scale = 1.0f / sqrtf(128.0f);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(attn_rows_kernel, dim3(splits, (n + tpw - 1) / tpw, kvh), dim3(256), 0, st,
                       q, kcache, vcache, pos, n, heads, kvh, scale, part, splits, span, context);
    return launch_attention_merge_rows(part, splits, span, heads, pos, n, out, stream);
}

} // namespace hyq
