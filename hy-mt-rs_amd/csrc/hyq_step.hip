// Device-resident glue of the batch-1 decode step of the dense graph
// (Model::forward_into, src/model.rs:374-546) around the int8 GEMVs:
//   embed_row        embedding.row_into(token)              (src/model.rs:376)
//   rms_norm_q8      rms_norm_into + Q8::quantize_into      (:396-416, :785-830)
//   rope_norm_kv     rope_with_cache, per-head rms_norm of q and k (dense
//                    order: RoPE first), KvCache::append    (:425-452, :874-917)
//   attention        attention_into for one query token    (:949-1035)
//   argmax           greedy sampling                        (src/generation.rs:281-290)
// The current position and token live in device memory, so a whole step can
// be captured once in a HIP graph and replayed without host work.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hyq_decode.hpp"
#include "hyq_q8.hpp"
#include "hyq_step.hpp"
#include "hyq_wave.hpp"

namespace hyq {

namespace {

__device__ __forceinline__ float wave_sum(float v) { return wave::sum64(v); }

// ---- embedding rows (Weight::row_into with device-resident token ids) ----
// Grid (cols / 256, tokens): row blockIdx.y of out takes token[blockIdx.y]
// (clamped into [0, rows): the reference rejects an id past the table, which
// a device-side id cannot report, so it never reads outside the table).
template <int F>
__global__ __launch_bounds__(256) void embed_kernel(WView w, int cols, const int *__restrict__ token,
                                                    float *__restrict__ out)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= cols) return;
    // a device-resident id the host cannot check: clamped into the table
    const size_t row = (size_t)min(max(token[blockIdx.y], 0), w.rows - 1);
    out += (size_t)blockIdx.y * cols;
    const size_t blk = row * (size_t)w.nb + i / block_len(F);
    out[i] = dec::decode_plane_value<F>(w, blk, i % block_len(F));
}

// ---- rms_norm_into fused with the Q8 quantizer ----
// One workgroup per 256-value group; each recomputes sum(x^2) over the whole
// row (n <= 64 Ki values, read from L2) so that no cross-workgroup sync is
// needed. y = x * (w * scale) with scale = 1 / sqrt(mean(x^2) + eps) over
// whole 16-value steps and x * scale * w over the tail, the aarch64 arm's
// operation order (src/model.rs:791-822).
// x is the row ((x + p_0) + p_1) + ... with nparts partial rows p_k at
// parts + k * pstride (a K-split product's slices, added in the order the
// GEMV input stage adds them).
__global__ __launch_bounds__(256) void rms_norm_q8_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ w, int n,
                                                          float eps, float *__restrict__ y,
                                                          int8_t *q, float *s, int32_t *s16,
                                                          int32_t *s32, int32_t *s256,
                                                          const float *__restrict__ parts,
                                                          int nparts, int pstride)
{
    __shared__ float part[4];
    const int t = threadIdx.x;
    auto row4 = [&](int i) {
        float4 v = reinterpret_cast<const float4 *>(x)[i];
        for (int k = 0; k < nparts; ++k) {
            const float4 p = reinterpret_cast<const float4 *>(parts + (size_t)k * pstride)[i];
            v = make_float4(v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w);
        }
        return v;
    };
    auto row1 = [&](int i) {
        float v = x[i];
        for (int k = 0; k < nparts; ++k) v = v + parts[(size_t)k * pstride + i];
        return v;
    };
    float ss = 0.f;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (nparts == 0 || ((reinterpret_cast<uintptr_t>(parts) & 15) == 0 && pstride % 4 == 0))) {
        // all of this thread's float4 loads in flight together
        const int n4 = n / 4;
        int i = t;
        for (; i + 768 < n4; i += 1024) {
            const float4 a = row4(i), b = row4(i + 256), c = row4(i + 512), d = row4(i + 768);
            ss += (a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w) +
                  (b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w) +
                  (c.x * c.x + c.y * c.y + c.z * c.z + c.w * c.w) +
                  (d.x * d.x + d.y * d.y + d.z * d.z + d.w * d.w);
        }
        for (; i < n4; i += 256) {
            const float4 a = row4(i);
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
        for (int j = n4 * 4 + t; j < n; j += 256) {
            const float v = row1(j);
            ss += v * v;
        }
    } else {
        for (int i = t; i < n; i += 256) {
            const float v = row1(i);
            ss += v * v;
        }
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float variance = ss / (float)n;
    const float scale = 1.0f / sqrtf(variance + eps);
    const int g = blockIdx.x;
    const int len = min(256, n - g * 256);
    float v = 0.f;
    if (t < len) {
        const int i = g * 256 + t;
        v = i < (n & ~15) ? row1(i) * (w[i] * scale) : row1(i) * scale * w[i];
        if (y) y[i] = v;
    }
    q8_quantize_group(v, g, len, q, s, s16, s32, s256);
}

// ---- RoPE + per-head Q/K RMSNorm + KV append ----
// The per-head rms_norm follows RoPE in the dense graph and precedes it in
// hy_v3 (norm_first, src/model.rs:425-446); RoPE keeps each pair's length,
// so both orders normalise by the same mean square up to rounding.
// Workgroups [0, heads) rotate and normalise the query heads in place,
// [heads, heads+kv) the key heads into kcache[pos], [heads+kv, heads+2kv)
// copy the value heads into vcache[pos]. Lane j owns the NeoX pair
// (j, j + dim/2) (docs/reference.md:79), so dim/2 lanes per head. Grid y
// walks the tokens of a chunk: token y has rows q[y], k[y], v[y] and
// position *pos_p + y (rope at start + token, src/model.rs:919-925).
__global__ void rope_norm_kv_kernel(float *__restrict__ q, const float *__restrict__ k,
                                    const float *__restrict__ v, const float *__restrict__ qn,
                                    const float *__restrict__ kn,
                                    const float *__restrict__ freq, const int *__restrict__ pos_p,
                                    int heads, int kvh, int dim, float eps, int norm_first,
                                    float *__restrict__ kcache, float *__restrict__ vcache)
{
    const int b = blockIdx.x;
    const int j = threadIdx.x;
    const int half = dim / 2;
    const int pos = *pos_p + (int)blockIdx.y;
    const size_t kvw = (size_t)kvh * dim;
    q += (size_t)blockIdx.y * heads * dim;
    k += (size_t)blockIdx.y * kvw;
    v += (size_t)blockIdx.y * kvw;
    if (b >= heads + kvh) {
        if (pos < 0) return; // (a negative device position appends nothing)
        const int h = b - heads - kvh;
        float *dst = vcache + (size_t)pos * kvw + (size_t)h * dim;
        dst[j] = v[h * dim + j];
        dst[j + half] = v[h * dim + j + half];
        return;
    }
    const bool is_q = b < heads;
    const int h = is_q ? b : b - heads;
    const float *src = is_q ? q + (size_t)h * dim : k + (size_t)h * dim;
    const float a = src[j], c2 = src[j + half];
    const float ang = (float)pos * freq[j];
    const float cs = cosf(ang), sn = sinf(ang);
    const float *nw = is_q ? qn : kn;
    // rms_norm over the head (src/model.rs:832-870): scale = 1/sqrt(mean + eps)
    __shared__ float part[4];
    auto head_scale = [&](float u0, float u1) {
        float ss = wave_sum(u0 * u0 + u1 * u1);
        if ((j & 63) == 0) part[j >> 6] = ss;
        __syncthreads();
        ss = 0.f;
        for (int i = 0; i < (half + 63) / 64; ++i) ss += part[i];
        return 1.0f / sqrtf(ss / (float)dim + eps);
    };
    // the aarch64 arm's x * (w * scale) over whole 16-value steps, x * scale
    // * w over a tail (src/model.rs:837-865)
    const int body = dim & ~15;
    auto nrm = [&](float x, int i, float scale) {
        return i < body ? x * (nw[i] * scale) : x * scale * nw[i];
    };
    float o0, o1;
    if (norm_first) {
        const float scale = head_scale(a, c2);
        const float n0 = nrm(a, j, scale), n1 = nrm(c2, j + half, scale);
        o0 = n0 * cs - n1 * sn;
        o1 = n0 * sn + n1 * cs;
    } else {
        const float r0 = a * cs - c2 * sn;
        const float r1 = a * sn + c2 * cs;
        const float scale = head_scale(r0, r1);
        o0 = nrm(r0, j, scale);
        o1 = nrm(r1, j + half, scale);
    }
    if (is_q) {
        q[(size_t)h * dim + j] = o0;
        q[(size_t)h * dim + j + half] = o1;
    } else if (pos >= 0) {
        float *dst = kcache + (size_t)pos * kvw + (size_t)h * dim;
        dst[j] = o0;
        dst[j + half] = o1;
    }
}

// ---- attention over positions 0..=pos, in splits of `chunk` positions ----
// Grid (splits, kv_heads), 512 threads (8 waves, two per SIMD); only the
// splits that hold visible positions do work. Splits are small (32
// positions at contexts up to 2048) so that many CUs share the VALU work. A
// workgroup walks its split in ATT_SUB-position slices: thread t fetches
// float4 t % 32 of slice rows t / 32 and t / 32 + 16 of K and V, all loads in
// flight at once (the next slice's are issued before the current one is
// used), and stages them in LDS. The `rep` (<= 4) query heads of the KV head
// share every LDS read: head h = lane % 4, so the four heads' lanes of a
// 16-lane LDS pass read the same address.
//   scores  lane (h, q = lane / 4 % 4) of wave w dots head h with slice row
//           4w + lane / 16 over dims {4q + 16i .. +3}; row_ror DPP adds the
//           four quarters.
//   softmax the slice maximum and exp-sum per head over the wave's 4 rows by
//           permlane16/32 swaps, then over the 8 waves through LDS; the
//           workgroup keeps an online softmax (running max, exp-sum and
//           exp-weighted V sum).
//   V       lane (h, x = lane / 4) of wave w accumulates dim 16w + x of head h
//           over the slice rows.
// The split's (max, exp-sum, V sum) per query head goes to `part`
// ([heads][splits][PART_STRIDE]) for the merge (attn_merge_kernel).
//
// Grid z walks the query tokens of a prefill chunk whose keys and values are
// already in the cache: token z reads query row q[z], sees positions
// 0..=*pos_p + z (causal, src/model.rs:956-961) and writes partials block z.
//
// With `rope` set the workgroup first forms its query heads from the raw
// projection (rope_with_cache + the dense order's per-head rms_norm,
// src/model.rs:425-446, 874-917), and the split holding `pos` also forms the
// new key (RoPE + norm) and value, appends them to the caches
// (KvCache::append, src/model.rs:650-669) and uses them from LDS.

// RoPE (NeoX halves j, j+64) of one 128-wide head and its rms_norm (the
// aarch64 arm's x * (w * scale), src/model.rs:837-865), in the dense order
// (RoPE first) or the hy_v3 one (norm first); lane j of a full wave owns the
// pair.
__device__ __forceinline__ void rope_norm_pair(float a, float c2, float cs, float sn, float n0,
                                               float n1, float eps, bool norm_first, float &o0,
                                               float &o1)
{
    if (norm_first) {
        const float ss = wave_sum(a * a + c2 * c2);
        const float scale = 1.0f / sqrtf(ss / (float)ATT_D + eps);
        const float u0 = a * (n0 * scale), u1 = c2 * (n1 * scale);
        o0 = u0 * cs - u1 * sn;
        o1 = u0 * sn + u1 * cs;
        return;
    }
    const float r0 = a * cs - c2 * sn;
    const float r1 = a * sn + c2 * cs;
    const float ss = wave_sum(r0 * r0 + r1 * r1);
    const float scale = 1.0f / sqrtf(ss / (float)ATT_D + eps);
    o0 = r0 * (n0 * scale);
    o1 = r1 * (n1 * scale);
}

constexpr int ATT_WAVES = 8;
constexpr int ATT_THREADS = 64 * ATT_WAVES;

__global__ __launch_bounds__(ATT_THREADS) void attn_kernel(
    bool rope, bool norm_first, const float *__restrict__ q, const float *__restrict__ knew,
    const float *__restrict__ vnew, const float *__restrict__ qn, const float *__restrict__ kn,
    const float *__restrict__ freq, float eps, float *__restrict__ kcache,
    float *__restrict__ vcache, const int *__restrict__ pos_p, int heads, int kvh, float scale,
    float *__restrict__ part, int splits, int chunk, int context)
{
    constexpr int D = ATT_D;
    static_assert(ATT_SUB == 32 && ATT_WAVES == 8 && ATT_MAX_REP == 4 && D == 128,
                  "lane roles assume these");
    // (16-byte aligned: read and written as float4)
    __shared__ __align__(16) float Ks[ATT_SUB][D + 4];
    __shared__ __align__(16) float Vs[ATT_SUB][D];
    __shared__ __align__(16) float Qs[ATT_MAX_REP][D];
    __shared__ __align__(16) float Kn[D];
    __shared__ __align__(16) float Vn[D];
    __shared__ __align__(16) float Es[ATT_MAX_REP][ATT_SUB];     // the slice's exp weights
    __shared__ __align__(16) float Red[2][ATT_MAX_REP][ATT_WAVES]; // per-wave max / exp-sum
    const int split = blockIdx.x, kh = blockIdx.y, tq = blockIdx.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const size_t kvw = (size_t)kvh * D;
    q += (size_t)tq * heads * D;
    part += (size_t)tq * heads * splits * PART_STRIDE;
    const int p0 = split * chunk;
    const int rep = heads / kvh;
    // rope: wave w < rep forms query head w of the group (waves past `rep`
    // read the last head's row, in bounds, and do not use it)
    const bool has_q = wave < rep;
    const int hql = kh * rep + min(wave, rep - 1);
    // Loads in the order their values are needed, since they complete in
    // issue order: the small operands (query row, RoPE frequencies, norm
    // weights, the new key/value rows), then the first slice's K/V rows of
    // the allocated cache (clamped to `context`; rows past the visible ones
    // are masked out below), then the position. None of them depends on the
    // position, so all latencies overlap.
    float qa = 0.f, qb = 0.f, fr = 0.f, qn0 = 0.f, qn1 = 0.f, kn0 = 0.f, kn1 = 0.f;
    float ka = 0.f, kb = 0.f, va = 0.f, vb = 0.f;
    if (wave < ATT_MAX_REP) {
        qa = q[hql * D + lane];
        qb = q[hql * D + lane + D / 2];
        if (rope) {
            fr = freq[lane];
            qn0 = qn[lane];
            qn1 = qn[lane + D / 2];
            kn0 = kn[lane];
            kn1 = kn[lane + D / 2];
            ka = knew[kh * D + lane];
            kb = knew[kh * D + lane + D / 2];
            va = vnew[kh * D + lane];
            vb = vnew[kh * D + lane + D / 2];
        }
    }
    const float *kbase = kcache + (size_t)p0 * kvw + (size_t)kh * D;
    const float *vbase = vcache + (size_t)p0 * kvw + (size_t)kh * D;
    const int r0 = t >> 5, d4 = t & 31;
    float4 kr[2], vr[2];
    const int rows0 = min(ATT_SUB, context - p0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int pp = min(r0 + 16 * j, rows0 - 1);
        kr[j] = reinterpret_cast<const float4 *>(kbase + (size_t)pp * kvw)[d4];
        vr[j] = reinterpret_cast<const float4 *>(vbase + (size_t)pp * kvw)[d4];
    }
    const int pos = *pos_p + tq;
    const int visible = min(pos + 1, context); // no cache row past the allocation
    const int nact = (visible + chunk - 1) / chunk;
    if (split >= nact) {
        // The idle split consumes its loads as well (a store that a valid
        // position never takes), so the compiler cannot sink them below
        // this branch and behind the position's latency.
        const float z = (kr[0].x + vr[0].x) + (kr[1].x + vr[1].x);
        if (pos < 0 && z == 0.f) part[0] = z;
        return;
    }
    const int n = min(chunk, visible - p0);
    // the new position's row of this head is formed here, not read (and
    // appended only inside the allocation: a position the caller let reach
    // `context` attends to the cache without writing past it)
    const int pnew = rope && split == nact - 1 && pos < context ? pos - p0 : -1;
#define HYQ_ATT_LOAD(SB)                                                                       \
    _Pragma("unroll") for (int j = 0; j < 2; ++j)                                             \
    {                                                                                          \
        const int pp = (SB) + r0 + 16 * j;                                                     \
        if (pp < n && pp != pnew) {                                                            \
            kr[j] = reinterpret_cast<const float4 *>(kbase + (size_t)pp * kvw)[d4];             \
            vr[j] = reinterpret_cast<const float4 *>(vbase + (size_t)pp * kvw)[d4];             \
        } else {                                                                               \
            kr[j] = vr[j] = make_float4(0.f, 0.f, 0.f, 0.f);                                   \
        }                                                                                      \
    }
    if (wave < ATT_MAX_REP) {
        if (rope) {
            const float ang = (float)pos * fr;
            const float cs = cosf(ang), sn = sinf(ang);
            if (has_q) {
                float o0, o1;
                rope_norm_pair(qa, qb, cs, sn, qn0, qn1, eps, norm_first, o0, o1);
                Qs[wave][lane] = o0;
                Qs[wave][lane + D / 2] = o1;
            }
            if (pnew >= 0 && wave == 0) {
                float o0, o1;
                rope_norm_pair(ka, kb, cs, sn, kn0, kn1, eps, norm_first, o0, o1);
                Kn[lane] = o0;
                Kn[lane + D / 2] = o1;
                float *kdst = kcache + (size_t)pos * kvw + (size_t)kh * D;
                kdst[lane] = o0;
                kdst[lane + D / 2] = o1;
            }
            if (pnew >= 0 && wave == 1) {
                Vn[lane] = va;
                Vn[lane + D / 2] = vb;
                float *vdst = vcache + (size_t)pos * kvw + (size_t)kh * D;
                vdst[lane] = va;
                vdst[lane + D / 2] = vb;
            }
        } else if (has_q) {
            Qs[wave][lane] = qa;
            Qs[wave][lane + D / 2] = qb;
        }
    }
    // lane roles (see above); heads past `rep` idle
    const int hl = lane & 3;
    const bool hq_ok = hl < rep;
    const int qq = (lane >> 2) & 3;          // score phase: dim quarter
    const int srow = 4 * wave + (lane >> 4); // score phase: slice row
    const int vdim = 16 * wave + (lane >> 2); // V phase: output dim
    float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
    for (int sb = 0; sb < n; sb += ATT_SUB) {
        const int nn = min(ATT_SUB, n - sb);
        __syncthreads(); // the previous slice's readers are done (and Qs/Kn/Vn are ready)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int pp = r0 + 16 * j;
            float4 kv = kr[j], vv = vr[j];
            if (sb + pp >= n) kv = vv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sb + pp == pnew) {
                kv = *reinterpret_cast<const float4 *>(&Kn[4 * d4]);
                vv = *reinterpret_cast<const float4 *>(&Vn[4 * d4]);
            }
            *reinterpret_cast<float4 *>(&Ks[pp][4 * d4]) = kv;
            *reinterpret_cast<float4 *>(&Vs[pp][4 * d4]) = vv;
        }
        if (sb + ATT_SUB < n) HYQ_ATT_LOAD(sb + ATT_SUB)
        __syncthreads();
        // scores: four partial dots per lane (explicit fmaf: this file is
        // compiled without contraction for the decoders), then the quarters
        // by row_ror
        float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
            const float4 qv = *reinterpret_cast<const float4 *>(&Qs[hl][4 * qq + 16 * i]);
            const float4 kv = *reinterpret_cast<const float4 *>(&Ks[srow][4 * qq + 16 * i]);
            d0 = fmaf(qv.x, kv.x, d0);
            d1 = fmaf(qv.y, kv.y, d1);
            d2 = fmaf(qv.z, kv.z, d2);
            d3 = fmaf(qv.w, kv.w, d3);
        }
        float dot = (d0 + d1) + (d2 + d3);
        dot += wave::dpp<wave::DPP_ROR4>(dot);
        dot += wave::dpp<wave::DPP_ROR8>(dot);
        const bool live = hq_ok && srow < nn;
        const float sc = live ? dot * scale : -INFINITY;
        const float wmax = wave::max_halves(wave::max_rows2(sc));
        if (lane < ATT_MAX_REP) Red[0][hl][wave] = wmax;
        __syncthreads();
        float smax = -INFINITY;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; w += 4) {
            const float4 m4 = *reinterpret_cast<const float4 *>(&Red[0][hl][w]);
            smax = fmaxf(smax, fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w)));
        }
        const float m_new = fmaxf(m_run, smax);
        const float corr = expf(m_run - m_new);
        const float e = live ? expf(sc - m_new) : 0.f;
        if (qq == 0) Es[hl][srow] = e;
        const float wsum = wave::sum_halves(wave::sum_rows2(e));
        if (lane < ATT_MAX_REP) Red[1][hl][wave] = wsum;
        __syncthreads();
        float ssum = 0.f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; w += 4) {
            const float4 s4 = *reinterpret_cast<const float4 *>(&Red[1][hl][w]);
            ssum += (s4.x + s4.y) + (s4.z + s4.w);
        }
        l_run = l_run * corr + ssum;
        // V over the slice rows (rows past `nn` hold zeros and have e = 0),
        // even and odd rows in separate sums
        float ae = 0.f, ao = 0.f;
#pragma unroll
        for (int pp = 0; pp < ATT_SUB; pp += 4) {
            const float4 ev = *reinterpret_cast<const float4 *>(&Es[hl][pp]);
            ae = fmaf(ev.x, Vs[pp][vdim], ae);
            ao = fmaf(ev.y, Vs[pp + 1][vdim], ao);
            ae = fmaf(ev.z, Vs[pp + 2][vdim], ae);
            ao = fmaf(ev.w, Vs[pp + 3][vdim], ao);
        }
        acc = acc * corr + (ae + ao);
        m_run = m_new;
    }
#undef HYQ_ATT_LOAD
    if (hq_ok) {
        float *o = part + ((size_t)(kh * rep + hl) * splits + split) * PART_STRIDE;
        if (wave == 0 && lane < ATT_MAX_REP) {
            o[0] = m_run;
            o[1] = l_run;
        }
        o[4 + vdim] = acc;
    }
}

// Merge of the splits of one head: out = sum_s exp(m_s - M) acc_s /
// sum_s exp(m_s - M) l_s with M = max_s m_s. Grid (heads, 2), 256 threads:
// workgroup (h, y) forms dims 64y .. 64y + 63, wave g the splits g, g + 4,
// ... (lane = dim), and the four waves' sums are added through LDS in a
// fixed order. Lane s of every wave loads split s's (max, exp-sum) and forms
// its weight, which reaches the accumulation by readlane. All loads (split
// slots past `splits` clamped into bounds, slots past the visible splits
// ignored) are issued together with the position's, so one memory round
// trip is paid. Grid z walks the query tokens of a prefill chunk (token z at
// position *pos_p + z, partials block z, output row z).
template <int MS>
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ part,
                                                         int splits, int chunk,
                                                         const int *__restrict__ pos_p,
                                                         float *__restrict__ out)
{
    static_assert(MS % 4 == 0 && MS <= 64, "one split per lane, four waves");
    __shared__ float red[4][64];
    const int h = blockIdx.x, lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int d = 64 * blockIdx.y + lane;
    const int tq = blockIdx.z;
    const float *ph = part + ((size_t)tq * gridDim.x + h) * splits * PART_STRIDE;
    out += (size_t)tq * gridDim.x * ATT_D;
    const float2 ml =
        *reinterpret_cast<const float2 *>(ph + (size_t)min(lane, splits - 1) * PART_STRIDE);
    float a[MS / 4];
#pragma unroll
    for (int k = 0; k < MS / 4; ++k)
        a[k] = ph[(size_t)min(g + 4 * k, splits - 1) * PART_STRIDE + 4 + d];
    const int nact = min((*pos_p + tq + chunk) / chunk, splits);
    const bool live = lane < nact;
    const float M = wave::max64(live ? ml.x : -INFINITY);
    const float w = live ? expf(ml.x - M) : 0.f;
    const float den = wave::sum64(w * (live ? ml.y : 0.f));
    float num = 0.f;
#pragma unroll
    for (int k = 0; k < MS / 4; ++k) // a select, not a branch: the loads stay hoisted
        num += wave::lane(w, g + 4 * k) * (g + 4 * k < nact ? a[k] : 0.f);
    red[g][lane] = num;
    __syncthreads();
    if (g == 0) out[h * ATT_D + d] = ((red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane])) / den;
}

// out = ((x + p[0]) + p[1]) + ... over np partial rows (p[k] = parts + k *
// stride): the hidden row as the next stage forms it.
__global__ void sum_parts_kernel(const float *__restrict__ x, const float *__restrict__ parts,
                                 int np, int stride, int n, float *__restrict__ out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = x[i];
    for (int k = 0; k < np; ++k) v += parts[(size_t)k * stride + i];
    out[i] = v;
}

__global__ void zero_u32_kernel(unsigned *p, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// ---- greedy argmax (src/generation.rs:281-290) ----
// The reference keeps (best, value) = (0, x[0]) and takes index i only when
// x[i] > value: the first maximum wins, a NaN is never taken, and a NaN at
// index 0 keeps token 0 (no later value compares greater than it). In
// parallel: every non-NaN value is a candidate, candidates reduce by larger
// value then smaller index, and a NaN x[0] forces token 0. Whenever x[0] is
// not NaN it is itself a candidate, so the result is a valid index; it is
// still clamped into [0, n) before it is stored, because the decode loop
// embeds it as the next token. Pass 1: each workgroup reduces a slice to
// (value, index), with bit 31 of the index set when the slice holds a
// non-finite value (forward_into rejects non-finite logits,
// src/model.rs:540-543); pass 2: one workgroup reduces the partials, stores
// the token and (in the decode loop) advances the step state and records the
// non-finite flag there.
constexpr int ARGMAX_NONFINITE = (int)0x80000000;

__device__ __forceinline__ void better(float &v, int &i, float ov, int oi)
{
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ x, int n,
                                                             float *__restrict__ pv,
                                                             int *__restrict__ pi)
{
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ int sf[4];
    const int t = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    bool nonfinite = false;
    // eight values per thread in flight at once (clamped into bounds, the
    // surplus ignored); the grid makes one round enough up to 131072 values
    const int stride = gridDim.x * 256;
    for (int base = blockIdx.x * 256 + t; base < n; base += 8 * stride) {
        float xv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) xv[u] = x[min(base + u * stride, n - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (base + u * stride < n) {
                nonfinite |= !isfinite(xv[u]);
                if (!isnan(xv[u])) better(v, idx, xv[u], base + u * stride);
            }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    const bool any_nf = __any(nonfinite);
    if ((t & 63) == 0) {
        sv[t >> 6] = v;
        si[t >> 6] = idx;
        sf[t >> 6] = any_nf;
    }
    __syncthreads();
    if (t == 0) {
        int f = sf[0];
        for (int w = 1; w < 4; ++w) {
            better(v, idx, sv[w], si[w]);
            f |= sf[w];
        }
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = idx | (f ? ARGMAX_NONFINITE : 0);
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float *__restrict__ x, int n,
                                                          const float *__restrict__ pv,
                                                          const int *__restrict__ pi, int np,
                                                          int *__restrict__ token,
                                                          StepState *st, int *history)
{
    const int t = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    bool nonfinite = false;
    for (int i = t; i < np; i += 64) {
        const int pii = pi[i];
        nonfinite |= (pii & ARGMAX_NONFINITE) != 0;
        better(v, idx, pv[i], pii & ~ARGMAX_NONFINITE);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    const bool any_nf = __any(nonfinite);
    if (t == 0) {
        if (isnan(x[0])) idx = 0;
        idx = min(max(idx, 0), n - 1);
        *token = idx;
        if (st) {
            if (history && st->step < st->history_cap) history[st->step] = idx;
            st->step += 1;
            st->pos += 1;
            if (any_nf) st->nonfinite = 1;
        }
    }
}

// The argmax's final pass fused with the next step's embedding row: every
// workgroup's first wave reduces the np partials (as argmax_final_kernel),
// workgroup 0 alone stores the token and advances the step state, and each
// workgroup decodes 256 values of the token's row of w into out (as
// embed_kernel does), so the decode loop needs no embedding launch.
template <int F>
__global__ __launch_bounds__(256) void argmax_final_embed_kernel(
    const float *__restrict__ x, int n, const float *__restrict__ pv, const int *__restrict__ pi,
    int np, int *__restrict__ token, StepState *st, int *history, WView w, int cols,
    float *__restrict__ out)
{
    __shared__ int s_idx;
    const int t = threadIdx.x;
    if (t < 64) {
        float v = -INFINITY;
        int idx = 0x7fffffff;
        bool nonfinite = false;
        for (int i = t; i < np; i += 64) {
            const int pii = pi[i];
            nonfinite |= (pii & ARGMAX_NONFINITE) != 0;
            better(v, idx, pv[i], pii & ~ARGMAX_NONFINITE);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
        const bool any_nf = __any(nonfinite);
        if (t == 0) {
            if (isnan(x[0])) idx = 0;
            idx = min(max(idx, 0), n - 1);
            s_idx = idx;
            if (blockIdx.x == 0) {
                *token = idx;
                if (st) {
                    if (history && st->step < st->history_cap) history[st->step] = idx;
                    st->step += 1;
                    st->pos += 1;
                    if (any_nf) st->nonfinite = 1;
                }
            }
        }
    }
    __syncthreads();
    const int i = blockIdx.x * 256 + t;
    if (i >= cols) return;
    const size_t row = (size_t)min(s_idx, w.rows - 1);
    const size_t blk = row * (size_t)w.nb + i / block_len(F);
    out[i] = dec::decode_plane_value<F>(w, blk, i % block_len(F));
}

} // namespace

int launch_argmax_embed(const float *x, int n, float *pv, int *pi, int *token, StepState *st,
                        int *history, int fmt, WView w, int cols, float *out, void *stream)
{
    const int np = argmax_partials(n);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(np), dim3(256), 0, s, x, n, pv, pi);
    const dim3 grid((cols + 255) / 256), block(256);
#define HYQ_AE(F)                                                                              \
    case F: hipLaunchKernelGGL(argmax_final_embed_kernel<F>, grid, block, 0, s, x, n, pv, pi,     \
                               np, token, st, history, w, cols, out);                            \
        break;
    switch (fmt) {
        HYQ_AE(Q2_0C)
        HYQ_AE(STQ1_0)
        HYQ_AE(Q4_K)
        HYQ_AE(Q6_K)
        HYQ_AE(Q8_0)
        HYQ_AE(F32)
        HYQ_AE(F16)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_AE
    return (int)hipGetLastError();
}

int launch_embed_row(int fmt, WView w, int cols, const int *token, float *out, void *stream)
{
    return launch_embed_rows(fmt, w, cols, token, 1, out, stream);
}

int launch_embed_rows(int fmt, WView w, int cols, const int *tokens, int n, float *out,
                      void *stream)
{
    if (n <= 0) return 0;
    dim3 grid((cols + 255) / 256, n), block(256);
    hipStream_t st = (hipStream_t)stream;
#define HYQ_EMB(F)                                                                             \
    case F: hipLaunchKernelGGL(embed_kernel<F>, grid, block, 0, st, w, cols, tokens, out); break;
    switch (fmt) {
        HYQ_EMB(Q2_0C)
        HYQ_EMB(STQ1_0)
        HYQ_EMB(Q4_K)
        HYQ_EMB(Q6_K)
        HYQ_EMB(Q8_0)
        HYQ_EMB(F32)
        HYQ_EMB(F16)
    default: return (int)hipErrorInvalidValue;
    }
#undef HYQ_EMB
    return (int)hipGetLastError();
}

int launch_rms_norm_q8(const float *x, const float *w, int n, float eps, float *y, int8_t *q,
                       float *s, int32_t *s16, int32_t *s32, int32_t *s256, void *stream,
                       const float *parts, int nparts, int pstride)
{
    hipLaunchKernelGGL(rms_norm_q8_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, x, w, n, eps, y, q, s, s16, s32, s256, parts, nparts,
                       pstride);
    return (int)hipGetLastError();
}

int launch_rope_norm_kv(float *q, const float *k, const float *v, const float *qn,
                        const float *kn, const float *freq, const int *pos, int heads, int kvh,
                        int dim, float eps, float *kcache, float *vcache, void *stream,
                        bool norm_first)
{
    return launch_rope_norm_kv_rows(q, k, v, qn, kn, freq, pos, 1, heads, kvh, dim, eps, kcache,
                                    vcache, stream, norm_first);
}

int launch_rope_norm_kv_rows(float *q, const float *k, const float *v, const float *qn,
                             const float *kn, const float *freq, const int *pos, int n,
                             int heads, int kvh, int dim, float eps, float *kcache,
                             float *vcache, void *stream, bool norm_first)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(rope_norm_kv_kernel, dim3(heads + 2 * kvh, n), dim3(dim / 2), 0,
                       (hipStream_t)stream, q, k, v, qn, kn, freq, pos, heads, kvh, dim, eps,
                       (int)norm_first, kcache, vcache);
    return (int)hipGetLastError();
}

int attention_chunk(int context)
{
    // ATT_SUB-position multiples, at most ATT_MAX_SPLITS splits (the merge
    // holds one split per lane)
    const int per = (context + ATT_MAX_SPLITS - 1) / ATT_MAX_SPLITS;
    return (per + ATT_SUB - 1) / ATT_SUB * ATT_SUB;
}

int attention_splits(int context)
{
    const int c = attention_chunk(context);
    return (context + c - 1) / c;
}

int prefill_attention_chunk(int context)
{
    // n query tokens already fill the machine; splits of at least 128
    // positions keep partials and merge work small
    return std::max(128, attention_chunk(context));
}

int prefill_attention_splits(int context)
{
    const int c = prefill_attention_chunk(context);
    return (context + c - 1) / c;
}

int launch_sum_parts(const float *x, const float *parts, int np, int stride, int n, float *out,
                     void *stream)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(sum_parts_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, x, parts, np, stride, n, out);
    return (int)hipGetLastError();
}

int launch_zero_u32(unsigned *p, int n, void *stream)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       p, n);
    return (int)hipGetLastError();
}

// The merge, instantiated for the smallest split bound that covers `splits`.
static void launch_merge(const float *part, int splits, int chunk, int heads, const int *pos,
                         float *out, hipStream_t st, int tokens = 1)
{
    const dim3 grid(heads, 2, tokens);
    if (splits <= 16)
        hipLaunchKernelGGL(attn_merge_kernel<16>, grid, dim3(256), 0, st, part, splits, chunk,
                           pos, out);
    else if (splits <= 32)
        hipLaunchKernelGGL(attn_merge_kernel<32>, grid, dim3(256), 0, st, part, splits, chunk,
                           pos, out);
    else
        hipLaunchKernelGGL(attn_merge_kernel<ATT_MAX_SPLITS>, grid, dim3(256), 0, st, part,
                           splits, chunk, pos, out);
}

int launch_attention(const float *q, const float *kcache, const float *vcache, const int *pos,
                     int context, int heads, int kvh, float *part, float *out, void *stream)
{
    const int splits = attention_splits(context), chunk = attention_chunk(context);
    const float scale = 1.0f / sqrtf(128.0f);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(attn_kernel, dim3(splits, kvh), dim3(ATT_THREADS), 0, st, false, false, q, nullptr,
                       nullptr, nullptr, nullptr, nullptr, 0.f, const_cast<float *>(kcache),
                       const_cast<float *>(vcache), pos, heads, kvh, scale, part, splits, chunk,
                       context);
    launch_merge(part, splits, chunk, heads, pos, out, st);
    return (int)hipGetLastError();
}

int launch_attention_merge_rows(const float *part, int splits, int chunk, int heads,
                                const int *pos, int n, float *out, void *stream)
{
    if (n <= 0) return 0;
    launch_merge(part, splits, chunk, heads, pos, out, (hipStream_t)stream, n);
    return (int)hipGetLastError();
}

int launch_attention_merge(const float *part, int context, int heads, const int *pos,
                           float *out, void *stream)
{
    launch_merge(part, attention_splits(context), attention_chunk(context), heads, pos, out,
                 (hipStream_t)stream);
    return (int)hipGetLastError();
}

int launch_attention_rope(const float *q, const float *k, const float *v, const float *qn,
                          const float *kn, const float *freq, float eps, float *kcache,
                          float *vcache, const int *pos, int context, int heads, int kvh,
                          float *part, void *stream, bool norm_first)
{
    const int splits = attention_splits(context), chunk = attention_chunk(context);
    const float scale = 1.0f / sqrtf(128.0f);
    hipLaunchKernelGGL(attn_kernel, dim3(splits, kvh), dim3(ATT_THREADS), 0, (hipStream_t)stream, true, norm_first, q,
                       k, v, qn, kn, freq, eps, kcache, vcache, pos, heads, kvh, scale, part,
                       splits, chunk, context);
    return (int)hipGetLastError();
}

int argmax_partials(int n) { return std::min(64, std::max(1, (n + 2047) / 2048)); }

int launch_argmax(const float *x, int n, float *pv, int *pi, int *token, StepState *st,
                  int *history, void *stream)
{
    const int np = argmax_partials(n);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(np), dim3(256), 0, s, x, n, pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, s, x, n, pv, pi, np, token, st,
                       history);
    return (int)hipGetLastError();
}

} // namespace hyq
