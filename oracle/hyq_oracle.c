/*
 * CPU oracle for the quantized matrix-product path of hy-mt-rs.
 *
 * TEST INFRASTRUCTURE ONLY: the reference results for tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg. Nothing in the product library links it.
 * The pinning of each function is listed in hyq_oracle.h.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so that a*b+c stays two
 * roundings as in the Rust source, which never contracts).
 */
#include "hyq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------ */
/* Geometry: DType::block_len / block_bytes (src/quant.rs:43-62).            */
/* ------------------------------------------------------------------------ */
int hyqo_block_len(int dtype)
{
    switch (dtype) {
    case HYQO_F32:
    case HYQO_F16: return 1;
    case HYQO_Q8_0: return 32;
    case HYQO_Q2_0C: return 512;
    case HYQO_Q4_K:
    case HYQO_Q6_K:
    case HYQO_STQ1_0: return 256;
    default: return -1;
    }
}

int hyqo_block_bytes(int dtype)
{
    switch (dtype) {
    case HYQO_F32: return 4;
    case HYQO_F16: return 2;
    case HYQO_Q4_K: return 144;
    case HYQO_Q6_K: return 210;
    case HYQO_Q8_0: return 34;
    case HYQO_Q2_0C: return 130;
    case HYQO_STQ1_0: return 42;
    default: return -1;
    }
}

static size_t row_bytes_of(int dtype, size_t cols)
{
    return cols / (size_t)hyqo_block_len(dtype) * (size_t)hyqo_block_bytes(dtype);
}

/* Exact IEEE binary16 -> binary32, as half::f16::to_f32 (half 2.7.1,
 * src/quant.rs:844-847): subnormals are scaled exactly, NaN gets the quiet bit. */
float hyqo_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            float f = (float)man * 5.9604644775390625e-08f; /* man * 2^-24, exact */
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static float half_at(const uint8_t *p)
{
    return hyqo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* STQ_CODEBOOK (src/quant.rs:1081-1084), ggml-derived (MIT; the notice is in
 * THIRD_PARTY_NOTICES.md at the top of this repository). Index = sign<<4 | nibble; entry
 * holds four 2-bit codes, digit = code - 1. */
static const uint8_t STQ_CODEBOOK[32] = {
    0xa9, 0x89, 0x29, 0x09, 0xa6, 0x86, 0x26, 0x06, 0x9a, 0x92, 0x1a, 0x12, 0x6a, 0x62, 0x4a, 0x42,
    0x01, 0x21, 0x81, 0xa1, 0x04, 0x24, 0x84, 0xa4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68,
};

/* STQ integer digits of one 42-byte block in output order: group g's lane p
 * goes to (g/16)*64 + g%16 + 16p (stq_digits_scalar, src/quant.rs:1104-1123;
 * docs/reference.md:53). */
static void stq_int_digits(const uint8_t *b, int8_t *digits)
{
    for (int g = 0; g < 64; ++g) {
        int code = (b[g >> 1] >> (4 * (g % 2))) & 15;
        int sign = (b[32 + (g >> 3)] >> (g & 7)) & 1;
        int e = STQ_CODEBOOK[(sign << 4) | code];
        for (int p = 0; p < 4; ++p)
            digits[(g / 16) * 64 + g % 16 + 16 * p] = (int8_t)(((e >> (2 * p)) & 3) - 1);
    }
}

/* Q4_K 6-bit scale/min unpacking (src/quant.rs:2441-2451). */
static void q4k_scale_min(const uint8_t *scales, int j, int *s, int *m)
{
    if (j < 4) {
        *s = scales[j] & 63;
        *m = scales[j + 4] & 63;
    } else {
        *s = (scales[j + 4] & 15) | ((scales[j - 4] >> 6) << 4);
        *m = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
    }
}

/* Q6_K 6-bit code of output lane (chunk, p, half, i) (src/quant.rs:2462-2483). */
static int q6k_code(const uint8_t *x, int chunk, int p, int hf, int i)
{
    const uint8_t *ql = x + chunk * 64;
    const uint8_t *qh = x + 128 + chunk * 32;
    int nib = (p >> 1) * 4;
    int bits = 2 * p;
    int qv = ql[hf * 16 + (p & 1) * 32 + i];
    int hv = qh[hf * 16 + i];
    return ((qv >> nib) & 15) | (((hv >> bits) & 3) << 4);
}

/* ------------------------------------------------------------------------ */
/* decode / decode_unchecked (src/quant.rs:1066-1079, 2405-2486).           */
/* Operation order follows the source exactly; every product is one f32     */
/* rounding (the file is built with -ffp-contract=off).                     */
/* ------------------------------------------------------------------------ */
static void decode_block(int dtype, const uint8_t *x, float *y)
{
    switch (dtype) {
    case HYQO_F32: memcpy(y, x, 4); break;
    case HYQO_F16: y[0] = half_at(x); break;
    case HYQO_Q8_0: {
        float d = half_at(x);
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)x[2 + i];
        break;
    }
    case HYQO_Q2_0C: {
        float d = half_at(x);
        for (int i = 0; i < 512; ++i)
            y[i] = (float)(2 * ((x[2 + i / 4] >> (2 * (i % 4))) & 3) - 3) * d;
        break;
    }
    case HYQO_STQ1_0: {
        float d = half_at(x + 40);
        int8_t digits[256];
        stq_int_digits(x, digits);
        for (int i = 0; i < 256; ++i) y[i] = (float)digits[i] * d;
        break;
    }
    case HYQO_Q4_K: {
        float d = half_at(x);
        float dmin = half_at(x + 2);
        const uint8_t *scales = x + 4;
        for (int group = 0; group < 4; ++group) {
            int s1, m1i, s2, m2i;
            q4k_scale_min(scales, group * 2, &s1, &m1i);
            q4k_scale_min(scales, group * 2 + 1, &s2, &m2i);
            float d1 = d * (float)s1, m1 = dmin * (float)m1i;
            float d2 = d * (float)s2, m2 = dmin * (float)m2i;
            for (int l = 0; l < 32; ++l) {
                int q = x[16 + group * 32 + l];
                y[group * 64 + l] = d1 * (float)(q & 15) - m1;
                y[group * 64 + 32 + l] = d2 * (float)(q >> 4) - m2;
            }
        }
        break;
    }
    case HYQO_Q6_K: {
        float d = half_at(x + 208);
        const uint8_t *sc = x + 192;
        for (int chunk = 0; chunk < 2; ++chunk)
            for (int p = 0; p < 4; ++p)
                for (int hf = 0; hf < 2; ++hf) {
                    float s = d * (float)(int8_t)sc[chunk * 8 + 2 * p + hf];
                    for (int i = 0; i < 16; ++i)
                        y[chunk * 128 + p * 32 + hf * 16 + i] =
                            s * (float)(q6k_code(x, chunk, p, hf, i) - 32);
                }
        break;
    }
    default: break;
    }
}

int hyqo_decode(int dtype, const uint8_t *bytes, size_t nbytes, float *out, size_t n)
{
    int bl = hyqo_block_len(dtype), bb = hyqo_block_bytes(dtype);
    if (bl <= 0) return -1;
    if (n % (size_t)bl != 0) return -1;                 /* partial output block */
    if (nbytes != n / (size_t)bl * (size_t)bb) return -1; /* wrong byte count */
    for (size_t b = 0; b < n / (size_t)bl; ++b)
        decode_block(dtype, bytes + b * (size_t)bb, out + b * (size_t)bl);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Q8 activations (src/quant.rs:849-991).                                   */
/* ------------------------------------------------------------------------ */
static int8_t sat_i8_from_rne(float v)
{
    /* vcvtnq_s32_f32 (round to nearest, ties to even; NaN -> 0; saturating),
     * then vqmovn_s32 / vqmovn_s16: saturate to [-128, 127]. */
    if (v != v) return 0;
    float r = rintf(v); /* default rounding mode is round-to-nearest-even */
    if (r > 127.f) return 127;
    if (r < -128.f) return -128;
    return (int8_t)r;
}

static int8_t tail_round(float v)
{
    /* (activations * inverse).round().clamp(-127., 127.) as i8 (src/quant.rs:988):
     * round half away from zero; NaN as i8 is 0. */
    if (v != v) return 0;
    float r = roundf(v);
    if (r > 127.f) r = 127.f;
    if (r < -127.f) r = -127.f;
    return (int8_t)r;
}

/* max_abs_neon (src/quant.rs:869-892): vmaxq_f32 / vmaxvq_f32 (FMAX,
 * FMAXV) over the whole 16-value steps, starting from 0: any NaN there makes
 * the maximum NaN. The tail then folds in with f32::max, which returns the
 * other operand when one is NaN (fmaxf), so a tail value replaces a NaN
 * maximum. With max NaN (or 0), `max > 0.` fails: scale and inverse are 0
 * and every code of the group is 0 (NaN * 0 converts to 0). */
static float group_max_abs(const float *x, size_t len)
{
    size_t vec = len / 16 * 16;
    float max = 0.f;
    int nan = 0;
    for (size_t i = 0; i < vec; ++i) {
        float a = fabsf(x[i]);
        if (a != a) nan = 1;
        else if (a > max) max = a;
    }
    if (nan) max = NAN;
    for (size_t i = vec; i < len; ++i) max = fmaxf(max, fabsf(x[i]));
    return max;
}

void hyqo_q8_quantize(const float *x, size_t n, int8_t *q, float *scales)
{
    for (size_t g0 = 0, gi = 0; g0 < n; g0 += 256, ++gi) {
        size_t len = n - g0 < 256 ? n - g0 : 256;
        float max = group_max_abs(x + g0, len);
        float scale = 0.f, inverse = 0.f;
        if (max > 0.f) {
            scale = max / 127.f;
            inverse = 127.f / max;
        }
        scales[gi] = scale;
        size_t vec = len / 16 * 16;
        for (size_t i = 0; i < vec; ++i) q[g0 + i] = sat_i8_from_rne(x[g0 + i] * inverse);
        for (size_t i = vec; i < len; ++i) q[g0 + i] = tail_round(x[g0 + i] * inverse);
    }
}

void hyqo_q8_deinterleave_q2c(const int8_t *q, size_t n, int8_t *out)
{
    size_t i = 0;
    for (; i + 64 <= n; i += 64)
        for (int k = 0; k < 4; ++k)
            for (int j = 0; j < 16; ++j) out[i + 16 * k + j] = q[i + 4 * j + k];
    for (; i < n; ++i) out[i] = q[i];
}

/* ------------------------------------------------------------------------ */
/* Integer block sums.                                                      */
/* ------------------------------------------------------------------------ */
int hyqo_isums_per_row(int dtype, size_t cols)
{
    switch (dtype) {
    case HYQO_STQ1_0: return (int)(cols / 256);
    case HYQO_Q2_0C: return (int)(cols / 256);
    case HYQO_Q6_K: return (int)(cols / 256 * 16);
    case HYQO_Q4_K: return (int)(cols / 256 * 2);
    case HYQO_Q8_0: return (int)(cols / 32);
    default: return -1;
    }
}

int hyqo_row_isums(int dtype, const uint8_t *row, size_t cols, const int8_t *q, int32_t *out)
{
    int bl = hyqo_block_len(dtype), bb = hyqo_block_bytes(dtype);
    if (bl <= 0 || dtype == HYQO_F32 || dtype == HYQO_F16 || cols % (size_t)bl) return -1;
    size_t nb = cols / (size_t)bl;
    int n = 0;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t *x = row + b * (size_t)bb;
        const int8_t *a = q + b * (size_t)bl;
        switch (dtype) {
        case HYQO_STQ1_0: {
            int8_t dg[256];
            stq_int_digits(x, dg);
            int32_t s = 0;
            for (int i = 0; i < 256; ++i) s += dg[i] * a[i];
            out[n++] = s;
            break;
        }
        case HYQO_Q2_0C:
            for (int h = 0; h < 2; ++h) {
                int32_t s = 0;
                for (int i = h * 256; i < h * 256 + 256; ++i)
                    s += (2 * ((x[2 + i / 4] >> (2 * (i % 4))) & 3) - 3) * a[i];
                out[n++] = s;
            }
            break;
        case HYQO_Q6_K:
            /* plane index = chunk*8 + 2p + half = the sub-scale index */
            for (int chunk = 0; chunk < 2; ++chunk)
                for (int p = 0; p < 4; ++p)
                    for (int hf = 0; hf < 2; ++hf) {
                        int32_t s = 0;
                        for (int i = 0; i < 16; ++i)
                            s += (q6k_code(x, chunk, p, hf, i) - 32) *
                                 a[chunk * 128 + p * 32 + hf * 16 + i];
                        out[n + chunk * 8 + 2 * p + hf] = s;
                    }
            n += 16;
            break;
        case HYQO_Q4_K: {
            int32_t A = 0, B = 0;
            for (int j = 0; j < 8; ++j) {
                int sj, mj;
                q4k_scale_min(x + 4, j, &sj, &mj);
                int group = j / 2, hi = j % 2;
                int32_t qx = 0, xs = 0;
                for (int l = 0; l < 32; ++l) {
                    int qb = x[16 + group * 32 + l];
                    int nib = hi ? (qb >> 4) : (qb & 15);
                    int act = a[group * 64 + hi * 32 + l];
                    qx += nib * act;
                    xs += act;
                }
                A += sj * qx;
                B += mj * xs;
            }
            out[n++] = A;
            out[n++] = B;
            break;
        }
        case HYQO_Q8_0: {
            int32_t s = 0;
            for (int i = 0; i < 32; ++i) s += (int8_t)x[2 + i] * a[i];
            out[n++] = s;
            break;
        }
        default: return -1;
        }
    }
    return n;
}

static double row_magnitude(int dtype, const uint8_t *row, size_t cols, const int8_t *q,
                            const float *s, float *scratch)
{
    hyqo_decode(dtype, row, row_bytes_of(dtype, cols), scratch, cols);
    double mag = 0.0;
    for (size_t i = 0; i < cols; ++i)
        mag += fabs((double)scratch[i] * (double)q[i] * (double)s[i / 256]);
    return mag;
}

void hyqo_gemv_q8_f64(int dtype, const uint8_t *w, size_t rows, size_t cols, const int8_t *q,
                      const float *s, double *y, double *mag)
{
    size_t rb = row_bytes_of(dtype, cols);
    int per = hyqo_isums_per_row(dtype, cols);
    int32_t *is = (int32_t *)malloc(sizeof(int32_t) * (size_t)(per > 0 ? per : 1));
    float *scratch = (float *)malloc(sizeof(float) * cols);
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t *row = w + r * rb;
        hyqo_row_isums(dtype, row, cols, q, is);
        double acc = 0.0;
        int bl = hyqo_block_len(dtype), bb = hyqo_block_bytes(dtype);
        for (size_t b = 0; b < cols / (size_t)bl; ++b) {
            const uint8_t *x = row + b * (size_t)bb;
            switch (dtype) {
            case HYQO_STQ1_0: {
                float bs = half_at(x + 40) * s[b]; /* src/quant.rs:1512 */
                acc += (double)is[b] * (double)bs;
                break;
            }
            case HYQO_Q2_0C: {
                float d = half_at(x);
                for (int h = 0; h < 2; ++h) {
                    float sc = d * s[2 * b + h]; /* src/quant.rs:1896,1925 */
                    acc += (double)is[2 * b + h] * (double)sc;
                }
                break;
            }
            case HYQO_Q6_K: {
                float d = half_at(x + 208) * s[b]; /* src/quant.rs:2258 */
                for (int k = 0; k < 16; ++k) {
                    float plane = d * (float)(int8_t)x[192 + k]; /* :2281 */
                    acc += (double)is[16 * b + k] * (double)plane;
                }
                break;
            }
            case HYQO_Q4_K: {
                double d = half_at(x), dmin = half_at(x + 2);
                acc += (double)s[b] * (d * (double)is[2 * b] - dmin * (double)is[2 * b + 1]);
                break;
            }
            case HYQO_Q8_0: {
                double d = half_at(x);
                acc += d * (double)s[b / 8] * (double)is[b];
                break;
            }
            default: break;
            }
        }
        y[r] = acc;
        if (mag) mag[r] = row_magnitude(dtype, row, cols, q, s, scratch);
    }
    free(is);
    free(scratch);
}

void hyqo_gemv_q8_bruteforce(int dtype, const uint8_t *w, size_t rows, size_t cols,
                             const int8_t *q, const float *s, double *y, double *mag)
{
    size_t rb = row_bytes_of(dtype, cols);
    float *dec = (float *)malloc(sizeof(float) * cols);
    for (size_t r = 0; r < rows; ++r) {
        hyqo_decode(dtype, w + r * rb, rb, dec, cols);
        double acc = 0.0, m = 0.0;
        for (size_t i = 0; i < cols; ++i) {
            double t = (double)dec[i] * (double)q[i] * (double)s[i / 256];
            acc += t;
            m += fabs(t);
        }
        y[r] = acc;
        if (mag) mag[r] = m;
    }
    free(dec);
}

/* ------------------------------------------------------------------------ */
/* f32 dot (src/quant.rs:2500-2596).                                        */
/* ------------------------------------------------------------------------ */
float hyqo_dot_scalar(const float *a, const float *b, size_t n)
{
    /* a.iter().zip(b).map(|(x, y)| x * y).sum(): a sequential fold from -0.0 */
    float s = -0.0f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static float dot_avx2(const float *a, const float *b, size_t n)
{
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    size_t chunks = n / 16;
    for (size_t c = 0; c < chunks; ++c) {
        size_t i = c * 16;
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), s1);
    }
    __m256 sum = _mm256_add_ps(s0, s1);
    size_t simd_end = chunks * 16, vec_end = n / 8 * 8;
    for (size_t i = simd_end; i < vec_end; i += 8)
        sum = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), sum);
    float lanes[8];
    _mm256_storeu_ps(lanes, sum);
    float t = -0.0f;
    for (int i = 0; i < 8; ++i) t += lanes[i];
    return t + hyqo_dot_scalar(a + vec_end, b + vec_end, n - vec_end);
}

static int have_avx2_fma(void)
{
    static int state = -1;
    if (state < 0) {
        __builtin_cpu_init();
        state = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return state;
}
#endif

float hyqo_dot(const float *a, const float *b, size_t n)
{
#if defined(__x86_64__)
    if (have_avx2_fma()) return dot_avx2(a, b, n);
#endif
    return hyqo_dot_scalar(a, b, n);
}

/* ------------------------------------------------------------------------ */
/* x86 batch-1 row dots (src/quant.rs:179-268).                             */
/* ------------------------------------------------------------------------ */
float hyqo_row_dot_f32(int dtype, const uint8_t *row, size_t cols, const float *x)
{
    switch (dtype) {
    case HYQO_STQ1_0: {
        /* stq_row_dot x86 arm (:1270-1279) over stq_dot (:1256-1261) */
        float sum = 0.f;
        for (size_t b = 0; b < cols / 256; ++b) {
            const uint8_t *bytes = row + b * 42;
            float d = half_at(bytes + 40);
            int8_t dg[256];
            float digits[256];
            stq_int_digits(bytes, dg);
            for (int i = 0; i < 256; ++i) digits[i] = (float)dg[i] * 1.f;
            sum += d * hyqo_dot(digits, x + b * 256, 256);
        }
        return sum;
    }
    case HYQO_Q6_K: {
        /* q6_row_dot x86 arm (:1734-1742) over q6_dot (:1720-1725) */
        float sum = 0.f;
        float dec[256];
        for (size_t b = 0; b < cols / 256; ++b) {
            decode_block(HYQO_Q6_K, row + b * 210, dec);
            sum += hyqo_dot(dec, x + b * 256, 256);
        }
        return sum;
    }
    case HYQO_Q2_0C: {
        /* q2c_row_dot x86 arm (:2175-2187): one scalar f32 chain */
        float sum = 0.f;
        for (size_t b = 0; b < cols / 512; ++b) {
            const uint8_t *bytes = row + b * 130;
            float d = half_at(bytes);
            const float *xs = x + b * 512;
            for (int i = 0; i < 512; ++i) {
                float w = (float)(2 * ((bytes[2 + i / 4] >> (2 * (i % 4))) & 3) - 3);
                sum += d * w * xs[i];
            }
        }
        return sum;
    }
    case HYQO_F32:
    case HYQO_F16: {
        float *values = (float *)malloc(sizeof(float) * (cols ? cols : 1));
        for (size_t i = 0; i < cols; ++i) {
            if (dtype == HYQO_F32)
                memcpy(&values[i], row + 4 * i, 4);
            else
                values[i] = half_at(row + 2 * i);
        }
        float r = hyqo_dot(values, x, cols);
        free(values);
        return r;
    }
    default: {
        /* Q4_K / Q8_0: decode each block into a scratch then dot (:239-267) */
        int bl = hyqo_block_len(dtype), bb = hyqo_block_bytes(dtype);
        float scratch[512];
        float sum = 0.f;
        for (size_t b = 0; b < cols / (size_t)bl; ++b) {
            decode_block(dtype, row + b * (size_t)bb, scratch);
            sum += hyqo_dot(scratch, x + b * (size_t)bl, (size_t)bl);
        }
        return sum;
    }
    }
}

/* ------------------------------------------------------------------------ */
/* Weight::matmul x86 (src/quant.rs:159-344).                               */
/* ------------------------------------------------------------------------ */
size_t hyqo_chunk_rows(size_t rows, int threads)
{
    size_t target = (size_t)(threads * 2 > 1 ? threads * 2 : 1);
    size_t chunk = rows / target;
    if (chunk < 32) chunk = 32;
    if (chunk > 2048) chunk = 2048;
    if (chunk % 2 && chunk < 2048) chunk += 1;
    return chunk;
}

static int resolve_threads(int threads)
{
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

/* w_tile [nrows x cols] times xs [cols x batch] -> out [nrows x batch].
 * Stand-in for candle's Tensor::matmul (gemm 0.19): its blocking and
 * summation order are not restated (parity unpinned at this boundary). */
#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static void tile_gemm_avx2(const float *w, size_t nrows,
                                                               size_t cols, const float *xs,
                                                               size_t batch, float *out)
{
    size_t b0 = 0;
    for (; b0 + 16 <= batch; b0 += 16) {
        size_t r0 = 0;
        for (; r0 + 4 <= nrows; r0 += 4) {
            __m256 acc[4][2];
            for (int i = 0; i < 4; ++i) acc[i][0] = acc[i][1] = _mm256_setzero_ps();
            for (size_t k = 0; k < cols; ++k) {
                __m256 x0 = _mm256_loadu_ps(xs + k * batch + b0);
                __m256 x1 = _mm256_loadu_ps(xs + k * batch + b0 + 8);
                for (int i = 0; i < 4; ++i) {
                    __m256 wv = _mm256_broadcast_ss(w + (r0 + i) * cols + k);
                    acc[i][0] = _mm256_fmadd_ps(wv, x0, acc[i][0]);
                    acc[i][1] = _mm256_fmadd_ps(wv, x1, acc[i][1]);
                }
            }
            for (int i = 0; i < 4; ++i) {
                _mm256_storeu_ps(out + (r0 + i) * batch + b0, acc[i][0]);
                _mm256_storeu_ps(out + (r0 + i) * batch + b0 + 8, acc[i][1]);
            }
        }
        for (; r0 < nrows; ++r0)
            for (size_t b = b0; b < b0 + 16; ++b) {
                float s = 0.f;
                for (size_t k = 0; k < cols; ++k) s += w[r0 * cols + k] * xs[k * batch + b];
                out[r0 * batch + b] = s;
            }
    }
    for (size_t r = 0; r < nrows; ++r)
        for (size_t b = b0; b < batch; ++b) {
            float s = 0.f;
            for (size_t k = 0; k < cols; ++k) s += w[r * cols + k] * xs[k * batch + b];
            out[r * batch + b] = s;
        }
}
#endif

static void tile_gemm(const float *w, size_t nrows, size_t cols, const float *xs, size_t batch,
                      float *out)
{
#if defined(__x86_64__)
    if (have_avx2_fma()) {
        tile_gemm_avx2(w, nrows, cols, xs, batch, out);
        return;
    }
#endif
    for (size_t r = 0; r < nrows; ++r)
        for (size_t b = 0; b < batch; ++b) {
            float s = 0.f;
            for (size_t k = 0; k < cols; ++k) s += w[r * cols + k] * xs[k * batch + b];
            out[r * batch + b] = s;
        }
}

int hyqo_matmul(int dtype, const uint8_t *w, size_t rows, size_t cols, const float *x,
                size_t batch, float *y, int threads)
{
    int bl = hyqo_block_len(dtype);
    if (bl <= 0 || batch == 0 || cols % (size_t)bl) return -1;
    size_t rb = row_bytes_of(dtype, cols);
    int T = resolve_threads(threads);
    if (batch == 1) {
        size_t chunk = hyqo_chunk_rows(rows, T);
        long nchunks = (long)((rows + chunk - 1) / chunk);
#pragma omp parallel for num_threads(T) schedule(dynamic, 1)
        for (long c = 0; c < nchunks; ++c) {
            size_t r0 = (size_t)c * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
            for (size_t r = r0; r < r1; ++r) y[r] = hyqo_row_dot_f32(dtype, w + r * rb, cols, x);
        }
        return 0;
    }
    float *transposed = (float *)malloc(sizeof(float) * rows * batch);
    if (batch >= 8) {
        float *xs = (float *)malloc(sizeof(float) * cols * batch);
        for (size_t b = 0; b < batch; ++b)
            for (size_t k = 0; k < cols; ++k) xs[k * batch + b] = x[b * cols + k];
        const size_t tile_rows = 64;
        long ntiles = (long)((rows + tile_rows - 1) / tile_rows);
#pragma omp parallel for num_threads(T) schedule(dynamic, 1)
        for (long t = 0; t < ntiles; ++t) {
            size_t r0 = (size_t)t * tile_rows;
            size_t nrows = rows - r0 < tile_rows ? rows - r0 : tile_rows;
            float *wt = (float *)malloc(sizeof(float) * nrows * cols);
            hyqo_decode(dtype, w + r0 * rb, nrows * rb, wt, nrows * cols);
            tile_gemm(wt, nrows, cols, xs, batch, transposed + r0 * batch);
            free(wt);
        }
        free(xs);
    } else {
        long ntiles = (long)((rows + 31) / 32);
#pragma omp parallel for num_threads(T) schedule(dynamic, 1)
        for (long t = 0; t < ntiles; ++t) {
            float *scratch = (float *)malloc(sizeof(float) * cols);
            for (size_t r = (size_t)t * 32; r < rows && r < (size_t)t * 32 + 32; ++r) {
                hyqo_decode(dtype, w + r * rb, rb, scratch, cols);
                for (size_t b = 0; b < batch; ++b)
                    transposed[r * batch + b] = hyqo_dot(scratch, x + b * cols, cols);
            }
            free(scratch);
        }
    }
    for (size_t b = 0; b < batch; ++b)
        for (size_t r = 0; r < rows; ++r) y[b * rows + r] = transposed[r * batch + b];
    free(transposed);
    return 0;
}

static float silu_mul(float g, float u)
{
    float silu = g / (1.0f + expf(-g));
    return silu * u;
}

int hyqo_gate_up_silu(int dtype, const uint8_t *gate, const uint8_t *up, size_t rows, size_t cols,
                      const float *x, float *y, int threads)
{
    int bl = hyqo_block_len(dtype);
    if (bl <= 0 || cols % (size_t)bl) return -1;
    size_t rb = row_bytes_of(dtype, cols);
    int T = resolve_threads(threads);
    if (dtype == HYQO_STQ1_0 || dtype == HYQO_Q6_K || dtype == HYQO_Q2_0C) {
        /* paired f32 row dots (src/quant.rs:768-830) */
        size_t chunk = hyqo_chunk_rows(rows, T);
        long nchunks = (long)((rows + chunk - 1) / chunk);
#pragma omp parallel for num_threads(T) schedule(dynamic, 1)
        for (long c = 0; c < nchunks; ++c) {
            size_t r0 = (size_t)c * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
            for (size_t r = r0; r < r1; ++r) {
                float g = hyqo_row_dot_f32(dtype, gate + r * rb, cols, x);
                float u = hyqo_row_dot_f32(dtype, up + r * rb, cols, x);
                y[r] = silu_mul(g, u);
            }
        }
        return 0;
    }
    /* separate matmuls then SiLU (src/quant.rs:831-838) */
    float *u = (float *)malloc(sizeof(float) * rows);
    hyqo_matmul(dtype, gate, rows, cols, x, 1, y, T);
    hyqo_matmul(dtype, up, rows, cols, x, 1, u, T);
    for (size_t r = 0; r < rows; ++r) y[r] = (y[r] / (1.f + expf(-y[r]))) * u[r];
    free(u);
    return 0;
}

void hyqo_matmul_f64(int dtype, const uint8_t *w, size_t rows, size_t cols, const float *x,
                     size_t batch, double *y, double *mag)
{
    size_t rb = row_bytes_of(dtype, cols);
    long R = (long)rows;
#pragma omp parallel for schedule(dynamic, 16)
    for (long r = 0; r < R; ++r) {
        float *dec = (float *)malloc(sizeof(float) * cols);
        hyqo_decode(dtype, w + (size_t)r * rb, rb, dec, cols);
        for (size_t b = 0; b < batch; ++b) {
            double acc = 0.0, m = 0.0;
            const float *xb = x + b * cols;
            for (size_t k = 0; k < cols; ++k) {
                double t = (double)dec[k] * (double)xb[k];
                acc += t;
                m += fabs(t);
            }
            y[b * rows + (size_t)r] = acc;
            if (mag) mag[b * rows + (size_t)r] = m;
        }
        free(dec);
    }
}

/* ------------------------------------------------------------------------ */
/* MoE (src/model.rs:687-767).                                              */
/* ------------------------------------------------------------------------ */
static float stable_sigmoid(float x)
{
    if (x >= 0.f) return 1.f / (1.f + expf(-x));
    float e = expf(x);
    return e / (1.f + e);
}

void hyqo_route(const float *logits, const float *bias, size_t experts, size_t used,
                int normalize, float scale, int32_t *idx, float *weight)
{
    float *sig = (float *)malloc(sizeof(float) * experts);
    size_t *order = (size_t *)malloc(sizeof(size_t) * experts);
    for (size_t i = 0; i < experts; ++i) {
        sig[i] = stable_sigmoid(logits[i]);
        order[i] = i;
    }
    /* sort descending by sigmoid+bias (total_cmp), ties by ascending index;
     * insertion sort keeps it simple and the order total. */
    for (size_t i = 1; i < experts; ++i) {
        size_t v = order[i];
        size_t j = i;
        while (j > 0) {
            size_t u = order[j - 1];
            float ku = sig[u] + bias[u], kv = sig[v] + bias[v];
            int before = (kv > ku) || (kv == ku && v < u);
            if (!before) break;
            order[j] = u;
            --j;
        }
        order[j] = v;
    }
    float sum = 1.f;
    if (normalize) {
        sum = -0.0f;
        for (size_t k = 0; k < used; ++k) sum += sig[order[k]];
        if (sum < 6.103515625e-05f) sum = 6.103515625e-05f; /* f16::MIN_POSITIVE */
    }
    for (size_t k = 0; k < used; ++k) {
        idx[k] = (int32_t)order[k];
        weight[k] = sig[order[k]] / sum * scale;
    }
    free(sig);
    free(order);
}

int hyqo_moe_experts(int dtype_gate, int dtype_down, const uint8_t *gate, const uint8_t *up,
                     const uint8_t *down, size_t experts, size_t hidden, size_t mid,
                     const float *x, size_t tokens, const int32_t *pair_token,
                     const int32_t *pair_expert, const float *pair_weight, size_t npairs,
                     float *out, int threads)
{
    (void)tokens;
    size_t gate_bytes = mid * row_bytes_of(dtype_gate, hidden);
    size_t down_bytes = hidden * row_bytes_of(dtype_down, mid);
    int32_t *tok = (int32_t *)malloc(sizeof(int32_t) * (npairs ? npairs : 1));
    float *wt = (float *)malloc(sizeof(float) * (npairs ? npairs : 1));
    for (size_t e = 0; e < experts; ++e) {
        size_t n = 0;
        for (size_t p = 0; p < npairs; ++p)
            if ((size_t)pair_expert[p] == e) {
                tok[n] = pair_token[p];
                wt[n] = pair_weight[p];
                ++n;
            }
        if (n == 0) continue;
        float *sel = (float *)malloc(sizeof(float) * n * hidden);
        for (size_t i = 0; i < n; ++i)
            memcpy(sel + i * hidden, x + (size_t)tok[i] * hidden, sizeof(float) * hidden);
        const uint8_t *g = gate + e * gate_bytes, *u = up + e * gate_bytes;
        const uint8_t *d = down + e * down_bytes;
        float *h = (float *)malloc(sizeof(float) * n * mid);
        float *res = (float *)malloc(sizeof(float) * n * hidden);
        /* DenseFfn::forward (src/model.rs:672-685) */
        if (n == 1) {
            hyqo_gate_up_silu(dtype_gate, g, u, mid, hidden, sel, h, threads);
            hyqo_matmul(dtype_down, d, hidden, mid, h, 1, res, threads);
        } else {
            float *uo = (float *)malloc(sizeof(float) * n * mid);
            hyqo_matmul(dtype_gate, g, mid, hidden, sel, n, h, threads);
            hyqo_matmul(dtype_gate, u, mid, hidden, sel, n, uo, threads);
            for (size_t i = 0; i < n * mid; ++i) h[i] = (h[i] / (1.f + expf(-h[i]))) * uo[i];
            free(uo);
            hyqo_matmul(dtype_down, d, hidden, mid, h, n, res, threads);
        }
        for (size_t i = 0; i < n; ++i)
            for (size_t k = 0; k < hidden; ++k)
                out[(size_t)tok[i] * hidden + k] += wt[i] * res[i * hidden + k];
        free(sel);
        free(h);
        free(res);
    }
    free(tok);
    free(wt);
    return 0;
}
