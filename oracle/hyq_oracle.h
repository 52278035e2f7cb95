/*
 * CPU oracle for the quantized matrix-product path of hy-mt-rs.
 *
 * TEST INFRASTRUCTURE ONLY. This library gives the reference results: it is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, never by the product library (hy-mt-rs_amd/libhyq.so), which has no
 * CPU fallback.
 *
 * Every function restates an algorithm of the reference (Rust, not buildable
 * here: no cargo/rustc, git dependency on candle-core, and src/quant.rs:1460
 * breaks the x86_64 build). Citations are path:line in the reference tree.
 *
 * Pinning (what fixes each function independently of this restatement):
 *   hyqo_decode            tests/fixtures/quant.json golden bit patterns (all
 *                          5 formats x 3 blocks, incl. negative and zero
 *                          scales) + closed forms src/quant.rs:2602-2644.
 *   hyqo_q8_quantize       hand-built vectors whose answer is fixed by
 *                          construction (max=127 => q=rint(x); ties to even;
 *                          all-zero group; +-max => +-127) and the invariant
 *                          |q*s - x| <= s/2 (src/quant.rs:2955-2978).
 *   hyqo_row_isums         must equal integer sums over the golden-pinned
 *                          decoder's output with unit block scales (exact).
 *   hyqo_gemv_q8_f64       must equal the f64 brute force over decoded
 *                          weights x dequantized activations
 *                          (src/quant.rs:2980-3079 recipe).
 *   hyqo_dot / row dots    src/quant.rs:2646-2711 (vs scalar / decode+dot).
 *   hyqo_route             src/model.rs:1088-1094 closed form.
 *   hyqo_matmul batch>=8   parity unpinned at the candle/gemm boundary: the
 *                          f64 brute force (hyqo_matmul_f64) is the oracle.
 */
#ifndef HYQ_ORACLE_H
#define HYQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType ids as GGUF stores them after profile resolution (src/quant.rs:30-41). */
enum {
    HYQO_F32 = 0,
    HYQO_F16 = 1,
    HYQO_Q8_0 = 8,
    HYQO_Q4_K = 12,
    HYQO_Q6_K = 14,
    HYQO_Q2_0C = 40,
    HYQO_STQ1_0 = 42
};

int hyqo_block_len(int dtype);
int hyqo_block_bytes(int dtype);
float hyqo_f16_to_f32(uint16_t bits);

/* decode (src/quant.rs:1066-1079) -> decode_unchecked (:2405-2486).
 * Returns 0, or -1 on a partial block / wrong byte count (the ensure! arms). */
int hyqo_decode(int dtype, const uint8_t *bytes, size_t nbytes, float *out, size_t n);

/* Q8::quantize_into (src/quant.rs:904-922, :965-991): one f32 scale per
 * 256-group; q = sat_i8(RNE(x * (127/max))); a group with max 0 gives 0/0. */
void hyqo_q8_quantize(const float *x, size_t n, int8_t *q, float *scales);
/* deinterleave_q2c (src/quant.rs:943-963): out[64c+16k+j] = q[64c+4j+k]. */
void hyqo_q8_deinterleave_q2c(const int8_t *q, size_t n, int8_t *out);

/* Integer partial sums of one row against Q8 values, in the granularity the
 * reference's int8 kernels accumulate them:
 *   STQ1_0  one isum per 256-weight block      (src/quant.rs:1511-1556)
 *   Q2_0C   two isums per 512-weight block      (src/quant.rs:1891-1951)
 *   Q6_K    sixteen isums per block (16-weight planes, q6-32) (:2257-2330)
 *   Q4_K    two per block: A = sum_j s_j*qx_j, B = sum_j m_j*xs_j (build-defined)
 *   Q8_0    one isum per 32-weight block (build-defined)
 * Returns the number written, or -1. */
int hyqo_row_isums(int dtype, const uint8_t *row, size_t cols, const int8_t *q, int32_t *out);
int hyqo_isums_per_row(int dtype, size_t cols);

/* int8 GEMV oracle in f64 from the isums and the f32 scale products the
 * reference forms (d*s per block/group, src/quant.rs:1512,1896,2258).
 * mag[r] = sum of |term| (the reference's tolerance magnitude). */
void hyqo_gemv_q8_f64(int dtype, const uint8_t *w, size_t rows, size_t cols,
                      const int8_t *q, const float *s, double *y, double *mag);
/* Brute force: sum_i decoded_w[i] * q[i] * s[i/256] in f64
 * (the recipe of src/quant.rs:3007-3024). */
void hyqo_gemv_q8_bruteforce(int dtype, const uint8_t *w, size_t rows, size_t cols,
                             const int8_t *q, const float *s, double *y, double *mag);

/* f32 dot product: dot_avx2 when the CPU has AVX2+FMA, else dot_scalar
 * (src/quant.rs:2500-2596). */
float hyqo_dot(const float *a, const float *b, size_t n);
float hyqo_dot_scalar(const float *a, const float *b, size_t n);

/* Batch-1 f32 row dot of the x86 path of Weight::matmul (src/quant.rs:179-268):
 * STQ stq_row_dot, Q6_K q6_row_dot, Q2_0C q2c_row_dot (scalar), F32/F16 decode
 * row + dot, Q4_K/Q8_0 decode-block + dot per block. */
float hyqo_row_dot_f32(int dtype, const uint8_t *row, size_t cols, const float *x);

/* Weight::matmul, x86 path (src/quant.rs:159-344). x is [batch, cols],
 * y is [batch, rows]. threads <= 0 uses all OpenMP threads. The batch >= 8
 * arm replaces candle's GEMM with an own AVX2 outer-product kernel. */
int hyqo_matmul(int dtype, const uint8_t *w, size_t rows, size_t cols,
                const float *x, size_t batch, float *y, int threads);
/* Weight::matmul_gate_up_silu, x86 path (src/quant.rs:724-841). */
int hyqo_gate_up_silu(int dtype, const uint8_t *gate, const uint8_t *up, size_t rows,
                      size_t cols, const float *x, float *y, int threads);
/* f64 brute force of decoded weights x f32 activations: y[b*rows + r]. */
void hyqo_matmul_f64(int dtype, const uint8_t *w, size_t rows, size_t cols,
                     const float *x, size_t batch, double *y, double *mag);

/* chunk_rows (src/quant.rs:1037-1045). */
size_t hyqo_chunk_rows(size_t rows, int threads);

/* route (src/model.rs:728-767). Writes `used` (expert, weight) pairs. */
void hyqo_route(const float *logits, const float *bias, size_t experts, size_t used,
                int normalize, float scale, int32_t *idx, float *weight);

/* Moe::forward minus the router and the shared expert (src/model.rs:699-725):
 * out[t] += w * DenseFfn(expert e)(x[t]) for experts in ascending order, with
 * each expert's token batch sent through the x86 matmul paths. gate/up are
 * [E][mid x hidden], down is [E][hidden x mid]; pairs are (token, expert, w). */
int hyqo_moe_experts(int dtype_gate, int dtype_down, const uint8_t *gate, const uint8_t *up,
                     const uint8_t *down, size_t experts, size_t hidden, size_t mid,
                     const float *x, size_t tokens, const int32_t *pair_token,
                     const int32_t *pair_expert, const float *pair_weight, size_t npairs,
                     float *out, int threads);

#ifdef __cplusplus
}
#endif
#endif
