// Decode-step glue launchers (kernels in hyq_step.hip).
#pragma once

#include <stdint.h>

#include "hyq_internal.hpp"

namespace hyq {

// Device-resident step state: the position of the token being decoded, the
// number of tokens generated so far (index into the history buffer), and a
// flag the argmax sets when a step's logits held a non-finite value.
struct StepState {
    int pos;
    int step;
    int history_cap;
    int nonfinite;
};

int launch_embed_row(int fmt, WView w, int cols, const int *token, float *out, void *stream);
// Rows out[i] = embedding row tokens[i] for i < n (tokens in device memory).
int launch_embed_rows(int fmt, WView w, int cols, const int *tokens, int n, float *out,
                      void *stream);
// x may carry nparts partial rows at parts + k * pstride, added to it first
int launch_rms_norm_q8(const float *x, const float *w, int n, float eps, float *y, int8_t *q,
                       float *s, int32_t *s16, int32_t *s32, int32_t *s256, void *stream,
                       const float *parts = nullptr, int nparts = 0, int pstride = 0);
// norm_first: the hy_v3 order (per-head rms_norm, then RoPE); otherwise the
// dense one (src/model.rs:425-446).
int launch_rope_norm_kv(float *q, const float *k, const float *v, const float *qn,
                        const float *kn, const float *freq, const int *pos, int heads, int kvh,
                        int dim, float eps, float *kcache, float *vcache, void *stream,
                        bool norm_first = false);
// The same for n tokens of a chunk: rows q[i], k[i], v[i] at position *pos + i.
int launch_rope_norm_kv_rows(float *q, const float *k, const float *v, const float *qn,
                             const float *kn, const float *freq, const int *pos, int n,
                             int heads, int kvh, int dim, float eps, float *kcache,
                             float *vcache, void *stream, bool norm_first = false);
// Attention splits: `chunk` positions each (a multiple of ATT_SUB), at most
// ATT_MAX_SPLITS; partials are [heads][splits][PART_STRIDE] floats holding
// (max, exp-sum, -, -, exp-weighted V sum[128]).
constexpr int ATT_SUB = 32;
constexpr int ATT_D = 128;
constexpr int ATT_MAX_SPLITS = 64;
static_assert(ATT_MAX_SPLITS <= 64, "the merge holds one split per lane of a wave");
constexpr int ATT_MAX_REP = 4; // query heads per KV head (one per wave)
constexpr int PART_STRIDE = 132;
int attention_chunk(int context);
int attention_splits(int context);
// Splits of the chunked-prefill attention (each of prefill_attention_chunk
// positions); its partials are [n][heads][splits][PART_STRIDE].
int prefill_attention_chunk(int context);
int prefill_attention_splits(int context);
int launch_zero_u32(unsigned *p, int n, void *stream);
// out[i] = ((x[i] + parts[i]) + parts[stride + i]) + ... over np partial rows.
int launch_sum_parts(const float *x, const float *parts, int np, int stride, int n, float *out,
                     void *stream);
// Attention of one query token over cache rows 0..=*pos (q already rotated
// and normalized), merged into out [heads*128].
int launch_attention(const float *q, const float *kcache, const float *vcache, const int *pos,
                     int context, int heads, int kvh, float *part, float *out, void *stream);
// Causal attention of the n query rows q [n][heads*128] of a chunk whose
// keys and values are in the cache: row i at position *pos + i sees cache
// rows 0..=*pos + i; merged into out [n][heads*128] (hyq_attn_rows.hip: f16
// matrix-core products of split f16 operand pairs).
int launch_attention_rows(const float *q, const float *kcache, const float *vcache,
                          const int *pos, int n, int context, int heads, int kvh, float *part,
                          float *out, void *stream);
// The same with the rows merged one workgroup per token, written as f32
// (out, if given) and/or as the attention-output GEMM's f16 operand rows
// with their power-of-two scales (xh, rscale, if given); hipErrorInvalidValue
// when a row's merge needs more than 64 KiB of LDS (merge_rows_lds).
int launch_attention_rows_f16(const float *q, const float *kcache, const float *vcache,
                              const int *pos, int n, int context, int heads, int kvh,
                              float *part, float *out, _Float16 *xh, float *rscale,
                              void *stream);
size_t merge_rows_lds(int heads, int splits);
// Merge of n query rows' split partials ([n][heads][splits][PART_STRIDE],
// `chunk` positions per split) into out [n][heads*128].
int launch_attention_merge_rows(const float *part, int splits, int chunk, int heads,
                                const int *pos, int n, float *out, void *stream);
// Merge of the split partials into out [heads*128].
int launch_attention_merge(const float *part, int context, int heads, const int *pos,
                           float *out, void *stream);
// The decode step's attention: RoPE + Q/K norm of the raw projections, KV
// append at *pos, split partials (merged by launch_attention_merge).
int launch_attention_rope(const float *q, const float *k, const float *v, const float *qn,
                          const float *kn, const float *freq, float eps, float *kcache,
                          float *vcache, const int *pos, int context, int heads, int kvh,
                          float *part, void *stream, bool norm_first = false);
int argmax_partials(int n);
int launch_argmax(const float *x, int n, float *pv, int *pi, int *token, StepState *st,
                  int *history, void *stream);
// The same argmax, whose final pass also writes the chosen token's row of
// the embedding w (format fmt, cols values) to out: the next decode step's
// input.
int launch_argmax_embed(const float *x, int n, float *pv, int *pi, int *token, StepState *st,
                        int *history, int fmt, WView w, int cols, float *out, void *stream);

} // namespace hyq
