/* CPU oracle, part 2: decode-step glue (test infrastructure only). */
#ifndef HYQ_ORACLE_STEP_H
#define HYQ_ORACLE_STEP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The MoE FFN of a HyV3 layer (src/model.rs:82-92, :206-235): an F32 router
 * [experts][hidden] with its selection bias, expert stacks gate/up
 * [experts][mid][hidden] and down [experts][hidden][mid] (GGUF bytes, expert
 * after expert) and the shared expert's gate/up [shared_mid][hidden] and
 * down [hidden][shared_mid]. */
typedef struct {
    int experts, used, mid, shared_mid, normalize;
    float scale;
    int dtype_gate, dtype_down, dtype_shared, dtype_shared_down;
    const float *router;
    const float *bias;
    const uint8_t *gate, *up, *down;
    const uint8_t *sgate, *sup, *sdown;
} hyqo_moe;

/* Weights of a Hunyuan model (src/model.rs:49-76), packed GGUF bytes. The
 * embedding doubles as the output matrix when output is NULL (tied, dense
 * only, src/model.rs:194-202). arch 0 is hunyuan-dense, 1 is hy_v3 (Q/K
 * norms before RoPE, src/model.rs:425-446); moe[l] is layer l's MoE FFN or
 * NULL for a dense FFN (moe itself may be NULL). */
typedef struct {
    int layers, hidden, heads, kv_heads, head_dim, ffn, vocab;
    float rope_base, eps;
    int dtype_linear, dtype_embed;
    int dtype_down; /* ffn_down's format (Q6_K in the Q4_K_M mix) */
    const uint8_t *embed;
    const uint8_t *output; /* NULL: tied to embed */
    const float *output_norm;
    const uint8_t *const *wq, *const *wk, *const *wv, *const *wo;
    const uint8_t *const *wgate, *const *wup, *const *wdown;
    const float *const *attn_norm, *const *ffn_norm, *const *q_norm, *const *k_norm;
    int arch;
    const hyqo_moe *const *moe;
} hyqo_model;

/* Moe::forward (src/model.rs:687-726) for n rows x [n][hidden]: router
 * matmul, route, shared expert, then the experts in ascending order,
 * out[t] += w * ffn_e(x_t); out [n][hidden] is written. With int8_path and
 * n == 1 every quantized product takes the int8 path; otherwise the f32
 * products of the reference's x86 arm. */
void hyqo_moe_forward(const hyqo_moe *e, size_t hidden, const float *x, size_t n, float *out,
                      int int8_path, int threads);

/* The int8 path's quantized inputs, stage by stage, for the parity tests of
 * the device's decode step. The stages of one layer (values per stage):
 *   HYQO_STAGE_ATTN_IN        the normalized hidden row (Q/K/V input)    hidden
 *   HYQO_STAGE_OUT_IN         the attention row (attention-output input) heads*head_dim
 *   HYQO_STAGE_FFN_IN         the normalized row (FFN input)             hidden
 *   HYQO_STAGE_DOWN_IN        silu(g) * u of the dense FFN, or of the MoE's
 *                             shared expert (down input)                 ffn / shared_mid
 *   HYQO_STAGE_EXPERT_DOWN_IN + j  the j-th routed expert's silu(g) * u,
 *                             experts in ascending order                 mid
 * and the output's one: HYQO_STAGE_ATTN_IN, the output-normalized row.
 * Stage i's values sit at own_x / own_q / use_q + i * stride and its scales
 * at own_s / use_s + i * stride / 256 (stride a multiple of 256). own_* (each
 * when set) receive the oracle's own f32 input, codes and scales; use_q and
 * use_s (each when set) replace the codes and scales that enter the
 * product. */
enum {
    HYQO_STAGE_ATTN_IN = 0,
    HYQO_STAGE_OUT_IN = 1,
    HYQO_STAGE_FFN_IN = 2,
    HYQO_STAGE_DOWN_IN = 3,
    HYQO_STAGE_EXPERT_DOWN_IN = 4
};
typedef struct {
    size_t stride;
    float *own_x;
    int8_t *own_q;
    float *own_s;
    const int8_t *use_q;
    const float *use_s;
} hyqo_q8_tap;

/* Moe::forward of one row on the int8 path with a tap (its stages FFN_IN,
 * DOWN_IN and EXPERT_DOWN_IN + j). */
void hyqo_moe_forward_tap(const hyqo_moe *e, size_t hidden, const float *x, float *out,
                          int threads, const hyqo_q8_tap *tap);

/* rms_norm_into / rms_norm (src/model.rs:785-870) in the operation order of
 * the aarch64 arm (aarch64 = 1: x * (w * scale) over whole 16-value steps) or
 * the x86 arm (0: x * scale * w). */
void hyqo_rms_norm_into(const float *x, const float *w, size_t n, float eps, float *out,
                        int aarch64);
void hyqo_rms_norm_rows(float *x, const float *w, size_t total, size_t wlen, float eps,
                        int aarch64);
void hyqo_rope_tables(size_t head_dim, float base, size_t pos, float *cos_s, float *sin_s);
void hyqo_rope(float *values, size_t heads, size_t dim, const float *cos_s, const float *sin_s);
void hyqo_attention(const float *q, const float *keys, const float *values, size_t heads,
                    size_t kv_heads, size_t dim, size_t visible, float *out);
/* One token through Model::forward_into batch 1 (src/model.rs:374-546).
 * kcache/vcache are [layers][ctx][kv_heads*head_dim]; the step writes
 * position `pos` and attends over 0..=pos. */
int hyqo_decode_step(const hyqo_model *m, float *kcache, float *vcache, size_t ctx, size_t pos,
                     int token, int int8_path, float *logits, int threads);
/* One chunk of Model::forward_into at batch n (src/model.rs:549-616): the
 * tokens take positions pos..pos+n-1 (written to the caches); logits are the
 * last row's, through the batch-1 matmul of the int8 or f32 arm. n == 1 is
 * hyqo_decode_step. Returns -1 on an empty chunk, the context limit or a
 * token outside the vocabulary. */
int hyqo_prefill_chunk(const hyqo_model *m, float *kcache, float *vcache, size_t ctx, size_t pos,
                       const int *tokens, size_t n, int int8_path, float *logits, int threads);
/* The pieces of those two: one layer of the batch-1 step on `hidden` [H]
 * (in place) with that layer's caches kc/vc [ctx][kv_heads*head_dim]; one
 * layer of the batch-n arm on hidden [n][H]; the output norm (in place) and
 * the output matmul of one row. */
int hyqo_layer_step(const hyqo_model *m, int l, float *hidden, float *kc, float *vc, size_t ctx,
                    size_t pos, int int8_path, int threads);
int hyqo_prefill_layer(const hyqo_model *m, int l, float *hidden, float *kc, float *vc,
                       size_t ctx, size_t pos, size_t n, int threads);
void hyqo_output_logits(const hyqo_model *m, float *hidden, int int8_path, float *logits,
                        int threads);
/* hyqo_layer_step and hyqo_output_logits on the int8 path with a tap. */
int hyqo_layer_step_tap(const hyqo_model *m, int l, float *hidden, float *kc, float *vc,
                        size_t ctx, size_t pos, int threads, const hyqo_q8_tap *tap);
void hyqo_output_logits_tap(const hyqo_model *m, float *hidden, float *logits, int threads,
                            const hyqo_q8_tap *tap);
int hyqo_argmax(const float *x, size_t n);
/* OpenMP threads the matmul/attention loops use when threads <= 0. */
int hyqo_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
