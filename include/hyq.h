/*
 * hyq: MI355X (gfx950) quantized matrix products for hy-mt-rs.
 *
 * A C ABI over hand-written HIP kernels. It replaces the bodies of the
 * reference's quantized-tensor interface (Rust, src/quant.rs) so that the
 * GGUF reader, tokenizer, KV cache, sampler and server stay unchanged. Each
 * declaration names the reference item it stands in for.
 *
 * Conventions
 *   - Return value: HYQ_OK (0) or a negative HYQ_E* code; hyq_last_error()
 *     gives a thread-local message. Shape/length violations return
 *     HYQ_EINVAL, the reference's `ensure!` arms (src/quant.rs:160-166,
 *     :665-671, :726-730, :1067-1076); an unsupported format/op pair returns
 *     HYQ_EDTYPE. No call has undefined behaviour on bad sizes.
 *   - Host-pointer calls (x, y, bytes in host memory) are synchronous, as the
 *     reference returns owned Vecs. Calls ending in _d take device pointers
 *     and are asynchronous on the context's stream (hyq_sync waits).
 *   - Shapes follow GGUF: dims[0] is the input width (cols), dims[1] the
 *     output rows, dims[2] the expert count (src/gguf.rs:32, quant.rs:161).
 *   - Activations are row-major [batch, cols]; outputs are [batch, rows].
 *   - A hyq_ctx is one device plus one HIP stream; use one per host thread.
 *     A hyq_weight is immutable after upload and may be shared by contexts
 *     of the same device.
 */
#ifndef HYQ_H
#define HYQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType ids after GGUF profile resolution (src/quant.rs:17-63). 40/42 are the
 * Tencent legacy ids, valid only under their profiles (src/quant.rs:37-38). */
typedef enum {
    HYQ_F32 = 0,
    HYQ_F16 = 1,
    HYQ_Q8_0 = 8,
    HYQ_Q4_K = 12,
    HYQ_Q6_K = 14,
    HYQ_Q2_0C = 40,
    HYQ_STQ1_0 = 42
} hyq_dtype;

enum {
    HYQ_OK = 0,
    HYQ_EINVAL = -1,  /* bad shape, length, index or null pointer */
    HYQ_EDTYPE = -2,  /* format not supported by this operation */
    HYQ_EDEVICE = -3, /* HIP runtime error */
    HYQ_ENOMEM = -4   /* device allocation failed */
};

typedef struct hyq_ctx hyq_ctx;
typedef struct hyq_weight hyq_weight;
typedef struct hyq_q8 hyq_q8;

/* Thread-local description of the last failure on this thread. */
const char *hyq_last_error(void);
/* DType::block_len / block_bytes (src/quant.rs:43-62); -1 if unknown. */
int hyq_block_len(int dtype);
int hyq_block_bytes(int dtype);

/* ---- context: the device and stream a rayon pool stood for ---- */
int hyq_ctx_create(int device, hyq_ctx **out);
/* Decoders created on a context (hyq_dense_*) use its stream: destroy them
 * first. Weights and Q8 buffers may outlive it. */
void hyq_ctx_destroy(hyq_ctx *ctx);
/* The context's hipStream_t, for callers that enqueue their own work. */
void *hyq_ctx_stream(hyq_ctx *ctx);
int hyq_sync(hyq_ctx *ctx);
/* Q8 tracing (no counterpart in the reference: it exposes the int8 codes
 * that Q8::quantize_into, src/quant.rs:904-922, forms inside the products).
 * While trace_d (256-byte aligned device memory of `bytes` bytes) is set,
 * every launch of the dense decoder's eager step (hyq_dense_forward) and of
 * hyq_moe_forward_d at one token that quantizes an f32 row to Q8 - a GEMV
 * input stage, the RMSNorm+Q8 and quantize kernels - also writes what it
 * quantized and formed to trace_d, one record of n values after another:
 * n int8 codes, n / 256 f32 scales and, from the next 256-byte boundary, the
 * n f32 values quantized (after any RMSNorm); each record starts on a
 * 256-byte boundary.
 * Setting a buffer (or NULL, which switches tracing off) clears the list.
 * hyq_ctx_q8_trace_records returns the number of records written since
 * (*count), the number dropped for want of space (*dropped, may be NULL)
 * and, for the first max_records of them, (byte offset, n) pairs. */
int hyq_ctx_set_q8_trace(hyq_ctx *ctx, void *trace_d, size_t bytes);
int hyq_ctx_q8_trace_records(hyq_ctx *ctx, size_t *pairs, size_t max_records, size_t *count,
                             size_t *dropped);

/* ---- device buffers for the _d entry points (no reference counterpart: the
 * reference is host-only; a host that drives the device-pointer calls needs
 * them). Copies are ordered on the context stream; the h2d/d2h calls return
 * after the copy completed. ---- */
int hyq_device_alloc(hyq_ctx *ctx, size_t bytes, void **ptr_d);
int hyq_device_free(hyq_ctx *ctx, void *ptr_d);
int hyq_memcpy_h2d(hyq_ctx *ctx, void *dst_d, const void *src, size_t bytes);
int hyq_memcpy_d2h(hyq_ctx *ctx, void *dst, const void *src_d, size_t bytes);
int hyq_memcpy_d2d(hyq_ctx *ctx, void *dst_d, const void *src_d, size_t bytes);

/* ---- weights: Weight::new over the mmap (src/quant.rs:65-97) ----
 * Copies gguf_bytes (byte_len == rows*row_bytes*experts) to the device and
 * re-lays it out for the kernels (same byte count); the host buffer may be
 * unmapped afterwards. rank 2: dims = {cols, rows}; rank 3: {cols, rows, E}. */
int hyq_weight_upload(hyq_ctx *ctx, int dtype, const uint8_t *gguf_bytes, size_t byte_len,
                      const uint64_t *dims, int rank, hyq_weight **out);
/* Weight::expert (src/quant.rs:144-154): a no-copy view of expert e. */
int hyq_weight_expert(const hyq_weight *w, size_t e, hyq_weight **view);
void hyq_weight_release(hyq_weight *w);
/* Weight::shape / dtype (src/quant.rs:75-80). dims must hold 3 entries. */
int hyq_weight_info(const hyq_weight *w, int *dtype, uint64_t *dims, int *rank);

/* ---- host-pointer products (synchronous) ---- */

/* Weight::matmul (src/quant.rs:159-344). batch == 1 runs the int8 GEMV
 * (x quantized to Q8 as Q8::quantize_into, src/quant.rs:904-922);
 * batch > 1 runs the f16-MFMA GEMM (weights dequantized to f16 in LDS). */
int hyq_matmul(hyq_ctx *ctx, const hyq_weight *w, const float *x, size_t batch, float *y);
/* Weight::gemv_qkv (src/quant.rs:658-721): one Q8 and one launch for all three. */
int hyq_gemv_qkv(hyq_ctx *ctx, const hyq_weight *q, const hyq_weight *k, const hyq_weight *v,
                 const float *x, float *yq, float *yk, float *yv);
/* Weight::matmul_gate_up_silu (src/quant.rs:724-841): y = silu(gate x) * (up x). */
int hyq_gate_up_silu(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                     const float *x, float *y);
/* decode (src/quant.rs:1066-1079) on the device: n values from whole blocks. */
int hyq_decode(hyq_ctx *ctx, int dtype, const uint8_t *bytes, size_t byte_len, float *out,
               size_t n);
/* Weight::row_into (src/quant.rs:123-142): decode one row (cols values). */
int hyq_weight_row(hyq_ctx *ctx, const hyq_weight *w, size_t row, float *out, size_t n);

/* ---- device-pointer products (asynchronous on the context stream) ---- */

/* Q8::new (src/quant.rs:896-902): int8 activations of length n with one f32
 * scale per 256 values, plus the per-16/32/256 integer sums the kernels use. */
int hyq_q8_create(hyq_ctx *ctx, size_t n, hyq_q8 **out);
void hyq_q8_release(hyq_q8 *q8);
/* Device addresses of the int8 values [n] and scales [ceil(n/256)]. */
int hyq_q8_buffers(const hyq_q8 *q8, int8_t **values_d, float **scales_d, size_t *n);
/* Q8::quantize_into (src/quant.rs:904-922). */
int hyq_quantize_q8_d(hyq_ctx *ctx, const float *x_d, size_t n, hyq_q8 *q8);
/* Weight::gemv_q8_fast (src/quant.rs:354-357); y = residual + W x when
 * residual_d is non-null (the `add` that follows, src/model.rs:476, :512). */
int hyq_gemv_q8_d(hyq_ctx *ctx, const hyq_weight *w, const hyq_q8 *x, const float *residual_d,
                  float *y_d);
/* Weight::gemv_qkv_fast (src/quant.rs:441-538). */
int hyq_gemv_qkv_q8_d(hyq_ctx *ctx, const hyq_weight *q, const hyq_weight *k,
                      const hyq_weight *v, const hyq_q8 *x, float *yq_d, float *yk_d,
                      float *yv_d);
/* Weight::matmul_gate_up_silu_fast (src/quant.rs:540-651). */
int hyq_gate_up_silu_q8_d(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                          const hyq_q8 *x, float *y_d);
/* The integer block sums of the int8 GEMV (isums_d is [rows][per_row] int32,
 * per_row from hyq_isums_per_row), from the same device code as
 * hyq_gemv_q8_d. Granularity as the reference's SDOT kernels accumulate:
 * STQ1_0 one per block (src/quant.rs:1511-1556), Q2_0C two per block
 * (:1891-1951), Q6_K sixteen per block (:2257-2330); Q4_K (A, B) and Q8_0 one
 * per 32-block are this library's definitions (no reference int path). */
int hyq_isums_per_row(int dtype, size_t cols);
int hyq_gemv_isums_d(hyq_ctx *ctx, const hyq_weight *w, const hyq_q8 *x, int32_t *isums_d);
/* Weight::matmul on device buffers: x_d [batch, cols] f32, y_d [batch, rows]
 * f32. Batch 1 is the int8 GEMV (src/quant.rs:159-270): a float4-aligned x_d
 * whose width is a multiple of 256 (at most 40960) is quantized inside the
 * GEMV launch, bit-identical to hyq_quantize_q8_d followed by hyq_gemv_q8_d;
 * batch >= 2 is the f16-MFMA GEMM (src/quant.rs:272-344). */
int hyq_matmul_d(hyq_ctx *ctx, const hyq_weight *w, const float *x_d, size_t batch,
                 float *y_d);
/* Weight::matmul on device buffers for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. Same arguments, results
 * and launches as hyq_matmul_d (bit for bit), but every temporary - the Q8
 * row of an unstaged batch-1 input, the f16 activation rows and their
 * scales, the K-slice partial sums of a batched product - lives in one
 * fixed per-device array of HYQ_NOALLOC_SCRATCH_BYTES, resident from the
 * first hyq_ctx_create on that device until the process ends; the call makes
 * no hipMalloc/hipFree or other allocating call. A product whose temporaries
 * exceed the array (batch * cols * 2 bytes of f16 rows plus, for batches of at
 * most 128, up to 8 * batch * rows * 4 bytes of partials) returns HYQ_EINVAL
 * before any work. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (several contexts or streams at once) race; serialize
 * them. The array keeps the last call's contents; nothing in it needs to
 * start at zero. */
#define HYQ_NOALLOC_SCRATCH_BYTES (32u * 1024u * 1024u)
int hyq_matmul_noalloc_d(hyq_ctx *ctx, const hyq_weight *w, const float *x_d, size_t batch,
                         float *y_d);
/* ---- MoE expert products: the expert loop of Moe::forward (src/model.rs:699-725).
 * gate and up are rank-3 weights {hidden, mid, E}, down is {mid, hidden, E}
 * (the expert stacks Weight::expert slices, src/quant.rs:144-154). The
 * routed pairs (token, expert, weight) are what route() returned
 * (src/model.rs:728-767) for each token; the caller seeds `out` [tokens,
 * hidden] (the reference seeds it with the shared expert, :699) and this
 * adds, for every token and in ascending expert order, weight * down_e(
 * silu(gate_e x) * (up_e x)) (:700-722). Each expert's token group runs as
 * f16-MFMA GEMMs (DenseFfn::forward at its batch, :672-685). At most 4096
 * tokens and experts and 65535 pairs per call. ---- */
size_t hyq_moe_scratch_bytes(size_t tokens, size_t npairs, size_t experts, size_t hidden,
                             size_t mid);
/* Device buffers, asynchronous. scratch_d: 256-byte aligned, at least
 * hyq_moe_scratch_bytes(...) bytes. Pairs naming a token or expert out of
 * range are skipped. */
int hyq_moe_experts_d(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                      const hyq_weight *down, const float *x_d, size_t tokens,
                      const int32_t *pair_token_d, const int32_t *pair_expert_d,
                      const float *pair_weight_d, size_t npairs, void *scratch_d,
                      size_t scratch_bytes, float *out_d);
/* Host buffers, synchronous; out is read and updated; pairs out of range are
 * HYQ_EINVAL. */
int hyq_moe_experts(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                    const hyq_weight *down, const float *x, size_t tokens,
                    const int32_t *pair_token, const int32_t *pair_expert,
                    const float *pair_weight, size_t npairs, float *out);
/* The expert loop with its seed: out_d = shared x_d (Weight::matmul of the
 * [hidden, hidden] shared projection at batch `tokens`, in the place of
 * Moe::forward's shared expert, src/model.rs:699), then the loop of
 * hyq_moe_experts_d adds into it. For a Q8_0 projection at 2..128 tokens
 * beside Q4_K experts of at most 16 tokens each on average, the shared
 * product runs inside the expert launches: its f16 rows are formed with the
 * experts' token operands and its tiles run beside the SiLU rows, with the
 * same arithmetic as hyq_matmul_d, so out_d holds the same bits as the two
 * calls in sequence (which is what other shapes run). Same pairs, scratch
 * and limits as hyq_moe_experts_d. */
int hyq_moe_shared_experts_d(hyq_ctx *ctx, const hyq_weight *shared, const hyq_weight *gate,
                             const hyq_weight *up, const hyq_weight *down, const float *x_d,
                             size_t tokens, const int32_t *pair_token_d,
                             const int32_t *pair_expert_d, const float *pair_weight_d,
                             size_t npairs, void *scratch_d, size_t scratch_bytes, float *out_d);

/* ---- the whole MoE FFN of a HyV3 layer: Moe::forward (src/model.rs:687-726)
 * ---- */
typedef struct {
    int experts;    /* expert_count */
    int used;       /* expert_used_count */
    int mid;        /* expert_feed_forward_length */
    int shared_mid; /* expert_shared_feed_forward_length */
    int normalize;  /* expert_weights_norm */
    float scale;    /* expert_weights_scale */
} hyq_moe_config;
/* route (src/model.rs:728-767) for `tokens` rows of router logits
 * [tokens][experts]: stable sigmoid, the `used` largest sigmoid + bias
 * (IEEE total order, ties to the lower index), weights sigmoid / sum * scale
 * with the sum of the chosen sigmoids floored at f16's smallest normal when
 * normalize is set (else sum = 1). Writes tokens * used pairs, token-major
 * and in ascending expert order within a token: the lists hyq_moe_experts_d
 * takes. pair_token_d may be null. At most 1024 experts. */
int hyq_moe_route_d(hyq_ctx *ctx, const float *logits_d, const float *bias_d, size_t tokens,
                    size_t experts, size_t used, int normalize, float scale,
                    int32_t *pair_token_d, int32_t *pair_expert_d, float *pair_weight_d);
/* Moe::forward of x_d [tokens][hidden] (rows already normalised) into out_d
 * [tokens][hidden]: router [hidden, experts] F32 (its logits by the F32
 * matmul), route with bias_d [experts] (device), the shared expert
 * (shared_gate/up [hidden, shared_mid], shared_down [shared_mid, hidden])
 * seeding the output, then each chosen expert (gate/up [hidden, mid, E],
 * down [mid, hidden, E]) adding weight * its FFN in ascending expert order.
 * One token runs the int8 GEMVs of the batch-1 path (src/model.rs:507-510);
 * more run the f16-MFMA products. Widths must be whole 256-value groups.
 * scratch_d: 256-byte aligned, hyq_moe_forward_scratch_bytes bytes (0 when
 * the call is not supported: too many tokens per call). */
size_t hyq_moe_forward_scratch_bytes(const hyq_moe_config *mc, size_t hidden, size_t tokens);
int hyq_moe_forward_d(hyq_ctx *ctx, const hyq_moe_config *mc, const hyq_weight *router,
                      const float *bias_d, const hyq_weight *gate, const hyq_weight *up,
                      const hyq_weight *down, const hyq_weight *shared_gate,
                      const hyq_weight *shared_up, const hyq_weight *shared_down,
                      const float *x_d, size_t tokens, void *scratch_d, size_t scratch_bytes,
                      float *out_d);

/* Measurement aid (no counterpart in the reference): reads `bytes` of
 * device memory at buf_d (16-byte aligned) once with `workgroups`
 * workgroups of 256 threads and writes one float per workgroup to sink_d -
 * the read-only HBM rate the HBM-bound products are compared with. */
int hyq_hbm_read_d(hyq_ctx *ctx, const void *buf_d, size_t bytes, int workgroups,
                   float *sink_d);
/* Measurement aid (no counterpart in the reference): `workgroups`
 * workgroups of 256 threads, each wave issuing `iters` rounds of four
 * independent f16 MFMAs (v_mfma_f32_32x32x16_f16, 32768 flop each) on
 * register operands; sink_d receives workgroups * 256 floats - the
 * sustained matrix-core rate the batched products are compared with. */
int hyq_mfma_stream_d(hyq_ctx *ctx, int workgroups, int iters, float *sink_d);

/* decode of rows [row0, row0+nrows) to f32 on the device (Weight::row_into /
 * to_vec, src/quant.rs:99-142). */
int hyq_dequant_rows_d(hyq_ctx *ctx, const hyq_weight *w, size_t row0, size_t nrows,
                       float *out_d);
/* decode of raw GGUF block bytes already on the device. */
int hyq_decode_d(hyq_ctx *ctx, int dtype, const uint8_t *bytes_d, size_t byte_len,
                 float *out_d, size_t n);

/* ---- batch-1 decode-step glue (device pointers, asynchronous) ----
 * Positions and token ids are read from device memory so that a caller can
 * capture a whole step in a HIP graph and replay it. */

/* Weight::row_into (src/quant.rs:123-142) with the row index in device memory.
 * The library cannot check a device-resident index: one outside [0, rows)
 * is clamped into it (the reference's bounds error has no device form). */
int hyq_embed_row_d(hyq_ctx *ctx, const hyq_weight *w, const int32_t *token_d, float *out_d);
/* rms_norm_into (src/model.rs:785-830) fused with Q8::quantize_into: the
 * normalized row y = x * (1/sqrt(mean(x^2)+eps)) * w goes to `out` as Q8 and,
 * when y_d is non-null, as f32. n must equal out's length. */
int hyq_rms_norm_q8_d(hyq_ctx *ctx, const float *x_d, const float *w_d, size_t n, float eps,
                      float *y_d, hyq_q8 *out);
/* For one token at position *pos_d: rope_with_cache on q and k (NeoX halves,
 * src/model.rs:874-917), then the dense order's per-head rms_norm of q and k
 * (src/model.rs:425-446), then KvCache::append (src/model.rs:650-669) of k and
 * v into row *pos_d of kcache/vcache ([context][kv_heads*head_dim] f32).
 * q is updated in place. freq_d[j] = rope_base^(-2j/head_dim). head_dim 128.
 * *pos_d is read on the device, so the library cannot check it: the caches
 * must hold row *pos_d (a negative position appends nothing). */
int hyq_rope_norm_append_d(hyq_ctx *ctx, float *q_d, const float *k_d, const float *v_d,
                           const float *q_norm_d, const float *k_norm_d, const float *freq_d,
                           const int32_t *pos_d, size_t heads, size_t kv_heads, size_t head_dim,
                           float eps, float *kcache_d, float *vcache_d);
/* attention_into (src/model.rs:949-1035) for one query token over cache rows
 * 0..=*pos_d (grouped-query, head_dim 128, scale 1/sqrt(128)). out_d
 * [heads*128] f32 and/or out_q8 (quantized for the output projection) may be
 * null. scratch_d holds hyq_attention_scratch_floats(context, heads) floats. */
size_t hyq_attention_scratch_floats(size_t context, size_t heads);
int hyq_attention_d(hyq_ctx *ctx, const float *q_d, const float *kcache_d,
                    const float *vcache_d, const int32_t *pos_d, size_t context, size_t heads,
                    size_t kv_heads, size_t head_dim, float *scratch_d, float *out_d,
                    hyq_q8 *out_q8);
/* The decode step's attention as the decoder launches it: for the token at
 * position *pos_d, RoPE and the per-head Q/K rms_norm of the raw projections
 * q_d [heads*128] and k_d [kv_heads*128] (dense order, or the hy_v3 one when
 * norm_first is set, src/model.rs:425-446), the append of the new key and
 * v_d to row *pos_d of the caches (KvCache::append, :650-669), then
 * attention_into over rows 0..=*pos_d (:949-1035) into out_d [heads*128].
 * q_d is not modified; scratch_d holds hyq_attention_scratch_floats floats.
 * *pos_d must lie in [0, context): the launch appends nothing outside the
 * caches' `context` rows, whatever the device value.
 * With out_d null only the split partials are formed (the first of the
 * step's two launches: its attention kernel without the merge). */
int hyq_attention_rope_d(hyq_ctx *ctx, const float *q_d, const float *k_d, const float *v_d,
                         const float *q_norm_d, const float *k_norm_d, const float *freq_d,
                         const int32_t *pos_d, size_t context, size_t heads, size_t kv_heads,
                         size_t head_dim, float eps, int norm_first, float *kcache_d,
                         float *vcache_d, float *scratch_d, float *out_d);
/* attention (src/model.rs:949-1037) for n query rows of a chunk whose keys
 * and values are already in the cache: row i (q_d [n][heads*128]) is the
 * token at position *pos_d + i and sees cache rows 0..=*pos_d + i (causal,
 * :956-961). out_d is [n][heads*128] f32; scratch_d holds
 * hyq_attention_rows_scratch_floats(context, heads, n) floats. Rows past
 * `context` are never read. */
size_t hyq_attention_rows_scratch_floats(size_t context, size_t heads, size_t n);
int hyq_attention_rows_d(hyq_ctx *ctx, const float *q_d, const float *kcache_d,
                         const float *vcache_d, const int32_t *pos_d, size_t n, size_t context,
                         size_t heads, size_t kv_heads, size_t head_dim, float *scratch_d,
                         float *out_d);
/* Greedy sampling (src/generation.rs:281-290): index of the first maximum.
 * scratch_d holds 128 floats. */
int hyq_argmax_d(hyq_ctx *ctx, const float *x_d, size_t n, float *scratch_d, int32_t *token_d);

/* ---- dense decoder: Model::forward_into at batch 1 (src/model.rs:374-546)
 * for the hunyuan-dense graph, device-resident, KV cache in HBM ---- */
typedef struct {
    int layers, hidden, heads, kv_heads, head_dim, ffn, vocab;
    float rope_base, rms_eps;
} hyq_dense_config;
typedef struct hyq_dense hyq_dense;

/* Model::new_session (src/model.rs:287-322) with `context` cached positions. */
int hyq_dense_create(hyq_ctx *ctx, const hyq_dense_config *cfg, size_t context,
                     hyq_dense **out);
void hyq_dense_destroy(hyq_dense *m);
/* Layer weights (borrowed: they must outlive the decoder) and f32 norm vectors
 * (copied), as Model::from_gguf binds them (src/model.rs:204-258). gate, up
 * and down may all be null for a layer whose FFN is an MoE
 * (hyq_dense_set_moe). */
int hyq_dense_set_layer(hyq_dense *m, int layer, const hyq_weight *q, const hyq_weight *k,
                        const hyq_weight *v, const hyq_weight *o, const hyq_weight *gate,
                        const hyq_weight *up, const hyq_weight *down, const float *attn_norm,
                        const float *ffn_norm, const float *q_norm, const float *k_norm);
/* Model::from_gguf's architecture (src/model.rs:137-142): hunyuan-dense
 * normalises q and k per head after RoPE, hy_v3 before it (:425-446). */
enum { HYQ_ARCH_DENSE = 0, HYQ_ARCH_HYV3 = 1 };
int hyq_dense_set_architecture(hyq_dense *m, int arch);
/* Ffn::Moe of one layer (src/model.rs:82-92, :206-235): the layer's FFN
 * becomes Moe::forward (see hyq_moe_forward_d for the weights' shapes) with
 * the selection bias `bias` [experts] (host, copied); hyq_dense_set_layer's
 * gate/up/down are then null for that layer. Every MoE layer of a decoder
 * shares one hyq_moe_config shape (the expert_* metadata is model-wide).
 * Weights are borrowed. */
int hyq_dense_set_moe(hyq_dense *m, int layer, const hyq_moe_config *mc,
                      const hyq_weight *router, const float *bias, const hyq_weight *gate,
                      const hyq_weight *up, const hyq_weight *down, const hyq_weight *shared_gate,
                      const hyq_weight *shared_up, const hyq_weight *shared_down);
/* token_embd / output (tied when the same weight, src/model.rs:194-202). */
int hyq_dense_set_output(hyq_dense *m, const hyq_weight *embedding, const hyq_weight *output,
                         const float *output_norm);
/* Writes cached keys/values [positions][kv_heads*head_dim] of one layer. */
int hyq_dense_load_kv(hyq_dense *m, int layer, size_t positions, const float *keys,
                      const float *values);
int hyq_dense_set_position(hyq_dense *m, size_t position);
int hyq_dense_get_position(hyq_dense *m, size_t *position);
/* One token through the model (Model::forward_into, batch 1): appends its
 * K/V at the current position, advances it, and returns the logits (if
 * non-null) and the greedy next token (if non-null). */
int hyq_dense_forward(hyq_dense *m, int32_t token, float *logits, int32_t *next);
/* Model::prefill_into (src/model.rs:630-646): the prompt through
 * forward_into at batch n (:549-616, f16-MFMA products), on the device in
 * passes of hyq_dense_set_prefill_rows tokens; as in the reference's
 * 256-token chunking (PREFILL_CHUNK, :18), a prompt of 256k + 1 tokens ends
 * with its last token through the batch-1 step.
 * Appends every token's K/V from the current position, advances it by n,
 * and returns the last token's logits (if non-null) and greedy next token
 * (if non-null). HYQ_EINVAL for an empty prompt, one that exceeds the
 * context, or a token outside the vocabulary (checked before any work). */
int hyq_dense_prefill(hyq_dense *m, const int32_t *tokens, size_t n, float *logits,
                      int32_t *next);
/* Tokens per device pass of hyq_dense_prefill (default 1024; 1..65536). The
 * results do not depend on it; it sets the activation memory: per row about
 * 4*hidden + 8*(heads + kv_heads)*head_dim + 6*ffn bytes, plus 528 bytes per
 * query head and attention split. No counterpart in the reference, whose
 * chunk is fixed. */
int hyq_dense_set_prefill_rows(hyq_dense *m, size_t rows);
/* Parity tracing (no counterpart in the reference: it exposes the hidden row
 * that Model::forward_into carries between layers, src/model.rs:394-513).
 * With trace_d set (device memory of `floats` floats, at least
 * (layers + 1) * hidden), hyq_dense_forward writes the hidden row after the
 * embedding and after each layer as [layers + 1][hidden]; a hyq_dense_prefill
 * pass of n rows writes [layers + 1][n][hidden] when it fits in `floats`.
 * Graph replays (hyq_dense_generate) never write it. NULL switches it off. */
int hyq_dense_set_trace(hyq_dense *m, float *trace_d, size_t floats);
/* Reads cached keys/values [positions][kv_heads*head_dim] of one layer
 * (the Session's KvCache, src/model.rs:650-669). */
int hyq_dense_read_kv(hyq_dense *m, int layer, size_t positions, float *keys, float *values);
/* Greedy decoding (Generator::generate at temperature 0 and repetition
 * penalty 1): feeds `token`, then each argmax, for `steps` steps; tokens[i]
 * is the argmax after step i. use_graph = 1 replays one captured HIP graph
 * per step; 0 launches the same kernels one by one. */
int hyq_dense_generate(hyq_dense *m, int32_t token, size_t steps, int use_graph,
                       int32_t *tokens);

/* ---- GGUF v3 files (Gguf::open / parse, src/gguf.rs:50-210) ---- */
/* Profiles (src/gguf.rs:17-26): type ids 40 and 42 are Q2_0C / STQ1_0 only
 * under their Tencent profiles; AUTO resolves a file carrying them by its
 * SHA-256 (the two known exports, :14-15) and fails otherwise. */
enum {
    HYQ_PROFILE_AUTO = 0,
    HYQ_PROFILE_STANDARD = 1,
    HYQ_PROFILE_TENCENT_Q2_0C = 2,
    HYQ_PROFILE_TENCENT_STQ1 = 3
};
typedef struct hyq_gguf hyq_gguf;
/* TensorInfo (src/gguf.rs:28-38); name is valid while the file is open. */
typedef struct {
    const char *name;
    uint64_t dims[4]; /* GGUF order: the contiguous input dimension first */
    int rank;
    uint32_t type_id; /* as stored */
    int dtype;        /* hyq_dtype after profile resolution */
    uint64_t offset;  /* absolute byte offset in the file */
    uint64_t byte_len;
} hyq_gguf_tensor;
/* Gguf::open: maps the file read-only and validates it like the reference
 * (every count, string, array and tensor extent bounds-checked; errors
 * HYQ_EINVAL, or HYQ_EDTYPE for a type id with no format under the profile).
 * The file must stay unchanged while open. */
int hyq_gguf_open(const char *path, int profile, hyq_gguf **out);
/* The same over caller memory, borrowed until hyq_gguf_close. */
int hyq_gguf_open_bytes(const uint8_t *bytes, size_t len, int profile, hyq_gguf **out);
void hyq_gguf_close(hyq_gguf *g);
/* The resolved profile (never HYQ_PROFILE_AUTO). */
int hyq_gguf_profile(const hyq_gguf *g);
size_t hyq_gguf_byte_len(const hyq_gguf *g);
const uint8_t *hyq_gguf_bytes(const hyq_gguf *g);
/* Tensors in name order (the reference's BTreeMap). */
size_t hyq_gguf_tensor_count(const hyq_gguf *g);
int hyq_gguf_tensor_at(const hyq_gguf *g, size_t index, hyq_gguf_tensor *out);
int hyq_gguf_find_tensor(const hyq_gguf *g, const char *name, hyq_gguf_tensor *out);
/* Metadata accessors (Gguf::usize / float / boolean / string, :220-258):
 * u64 takes non-negative integers, f64 any number; arrays give their
 * element type and length. HYQ_EINVAL when missing or of another type. */
int hyq_gguf_meta_u64(const hyq_gguf *g, const char *key, uint64_t *out);
int hyq_gguf_meta_f64(const hyq_gguf *g, const char *key, double *out);
int hyq_gguf_meta_bool(const hyq_gguf *g, const char *key, int *out);
int hyq_gguf_meta_str(const hyq_gguf *g, const char *key, const char **out, size_t *len);
int hyq_gguf_meta_array(const hyq_gguf *g, const char *key, uint32_t *elem_type,
                        uint64_t *count);
/* Gguf::tensor + upload: a rank-2 matrix or rank-3 expert stack as a
 * device weight (hyq_weight_upload of the tensor's bytes). */
int hyq_gguf_upload(hyq_ctx *ctx, const hyq_gguf *g, const char *name, hyq_weight **out);
/* Weight::to_vec of any tensor (norm vectors): n f32 values. */
int hyq_gguf_read_f32(hyq_ctx *ctx, const hyq_gguf *g, const char *name, float *out, size_t n);
/* SHA-256 (FIPS 180-4), the digest the AUTO profile checks. */
int hyq_sha256(const uint8_t *bytes, size_t len, uint8_t digest[32]);
/* Model::from_gguf (src/model.rs:136-262) + Model::new_session's context
 * check (:264-270): reads the hunyuan-dense or hy_v3 configuration, checks
 * every tensor's shape, uploads the weights (owned by the decoder) and the
 * norm vectors. vocab = the length of tokenizer.ggml.tokens. A hy_v3 file
 * gets the hy_v3 Q/K-norm order and, for every layer after the first, its
 * MoE FFN (expert_* metadata, sigmoid gating required, F32 router
 * ffn_gate_inp, bias exp_probs_b, ffn_{gate,up,down}_exps expert stacks,
 * ffn_{gate,up,down}_shexp shared expert) and needs a separate output. */
int hyq_dense_from_gguf(hyq_ctx *ctx, const hyq_gguf *g, size_t context, hyq_dense **out);

#ifdef __cplusplus
}
#endif
#endif
