// Decode-step glue entry points and the dense batch-1 decoder of the C ABI.
//
// hyq_dense composes, per token, the same kernels the reference's
// Model::forward_into batch-1 arm calls per layer (src/model.rs:394-513):
// rms_norm -> Q8 -> fused QKV GEMV -> RoPE + Q/K norm + KV append ->
// attention -> Q8 -> attn_output GEMV (+ residual) -> rms_norm -> Q8 ->
// gate/up SiLU GEMV -> Q8 -> down GEMV (+ residual); then output norm ->
// Q8 -> lm_head GEMV -> argmax. Position and token stay in device memory, so
// one step is captured once as a HIP graph and replayed per token.
//
// hyq_dense_prefill runs a prompt through the batch > 1 arm
// (src/model.rs:549-616, 630-646): per layer the RMSNorm of every row fused
// with its f16 rounding, one f16-MFMA GEMM for Q, K and V, RoPE + Q/K norm +
// KV append for all rows, causal attention of every row over the cache, the
// attention-output GEMM with the residual add in its epilogue, the FFN norm,
// the gate/up GEMM with silu(g)*u in its epilogue and the down GEMM with the
// residual add; then the last row's output norm, the lm_head GEMV and the
// argmax. Every row's result is independent of the other rows of its pass,
// so the device takes up to `prefill_rows` tokens per pass (default 1024)
// instead of the reference's 256-token chunks with identical results; the
// one case where the chunking shows is kept: a prompt of 256k + 1 tokens
// ends with a one-token chunk, which the reference runs through the batch-1
// arm, and so does this decoder (the decode step).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

#include "hyq_abi.hpp"
#include "hyq_moe_ffn.hpp"
#include "hyq_step.hpp"

using namespace hyq;

namespace {

int check_ctx(hyq_ctx *ctx, const char *who)
{
    if (!ctx) return fail(HYQ_EINVAL, "%s: null context", who);
    return HYQ_OK;
}

GemvArgs gemv_args(const hyq_weight *w, const Q8Ref &x, float *y, const float *residual)
{
    GemvArgs a{};
    a.nseg = 1;
    a.seg[0].w = w->view;
    a.seg[0].y = y;
    a.rows_total = (int)w->rows;
    a.groups = (int)(w->cols / 256);
    a.x = x.view();
    a.residual = residual;
    return a;
}

bool int8_ok(const hyq_weight *w)
{
    return w && w->rank == 2 && is_quant(w->dtype) && w->cols % 256 == 0 && w->cols <= 240 * 256;
}

} // namespace

// ---------------------------------------------------------------------------
// glue entry points
// ---------------------------------------------------------------------------
extern "C" {

int hyq_embed_row_d(hyq_ctx *ctx, const hyq_weight *w, const int32_t *token_d, float *out_d)
{
    int rc = check_ctx(ctx, "embed_row");
    if (rc) return rc;
    if (!w || !token_d || !out_d) return fail(HYQ_EINVAL, "embed_row: null argument");
    if (w->rank != 2) return fail(HYQ_EINVAL, "embed_row: weight is not a matrix");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_embed_row(w->dtype, w->view, (int)w->cols, token_d, out_d, ctx->stream),
               "embed_row");
    return HYQ_OK;
}

int hyq_rms_norm_q8_d(hyq_ctx *ctx, const float *x_d, const float *w_d, size_t n, float eps,
                      float *y_d, hyq_q8 *out)
{
    int rc = check_ctx(ctx, "rms_norm_q8");
    if (rc) return rc;
    if (!x_d || !w_d || !out) return fail(HYQ_EINVAL, "rms_norm_q8: null argument");
    if (n == 0 || n != out->ref.n) return fail(HYQ_EINVAL, "rms_norm_q8: length %zu", n);
    DeviceGuard g(ctx->device);
    const Q8Ref &q = out->ref;
    HYQ_LAUNCH(launch_rms_norm_q8(x_d, w_d, (int)n, eps, y_d, q.q, q.s, q.sum16, q.sum32,
                                  q.sum256, ctx->stream),
               "rms_norm_q8");
    return HYQ_OK;
}

int hyq_rope_norm_append_d(hyq_ctx *ctx, float *q_d, const float *k_d, const float *v_d,
                           const float *q_norm_d, const float *k_norm_d, const float *freq_d,
                           const int32_t *pos_d, size_t heads, size_t kv_heads, size_t head_dim,
                           float eps, float *kcache_d, float *vcache_d)
{
    int rc = check_ctx(ctx, "rope_norm_append");
    if (rc) return rc;
    if (!q_d || !k_d || !v_d || !q_norm_d || !k_norm_d || !freq_d || !pos_d || !kcache_d ||
        !vcache_d)
        return fail(HYQ_EINVAL, "rope_norm_append: null argument");
    if (head_dim != 128 || heads == 0 || kv_heads == 0 || heads % kv_heads)
        return fail(HYQ_EINVAL, "rope_norm_append: heads %zu/%zu of dim %zu", heads, kv_heads,
                    head_dim);
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_rope_norm_kv(q_d, k_d, v_d, q_norm_d, k_norm_d, freq_d, pos_d, (int)heads,
                                   (int)kv_heads, (int)head_dim, eps, kcache_d, vcache_d,
                                   ctx->stream),
               "rope_norm_append");
    return HYQ_OK;
}

size_t hyq_attention_scratch_floats(size_t context, size_t heads)
{
    // split partials, and an f32 output row for callers that only want Q8
    return (size_t)attention_splits((int)context) * heads * PART_STRIDE + heads * 128;
}

int hyq_attention_d(hyq_ctx *ctx, const float *q_d, const float *kcache_d,
                    const float *vcache_d, const int32_t *pos_d, size_t context, size_t heads,
                    size_t kv_heads, size_t head_dim, float *scratch_d, float *out_d,
                    hyq_q8 *out_q8)
{
    int rc = check_ctx(ctx, "attention");
    if (rc) return rc;
    if (!q_d || !kcache_d || !vcache_d || !pos_d || !scratch_d)
        return fail(HYQ_EINVAL, "attention: null argument");
    if (head_dim != 128 || heads == 0 || kv_heads == 0 || heads % kv_heads ||
        heads / kv_heads > (size_t)ATT_MAX_REP || context == 0 || context > 65536)
        return fail(HYQ_EINVAL, "attention: unsupported shape");
    if (out_q8 && out_q8->ref.n != heads * head_dim)
        return fail(HYQ_EINVAL, "attention: Q8 length %zu != %zu", out_q8->ref.n,
                    heads * head_dim);
    DeviceGuard g(ctx->device);
    const size_t part_floats = (size_t)attention_splits((int)context) * heads * PART_STRIDE;
    float *out = out_d ? out_d : scratch_d + part_floats;
    HYQ_LAUNCH(launch_attention(q_d, kcache_d, vcache_d, pos_d, (int)context, (int)heads,
                                (int)kv_heads, scratch_d, out, ctx->stream),
               "attention");
    if (out_q8) {
        const Q8Ref &q = out_q8->ref;
        HYQ_LAUNCH(launch_quantize_q8(out, (int)(heads * head_dim), q.q, q.s, q.sum16, q.sum32,
                                      q.sum256, ctx->stream),
                   "quantize_q8");
    }
    return HYQ_OK;
}

int hyq_attention_rope_d(hyq_ctx *ctx, const float *q_d, const float *k_d, const float *v_d,
                         const float *q_norm_d, const float *k_norm_d, const float *freq_d,
                         const int32_t *pos_d, size_t context, size_t heads, size_t kv_heads,
                         size_t head_dim, float eps, int norm_first, float *kcache_d,
                         float *vcache_d, float *scratch_d, float *out_d)
{
    int rc = check_ctx(ctx, "attention_rope");
    if (rc) return rc;
    if (!q_d || !k_d || !v_d || !q_norm_d || !k_norm_d || !freq_d || !pos_d || !kcache_d ||
        !vcache_d || !scratch_d)
        return fail(HYQ_EINVAL, "attention_rope: null argument");
    if (head_dim != 128 || heads == 0 || kv_heads == 0 || heads % kv_heads ||
        heads / kv_heads > (size_t)ATT_MAX_REP || context == 0 || context > 65536)
        return fail(HYQ_EINVAL, "attention_rope: unsupported shape");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_attention_rope(q_d, k_d, v_d, q_norm_d, k_norm_d, freq_d, eps, kcache_d,
                                     vcache_d, pos_d, (int)context, (int)heads, (int)kv_heads,
                                     scratch_d, ctx->stream, norm_first != 0),
               "attention_rope");
    if (out_d)
        HYQ_LAUNCH(launch_attention_merge(scratch_d, (int)context, (int)heads, pos_d, out_d,
                                          ctx->stream),
                   "attention_merge");
    return HYQ_OK;
}

size_t hyq_attention_rows_scratch_floats(size_t context, size_t heads, size_t n)
{
    return n * (size_t)prefill_attention_splits((int)context) * heads * PART_STRIDE;
}

int hyq_attention_rows_d(hyq_ctx *ctx, const float *q_d, const float *kcache_d,
                         const float *vcache_d, const int32_t *pos_d, size_t n, size_t context,
                         size_t heads, size_t kv_heads, size_t head_dim, float *scratch_d,
                         float *out_d)
{
    int rc = check_ctx(ctx, "attention_rows");
    if (rc) return rc;
    if (!q_d || !kcache_d || !vcache_d || !pos_d || !scratch_d || !out_d)
        return fail(HYQ_EINVAL, "attention_rows: null argument");
    if (head_dim != 128 || heads == 0 || kv_heads == 0 || heads % kv_heads ||
        heads / kv_heads > (size_t)ATT_MAX_REP || context == 0 || context > 65536)
        return fail(HYQ_EINVAL, "attention_rows: unsupported shape");
    if (n == 0 || n > context) return fail(HYQ_EINVAL, "attention_rows: %zu query rows", n);
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_attention_rows(q_d, kcache_d, vcache_d, pos_d, (int)n, (int)context,
                                     (int)heads, (int)kv_heads, scratch_d, out_d, ctx->stream),
               "attention_rows");
    return HYQ_OK;
}

int hyq_argmax_d(hyq_ctx *ctx, const float *x_d, size_t n, float *scratch_d, int32_t *token_d)
{
    int rc = check_ctx(ctx, "argmax");
    if (rc) return rc;
    if (!x_d || !scratch_d || !token_d || n == 0 || n > 0x7fffffff)
        return fail(HYQ_EINVAL, "argmax: bad argument");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_argmax(x_d, (int)n, scratch_d, (int *)(scratch_d + 64), token_d, nullptr,
                             nullptr, ctx->stream),
               "argmax");
    return HYQ_OK;
}

} // extern "C"

// ---------------------------------------------------------------------------
// dense decoder
// ---------------------------------------------------------------------------
struct hyq_dense {
    hyq_ctx *ctx = nullptr;
    hyq_dense_config cfg{};
    size_t context = 0;
    size_t pos_host = 0;
    // set when a forward produced non-finite logits (the reference poisons
    // the session, src/model.rs:348-351, :371, :540-545); cleared by a new
    // position
    bool poisoned = false;
    struct Layer {
        const hyq_weight *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
        // the dense FFN, or none when the layer's FFN is an MoE (moe set)
        const hyq_weight *gate = nullptr, *up = nullptr, *down = nullptr;
        float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
        std::unique_ptr<MoeFfn> moe;
        std::unique_ptr<DeviceBuffer> moe_bias; // the MoE's selection bias
    };
    std::vector<Layer> layers;
    int arch = HYQ_ARCH_DENSE;
    // the MoE shape every MoE layer shares (expert_* metadata is model-wide)
    hyq_moe_config moe_cfg{};
    bool has_moe = false;
    // batch-1 MoE temporaries: the normalized row, its Q8, the FFN's buffers
    std::unique_ptr<DeviceBuffer> moe_mem;
    float *moe_xn = nullptr;
    Q8Ref moe_q8;
    // the output row's normalised Q8 (the lm_head GEMV's input)
    Q8Ref out_q8;
    MoeRowBuf moe_row{};
    const hyq_weight *embedding = nullptr, *output = nullptr;
    float *output_norm = nullptr;

    DeviceBuffer mem;       // norms, freq, activations, scratch, state
    DeviceBuffer kv;        // [layers][2][context][kv_heads*head_dim]
    float *freq = nullptr, *hidden = nullptr, *qb = nullptr, *kb = nullptr, *vb = nullptr;
    float *gb = nullptr, *logits = nullptr, *att_scratch = nullptr, *argmax_scratch = nullptr;
    float *att_out = nullptr; // merged attention output [heads * head_dim]
    // The down projection runs as `down_ks` K slices writing partial rows
    // [down_ks][hidden]; the next layer's QKV stage (or the lm_head's) adds
    // them to the hidden row it normalizes, and the attention output adds
    // them to its residual, which materializes the hidden row again.
    float *parts = nullptr;
    int down_ks = 1;
    int32_t *token = nullptr, *history = nullptr;
    StepState *state = nullptr;
    size_t history_cap = 0;
    std::unique_ptr<DeviceBuffer> history_mem;

    // hidden rows after the embedding and after every layer, written by the
    // eager forward and prefill when set (hyq_dense_set_trace)
    float *trace = nullptr;
    size_t trace_floats = 0;

    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<hyq_weight *> owned; // weights this decoder releases

    // chunked prefill activations (allocated on the first prefill):
    // hid [n][H], q [n][QL], k/v [n][KV], att [n][QL], h [n][F] f32;
    // xh [n][max(H, QL, F)] f16 with row scales rs [n]; attention partials;
    // the chunk's token ids
    std::unique_ptr<DeviceBuffer> pf_mem;
    size_t pf_rows = 1024, pf_cap = 0; // rows per pass; rows the buffers hold
    float *pf_hid = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
    float *pf_att = nullptr, *pf_h = nullptr, *pf_rs = nullptr, *pf_part = nullptr;
    float *pf_kpart = nullptr; // K-slice partials of the output and down GEMMs
    size_t pf_kpart_floats = 0;
    float *pf_xn = nullptr;    // MoE layers: the normalized rows [n][H] f32
    MoeRowsBuf pf_moe{};
    _Float16 *pf_xh = nullptr;
    int32_t *pf_tok = nullptr;

    ~hyq_dense()
    {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        for (hyq_weight *w : owned) hyq_weight_release(w);
    }
    size_t kvw() const { return (size_t)cfg.kv_heads * cfg.head_dim; }
    float *kcache(int l) { return (float *)kv.ptr + (size_t)l * 2 * context * kvw(); }
    float *vcache(int l) { return kcache(l) + context * kvw(); }
    void drop_graph()
    {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
    }
};

void hyq::dense_adopt(hyq_dense *m, hyq_weight *w) { m->owned.push_back(w); }

namespace {

// One token: embedding row, then per layer five kernels - the QKV GEMV
// (RMSNorm + Q8 in its input stage), attention (RoPE, Q/K norm, KV append,
// merge), the output GEMV (Q8 of the attention row in its input stage,
// residual add), the gate/up GEMV (RMSNorm + Q8, SiLU product) and the down
// GEMV (Q8 of the SiLU row, residual add) - then the lm_head GEMV (output
// RMSNorm + Q8) and the argmax.
// K slices of the down projection: the most (up to GEMV_MAX_PARTS) that
// leave every slice at least 8 whole groups (one per sub-lane).
int down_kslices(int groups)
{
    for (int k = GEMV_MAX_PARTS; k > 1; --k)
        if (groups % k == 0 && groups / k >= 8) return k;
    return 1;
}

GemvArgs staged(const hyq_weight *w, const float *xin, const float *norm, float eps, float *y,
                const float *residual)
{
    GemvArgs a{};
    a.nseg = 1;
    a.seg[0].w = w->view;
    a.seg[0].y = y;
    a.rows_total = (int)w->rows;
    a.groups = (int)(w->cols / 256);
    a.residual = residual;
    a.xin = xin;
    a.norm = norm;
    a.eps = eps;
    return a;
}

// The output norm and lm_head (src/model.rs:374-380): the row (plus the
// last down projection's nparts partial rows) normalised and quantized to Q8
// once, then the Q8-input GEMV (one row per lane, no input stage repeated by
// each of its workgroups).
int lm_head(hyq_dense *m, const float *x, const float *parts, int nparts, hipStream_t st,
            Q8Trace *q8t)
{
    const hyq_dense_config &c = m->cfg;
    const Q8Ref &q = m->out_q8;
    // (traced: the normalized row goes straight into the record)
    int8_t *tq = nullptr;
    float *ts = nullptr, *tx = nullptr;
    const bool tr = q8t && q8t->take((size_t)c.hidden, &tq, &ts, &tx);
    HYQ_LAUNCH(launch_rms_norm_q8(x, m->output_norm, c.hidden, c.rms_eps, tr ? tx : nullptr, q.q,
                                  q.s, q.sum16, q.sum32, q.sum256, st, parts, nparts, c.hidden),
               "output_norm_q8");
    if (tr) {
        HYQ_HIP(hipMemcpyAsync(tq, q.q, c.hidden, hipMemcpyDeviceToDevice, st), "q8 trace");
        HYQ_HIP(hipMemcpyAsync(ts, q.s, c.hidden / 64, hipMemcpyDeviceToDevice, st), "q8 trace");
    }
    HYQ_LAUNCH(launch_gemv(m->output->dtype, GEMV_PLAIN, gemv_args(m->output, q, m->logits, nullptr),
                           st),
               "gemv_lm_head");
    return HYQ_OK;
}

// One decode step. It ends with the greedy token, whose final pass also
// writes that token's embedding row to the hidden row; embed = false starts
// from that row (the decode loop after its first step), embed = true embeds
// the state's token first.
int enqueue_step(hyq_dense *m, bool trace = false, bool embed = true)
{
    const hyq_dense_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    if (embed)
        HYQ_LAUNCH(launch_embed_row(m->embedding->dtype, m->embedding->view, c.hidden, m->token,
                                    m->hidden, st),
                   "embed_row");
    const int *pos = &m->state->pos;
    const int ks = m->down_ks;
    const bool norm_first = m->arch == HYQ_ARCH_HYV3;
    // the context's Q8 record (eager steps only: a captured graph keeps none)
    Q8Trace *q8t = trace ? m->ctx->q8t() : nullptr;
    trace = trace && m->trace;
    if (trace)
        HYQ_LAUNCH(launch_sum_parts(m->hidden, nullptr, 0, 0, c.hidden, m->trace, st), "trace");
    // partial rows the previous layer's down projection left (a dense layer
    // with a K-split down; an MoE layer writes the whole hidden row)
    int np = 0;
    for (int l = 0; l < c.layers; ++l) {
        const hyq_dense::Layer &L = m->layers[l];
        {
            GemvArgs a = staged(L.q, m->hidden, L.attn_norm, c.rms_eps, m->qb, nullptr);
            a.sparts = m->parts;
            a.nsparts = np;
            a.parts_stride = c.hidden;
            const hyq_weight *ws[3] = {L.q, L.k, L.v};
            float *ys[3] = {m->qb, m->kb, m->vb};
            int start = 0;
            for (int i = 0; i < 3; ++i) {
                a.seg[i].w = ws[i]->view;
                a.seg[i].y = ys[i];
                a.seg[i].row_start = start;
                start += (int)ws[i]->rows;
            }
            a.nseg = 3;
            a.rows_total = start;
            q8_trace_gemv(q8t, a);
            HYQ_LAUNCH(launch_gemv(L.q->dtype, GEMV_MULTI, a, st), "gemv_qkv");
        }
        HYQ_LAUNCH(launch_attention_rope(m->qb, m->kb, m->vb, L.q_norm, L.k_norm, m->freq,
                                         c.rms_eps, m->kcache(l), m->vcache(l), pos,
                                         (int)m->context, c.heads, c.kv_heads, m->att_scratch,
                                         st, norm_first),
                   "attention");
        HYQ_LAUNCH(launch_attention_merge(m->att_scratch, (int)m->context, c.heads, pos,
                                          m->att_out, st),
                   "attention_merge");
        {
            GemvArgs a = staged(L.o, m->att_out, nullptr, 0.f, m->hidden, m->hidden);
            a.rparts = m->parts;
            a.nrparts = np;
            a.parts_stride = c.hidden;
            q8_trace_gemv(q8t, a);
            HYQ_LAUNCH(launch_gemv(L.o->dtype, GEMV_PLAIN, a, st), "gemv_attn_output");
        }
        if (L.moe) {
            // Ffn::Moe (src/model.rs:507-510): the normalized row and its Q8,
            // then Moe::forward and the residual add (:512)
            const Q8Ref &q = m->moe_q8;
            HYQ_LAUNCH(launch_rms_norm_q8(m->hidden, L.ffn_norm, c.hidden, c.rms_eps, m->moe_xn,
                                          q.q, q.s, q.sum16, q.sum32, q.sum256, st),
                       "rms_norm_q8");
            if (int rc = q8_trace_copy(q8t, q, m->moe_xn, (size_t)c.hidden, st)) return rc;
            int rc = moe_ffn_row(st, *L.moe, m->moe_xn, q, m->moe_row, m->hidden, m->hidden,
                                 trace ? m->trace + (size_t)(l + 1) * c.hidden : nullptr, q8t);
            if (rc) return rc;
            np = 0;
            continue;
        }
        {
            GemvArgs a = staged(L.gate, m->hidden, L.ffn_norm, c.rms_eps, m->gb, nullptr);
            a.nseg = 2;
            a.seg[1].w = L.up->view;
            q8_trace_gemv(q8t, a);
            HYQ_LAUNCH(launch_gemv(L.gate->dtype, GEMV_SILU, a, st), "gemv_gate_up_silu");
        }
        if (ks > 1) {
            GemvArgs a = staged(L.down, m->gb, nullptr, 0.f, m->parts, nullptr);
            a.groups /= ks;
            a.kslices = ks;
            q8_trace_gemv(q8t, a);
            HYQ_LAUNCH(launch_gemv(L.down->dtype, GEMV_PLAIN, a, st), "gemv_down");
        } else {
            GemvArgs a = staged(L.down, m->gb, nullptr, 0.f, m->hidden, m->hidden);
            q8_trace_gemv(q8t, a);
            HYQ_LAUNCH(launch_gemv(L.down->dtype, GEMV_PLAIN, a, st), "gemv_down");
        }
        np = ks > 1 ? ks : 0;
        if (trace)
            HYQ_LAUNCH(launch_sum_parts(m->hidden, m->parts, np, c.hidden, c.hidden,
                                        m->trace + (size_t)(l + 1) * c.hidden, st),
                       "trace");
    }
    if (int rc = lm_head(m, m->hidden, m->parts, np, st, q8t)) return rc;
    HYQ_LAUNCH(launch_argmax_embed(m->logits, c.vocab, m->argmax_scratch,
                                   (int *)(m->argmax_scratch + 64), m->token, m->state, m->history,
                                   m->embedding->dtype, m->embedding->view, c.hidden, m->hidden,
                                   st),
               "argmax");
    return HYQ_OK;
}

// PREFILL_CHUNK (src/model.rs:18): tokens per forward_into call.
constexpr size_t PREFILL_CHUNK = 256;

// Rows per prefill pass: the set size, at most the context, and for a model
// with MoE layers at most what the grouped expert kernels take per call.
size_t pass_rows(const hyq_dense *m)
{
    size_t N = std::min(m->pf_rows, m->context);
    for (const hyq_dense::Layer &L : m->layers)
        if (L.moe) N = std::min(N, (size_t)moe_rows_max(*L.moe));
    return N;
}

int prefill_buffers(hyq_dense *m)
{
    const size_t N = pass_rows(m);
    if (m->pf_mem && m->pf_cap == N) return HYQ_OK;
    m->pf_mem.reset();
    m->pf_cap = 0;
    const hyq_dense_config &c = m->cfg;
    const size_t H = (size_t)c.hidden, F = (size_t)c.ffn;
    const size_t QL = (size_t)c.heads * c.head_dim, KV = (size_t)c.kv_heads * c.head_dim;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += align_up(bytes, 256);
        return o;
    };
    const size_t o_hid = take(N * H * 4), o_q = take(N * QL * 4), o_k = take(N * KV * 4);
    const size_t o_v = take(N * KV * 4), o_att = take(N * QL * 4), o_h = take(N * F * 4);
    const size_t o_xh = take(N * std::max(H, std::max(QL, F)) * 2), o_rs = take(N * 4);
    const size_t o_part = take(N * (size_t)c.heads *
                               (size_t)prefill_attention_splits((int)m->context) * PART_STRIDE * 4);
    const size_t o_tok = take(N * 4);
    // the split attention-output and down GEMMs' partials (every layer's
    // formats: they may differ)
    size_t kp = 0, moe_bytes = 0;
    const MoeFfn *moe = nullptr;
    for (const hyq_dense::Layer &L : m->layers) {
        kp = std::max(kp, gemm_split_floats(L.o->dtype, (int)H, (int)N, (int)QL));
        if (L.down) kp = std::max(kp, gemm_split_floats(L.down->dtype, (int)H, (int)N, (int)F));
        if (L.moe && moe_rows_bytes(*L.moe, (int)N) > moe_bytes) {
            moe = L.moe.get();
            moe_bytes = moe_rows_bytes(*moe, (int)N);
        }
    }
    const size_t o_kpart = take(kp * 4);
    const size_t o_xn = moe ? take(N * H * 4) : 0;
    const size_t o_moe = moe ? take(moe_bytes) : 0;
    auto buf = std::make_unique<DeviceBuffer>();
    int rc = buf->alloc(m->ctx->device, off);
    if (rc) return rc;
    uint8_t *b = (uint8_t *)buf->ptr;
    m->pf_hid = (float *)(b + o_hid);
    m->pf_q = (float *)(b + o_q);
    m->pf_k = (float *)(b + o_k);
    m->pf_v = (float *)(b + o_v);
    m->pf_att = (float *)(b + o_att);
    m->pf_h = (float *)(b + o_h);
    m->pf_xh = (_Float16 *)(b + o_xh);
    m->pf_rs = (float *)(b + o_rs);
    m->pf_part = (float *)(b + o_part);
    m->pf_tok = (int32_t *)(b + o_tok);
    m->pf_kpart = (float *)(b + o_kpart);
    m->pf_kpart_floats = kp;
    if (moe) {
        m->pf_xn = (float *)(b + o_xn);
        m->pf_moe = moe_rows_carve(*moe, (int)N, b + o_moe);
    }
    m->pf_mem = std::move(buf);
    m->pf_cap = N;
    return HYQ_OK;
}

// One chunk of n >= 2 tokens at position m->state->pos (the chunk's ids are
// in m->pf_tok); leaves the last row's logits in m->logits and the greedy
// token in m->token.
int enqueue_prefill_chunk(hyq_dense *m, int n)
{
    const hyq_dense_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int H = c.hidden, F = c.ffn, QL = c.heads * c.head_dim;
    const int *pos = &m->state->pos;
    HYQ_LAUNCH(launch_embed_rows(m->embedding->dtype, m->embedding->view, H, m->pf_tok, n,
                                 m->pf_hid, st),
               "embed_rows");
    const size_t rows = (size_t)n * H;
    const bool trace = m->trace && (size_t)(c.layers + 1) * rows <= m->trace_floats;
    if (trace)
        HYQ_HIP(hipMemcpyAsync(m->trace, m->pf_hid, rows * 4, hipMemcpyDeviceToDevice, st),
                "trace");
    for (int l = 0; l < c.layers; ++l) {
        const hyq_dense::Layer &L = m->layers[l];
        HYQ_LAUNCH(launch_norm_to_f16(m->pf_hid, n, H, L.attn_norm, c.rms_eps, m->pf_xh,
                                      m->pf_rs, st),
                   "norm_to_f16");
        {
            GemmSegs gs{};
            const hyq_weight *ws[3] = {L.q, L.k, L.v};
            float *ys[3] = {m->pf_q, m->pf_k, m->pf_v};
            for (int i = 0; i < 3; ++i) {
                gs.s[i].w = ws[i]->view;
                gs.s[i].y = ys[i];
                gs.s[i].rows = (int)ws[i]->rows;
            }
            gs.nseg = 3;
            HYQ_LAUNCH(launch_gemm_f16_segs(L.q->dtype, gs, H, m->pf_xh, m->pf_rs, n, st),
                       "gemm_qkv");
        }
        HYQ_LAUNCH(launch_rope_norm_kv_rows(m->pf_q, m->pf_k, m->pf_v, L.q_norm, L.k_norm,
                                            m->freq, pos, n, c.heads, c.kv_heads, c.head_dim,
                                            c.rms_eps, m->kcache(l), m->vcache(l), st,
                                            m->arch == HYQ_ARCH_HYV3),
                   "rope_norm_kv_rows");
        if (merge_rows_lds(c.heads, prefill_attention_splits((int)m->context)) <= 64 * 1024) {
            // attention with its rows merged straight into the GEMM's f16 operand
            HYQ_LAUNCH(launch_attention_rows_f16(m->pf_q, m->kcache(l), m->vcache(l), pos, n,
                                                 (int)m->context, c.heads, c.kv_heads,
                                                 m->pf_part, nullptr, m->pf_xh, m->pf_rs, st),
                       "attention_rows");
        } else {
            HYQ_LAUNCH(launch_attention_rows(m->pf_q, m->kcache(l), m->vcache(l), pos, n,
                                             (int)m->context, c.heads, c.kv_heads, m->pf_part,
                                             m->pf_att, st),
                       "attention_rows");
            HYQ_LAUNCH(launch_to_f16(m->pf_att, n, QL, m->pf_xh, m->pf_rs, st), "to_f16");
        }
        HYQ_LAUNCH(launch_gemm_f16(L.o->dtype, L.o->view, QL, m->pf_xh, m->pf_rs, n, m->pf_hid,
                                   m->pf_hid, st, m->pf_kpart, m->pf_kpart_floats),
                   "gemm_attn_output");
        if (L.moe) {
            // Moe::forward at batch n (src/model.rs:598-601) and the add (:602)
            HYQ_LAUNCH(launch_rms_rows(m->pf_hid, L.ffn_norm, n, H, c.rms_eps, m->pf_xn, st),
                       "rms_rows");
            int rc = moe_ffn_rows(st, *L.moe, m->pf_xn, n, m->pf_moe, m->pf_hid, m->pf_hid);
            if (rc) return rc;
        } else {
        HYQ_LAUNCH(launch_norm_to_f16(m->pf_hid, n, H, L.ffn_norm, c.rms_eps, m->pf_xh,
                                      m->pf_rs, st),
                   "norm_to_f16");
        HYQ_LAUNCH(launch_gate_up_f16(L.gate->dtype, L.gate->view, L.up->view, H, m->pf_xh,
                                      m->pf_rs, n, m->pf_h, st),
                   "gemm_gate_up");
        HYQ_LAUNCH(launch_to_f16(m->pf_h, n, F, m->pf_xh, m->pf_rs, st), "to_f16");
        HYQ_LAUNCH(launch_gemm_f16(L.down->dtype, L.down->view, F, m->pf_xh, m->pf_rs, n,
                                   m->pf_hid, m->pf_hid, st, m->pf_kpart, m->pf_kpart_floats),
                   "gemm_down");
        }
        if (trace)
            HYQ_HIP(hipMemcpyAsync(m->trace + (size_t)(l + 1) * rows, m->pf_hid, rows * 4,
                                   hipMemcpyDeviceToDevice, st),
                    "trace");
    }
    if (int rc = lm_head(m, m->pf_hid + (size_t)(n - 1) * H, nullptr, 0, st, m->ctx->q8t()))
        return rc;
    HYQ_LAUNCH(launch_argmax(m->logits, c.vocab, m->argmax_scratch,
                             (int *)(m->argmax_scratch + 64), m->token, m->state, nullptr, st),
               "argmax");
    return HYQ_OK;
}

int ready(hyq_dense *m)
{
    if (m->poisoned) return fail(HYQ_EINVAL, "session was invalidated by a failed forward");
    for (size_t l = 0; l < m->layers.size(); ++l) {
        const hyq_dense::Layer &L = m->layers[l];
        if (!L.q) return fail(HYQ_EINVAL, "dense: layer %zu has no weights", l);
        if (!L.gate && !L.moe) return fail(HYQ_EINVAL, "dense: layer %zu has no FFN", l);
    }
    if (!m->embedding || !m->output) return fail(HYQ_EINVAL, "dense: output weights not set");
    return HYQ_OK;
}

int write_state(hyq_dense *m, int32_t token, int step, int cap)
{
    StepState s{(int)m->pos_host, step, cap, 0};
    HYQ_HIP(hipMemcpyAsync(m->state, &s, sizeof s, hipMemcpyHostToDevice, m->ctx->stream),
            "hipMemcpy(state)");
    HYQ_HIP(hipMemcpyAsync(m->token, &token, sizeof token, hipMemcpyHostToDevice,
                           m->ctx->stream),
            "hipMemcpy(token)");
    return HYQ_OK;
}

// After the stream has drained: the argmax's non-finite flag of the steps
// since the last write_state. forward_into rejects non-finite logits
// (src/model.rs:540-543, :609-612) and the failed forward poisons the session.
int check_finite(hyq_dense *m)
{
    StepState s{};
    HYQ_HIP(hipMemcpy(&s, m->state, sizeof s, hipMemcpyDeviceToHost), "hipMemcpy(state)");
    if (s.nonfinite) {
        m->poisoned = true;
        return fail(HYQ_EINVAL, "model produced non-finite logits; check model format and weights");
    }
    return HYQ_OK;
}

} // namespace

extern "C" {

int hyq_dense_create(hyq_ctx *ctx, const hyq_dense_config *cfg, size_t context, hyq_dense **out)
{
    int rc = check_ctx(ctx, "dense_create");
    if (rc) return rc;
    if (!cfg || !out) return fail(HYQ_EINVAL, "dense_create: null argument");
    const hyq_dense_config &c = *cfg;
    if (c.layers <= 0 || c.layers > 1024 || c.hidden <= 0 || c.vocab <= 0 || c.ffn <= 0)
        return fail(HYQ_EINVAL, "invalid model dimensions");
    if (c.heads <= 0 || c.kv_heads <= 0 || c.heads % c.kv_heads ||
        c.heads / c.kv_heads > ATT_MAX_REP)
        return fail(HYQ_EINVAL, "invalid grouped-query head counts");
    if (c.head_dim != 128) return fail(HYQ_EINVAL, "dense: head_dim %d (128 supported)", c.head_dim);
    if (c.hidden % 256 || c.ffn % 256 || (c.heads * c.head_dim) % 256)
        return fail(HYQ_EINVAL, "dense: widths must be multiples of 256");
    if (!(c.rope_base > 0.f) || !(c.rms_eps > 0.f))
        return fail(HYQ_EINVAL, "invalid context, RoPE, or RMS settings");
    if (context == 0 || context > 65536) return fail(HYQ_EINVAL, "dense: context %zu", context);
    DeviceGuard g(ctx->device);

    auto m = std::make_unique<hyq_dense>();
    m->ctx = ctx;
    m->cfg = c;
    m->context = context;
    m->layers.resize((size_t)c.layers);
    const size_t H = (size_t)c.hidden, F = (size_t)c.ffn, D = (size_t)c.head_dim;
    const size_t QL = (size_t)c.heads * D, KV = (size_t)c.kv_heads * D, V = (size_t)c.vocab;
    // one arena: norms (per layer 2*H + 2*D, plus H), freq, activations, scratch
    size_t off = 0;
    auto take = [&](size_t floats) {
        size_t o = off;
        off += align_up(floats * 4, 256);
        return o;
    };
    const size_t o_norms = take((size_t)c.layers * (2 * H + 2 * D) + H);
    const size_t o_freq = take(D / 2);
    const size_t o_hidden = take(H), o_q = take(QL), o_k = take(KV), o_v = take(KV);
    const size_t o_g = take(F), o_logits = take(V);
    const size_t o_att = take((size_t)attention_splits((int)context) * c.heads * PART_STRIDE);
    const size_t o_att_out = take(QL);
    const size_t o_parts = take((size_t)GEMV_MAX_PARTS * H);
    const size_t o_arg = take(128), o_tok = take(4), o_state = take(4);
    const size_t ng = (H + 255) / 256;
    const size_t o_oq = take((H + 3) / 4), o_os = take(ng), o_o16 = take(16 * ng);
    const size_t o_o32 = take(8 * ng), o_o256 = take(ng);
    rc = m->mem.alloc(ctx->device, off);
    if (rc) return rc;
    uint8_t *base = (uint8_t *)m->mem.ptr;
    float *norms = (float *)(base + o_norms);
    for (int l = 0; l < c.layers; ++l) {
        float *p = norms + (size_t)l * (2 * H + 2 * D);
        m->layers[l].attn_norm = p;
        m->layers[l].ffn_norm = p + H;
        m->layers[l].q_norm = p + 2 * H;
        m->layers[l].k_norm = p + 2 * H + D;
    }
    m->output_norm = norms + (size_t)c.layers * (2 * H + 2 * D);
    m->freq = (float *)(base + o_freq);
    m->hidden = (float *)(base + o_hidden);
    m->qb = (float *)(base + o_q);
    m->kb = (float *)(base + o_k);
    m->vb = (float *)(base + o_v);
    m->gb = (float *)(base + o_g);
    m->logits = (float *)(base + o_logits);
    m->att_scratch = (float *)(base + o_att);
    m->att_out = (float *)(base + o_att_out);
    m->parts = (float *)(base + o_parts);
    m->down_ks = down_kslices((int)(F / 256));
    m->argmax_scratch = (float *)(base + o_arg);
    m->token = (int32_t *)(base + o_tok);
    m->state = (StepState *)(base + o_state);
    m->out_q8.q = (int8_t *)(base + o_oq);
    m->out_q8.s = (float *)(base + o_os);
    m->out_q8.sum16 = (int32_t *)(base + o_o16);
    m->out_q8.sum32 = (int32_t *)(base + o_o32);
    m->out_q8.sum256 = (int32_t *)(base + o_o256);
    m->out_q8.n = H;
    // rope_frequencies (src/model.rs:263-269): base^(-2j/head_dim) in f32
    std::vector<float> freq(D / 2);
    for (size_t j = 0; j < D / 2; ++j)
        freq[j] = std::pow(c.rope_base, -2.0f * (float)j / (float)D);
    HYQ_HIP(hipMemcpy(m->freq, freq.data(), freq.size() * 4, hipMemcpyHostToDevice),
            "hipMemcpy(freq)");
    rc = m->kv.alloc(ctx->device, (size_t)c.layers * 2 * context * KV * 4);
    if (rc) return rc;
    HYQ_HIP(hipMemset(m->kv.ptr, 0, m->kv.bytes), "hipMemset(kv)");
    if ((rc = write_state(m.get(), 0, 0, 0))) return rc;
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    *out = m.release();
    return HYQ_OK;
}

void hyq_dense_destroy(hyq_dense *m)
{
    if (!m) return;
    DeviceGuard g(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    delete m;
}

static int check_weight(const hyq_dense *m, const hyq_weight *w, size_t cols, size_t rows,
                        const char *name)
{
    if (!w) return fail(HYQ_EINVAL, "dense: null %s weight", name);
    if (w->device != m->ctx->device) return fail(HYQ_EINVAL, "dense: %s on another device", name);
    if (w->rank != 2 || w->cols != cols || w->rows != rows)
        return fail(HYQ_EINVAL, "%s: expected GGUF shape [%zu, %zu], got [%zu, %zu]", name, cols,
                    rows, w->cols, w->rows);
    if (!int8_ok(w)) return fail(HYQ_EDTYPE, "%s: dtype %d has no int8 path", name, w->dtype);
    return HYQ_OK;
}

int hyq_dense_set_layer(hyq_dense *m, int layer, const hyq_weight *q, const hyq_weight *k,
                        const hyq_weight *v, const hyq_weight *o, const hyq_weight *gate,
                        const hyq_weight *up, const hyq_weight *down, const float *attn_norm,
                        const float *ffn_norm, const float *q_norm, const float *k_norm)
{
    if (!m) return fail(HYQ_EINVAL, "dense_set_layer: null decoder");
    const hyq_dense_config &c = m->cfg;
    if (layer < 0 || layer >= c.layers) return fail(HYQ_EINVAL, "dense: layer %d", layer);
    const size_t H = c.hidden, F = c.ffn, QL = (size_t)c.heads * c.head_dim,
                 KV = (size_t)c.kv_heads * c.head_dim, D = c.head_dim;
    int rc = check_weight(m, q, H, QL, "attn_q");
    if (!rc) rc = check_weight(m, k, H, KV, "attn_k");
    if (!rc) rc = check_weight(m, v, H, KV, "attn_v");
    if (!rc) rc = check_weight(m, o, QL, H, "attn_output");
    // no dense FFN: the layer's FFN is an MoE (hyq_dense_set_moe)
    const bool dense_ffn = gate || up || down;
    if (dense_ffn) {
        if (!rc) rc = check_weight(m, gate, H, F, "ffn_gate");
        if (!rc) rc = check_weight(m, up, H, F, "ffn_up");
        if (!rc) rc = check_weight(m, down, F, H, "ffn_down");
    }
    if (rc) return rc;
    if (!(q->dtype == k->dtype && k->dtype == v->dtype))
        return fail(HYQ_EDTYPE, "dense: q/k/v formats differ");
    if (dense_ffn && gate->dtype != up->dtype)
        return fail(HYQ_EDTYPE, "dense: gate/up formats differ");
    if (!attn_norm || !ffn_norm || !q_norm || !k_norm)
        return fail(HYQ_EINVAL, "dense: null norm vector");
    for (const float *vec : {attn_norm, ffn_norm})
        for (size_t i = 0; i < H; ++i)
            if (!std::isfinite(vec[i])) return fail(HYQ_EINVAL, "non-finite normalization tensor");
    DeviceGuard g(m->ctx->device);
    hyq_dense::Layer &L = m->layers[layer];
    L.q = q;
    L.k = k;
    L.v = v;
    L.o = o;
    L.gate = gate;
    L.up = up;
    L.down = down;
    if (dense_ffn) {
        L.moe.reset();
        L.moe_bias.reset();
    }
    m->pf_mem.reset(); // the prefill buffers depend on the layers' FFNs
    m->pf_cap = 0;
    HYQ_HIP(hipMemcpy(L.attn_norm, attn_norm, H * 4, hipMemcpyHostToDevice), "hipMemcpy");
    HYQ_HIP(hipMemcpy(L.ffn_norm, ffn_norm, H * 4, hipMemcpyHostToDevice), "hipMemcpy");
    HYQ_HIP(hipMemcpy(L.q_norm, q_norm, D * 4, hipMemcpyHostToDevice), "hipMemcpy");
    HYQ_HIP(hipMemcpy(L.k_norm, k_norm, D * 4, hipMemcpyHostToDevice), "hipMemcpy");
    m->drop_graph();
    return HYQ_OK;
}

int hyq_dense_set_architecture(hyq_dense *m, int arch)
{
    if (!m) return fail(HYQ_EINVAL, "dense_set_architecture: null decoder");
    if (arch != HYQ_ARCH_DENSE && arch != HYQ_ARCH_HYV3)
        return fail(HYQ_EINVAL, "unsupported model architecture %d", arch);
    m->arch = arch;
    m->drop_graph();
    return HYQ_OK;
}

int hyq_dense_set_moe(hyq_dense *m, int layer, const hyq_moe_config *mc,
                      const hyq_weight *router, const float *bias, const hyq_weight *gate,
                      const hyq_weight *up, const hyq_weight *down, const hyq_weight *shared_gate,
                      const hyq_weight *shared_up, const hyq_weight *shared_down)
{
    if (!m || !mc) return fail(HYQ_EINVAL, "dense_set_moe: null argument");
    const hyq_dense_config &c = m->cfg;
    if (layer < 0 || layer >= c.layers) return fail(HYQ_EINVAL, "dense: layer %d", layer);
    if (m->has_moe && (mc->experts != m->moe_cfg.experts || mc->used != m->moe_cfg.used ||
                       mc->mid != m->moe_cfg.mid || mc->shared_mid != m->moe_cfg.shared_mid))
        return fail(HYQ_EINVAL, "dense: MoE layers must share one expert shape");
    if (!bias) return fail(HYQ_EINVAL, "dense: null selection bias");
    for (int e = 0; e < mc->experts; ++e)
        if (!std::isfinite(bias[e])) return fail(HYQ_EINVAL, "non-finite normalization/router tensor");
    DeviceGuard g(m->ctx->device);
    auto bias_d = std::make_unique<DeviceBuffer>();
    int rc = mc->experts > 0 ? bias_d->alloc(m->ctx->device, (size_t)mc->experts * 4)
                             : fail(HYQ_EINVAL, "invalid expert dimensions");
    if (rc) return rc;
    auto f = std::make_unique<MoeFfn>();
    f->router = router;
    f->bias_d = (const float *)bias_d->ptr;
    f->gate = gate;
    f->up = up;
    f->down = down;
    f->sgate = shared_gate;
    f->sup = shared_up;
    f->sdown = shared_down;
    f->hidden = c.hidden;
    f->experts = mc->experts;
    f->used = mc->used;
    f->mid = mc->mid;
    f->smid = mc->shared_mid;
    f->normalize = mc->normalize;
    f->scale = mc->scale;
    if ((rc = moe_ffn_check(*f, m->ctx->device))) return rc;
    HYQ_HIP(hipMemcpy(bias_d->ptr, bias, (size_t)mc->experts * 4, hipMemcpyHostToDevice),
            "hipMemcpy(bias)");
    if (!m->moe_mem) {
        // the batch-1 temporaries: normalized row, its Q8, the FFN's buffers
        const size_t H = c.hidden, ng = H / 256;
        size_t off = 0;
        auto take = [&](size_t bytes) {
            const size_t o = off;
            off += align_up(bytes, 256);
            return o;
        };
        const size_t o_xn = take(H * 4), o_q = take(H), o_s = take(ng * 4);
        const size_t o_16 = take(H / 4), o_32 = take(H / 8), o_256 = take(ng * 4);
        const size_t o_row = take(moe_row_bytes(*f));
        auto mem = std::make_unique<DeviceBuffer>();
        if ((rc = mem->alloc(m->ctx->device, off))) return rc;
        uint8_t *b = (uint8_t *)mem->ptr;
        m->moe_xn = (float *)(b + o_xn);
        m->moe_q8.q = (int8_t *)(b + o_q);
        m->moe_q8.s = (float *)(b + o_s);
        m->moe_q8.sum16 = (int32_t *)(b + o_16);
        m->moe_q8.sum32 = (int32_t *)(b + o_32);
        m->moe_q8.sum256 = (int32_t *)(b + o_256);
        m->moe_q8.n = H;
        m->moe_row = moe_row_carve(*f, b + o_row);
        m->moe_mem = std::move(mem);
    }
    hyq_dense::Layer &L = m->layers[layer];
    L.gate = L.up = L.down = nullptr;
    L.moe = std::move(f);
    L.moe_bias = std::move(bias_d);
    m->moe_cfg = *mc;
    m->has_moe = true;
    m->pf_mem.reset();
    m->pf_cap = 0;
    m->drop_graph();
    return HYQ_OK;
}

int hyq_dense_set_output(hyq_dense *m, const hyq_weight *embedding, const hyq_weight *output,
                         const float *output_norm)
{
    if (!m) return fail(HYQ_EINVAL, "dense_set_output: null decoder");
    const hyq_dense_config &c = m->cfg;
    int rc = check_weight(m, output, c.hidden, c.vocab, "output");
    if (rc) return rc;
    if (!embedding || embedding->rank != 2 || embedding->cols != (size_t)c.hidden ||
        embedding->rows != (size_t)c.vocab)
        return fail(HYQ_EINVAL, "token_embd: shape mismatch");
    if (!output_norm) return fail(HYQ_EINVAL, "dense: null output norm");
    DeviceGuard g(m->ctx->device);
    m->embedding = embedding;
    m->output = output;
    HYQ_HIP(hipMemcpy(m->output_norm, output_norm, (size_t)c.hidden * 4, hipMemcpyHostToDevice),
            "hipMemcpy");
    m->drop_graph();
    return HYQ_OK;
}

int hyq_dense_load_kv(hyq_dense *m, int layer, size_t positions, const float *keys,
                      const float *values)
{
    if (!m || !keys || !values) return fail(HYQ_EINVAL, "dense_load_kv: null argument");
    if (layer < 0 || layer >= m->cfg.layers) return fail(HYQ_EINVAL, "dense: layer %d", layer);
    if (positions > m->context) return fail(HYQ_EINVAL, "context limit exceeded");
    DeviceGuard g(m->ctx->device);
    const size_t bytes = positions * m->kvw() * 4;
    HYQ_HIP(hipMemcpy(m->kcache(layer), keys, bytes, hipMemcpyHostToDevice), "hipMemcpy(k)");
    HYQ_HIP(hipMemcpy(m->vcache(layer), values, bytes, hipMemcpyHostToDevice), "hipMemcpy(v)");
    return HYQ_OK;
}

int hyq_dense_set_position(hyq_dense *m, size_t position)
{
    if (!m) return fail(HYQ_EINVAL, "dense_set_position: null decoder");
    if (position > m->context) return fail(HYQ_EINVAL, "context limit exceeded");
    m->pos_host = position;
    m->poisoned = false;
    return HYQ_OK;
}

int hyq_dense_get_position(hyq_dense *m, size_t *position)
{
    if (!m || !position) return fail(HYQ_EINVAL, "dense_get_position: null argument");
    *position = m->pos_host;
    return HYQ_OK;
}

int hyq_dense_forward(hyq_dense *m, int32_t token, float *logits, int32_t *next)
{
    if (!m) return fail(HYQ_EINVAL, "dense_forward: null decoder");
    int rc = ready(m);
    if (rc) return rc;
    if (token < 0 || token >= m->cfg.vocab) return fail(HYQ_EINVAL, "input token outside vocabulary");
    if (m->pos_host + 1 > m->context) return fail(HYQ_EINVAL, "context limit exceeded");
    DeviceGuard g(m->ctx->device);
    if ((rc = write_state(m, token, 0, 0))) return rc;
    if ((rc = enqueue_step(m, true))) return rc;
    if (logits)
        HYQ_HIP(hipMemcpyAsync(logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost,
                               m->ctx->stream),
                "hipMemcpy(logits)");
    int32_t nt = 0;
    HYQ_HIP(hipMemcpyAsync(&nt, m->token, 4, hipMemcpyDeviceToHost, m->ctx->stream),
            "hipMemcpy(token)");
    HYQ_HIP(hipStreamSynchronize(m->ctx->stream), "hipStreamSynchronize");
    if ((rc = check_finite(m))) return rc;
    m->pos_host += 1;
    if (next) *next = nt;
    return HYQ_OK;
}

int hyq_dense_prefill(hyq_dense *m, const int32_t *tokens, size_t n, float *logits,
                      int32_t *next)
{
    if (!m) return fail(HYQ_EINVAL, "dense_prefill: null decoder");
    int rc = ready(m);
    if (rc) return rc;
    if (n == 0 || !tokens) return fail(HYQ_EINVAL, "prompt must contain at least one token");
    if (n > m->context - m->pos_host) return fail(HYQ_EINVAL, "prompt exceeds context limit");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab)
            return fail(HYQ_EINVAL, "input token outside vocabulary");
    // the reference's chunks of PREFILL_CHUNK tokens take the batch-1 arm
    // only when one token is left over
    const size_t batched = n % PREFILL_CHUNK == 1 ? n - 1 : n;
    if (batched) // the batched products' f16 operands
        for (const hyq_dense::Layer &L : m->layers) {
            for (const hyq_weight *w : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down})
                if (w && (rc = check_f16_range(w, "prefill"))) return rc;
            if (L.moe)
                for (const hyq_weight *w : {L.moe->gate, L.moe->up, L.moe->down, L.moe->sgate,
                                            L.moe->sup, L.moe->sdown})
                    if ((rc = check_f16_range(w, "prefill"))) return rc;
        }
    DeviceGuard g(m->ctx->device);
    hipStream_t st = m->ctx->stream;
    if (batched && (rc = prefill_buffers(m))) return rc;
    for (size_t s = 0; s < n;) {
        const size_t cn = s < batched ? std::min(m->pf_cap, batched - s) : 1;
        if ((rc = write_state(m, tokens[s], 0, 0))) return rc;
        if (s < batched) {
            HYQ_HIP(hipMemcpyAsync(m->pf_tok, tokens + s, cn * 4, hipMemcpyHostToDevice, st),
                    "hipMemcpy(tokens)");
            if ((rc = enqueue_prefill_chunk(m, (int)cn))) return rc;
        } else if ((rc = enqueue_step(m, true))) {
            return rc;
        }
        // the host-side state and token words are rewritten by the next pass
        HYQ_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
        if ((rc = check_finite(m))) return rc;
        m->pos_host += cn;
        s += cn;
    }
    if (logits)
        HYQ_HIP(hipMemcpyAsync(logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost,
                               st),
                "hipMemcpy(logits)");
    int32_t nt = 0;
    HYQ_HIP(hipMemcpyAsync(&nt, m->token, 4, hipMemcpyDeviceToHost, st), "hipMemcpy(token)");
    HYQ_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
    if (next) *next = nt;
    return HYQ_OK;
}

int hyq_dense_set_trace(hyq_dense *m, float *trace_d, size_t floats)
{
    if (!m) return fail(HYQ_EINVAL, "dense_set_trace: null decoder");
    const size_t need = (size_t)(m->cfg.layers + 1) * (size_t)m->cfg.hidden;
    if (trace_d && floats < need)
        return fail(HYQ_EINVAL, "dense_set_trace: %zu floats < %zu", floats, need);
    m->trace = trace_d;
    m->trace_floats = trace_d ? floats : 0;
    return HYQ_OK;
}

int hyq_dense_set_prefill_rows(hyq_dense *m, size_t rows)
{
    if (!m) return fail(HYQ_EINVAL, "dense_set_prefill_rows: null decoder");
    if (rows == 0 || rows > 65536) return fail(HYQ_EINVAL, "dense: prefill rows %zu", rows);
    m->pf_rows = rows;
    return HYQ_OK;
}

int hyq_dense_read_kv(hyq_dense *m, int layer, size_t positions, float *keys, float *values)
{
    if (!m || !keys || !values) return fail(HYQ_EINVAL, "dense_read_kv: null argument");
    if (layer < 0 || layer >= m->cfg.layers) return fail(HYQ_EINVAL, "dense: layer %d", layer);
    if (positions > m->context) return fail(HYQ_EINVAL, "context limit exceeded");
    DeviceGuard g(m->ctx->device);
    HYQ_HIP(hipStreamSynchronize(m->ctx->stream), "hipStreamSynchronize");
    const size_t bytes = positions * m->kvw() * 4;
    HYQ_HIP(hipMemcpy(keys, m->kcache(layer), bytes, hipMemcpyDeviceToHost), "hipMemcpy(k)");
    HYQ_HIP(hipMemcpy(values, m->vcache(layer), bytes, hipMemcpyDeviceToHost), "hipMemcpy(v)");
    return HYQ_OK;
}

int hyq_dense_generate(hyq_dense *m, int32_t token, size_t steps, int use_graph, int32_t *tokens)
{
    if (!m) return fail(HYQ_EINVAL, "dense_generate: null decoder");
    int rc = ready(m);
    if (rc) return rc;
    if (token < 0 || token >= m->cfg.vocab) return fail(HYQ_EINVAL, "input token outside vocabulary");
    if (steps == 0) return HYQ_OK;
    if (!tokens) return fail(HYQ_EINVAL, "dense_generate: null output");
    if (m->pos_host + steps > m->context) return fail(HYQ_EINVAL, "context limit exceeded");
    DeviceGuard g(m->ctx->device);
    hipStream_t st = m->ctx->stream;
    if (m->history_cap < steps) {
        m->drop_graph(); // the graph bakes the history address in
        m->history_mem.reset();
        m->history = nullptr;
        m->history_cap = 0;
        auto buf = std::make_unique<DeviceBuffer>();
        if ((rc = buf->alloc(m->ctx->device, steps * 4))) return rc;
        m->history_mem = std::move(buf);
        m->history = (int32_t *)m->history_mem->ptr;
        m->history_cap = steps;
    }
    if ((rc = write_state(m, token, 0, (int)steps))) return rc;
    // the first step's input row; every step's argmax then writes the next
    HYQ_LAUNCH(launch_embed_row(m->embedding->dtype, m->embedding->view, m->cfg.hidden, m->token,
                                m->hidden, st),
               "embed_row");
    if (use_graph) {
        if (!m->exec) {
            HYQ_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
            HYQ_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "BeginCapture");
            rc = enqueue_step(m, false, false);
            hipGraph_t graph = nullptr;
            hipError_t e = hipStreamEndCapture(st, &graph);
            if (rc) {
                if (graph) (void)hipGraphDestroy(graph);
                return rc;
            }
            if (e != hipSuccess) return hip_fail(e, "EndCapture");
            m->graph = graph;
            HYQ_HIP(hipGraphInstantiate(&m->exec, m->graph, nullptr, nullptr, 0),
                    "hipGraphInstantiate");
        }
        for (size_t i = 0; i < steps; ++i) HYQ_HIP(hipGraphLaunch(m->exec, st), "hipGraphLaunch");
    } else {
        for (size_t i = 0; i < steps; ++i)
            if ((rc = enqueue_step(m, false, false))) return rc;
    }
    HYQ_HIP(hipMemcpyAsync(tokens, m->history, steps * 4, hipMemcpyDeviceToHost, st),
            "hipMemcpy(tokens)");
    HYQ_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
    if ((rc = check_finite(m))) return rc;
    m->pos_host += steps;
    return HYQ_OK;
}

} // extern "C"
