/*
 * CPU oracle, part 2: the batch-1 decode step of the dense Hunyuan graph
 * (src/model.rs:374-546) around the quantized matmuls.
 *
 * TEST INFRASTRUCTURE ONLY (checker and CPU baseline). Two arms:
 *   int8_path = 0  the x86 path: f32 activations through Weight::matmul /
 *                  matmul_gate_up_silu (src/model.rs:418-422, 473-474, 503,
 *                  535-537). This is the CPU baseline of the decode step.
 *   int8_path = 1  the int8 path the reference takes with SDOT
 *                  (src/model.rs:403-416, 461-471, 487-501, 522-531): every
 *                  matmul input is Q8-quantized and each output is the exact
 *                  value of the integer formula rounded once to f32. The
 *                  int8 path exists only in the aarch64 build, so its
 *                  RMSNorms take that arm's operation order (x * (w *
 *                  scale), src/model.rs:791-822, 837-865).
 * The rest of the glue follows rope_with_cache (src/model.rs:874-917),
 * attention_into (:949-1035), add (:1043-1077) and, with int8_path = 0, the
 * x86 arms of rms_norm_into (:824-829) and rms_norm (:866-869); the
 * hyqo_q8_tap of hyqo_layer_step_tap records and replaces the int8 path's
 * quantized inputs stage by stage. hyqo_prefill_chunk is the batch > 1
 * arm of forward_into (src/model.rs:549-616): f32 activations through the
 * batched Weight::matmul (src/quant.rs:272-343), and the last row's logits
 * through the batch-1 matmul of the chosen arm.
 */
#include "hyq_oracle.h"
#include "hyq_oracle_step.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static size_t rb_of(int dtype, size_t cols)
{
    return cols / (size_t)hyqo_block_len(dtype) * (size_t)hyqo_block_bytes(dtype);
}

/* One normalized value. The aarch64 arm multiplies x by (w * scale) over
 * whole 16-value steps (src/model.rs:791-815, :837-860) and by scale, then
 * w, over the tail (:816-822, :861-864); the x86 arm always x * scale * w
 * (:824-829, :866-869). */
static float rms_value(float x, float w, float scale, size_t i, size_t n, int aarch64)
{
    if (aarch64 && i < n / 16 * 16) return x * (w * scale);
    return x * scale * w;
}

void hyqo_rms_norm_into(const float *x, const float *w, size_t n, float eps, float *out,
                        int aarch64)
{
    float variance = hyqo_dot(x, x, n) / (float)n;
    float scale = 1.0f / sqrtf(variance + eps);
    for (size_t i = 0; i < n; ++i) out[i] = rms_value(x[i], w[i], scale, i, n, aarch64);
}

void hyqo_rms_norm_rows(float *x, const float *w, size_t total, size_t wlen, float eps,
                        int aarch64)
{
    for (size_t r = 0; r + wlen <= total; r += wlen) {
        float *row = x + r;
        float variance = hyqo_dot(row, row, wlen) / (float)wlen;
        float scale = 1.0f / sqrtf(variance + eps);
        for (size_t i = 0; i < wlen; ++i)
            row[i] = rms_value(row[i], w[i], scale, i, wlen, aarch64);
    }
}

void hyqo_rope_tables(size_t head_dim, float base, size_t pos, float *cos_s, float *sin_s)
{
    size_t half = head_dim / 2;
    float p = (float)pos;
    for (size_t j = 0; j < half; ++j) {
        float freq = powf(base, -2.0f * (float)j / (float)head_dim); /* src/model.rs:263-269 */
        float a = p * freq;
        sin_s[j] = sinf(a);
        cos_s[j] = cosf(a);
    }
}

void hyqo_rope(float *values, size_t heads, size_t dim, const float *cos_s, const float *sin_s)
{
    size_t half = dim / 2;
    for (size_t h = 0; h < heads; ++h) {
        float *head = values + h * dim;
        for (size_t j = 0; j < half; ++j) {
            float a = head[j], b = head[j + half];
            head[j] = a * cos_s[j] - b * sin_s[j];
            head[j + half] = a * sin_s[j] + b * cos_s[j];
        }
    }
}

void hyqo_attention(const float *q, const float *keys, const float *values, size_t heads,
                    size_t kv_heads, size_t dim, size_t visible, float *out)
{
    size_t kv_width = kv_heads * dim;
    size_t repeats = heads / kv_heads;
    float scale = 1.0f / sqrtf((float)dim);
    memset(out, 0, sizeof(float) * heads * dim);
    /* heads in parallel, as the reference does once past >= 64 (src/model.rs:1024-1034) */
    long nh = (long)heads;
#pragma omp parallel for schedule(static) if (visible >= 64)
    for (long hl = 0; hl < nh; ++hl) {
        size_t h = (size_t)hl;
        float *scores = (float *)malloc(sizeof(float) * (visible ? visible : 1));
        size_t kvh = h / repeats;
        const float *query = q + h * dim;
        for (size_t p = 0; p < visible; ++p)
            scores[p] = hyqo_dot(query, keys + p * kv_width + kvh * dim, dim) * scale;
        float max = -INFINITY;
        for (size_t p = 0; p < visible; ++p) max = fmaxf(max, scores[p]);
        float sum = 0.f;
        for (size_t p = 0; p < visible; ++p) {
            scores[p] = expf(scores[p] - max);
            sum += scores[p];
        }
        float inv = 1.0f / sum;
        float *o = out + h * dim;
        for (size_t p = 0; p < visible; ++p) {
            float pr = scores[p] * inv;
            const float *v = values + p * kv_width + kvh * dim;
            for (size_t i = 0; i < dim; ++i) o[i] += pr * v[i];
        }
        free(scores);
    }
}

int hyqo_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* One int8-path GEMV: y = round_f32(exact integer formula) (see hyq_oracle.h),
 * its input being quantized stage `stage` of the tap (when set). */
static void gemv_int8(int dtype, const uint8_t *w, size_t rows, size_t cols, const float *x,
                      float *y, const hyqo_q8_tap *tap, int stage)
{
    int8_t *q = (int8_t *)malloc(cols);
    float *s = (float *)malloc(sizeof(float) * (cols / 256 + 1));
    double *yd = (double *)malloc(sizeof(double) * rows);
    hyqo_q8_quantize(x, cols, q, s);
    if (tap) {
        size_t o = (size_t)stage * tap->stride, os = o / 256;
        if (tap->own_x) memcpy(tap->own_x + o, x, sizeof(float) * cols);
        if (tap->own_q) memcpy(tap->own_q + o, q, cols);
        if (tap->own_s) memcpy(tap->own_s + os, s, sizeof(float) * ((cols + 255) / 256));
        if (tap->use_q) memcpy(q, tap->use_q + o, cols);
        if (tap->use_s) memcpy(s, tap->use_s + os, sizeof(float) * ((cols + 255) / 256));
    }
    hyqo_gemv_q8_f64(dtype, w, rows, cols, q, s, yd, NULL);
    for (size_t r = 0; r < rows; ++r) y[r] = (float)yd[r];
    free(q);
    free(s);
    free(yd);
}

static void linear(const hyqo_model *m, int dtype, const uint8_t *w, size_t rows, size_t cols,
                   const float *x, float *y, int int8_path, int threads, const hyqo_q8_tap *tap,
                   int stage)
{
    if (int8_path)
        gemv_int8(dtype, w, rows, cols, x, y, tap, stage);
    else
        hyqo_matmul(dtype, w, rows, cols, x, 1, y, threads);
    (void)m;
}

/* DenseFfn::forward at batch 1 on the int8 path (src/model.rs:487-501):
 * silu(gate x) * (up x) from Q8 inputs, then down of the product's Q8 (tap
 * stages in_stage and down_stage). */
static void ffn_int8(int dtype_gu, int dtype_down, const uint8_t *gate, const uint8_t *up,
                     const uint8_t *down, size_t hidden, size_t mid, const float *x, float *out,
                     const hyqo_q8_tap *tap, int in_stage, int down_stage)
{
    float *g = (float *)malloc(sizeof(float) * mid);
    float *u = (float *)malloc(sizeof(float) * mid);
    gemv_int8(dtype_gu, gate, mid, hidden, x, g, tap, in_stage);
    gemv_int8(dtype_gu, up, mid, hidden, x, u, tap, in_stage);
    for (size_t i = 0; i < mid; ++i) {
        float v = g[i];
        g[i] = (v / (1.0f + expf(-v))) * u[i];
    }
    gemv_int8(dtype_down, down, hidden, mid, g, out, tap, down_stage);
    free(g);
    free(u);
}

/* DenseFfn::forward (src/model.rs:672-685) on f32 activations: batch 1
 * through matmul_gate_up_silu, batch n through two matmuls and silu(g) * u. */
static void ffn_f32(int dtype_gu, int dtype_down, const uint8_t *gate, const uint8_t *up,
                    const uint8_t *down, size_t hidden, size_t mid, const float *x, size_t n,
                    float *out, int threads)
{
    float *g = (float *)malloc(sizeof(float) * n * mid);
    if (n == 1) {
        hyqo_gate_up_silu(dtype_gu, gate, up, mid, hidden, x, g, threads);
    } else {
        float *u = (float *)malloc(sizeof(float) * n * mid);
        hyqo_matmul(dtype_gu, gate, mid, hidden, x, n, g, threads);
        hyqo_matmul(dtype_gu, up, mid, hidden, x, n, u, threads);
        for (size_t i = 0; i < n * mid; ++i) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        free(u);
    }
    hyqo_matmul(dtype_down, down, hidden, mid, g, n, out, threads);
    free(g);
}

static void moe_forward(const hyqo_moe *e, size_t hidden, const float *x, size_t n, float *out,
                        int int8_path, int threads, const hyqo_q8_tap *tap)
{
    size_t E = (size_t)e->experts, U = (size_t)e->used, mid = (size_t)e->mid;
    /* router.matmul (F32, src/model.rs:691) and route per token (:692-698);
     * assignments in token order per expert */
    float *logits = (float *)malloc(sizeof(float) * n * E);
    hyqo_matmul(0 /* F32 */, (const uint8_t *)e->router, E, hidden, x, n, logits, threads);
    int32_t *pt = (int32_t *)malloc(sizeof(int32_t) * n * U);
    int32_t *pe = (int32_t *)malloc(sizeof(int32_t) * n * U);
    float *pw = (float *)malloc(sizeof(float) * n * U);
    for (size_t t = 0; t < n; ++t) {
        hyqo_route(logits + t * E, e->bias, E, U, e->normalize, e->scale, pe + t * U, pw + t * U);
        for (size_t k = 0; k < U; ++k) pt[t * U + k] = (int32_t)t;
    }
    /* output = shared.forward(input, batch) (:699) */
    if (int8_path && n == 1)
        ffn_int8(e->dtype_shared, e->dtype_shared_down, e->sgate, e->sup, e->sdown, hidden,
                 (size_t)e->shared_mid, x, out, tap, HYQO_STAGE_FFN_IN, HYQO_STAGE_DOWN_IN);
    else
        ffn_f32(e->dtype_shared, e->dtype_shared_down, e->sgate, e->sup, e->sdown, hidden,
                (size_t)e->shared_mid, x, n, out, threads);
    /* experts in ascending order, out[t] += w * ffn (:700-722) */
    if (int8_path && n == 1) {
        size_t gb = mid * (size_t)hyqo_block_bytes(e->dtype_gate) * hidden /
                    (size_t)hyqo_block_len(e->dtype_gate);
        size_t db = hidden * (size_t)hyqo_block_bytes(e->dtype_down) * mid /
                    (size_t)hyqo_block_len(e->dtype_down);
        float *res = (float *)malloc(sizeof(float) * hidden);
        int visited = 0;
        for (size_t ex = 0; ex < E; ++ex)
            for (size_t k = 0; k < U; ++k) {
                if ((size_t)pe[k] != ex) continue;
                ffn_int8(e->dtype_gate, e->dtype_down, e->gate + ex * gb, e->up + ex * gb,
                         e->down + ex * db, hidden, mid, x, res, tap, HYQO_STAGE_FFN_IN,
                         HYQO_STAGE_EXPERT_DOWN_IN + visited++);
                for (size_t i = 0; i < hidden; ++i) out[i] += pw[k] * res[i];
            }
        free(res);
    } else {
        hyqo_moe_experts(e->dtype_gate, e->dtype_down, e->gate, e->up, e->down, E, hidden, mid,
                         x, n, pt, pe, pw, n * U, out, threads);
    }
    free(logits);
    free(pt);
    free(pe);
    free(pw);
}

void hyqo_moe_forward(const hyqo_moe *e, size_t hidden, const float *x, size_t n, float *out,
                      int int8_path, int threads)
{
    moe_forward(e, hidden, x, n, out, int8_path, threads, NULL);
}

void hyqo_moe_forward_tap(const hyqo_moe *e, size_t hidden, const float *x, float *out,
                          int threads, const hyqo_q8_tap *tap)
{
    moe_forward(e, hidden, x, 1, out, 1, threads, tap);
}

static int layer_step(const hyqo_model *m, int l, float *hidden, float *kc, float *vc,
                      size_t ctx, size_t pos, int int8_path, int threads, const hyqo_q8_tap *tap)
{
    size_t H = (size_t)m->hidden, D = (size_t)m->head_dim;
    size_t qlen = (size_t)m->heads * D, kvw = (size_t)m->kv_heads * D, F = (size_t)m->ffn;
    if (l < 0 || l >= m->layers || pos >= ctx) return -1;
    float *xn = (float *)malloc(sizeof(float) * H);
    float *q = (float *)malloc(sizeof(float) * qlen);
    float *k = (float *)malloc(sizeof(float) * kvw);
    float *v = (float *)malloc(sizeof(float) * kvw);
    float *att = (float *)malloc(sizeof(float) * qlen);
    float *proj = (float *)malloc(sizeof(float) * H);
    float *gate = (float *)malloc(sizeof(float) * F);
    float *up = (float *)malloc(sizeof(float) * F);
    float cos_s[512], sin_s[512];
    /* the step's RoPE tables at `pos` (src/model.rs:378-392) */
    hyqo_rope_tables(D, m->rope_base, pos, cos_s, sin_s);

    hyqo_rms_norm_into(hidden, m->attn_norm[l], H, m->eps, xn, int8_path);
    linear(m, m->dtype_linear, m->wq[l], qlen, H, xn, q, int8_path, threads, tap,
           HYQO_STAGE_ATTN_IN);
    linear(m, m->dtype_linear, m->wk[l], kvw, H, xn, k, int8_path, threads, tap,
           HYQO_STAGE_ATTN_IN);
    linear(m, m->dtype_linear, m->wv[l], kvw, H, xn, v, int8_path, threads, tap,
           HYQO_STAGE_ATTN_IN);
    /* per-head Q/K RMSNorm before RoPE (hy_v3) or after it (dense)
     * (src/model.rs:425-446) */
    if (m->arch == 1) {
        hyqo_rms_norm_rows(q, m->q_norm[l], qlen, D, m->eps, int8_path);
        hyqo_rms_norm_rows(k, m->k_norm[l], kvw, D, m->eps, int8_path);
    }
    hyqo_rope(q, (size_t)m->heads, D, cos_s, sin_s);
    hyqo_rope(k, (size_t)m->kv_heads, D, cos_s, sin_s);
    if (m->arch != 1) {
        hyqo_rms_norm_rows(q, m->q_norm[l], qlen, D, m->eps, int8_path);
        hyqo_rms_norm_rows(k, m->k_norm[l], kvw, D, m->eps, int8_path);
    }
    memcpy(kc + pos * kvw, k, sizeof(float) * kvw);
    memcpy(vc + pos * kvw, v, sizeof(float) * kvw);
    hyqo_attention(q, kc, vc, (size_t)m->heads, (size_t)m->kv_heads, D, pos + 1, att);
    linear(m, m->dtype_linear, m->wo[l], H, qlen, att, proj, int8_path, threads, tap,
           HYQO_STAGE_OUT_IN);
    for (size_t i = 0; i < H; ++i) hidden[i] += proj[i];
    hyqo_rms_norm_into(hidden, m->ffn_norm[l], H, m->eps, xn, int8_path);
    if (m->moe && m->moe[l]) {
        /* Ffn::Moe (src/model.rs:507-510) */
        moe_forward(m->moe[l], H, xn, 1, proj, int8_path, threads, tap);
    } else if (int8_path) {
        gemv_int8(m->dtype_linear, m->wgate[l], F, H, xn, gate, tap, HYQO_STAGE_FFN_IN);
        gemv_int8(m->dtype_linear, m->wup[l], F, H, xn, up, tap, HYQO_STAGE_FFN_IN);
        for (size_t i = 0; i < F; ++i) {
            float g = gate[i];
            float silu = g / (1.0f + expf(-g));
            gate[i] = silu * up[i];
        }
    } else {
        hyqo_gate_up_silu(m->dtype_linear, m->wgate[l], m->wup[l], F, H, xn, gate, threads);
    }
    if (!(m->moe && m->moe[l]))
        linear(m, m->dtype_down, m->wdown[l], H, F, gate, proj, int8_path, threads, tap,
               HYQO_STAGE_DOWN_IN);
    for (size_t i = 0; i < H; ++i) hidden[i] += proj[i];

    free(xn);
    free(q);
    free(k);
    free(v);
    free(att);
    free(proj);
    free(gate);
    free(up);
    return 0;
}

int hyqo_layer_step(const hyqo_model *m, int l, float *hidden, float *kc, float *vc, size_t ctx,
                    size_t pos, int int8_path, int threads)
{
    return layer_step(m, l, hidden, kc, vc, ctx, pos, int8_path, threads, NULL);
}

int hyqo_layer_step_tap(const hyqo_model *m, int l, float *hidden, float *kc, float *vc,
                        size_t ctx, size_t pos, int threads, const hyqo_q8_tap *tap)
{
    return layer_step(m, l, hidden, kc, vc, ctx, pos, 1, threads, tap);
}

static void output_logits(const hyqo_model *m, float *hidden, int int8_path, float *logits,
                          int threads, const hyqo_q8_tap *tap)
{
    size_t H = (size_t)m->hidden;
    /* rms_norm(hidden, output_norm), then the output matmul (src/model.rs:515-538) */
    hyqo_rms_norm_rows(hidden, m->output_norm, H, H, m->eps, int8_path);
    linear(m, m->dtype_embed, m->output ? m->output : m->embed, (size_t)m->vocab, H, hidden,
           logits, int8_path, threads, tap, HYQO_STAGE_ATTN_IN);
}

void hyqo_output_logits(const hyqo_model *m, float *hidden, int int8_path, float *logits,
                        int threads)
{
    output_logits(m, hidden, int8_path, logits, threads, NULL);
}

void hyqo_output_logits_tap(const hyqo_model *m, float *hidden, float *logits, int threads,
                            const hyqo_q8_tap *tap)
{
    output_logits(m, hidden, 1, logits, threads, tap);
}

int hyqo_decode_step(const hyqo_model *m, float *kcache, float *vcache, size_t ctx, size_t pos,
                     int token, int int8_path, float *logits, int threads)
{
    size_t H = (size_t)m->hidden, kvw = (size_t)m->kv_heads * m->head_dim;
    if (pos >= ctx || token < 0 || token >= m->vocab) return -1;
    float *hidden = (float *)malloc(sizeof(float) * H);
    /* embedding.row_into (src/model.rs:376) */
    size_t erb = rb_of(m->dtype_embed, H);
    hyqo_decode(m->dtype_embed, m->embed + (size_t)token * erb, erb, hidden, H);
    for (int l = 0; l < m->layers; ++l)
        hyqo_layer_step(m, l, hidden, kcache + (size_t)l * ctx * kvw,
                        vcache + (size_t)l * ctx * kvw, ctx, pos, int8_path, threads);
    hyqo_output_logits(m, hidden, int8_path, logits, threads);
    free(hidden);
    return 0;
}

int hyqo_prefill_layer(const hyqo_model *m, int l, float *hidden, float *kc, float *vc,
                       size_t ctx, size_t pos, size_t n, int threads)
{
    size_t H = (size_t)m->hidden, D = (size_t)m->head_dim;
    size_t qlen = (size_t)m->heads * D, kvw = (size_t)m->kv_heads * D, F = (size_t)m->ffn;
    if (l < 0 || l >= m->layers || n == 0 || pos + n > ctx) return -1;
    float *xn = (float *)malloc(sizeof(float) * n * H);
    float *q = (float *)malloc(sizeof(float) * n * qlen);
    float *k = (float *)malloc(sizeof(float) * n * kvw);
    float *v = (float *)malloc(sizeof(float) * n * kvw);
    float *att = (float *)malloc(sizeof(float) * n * qlen);
    float *proj = (float *)malloc(sizeof(float) * n * H);
    float *gate = (float *)malloc(sizeof(float) * n * F);
    float *up = (float *)malloc(sizeof(float) * n * F);
    float cos_s[512], sin_s[512];

    /* normalized = rms_norm(hidden) row by row; q/k/v = matmul(., batch) (:555-564) */
    memcpy(xn, hidden, sizeof(float) * n * H);
    hyqo_rms_norm_rows(xn, m->attn_norm[l], n * H, H, m->eps, 0);
    hyqo_matmul(m->dtype_linear, m->wq[l], qlen, H, xn, n, q, threads);
    hyqo_matmul(m->dtype_linear, m->wk[l], kvw, H, xn, n, k, threads);
    hyqo_matmul(m->dtype_linear, m->wv[l], kvw, H, xn, n, v, threads);
    /* rope at start + token (src/model.rs:570-583, 919-947), then the dense
     * order's per-head norms (:584-587) */
    if (m->arch == 1) {
        hyqo_rms_norm_rows(q, m->q_norm[l], n * qlen, D, m->eps, 0);
        hyqo_rms_norm_rows(k, m->k_norm[l], n * kvw, D, m->eps, 0);
    }
    for (size_t t = 0; t < n; ++t) {
        hyqo_rope_tables(D, m->rope_base, pos + t, cos_s, sin_s);
        hyqo_rope(q + t * qlen, (size_t)m->heads, D, cos_s, sin_s);
        hyqo_rope(k + t * kvw, (size_t)m->kv_heads, D, cos_s, sin_s);
    }
    if (m->arch != 1) {
        hyqo_rms_norm_rows(q, m->q_norm[l], n * qlen, D, m->eps, 0);
        hyqo_rms_norm_rows(k, m->k_norm[l], n * kvw, D, m->eps, 0);
    }
    /* cache.append (:588-593, 650-669), then causal attention: token t sees
     * positions 0..=pos+t (src/model.rs:956-961) */
    memcpy(kc + pos * kvw, k, sizeof(float) * n * kvw);
    memcpy(vc + pos * kvw, v, sizeof(float) * n * kvw);
    for (size_t t = 0; t < n; ++t)
        hyqo_attention(q + t * qlen, kc, vc, (size_t)m->heads, (size_t)m->kv_heads, D,
                       pos + t + 1, att + t * qlen);
    hyqo_matmul(m->dtype_linear, m->wo[l], H, qlen, att, n, proj, threads);
    for (size_t i = 0; i < n * H; ++i) hidden[i] += proj[i];
    /* DenseFfn::forward at batch n (src/model.rs:672-685): two matmuls,
     * silu(g) * u, down */
    memcpy(xn, hidden, sizeof(float) * n * H);
    hyqo_rms_norm_rows(xn, m->ffn_norm[l], n * H, H, m->eps, 0);
    if (m->moe && m->moe[l]) {
        /* Moe::forward at batch n (src/model.rs:598-601) */
        hyqo_moe_forward(m->moe[l], H, xn, n, proj, 0, threads);
    } else {
        hyqo_matmul(m->dtype_linear, m->wgate[l], F, H, xn, n, gate, threads);
        hyqo_matmul(m->dtype_linear, m->wup[l], F, H, xn, n, up, threads);
        for (size_t i = 0; i < n * F; ++i) {
            float g = gate[i];
            gate[i] = (g / (1.0f + expf(-g))) * up[i];
        }
        hyqo_matmul(m->dtype_down, m->wdown[l], H, F, gate, n, proj, threads);
    }
    for (size_t i = 0; i < n * H; ++i) hidden[i] += proj[i];

    free(xn);
    free(q);
    free(k);
    free(v);
    free(att);
    free(proj);
    free(gate);
    free(up);
    return 0;
}

int hyqo_prefill_chunk(const hyqo_model *m, float *kcache, float *vcache, size_t ctx, size_t pos,
                       const int *tokens, size_t n, int int8_path, float *logits, int threads)
{
    size_t H = (size_t)m->hidden, kvw = (size_t)m->kv_heads * m->head_dim;
    if (n == 0 || pos + n > ctx) return -1;
    for (size_t t = 0; t < n; ++t)
        if (tokens[t] < 0 || tokens[t] >= m->vocab) return -1;
    /* a one-token chunk takes the batch-1 arm (src/model.rs:557-558) */
    if (n == 1) return hyqo_decode_step(m, kcache, vcache, ctx, pos, tokens[0], int8_path, logits,
                                        threads);
    float *hidden = (float *)malloc(sizeof(float) * n * H);
    /* embedding rows (src/model.rs:549-552) */
    size_t erb = rb_of(m->dtype_embed, H);
    for (size_t t = 0; t < n; ++t)
        hyqo_decode(m->dtype_embed, m->embed + (size_t)tokens[t] * erb, erb, hidden + t * H, H);
    for (int l = 0; l < m->layers; ++l)
        hyqo_prefill_layer(m, l, hidden, kcache + (size_t)l * ctx * kvw,
                           vcache + (size_t)l * ctx * kvw, ctx, pos, n, threads);
    /* the last row's output norm and a batch-1 matmul (src/model.rs:605-607) */
    hyqo_output_logits(m, hidden + (n - 1) * H, int8_path, logits, threads);
    free(hidden);
    return 0;
}

int hyqo_argmax(const float *x, size_t n)
{
    /* greedy sampling (src/generation.rs:281-290): first maximum wins */
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return (int)best;
}
