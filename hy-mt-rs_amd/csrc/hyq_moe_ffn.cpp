// Moe::forward (src/model.rs:687-726) on the device: the launch sequences
// declared in hyq_moe_ffn.hpp and the standalone C ABI entry points
// (hyq_moe_route_d, hyq_moe_forward_d).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "hyq_moe_ffn.hpp"

namespace hyq {

namespace {

size_t carve(size_t &off, size_t bytes)
{
    const size_t o = off;
    off += align_up(bytes, 256);
    return o;
}

bool int8_width(size_t w) { return w % 256 == 0 && w / 256 <= 160; }

int check_shape(const hyq_weight *w, size_t cols, size_t rows, size_t experts, const char *name,
                int device)
{
    if (!w) return fail(HYQ_EINVAL, "moe: null %s weight", name);
    if (w->device != device) return fail(HYQ_EINVAL, "moe: %s on another device", name);
    const int rank = experts ? 3 : 2;
    if (w->rank != rank || w->dims[0] != cols || w->dims[1] != rows ||
        (experts && w->dims[2] != experts))
        return fail(HYQ_EINVAL, "%s: expected GGUF shape [%zu, %zu%s], got [%llu, %llu, %llu]",
                    name, cols, rows, experts ? ", experts" : "",
                    (unsigned long long)w->dims[0], (unsigned long long)w->dims[1],
                    (unsigned long long)w->dims[2]);
    return HYQ_OK;
}

} // namespace

int moe_ffn_check(const MoeFfn &f, int device)
{
    if (f.experts <= 0 || f.used <= 0 || f.used > f.experts || f.mid <= 0 || f.smid <= 0 ||
        f.hidden <= 0)
        return fail(HYQ_EINVAL, "invalid expert dimensions");
    if (!(f.scale > 0.f)) return fail(HYQ_EINVAL, "invalid expert weight scale");
    if (f.experts > route_max_experts())
        return fail(HYQ_EINVAL, "moe: %d experts exceed %d", f.experts, route_max_experts());
    const size_t H = f.hidden, E = f.experts, M = f.mid, S = f.smid;
    int rc = check_shape(f.router, H, E, 0, "ffn_gate_inp", device);
    if (!rc && f.router->dtype != F32) rc = fail(HYQ_EDTYPE, "HYV3 router must use F32");
    if (!rc) rc = check_shape(f.gate, H, M, E, "ffn_gate_exps", device);
    if (!rc) rc = check_shape(f.up, H, M, E, "ffn_up_exps", device);
    if (!rc) rc = check_shape(f.down, M, H, E, "ffn_down_exps", device);
    if (!rc) rc = check_shape(f.sgate, H, S, 0, "ffn_gate_shexp", device);
    if (!rc) rc = check_shape(f.sup, H, S, 0, "ffn_up_shexp", device);
    if (!rc) rc = check_shape(f.sdown, S, H, 0, "ffn_down_shexp", device);
    if (rc) return rc;
    if (!f.bias_d) return fail(HYQ_EINVAL, "moe: null selection bias");
    for (const hyq_weight *w : {f.gate, f.up, f.down, f.sgate, f.sup, f.sdown})
        if (!is_quant(w->dtype)) return fail(HYQ_EDTYPE, "moe: dtype %d has no int8 path", w->dtype);
    if (f.gate->dtype != f.up->dtype || f.sgate->dtype != f.sup->dtype)
        return fail(HYQ_EDTYPE, "moe: gate and up formats differ");
    if (!int8_width(H) || !int8_width(M) || !int8_width(S))
        return fail(HYQ_EINVAL, "moe: hidden %zu, mid %zu and shared %zu must be whole 256-value "
                                "groups (at most 40960)",
                    H, M, S);
    return HYQ_OK;
}

size_t moe_row_bytes(const MoeFfn &f)
{
    size_t off = 0;
    carve(off, 4 * (size_t)f.experts);
    carve(off, 4 * (size_t)f.used);
    carve(off, 4 * (size_t)f.used);
    carve(off, 4 * (size_t)f.smid);
    carve(off, 4 * (size_t)f.used * f.mid);
    carve(off, 4 * (size_t)f.hidden);
    carve(off, 4 * (size_t)f.used * f.hidden);
    return off;
}

MoeRowBuf moe_row_carve(const MoeFfn &f, uint8_t *base)
{
    size_t off = 0;
    MoeRowBuf b{};
    b.logits = (float *)(base + carve(off, 4 * (size_t)f.experts));
    b.se = (int *)(base + carve(off, 4 * (size_t)f.used));
    b.sw = (float *)(base + carve(off, 4 * (size_t)f.used));
    b.hs = (float *)(base + carve(off, 4 * (size_t)f.smid));
    b.he = (float *)(base + carve(off, 4 * (size_t)f.used * f.mid));
    b.ps = (float *)(base + carve(off, 4 * (size_t)f.hidden));
    b.pe = (float *)(base + carve(off, 4 * (size_t)f.used * f.hidden));
    return b;
}

int moe_ffn_row(hipStream_t st, const MoeFfn &f, const float *xn, const Q8Ref &xq,
                const MoeRowBuf &b, const float *residual, float *out, float *trace,
                Q8Trace *q8t)
{
    const int H = f.hidden;
    // router logits (F32 decoded rows, src/model.rs:691) and route (:694)
    HYQ_LAUNCH(launch_f32_gemv(F32, f.router->view, nullptr, H, xn, b.logits, st), "router");
    HYQ_LAUNCH(launch_route(b.logits, f.bias_d, 1, f.experts, f.used, f.normalize != 0, f.scale,
                            b.se, b.sw, nullptr, st),
               "route");
    // gate/up SiLU rows: the shared expert, then the chosen experts' slots
    {
        GemvArgs a{};
        a.nseg = 2;
        a.seg[0].w = f.sgate->view;
        a.seg[0].y = b.hs;
        a.seg[1].w = f.sup->view;
        a.rows_total = f.smid;
        a.groups = H / 256;
        a.x = xq.view();
        HYQ_LAUNCH(launch_gemv(f.sgate->dtype, GEMV_SILU, a, st), "moe_shared_gate_up");
    }
    {
        GemvArgs a{};
        a.nseg = 2;
        a.seg[0].w = f.gate->view;
        a.seg[0].y = b.he;
        a.seg[1].w = f.up->view;
        a.rows_total = f.used * f.mid;
        a.groups = H / 256;
        a.x = xq.view();
        a.slot_expert = b.se;
        a.slot_experts = f.experts;
        a.slot_rows = f.mid;
        HYQ_LAUNCH(launch_gemv(f.gate->dtype, GEMV_SILU, a, st), "moe_experts_gate_up");
    }
    // down rows, each from its SiLU row quantized in the launch's input stage
    {
        GemvArgs a{};
        a.nseg = 1;
        a.seg[0].w = f.sdown->view;
        a.seg[0].y = b.ps;
        a.rows_total = H;
        a.groups = f.smid / 256;
        a.xin = b.hs;
        q8_trace_gemv(q8t, a);
        HYQ_LAUNCH(launch_gemv(f.sdown->dtype, GEMV_PLAIN, a, st), "moe_shared_down");
    }
    {
        GemvArgs a{};
        a.nseg = 1;
        a.seg[0].w = f.down->view;
        a.seg[0].y = b.pe;
        a.rows_total = H;
        a.groups = f.mid / 256;
        a.xin = b.he;
        a.slot_expert = b.se;
        a.slot_experts = f.experts;
        a.nslots = f.used;
        a.slot_xin_stride = f.mid;
        q8_trace_gemv(q8t, a);
        HYQ_LAUNCH(launch_gemv(f.down->dtype, GEMV_PLAIN, a, st), "moe_experts_down");
    }
    HYQ_LAUNCH(launch_ffn_combine(residual, b.ps, b.pe, b.sw, f.used, H, 1, out, trace, st),
               "moe_combine");
    return HYQ_OK;
}

int moe_rows_max(const MoeFfn &f)
{
    return std::max(1, std::min(moe_plan_max(), 65535 / std::max(f.used, 1)));
}

size_t moe_rows_bytes(const MoeFfn &f, int n)
{
    const size_t N = n, np = (size_t)n * f.used, W = std::max(f.hidden, f.smid);
    size_t off = 0;
    carve(off, 4 * N * f.experts);
    carve(off, 4 * np);
    carve(off, 4 * N);
    carve(off, 4 * N * f.smid);
    carve(off, 4 * N * f.hidden);
    carve(off, 4 * np);
    carve(off, 4 * np);
    carve(off, 2 * N * W);
    carve(off, moe_layout(n, (int)np, f.experts, f.hidden, f.mid).bytes);
    return off;
}

MoeRowsBuf moe_rows_carve(const MoeFfn &f, int n, uint8_t *base)
{
    const size_t N = n, np = (size_t)n * f.used, W = std::max(f.hidden, f.smid);
    size_t off = 0;
    MoeRowsBuf b{};
    b.logits = (float *)(base + carve(off, 4 * N * f.experts));
    b.pw = (float *)(base + carve(off, 4 * np));
    b.rs = (float *)(base + carve(off, 4 * N));
    b.h = (float *)(base + carve(off, 4 * N * f.smid));
    b.ffo = (float *)(base + carve(off, 4 * N * f.hidden));
    b.pt = (int *)(base + carve(off, 4 * np));
    b.pe = (int *)(base + carve(off, 4 * np));
    b.xh = (_Float16 *)(base + carve(off, 2 * N * W));
    b.L = moe_layout(n, (int)np, f.experts, f.hidden, f.mid);
    b.scratch = base + carve(off, b.L.bytes);
    return b;
}

int moe_ffn_rows(hipStream_t st, const MoeFfn &f, const float *xn, int n, const MoeRowsBuf &b,
                 const float *residual, float *out)
{
    const int H = f.hidden;
    // router logits at batch n (F32, src/model.rs:691) and the pairs (:692-698)
    HYQ_LAUNCH(launch_f32_gemm(F32, f.router->view, H, xn, n, b.logits, st), "router");
    HYQ_LAUNCH(launch_route(b.logits, f.bias_d, n, f.experts, f.used, f.normalize != 0, f.scale,
                            b.pe, b.pw, b.pt, st),
               "route");
    // output = shared.forward(input, n) (:699): two products, silu(g) * u, down
    HYQ_LAUNCH(launch_to_f16(xn, n, H, b.xh, b.rs, st), "to_f16");
    HYQ_LAUNCH(launch_gate_up_f16(f.sgate->dtype, f.sgate->view, f.sup->view, H, b.xh, b.rs, n,
                                  b.h, st),
               "moe_shared_gate_up");
    HYQ_LAUNCH(launch_to_f16(b.h, n, f.smid, b.xh, b.rs, st), "to_f16");
    HYQ_LAUNCH(launch_gemm_f16(f.sdown->dtype, f.sdown->view, f.smid, b.xh, b.rs, n, b.ffo,
                               nullptr, st),
               "moe_shared_down");
    // the experts, added per token in ascending expert order (:700-722)
    HYQ_LAUNCH(launch_moe(f.gate->dtype, f.down->dtype, f.gate->view, f.up->view, f.down->view, H,
                          f.mid, xn, n, b.pt, b.pe, b.pw, n * f.used, f.experts, b.scratch, b.L,
                          b.ffo, st),
               "moe_experts");
    HYQ_LAUNCH(launch_ffn_combine(residual, b.ffo, nullptr, nullptr, 0, H, n, out, nullptr, st),
               "moe_residual");
    return HYQ_OK;
}

} // namespace hyq

using namespace hyq;

namespace {

MoeFfn ffn_of(const hyq_moe_config *mc, const hyq_weight *router, const float *bias_d,
              const hyq_weight *gate, const hyq_weight *up, const hyq_weight *down,
              const hyq_weight *sgate, const hyq_weight *sup, const hyq_weight *sdown)
{
    MoeFfn f;
    f.router = router;
    f.bias_d = bias_d;
    f.gate = gate;
    f.up = up;
    f.down = down;
    f.sgate = sgate;
    f.sup = sup;
    f.sdown = sdown;
    f.hidden = router ? (int)router->dims[0] : 0;
    f.experts = mc->experts;
    f.used = mc->used;
    f.mid = mc->mid;
    f.smid = mc->shared_mid;
    f.normalize = mc->normalize;
    f.scale = mc->scale;
    return f;
}

// The Q8 buffers of one row of H values (values, scales and the
// 16/32/256-value sums) carved from base at off (base may be null to size).
Q8Ref q8_carve(uint8_t *base, size_t &off, size_t H)
{
    const size_t ng = H / 256;
    Q8Ref q;
    q.q = (int8_t *)(base + carve(off, H));
    q.s = (float *)(base + carve(off, 4 * ng));
    q.sum16 = (int32_t *)(base + carve(off, H / 4));
    q.sum32 = (int32_t *)(base + carve(off, H / 8));
    q.sum256 = (int32_t *)(base + carve(off, 4 * ng));
    q.n = H;
    return q;
}

size_t forward_bytes(const MoeFfn &f, size_t tokens)
{
    if (tokens == 1) {
        size_t off = 0;
        (void)q8_carve(nullptr, off, (size_t)f.hidden);
        return off + moe_row_bytes(f);
    }
    return moe_rows_bytes(f, (int)tokens);
}

} // namespace

extern "C" {

int hyq_moe_route_d(hyq_ctx *ctx, const float *logits_d, const float *bias_d, size_t tokens,
                    size_t experts, size_t used, int normalize, float scale,
                    int32_t *pair_token_d, int32_t *pair_expert_d, float *pair_weight_d)
{
    if (!ctx) return fail(HYQ_EINVAL, "route: null context");
    if (experts == 0 || used == 0 || used > experts || experts > (size_t)route_max_experts())
        return fail(HYQ_EINVAL, "route: %zu of %zu experts (at most %d)", used, experts,
                    route_max_experts());
    if (tokens > 65535) return fail(HYQ_EINVAL, "route: %zu tokens exceed 65535", tokens);
    if (tokens == 0) return HYQ_OK;
    if (!logits_d || !bias_d || !pair_expert_d || !pair_weight_d)
        return fail(HYQ_EINVAL, "route: null buffer");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_route(logits_d, bias_d, (int)tokens, (int)experts, (int)used,
                            normalize != 0, scale, pair_expert_d, pair_weight_d, pair_token_d,
                            ctx->stream),
               "route");
    return HYQ_OK;
}

size_t hyq_moe_forward_scratch_bytes(const hyq_moe_config *mc, size_t hidden, size_t tokens)
{
    if (!mc || tokens == 0 || hidden == 0 || hidden > (1u << 20) || mc->experts <= 0 ||
        mc->used <= 0 || mc->mid <= 0 || mc->shared_mid <= 0 || mc->experts > (1 << 20) ||
        mc->mid > (1 << 20) || mc->shared_mid > (1 << 20))
        return 0;
    MoeFfn f;
    f.hidden = (int)hidden;
    f.experts = mc->experts;
    f.used = mc->used;
    f.mid = mc->mid;
    f.smid = mc->shared_mid;
    if (tokens > 1 && tokens > (size_t)moe_rows_max(f)) return 0;
    return forward_bytes(f, tokens);
}

int hyq_moe_forward_d(hyq_ctx *ctx, const hyq_moe_config *mc, const hyq_weight *router,
                      const float *bias_d, const hyq_weight *gate, const hyq_weight *up,
                      const hyq_weight *down, const hyq_weight *shared_gate,
                      const hyq_weight *shared_up, const hyq_weight *shared_down,
                      const float *x_d, size_t tokens, void *scratch_d, size_t scratch_bytes,
                      float *out_d)
{
    if (!ctx || !mc) return fail(HYQ_EINVAL, "moe_forward: null argument");
    const MoeFfn f = ffn_of(mc, router, bias_d, gate, up, down, shared_gate, shared_up,
                            shared_down);
    int rc = moe_ffn_check(f, ctx->device);
    if (rc) return rc;
    if (tokens == 0) return HYQ_OK;
    if (tokens > (size_t)moe_rows_max(f))
        return fail(HYQ_EINVAL, "moe_forward: %zu tokens exceed %d per call", tokens,
                    moe_rows_max(f));
    if (tokens > 1)
        for (const hyq_weight *w : {gate, up, down, shared_gate, shared_up, shared_down})
            if ((rc = check_f16_range(w, "moe_forward"))) return rc;
    if (!x_d || !out_d || !scratch_d) return fail(HYQ_EINVAL, "moe_forward: null buffer");
    if ((uintptr_t)x_d % 16 || (uintptr_t)scratch_d % 256)
        return fail(HYQ_EINVAL, "moe_forward: x must be 16-byte and scratch 256-byte aligned");
    const size_t need = forward_bytes(f, tokens);
    if (scratch_bytes < need)
        return fail(HYQ_EINVAL, "moe_forward: scratch %zu bytes < %zu", scratch_bytes, need);
    DeviceGuard g(ctx->device);
    uint8_t *base = (uint8_t *)scratch_d;
    if (tokens == 1) {
        size_t off = 0;
        const Q8Ref q = q8_carve(base, off, (size_t)f.hidden);
        HYQ_LAUNCH(launch_quantize_q8(x_d, f.hidden, q.q, q.s, q.sum16, q.sum32, q.sum256,
                                      ctx->stream),
                   "quantize_q8");
        if ((rc = q8_trace_copy(ctx->q8t(), q, x_d, (size_t)f.hidden, ctx->stream))) return rc;
        return moe_ffn_row(ctx->stream, f, x_d, q, moe_row_carve(f, base + off), nullptr, out_d,
                           nullptr, ctx->q8t());
    }
    return moe_ffn_rows(ctx->stream, f, x_d, (int)tokens, moe_rows_carve(f, (int)tokens, base),
                        nullptr, out_d);
}

} // extern "C"
