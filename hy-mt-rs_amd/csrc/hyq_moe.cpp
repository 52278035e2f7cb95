// C ABI of the MoE expert products (include/hyq.h: hyq_moe_*): the expert
// loop of Moe::forward (src/model.rs:699-725) on one device. The router
// matmul, route() and the shared expert stay with the caller, as in the
// reference they run before the loop and seed its output.
#include <hip/hip_runtime.h>

#include <vector>

#include "hyq_abi.hpp"

using namespace hyq;

namespace {

struct MoeShape {
    size_t hidden, mid, experts;
};

int check_experts(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                  const hyq_weight *down, MoeShape *out)
{
    if (!ctx) return fail(HYQ_EINVAL, "moe: null context");
    if (!gate || !up || !down) return fail(HYQ_EINVAL, "moe: null expert weight");
    for (const hyq_weight *w : {gate, up, down}) {
        if (w->rank != 3) return fail(HYQ_EINVAL, "moe: expert weights must have rank 3");
        if (w->device != ctx->device) return fail(HYQ_EINVAL, "moe: weight on another device");
        if (!is_quant(w->dtype)) return fail(HYQ_EDTYPE, "moe: dtype %d has no batched path", w->dtype);
        int rc = check_f16_range(w, "moe");
        if (rc) return rc;
    }
    const size_t hidden = gate->dims[0], mid = gate->dims[1], E = gate->dims[2];
    if (up->dims[0] != hidden || up->dims[1] != mid || up->dims[2] != E)
        return fail(HYQ_EINVAL, "moe: up shape differs from gate");
    if (down->dims[0] != mid || down->dims[1] != hidden || down->dims[2] != E)
        return fail(HYQ_EINVAL, "moe: down must be [mid, hidden, experts]");
    if (gate->dtype != up->dtype) return fail(HYQ_EDTYPE, "moe: gate and up formats differ");
    if (hidden % 64 || mid % 64)
        return fail(HYQ_EINVAL, "moe: hidden %zu and mid %zu must be multiples of 64", hidden, mid);
    if (E > (size_t)moe_plan_max())
        return fail(HYQ_EINVAL, "moe: %zu experts exceed %d", E, moe_plan_max());
    *out = MoeShape{hidden, mid, E};
    return HYQ_OK;
}

int check_counts(size_t tokens, size_t npairs)
{
    if (tokens == 0 || tokens > (size_t)moe_plan_max())
        return fail(HYQ_EINVAL, "moe: %zu tokens (1..%d per call)", tokens, moe_plan_max());
    if (npairs > 65535) return fail(HYQ_EINVAL, "moe: %zu pairs exceed 65535", npairs);
    return HYQ_OK;
}

int check_device_args(const float *x_d, const float *out_d, const int32_t *pt, const int32_t *pe,
                      const float *pw, const void *scratch_d)
{
    if (!x_d || !out_d || !pt || !pe || !pw || !scratch_d)
        return fail(HYQ_EINVAL, "moe: null buffer");
    if ((uintptr_t)x_d % 16 || (uintptr_t)scratch_d % 256)
        return fail(HYQ_EINVAL, "moe: x must be 16-byte and scratch 256-byte aligned");
    return HYQ_OK;
}

// The expert loop on the context's stream (buffers checked); with `shared`
// (moe_fuses_shared holds) its product seeds out inside the same launches.
int experts_into(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                 const hyq_weight *down, const MoeShape &s, const float *x_d, size_t tokens,
                 const int32_t *pt, const int32_t *pe, const float *pw, size_t npairs,
                 void *scratch_d, size_t scratch_bytes, float *out_d, const WView *shared)
{
    const MoeLayout L =
        moe_layout((int)tokens, (int)npairs, (int)s.experts, (int)s.hidden, (int)s.mid);
    if (scratch_bytes < L.bytes)
        return fail(HYQ_EINVAL, "moe: scratch %zu bytes < %zu", scratch_bytes, L.bytes);
    HYQ_LAUNCH(launch_moe(gate->dtype, down->dtype, gate->view, up->view, down->view,
                          (int)s.hidden, (int)s.mid, x_d, (int)tokens, pt, pe, pw, (int)npairs,
                          (int)s.experts, (uint8_t *)scratch_d, L, out_d, ctx->stream, shared),
               "moe");
    return HYQ_OK;
}

} // namespace

extern "C" {

size_t hyq_moe_scratch_bytes(size_t tokens, size_t npairs, size_t experts, size_t hidden,
                             size_t mid)
{
    if (tokens > (size_t)moe_plan_max() || npairs > 65535 || experts > (size_t)moe_plan_max() ||
        hidden > (1u << 20) || mid > (1u << 20))
        return 0;
    return moe_layout((int)tokens, (int)npairs, (int)experts, (int)hidden, (int)mid).bytes;
}

int hyq_moe_experts_d(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                      const hyq_weight *down, const float *x_d, size_t tokens,
                      const int32_t *pair_token_d, const int32_t *pair_expert_d,
                      const float *pair_weight_d, size_t npairs, void *scratch_d,
                      size_t scratch_bytes, float *out_d)
{
    MoeShape s;
    int rc = check_experts(ctx, gate, up, down, &s);
    if (!rc) rc = check_counts(tokens, npairs);
    if (!rc && npairs)
        rc = check_device_args(x_d, out_d, pair_token_d, pair_expert_d, pair_weight_d, scratch_d);
    if (rc || npairs == 0) return rc;
    DeviceGuard g(ctx->device);
    return experts_into(ctx, gate, up, down, s, x_d, tokens, pair_token_d, pair_expert_d,
                        pair_weight_d, npairs, scratch_d, scratch_bytes, out_d, nullptr);
}

int hyq_moe_shared_experts_d(hyq_ctx *ctx, const hyq_weight *shared, const hyq_weight *gate,
                             const hyq_weight *up, const hyq_weight *down, const float *x_d,
                             size_t tokens, const int32_t *pair_token_d,
                             const int32_t *pair_expert_d, const float *pair_weight_d,
                             size_t npairs, void *scratch_d, size_t scratch_bytes, float *out_d)
{
    MoeShape s;
    int rc = check_experts(ctx, gate, up, down, &s);
    if (!rc) rc = check_counts(tokens, npairs);
    if (rc) return rc;
    if (!shared) return fail(HYQ_EINVAL, "moe: null shared weight");
    if (shared->rank != 2 || shared->cols != s.hidden || shared->rows != s.hidden)
        return fail(HYQ_EINVAL, "moe: the shared projection must be [%zu, %zu]", s.hidden,
                    s.hidden);
    if (shared->device != ctx->device) return fail(HYQ_EINVAL, "moe: shared weight on another device");
    if (npairs &&
        (rc = check_device_args(x_d, out_d, pair_token_d, pair_expert_d, pair_weight_d, scratch_d)))
        return rc;
    DeviceGuard g(ctx->device);
    if (shared->dtype == Q8_0 && !check_f16_range(shared, "moe") &&
        moe_fuses_shared(gate->dtype, down->dtype, gate->view, up->view, down->view,
                         (int)s.hidden, (int)s.mid, (int)tokens, (int)npairs, (int)s.experts))
        // the shared product's tiles run in the expert launches (its f16
        // rows formed with the experts' row operands, its tiles beside the
        // SiLU rows), before the routed sum
        return experts_into(ctx, gate, up, down, s, x_d, tokens, pair_token_d, pair_expert_d,
                            pair_weight_d, npairs, scratch_d, scratch_bytes, out_d,
                            &shared->view);
    // else the two calls: the seed (src/model.rs:699), then the loop
    rc = hyq_matmul_d(ctx, shared, x_d, tokens, out_d);
    if (rc || npairs == 0) return rc;
    return experts_into(ctx, gate, up, down, s, x_d, tokens, pair_token_d, pair_expert_d,
                        pair_weight_d, npairs, scratch_d, scratch_bytes, out_d, nullptr);
}

int hyq_moe_experts(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                    const hyq_weight *down, const float *x, size_t tokens,
                    const int32_t *pair_token, const int32_t *pair_expert,
                    const float *pair_weight, size_t npairs, float *out)
{
    MoeShape s;
    int rc = check_experts(ctx, gate, up, down, &s);
    if (!rc) rc = check_counts(tokens, npairs);
    if (rc) return rc;
    if (!x || !out) return fail(HYQ_EINVAL, "moe: null buffer");
    if (npairs && (!pair_token || !pair_expert || !pair_weight))
        return fail(HYQ_EINVAL, "moe: null routing list");
    for (size_t p = 0; p < npairs; ++p) {
        if (pair_token[p] < 0 || (size_t)pair_token[p] >= tokens)
            return fail(HYQ_EINVAL, "moe: pair %zu names token %d of %zu", p, pair_token[p], tokens);
        if (pair_expert[p] < 0 || (size_t)pair_expert[p] >= s.experts)
            return fail(HYQ_EINVAL, "moe: pair %zu names expert %d of %zu", p, pair_expert[p],
                        s.experts);
    }
    if (npairs == 0) return HYQ_OK;
    DeviceGuard g(ctx->device);
    const MoeLayout L =
        moe_layout((int)tokens, (int)npairs, (int)s.experts, (int)s.hidden, (int)s.mid);
    const size_t xbytes = tokens * s.hidden * 4;
    const size_t pbytes = align_up(npairs * 4, 256);
    // x | out | tokens | experts | weights in ctx->x, the plan in ctx->moe
    rc = ctx->x.reserve(ctx->device, 2 * align_up(xbytes, 256) + 3 * pbytes);
    if (!rc) rc = ctx->moe.reserve(ctx->device, L.bytes);
    if (rc) return rc;
    uint8_t *base = (uint8_t *)ctx->x.ptr();
    float *xd = (float *)base;
    float *od = (float *)(base + align_up(xbytes, 256));
    uint8_t *pd = base + 2 * align_up(xbytes, 256);
    hipStream_t st = ctx->stream;
    HYQ_HIP(hipMemcpyAsync(xd, x, xbytes, hipMemcpyHostToDevice, st), "hipMemcpy");
    HYQ_HIP(hipMemcpyAsync(od, out, xbytes, hipMemcpyHostToDevice, st), "hipMemcpy");
    HYQ_HIP(hipMemcpyAsync(pd, pair_token, npairs * 4, hipMemcpyHostToDevice, st), "hipMemcpy");
    HYQ_HIP(hipMemcpyAsync(pd + pbytes, pair_expert, npairs * 4, hipMemcpyHostToDevice, st),
            "hipMemcpy");
    HYQ_HIP(hipMemcpyAsync(pd + 2 * pbytes, pair_weight, npairs * 4, hipMemcpyHostToDevice, st),
            "hipMemcpy");
    HYQ_LAUNCH(launch_moe(gate->dtype, down->dtype, gate->view, up->view, down->view,
                          (int)s.hidden, (int)s.mid, xd, (int)tokens, (const int *)pd,
                          (const int *)(pd + pbytes), (const float *)(pd + 2 * pbytes),
                          (int)npairs, (int)s.experts, (uint8_t *)ctx->moe.ptr(), L, od, st),
               "moe");
    HYQ_HIP(hipMemcpyAsync(out, od, xbytes, hipMemcpyDeviceToHost, st), "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
    return HYQ_OK;
}

} // extern "C"
