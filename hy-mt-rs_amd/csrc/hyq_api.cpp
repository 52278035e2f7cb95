// C ABI of hyq (include/hyq.h): validation, device memory and launches.
//
// Every entry point checks shapes the way the reference's `ensure!` arms do
// (src/quant.rs:160-166, :665-671, :726-730, :1067-1076) before any device
// work, so bad sizes become HYQ_EINVAL instead of out-of-bounds accesses.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "hyq_abi.hpp"

using namespace hyq;

namespace hyq {
namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what)
{
    // A failed runtime call (an allocation past the device's memory, say)
    // stays the thread's last error until read, and every launcher reports
    // hipGetLastError after its launch: read it here, so that the next launch
    // is not reported as this call's failure.
    (void)hipGetLastError();
    return fail(e == hipErrorOutOfMemory ? HYQ_ENOMEM : HYQ_EDEVICE, "%s: %s", what,
                hipGetErrorString(e));
}

namespace {
float f16_bits(const uint8_t *p)
{
    _Float16 h;
    std::memcpy(&h, p, 2);
    return (float)h;
}
} // namespace

float weight_max_abs(int dtype, const uint8_t *b, size_t nblocks)
{
    const size_t bb = (size_t)block_bytes(dtype);
    float m = 0.f;
    auto upd = [&](float v) {
        v = std::fabs(v);
        if (!(v <= m)) m = v; // NaN propagates
    };
    for (size_t i = 0; i < nblocks; ++i) {
        const uint8_t *x = b + i * bb;
        switch (dtype) {
        case F32: {
            float v;
            std::memcpy(&v, x, 4);
            upd(v);
            break;
        }
        case F16: upd(f16_bits(x)); break;
        case Q8_0: upd(f16_bits(x) * 128.f); break;   // d * q, |q| <= 128
        case Q2_0C: upd(f16_bits(x) * 3.f); break;    // (2c - 3) d
        case STQ1_0: upd(f16_bits(x + 40)); break;    // digit * d, |digit| <= 1
        case Q4_K: {                                   // d s q - dmin m, q <= 15, s, m <= 63
            int smax = 0, mmax = 0;
            for (int j = 0; j < 8; ++j) {
                const uint8_t *sc = x + 4;
                const int s6 = j < 4 ? sc[j] & 63 : (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
                const int m6 = j < 4 ? sc[j + 4] & 63 : (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
                smax = s6 > smax ? s6 : smax;
                mmax = m6 > mmax ? m6 : mmax;
            }
            upd(std::fabs(f16_bits(x)) * (float)(15 * smax) + std::fabs(f16_bits(x + 2)) * (float)mmax);
            break;
        }
        case Q6_K: { // (d sc) (q - 32), |q - 32| <= 32
            int smax = 0;
            for (int j = 0; j < 16; ++j) {
                const int v = std::abs((int)(int8_t)x[192 + j]);
                smax = v > smax ? v : smax;
            }
            upd(f16_bits(x + 208) * (float)(32 * smax));
            break;
        }
        default: break;
        }
    }
    return m;
}

int check_f16_range(const hyq_weight *w, const char *who)
{
    const float m = w->max_abs;
    if (!(m <= 65504.f))
        return fail(HYQ_EINVAL,
                    "%s: weight values up to %g leave the f16 range of the batched products",
                    who, (double)m);
    if (m > 0.f && m < 6.103515625e-05f)
        return fail(HYQ_EINVAL,
                    "%s: all weight values are below %g, f16's smallest normal: the batched "
                    "products would lose them",
                    who, 6.103515625e-05);
    return HYQ_OK;
}

int q8_alloc(int device, size_t n, hyq_q8 **out)
{
    auto q = std::make_unique<hyq_q8>();
    q->ref.n = n;
    q->device = device;
    const size_t ng = (n + 255) / 256, n16 = (n + 15) / 16, n32 = (n + 31) / 32;
    const size_t off_s = align_up(n, 256);
    const size_t off_16 = off_s + align_up(ng * 4, 256);
    const size_t off_32 = off_16 + align_up(n16 * 4, 256);
    const size_t off_256 = off_32 + align_up(n32 * 4, 256);
    const size_t total = off_256 + align_up(ng * 4, 256);
    q->mem = std::make_unique<DeviceBuffer>();
    int rc = q->mem->alloc(device, total);
    if (rc) return rc;
    uint8_t *base = (uint8_t *)q->mem->ptr;
    q->ref.q = (int8_t *)base;
    q->ref.s = (float *)(base + off_s);
    q->ref.sum16 = (int32_t *)(base + off_16);
    q->ref.sum32 = (int32_t *)(base + off_32);
    q->ref.sum256 = (int32_t *)(base + off_256);
    *out = q.release();
    return HYQ_OK;
}

bool Q8Trace::take(size_t n, int8_t **codes, float **scales, float **values)
{
    const size_t xoff = align_up(n + n / 64, 256);
    const size_t need = xoff + align_up(4 * n, 256);
    if (!base || n % 256 || used + need > bytes) {
        if (base) ++dropped;
        return false;
    }
    *codes = (int8_t *)(base + used);
    *scales = (float *)(base + used + n);
    *values = (float *)(base + used + xoff);
    records.emplace_back(used, n);
    used += need;
    return true;
}

void q8_trace_gemv(Q8Trace *t, GemvArgs &a)
{
    if (!t || !a.xin) return;
    const size_t parts = a.nslots > 0 ? (size_t)a.nslots : a.kslices > 1 ? (size_t)a.kslices : 1;
    if (!t->take((size_t)a.groups * 256 * parts, &a.q8t_codes, &a.q8t_scales, &a.q8t_x)) {
        a.q8t_codes = nullptr;
        a.q8t_scales = nullptr;
        a.q8t_x = nullptr;
    }
}

int q8_trace_copy(Q8Trace *t, const Q8Ref &q, const float *x, size_t n, hipStream_t st)
{
    int8_t *codes;
    float *scales, *values;
    if (!t || !t->take(n, &codes, &scales, &values)) return HYQ_OK;
    HYQ_HIP(hipMemcpyAsync(codes, q.q, n, hipMemcpyDeviceToDevice, st), "q8 trace");
    HYQ_HIP(hipMemcpyAsync(scales, q.s, n / 256 * 4, hipMemcpyDeviceToDevice, st), "q8 trace");
    HYQ_HIP(hipMemcpyAsync(values, x, n * 4, hipMemcpyDeviceToDevice, st), "q8 trace");
    return HYQ_OK;
}

} // namespace hyq

namespace {

// The context's own Q8 buffers, grown on demand, as a prefix of length n.
int ctx_q8(hyq_ctx *ctx, size_t n, Q8Ref *out)
{
    if (!ctx->q8 || ctx->q8->ref.n < n) {
        delete ctx->q8;
        ctx->q8 = nullptr;
        int rc = q8_alloc(ctx->device, align_up(n, 4096), &ctx->q8);
        if (rc) return rc;
    }
    *out = ctx->q8->ref.prefix(n);
    return HYQ_OK;
}

int quantize_into(hyq_ctx *ctx, const float *x_d, const Q8Ref &q8)
{
    HYQ_LAUNCH(launch_quantize_q8(x_d, (int)q8.n, q8.q, q8.s, q8.sum16, q8.sum32, q8.sum256,
                                  ctx->stream),
               "quantize_q8");
    return HYQ_OK;
}

bool is_raw(int d) { return d == HYQ_F32 || d == HYQ_F16; }

bool dtype_known(int d)
{
    return d == HYQ_F32 || d == HYQ_F16 || d == HYQ_Q8_0 || d == HYQ_Q4_K || d == HYQ_Q6_K ||
           d == HYQ_Q2_0C || d == HYQ_STQ1_0;
}

int check_matrix(const hyq_weight *w, const char *who)
{
    if (!w) return fail(HYQ_EINVAL, "%s: null weight", who);
    if (w->rank != 2) return fail(HYQ_EINVAL, "%s: weight is not a matrix (rank %d)", who, w->rank);
    return HYQ_OK;
}

// The int8 GEMV reads whole 256-value groups.
int check_int8_path(const hyq_weight *w, const char *who)
{
    if (!is_quant(w->dtype))
        return fail(HYQ_EDTYPE, "%s: dtype %d has no int8 path", who, w->dtype);
    if (w->cols % 256 != 0)
        return fail(HYQ_EINVAL, "%s: cols %zu is not a multiple of 256", who, w->cols);
    // the Q8 row is staged in LDS at 272 bytes per 256 values (64 KiB at most)
    if (w->cols > 240 * 256)
        return fail(HYQ_EINVAL, "%s: cols %zu exceeds %d", who, w->cols, 240 * 256);
    return HYQ_OK;
}

int check_q8(const hyq_q8 *x, size_t cols, const char *who)
{
    if (!x) return fail(HYQ_EINVAL, "%s: null activations", who);
    if (x->ref.n != cols)
        return fail(HYQ_EINVAL, "%s: activation length %zu != cols %zu", who, x->ref.n, cols);
    return HYQ_OK;
}

// An f32 row that the GEMV quantizes itself into LDS (one launch, no
// separate quantize pass): float4-aligned, with the Q8 row and its sums
// (380 bytes per 256 values) within 60 KiB of LDS.
constexpr size_t STAGED_MAX_GROUPS = 160;

bool can_stage(const float *x_d, size_t cols)
{
    return (uintptr_t)x_d % 16 == 0 && cols % 256 == 0 && cols / 256 <= STAGED_MAX_GROUPS;
}

GemvArgs base_args(const hyq_weight *w, const Q8Ref &x)
{
    GemvArgs a{};
    a.nseg = 1;
    a.seg[0].w = w->view;
    a.seg[0].row_start = 0;
    a.rows_total = (int)w->rows;
    a.groups = (int)(w->cols / 256);
    a.x = x.view();
    return a;
}

int gemv_plain(hyq_ctx *ctx, const hyq_weight *w, const Q8Ref &x, const float *residual,
               float *y)
{
    GemvArgs a = base_args(w, x);
    a.seg[0].y = y;
    a.residual = residual;
    HYQ_LAUNCH(launch_gemv(w->dtype, GEMV_PLAIN, a, ctx->stream), "gemv");
    return HYQ_OK;
}

int gemv_qkv(hyq_ctx *ctx, const hyq_weight *q, const hyq_weight *k, const hyq_weight *v,
             const Q8Ref &x, float *yq, float *yk, float *yv)
{
    if (q->dtype == k->dtype && k->dtype == v->dtype) {
        GemvArgs a = base_args(q, x);
        const hyq_weight *ws[3] = {q, k, v};
        float *ys[3] = {yq, yk, yv};
        int start = 0;
        for (int i = 0; i < 3; ++i) {
            a.seg[i].w = ws[i]->view;
            a.seg[i].y = ys[i];
            a.seg[i].row_start = start;
            start += (int)ws[i]->rows;
        }
        a.nseg = 3;
        a.rows_total = start;
        HYQ_LAUNCH(launch_gemv(q->dtype, GEMV_MULTI, a, ctx->stream), "gemv_qkv");
        return HYQ_OK;
    }
    // mixed formats: three launches sharing the one Q8 vector
    int rc = gemv_plain(ctx, q, x, nullptr, yq);
    if (!rc) rc = gemv_plain(ctx, k, x, nullptr, yk);
    if (!rc) rc = gemv_plain(ctx, v, x, nullptr, yv);
    return rc;
}

int gate_up(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up, const Q8Ref &x,
            float *y)
{
    GemvArgs a = base_args(gate, x);
    a.nseg = 2;
    a.seg[0].y = y;
    a.seg[1].w = up->view;
    a.seg[1].row_start = 0;
    HYQ_LAUNCH(launch_gemv(gate->dtype, GEMV_SILU, a, ctx->stream), "gate_up_silu");
    return HYQ_OK;
}

int check_qkv(const hyq_weight *q, const hyq_weight *k, const hyq_weight *v)
{
    int rc = check_matrix(q, "gemv_qkv");
    if (!rc) rc = check_matrix(k, "gemv_qkv");
    if (!rc) rc = check_matrix(v, "gemv_qkv");
    if (rc) return rc;
    if (k->cols != q->cols || v->cols != q->cols)
        return fail(HYQ_EINVAL, "query, key and value must be matrices that share an input width");
    if (q->device != k->device || q->device != v->device)
        return fail(HYQ_EINVAL, "gemv_qkv: weights live on different devices");
    if (is_raw(q->dtype) || is_raw(k->dtype) || is_raw(v->dtype)) {
        if (!(is_raw(q->dtype) && is_raw(k->dtype) && is_raw(v->dtype)))
            return fail(HYQ_EDTYPE, "gemv_qkv: F32/F16 mixed with quantized weights");
        return HYQ_OK;
    }
    rc = check_int8_path(q, "gemv_qkv");
    if (!rc) rc = check_int8_path(k, "gemv_qkv");
    if (!rc) rc = check_int8_path(v, "gemv_qkv");
    return rc;
}

int check_gate_up(const hyq_weight *gate, const hyq_weight *up)
{
    int rc = check_matrix(gate, "gate_up_silu");
    if (!rc) rc = check_matrix(up, "gate_up_silu");
    if (rc) return rc;
    if (gate->rows != up->rows || gate->cols != up->cols)
        return fail(HYQ_EINVAL, "gate and up shape mismatch");
    if (gate->dtype != up->dtype)
        return fail(HYQ_EDTYPE, "gate_up_silu: gate and up formats differ (%d vs %d)",
                    gate->dtype, up->dtype);
    if (is_raw(gate->dtype)) return HYQ_OK;
    return check_int8_path(gate, "gate_up_silu");
}

int check_ctx_weight(hyq_ctx *ctx, const hyq_weight *w, const char *who)
{
    if (!ctx) return fail(HYQ_EINVAL, "%s: null context", who);
    if (w && w->device != ctx->device)
        return fail(HYQ_EINVAL, "%s: weight is on device %d, context on %d", who, w->device,
                    ctx->device);
    return HYQ_OK;
}

// ---- Weight::matmul on device buffers, with its temporaries either from the
// context (grown by hipMalloc on demand) or from the fixed per-device array
// of hyq_matmul_noalloc_d ----

// `scratch`: the no-allocation entry point's temporaries, one copy per GPU
// (a module global, resident while the library is loaded). Host code never
// passes this name to a kernel: it uses the per-device address that
// hipGetSymbolAddress returned (g_scratch), resolved once per device by
// hyq_ctx_create with that device current.
static __device__ __align__(256) uint8_t scratch[HYQ_NOALLOC_SCRATCH_BYTES];
std::mutex g_scratch_mu;
std::unordered_map<int, void *> g_scratch;

int resolve_scratch(int device)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch.count(device)) return HYQ_OK;
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch[device] = ptr;
    return HYQ_OK;
}

struct FixedScratch {
    uint8_t *base;
    size_t bytes;
};

// Carves [offset, offset + bytes) out of the fixed array, or fails when the
// request exceeds it.
int take_fixed(const FixedScratch &fs, size_t &off, size_t bytes, void **out, const char *what)
{
    const size_t o = align_up(off, 256);
    if (o + bytes > fs.bytes)
        return fail(HYQ_EINVAL,
                    "matmul_noalloc: %s needs %zu bytes of scratch beyond the %zu-byte maximum",
                    what, o + bytes - fs.bytes, fs.bytes);
    *out = fs.base + o;
    off = o + bytes;
    return HYQ_OK;
}

// Q8 buffers of length n laid out like q8_alloc's, inside the fixed array.
int fixed_q8(const FixedScratch &fs, size_t &off, size_t n, Q8Ref *out)
{
    const size_t ng = (n + 255) / 256, n16 = (n + 15) / 16, n32 = (n + 31) / 32;
    void *q = nullptr, *sc = nullptr, *s16 = nullptr, *s32 = nullptr, *s256 = nullptr;
    int rc = take_fixed(fs, off, n, &q, "Q8 values");
    if (!rc) rc = take_fixed(fs, off, ng * 4, &sc, "Q8 scales");
    if (!rc) rc = take_fixed(fs, off, n16 * 4, &s16, "Q8 sums");
    if (!rc) rc = take_fixed(fs, off, n32 * 4, &s32, "Q8 sums");
    if (!rc) rc = take_fixed(fs, off, ng * 4, &s256, "Q8 sums");
    if (rc) return rc;
    out->q = (int8_t *)q;
    out->s = (float *)sc;
    out->sum16 = (int32_t *)s16;
    out->sum32 = (int32_t *)s32;
    out->sum256 = (int32_t *)s256;
    out->n = n;
    return HYQ_OK;
}

int matmul_dev(hyq_ctx *ctx, const hyq_weight *w, const float *x_d, size_t batch, float *y_d,
               const FixedScratch *fs)
{
    int rc = check_ctx_weight(ctx, w, "matmul");
    if (!rc) rc = check_matrix(w, "matmul");
    if (rc) return rc;
    if (batch == 0) return fail(HYQ_EINVAL, "%s: invalid activation shape", "matmul");
    if (!x_d || !y_d) return fail(HYQ_EINVAL, "matmul: null buffer");
    DeviceGuard g(ctx->device);
    // Q8_0 of a width the int8 GEMV (256-value groups) or the GEMM (64-column
    // slices) does not tile: the decoded-row path, as F32/F16
    const bool q80_odd = w->dtype == HYQ_Q8_0 && w->cols % (batch == 1 ? 256 : 64) != 0;
    if (is_raw(w->dtype) || q80_odd) {
        // decode rows to f32 + dot (src/quant.rs:225-267; batched :312-343)
        if (batch > 65535 * 64) return fail(HYQ_EINVAL, "matmul: batch %zu too large", batch);
        if (batch == 1)
            HYQ_LAUNCH(launch_f32_gemv(w->dtype, w->view, nullptr, (int)w->cols, x_d, y_d,
                                       ctx->stream),
                       "f32_gemv");
        else
            HYQ_LAUNCH(launch_f32_gemm(w->dtype, w->view, (int)w->cols, x_d, (int)batch, y_d,
                                       ctx->stream),
                       "f32_gemm");
        return HYQ_OK;
    }
    if (batch == 1) {
        rc = check_int8_path(w, "matmul");
        if (rc) return rc;
        if (can_stage(x_d, w->cols)) {
            GemvArgs a{};
            a.nseg = 1;
            a.seg[0].w = w->view;
            a.seg[0].y = y_d;
            a.rows_total = (int)w->rows;
            a.groups = (int)(w->cols / 256);
            a.xin = x_d;
            HYQ_LAUNCH(launch_gemv(w->dtype, GEMV_PLAIN, a, ctx->stream), "gemv");
            return HYQ_OK;
        }
        Q8Ref q8;
        size_t off = 0;
        rc = fs ? fixed_q8(*fs, off, w->cols, &q8) : ctx_q8(ctx, w->cols, &q8);
        if (!rc) rc = quantize_into(ctx, x_d, q8);
        if (!rc) rc = gemv_plain(ctx, w, q8, nullptr, y_d);
        return rc;
    }
    if (!is_quant(w->dtype)) return fail(HYQ_EDTYPE, "matmul: dtype %d has no batched path", w->dtype);
    if ((rc = check_f16_range(w, "matmul"))) return rc;
    // the GEMM walks K in 64-column slices and loads x as float4
    if (w->cols % 64) return fail(HYQ_EINVAL, "matmul: cols %zu is not a multiple of 64", w->cols);
    if ((uintptr_t)x_d % 16 || (uintptr_t)y_d % 16)
        return fail(HYQ_EINVAL, "matmul: device buffers must be 16-byte aligned");
    if (batch > 65535) return fail(HYQ_EINVAL, "matmul: batch %zu exceeds 65535", batch);
    // Q8_0 at up to 128 tokens: one register-operand launch (no K split)
    const bool few = w->dtype == Q8_0 && few_q80_fits((int)w->rows, (int)w->cols, (int)batch);
    const int ks = few ? 1 : matmul_kslices(w->dtype, (int)w->rows, (int)w->cols, (int)batch);
    // the 256-token tiles take their f16 rows in MFMA fragment order
    const bool frag =
        !few && gemm_frag_operand(w->dtype, (int)w->rows, (int)w->cols, (int)batch, ks);
    const size_t xh_bytes =
        align_up(few ? few_q80_operand_bytes((int)w->cols, (int)batch)
                     : (frag ? frag_rows((int)batch) : batch) * w->cols * 2,
                 256);
    const size_t part = ks > 1 ? (size_t)ks * batch * w->rows : 0;
    void *xh_mem = nullptr, *part_mem = nullptr;
    if (fs) {
        size_t off = 0;
        rc = take_fixed(*fs, off, xh_bytes + batch * 4, &xh_mem, "f16 activation rows");
        if (!rc && part) rc = take_fixed(*fs, off, part * 4, &part_mem, "K-slice partials");
        if (rc) return rc;
    } else {
        rc = ctx->xh.reserve(ctx->device, xh_bytes + batch * 4);
        if (!rc && part) rc = ctx->kpart.reserve(ctx->device, part * 4);
        if (rc) return rc;
        xh_mem = ctx->xh.ptr();
        part_mem = ctx->kpart.ptr();
    }
    _Float16 *xh = (_Float16 *)xh_mem;
    float *rscale = (float *)((uint8_t *)xh_mem + xh_bytes);
    if (few) {
        HYQ_LAUNCH(launch_few_q80(w->view, (int)w->cols, x_d, xh, rscale, (int)batch, y_d,
                                  ctx->stream),
                   "few_q80");
        return HYQ_OK;
    }
    HYQ_LAUNCH(launch_to_f16(x_d, (int)batch, (int)w->cols, xh, rscale, ctx->stream, frag),
               "to_f16");
    HYQ_LAUNCH(launch_gemm_f16(w->dtype, w->view, (int)w->cols, xh, rscale, (int)batch, y_d,
                               nullptr, ctx->stream, (float *)part_mem, part, ks, frag),
               "gemm_f16");
    return HYQ_OK;
}

} // namespace

// ---------------------------------------------------------------------------
// exported
// ---------------------------------------------------------------------------
extern "C" {

const char *hyq_last_error(void) { return hyq::g_last_error.c_str(); }
int hyq_block_len(int dtype) { return dtype_known(dtype) ? block_len(dtype) : -1; }
int hyq_block_bytes(int dtype) { return dtype_known(dtype) ? block_bytes(dtype) : -1; }

int hyq_ctx_create(int device, hyq_ctx **out)
{
    if (!out) return fail(HYQ_EINVAL, "hyq_ctx_create: null output");
    int count = 0;
    HYQ_HIP(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return fail(HYQ_EINVAL, "hyq_ctx_create: device %d of %d", device, count);
    DeviceGuard g(device);
    if (!g.ok) return fail(HYQ_EDEVICE, "hipSetDevice(%d) failed", device);
    auto ctx = std::make_unique<hyq_ctx>();
    ctx->device = device;
    // the no-allocation entry point's per-device scratch address
    int rc = resolve_scratch(device);
    if (rc) return rc;
    HYQ_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
    *out = ctx.release();
    return HYQ_OK;
}

void hyq_ctx_destroy(hyq_ctx *ctx)
{
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    delete ctx->q8;
    ctx->x.buf.reset();
    ctx->y.buf.reset();
    ctx->bytes.buf.reset();
    ctx->xh.buf.reset();
    ctx->moe.buf.reset();
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void *hyq_ctx_stream(hyq_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int hyq_ctx_set_q8_trace(hyq_ctx *ctx, void *trace_d, size_t bytes)
{
    if (!ctx) return fail(HYQ_EINVAL, "ctx_set_q8_trace: null context");
    if (trace_d && (uintptr_t)trace_d % 256)
        return fail(HYQ_EINVAL, "ctx_set_q8_trace: buffer must be 256-byte aligned");
    ctx->q8trace = Q8Trace{};
    if (trace_d) {
        ctx->q8trace.base = (uint8_t *)trace_d;
        ctx->q8trace.bytes = bytes;
    }
    return HYQ_OK;
}

int hyq_ctx_q8_trace_records(hyq_ctx *ctx, size_t *pairs, size_t max_records, size_t *count,
                             size_t *dropped)
{
    if (!ctx || !count) return fail(HYQ_EINVAL, "ctx_q8_trace_records: null argument");
    const Q8Trace &t = ctx->q8trace;
    *count = t.records.size();
    if (dropped) *dropped = t.dropped;
    if (pairs)
        for (size_t i = 0; i < t.records.size() && i < max_records; ++i) {
            pairs[2 * i] = t.records[i].first;
            pairs[2 * i + 1] = t.records[i].second;
        }
    return HYQ_OK;
}

int hyq_sync(hyq_ctx *ctx)
{
    if (!ctx) return fail(HYQ_EINVAL, "hyq_sync: null context");
    DeviceGuard g(ctx->device);
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_device_alloc(hyq_ctx *ctx, size_t bytes, void **ptr_d)
{
    if (!ctx || !ptr_d) return fail(HYQ_EINVAL, "hyq_device_alloc: null argument");
    DeviceGuard g(ctx->device);
    *ptr_d = nullptr;
    HYQ_HIP(hipMalloc(ptr_d, bytes ? bytes : 1), "hipMalloc");
    return HYQ_OK;
}

int hyq_device_free(hyq_ctx *ctx, void *ptr_d)
{
    if (!ctx) return fail(HYQ_EINVAL, "hyq_device_free: null context");
    if (!ptr_d) return HYQ_OK;
    DeviceGuard g(ctx->device);
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    HYQ_HIP(hipFree(ptr_d), "hipFree");
    return HYQ_OK;
}

int hyq_memcpy_h2d(hyq_ctx *ctx, void *dst_d, const void *src, size_t bytes)
{
    if (!ctx || (bytes && (!dst_d || !src))) return fail(HYQ_EINVAL, "hyq_memcpy_h2d: null");
    if (!bytes) return HYQ_OK;
    DeviceGuard g(ctx->device);
    HYQ_HIP(hipMemcpyAsync(dst_d, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_memcpy_d2h(hyq_ctx *ctx, void *dst, const void *src_d, size_t bytes)
{
    if (!ctx || (bytes && (!dst || !src_d))) return fail(HYQ_EINVAL, "hyq_memcpy_d2h: null");
    if (!bytes) return HYQ_OK;
    DeviceGuard g(ctx->device);
    HYQ_HIP(hipMemcpyAsync(dst, src_d, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_memcpy_d2d(hyq_ctx *ctx, void *dst_d, const void *src_d, size_t bytes)
{
    if (!ctx || (bytes && (!dst_d || !src_d))) return fail(HYQ_EINVAL, "hyq_memcpy_d2d: null");
    if (!bytes) return HYQ_OK;
    DeviceGuard g(ctx->device);
    HYQ_HIP(hipMemcpyAsync(dst_d, src_d, bytes, hipMemcpyDeviceToDevice, ctx->stream),
            "hipMemcpy");
    return HYQ_OK;
}

int hyq_weight_upload(hyq_ctx *ctx, int dtype, const uint8_t *gguf_bytes, size_t byte_len,
                      const uint64_t *dims, int rank, hyq_weight **out)
{
    if (!ctx || !out || !dims) return fail(HYQ_EINVAL, "hyq_weight_upload: null argument");
    if (!dtype_known(dtype)) return fail(HYQ_EDTYPE, "hyq_weight_upload: unknown dtype %d", dtype);
    if (rank != 2 && rank != 3) return fail(HYQ_EINVAL, "hyq_weight_upload: rank %d", rank);
    const uint64_t cols = dims[0], rows = dims[1], experts = rank == 3 ? dims[2] : 1;
    if (cols == 0 || rows == 0 || experts == 0)
        return fail(HYQ_EINVAL, "hyq_weight_upload: empty dimension");
    const int bl = block_len(dtype), bb = block_bytes(dtype);
    if (cols % (uint64_t)bl) return fail(HYQ_EINVAL, "partial %d output block", dtype);
    const uint64_t nb = cols / (uint64_t)bl;
    const uint64_t nblocks = nb * rows * experts;
    if (nblocks > (1ull << 40) || byte_len != nblocks * (uint64_t)bb)
        return fail(HYQ_EINVAL, "wrong byte count for dtype %d: %zu != %llu", dtype, byte_len,
                    (unsigned long long)(nblocks * (uint64_t)bb));
    if (!gguf_bytes) return fail(HYQ_EINVAL, "hyq_weight_upload: null bytes");
    // (every launch takes rows and columns as int)
    if (rows * experts > 0x7fffffffull || cols > 0x7fffffffull)
        return fail(HYQ_EINVAL, "hyq_weight_upload: shape too large");
    DeviceGuard g(ctx->device);

    size_t sz[3];
    for (int p = 0; p < 3; ++p) sz[p] = align_up(nblocks * (size_t)plane_bytes(dtype, p), 256);
    // A Q4_K expert stack also keeps its headers in 16-row tiles (plane 2,
    // which Q4_K does not otherwise use): the few-token expert kernels read
    // the headers of 16 rows of one superblock as 256 contiguous bytes.
    const bool q4k_tiles = dtype == Q4_K && rank == 3 && rows % 16 == 0;
    if (q4k_tiles) sz[2] = align_up(nblocks * 16, 256);
    auto storage = std::make_shared<DeviceBuffer>();
    storage->device = ctx->device;
    storage->bytes = sz[0] + sz[1] + sz[2];
    storage->ptr = pool_alloc(ctx->device, storage->bytes, &storage->chunk);
    if (!storage->ptr) return fail(HYQ_ENOMEM, "weight pool: out of device memory");
    int rc = ctx->bytes.reserve(ctx->device, byte_len);
    if (rc) return rc;
    uint8_t *stage = (uint8_t *)ctx->bytes.ptr();
    HYQ_HIP(hipMemcpyAsync(stage, gguf_bytes, byte_len, hipMemcpyHostToDevice, ctx->stream),
            "hipMemcpy(weight)");
    uint8_t *base = (uint8_t *)storage->ptr;
    HYQ_LAUNCH(launch_repack(dtype, stage, nblocks, (int)nb, base, base + sz[0],
                             base + sz[0] + sz[1], ctx->stream),
               "repack");
    if (q4k_tiles)
        HYQ_LAUNCH(launch_tile_headers(base + sz[0], (size_t)(rows * experts), (int)nb,
                                       base + sz[0] + sz[1], ctx->stream),
                   "tile_headers");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(upload)");

    auto w = std::make_unique<hyq_weight>();
    w->storage = storage;
    w->dtype = dtype;
    w->rank = rank;
    w->dims[0] = cols;
    w->dims[1] = rows;
    w->dims[2] = experts;
    w->cols = cols;
    w->rows = rows;
    w->device = ctx->device;
    w->view.p0 = base;
    w->view.p1 = base + sz[0];
    w->view.p2 = dtype == Q4_K && !q4k_tiles ? nullptr : base + sz[0] + sz[1];
    w->view.rows = (int)(rows * experts);
    w->view.nb = (int)nb;
    w->max_abs = weight_max_abs(dtype, gguf_bytes, nblocks);
    *out = w.release();
    return HYQ_OK;
}

int hyq_weight_expert(const hyq_weight *w, size_t e, hyq_weight **view)
{
    if (!w || !view) return fail(HYQ_EINVAL, "hyq_weight_expert: null argument");
    if (w->rank != 3 || e >= w->dims[2]) return fail(HYQ_EINVAL, "invalid expert %zu", e);
    auto v = std::make_unique<hyq_weight>(*w);
    v->rank = 2;
    v->dims[2] = 1;
    const size_t rows = w->dims[1], nb = (size_t)w->view.nb;
    v->view.p0 = w->view.p0 + e * rows * nb * plane_bytes(w->dtype, 0);
    v->view.p1 = w->view.p1 + e * rows * nb * plane_bytes(w->dtype, 1);
    // (a Q4_K stack's header tiles: 16 bytes per block, whole tiles per expert)
    const size_t p2b = w->dtype == Q4_K ? (w->view.p2 ? 16 : 0) : plane_bytes(w->dtype, 2);
    v->view.p2 = w->view.p2 ? w->view.p2 + e * rows * nb * p2b : nullptr;
    v->view.rows = (int)rows;
    *view = v.release();
    return HYQ_OK;
}

void hyq_weight_release(hyq_weight *w) { delete w; }

int hyq_weight_info(const hyq_weight *w, int *dtype, uint64_t *dims, int *rank)
{
    if (!w) return fail(HYQ_EINVAL, "hyq_weight_info: null weight");
    if (dtype) *dtype = w->dtype;
    if (rank) *rank = w->rank;
    if (dims)
        for (int i = 0; i < 3; ++i) dims[i] = w->dims[i];
    return HYQ_OK;
}

int hyq_q8_create(hyq_ctx *ctx, size_t n, hyq_q8 **out)
{
    if (!ctx || !out) return fail(HYQ_EINVAL, "hyq_q8_create: null argument");
    if (n == 0 || n > (1u << 30)) return fail(HYQ_EINVAL, "hyq_q8_create: length %zu", n);
    DeviceGuard g(ctx->device);
    hyq_q8 *q = nullptr;
    int rc = q8_alloc(ctx->device, n, &q);
    if (rc) return rc;
    *out = q;
    return HYQ_OK;
}

void hyq_q8_release(hyq_q8 *q8) { delete q8; }

int hyq_q8_buffers(const hyq_q8 *q8, int8_t **values_d, float **scales_d, size_t *n)
{
    if (!q8) return fail(HYQ_EINVAL, "hyq_q8_buffers: null");
    if (values_d) *values_d = q8->ref.q;
    if (scales_d) *scales_d = q8->ref.s;
    if (n) *n = q8->ref.n;
    return HYQ_OK;
}

int hyq_quantize_q8_d(hyq_ctx *ctx, const float *x_d, size_t n, hyq_q8 *q8)
{
    if (!ctx || !q8 || !x_d) return fail(HYQ_EINVAL, "hyq_quantize_q8_d: null argument");
    if (n != q8->ref.n) return fail(HYQ_EINVAL, "quantize: length %zu != %zu", n, q8->ref.n);
    DeviceGuard g(ctx->device);
    return quantize_into(ctx, x_d, q8->ref);
}

int hyq_gemv_q8_d(hyq_ctx *ctx, const hyq_weight *w, const hyq_q8 *x, const float *residual_d,
                  float *y_d)
{
    int rc = check_ctx_weight(ctx, w, "gemv_q8");
    if (!rc) rc = check_matrix(w, "gemv_q8");
    if (!rc) rc = check_int8_path(w, "gemv_q8");
    if (!rc) rc = check_q8(x, w->cols, "gemv_q8");
    if (rc) return rc;
    if (!y_d) return fail(HYQ_EINVAL, "gemv_q8: null output");
    DeviceGuard g(ctx->device);
    return gemv_plain(ctx, w, x->ref, residual_d, y_d);
}

int hyq_gemv_qkv_q8_d(hyq_ctx *ctx, const hyq_weight *q, const hyq_weight *k,
                      const hyq_weight *v, const hyq_q8 *x, float *yq_d, float *yk_d,
                      float *yv_d)
{
    int rc = check_ctx_weight(ctx, q, "gemv_qkv");
    if (!rc) rc = check_qkv(q, k, v);
    if (!rc) rc = check_int8_path(q, "gemv_qkv");
    if (!rc) rc = check_q8(x, q->cols, "gemv_qkv");
    if (rc) return rc;
    if (!yq_d || !yk_d || !yv_d) return fail(HYQ_EINVAL, "gemv_qkv: null output");
    DeviceGuard g(ctx->device);
    return gemv_qkv(ctx, q, k, v, x->ref, yq_d, yk_d, yv_d);
}

int hyq_gate_up_silu_q8_d(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                          const hyq_q8 *x, float *y_d)
{
    int rc = check_ctx_weight(ctx, gate, "gate_up_silu");
    if (!rc) rc = check_gate_up(gate, up);
    if (!rc) rc = check_int8_path(gate, "gate_up_silu");
    if (!rc) rc = check_q8(x, gate->cols, "gate_up_silu");
    if (rc) return rc;
    if (!y_d) return fail(HYQ_EINVAL, "gate_up_silu: null output");
    DeviceGuard g(ctx->device);
    return gate_up(ctx, gate, up, x->ref, y_d);
}

int hyq_isums_per_row(int dtype, size_t cols)
{
    const int per = isums_per_group(dtype);
    if (per < 0 || cols % 256) return -1;
    return (int)(cols / 256) * per;
}

int hyq_gemv_isums_d(hyq_ctx *ctx, const hyq_weight *w, const hyq_q8 *x, int32_t *isums_d)
{
    int rc = check_ctx_weight(ctx, w, "gemv_isums");
    if (!rc) rc = check_matrix(w, "gemv_isums");
    if (!rc) rc = check_int8_path(w, "gemv_isums");
    if (!rc) rc = check_q8(x, w->cols, "gemv_isums");
    if (rc) return rc;
    if (!isums_d) return fail(HYQ_EINVAL, "gemv_isums: null output");
    DeviceGuard g(ctx->device);
    GemvArgs a = base_args(w, x->ref);
    a.isums = isums_d;
    HYQ_LAUNCH(launch_gemv(w->dtype, GEMV_ISUMS, a, ctx->stream), "gemv_isums");
    return HYQ_OK;
}

int hyq_matmul_d(hyq_ctx *ctx, const hyq_weight *w, const float *x_d, size_t batch, float *y_d)
{
    return matmul_dev(ctx, w, x_d, batch, y_d, nullptr);
}

int hyq_matmul_noalloc_d(hyq_ctx *ctx, const hyq_weight *w, const float *x_d, size_t batch,
                         float *y_d)
{
    if (!ctx) return fail(HYQ_EINVAL, "matmul_noalloc: null context");
    FixedScratch fs{};
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        auto it = g_scratch.find(ctx->device);
        if (it == g_scratch.end() || !it->second)
            return fail(HYQ_EDEVICE, "matmul_noalloc: no scratch address for device %d",
                        ctx->device);
        fs.base = (uint8_t *)it->second;
    }
    fs.bytes = HYQ_NOALLOC_SCRATCH_BYTES;
    return matmul_dev(ctx, w, x_d, batch, y_d, &fs);
}

int hyq_hbm_read_d(hyq_ctx *ctx, const void *buf_d, size_t bytes, int workgroups,
                   float *sink_d)
{
    if (!ctx || !buf_d || !sink_d) return fail(HYQ_EINVAL, "hbm_read: null argument");
    if ((uintptr_t)buf_d % 16 || bytes < 16 || workgroups <= 0 || workgroups > (1 << 20))
        return fail(HYQ_EINVAL, "hbm_read: bad buffer or workgroup count");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_hbm_read(buf_d, bytes, workgroups, sink_d, ctx->stream), "hbm_read");
    return HYQ_OK;
}

int hyq_mfma_stream_d(hyq_ctx *ctx, int workgroups, int iters, float *sink_d)
{
    if (!ctx || !sink_d) return fail(HYQ_EINVAL, "mfma_stream: null argument");
    if (workgroups <= 0 || workgroups > (1 << 20) || iters <= 0 || iters > (1 << 24))
        return fail(HYQ_EINVAL, "mfma_stream: bad workgroup or iteration count");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_mfma_stream(workgroups, iters, sink_d, ctx->stream), "mfma_stream");
    return HYQ_OK;
}

int hyq_dequant_rows_d(hyq_ctx *ctx, const hyq_weight *w, size_t row0, size_t nrows,
                       float *out_d)
{
    int rc = check_ctx_weight(ctx, w, "dequant_rows");
    if (rc) return rc;
    if (!w) return fail(HYQ_EINVAL, "dequant_rows: null weight");
    if (row0 + nrows > (size_t)w->view.rows || row0 + nrows < row0)
        return fail(HYQ_EINVAL, "row %zu out of range", row0 + nrows);
    if (!out_d) return fail(HYQ_EINVAL, "dequant_rows: null output");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_dequant_rows(w->dtype, w->view, (int)row0, (int)nrows, (int)w->cols, out_d,
                                   ctx->stream),
               "dequant_rows");
    return HYQ_OK;
}

int hyq_decode_d(hyq_ctx *ctx, int dtype, const uint8_t *bytes_d, size_t byte_len, float *out_d,
                 size_t n)
{
    if (!ctx) return fail(HYQ_EINVAL, "decode: null context");
    if (!dtype_known(dtype)) return fail(HYQ_EDTYPE, "decode: unknown dtype %d", dtype);
    const size_t bl = (size_t)block_len(dtype), bb = (size_t)block_bytes(dtype);
    if (n % bl) return fail(HYQ_EINVAL, "partial %d output block", dtype);
    if (byte_len != n / bl * bb) return fail(HYQ_EINVAL, "wrong %d byte count", dtype);
    if (n && (!bytes_d || !out_d)) return fail(HYQ_EINVAL, "decode: null buffer");
    DeviceGuard g(ctx->device);
    HYQ_LAUNCH(launch_decode_gguf(dtype, bytes_d, n / bl, out_d, ctx->stream), "decode");
    return HYQ_OK;
}

// ---- host-pointer wrappers ----

int hyq_decode(hyq_ctx *ctx, int dtype, const uint8_t *bytes, size_t byte_len, float *out,
               size_t n)
{
    if (!ctx) return fail(HYQ_EINVAL, "decode: null context");
    if (!dtype_known(dtype)) return fail(HYQ_EDTYPE, "decode: unknown dtype %d", dtype);
    const size_t bl = (size_t)block_len(dtype), bb = (size_t)block_bytes(dtype);
    if (n % bl) return fail(HYQ_EINVAL, "partial %d output block", dtype);
    if (byte_len != n / bl * bb) return fail(HYQ_EINVAL, "wrong %d byte count", dtype);
    if (n == 0) return HYQ_OK;
    if (!bytes || !out) return fail(HYQ_EINVAL, "decode: null buffer");
    DeviceGuard g(ctx->device);
    int rc = ctx->bytes.reserve(ctx->device, byte_len);
    if (!rc) rc = ctx->y.reserve(ctx->device, n * 4);
    if (rc) return rc;
    HYQ_HIP(hipMemcpyAsync(ctx->bytes.ptr(), bytes, byte_len, hipMemcpyHostToDevice, ctx->stream),
            "hipMemcpy");
    HYQ_LAUNCH(launch_decode_gguf(dtype, (const uint8_t *)ctx->bytes.ptr(), n / bl,
                                  (float *)ctx->y.ptr(), ctx->stream),
               "decode");
    HYQ_HIP(hipMemcpyAsync(out, ctx->y.ptr(), n * 4, hipMemcpyDeviceToHost, ctx->stream),
            "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_weight_row(hyq_ctx *ctx, const hyq_weight *w, size_t row, float *out, size_t n)
{
    int rc = check_ctx_weight(ctx, w, "row_into");
    if (rc) return rc;
    if (!w || !out) return fail(HYQ_EINVAL, "row_into: null argument");
    if (n != w->cols) return fail(HYQ_EINVAL, "out buffer length mismatch");
    if (row >= (size_t)w->view.rows) return fail(HYQ_EINVAL, "row %zu out of range", row);
    DeviceGuard g(ctx->device);
    rc = ctx->y.reserve(ctx->device, n * 4);
    if (rc) return rc;
    HYQ_LAUNCH(launch_dequant_rows(w->dtype, w->view, (int)row, 1, (int)w->cols,
                                   (float *)ctx->y.ptr(), ctx->stream),
               "dequant_rows");
    HYQ_HIP(hipMemcpyAsync(out, ctx->y.ptr(), n * 4, hipMemcpyDeviceToHost, ctx->stream),
            "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_matmul(hyq_ctx *ctx, const hyq_weight *w, const float *x, size_t batch, float *y)
{
    int rc = check_ctx_weight(ctx, w, "matmul");
    if (!rc) rc = check_matrix(w, "matmul");
    if (rc) return rc;
    if (batch == 0 || !x || !y) return fail(HYQ_EINVAL, "matmul: invalid activation shape");
    DeviceGuard g(ctx->device);
    const size_t xin = batch * w->cols * 4, yout = batch * w->rows * 4;
    rc = ctx->x.reserve(ctx->device, xin);
    if (!rc) rc = ctx->y.reserve(ctx->device, yout);
    if (rc) return rc;
    HYQ_HIP(hipMemcpyAsync(ctx->x.ptr(), x, xin, hipMemcpyHostToDevice, ctx->stream), "hipMemcpy");
    rc = hyq_matmul_d(ctx, w, (const float *)ctx->x.ptr(), batch, (float *)ctx->y.ptr());
    if (rc) return rc;
    HYQ_HIP(hipMemcpyAsync(y, ctx->y.ptr(), yout, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_gemv_qkv(hyq_ctx *ctx, const hyq_weight *q, const hyq_weight *k, const hyq_weight *v,
                 const float *x, float *yq, float *yk, float *yv)
{
    int rc = check_ctx_weight(ctx, q, "gemv_qkv");
    if (!rc) rc = check_qkv(q, k, v);
    if (rc) return rc;
    if (!x || !yq || !yk || !yv) return fail(HYQ_EINVAL, "invalid activation shape for qkv");
    DeviceGuard g(ctx->device);
    const size_t cols = q->cols, nq = q->rows, nk = k->rows, nv = v->rows;
    rc = ctx->x.reserve(ctx->device, cols * 4);
    if (!rc) rc = ctx->y.reserve(ctx->device, (nq + nk + nv) * 4);
    if (rc) return rc;
    float *yd = (float *)ctx->y.ptr();
    const float *xd = (const float *)ctx->x.ptr();
    HYQ_HIP(hipMemcpyAsync(ctx->x.ptr(), x, cols * 4, hipMemcpyHostToDevice, ctx->stream),
            "hipMemcpy");
    if (is_raw(q->dtype)) {
        // three matmuls (src/quant.rs:716-720)
        const hyq_weight *ws[3] = {q, k, v};
        float *ys[3] = {yd, yd + nq, yd + nq + nk};
        for (int i = 0; i < 3; ++i)
            HYQ_LAUNCH(launch_f32_gemv(ws[i]->dtype, ws[i]->view, nullptr, (int)cols, xd, ys[i],
                                       ctx->stream),
                       "f32_gemv");
    } else {
        Q8Ref q8;
        rc = ctx_q8(ctx, cols, &q8);
        if (!rc) rc = quantize_into(ctx, xd, q8);
        if (!rc) rc = gemv_qkv(ctx, q, k, v, q8, yd, yd + nq, yd + nq + nk);
        if (rc) return rc;
    }
    HYQ_HIP(hipMemcpyAsync(yq, yd, nq * 4, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy");
    HYQ_HIP(hipMemcpyAsync(yk, yd + nq, nk * 4, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy");
    HYQ_HIP(hipMemcpyAsync(yv, yd + nq + nk, nv * 4, hipMemcpyDeviceToHost, ctx->stream),
            "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

int hyq_gate_up_silu(hyq_ctx *ctx, const hyq_weight *gate, const hyq_weight *up,
                     const float *x, float *y)
{
    int rc = check_ctx_weight(ctx, gate, "gate_up_silu");
    if (!rc) rc = check_gate_up(gate, up);
    if (rc) return rc;
    if (!x || !y) return fail(HYQ_EINVAL, "invalid activation shape for gate_up_silu");
    DeviceGuard g(ctx->device);
    const size_t cols = gate->cols, rows = gate->rows;
    rc = ctx->x.reserve(ctx->device, cols * 4);
    if (!rc) rc = ctx->y.reserve(ctx->device, rows * 4);
    if (rc) return rc;
    HYQ_HIP(hipMemcpyAsync(ctx->x.ptr(), x, cols * 4, hipMemcpyHostToDevice, ctx->stream),
            "hipMemcpy");
    if (is_raw(gate->dtype)) {
        // two matmuls and silu(g) * u (src/quant.rs:831-838)
        HYQ_LAUNCH(launch_f32_gemv(gate->dtype, gate->view, &up->view, (int)cols,
                                   (const float *)ctx->x.ptr(), (float *)ctx->y.ptr(),
                                   ctx->stream),
                   "f32_gate_up");
    } else {
        Q8Ref q8;
        rc = ctx_q8(ctx, cols, &q8);
        if (!rc) rc = quantize_into(ctx, (const float *)ctx->x.ptr(), q8);
        if (!rc) rc = gate_up(ctx, gate, up, q8, (float *)ctx->y.ptr());
        if (rc) return rc;
    }
    HYQ_HIP(hipMemcpyAsync(y, ctx->y.ptr(), rows * 4, hipMemcpyDeviceToHost, ctx->stream),
            "hipMemcpy");
    HYQ_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return HYQ_OK;
}

} // extern "C"
