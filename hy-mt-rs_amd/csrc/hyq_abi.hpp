// Internal state behind the C ABI handles, shared by hyq_api.cpp and
// hyq_dense.cpp (not installed; include/hyq.h is the public boundary).
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../include/hyq.h"
#include "hyq_internal.hpp"

namespace hyq {

// Records a thread-local message for hyq_last_error and returns code.
int fail(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);

#define HYQ_HIP(call, what)                                                                    \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) return ::hyq::hip_fail(e_, what);                                \
    } while (0)

#define HYQ_LAUNCH(call, what)                                                                 \
    do {                                                                                       \
        int e_ = (call);                                                                       \
        if (e_ != 0) return ::hyq::hip_fail((hipError_t)e_, what);                             \
    } while (0)

// Makes the context's device current for the scope of one call.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev)
    {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard()
    {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Weight storage comes from large per-device pool chunks (hyq_pool.cpp):
// packing a model's tensors into a few big, 2 MiB-aligned allocations keeps
// them on large-page mappings, so the first touch of a tensor by a kernel
// does not walk page tables for every few kilobytes.
struct PoolChunk;
void *pool_alloc(int device, size_t bytes, PoolChunk **chunk);
// Returns [ptr, ptr + bytes) that pool_alloc(.., bytes, &chunk) gave.
void pool_release(PoolChunk *chunk, void *ptr, size_t bytes);

struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    int device = 0;
    PoolChunk *chunk = nullptr; // set when ptr lives in a pool chunk
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    ~DeviceBuffer()
    {
        if (chunk) {
            pool_release(chunk, ptr, bytes);
        } else if (ptr) {
            DeviceGuard g(device);
            (void)hipFree(ptr);
        }
    }
    int alloc(int dev, size_t n)
    {
        device = dev;
        bytes = n;
        hipError_t e = hipMalloc(&ptr, n ? n : 1);
        if (e != hipSuccess) {
            ptr = nullptr;
            return hip_fail(e, "hipMalloc");
        }
        return HYQ_OK;
    }
};

// Grow-only device scratch owned by a context.
struct Scratch {
    std::unique_ptr<DeviceBuffer> buf;
    int reserve(int device, size_t bytes)
    {
        if (buf && buf->bytes >= bytes) return HYQ_OK;
        buf.reset();
        auto b = std::make_unique<DeviceBuffer>();
        int rc = b->alloc(device, align_up(bytes < 4096 ? 4096 : bytes, 4096));
        if (rc) return rc;
        buf = std::move(b);
        return HYQ_OK;
    }
    void *ptr() const { return buf ? buf->ptr : nullptr; }
};

// Non-owning Q8 buffers (a hyq_q8 or a prefix of the context's own).
struct Q8Ref {
    int8_t *q = nullptr;
    float *s = nullptr;
    int32_t *sum16 = nullptr, *sum32 = nullptr, *sum256 = nullptr;
    size_t n = 0;
    Q8View view() const { return Q8View{q, s, sum16, sum32, sum256, (int)n}; }
    Q8Ref prefix(size_t len) const
    {
        Q8Ref r = *this;
        r.n = len;
        return r;
    }
};

// The Q8 record of a context (hyq_ctx_set_q8_trace, a test hook): each
// traced launch takes the next record of n values (a multiple of 256):
// n int8 codes, n / 256 f32 scales, then (from the next 256-byte boundary)
// the n f32 values that were quantized; every record starts on a 256-byte
// boundary. Records that do not fit are counted and dropped.
struct Q8Trace {
    uint8_t *base = nullptr;
    size_t bytes = 0, used = 0, dropped = 0;
    std::vector<std::pair<size_t, size_t>> records; // (offset, n)
    // the next record of n values, or false
    bool take(size_t n, int8_t **codes, float **scales, float **values);
};
// Gives a launch with an f32 input stage its record (when t is set): the
// launch's groups over all of its K slices or slots.
void q8_trace_gemv(Q8Trace *t, GemvArgs &a);
// Records the first n values of a Q8 row already in device memory and the
// f32 row x it was quantized from (copies on st; t may be null).
int q8_trace_copy(Q8Trace *t, const Q8Ref &q, const float *x, size_t n, hipStream_t st);

int q8_alloc(int device, size_t n, hyq_q8 **out);
// Hands a weight to a dense decoder, which releases it when destroyed (the
// weights a GGUF loader uploads for it).
void dense_adopt(hyq_dense *m, hyq_weight *w);

} // namespace hyq

struct hyq_q8 {
    std::unique_ptr<hyq::DeviceBuffer> mem;
    int device = 0;
    hyq::Q8Ref ref;
};

struct hyq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hyq::Scratch x, y, bytes, xh, moe, kpart; // kpart: K-slice partials of batched products
    hyq_q8 *q8 = nullptr; // grown on demand for host-pointer calls
    hyq::Q8Trace q8trace;  // hyq_ctx_set_q8_trace
    // the record the traced launches use (null while the trace is off)
    hyq::Q8Trace *q8t() { return q8trace.base ? &q8trace : nullptr; }
};

struct hyq_weight {
    std::shared_ptr<hyq::DeviceBuffer> storage;
    int dtype = 0;
    int rank = 2;
    uint64_t dims[3] = {0, 0, 1};
    size_t cols = 0, rows = 0;
    int device = 0;
    hyq::WView view{};
    // an upper bound of |value| over the tensor (all experts), from its
    // scales at upload; the f16-MFMA products need it inside f16's range
    float max_abs = 0.f;
};

namespace hyq {
// Bound of |decoded value| over n blocks of GGUF bytes (host memory).
float weight_max_abs(int dtype, const uint8_t *bytes, size_t nblocks);
// HYQ_EINVAL unless the tensor's values fit the f16 operands of the batched
// products: none above f16's largest finite value, and not all of them
// below its smallest normal (an all-zero tensor is fine).
int check_f16_range(const hyq_weight *w, const char *who);
} // namespace hyq
