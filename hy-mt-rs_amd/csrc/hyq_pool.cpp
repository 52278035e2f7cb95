// Per-device pool of large allocations for weight storage.
//
// Tensors are placed (256-byte aligned) in chunks of at least 1 GiB, each a
// single 2 MiB-aligned hipMalloc, so that a model's weights sit in a few
// large mappings. Inside a chunk, released tensors' space is reused
// first-fit (hyq_ranges.hpp); a chunk is freed when its last tensor is
// released. When a 1 GiB chunk cannot be had, a chunk of the tensor's own
// size is tried before failing.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "hyq_abi.hpp"
#include "hyq_ranges.hpp"

namespace hyq {

struct PoolChunk {
    int device;
    uint8_t *base;
    Ranges ranges;
    int refs;
};

namespace {
std::mutex g_mu;
std::vector<PoolChunk *> g_chunks;
constexpr size_t CHUNK_MIN = size_t(1) << 30;
constexpr size_t PAGE = size_t(2) << 20;
} // namespace

void *pool_alloc(int device, size_t bytes, PoolChunk **chunk)
{
    const size_t need = align_up(bytes ? bytes : 1, 256);
    std::lock_guard<std::mutex> lk(g_mu);
    for (PoolChunk *c : g_chunks) {
        size_t off;
        if (c->device == device && c->ranges.take(need, &off)) {
            c->refs += 1;
            *chunk = c;
            return c->base + off;
        }
    }
    DeviceGuard g(device);
    void *base = nullptr;
    size_t size = align_up(need > CHUNK_MIN ? need : CHUNK_MIN, PAGE);
    if (hipMalloc(&base, size) != hipSuccess) {
        (void)hipGetLastError(); // clear the failed allocation's error
        size = align_up(need, PAGE);
        if (hipMalloc(&base, size) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    auto *c = new PoolChunk{device, (uint8_t *)base, Ranges{}, 1};
    c->ranges.size = size;
    size_t off;
    c->ranges.take(need, &off); // off == 0
    g_chunks.push_back(c);
    *chunk = c;
    return base;
}

void pool_release(PoolChunk *c, void *ptr, size_t bytes)
{
    std::lock_guard<std::mutex> lk(g_mu);
    c->ranges.give((size_t)((uint8_t *)ptr - c->base), align_up(bytes ? bytes : 1, 256));
    if (--c->refs > 0) return;
    for (size_t i = 0; i < g_chunks.size(); ++i)
        if (g_chunks[i] == c) {
            g_chunks.erase(g_chunks.begin() + (long)i);
            break;
        }
    DeviceGuard g(c->device);
    (void)hipFree(c->base);
    delete c;
}

} // namespace hyq
