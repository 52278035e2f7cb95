// Per-device pool of large allocations for weight storage.
//
// Tensors are bump-allocated (256-byte aligned) from chunks of at least
// 1 GiB, each a single 2 MiB-aligned hipMalloc, so that a model's weights
// sit in a few large mappings. A chunk is freed when the last tensor placed
// in it is released; space inside a live chunk is not reused.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "hyq_abi.hpp"

namespace hyq {

struct PoolChunk {
    int device;
    uint8_t *base;
    size_t size, used;
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
    for (PoolChunk *c : g_chunks)
        if (c->device == device && c->size - c->used >= need) {
            void *p = c->base + c->used;
            c->used += need;
            c->refs += 1;
            *chunk = c;
            return p;
        }
    const size_t size = align_up(need > CHUNK_MIN ? need : CHUNK_MIN, PAGE);
    DeviceGuard g(device);
    void *base = nullptr;
    if (hipMalloc(&base, size) != hipSuccess) return nullptr;
    auto *c = new PoolChunk{device, (uint8_t *)base, size, need, 1};
    g_chunks.push_back(c);
    *chunk = c;
    return base;
}

void pool_release(PoolChunk *c)
{
    std::lock_guard<std::mutex> lk(g_mu);
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
