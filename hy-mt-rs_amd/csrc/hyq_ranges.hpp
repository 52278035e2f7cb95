// Sub-allocation of one pool chunk: a bump pointer plus a free list of
// released ranges, reused first-fit and coalesced with their neighbours; a
// free range that reaches the bump pointer lowers it. Pure bookkeeping (no
// device calls), so it is unit-tested on the host.
#pragma once

#include <stddef.h>

#include <utility>
#include <vector>

namespace hyq {

struct Ranges {
    size_t size = 0; // bytes the chunk holds
    size_t top = 0;  // everything at or above top is free
    // released ranges below top: (offset, length), sorted, disjoint, not adjacent
    std::vector<std::pair<size_t, size_t>> free;

    // Takes `need` bytes: the first free range that holds them, else the top.
    bool take(size_t need, size_t *off)
    {
        for (size_t i = 0; i < free.size(); ++i)
            if (free[i].second >= need) {
                *off = free[i].first;
                free[i].first += need;
                free[i].second -= need;
                if (free[i].second == 0) free.erase(free.begin() + (long)i);
                return true;
            }
        if (size - top < need) return false;
        *off = top;
        top += need;
        return true;
    }

    // Returns [off, off + len) taken earlier.
    void give(size_t off, size_t len)
    {
        size_t i = 0;
        while (i < free.size() && free[i].first < off) ++i;
        free.insert(free.begin() + (long)i, {off, len});
        // merge with the next range, then with the previous one
        if (i + 1 < free.size() && free[i].first + free[i].second == free[i + 1].first) {
            free[i].second += free[i + 1].second;
            free.erase(free.begin() + (long)i + 1);
        }
        if (i > 0 && free[i - 1].first + free[i - 1].second == free[i].first) {
            free[i - 1].second += free[i].second;
            free.erase(free.begin() + (long)i);
            --i;
        }
        if (free[i].first + free[i].second == top) {
            top = free[i].first;
            free.erase(free.begin() + (long)i);
        }
    }
};

} // namespace hyq
