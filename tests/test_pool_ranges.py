"""CPU test of the weight pool's chunk bookkeeping (hy-mt-rs_amd/csrc/
hyq_ranges.hpp): first-fit reuse of released ranges, coalescing, the bump
pointer lowered when the top range is released, and a full chunk refusing.
The header is pure host code; the test compiles it with g++ into a small
program that replays allocation scripts against a brute-force byte map."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "hy-mt-rs_amd", "csrc", "hyq_ranges.hpp")

PROGRAM = r'''
#include "HEADER"
#include <cstdio>
#include <cstdlib>
#include <vector>
using hyq::Ranges;
// A chunk of 64 units; each operation is checked against a byte map.
static int fails = 0;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL line %d\n", __LINE__); ++fails; } } while (0)
struct Model {
    Ranges r; std::vector<int> owner;
    explicit Model(size_t n) { r.size = n; owner.assign(n, 0); }
    bool take(size_t need, int id, size_t *off) {
        if (!r.take(need, off)) return false;
        for (size_t i = *off; i < *off + need; ++i) { CHECK(owner[i] == 0); owner[i] = id; }
        return true;
    }
    void give(size_t off, size_t len, int id) {
        for (size_t i = off; i < off + len; ++i) { CHECK(owner[i] == id); owner[i] = 0; }
        r.give(off, len);
        // invariants: sorted, disjoint, non-adjacent, below top; bytes >= top are free
        for (size_t k = 0; k < r.free.size(); ++k) {
            CHECK(r.free[k].second > 0);
            if (k) CHECK(r.free[k - 1].first + r.free[k - 1].second < r.free[k].first);
        }
        if (!r.free.empty()) CHECK(r.free.back().first + r.free.back().second < r.top);
        for (size_t i = r.top; i < owner.size(); ++i) CHECK(owner[i] == 0);
    }
};
int main() {
    Model m(64);
    size_t a, b, c, d, e;
    CHECK(m.take(16, 1, &a) && a == 0);
    CHECK(m.take(16, 2, &b) && b == 16);
    CHECK(m.take(16, 3, &c) && c == 32);
    CHECK(!m.take(32, 9, &e));            // only 16 left at the top
    m.give(b, 16, 2);                      // a hole in the middle
    CHECK(m.take(8, 4, &d) && d == 16);   // first fit reuses it
    CHECK(m.take(8, 5, &e) && e == 24);
    m.give(d, 8, 4);
    m.give(e, 8, 5);                       // coalesced back to [16, 32)
    CHECK(m.r.free.size() == 1 && m.r.free[0].first == 16 && m.r.free[0].second == 16);
    m.give(c, 16, 3);                      // [16, 48) reaches the top: top drops to 16
    CHECK(m.r.top == 16 && m.r.free.empty());
    CHECK(m.take(48, 6, &e) && e == 16);  // the whole rest is one range again
    m.give(a, 16, 1);
    m.give(e, 48, 6);
    CHECK(m.r.top == 0 && m.r.free.empty());
    // random scripts against the byte map
    std::srand(7);
    for (int round = 0; round < 200; ++round) {
        Model r(256);
        std::vector<std::pair<size_t, size_t>> live;
        int id = 1;
        for (int op = 0; op < 200; ++op) {
            if (live.empty() || std::rand() % 3) {
                size_t need = 1 + std::rand() % 40, off;
                if (r.take(need, id, &off)) live.push_back({off, need}), ++id;
            } else {
                size_t k = std::rand() % live.size();
                r.give(live[k].first, live[k].second, r.owner[live[k].first]);
                live.erase(live.begin() + (long)k);
            }
        }
        for (auto &x : live) r.give(x.first, x.second, r.owner[x.first]);
        CHECK(r.r.top == 0 && r.r.free.empty());
    }
    std::printf(fails ? "failed\n" : "ok\n");
    return fails ? 1 : 0;
}
'''


def test_chunk_ranges(tmp_path):
    src = tmp_path / "ranges_test.cpp"
    src.write_text(PROGRAM.replace("HEADER", HEADER))
    exe = tmp_path / "ranges_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout
