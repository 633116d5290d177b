// CPU check of the stream-K partition arithmetic of the 8-wave prefill (mx_kernels.hpp: prefill_tile_blocks, sk_lo,
// sk_range_of, sk_locate, sk_slot), over many launch shapes and range counts. It walks every range's segments exactly as
// prefill_sk_kernel does and checks: each unit belongs to exactly one segment; sk_locate returns the tile holding the
// unit; a tile split between ranges has its segments in the ranges sk_range_of names for its first and last unit, each
// in the slot the merging range computes for it; no two partial segments share a slot. Exit status 0 when all hold.
#include <cstdio>
#include <map>
#include <set>
#include <vector>

#include "mx_kernels.hpp"

static int failures = 0;
#define CHECK(c, ...)                                  \
    do {                                               \
        if (!(c)) {                                    \
            if (failures++ < 20) {                     \
                std::printf("FAIL %s: ", #c);          \
                std::printf(__VA_ARGS__);              \
                std::printf("\n");                     \
            }                                          \
        }                                              \
    } while (0)

static void check_shape(int n_q, int p0, int n_kv, int causal, int n_head, int group, int ranges) {
    const int n_qtiles = (n_q + mx::kPrefillSkRows - 1) / mx::kPrefillSkRows;
    const int n_kvh = n_head / group;
    // tiles in launch order (kv head, query tile, head of the group)
    std::vector<int64_t> start;
    std::vector<int> nblk;
    int64_t total = 0;
    for (int kvh = 0; kvh < n_kvh; kvh++)
        for (int qt = 0; qt < n_qtiles; qt++)
            for (int gi = 0; gi < group; gi++) {
                start.push_back(total);
                nblk.push_back(mx::prefill_tile_blocks(qt, n_q, p0, n_kv, causal));
                total += nblk.back();
            }
    if (total < ranges) return;  // the plan never runs such a launch
    int64_t per_kv = 0;
    for (int q = 0; q < n_qtiles; q++) per_kv += mx::prefill_tile_blocks(q, n_q, p0, n_kv, causal);
    per_kv *= group;
    std::vector<int> covered(total, 0);
    std::map<int64_t, std::set<std::pair<int, int64_t>>> parts;  // tile -> (range, slot) of its partial segments
    std::set<int64_t> used_slots;
    for (int r = 0; r < ranges; r++) {
        const int64_t lo = mx::sk_lo(total, ranges, r), hi = mx::sk_lo(total, ranges, r + 1);
        CHECK(hi > lo, "empty range %d (total %lld, ranges %d)", r, (long long)total, ranges);
        for (int64_t x = lo; x < hi;) {
            const mx::SkTile t = mx::sk_locate(x, per_kv, group, n_qtiles, n_q, p0, n_kv, causal);
            const int64_t tile = ((int64_t)t.kvh * n_qtiles + t.qt) * group + t.gi;
            CHECK(tile >= 0 && tile < (int64_t)start.size(), "tile %lld out of range", (long long)tile);
            if (tile < 0 || tile >= (int64_t)start.size()) return;
            CHECK(t.start == start[tile] && t.nblk == nblk[tile] && x >= t.start && x < t.start + t.nblk,
                  "locate(%lld): tile %lld start %lld nblk %d", (long long)x, (long long)tile, (long long)t.start, t.nblk);
            const int ib0 = (int)(x - t.start), ib1 = (int)(hi - t.start < t.nblk ? hi - t.start : t.nblk);
            for (int b = ib0; b < ib1; b++) covered[t.start + b]++;
            if (ib0 != 0 || ib1 != t.nblk) {
                const int64_t slot = mx::sk_slot(total, ranges, r, t.start);
                CHECK(slot >= 0 && slot < 2 * (int64_t)ranges, "slot %lld", (long long)slot);
                CHECK(used_slots.insert(slot).second, "slot %lld used twice", (long long)slot);
                parts[tile].insert({r, slot});
            }
            CHECK(ib1 > ib0, "empty segment");
            if (ib1 <= ib0) return;
            x = t.start + ib1;
        }
    }
    for (int64_t u = 0; u < total; u++) CHECK(covered[u] == 1, "unit %lld covered %d times", (long long)u, covered[u]);
    for (const auto & kv : parts) {
        const int64_t s = start[kv.first];
        const int rf = mx::sk_range_of(total, ranges, s), rl = mx::sk_range_of(total, ranges, s + nblk[kv.first] - 1);
        std::set<std::pair<int, int64_t>> want;
        for (int r = rf; r <= rl; r++) want.insert({r, mx::sk_slot(total, ranges, r, s)});
        CHECK(want == kv.second && rl > rf, "tile %lld: %zu segments, ranges %d..%d", (long long)kv.first, kv.second.size(), rf, rl);
    }
}

int main() {
    int shapes = 0;
    const int heads[][2] = {{28, 7}, {32, 4}, {14, 7}, {20, 1}, {8, 8}, {40, 5}};
    for (const auto & hg : heads)
        for (int n_q : {1, 255, 256, 257, 700, 2048, 3000, 4096})
            for (int p0 : {0, 1, 63, 64, 1000, 30720})
                for (int causal : {0, 1})
                    for (int extra : {0, 37})
                        for (int ranges : {8, 64, 256}) {
                            check_shape(n_q, p0, p0 + n_q + extra, causal, hg[0], hg[1], ranges);
                            shapes++;
                        }
    std::printf("%d shapes, %d failures\n", shapes, failures);
    return failures ? 1 : 0;
}
