// Host tests of the block-granular pool's bookkeeping (BlockAllocator).
// Built with g++ (address and undefined-behaviour sanitizers) and run by
// tests/test_block_allocator.py; prints one line per test and exits non-zero
// on the first failed check.
//
// The randomized test follows the reference's property tests of the slot
// allocator (tests/test_kv_cache.cpp:298-440: allocation, release, memory
// and exhaustion invariants), restated for blocks.
#include "block_allocator.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <stdexcept>
#include <vector>

using tiny_llm::detail::BlockAllocator;

#define CHECK(c)                                                                  \
    do {                                                                          \
        if (!(c)) {                                                               \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #c); \
            std::exit(1);                                                         \
        }                                                                         \
    } while (0)

static void fresh_pool_is_empty() {
    BlockAllocator a(3, 4, 5);
    CHECK(a.freeBlocks() == 5 && a.usedBlocks() == 0 && a.spare() == 5);
    for (int32_t v : a.table()) CHECK(v == 5);
    for (int r = 0; r < 3; ++r) CHECK(a.mapped(r) == 0);
    CHECK(!a.hasUpdates());
}

static void ensure_maps_in_order_and_records_updates() {
    BlockAllocator a(2, 4, 6);
    CHECK(a.ensure(1, 3));
    CHECK(a.mapped(1) == 3 && a.freeBlocks() == 3);
    CHECK(a.table()[4] == 0 && a.table()[5] == 1 && a.table()[6] == 2 && a.table()[7] == 6);
    CHECK(a.ensure(1, 2));  // already covered: no change
    CHECK(a.mapped(1) == 3 && a.freeBlocks() == 3);
    auto u = a.takeUpdates();
    CHECK(u.size() == 3);
    CHECK(u[0].first == 4 && u[0].second == 0 && u[2].first == 6 && u[2].second == 2);
    CHECK(!a.hasUpdates());
    CHECK(a.ensure(0, 1) && a.table()[0] == 3);
}

static void ensure_is_all_or_nothing() {
    BlockAllocator a(2, 8, 4);
    CHECK(a.ensure(0, 3));
    (void)a.takeUpdates();
    CHECK(!a.ensure(1, 2));  // only one block free
    CHECK(a.mapped(1) == 0 && a.freeBlocks() == 1 && !a.hasUpdates());
    CHECK(!a.ensure(0, 9));  // beyond the row
    CHECK(!a.ensure(-1, 1) && !a.ensure(2, 1));
    CHECK(a.ensure(1, 1) && a.freeBlocks() == 0);
}

static void release_returns_blocks_and_resets_entries() {
    BlockAllocator a(2, 4, 4);
    CHECK(a.ensure(0, 2) && a.ensure(1, 2));
    (void)a.takeUpdates();
    a.release(0);
    CHECK(a.mapped(0) == 0 && a.freeBlocks() == 2);
    CHECK(a.table()[0] == 4 && a.table()[1] == 4);
    auto u = a.takeUpdates();
    CHECK(u.size() == 2);
    for (auto &p : u) CHECK(p.second == 4);
    // The released row's first block is handed out first again.
    CHECK(a.ensure(1, 3) && a.table()[6] == 0);
    a.release(1);
    a.release(1);  // releasing an empty row is a no-op
    CHECK(a.freeBlocks() == 4);
}

static void updates_coalesce_to_the_final_value() {
    BlockAllocator a(2, 2, 2);
    CHECK(a.ensure(0, 2));
    a.release(0);
    CHECK(a.ensure(1, 1));
    auto u = a.takeUpdates();
    CHECK(u.size() == 3);  // entries 0, 1 (back to spare) and 2
    std::vector<int32_t> mirror(4, 2);
    for (auto &p : u) mirror[static_cast<size_t>(p.first)] = p.second;
    CHECK(mirror == a.table());
}

static void shortfall_counts_missing_blocks() {
    BlockAllocator a(3, 4, 5);
    CHECK(a.ensure(0, 2));
    const int rows[3] = {0, 1, 2}, blocks[3] = {3, 2, 1};
    CHECK(a.shortfall(rows, blocks, 3) == (1 + 2 + 1) - 3);
    const int blocks2[3] = {1, 1, 1};
    CHECK(a.shortfall(rows, blocks2, 3) == 2 - 3);
}

static void invalid_geometry_throws() {
    int thrown = 0;
    for (auto g : {std::vector<int>{0, 1, 1}, {1, 0, 1}, {1, 1, 0}, {-1, 2, 2}}) {
        try {
            BlockAllocator a(g[0], g[1], g[2]);
        } catch (const std::invalid_argument &) {
            ++thrown;
        }
    }
    CHECK(thrown == 4);
}

// Random ensure / release / takeUpdates; after every op:
//  - mapped entries of each row are non-spare, the rest are spare;
//  - no block is mapped twice, and mapped + free covers every block once;
//  - used + free == num_blocks, used == sum of mapped counts;
//  - a device mirror patched with the updates equals the host table.
static void random_operations_keep_invariants() {
    for (int seed = 0; seed < 20; ++seed) {
        std::mt19937 rng(static_cast<unsigned>(seed));
        const int    rows = 1 + static_cast<int>(rng() % 12), bpr = 1 + static_cast<int>(rng() % 16);
        const int    nb = 1 + static_cast<int>(rng() % (rows * bpr + 4));
        BlockAllocator       a(rows, bpr, nb);
        std::vector<int32_t> mirror(a.table());
        for (int op = 0; op < 3000; ++op) {
            const int r = static_cast<int>(rng() % static_cast<unsigned>(rows));
            const int kind = static_cast<int>(rng() % 10);
            if (kind < 6) {
                const int want = static_cast<int>(rng() % static_cast<unsigned>(bpr + 2));
                const int before = a.mapped(r), free_before = a.freeBlocks();
                const bool ok = a.ensure(r, want);
                const bool fits = want <= bpr && (want <= before || want - before <= free_before);
                CHECK(ok == fits);
                CHECK(a.mapped(r) == (ok ? std::max(before, want) : before));
            } else if (kind < 8) {
                a.release(r);
                CHECK(a.mapped(r) == 0);
            } else {
                for (auto &p : a.takeUpdates()) mirror[static_cast<size_t>(p.first)] = p.second;
                CHECK(mirror == a.table());
            }
            std::set<int32_t> seen;
            int               used = 0;
            for (int rr = 0; rr < rows; ++rr) {
                for (int j = 0; j < bpr; ++j) {
                    const int32_t v = a.table()[static_cast<size_t>(rr * bpr + j)];
                    if (j < a.mapped(rr)) {
                        CHECK(v >= 0 && v < nb);
                        CHECK(seen.insert(v).second);
                    } else {
                        CHECK(v == nb);
                    }
                }
                used += a.mapped(rr);
            }
            CHECK(used == a.usedBlocks() && a.usedBlocks() + a.freeBlocks() == nb);
        }
        // Exhaustion: fill every row as far as blocks last, then release all.
        for (int r = 0; r < rows; ++r) a.release(r);
        int mapped = 0;
        for (int r = 0; r < rows; ++r)
            while (a.ensure(r, a.mapped(r) + 1)) ++mapped;
        CHECK(mapped == std::min(nb, rows * bpr) && a.freeBlocks() == nb - mapped);
        for (int r = 0; r < rows; ++r) a.release(r);
        CHECK(a.freeBlocks() == nb);
    }
}

int main() {
    struct {
        const char *name;
        void (*fn)();
    } tests[] = {
        {"fresh_pool_is_empty", fresh_pool_is_empty},
        {"ensure_maps_in_order_and_records_updates", ensure_maps_in_order_and_records_updates},
        {"ensure_is_all_or_nothing", ensure_is_all_or_nothing},
        {"release_returns_blocks_and_resets_entries", release_returns_blocks_and_resets_entries},
        {"updates_coalesce_to_the_final_value", updates_coalesce_to_the_final_value},
        {"shortfall_counts_missing_blocks", shortfall_counts_missing_blocks},
        {"invalid_geometry_throws", invalid_geometry_throws},
        {"random_operations_keep_invariants", random_operations_keep_invariants},
    };
    for (auto &t : tests) {
        t.fn();
        std::printf("ok %s\n", t.name);
    }
    return 0;
}
