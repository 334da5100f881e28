// CPU check of llm-kv260_amd/csrc/pool_ranges.h, the udmabuf pools'
// host-current ranges: random adds and removes over a small pool, each
// followed by a check of the set against a byte map kept beside it (the set
// disjoint, sorted, merged, and holding exactly the marked bytes) and of
// parts() inside and outside random windows against the same map.
//
//   pool_ranges_sim <pool bytes> <operations> <seed> <plant>
//     plant: 1 = add() without merging a range that only touches its
//            neighbour (a planted mistake the check must catch)
// Prints "ops N ok" and exits 0, or names the first mismatch and exits 1.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "pool_ranges.h"

using namespace w4a8;

static bool g_plant = false;

static void add_planted(pool_ranges::Set &m, size_t a, size_t b) {
    // Merges overlaps only, not ranges that merely touch: the set then holds
    // two adjacent ranges, which the merged-set check rejects.
    auto it = m.upper_bound(a);
    if (it != m.begin()) {
        auto p = std::prev(it);
        if (p->second > a) {
            a = p->first;
            b = b > p->second ? b : p->second;
            m.erase(p);
        }
    }
    while (it != m.end() && it->first < b) {
        b = b > it->second ? b : it->second;
        it = m.erase(it);
    }
    m.emplace(a, b);
}

static bool check(const pool_ranges::Set &m, const std::vector<char> &bytes, const char *after, long op) {
    size_t prev_end = 0;
    bool first = true;
    std::vector<char> got(bytes.size(), 0);
    for (const auto &r : m) {
        if (r.first >= r.second || r.second > bytes.size() || (!first && r.first <= prev_end)) {
            std::printf("op %ld (%s): bad or unmerged range [%zu, %zu)\n", op, after, r.first, r.second);
            return false;
        }
        for (size_t i = r.first; i < r.second; ++i) got[i] = 1;
        prev_end = r.second;
        first = false;
    }
    if (got != bytes) {
        std::printf("op %ld (%s): set differs from the byte map\n", op, after);
        return false;
    }
    return true;
}

static bool check_parts(const pool_ranges::Set &m, const std::vector<char> &bytes, size_t a, size_t b, long op) {
    for (int inside = 0; inside < 2; ++inside) {
        std::vector<char> got(bytes.size(), 0);
        size_t last = a;
        for (const auto &r : pool_ranges::parts(m, a, b, inside != 0)) {
            if (r.first < last || r.first >= r.second || r.second > b) {
                std::printf("op %ld: parts out of order or outside the window\n", op);
                return false;
            }
            for (size_t i = r.first; i < r.second; ++i) got[i] = 1;
            last = r.second;
        }
        for (size_t i = 0; i < bytes.size(); ++i) {
            const char want = (i >= a && i < b) ? (char)((bytes[i] != 0) == (inside != 0)) : 0;
            if (got[i] != want) {
                std::printf("op %ld: parts(inside=%d) wrong at byte %zu\n", op, inside, i);
                return false;
            }
        }
    }
    return true;
}

int main(int argc, char **argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: pool_ranges_sim bytes ops seed plant\n");
        return 2;
    }
    const size_t n = std::strtoull(argv[1], nullptr, 10);
    const long ops = std::atol(argv[2]);
    std::mt19937_64 rng(std::strtoull(argv[3], nullptr, 10));
    g_plant = std::atoi(argv[4]) != 0;
    pool_ranges::Set m;
    std::vector<char> bytes(n, 0);
    auto pick = [&](size_t &a, size_t &b) {
        a = rng() % n;
        // Mostly short ranges, some long, some empty.
        const size_t len = rng() % 4 == 0 ? rng() % n : rng() % 24;
        b = a + len < n ? a + len : n;
    };
    for (long op = 0; op < ops; ++op) {
        size_t a, b;
        pick(a, b);
        const int kind = (int)(rng() % 3);
        if (kind == 0) {
            if (g_plant) add_planted(m, a, b); else pool_ranges::add(m, a, b);
            for (size_t i = a; i < b; ++i) bytes[i] = 1;
        } else if (kind == 1) {
            pool_ranges::remove(m, a, b);
            for (size_t i = a; i < b; ++i) bytes[i] = 0;
        }
        if (!check(m, bytes, kind == 0 ? "add" : kind == 1 ? "remove" : "none", op)) return 1;
        pick(a, b);
        if (!check_parts(m, bytes, a, b, op)) return 1;
    }
    std::printf("ops %ld ok\n", ops);
    return 0;
}
