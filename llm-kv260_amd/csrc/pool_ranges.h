// A set of disjoint byte ranges [start, end) of a pool, kept merged: which
// parts of a udmabuf pool have their current bytes in the host copy
// (shim.hip). Free of HIP types so that a CPU test (tests/pool_ranges_sim.cpp)
// checks it against a byte map.
#pragma once
#include <cstddef>
#include <iterator>
#include <map>
#include <utility>
#include <vector>

namespace w4a8 {
namespace pool_ranges {

using Set = std::map<size_t, size_t>;   // start -> end

// [a, b) joins the set; touching or overlapping ranges merge.
inline void add(Set &m, size_t a, size_t b) {
    if (a >= b) return;
    auto it = m.upper_bound(a);
    if (it != m.begin()) {
        auto p = std::prev(it);
        if (p->second >= a) {
            a = p->first;
            b = b > p->second ? b : p->second;
            m.erase(p);
        }
    }
    while (it != m.end() && it->first <= b) {
        b = b > it->second ? b : it->second;
        it = m.erase(it);
    }
    m.emplace(a, b);
}

// [a, b) leaves the set; a range that straddles either end is cut there.
inline void remove(Set &m, size_t a, size_t b) {
    if (a >= b) return;
    auto it = m.upper_bound(a);
    if (it != m.begin()) --it;
    while (it != m.end() && it->first < b) {
        const size_t s = it->first, e = it->second;
        if (e <= a) {
            ++it;
            continue;
        }
        it = m.erase(it);
        if (s < a) m.emplace(s, a);
        if (e > b) {
            m.emplace(b, e);
            break;
        }
    }
}

// The parts of [a, b) inside the set (inside = true) or outside it, in order.
inline std::vector<std::pair<size_t, size_t>> parts(const Set &m, size_t a, size_t b, bool inside) {
    std::vector<std::pair<size_t, size_t>> out;
    if (a >= b) return out;
    size_t pos = a;
    auto it = m.upper_bound(a);
    if (it != m.begin()) --it;
    for (; it != m.end() && it->first < b; ++it) {
        const size_t s = it->first > a ? it->first : a, e = it->second < b ? it->second : b;
        if (e <= s) continue;
        if (inside)
            out.emplace_back(s, e);
        else if (s > pos)
            out.emplace_back(pos, s);
        pos = e;
    }
    if (!inside && pos < b) out.emplace_back(pos, b);
    return out;
}

}  // namespace pool_ranges
}  // namespace w4a8
