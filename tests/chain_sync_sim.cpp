// CPU simulation of the one-launch chain's grid barrier (chain.hip), built on
// the same state layout and epoch arithmetic (llm-kv260_amd/csrc/chain_sync.h):
// G threads play the workgroups of a launch, running n steps with the
// kernel's arrive / poll / give-up / exit-ticket sequence on std::atomic
// words. After passing barrier b a thread checks that every thread finished
// step b, which is what the barrier exists for.
//
//   chain_sync_sim <G> <n> <launches> <spin_limit> <stall_launch> <gen0> <plant>
//     stall_launch: the launch in which workgroup G-1 stalls at barrier 1 for
//                   longer than the others' spin limit (-1: none)
//     gen0:         the generation (and matching counters) to start from, so a
//                   run can cross 2^32
//     plant:        1 = poll for the previous epoch (a deliberate bug the
//                   check must catch)
// Prints one line per launch and exits 0 when every launch behaved as
// expected: no thread passed a barrier early, timeouts only where a stall was
// planted, the state restored after one, GEN advanced by n - 1 otherwise.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "chain_sync.h"

using namespace w4a8::chain_sync;

namespace {

std::atomic<uint32_t> words[WORDS];

struct Launch {
    int G, n, spin_limit;
    bool stall;
    bool plant;
    std::vector<std::atomic<int>> done;   // workgroups that finished step j
    std::atomic<int> early{0};            // passes of a barrier before every workgroup finished the step
    std::atomic<int> gave_up{0};
    Launch(int g, int n_, int spin, bool st, bool pl) : G(g), n(n_), spin_limit(spin), stall(st), plant(pl), done(n_) {
        for (auto &d : done) d.store(0);
    }
};

void workgroup(Launch &L, int g, unsigned seed) {
    std::mt19937 rng(seed);
    const uint32_t gen = words[GEN].load();
    const uint32_t tag = abort_tag(gen);
    bool quit = false;
    for (int j = 0; j < L.n; ++j) {
        if (j > 0 && !quit) {
            const int b = j - 1;
            if (L.stall && g == L.G - 1 && b == 1) std::this_thread::sleep_for(std::chrono::milliseconds(200));
            words[counter_word(counter_of(g))].fetch_add(1u);
            const uint32_t ep = epoch(gen, L.plant ? b - 1 : b);
            bool ok = false;
            for (int spin = 0; spin < L.spin_limit; ++spin) {
                if (words[ABORT].load() == tag) break;
                bool all = true;
                for (int c = 0; c < COUNTERS; ++c)
                    if (!reached(words[counter_word(c)].load(), target(c, L.G, ep))) all = false;
                if (all) {
                    ok = true;
                    break;
                }
                std::this_thread::yield();
            }
            if (!ok) {
                // Gave up, or saw another workgroup give up.
                if (words[ABORT].load() != tag) {
                    words[ABORT].store(tag);
                    L.gave_up.fetch_add(1);
                }
                quit = true;
            } else if (L.done[b].load() != L.G) {
                L.early.fetch_add(1);
            }
        }
        if (!quit) {
            if (rng() % 4 == 0) std::this_thread::sleep_for(std::chrono::microseconds(rng() % 200));
            L.done[j].fetch_add(1);
        }
    }
    const uint32_t t = words[TICKET].fetch_add(1u);
    if (t == (uint32_t)(L.G - 1)) {
        if (words[ABORT].load() == tag) {
            for (int c = 0; c < COUNTERS; ++c) words[counter_word(c)].store(0u);
            words[GEN].store(0u);
            words[ABORT].store(0u);
            words[TIMEOUTS].fetch_add(1u);
        } else {
            words[GEN].store(gen + (uint32_t)(L.n - 1));
        }
        words[TICKET].store(0u);
    }
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 8) {
        std::fprintf(stderr, "usage: %s G n launches spin_limit stall_launch gen0 plant\n", argv[0]);
        return 2;
    }
    const int G = std::atoi(argv[1]), n = std::atoi(argv[2]), launches = std::atoi(argv[3]);
    const int spin = std::atoi(argv[4]), stall_launch = std::atoi(argv[5]);
    const uint32_t gen0 = (uint32_t)std::strtoul(argv[6], nullptr, 0);
    const bool plant = std::atoi(argv[7]) != 0;
    for (auto &w : words) w.store(0u);
    words[GEN].store(gen0);
    for (int c = 0; c < COUNTERS; ++c) words[counter_word(c)].store(members(c, G) * gen0);
    int failures = 0, early_total = 0;
    for (int l = 0; l < launches; ++l) {
        const uint32_t gen_before = words[GEN].load(), timeouts_before = words[TIMEOUTS].load();
        Launch L(G, n, spin, l == stall_launch, plant);
        std::vector<std::thread> th;
        for (int g = 0; g < G; ++g) th.emplace_back(workgroup, std::ref(L), g, 1000u * l + g);
        for (auto &t : th) t.join();
        const bool stalled = l == stall_launch;
        const uint32_t gen_after = words[GEN].load();
        bool ok = words[TICKET].load() == 0 && words[ABORT].load() == 0;
        if (stalled) {
            ok = ok && L.gave_up.load() >= 1 && gen_after == 0 && words[TIMEOUTS].load() == timeouts_before + 1;
            for (int c = 0; c < COUNTERS; ++c) ok = ok && words[counter_word(c)].load() == 0;
        } else {
            ok = ok && L.gave_up.load() == 0 && gen_after == gen_before + (uint32_t)(n - 1) &&
                 words[TIMEOUTS].load() == timeouts_before;
            for (int c = 0; c < COUNTERS; ++c) ok = ok && words[counter_word(c)].load() == members(c, G) * gen_after;
        }
        ok = ok && L.early.load() == 0;
        early_total += L.early.load();
        std::printf("launch %d: gen %u -> %u, early passes %d, gave up %d, %s\n", l, gen_before, gen_after,
                    L.early.load(), L.gave_up.load(), ok ? "ok" : "FAILED");
        failures += !ok;
    }
    std::printf("early passes in all: %d\n", early_total);
    return failures ? 1 : 0;
}
