// The chain plan's packet ring discipline (chain_plan.hip), free of HSA types
// so that a CPU test (tests/plan_ring_sim.cpp) drives the same code against a
// simulated queue.
//
// The plan is the only producer on its device's queue while it holds the
// runtime's lock, so it owns the write index outright: a packet slot is taken
// only once the consumer has freed it, then written, then published by
// storing the write index past it. Nothing is ever claimed ahead of being
// written, so giving up leaves no hole that would stall the packet processor
// (a claimed slot with an invalid header blocks every later packet).
#pragma once
#include <chrono>
#include <cstdint>

namespace w4a8 {
namespace plan_ring {

enum class Room { OK, STALLED };

// Waits until slot `idx` of a ring of `size` packets is free: the consumer's
// read index has passed idx - size. `read()` loads that index; `ring(last)`
// tells the consumer that every packet up to `last` is ready, and is called
// once before waiting, so that a ring full of written packets drains. The
// wait gives up (STALLED) only when the read index has not moved for
// `stall_s` seconds: a long launch that keeps the device busy but keeps
// taking packets never gives up, however long it runs.
template <class Read, class Ring>
Room wait_for_room(uint64_t idx, uint64_t size, Read read, Ring ring, double stall_s) {
    uint64_t r = read();
    if (idx - r < size) return Room::OK;
    ring(idx - 1);   // idx >= size here, so idx - 1 is a written packet
    auto moved = std::chrono::steady_clock::now();
    for (;;) {
        const uint64_t now_r = read();
        if (idx - now_r < size) return Room::OK;
        const auto now = std::chrono::steady_clock::now();
        if (now_r != r) {
            r = now_r;
            moved = now;
        } else if (std::chrono::duration<double>(now - moved).count() > stall_s) {
            return Room::STALLED;
        }
    }
}

// Ring the doorbell after packet `idx` of a launch whose pass has n steps
// (j = idx's step): at the end of every pass, so that the device starts while
// later passes are written, and at the ring's last slot, so that no rung
// range of packets wraps around the ring's end (a queue interceptor, such as
// a profiler's, may copy a rung range as one block: with ranges that wrapped,
// rocprofv3's kernel trace read past the ring and crashed).
inline bool ring_after(uint64_t idx, uint64_t size, int j, int n) { return j == n - 1 || ((idx + 1) & (size - 1)) == 0; }

}  // namespace plan_ring
}  // namespace w4a8
