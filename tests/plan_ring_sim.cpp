// CPU simulation of the chain plan's packet ring (chain_plan.hip's launch
// loop over llm-kv260_amd/csrc/plan_ring.h): a producer thread writes
// `packets` packets into a ring of `size` slots the way a plan launch does
// (wait for room, write the slot, publish the write index, ring at the end
// of each pass and at the ring's last slot), while a consumer thread plays
// the packet processor: it takes the packet at its read index once that
// packet is both published and rung, checks that the slot holds exactly the
// packet expected there (a hole or an overwritten slot is an error), and
// advances the read index.
//
//   plan_ring_sim <size> <packets> <n> <per_packet_us> <stall_at> <stall_ms> <stall_s> <plant>
//     n:            steps per pass (the ring is rung after every n packets)
//     stall_at:     the packet before which the consumer stops for stall_ms
//                   (-1: never)
//     stall_s:      the producer's give-up bound (seconds without progress)
//     plant:        1 = give up stall_s after the launch began instead of
//                   after the read index last moved (the old bound, which
//                   stops a long launch that is progressing)
// Prints "written W read R result OK|STALLED errors E" and exits 0 when the
// consumer saw no error and took exactly the packets the producer wrote.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

#include "plan_ring.h"

using namespace w4a8::plan_ring;
using clk = std::chrono::steady_clock;

int main(int argc, char **argv) {
    if (argc != 9) {
        std::fprintf(stderr, "usage: plan_ring_sim size packets n per_packet_us stall_at stall_ms stall_s plant\n");
        return 2;
    }
    const uint64_t size = std::strtoull(argv[1], nullptr, 10);
    const long packets = std::atol(argv[2]);
    const int n = std::atoi(argv[3]);
    const int per_us = std::atoi(argv[4]);
    const long stall_at = std::atol(argv[5]);
    const int stall_ms = std::atoi(argv[6]);
    const double stall_s = std::atof(argv[7]);
    const bool plant = std::atoi(argv[8]) != 0;

    std::vector<std::atomic<long>> slot(size);
    for (auto &s : slot) s.store(-1);
    std::atomic<uint64_t> read{0}, write{0}, doorbell{0};
    std::atomic<bool> rung_any{false}, producer_done{false};
    std::atomic<long> errors{0};

    std::thread consumer([&] {
        bool stalled_once = false;
        for (;;) {
            const uint64_t r = read.load();
            const bool ready = r < write.load() && rung_any.load() && r <= doorbell.load();
            if (!ready) {
                if (producer_done.load() && r >= write.load()) break;
                std::this_thread::yield();
                continue;
            }
            if ((long)r == stall_at && !stalled_once) {
                stalled_once = true;
                std::this_thread::sleep_for(std::chrono::milliseconds(stall_ms));
            }
            const long got = slot[r & (size - 1)].load();
            if (got != (long)r) errors.fetch_add(1);
            slot[r & (size - 1)].store(-1);
            if (per_us) std::this_thread::sleep_for(std::chrono::microseconds(per_us));
            read.store(r + 1);
        }
    });

    auto ring = [&](uint64_t last) {
        doorbell.store(last);
        rung_any.store(true);
    };
    const auto t0 = clk::now();
    Room result = Room::OK;
    uint64_t idx = write.load();
    for (long i = 0; i < packets; ++i, ++idx) {
        const int j = (int)(i % n);
        if (plant) {
            // The old bound: measured from the launch's start.
            while (idx - read.load() >= size) {
                ring(idx - 1);
                if (std::chrono::duration<double>(clk::now() - t0).count() > stall_s) {
                    result = Room::STALLED;
                    break;
                }
            }
        } else {
            result = wait_for_room(idx, size, [&] { return read.load(); }, ring, stall_s);
        }
        if (result != Room::OK) break;
        if (slot[idx & (size - 1)].load() != -1) errors.fetch_add(1);   // overwriting an untaken packet
        slot[idx & (size - 1)].store((long)idx);
        write.store(idx + 1);
        if (ring_after(idx, size, j, n)) ring(idx);
    }
    // Ring whatever was written, as the device would eventually see it once
    // it resumes; the consumer must then take exactly those packets.
    if (write.load() > 0) ring(write.load() - 1);
    producer_done.store(true);
    consumer.join();
    const bool ok = errors.load() == 0 && read.load() == write.load();
    std::printf("written %llu read %llu result %s errors %ld\n", (unsigned long long)write.load(),
                (unsigned long long)read.load(), result == Room::OK ? "OK" : "STALLED", errors.load());
    return ok ? 0 : 1;
}
