// The grid barrier of the one-launch decode chain: layout of its state words
// and the arithmetic of its epochs, shared by the kernel (chain.hip) and the
// CPU simulation that checks the protocol with threads
// (tests/chain_sync_sim.cpp). Everything here is constexpr, so the same
// functions compile for the host and for gfx950.
//
// Protocol, per launch of G workgroups running n steps (n - 1 barriers):
//  * At the start every workgroup reads GEN, the number of barriers all
//    earlier launches completed (mod 2^32).
//  * Barrier b (after step b): each workgroup g, once its part of step b is
//    done, adds 1 to counter g % COUNTERS (one relaxed device-scope atomic, no
//    return), then polls every counter until counter c holds members(c) *
//    epoch(GEN, b) or more, compared modulo 2^32. Spreading the arrivals over
//    sixteen counters 4 KB apart keeps any one address from serialising 256
//    atomics (one counter: 10 us per barrier; sixteen: 1.3 us on MI355X).
//  * A poll that gives up (spin limit) stores abort_tag(GEN) into ABORT;
//    every poll also watches ABORT, so one give-up ends every workgroup's
//    wait. Such a workgroup skips the rest of its work.
//  * At the end every workgroup takes a ticket. The last one advances GEN by
//    n - 1 when the launch completed, or, when ABORT holds this launch's tag,
//    clears the counters, GEN and ABORT and counts a timeout, so the next
//    launch starts from a clean state. Then it clears TICKET.
// A counter is never more than one barrier ahead of the epoch a poller
// waits for (a workgroup cannot arrive at barrier b + 1 before barrier b is
// complete), so the modular comparison is exact for any GEN.
#pragma once

#include <stdint.h>

namespace w4a8 {
namespace chain_sync {

constexpr int COUNTERS = 16;
constexpr int STRIDE_WORDS = 1024;                 // 4 KB between counters
constexpr int GEN = COUNTERS * STRIDE_WORDS;       // word indices of the control words,
constexpr int ABORT = GEN + 64;                    // each in its own 256-byte line
constexpr int TICKET = GEN + 128;
constexpr int TIMEOUTS = GEN + 192;
constexpr int WORDS = GEN + 256;

// Word index of counter c.
constexpr int counter_word(int c) { return c * STRIDE_WORDS; }

// The counter workgroup g arrives at.
constexpr int counter_of(int g) { return g % COUNTERS; }

// How many of G workgroups arrive at counter c.
constexpr uint32_t members(int c, int G) { return c < G ? (uint32_t)((G - 1 - c) / COUNTERS + 1) : 0u; }

// Epoch of barrier b of a launch that started at gen.
constexpr uint32_t epoch(uint32_t gen, int b) { return gen + (uint32_t)b + 1u; }

// Value counter c holds once all its members have arrived at the barrier of `ep`.
constexpr uint32_t target(int c, int G, uint32_t ep) { return members(c, G) * ep; }

// v has reached t, modulo 2^32 (the two are never 2^31 apart).
constexpr bool reached(uint32_t v, uint32_t t) { return (int32_t)(v - t) >= 0; }

// ABORT's value for a launch that started at gen: never zero.
constexpr uint32_t abort_tag(uint32_t gen) { return (gen << 1) | 1u; }

}  // namespace chain_sync
}  // namespace w4a8
