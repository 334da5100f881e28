// M = 1 W4A8 GEMV for gfx950: y[N] = W[N, K] x, W in ggml Q4_0, x in Q8_0.
//
// A bandwidth problem with a latency tail, so no MFMA. What bounds it is how
// many weight bytes each CU keeps in flight (HBM3E needs ~150 KB per CU to
// run near its plateau) and how cleanly they stream, so the kernel is built
// around wide, fully coalesced, non-temporal loads held in registers:
//
//  * The unit of work is a chunk: eight consecutive blocks of a row, 144
//    bytes, i.e. nine 16-byte pieces (the 9-beat chunk hls/int4_core/q4_0.h:
//    21-25 streams). A wave tile is 64 / C whole rows (C = K / 256 chunks per
//    row), at most 64 chunks = 9,216 contiguous bytes: nine
//    global_load_dwordx4, lane l loading bytes 1024 p + 16 l of the tile.
//  * Each wave keeps two tiles in registers: while it computes one, the next
//    is in flight, and the one it just consumed is refilled before its terms
//    are computed (18 KB per wave). Large matrices launch two 4-wave
//    workgroups per CU, both resident.
//  * A tile's pieces go through a per-wave 9 KB LDS slab (ds_write_b128 in
//    load order, ds_read_b128 in chunk order), so that lane l ends up with
//    chunk l: 144 bytes, eight whole blocks.
//  * Lane l owns chunk column c = l % C of the tile's rows. The tile is whole
//    rows, so c never changes: the 256 activations (as block_dot_nib takes
//    them), 8 scales and 8 block corrections of column c are read from LDS
//    into registers once.
//  * The activation is staged once per workgroup in LDS (quantized there from
//    fp32 by the fused entry points); its loads are issued before the first
//    tiles', so they do not wait behind the weights.
//  * Each block's dot is exact in int32: twelve v_dot8_u32_u4 straight on the
//    packed nibbles against the activation split into nibbles at staging
//    (block_dot_nib). Then t = (f32(sumi) * d_w) * d_x.
//  * The contract's order (src/llm_kv260/q4_0.py:170-182): lane a of a row
//    adds the terms of blocks a, a + 8, a + 16, ... in that order, from +0.0f.
//    Chunk c holds terms 8c .. 8c + 7, so accumulator a needs term a of every
//    chunk of the row, in chunk order: each lane writes its eight terms to
//    the slab, and lane 8r + a of the wave reads term a of chunks 0 .. C-1 of
//    row r and adds them one by one. The eight lane sums of a row then meet
//    in a DPP adjacent-pair tree.
// The device side (parameters, tiles, the kernel body and the kernels) lives
// here so that the chain plan's code object (chain_plan_kernels.hip) builds
// the same body; the host launchers are in gemv_m1.hip.
#pragma once
#include <type_traits>
#include <utility>

#include "../../include/w4a8.h"
#include "kernels.h"
#include "gemv_tile.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

constexpr int MAX_THREADS = 512;
constexpr size_t LDS_BUDGET = 160 * 1024;   // per CU on gfx950

struct GemvParams {
    const uint8_t *seg[4];
    const void *x;
    float *y;
    int seg_rows;     // rows per segment
    int nseg;
    int k;
    int rows;         // seg_rows * nseg
    int C;            // chunks per row, k / 256
    int rpw;          // rows per wave tile, 64 / C
    int tiles;        // ceil(rows / rpw); board layouts: nseg * tps
    int paired;       // v2 port layout
    int tps;          // board layouts: tiles per segment
    int prw;          // v2 port layout: row pairs per tile
    // Argmax epilogue (LM head): the first row of the largest y, written to
    // *argmax by the last workgroup to finish; the merged key and the ticket
    // counter live in the caller's workspace (both zero between calls).
    int32_t *argmax;
    unsigned long long *key;
    unsigned int *ticket;
    // X_RMS: the norm weight float32[k] and epsilon.
    const float *norm_w;
    float eps;
};

// Argmax key of y[row] = v: the largest v wins, and among equal values the
// smallest row, which is the reference's scan (board/tp/tp_llama.cpp:879-880,
// "if (y[i] > y[best]) best = i"). -0 compares equal to +0 there, so it is
// keyed as +0; a NaN never compares greater, so it gets key 0 and never wins,
// except at row 0, where the scan starts and then keeps 0: that NaN gets the
// largest key of all. Every other value has a key in between.
constexpr unsigned long long ARGMAX_ROW0_NAN = ~0ull;
__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
    if (v != v) return row == 0 ? ARGMAX_ROW0_NAN : 0ull;
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)row);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max_u64(v, __shfl_xor(v, off));
    return v;
}

constexpr int BATCH_THREADS = 64 * 4;
constexpr int BATCH_TILES_PER_WAVE = 20;
constexpr int MID_TILES_PER_WAVE = 1;

struct BatchEntry {
    const uint8_t *w;
    const void *x;
    float *y;
    int rows;
    int k;
};

// Passed by value (kernel arguments): 32 B per entry.
struct BatchParams {
    int n;
    int tiles_per_block;
    BatchEntry e[W4A8_CHAIN_MAX_STEPS];
};

// Board layouts (four segments at separate addresses: the v1 quarters, or
// the v2 port regions, where row i of a region pairs with row i + R/2 and
// their 144-byte chunks alternate). Tiles are numbered segment by segment,
// tps to a segment, so that none straddles two; a v2 tile takes prw whole
// row pairs. Every tile is then one contiguous run of its segment, read with
// the plain layout's coalesced, range-checked loads. A tile past the end
// (segment index nseg or more) reads nothing.
struct TileSpan {
    const uint8_t *base;
    uint32_t bytes;
};

__device__ __forceinline__ TileSpan board_tile(const GemvParams &P, int tile) {
    const int t = __builtin_amdgcn_readfirstlane(tile);
    const int seg = t / P.tps, lt = t - seg * P.tps;
    TileSpan s{P.seg[0], 0u};
    if (seg < P.nseg) {
        const size_t row_bytes = (size_t)P.C * CHUNK_BYTES;
        const size_t seg_bytes = (size_t)P.seg_rows * row_bytes;
        const size_t tile_bytes = (size_t)(P.paired ? 2 * P.prw : P.rpw) * row_bytes;
        const size_t off = (size_t)lt * tile_bytes;
        s.base = P.seg[seg] + off;
        s.bytes = (uint32_t)(seg_bytes - off < tile_bytes ? seg_bytes - off : tile_bytes);
    }
    return s;
}

// Matrix row of row r of a board-layout tile (r < 2 prw for v2: pair r / 2,
// its first row when r is even), or -1 when the tile has no such row.
__device__ __forceinline__ int board_row(const GemvParams &P, int tile, int r) {
    const int t = __builtin_amdgcn_readfirstlane(tile);
    const int seg = t / P.tps, lt = t - seg * P.tps;
    if (seg >= P.nseg) return -1;
    if (P.paired) {
        const int half = P.seg_rows >> 1, i = lt * P.prw + (r >> 1);
        return (r >> 1) < P.prw && i < half ? seg * P.seg_rows + (r & 1) * half + i : -1;
    }
    const int local = lt * P.rpw + r;
    return r < P.rpw && local < P.seg_rows ? seg * P.seg_rows + local : -1;
}

// Argmax workspace: the ticket counter and the merged key, each in its own 64-byte line.
constexpr size_t ARGMAX_KEY_OFFSET = 64;
// Tiles per wave held in registers. Two: a third raised no shape's rate and
// took 36 VGPRs.
template <bool PLAIN>
constexpr int depth_of() { return 2; }

struct Tile {
    u32x4 p[CHUNK_PIECES];
};

// Load the nine pieces of `tile` (lane l: bytes 1024 p + 16 l of the tile).
// A tile past the end of the matrix reads nothing, and the pieces of the last
// tile past the matrix's (or the segment's) last byte read zeros (their terms
// are never stored).
template <bool PLAIN>
__device__ __forceinline__ void load_tile(const GemvParams &P, int tile, int lane, Tile &t) {
    __amdgpu_buffer_rsrc_t tb;
    if constexpr (PLAIN) {
        const size_t tile_bytes = (size_t)P.rpw * (size_t)P.C * CHUNK_BYTES;
        const size_t total = (size_t)P.rows * (size_t)P.C * CHUNK_BYTES;
        const size_t off0 = (size_t)__builtin_amdgcn_readfirstlane(tile) * tile_bytes;
        const bool in = off0 < total;
        const uint32_t n = in ? (uint32_t)(total - off0 < (size_t)TILE_BYTES ? total - off0 : (size_t)TILE_BYTES) : 0u;
        tb = buffer_of(P.seg[0] + (in ? off0 : 0), n);
    } else {
        const TileSpan sp = board_tile(P, tile);
        tb = buffer_of(sp.base, sp.bytes);
    }
#pragma unroll
    for (int p = 0; p < CHUNK_PIECES; ++p) t.p[p] = __builtin_amdgcn_raw_buffer_load_b128(tb, 1024 * p + 16 * lane, 0, CACHE_NT);
}

// LDS layout (dynamic): per-wave slabs [waves][9216] | the staged activation
// (nb / 8 columns of XCOL_DWORDS) | for X_RMS the float64 squares of x
// (rms_sq_doubles(k), chain by chain) and the scale. `block` / `nblocks` are this workgroup's index and the
// number of workgroups sharing the matrix.
// ONE_PASS: a tile holds at most eight rows (K >= 2048), so one pass of the
// ordered sums covers it and each lane stores at most one value per tile.
// The workgroup's best key (its waves' keys through LDS) goes into the
// launch's key with one device-scope atomic max; then the workgroup takes a
// ticket. Both are relaxed atomics performed where every XCD sees them, and
// the ticket is taken only after the max has returned, so the workgroup that
// draws the last ticket reads a key every other workgroup has already merged.
// No fence is needed (an agent-scope release or acquire would write back or
// invalidate the whole L2 of every XCD in turn). The last workgroup writes the
// row and clears the key and the ticket for the next call.
__device__ __forceinline__ void argmax_finish(const GemvParams &P, unsigned long long best, int nblocks, int waves,
                                              uint8_t *lds) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    unsigned long long *keys = reinterpret_cast<unsigned long long *>(lds);   // the slabs are free by now
    best = wave_max_u64(best);
    __syncthreads();
    if (lane == 0) keys[wave] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = 0;
        for (int w = 0; w < waves; ++w) b = max_u64(b, keys[w]);
        const unsigned long long seen = __hip_atomic_fetch_max(P.key, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The ticket depends on the max's result (no key equals ARGMAX_ROW0_NAN - 1),
        // so it is taken after the max is done.
        const unsigned inc = seen == ARGMAX_ROW0_NAN - 1 ? 2u : 1u;
        const unsigned t = __hip_atomic_fetch_add(P.ticket, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == (unsigned)(nblocks - 1)) {
            const unsigned long long k = __hip_atomic_load(P.key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int32_t row = (k == 0ull || k == ARGMAX_ROW0_NAN) ? 0 : (int32_t)(0xFFFFFFFFu - (uint32_t)k);
            __hip_atomic_store(P.argmax, row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(P.key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(P.ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// PAIR: the gate|up GEMV with silu(gate) * up as its epilogue. Gate tile t
// (rows of y[0 .. rows / 2)) and up tile t + tiles / 2 (the up rows of the
// same outputs) go to partner waves of one workgroup: its first waves / 2
// waves take gate tiles V b .. V b + V - 1 (V = waves / 2, b the workgroup),
// the others the matching up tiles, one tile each (the grid is exactly
// tiles / 2 / V workgroups). A gate wave leaves its rows' y in its slab, and
// after a workgroup barrier its partner stores act[r] = silu_mul(gate, up)
// to y[0 .. rows / 2) (PAIR_F32). PAIR_Q8: act quantized to Q8_0 in the
// epilogue instead, y the engine layout of act (int8[n] | float32[n / 32],
// n = rows / 2), the input of down as the reference's caller quantizes it
// (tp_llama.cpp:330-352). Needs V * rpw = 32 (k = 2048, V = 4): a
// workgroup's outputs are then exactly Q8_0 block b of act, quantized by
// eight lanes of its first up wave as the fused activation quantizer does.
// COH (the chain plan's dispatches, which carry no cache fences between
// them): bit 0, x is an earlier step's output, read from the device's
// coherence point (past the L2 of this XCD); bit 1, y is a later step's x,
// written through to it and waited for before the wave ends. ONE_PASS (and
// PAIR) only; fp32 and engine-layout x formats.
constexpr int COH_X = 1, COH_Y = 2;
constexpr int PAIR_F32 = 1, PAIR_Q8 = 2;

// The overlapped chain plan's step-to-step wait (chain_plan.hip): a step's
// dispatch goes out without the barrier bit, so its workgroups start while
// the step before is still running. Each workgroup issues its weight loads
// (weights never depend on the chain), then waits until every workgroup of
// the step before has finished (a flag byte each), and only then loads and
// stages x. Each workgroup of a step stores its own flag byte once its
// outputs have landed: the instance number it finished, modulo 256, read
// from that same byte when it starts (every instance of the step before has
// the same workgroups, and passes do not overlap: the first step of each
// pass keeps the barrier bit). Loads and stores of the flags are device-
// coherent (sc1). Every wait is bounded: one that gives up sets the abort
// word, which ends every other wait at once, and the plan reports it.
struct StreamSync {
    const uint8_t *prev;     // the previous step's flags (one byte per workgroup), or null
    uint8_t *mine;           // this step's
    uint32_t *abort;
    int prev_groups;
    int spin_limit;
};

// Wave 0 polls; every wave of the workgroup calls this once (it ends with a
// workgroup barrier). Returns the flag value this workgroup stores at its end
// (valid in wave 0).
__device__ __forceinline__ uint32_t stream_wait(const StreamSync &S, int block, int wave, int lane) {
    uint32_t target = 0;
    if (wave == 0) {
        const __amdgpu_buffer_rsrc_t mb = buffer_of(S.mine, (uint32_t)block + 1u);
        const uint32_t e = __builtin_amdgcn_readfirstlane((uint32_t)__builtin_amdgcn_raw_buffer_load_b8(mb, block, 0, SC1));
        target = (e + 1u) & 0xFFu;
        if (S.prev) {
            const uint32_t want = target * 0x01010101u;
            const int words = (S.prev_groups + 3) >> 2;
            const __amdgpu_buffer_rsrc_t pb = buffer_of(S.prev, 4u * (uint32_t)words);
            const __amdgpu_buffer_rsrc_t ab = buffer_of(S.abort, 4u);
            for (int spin = 0;; ++spin) {
                bool done = true;
                for (int w = lane; w < words; w += 64) {
                    const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(pb, 4 * w, 0, SC1);
                    const int valid = S.prev_groups - 4 * w;
                    const uint32_t mask = valid >= 4 ? ~0u : (1u << (8 * valid)) - 1u;
                    if ((v & mask) != (want & mask)) done = false;
                }
                const uint32_t aborted = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_raw_buffer_load_b32(ab, 0, 0, SC1));
                if (__builtin_amdgcn_ballot_w64(!done) == 0) break;
                if (aborted != 0u) break;
                if (spin >= S.spin_limit) {
                    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(1u, ab, 0, 0, SC1);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    __syncthreads();
    return target;
}

// After the workgroup's outputs have landed: its flag for the next step.
__device__ __forceinline__ void stream_arrive(const StreamSync &S, int block, uint32_t target) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)target, buffer_of(S.mine, (uint32_t)block + 1u), block, 0, SC1);
}

template <int XF, bool PLAIN, bool ONE_PASS, bool ARGMAX = false, int PAIR = 0, int COH = 0, bool STREAM = false>
__device__ __forceinline__ void gemv_m1_body(const GemvParams &P, int block, int nblocks, int nthreads, uint8_t *lds,
                                             const StreamSync *S = nullptr) {
    const int nb = P.k >> 5;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int waves = nthreads >> 6;
    uint8_t *slab = lds + (size_t)wave * TILE_BYTES;
    uint32_t *s_x = reinterpret_cast<uint32_t *>(lds + (size_t)waves * TILE_BYTES);

    const int C = P.C, rpw = P.rpw;
    // Lane l takes chunk l of the tile: row l / C, column l % C; in a v2
    // tile the chunks of a row pair alternate, so chunk l is column
    // (l / 2) % C of row 2 (l / 2C) + l % 2 of the tile.
    const bool paired = !PLAIN && P.paired;
    const int pq = paired ? lane >> 1 : lane;
    const int my_c = pq - lane_quot(pq, C) * C;
    const bool lane_live = paired ? lane < 2 * P.prw * C : lane_quot(lane, C) < rpw;
    // Rows per tile as the ordered sums see them.
    const int trows = paired ? 2 * P.prw : rpw;

    constexpr int DEPTH = depth_of<PLAIN>();
    const int pv = waves >> 1;            // PAIR: gate waves per workgroup
    const bool up_wave = PAIR && wave >= pv;
    int tile = PAIR ? (up_wave ? (P.tiles >> 1) + block * pv + wave - pv : block * pv + wave) : block * waves + wave;
    const int tstride = PAIR ? P.tiles : nblocks * waves;
    // Tiles of this wave; the division only where a wave has two or more.
    const int n_my = tile >= P.tiles ? 0 : tile + tstride >= P.tiles ? 1 : (P.tiles - 1 - tile) / tstride + 1;

    // 1. The activation. Its loads go out before any weight tile's; the
    // staging below waits for them only. (STREAM: after the weight loads and
    // the wait for the step before, since x may be that step's output.)
    XRaw<XF> xr;
    constexpr int XAUX = (COH & COH_X) ? SC1 : 0;
    // X_RMS with four threads per block (every launch shape at K = 2048):
    // each thread loads, squares and stages a quarter of a block.
    [[maybe_unused]] XQuarter xq;
    const bool quarter = XF == X_RMS && nthreads >= 4 * nb;
    // X_F32 with a thread per block: by whole lines, in the waves that hold
    // blocks only (a wave-uniform branch: the others issue no activation
    // load at all).
    [[maybe_unused]] XLines xl;
    const bool lines = XF == X_F32 && nthreads >= nb;
    const bool x_wave = __builtin_amdgcn_readfirstlane(wave) * 64 < nb;
    auto load_x = [&]() {
        if constexpr (XF == X_RMS) {
            if (quarter)
                x_load_quarter<XAUX>(P.x, P.norm_w, P.k, tid >> 2, tid & 3, tid < 4 * nb, xq);
            else
                x_load<XF, XAUX>(P.x, P.k, tid, tid < nb, xr, P.norm_w);
        } else if constexpr (XF == X_F32) {
            if (lines) {
                if (x_wave) x_load_lines<XAUX>(P.x, P.k, wave, lane, xl);
            } else {
                x_load<XF, XAUX>(P.x, P.k, tid, tid < nb, xr, P.norm_w);
            }
        } else {
            x_load<XF, XAUX>(P.x, P.k, tid, tid < nb, xr, P.norm_w);
        }
    };
    if constexpr (!STREAM) load_x();
    [[maybe_unused]] uint32_t flag = 0;
    auto after_weights = [&]() {
        if constexpr (STREAM) {
            flag = stream_wait(*S, block, wave, lane);
            load_x();
        }
    };


    uint32_t xv[8][8];
    float xd[8];
    int32_t xs[8];
    // 2. Stage the activation, then pull this lane's chunk column into registers.
    auto stage_x = [&]() {
        float rms = 0.0f;
        if constexpr (XF == X_RMS) {
            // rmsnorm's scale needs the whole of x: its squares go to LDS as
            // float64 after the staged x (chain by chain, rms_sq_index), wave
            // 0 reduces them, and the scale comes back through LDS. Block b's
            // elements 32 b + 4 m + c are square 8 b + m of chain c.
            double *sq = reinterpret_cast<double *>(s_x + (nb / 8) * XCOL_DWORDS);
            float *s_rms = reinterpret_cast<float *>(sq + rms_sq_doubles(P.k));
            const int cs = P.k / 4 + 2;
            auto squares = [&](const XRaw<XF> &r, int b) {
                double *c0 = sq + 8 * b;
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    const double a = r.v[m].x, c = r.v[m].y, d = r.v[m].z, e = r.v[m].w;
                    c0[m] = a * a;
                    c0[cs + m] = c * c;
                    c0[2 * cs + m] = d * d;
                    c0[3 * cs + m] = e * e;
                }
            };
            if (quarter) {
                // Element 32 b + 4 q + c is square 8 b + q of chain c; element
                // 32 b + 16 + 4 q + c square 8 b + 4 + q.
                if (tid < 4 * nb) {
                    double *c0 = sq + 8 * (tid >> 2) + (tid & 3);
                    const double a[4] = {xq.xa.x, xq.xa.y, xq.xa.z, xq.xa.w};
                    const double e[4] = {xq.xb.x, xq.xb.y, xq.xb.z, xq.xb.w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        c0[c * cs] = a[c] * a[c];
                        c0[c * cs + 4] = e[c] * e[c];
                    }
                }
            } else {
                if (tid < nb) squares(xr, tid);
                for (int b = tid + nthreads; b < nb; b += nthreads) {
                    XRaw<XF> xb;
                    x_load<XF, XAUX>(P.x, P.k, b, true, xb, P.norm_w);
                    squares(xb, b);
                }
            }
            __syncthreads();
            if (wave == 0) {
                const float sc = rms_scale_wave(sq, P.k, P.eps);
                if (lane == 0) *s_rms = sc;
            }
            __syncthreads();
            rms = *s_rms;
        }
        if (quarter) {
            if constexpr (XF == X_RMS) {
                if (tid < 4 * nb) x_stage_quarter(xq, tid >> 2, tid & 3, s_x, rms);
            }
        } else {
            if constexpr (XF == X_F32) {
                if (lines && x_wave) x_lines_to_block(xl, lane, slab, xr);
            }
            if (tid < nb) x_stage<XF>(xr, tid, s_x, rms);
            for (int b = tid + nthreads; b < nb; b += nthreads) {   // only if a launch has fewer threads than blocks
                XRaw<XF> xb;
                x_load<XF, XAUX>(P.x, P.k, b, true, xb, P.norm_w);
                x_stage<XF>(xb, b, s_x, rms);
            }
        }
        __syncthreads();
        const uint32_t *col = s_x + (lane_live ? my_c : 0) * XCOL_DWORDS;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const u32x4 *src = reinterpret_cast<const u32x4 *>(col + 8 * j);
            const u32x4 a = src[0], c = src[1];
            xv[j][0] = a.x; xv[j][1] = a.y; xv[j][2] = a.z; xv[j][3] = a.w;
            xv[j][4] = c.x; xv[j][5] = c.y; xv[j][6] = c.z; xv[j][7] = c.w;
            xd[j] = __uint_as_float(col[XCOL_D + j]);
            xs[j] = (int32_t)col[XCOL_S + j];
        }
    };

    const int acc_r = lane >> 3, acc_a = lane & 7;
    unsigned long long best = 0;          // argmax epilogue: this lane's best key
    // y's buffer resource is made where y is stored, not here: P.y is not
    // among the preloaded arguments, and a resource made up front has the
    // wave wait for its argument fetch before the weight loads go out.
    auto y_rsrc_of = [&]() {
        return __builtin_amdgcn_make_buffer_rsrc(P.y, 0,
                                                 PAIR == PAIR_Q8 ? P.rows / 2 + P.rows / 16
                                                                 : 4 * (PAIR ? P.rows / 2 : P.rows),
                                                 BUFFER_DWORD3);
    };
    // One tile: buffer -> slab (load order) -> chunk (lane order) -> terms ->
    // slab -> ordered lane sums -> tree -> y; with REFILL the buffer then
    // receives the tile DEPTH strides ahead while the terms are computed.
    auto step = [&](Tile &b, auto refill) {
        u32x4 *wslab = reinterpret_cast<u32x4 *>(slab);
#pragma unroll
        for (int p = 0; p < CHUNK_PIECES; ++p) wslab[64 * p + lane] = b.p[p];
        wave_sync_lds();
        uint32_t w[CHUNK_DWORDS];
        {
            const u32x4 *src = reinterpret_cast<const u32x4 *>(slab + CHUNK_BYTES * lane);
#pragma unroll
            for (int q = 0; q < CHUNK_PIECES; ++q) {
                const u32x4 v = src[q];
                w[4 * q] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
            }
        }
        if constexpr (decltype(refill)::value) load_tile<PLAIN>(P, tile + DEPTH * tstride, lane, b);
        float t[8];
        chunk_terms(w, xv, xd, xs, t);
        wave_sync_lds();
        // Terms at a stride of nine floats per lane: both the writes (lane l,
        // term j -> 9 l + j) and the ordered reads below hit distinct banks.
        float *s_t = reinterpret_cast<float *>(slab);
#pragma unroll
        for (int j = 0; j < 8; ++j) s_t[9 * lane + j] = t[j];
        wave_sync_lds();
        // Accumulator a of row r: term a of chunks 0 .. C-1, in order, from
        // +0.0f. Eight rows per pass (more than one pass only when C < 8).
        // Row r of a v2 tile has its chunks at 2 (r / 2) C + r % 2 + 2 c.
        auto lane_sum = [&](int r) {
            if (paired) return ordered_lane_sum_at(s_t, 2 * (r >> 1) * C + (r & 1), 2, r < trows, C, acc_a);
            return ordered_lane_sum(s_t, r, rpw, C, acc_a);
        };
        auto row_of = [&](int r) { return PLAIN ? (r < rpw && tile * rpw + r < P.rows ? tile * rpw + r : -1) : board_row(P, tile, r); };
        if constexpr (PAIR) {
            // The gate wave's y goes to the first floats of its slab (its
            // ordered sums, read above by this same wave, are done with it);
            // the up wave reads its partner's after the barrier. Every wave
            // of the workgroup has exactly one tile, so each reaches it once.
            const float yv = tree8_dpp(lane_sum(acc_r));
            const bool mine = acc_r < rpw && acc_a == 0;
            if (!up_wave && mine) s_t[acc_r] = yv;
            __syncthreads();
            if constexpr (PAIR == PAIR_F32) {
                if (up_wave) {
                    const float gate = reinterpret_cast<const float *>(lds + (size_t)(wave - pv) * TILE_BYTES)[acc_r < rpw ? acc_r : 0];
                    const int row = (tile - (P.tiles >> 1)) * rpw + acc_r;
                    const float act = silu_mul(gate, yv);
                    store_y<(COH & COH_Y) ? SC1 : 0>(y_rsrc_of(), mine && row < (P.rows >> 1) ? 4 * row : OUT_OF_RANGE, act);
                }
            } else {
                // The block's 32 act values go to the first floats of the
                // first up wave's slab (its sums are done: the barrier above
                // came after them), in row order; after a second barrier its
                // lanes 0..7 quantize four each, amax met over the eight by
                // DPP, exactly as a thread holding the whole block would
                // (quantize.hip's quantize_store8).
                float *s_q = reinterpret_cast<float *>(lds + (size_t)pv * TILE_BYTES);
                if (up_wave && mine) {
                    const float gate = reinterpret_cast<const float *>(lds + (size_t)(wave - pv) * TILE_BYTES)[acc_r];
                    s_q[(wave - pv) * rpw + acc_r] = silu_mul(gate, yv);
                }
                __syncthreads();
                if (wave == pv && lane < 8) {
                    const float4 v = reinterpret_cast<const float4 *>(s_q)[lane];
                    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
                    amax = fmaxf(amax, dpp_mov<0xB1>(amax));
                    amax = fmaxf(amax, dpp_mov<0x4E>(amax));
                    amax = fmaxf(amax, dpp_mov<0x141>(amax));
                    const float d = q8_scale(amax);
                    const float inv = safe_recip(d);
                    const uint32_t word = (uint32_t)(uint8_t)q8_round(v.x, inv) |
                                          ((uint32_t)(uint8_t)q8_round(v.y, inv) << 8) |
                                          ((uint32_t)(uint8_t)q8_round(v.z, inv) << 16) |
                                          ((uint32_t)(uint8_t)q8_round(v.w, inv) << 24);
                    const int n = P.rows >> 1;
                    store_y<(COH & COH_Y) ? SC1 : 0>(y_rsrc_of(), 32 * block + 4 * lane, __uint_as_float(word));
                    store_y<(COH & COH_Y) ? SC1 : 0>(y_rsrc_of(), lane == 0 ? n + 4 * block : OUT_OF_RANGE,
                                                     half_bits_to_float(float_to_half_bits(d)));
                }
            }
        } else if constexpr (ONE_PASS) {
            const float yv = tree8_dpp(lane_sum(acc_r));
            const int row = row_of(acc_r);
            const bool mine = acc_a == 0 && row >= 0;
            store_y<(COH & COH_Y) ? SC1 : 0>(y_rsrc_of(), mine ? 4 * row : OUT_OF_RANGE, yv);
            if constexpr (ARGMAX) {
                if (mine) best = max_u64(best, argmax_key(yv, row));
            }
        } else {
            for (int r = acc_r; r - acc_r < trows; r += 8) {
                const float yv = tree8_dpp(lane_sum(r));
                const int row = row_of(r);
                if (acc_a == 0 && row >= 0) {
                    P.y[row] = yv;
                    if constexpr (ARGMAX) best = max_u64(best, argmax_key(yv, row));
                }
            }
        }
        wave_sync_lds();
        tile += tstride;
    };

    // 3. Three straight-line paths, chosen per wave, so that every wait on
    // the loads in flight is exact: no tile, one tile, or the DEPTH-deep
    // pipeline (whole rounds with refills, then the remainder without).
    using refill_t = std::true_type;
    using last_t = std::false_type;
    if (n_my >= 2) {
        Tile buf[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load_tile<PLAIN>(P, tile + d * tstride, lane, buf[d]);
        after_weights();
        stage_x();
        int done = 0;
        for (; done + DEPTH <= n_my; done += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) step(buf[d], refill_t{});
        }
#pragma unroll
        for (int d = 0; d + 1 < DEPTH; ++d)
            if (done + d < n_my) step(buf[d], last_t{});
    } else if (n_my == 1) {
        Tile b;
        load_tile<PLAIN>(P, tile, lane, b);
        after_weights();
        stage_x();
        step(b, last_t{});
    } else {
        after_weights();
        stage_x();
    }
    if constexpr (ARGMAX) argmax_finish(P, best, nblocks, waves, lds);
    if constexpr (STREAM)
        stream_arrive(*S, block, flag);
    else if constexpr ((COH & COH_Y) != 0)
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The fields the first loads need (and the grid and workgroup sizes, which
// otherwise come from the dispatch's hidden arguments) also come as leading
// scalar arguments, which the build preloads into SGPRs: the first loads
// then wait for no argument fetch. y is not among them: read from the
// argument block with one scalar load at the start, as now, the decode chain
// ran in 270 us per step; with y preloaded as well, so that the wave reads
// nothing of the block, in 277 (the same as with nothing preloaded), and
// delaying the weight loads by other means (a sleep, or a wait for the
// activation's loads) did not recover it.
template <int XF, bool PLAIN, bool ONE_PASS, bool ARGMAX = false, int PAIR = 0>
__global__ __launch_bounds__(MAX_THREADS) void gemv_m1_kernel(const uint8_t *w0, const void *x, int rows, int k, int C,
                                                              int rpw, int tiles, int nblocks, int nthreads,
                                                              GemvParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if constexpr (PLAIN) {
        P.seg[0] = w0;
        P.x = x;
        P.rows = rows;
        P.k = k;
        P.C = C;
        P.rpw = rpw;
        P.tiles = tiles;
        gemv_m1_body<XF, PLAIN, ONE_PASS, ARGMAX, PAIR>(P, blockIdx.x, nblocks, nthreads, lds);
    } else {
        // The board layouts index P.seg at run time: P stays as the host wrote
        // it (the leading scalars repeat its fields) and is read from the
        // argument block. Writing to it would make it a local copy, which the
        // run-time index puts in scratch memory (the gemv2 LM head then took
        // 60 us instead of 35).
        gemv_m1_body<XF, PLAIN, ONE_PASS, ARGMAX, PAIR>(P, blockIdx.x, nblocks, nthreads, lds);
    }
}

__host__ __device__ inline void derive_plain(GemvParams &P, const uint8_t *w, const void *x, float *y, int rows, int k) {
    P.seg[0] = P.seg[1] = P.seg[2] = P.seg[3] = w;
    P.x = x;
    P.y = y;
    P.seg_rows = rows;
    P.nseg = 1;
    P.k = k;
    P.rows = rows;
    P.C = k >> 8;
    P.rpw = 64 / P.C;
    P.tiles = (rows + P.rpw - 1) / P.rpw;
    P.paired = 0;
}

// Workgroups of one batch entry: enough that each wave owns about
// BATCH_TILES_PER_WAVE tiles.
__host__ __device__ inline int batch_blocks(int rows, int k, int tiles_per_block) {
    const int rpw = 64 / (k >> 8);
    const int tiles = (rows + rpw - 1) / rpw;
    return (tiles + tiles_per_block - 1) / tiles_per_block;
}

// Many independent GEMVs in one launch: each entry j gets n_j workgroups
// (n_j = batch_blocks of its shape), each working exactly as the
// single-matrix kernel would with a grid of n_j workgroups. The entries take
// the workgroup indices from the last one backwards, so the largest matrix
// of a decode step (the LM head, listed last) is dispatched first and the
// small ones fill the end of the launch.
// Two waves per SIMD (two workgroups per CU), as the single-matrix kernel runs.
// ONE_PASS: every entry has K >= 2048 (at most eight rows per tile).
template <bool ONE_PASS>
__global__ __launch_bounds__(BATCH_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemv_batch_kernel(BatchParams B) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int b = blockIdx.x;
    int j = B.n - 1, nblk = 0;
    for (; j >= 0; --j) {
        nblk = batch_blocks(B.e[j].rows, B.e[j].k, B.tiles_per_block);
        if (b < nblk) break;
        b -= nblk;
    }
    if (j < 0) return;
    GemvParams P{};
    derive_plain(P, B.e[j].w, B.e[j].x, B.e[j].y, B.e[j].rows, B.e[j].k);
    gemv_m1_body<X_F32, true, ONE_PASS>(P, b, nblk, BATCH_THREADS, lds);
}

}  // namespace

}  // namespace w4a8
