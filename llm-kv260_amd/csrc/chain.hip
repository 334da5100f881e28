// The decode chain in one launch: every matrix of a token, in order, with
// the weights of the next matrices streaming while the current one is
// computed -- the split of the reference's gemv2 engine (hls/gemv2/gemv2.h:
// 1-18), whose fetch kernel streams the next matrix while the MAC kernel
// finishes the current one, and of its caller's prefetch of the next matrix
// after each MAC (board/tp/tp_llama.cpp:318-323, 364-368), built for one
// MI355X:
//
//  * One workgroup per CU (a cooperative launch, so all are resident), each
//    holding a ring of sixteen 9,216-byte tile slots in LDS (144 KB of its
//    160 KB) and the staged activation of the current matrix.
//  * Two streamer waves play the fetch kernel: they walk the workgroup's
//    tiles of every matrix of the chain in order and copy each one from HBM
//    straight into a free ring slot with buffer_load ... lds (no registers),
//    as far ahead as the ring allows -- about one transformer layer, since a
//    layer's share per CU is 15 tiles. A slot frees when the matrix (or,
//    past eight tiles, the round) that used it is done.
//  * Eight compute waves play the MAC kernel: per matrix they stage the
//    activation (the fused Q8_0 quantize of the M = 1 GEMV), then each takes
//    one tile of the round from the ring and computes it exactly as the
//    M = 1 GEMV does (same block dots, same ordered lane sums, same tree).
//  * Between matrices a grid barrier over sixteen device-scope counters
//    (chain_sync.h) replaces the kernel boundary: matrix j + 1 reads its
//    activation only after every workgroup has finished matrix j. When a
//    later step of the same launch reads this step's output as its
//    activation, the output is written through to the device's coherence
//    point and waited for before the barrier, and that step reads its
//    activation from there; other outputs and activations use the caches.
//  * Every wait is bounded: a poll that runs out of spins raises the abort
//    word, every workgroup then skips its remaining work but keeps the
//    workgroup barriers in step, and the last workgroup to leave restores
//    the barrier state (chain_sync.h). w4a8_chain_timeouts reports it.
//
// The streamers' waits are explicit (s_waitcnt vmcnt(n) with n the loads
// they issued after the tile they need), and the streamer code never reads
// LDS, so nothing makes it wait for loads it issued later. The compute waves
// never issue an LDS-DMA load.
#include <atomic>
#include <mutex>

#include "../../include/w4a8.h"
#include "chain_sync.h"
#include "gemv_tile.h"
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace cs = chain_sync;

namespace {

constexpr int CW = 8;                          // compute waves
constexpr int SW = 2;                          // streamer waves
constexpr int CHAIN_THREADS = 64 * (CW + SW);  // 640
constexpr int RING = 16;                       // tile slots
constexpr int PIECES = 9;                      // 1 KB loads per tile
// A streamer's tiles in flight: 6 (54 loads, under vmcnt's 63). With 1 or 2
// the streamers waited on their own loads and reached the workgroup barriers
// late (chain 441-447 us/step against 398).
constexpr int MAX_OUT_TILES = 6;
// Tiles a streamer issues once the grid barrier has passed, and once a
// round's tiles are ready: at most two each, so that no burst of 16 tiles per
// CU lands in the next barrier's window (nothing issued at the round's end).
constexpr int ISSUE_CAP = 2;
constexpr int ISSUE_CAP_B1 = 2;
constexpr int CHAIN_MIN_K = 2048;              // one pass of ordered sums per tile
constexpr int CHAIN_MAX_K = 8192;
constexpr size_t RING_BYTES = (size_t)RING * TILE_BYTES;
constexpr size_t CHAIN_LDS = RING_BYTES + x_lds_bytes(CHAIN_MAX_K / QK);
constexpr int DEFAULT_SPIN_LIMIT = 1 << 22;    // polls (~0.5 us each) before a wait gives up

// One step as the kernel takes it (32 bytes), its tile geometry worked out on
// the host so that the kernel divides nothing: C chunks per row, rpw rows per
// tile, and the step's tiles split over the G workgroups as tiles = tq * G +
// tr, workgroup g taking tq tiles plus one more when g < tr. geo packs
// C (6 bits) | rpw (4) | tr (11) | tq (11); rf packs rows (30 bits) and two
// flags: X_COH, x is an earlier step's output (read it from the coherence
// point), and Y_COH, y is a later step's x (write it through, and wait for
// it, before the barrier).
struct ChainStep {
    const uint8_t *w;
    const float *x;
    float *y;
    uint32_t rf;
    uint32_t geo;
};
constexpr uint32_t X_COH = 1u << 30, Y_COH = 1u << 31, ROWS_MASK = X_COH - 1;
constexpr uint32_t pack_geo(int C, int rpw, int tr, int tq) {
    return (uint32_t)C | ((uint32_t)rpw << 6) | ((uint32_t)tr << 10) | ((uint32_t)tq << 21);
}
constexpr int GEO_MAX_T = 2047;

// Passed by value (kernel arguments).
struct ChainArgs {
    int n;
    int spin_limit;
    ChainStep s[W4A8_CHAIN_MAX_STEPS];
    // Barrier counters, generation, abort word, exit ticket and timeout
    // count (chain_sync.h): device memory of this device, zero at first use.
    uint32_t *st;
};

// Shape of step j as the workgroup sees it.
struct StepShape {
    int C, rpw, tiles, lo, cnt;
    uint32_t tile_bytes, total_bytes;
};

__device__ __forceinline__ StepShape shape_of(const ChainStep &st, int g, int G) {
    StepShape s;
    const uint32_t geo = st.geo;
    const int tq = (int)(geo >> 21), tr = (int)((geo >> 10) & 2047u);
    s.C = (int)(geo & 63u);
    s.rpw = (int)((geo >> 6) & 15u);
    s.tiles = tq * G + tr;
    s.lo = g * tq + (g < tr ? g : tr);
    s.cnt = tq + (g < tr ? 1 : 0);
    s.tile_bytes = (uint32_t)(s.rpw * s.C * CHUNK_BYTES);
    s.total_bytes = (st.rf & ROWS_MASK) * (uint32_t)s.C * CHUNK_BYTES;
    return s;
}

__device__ __forceinline__ int rounds_of(int cnt) { return cnt > CW ? (cnt + CW - 1) / CW : 1; }

// Waves per tile: a step with fewer tiles per workgroup than compute waves
// shares each tile among S waves (a power of two), each computing 8 / S of
// the eight blocks of every chunk, so the latency of a small matrix is not
// one wave's whole tile. The streamers keep the same count to mirror the two
// extra barriers such a step takes.
__device__ __forceinline__ int split_of(int cnt) {
    if (cnt > CW / 2) return 1;
    if (cnt > CW / 4) return 2;
    if (cnt > CW / 8) return 4;
    return 8;
}

// Workgroup barrier. The compute waves first make their LDS writes visible;
// no wait on vector memory (the streamers' loads stay in flight).
__device__ __forceinline__ void wg_barrier_lds() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wg_barrier() { __asm__ volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void wait_vm0() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// s_waitcnt vmcnt(9 * newer): the wave's loads issued before its last
// `newer` tiles have landed (loads complete in order).
__device__ __forceinline__ void wait_tiles_but(int newer) {
    switch (newer) {
        case 0: __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 1: __asm__ volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
        case 2: __asm__ volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
        case 3: __asm__ volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
        case 4: __asm__ volatile("s_waitcnt vmcnt(36)" ::: "memory"); break;
        case 5: __asm__ volatile("s_waitcnt vmcnt(45)" ::: "memory"); break;
        default: __asm__ volatile("s_waitcnt vmcnt(54)" ::: "memory"); break;
    }
}

typedef __attribute__((address_space(3))) void lds_void;

// ---------------------------------------------------------------- streamer

// The streamer's walk over the workgroup's tiles of the whole chain, in
// order: sequence number q is tile `t` (local, 0 .. cnt - 1) of step `j`,
// whose descriptor and shape the cursor holds.
struct Cursor {
    int j, t;
    ChainStep d;
    StepShape sh;
};

__device__ __forceinline__ void cursor_skip_empty(const ChainArgs &A, Cursor &c, int g, int G) {
    while (c.j < A.n && c.t >= c.sh.cnt) {
        c.t -= c.sh.cnt;
        if (++c.j < A.n) {
            c.d = A.s[c.j];
            c.sh = shape_of(c.d, g, G);
        }
    }
}

__device__ __forceinline__ void issue_tile(const Cursor &c, uint8_t *ring, int q, int lane) {
    const StepShape &s = c.sh;
    const uint32_t off0 = (uint32_t)(s.lo + c.t) * s.tile_bytes;
    const uint32_t left = s.total_bytes - off0;
    const __amdgpu_buffer_rsrc_t rb = buffer_of(c.d.w + off0, left < s.tile_bytes ? left : s.tile_bytes);
    uint8_t *slot = ring + (size_t)(q % RING) * TILE_BYTES;
#pragma unroll
    for (int p = 0; p < PIECES; ++p)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(slot + 1024 * p), 16, 1024 * p + 16 * lane, 0, 0,
                                                 CACHE_NT);
}

__device__ void streamer(const ChainArgs &A, int g, int G, int s, uint8_t *ring) {
    const int lane = threadIdx.x & 63;
    Cursor c;
    c.j = 0;
    c.t = s;
    c.d = A.s[0];
    c.sh = shape_of(c.d, g, G);
    cursor_skip_empty(A, c, g, G);
    int next = s;          // next sequence number this streamer issues (s, s + SW, ...)
    int issued = 0;        // tiles this streamer has issued
    int landed = 0;        // of those, known to have landed
    auto issue_upto = [&](int limit, int cap) {
        for (int n_issued = 0; next < limit && c.j < A.n && n_issued < cap; ++n_issued) {
            if (issued - landed >= MAX_OUT_TILES) {
                wait_tiles_but(MAX_OUT_TILES - 1);
                landed = issued - (MAX_OUT_TILES - 1);
            }
            issue_tile(c, ring, next, lane);
            ++issued;
            next += SW;
            c.t += SW;
            cursor_skip_empty(A, c, g, G);
        }
    };
    issue_upto(RING, RING);
    int q = 0;
    for (int j = 0; j < A.n; ++j) {
        const int cnt = shape_of(A.s[j], g, G).cnt;
        if (j > 0) {
            wg_barrier();                                          // B0: the grid barrier passed
            issue_upto(q + RING, ISSUE_CAP);
        }
        const int rounds = rounds_of(cnt);
        for (int r = 0; r < rounds; ++r) {
            const int q0 = q + r * CW;
            const int q1 = q + (cnt < (r + 1) * CW ? cnt : (r + 1) * CW);
            // My last tile of the round: the largest q in [q0, q1) with q % SW == s.
            int last = q1 - 1 - (((q1 - 1 - s) % SW + SW) % SW);
            if (last >= q0) {
                const int idx = last / SW;                         // its index among my tiles
                if (idx >= landed) {
                    wait_tiles_but(issued - idx - 1);
                    landed = idx + 1;
                }
            }
            wg_barrier();                                          // B1: tiles and activation ready
            issue_upto(q0 + RING, ISSUE_CAP_B1);
            if (rounds == 1 && split_of(cnt) > 1) {
                wg_barrier();                                      // BT
                wg_barrier();                                      // BS
            }
            wg_barrier();                                          // B2: the round's slots are free
            if (rounds > 1) issue_upto(q1 + RING, RING);
        }
        q += cnt;
    }
    wait_vm0();   // nothing may land in LDS after the workgroup ends
}

// ---------------------------------------------------------------- compute

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}

// Q8_0 of values 4g .. 4g + 3 of activation block b, thread g (0..7) of an
// aligned group of eight (q4_0.py:83-97), written to the LDS column layout
// x_stage writes (gemv_tile.h) -- the same bytes, with each block shared by
// eight threads instead of done by one:
//  * amax is the group's max (DPP quad_perm [1,0,3,2], [2,3,0,1], then
//    row_half_mirror), so d and inv are those of a thread holding the block;
//  * the block's sum of int8 values is the group's sum (exact integer adds);
//  * the nibble split pairs dword m of the block with dword m + 4 (x_nibbles,
//    q4_0_device.h): thread g takes its partner g ^ 4's dword through
//    quad_perm [3,2,1,0] then row_half_mirror, and writes split word g.
// Every lane of the group must be active (the DPP moves read all eight).
__device__ __forceinline__ void stage8(const float4 v, int b, int g, bool live, uint32_t *s_x) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, dpp_mov<0xB1>(amax));
    amax = fmaxf(amax, dpp_mov<0x4E>(amax));
    amax = fmaxf(amax, dpp_mov<0x141>(amax));
    const float d = q8_scale(amax);
    const float inv = safe_recip(d);
    const uint32_t word = (uint32_t)(uint8_t)q8_round(v.x, inv) | ((uint32_t)(uint8_t)q8_round(v.y, inv) << 8) |
                          ((uint32_t)(uint8_t)q8_round(v.z, inv) << 16) | ((uint32_t)(uint8_t)q8_round(v.w, inv) << 24);
    int32_t sum = __builtin_amdgcn_sdot4((int)word, 0x01010101, 0, false);
    sum += (int32_t)dpp_u32<0xB1>((uint32_t)sum);
    sum += (int32_t)dpp_u32<0x4E>((uint32_t)sum);
    sum += (int32_t)dpp_u32<0x141>((uint32_t)sum);
    const uint32_t other = dpp_u32<0x141>(dpp_u32<0x1B>(word));
    const bool low = g < 4;
    const uint32_t lo = (low ? word : other) ^ 0x80808080u, hi = (low ? other : word) ^ 0x80808080u;
    const uint32_t xn = low ? (((lo >> 4) & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u))
                            : ((lo & 0x0F0F0F0Fu) | ((hi << 4) & 0xF0F0F0F0u));
    if (live) {
        uint32_t *col = s_x + (b >> 3) * XCOL_DWORDS;
        const int j = b & 7;
        col[8 * j + g] = xn;
        if (g == 0) {
            col[XCOL_D + j] = __float_as_uint(half_bits_to_float(float_to_half_bits(d)));
            col[XCOL_S + j] = (uint32_t)(-8 * sum);
        }
    }
}

constexpr int STAGE_GROUPS = CW * 64 / 8;                         // groups of eight compute threads
constexpr int STAGE_PASSES = CHAIN_MAX_K / QK / STAGE_GROUPS;      // blocks per group at the largest k

// The activation of a step, float32[k], quantized and staged in LDS by the
// compute threads: group `grp` takes blocks grp, grp + 64, ...; all its loads
// go out first. Coherent: read from the device's coherence point.
template <bool COHERENT>
__device__ __forceinline__ void stage_x(const float *x, int k, int tid, uint32_t *s_x) {
    const int nb = k >> 5, grp = tid >> 3, g = tid & 7;
    const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)(4 * k));
    float4 v[STAGE_PASSES];
#pragma unroll
    for (int p = 0; p < STAGE_PASSES; ++p) {
        const int b = grp + p * STAGE_GROUPS;
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(xb, b < nb ? 128 * b + 16 * g : OUT_OF_RANGE, 0,
                                                              COHERENT ? SC1 : 0);
        v[p] = make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
    }
#pragma unroll
    for (int p = 0; p < STAGE_PASSES; ++p) {
        const int b = grp + p * STAGE_GROUPS;
        if (p * STAGE_GROUPS < nb) stage8(v[p], b, g, b < nb, s_x);
    }
}

// Wave 0 of a workgroup: arrive at the barrier after step `b`, then wait for
// every workgroup. Returns false when the wait gave up or saw the abort word.
__device__ bool grid_barrier(uint32_t *st, int g, int G, uint32_t gen, int b, int spin_limit) {
    const int lane = threadIdx.x & 63;
    if (lane == 0)
        __hip_atomic_fetch_add(st + cs::counter_word(cs::counter_of(g)), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t ep = cs::epoch(gen, b);
    const uint32_t tag = cs::abort_tag(gen);
    // Lanes 0..15 watch the counters, lane 16 the abort word.
    const bool is_ctr = lane < cs::COUNTERS;
    const uint32_t *src = is_ctr ? st + cs::counter_word(lane) : st + cs::ABORT;
    const uint32_t want = is_ctr ? cs::target(lane, G, ep) : 0u;
    for (int spin = 0; spin < spin_limit; ++spin) {
        uint32_t v = 0;
        if (lane <= cs::COUNTERS) v = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__ballot(lane == cs::COUNTERS && v == tag)) return false;
        if (!__ballot(is_ctr && !cs::reached(v, want))) return true;
    }
    if (lane == 0) __hip_atomic_store(st + cs::ABORT, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

// One tile of step j, from ring slot `slot`, into y.
template <bool Y_SC1>
__device__ __forceinline__ void compute_tile(uint8_t *slot, const uint32_t xv[8][8], const float xd[8],
                                             const int32_t xs[8], int tile, int rpw, int C, int rows, float *y) {
    const int lane = threadIdx.x & 63;
    uint32_t w[CHUNK_DWORDS];
    {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(slot + CHUNK_BYTES * lane);
#pragma unroll
        for (int q = 0; q < CHUNK_PIECES; ++q) {
            const u32x4 v = src[q];
            w[4 * q] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
        }
    }
    float t[8];
    chunk_terms(w, xv, xd, xs, t);
    wave_sync_lds();
    float *s_t = reinterpret_cast<float *>(slot);
#pragma unroll
    for (int j = 0; j < 8; ++j) s_t[9 * lane + j] = t[j];
    wave_sync_lds();
    const int acc_r = lane >> 3, acc_a = lane & 7;
    const float yv = tree8_dpp(ordered_lane_sum(s_t, acc_r, rpw, C, acc_a));
    const int row = tile * rpw + acc_r;
    const bool mine = acc_r < rpw && acc_a == 0 && row < rows;
    const __amdgpu_buffer_rsrc_t yr = buffer_of(y, 4u * (uint32_t)rows);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv), yr, mine ? 4 * row : OUT_OF_RANGE, 0, Y_SC1 ? SC1 : 0);
}

// Block j of a chunk held in LDS as 36 dwords at `wd` (the layout chunk_block
// reads from registers; j is uniform across the wave).
__device__ __forceinline__ void lds_block(const uint32_t *wd, int j, uint32_t &d_bits, uint32_t qs[4]) {
    if ((j & 1) == 0) {
        const int base = (j >> 1) * 9;
        uint32_t w[5];
#pragma unroll
        for (int m = 0; m < 5; ++m) w[m] = wd[base + m];
        d_bits = w[0] & 0xFFFFu;
#pragma unroll
        for (int m = 0; m < 4; ++m) qs[m] = __builtin_amdgcn_alignbyte(w[m + 1], w[m], 2);
    } else {
        const int base = (j >> 1) * 9 + 4;
        d_bits = wd[base] >> 16;
#pragma unroll
        for (int m = 0; m < 4; ++m) qs[m] = wd[base + 1 + m];
    }
}

// Blocks j0 .. j0 + NB - 1 of this lane's chunk of the tile in `slot`, against
// activation column `colx`: their terms, written to the tile's term area
// (lane l, block j at 9 l + j) once every wave sharing the tile has read its
// blocks (the caller's barrier between the two calls).
template <int NB>
__device__ __forceinline__ void part_terms(const uint8_t *slot, const uint32_t *s_x, int lane, int colx, int j0,
                                           float t[NB]) {
    const uint32_t *wd = reinterpret_cast<const uint32_t *>(slot + CHUNK_BYTES * lane);
    const uint32_t *col = s_x + colx * XCOL_DWORDS;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int jj = j0 + i;
        uint32_t d_bits, qs[4];
        lds_block(wd, jj, d_bits, qs);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(col + 8 * jj);
        const u32x4 a = src[0], c = src[1];
        const uint32_t xv[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        const int32_t sumi = block_dot_nib(qs, xv, (int32_t)col[XCOL_S + jj]);
        t[i] = block_term(sumi, d_bits, __uint_as_float(col[XCOL_D + jj]));
    }
}

// The ordered lane sums, tree and store of one tile whose terms are in `slot`.
template <bool Y_SC1>
__device__ __forceinline__ void tile_finish(const uint8_t *slot, int tile, int rpw, int C, int rows, float *y) {
    const int lane = threadIdx.x & 63;
    const float *s_t = reinterpret_cast<const float *>(slot);
    const int acc_r = lane >> 3, acc_a = lane & 7;
    const float yv = tree8_dpp(ordered_lane_sum(s_t, acc_r, rpw, C, acc_a));
    const int row = tile * rpw + acc_r;
    const bool mine = acc_r < rpw && acc_a == 0 && row < rows;
    const __amdgpu_buffer_rsrc_t yr = buffer_of(y, 4u * (uint32_t)rows);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv), yr, mine ? 4 * row : OUT_OF_RANGE, 0, Y_SC1 ? SC1 : 0);
}

template <int NB, bool Y_SC1>
__device__ __forceinline__ void shared_tile(uint8_t *slot, const uint32_t *s_x, int lane, int colx, int h, bool live,
                                            int tile, int rpw, int C, int rows, float *y) {
    float t[NB];
    if (live) part_terms<NB>(slot, s_x, lane, colx, h * NB, t);
    wg_barrier_lds();                                              // BT: every part read its blocks
    if (live) {
        float *s_t = reinterpret_cast<float *>(slot);
#pragma unroll
        for (int i = 0; i < NB; ++i) s_t[9 * lane + h * NB + i] = t[i];
    }
    wg_barrier_lds();                                              // BS: the tile's terms are complete
    if (live && h == 0) tile_finish<Y_SC1>(slot, tile, rpw, C, rows, y);
}

__device__ void compute(const ChainArgs &A, int g, int G, uint8_t *ring, uint32_t *s_x, uint32_t *s_quit, int wave) {
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t gen = 0;
    if (wave == 0) gen = __hip_atomic_load(A.st + cs::GEN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool quit = false;
    int q = 0;
    // Lines of the next step's activation, loaded while this step runs so that
    // its staging after the barrier hits L2 (warming only: the values staged
    // are loaded again after the barrier). Folded into `warm` one step later,
    // when the loads have long landed.
    uint32_t warm = 0, warm_next = 0;
    // Each step's descriptor is loaded one step ahead: a kernel argument's
    // first read misses the scalar cache, and this one would sit right after
    // the barrier.
    ChainStep cur = A.s[0];
    for (int j = 0; j < A.n; ++j) {
        const ChainStep nxt = A.s[j + 1 < A.n ? j + 1 : j];
        const StepShape s = shape_of(cur, g, G);
        const int rows = (int)(cur.rf & ROWS_MASK);
        if (j > 0) {
            if (wave == 0) {
                const bool ok = quit ? false : grid_barrier(A.st, g, G, gen, j - 1, A.spin_limit);
                if (lane == 0) *s_quit = ok ? 0u : 1u;
            }
            wg_barrier_lds();                                      // B0
            quit = *s_quit != 0;
        }
        const int k = s.C << 8;
        warm ^= warm_next;
        if (!quit) {
            if (cur.rf & X_COH)
                stage_x<true>(cur.x, k, tid, s_x);
            else
                stage_x<false>(cur.x, k, tid, s_x);
            // An activation that is an earlier step's output is read from the
            // coherence point, past L2: nothing to warm.
            if (j + 1 < A.n && !(nxt.rf & X_COH)) {
                const int k1 = (int)(nxt.geo & 63u) << 8;
                const __amdgpu_buffer_rsrc_t xb = buffer_of(nxt.x, (uint32_t)(4 * k1));
                warm_next = __builtin_amdgcn_raw_buffer_load_b32(xb, 64 * tid, 0, 0);   // one dword per 64-byte line
            }
        }
        const int rounds = rounds_of(s.cnt);
        const int S = rounds > 1 ? 1 : split_of(s.cnt);
        const int colx = lane / s.C < s.rpw ? lane % s.C : 0;
        const bool ycoh = (cur.rf & Y_COH) != 0;
        if (S == 1) {
            uint32_t xv[8][8];
            float xd[8];
            int32_t xs[8];
            for (int r = 0; r < rounds; ++r) {
                wg_barrier_lds();                                  // B1
                if (r == 0) {
                    const uint32_t *col = s_x + colx * XCOL_DWORDS;
#pragma unroll
                    for (int b = 0; b < 8; ++b) {
                        const u32x4 *src = reinterpret_cast<const u32x4 *>(col + 8 * b);
                        const u32x4 a = src[0], c = src[1];
                        xv[b][0] = a.x; xv[b][1] = a.y; xv[b][2] = a.z; xv[b][3] = a.w;
                        xv[b][4] = c.x; xv[b][5] = c.y; xv[b][6] = c.z; xv[b][7] = c.w;
                        xd[b] = __uint_as_float(col[XCOL_D + b]);
                        xs[b] = (int32_t)col[XCOL_S + b];
                    }
                }
                const int mine = r * CW + wave;
                if (!quit && mine < s.cnt) {
                    uint8_t *slot = ring + (size_t)((q + mine) % RING) * TILE_BYTES;
                    if (ycoh)
                        compute_tile<true>(slot, xv, xd, xs, s.lo + mine, s.rpw, s.C, rows, cur.y);
                    else
                        compute_tile<false>(slot, xv, xd, xs, s.lo + mine, s.rpw, s.C, rows, cur.y);
                }
                if (r == rounds - 1 && ycoh) wait_vm0();           // y visible before the barrier
                wg_barrier_lds();                                  // B2
            }
        } else {
            wg_barrier_lds();                                      // B1
            const int ti = wave / S, h = wave % S;
            const bool live = !quit && ti < s.cnt;
            uint8_t *slot = ring + (size_t)((q + (live ? ti : 0)) % RING) * TILE_BYTES;
            const int tile = s.lo + ti;
            switch (S) {
                case 2:
                    if (ycoh) shared_tile<4, true>(slot, s_x, lane, colx, h, live, tile, s.rpw, s.C, rows, cur.y);
                    else shared_tile<4, false>(slot, s_x, lane, colx, h, live, tile, s.rpw, s.C, rows, cur.y);
                    break;
                case 4:
                    if (ycoh) shared_tile<2, true>(slot, s_x, lane, colx, h, live, tile, s.rpw, s.C, rows, cur.y);
                    else shared_tile<2, false>(slot, s_x, lane, colx, h, live, tile, s.rpw, s.C, rows, cur.y);
                    break;
                default:
                    if (ycoh) shared_tile<1, true>(slot, s_x, lane, colx, h, live, tile, s.rpw, s.C, rows, cur.y);
                    else shared_tile<1, false>(slot, s_x, lane, colx, h, live, tile, s.rpw, s.C, rows, cur.y);
                    break;
            }
            if (ycoh) wait_vm0();                                  // y visible before the barrier
            wg_barrier_lds();                                      // B2
        }
        q += s.cnt;
        cur = nxt;
    }
    // Keeps the warming loads (never true: spin_limit > 0).
    if (A.spin_limit < 0 && (warm ^ warm_next) == 0x5eed) A.st[cs::TIMEOUTS + 1] = warm;
    // Leave: the last workgroup out advances the generation, or restores the
    // barrier state after an abort.
    if (wave == 0 && lane == 0) {
        uint32_t *st = A.st;
        wait_vm0();   // this workgroup's arrivals and abort store are performed before its ticket
        const uint32_t t = __hip_atomic_fetch_add(st + cs::TICKET, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == (uint32_t)(G - 1)) {
            const uint32_t ab = __hip_atomic_load(st + cs::ABORT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ab == cs::abort_tag(gen)) {
                for (int c = 0; c < cs::COUNTERS; ++c)
                    __hip_atomic_store(st + cs::counter_word(c), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(st + cs::GEN, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(st + cs::ABORT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(st + cs::TIMEOUTS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __hip_atomic_store(st + cs::GEN, gen + (uint32_t)(A.n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(st + cs::TICKET, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

__global__ __launch_bounds__(CHAIN_THREADS) void chain_kernel(ChainArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t *ring = lds;
    uint32_t *s_x = reinterpret_cast<uint32_t *>(lds + RING_BYTES);
    __shared__ uint32_t s_quit;
    // The wave index as a scalar: everything the streamers derive from it
    // (tile walks, buffer resources, the kernel arguments they index) then
    // stays in SGPRs, with scalar loads that never wait behind their DMA.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave < CW)
        compute(A, blockIdx.x, gridDim.x, ring, s_x, &s_quit, wave);
    else
        streamer(A, blockIdx.x, gridDim.x, wave - CW, ring);
}

std::atomic<int> g_spin_limit{DEFAULT_SPIN_LIMIT};

// The barrier state of each device, allocated and zeroed at its first
// one-launch chain (device memory: a code object's __device__ array served
// the polls about 1 us slower per barrier on MI355X).
constexpr int MAX_DEVICES = 64;
std::mutex g_state_mu;
uint32_t *g_state[MAX_DEVICES];

hipError_t chain_state(uint32_t **out, bool create) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_state_mu);
    if (!g_state[dev] && create) {
        uint32_t *p = nullptr;
        e = hipMalloc(&p, cs::WORDS * sizeof(uint32_t));
        if (e != hipSuccess) return e;
        e = hipMemset(p, 0, cs::WORDS * sizeof(uint32_t));
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipFree(p);
            return e;
        }
        g_state[dev] = p;
    }
    *out = g_state[dev];
    return hipSuccess;
}
std::atomic<int> g_chain_mode{1};   // W4A8_CHAIN_PER_STEP

bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
    return pa < pb + nb && pb < pa + na;
}

}  // namespace

bool chain_one_launch_fits(const w4a8_chain_step *steps, int n) {
    if (g_chain_mode.load(std::memory_order_relaxed) != 0) return false;
    for (int i = 0; i < n; ++i) {
        const int k = steps[i].k;
        if (k < CHAIN_MIN_K || k > CHAIN_MAX_K || k % 256) return false;
        // Tile offsets and the buffer resources' sizes are 32-bit.
        if ((size_t)steps[i].rows * (size_t)(k / 32 * 18) >= (1ull << 31)) return false;
    }
    return true;
}

hipError_t launch_chain_one(const w4a8_chain_step *steps, int n, hipStream_t stream) {
    ChainArgs A{};
    A.n = n;
    A.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
    const int grid = device_cu_count();
    for (int i = 0; i < n; ++i) {
        const int C = steps[i].k / 256, rpw = 64 / C;
        const int tiles = (steps[i].rows + rpw - 1) / rpw;
        if (tiles / grid > GEO_MAX_T || grid > GEO_MAX_T + 1) return hipErrorInvalidValue;
        A.s[i] = ChainStep{static_cast<const uint8_t *>(steps[i].w), steps[i].x, steps[i].y, (uint32_t)steps[i].rows,
                           pack_geo(C, rpw, tiles % grid, tiles / grid)};
    }
    // Which outputs feed a later step's activation within this launch; and
    // outputs that share bytes with another step's output, which are written
    // through as well: the two steps map those rows to different workgroups,
    // and so to different XCDs' L2s, whose dirty copies the launch's closing
    // release would write back in no defined order.
    for (int j = 0; j < n; ++j)
        for (int i = 0; i < j; ++i) {
            if (overlaps(steps[j].x, 4 * (size_t)steps[j].k, steps[i].y, 4 * (size_t)steps[i].rows)) {
                A.s[j].rf |= X_COH;
                A.s[i].rf |= Y_COH;
            }
            if (overlaps(steps[j].y, 4 * (size_t)steps[j].rows, steps[i].y, 4 * (size_t)steps[i].rows)) {
                A.s[j].rf |= Y_COH;
                A.s[i].rf |= Y_COH;
            }
        }
    hipError_t e = allow_dynamic_lds(reinterpret_cast<const void *>(&chain_kernel), 160 * 1024);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    hipError_t oe = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&chain_kernel),
                                                                 CHAIN_THREADS, CHAIN_LDS);
    if (oe != hipSuccess) return oe;
    if (per_cu < 1) return hipErrorCooperativeLaunchTooLarge;
    // The state is made once per device, outside any capture: a chain first
    // met under stream capture runs one launch per step (capturable).
    uint32_t *st = nullptr;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess) return e;
    e = chain_state(&st, cap == hipStreamCaptureStatusNone);
    if (e != hipSuccess) return e;
    if (!st) return hipErrorCooperativeLaunchTooLarge;
    A.st = st;
    void *args[] = {&A};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&chain_kernel), dim3(grid), dim3(CHAIN_THREADS),
                                      args, CHAIN_LDS, stream);
}

void chain_set_spin_limit(int polls) { g_spin_limit.store(polls > 0 ? polls : DEFAULT_SPIN_LIMIT); }
void chain_set_mode(int mode) { g_chain_mode.store(mode); }
int chain_mode() { return g_chain_mode.load(); }

hipError_t chain_take_timeouts(int *out) {
    *out = 0;
    uint32_t *st = nullptr;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = chain_state(&st, false);
    if (e != hipSuccess || !st) return e;
    uint32_t v = 0;
    e = hipMemcpy(&v, st + cs::TIMEOUTS, sizeof(v), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    if (v) {
        e = hipMemset(st + cs::TIMEOUTS, 0, sizeof(uint32_t));
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) return e;
    }
    *out = (int)v;
    return hipSuccess;
}

}  // namespace w4a8
