// W4A8 GEMV for a few tokens at once (2 <= m <= 8): Y[t][n] = W[n, K] x_t for
// m engine-layout activation rows, each output byte-identical to the M = 1
// GEMV on that row alone (the contract takes one x at a time,
// src/llm_kv260/q4_0.py:164-165).
//
// At small m the work is still the weight stream: m = 8 adds 0.4% to the
// bytes of an 8,192-column matrix. So this is the M = 1 kernel's streaming
// (gemv_m1.hip) with the arithmetic repeated per token, not a contraction on
// MFMA, whose 16-token tiles would be mostly padding here:
//  * Each wave streams 9,216-byte tiles of whole rows with nine coalesced
//    16-byte raw buffer loads per lane, two tiles in flight, through a per-wave
//    LDS slab, so that lane l holds chunk l (eight consecutive blocks of a
//    row, 144 bytes).
//  * A lane pulls its eight blocks' fp16 scales and packed nibbles out of the
//    chunk once; each block's nibbles are unpacked to bytes once and meet
//    every token's int8 values in v_dot4_i32_i8 block dots (block_dot_raw,
//    q4_0_device.h: eight dots per block and token, where the M = 1 GEMV's
//    nibble-split form takes twelve and two integer ops).
//  * Per token it reads its chunk column of that token's staged activation
//    (LDS, one copy per token, the layout x_stage writes, with the int8
//    values as they are) and computes the eight terms (f32(sumi) * d_w) *
//    d_x, then the contract's ordered lane sums and adjacent-pair tree
//    through the slab, exactly as for M = 1.
// The activation rows are staged once per workgroup, their loads issued
// before the first weight tile's so that the staging waits for them only.
#include <atomic>

#include "../../include/w4a8.h"
#include "gemv_tile.h"
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

constexpr int MT_MAX = 8;                        // tokens per launch
constexpr int MT_THREADS = 512;
constexpr size_t MT_LDS_BUDGET = 160 * 1024;


struct MtParams {
    const uint8_t *w;
    const uint8_t *x;      // m rows of the engine layout, x_stride bytes apart
    float *y;              // y[m][rows]
    int m, rows, k, C, rpw, tiles, x_stride;
    uint32_t nb_mul, c_mul, tok_mul;   // div_mul of k / 32, C and 8 rpw
};

// n / d for 0 <= n < 2^16 and 2 <= d <= 2^16 as one high multiply by
// m = floor(2^32 / d) + 1 (div_mul), in place of the VALU division sequence
// the compiler emits for a run-time divisor. Exact: n m / 2^32 = n / d + n e
// / 2^32 with 0 < e <= 1, the excess is below 2^-16 <= 1 / d, and the
// fractional part of n / d is at most 1 - 1 / d.
__host__ __device__ constexpr uint32_t div_mul(uint32_t d) { return (uint32_t)((1ull << 32) / d + 1); }
__device__ __forceinline__ int small_div(int n, uint32_t mul) { return (int)__umulhi((uint32_t)n, mul); }

struct MtTile {
    u32x4 p[CHUNK_PIECES];
};

// Tile `tile` of the matrix (lane l: bytes 1024 p + 16 l of it); a tile past
// the end reads nothing, and the last tile's bytes past the matrix read zeros.
__device__ __forceinline__ void mt_load_tile(const MtParams &P, int tile, int lane, MtTile &t) {
    const size_t tile_bytes = (size_t)P.rpw * (size_t)P.C * CHUNK_BYTES;
    const size_t total = (size_t)P.rows * (size_t)P.C * CHUNK_BYTES;
    const size_t off0 = (size_t)__builtin_amdgcn_readfirstlane(tile) * tile_bytes;
    const bool in = off0 < total;
    const uint32_t n = in ? (uint32_t)(total - off0 < (size_t)TILE_BYTES ? total - off0 : (size_t)TILE_BYTES) : 0u;
    const __amdgpu_buffer_rsrc_t tb = buffer_of(P.w + (in ? off0 : 0), n);
#pragma unroll
    for (int p = 0; p < CHUNK_PIECES; ++p) t.p[p] = __builtin_amdgcn_raw_buffer_load_b128(tb, 1024 * p + 16 * lane, 0, CACHE_NT);
}

// The eight block terms of this lane's chunk for TG tokens t0 .. t0 + TG - 1
// (a token past m reads token `past` instead and is never stored): each
// block's weights unpacked to bytes once, then one v_dot4 block dot per token
// (block_dot_raw) on the token's staged int8 values, and the contract's term.
template <int TG>
__device__ __forceinline__ void mt_terms(const uint32_t qs[8][4], const uint32_t dw[8], const uint32_t *s_x,
                                         int tok_dwords, int colx, int t0, int m, float term[TG][8], int past = -1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t lo[4], hi[4];
        unpack_nibbles(qs[j], lo, hi);
#pragma unroll
        for (int u = 0; u < TG; ++u) {
            const int t = t0 + u < m ? t0 + u : (past < 0 ? t0 : past);
            const uint32_t *col = s_x + t * tok_dwords + colx * XCOL_DWORDS;
            const u32x4 *src = reinterpret_cast<const u32x4 *>(col + 8 * j);
            const u32x4 a = src[0], c = src[1];
            const uint32_t xr[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            const int32_t sumi = block_dot_raw(lo, hi, xr, (int32_t)col[XCOL_S + j]);
            term[u][j] = block_term(sumi, dw[j], __uint_as_float(col[XCOL_D + j]));
        }
    }
}

// PASSES: staging rounds of blocks per thread, m * nb <= PASSES * threads.
// TG: tokens computed per round of ordered sums.
// SHARED_SUMS: a tile's rows take at most 32 lanes per token (K >= 4096), so
// the ordered sums of several tokens share one pass (otherwise one per token).
template <int PASSES, int TG, bool SHARED_SUMS>
__device__ void gemv_mt_body(const MtParams &P, int block, int nblocks, uint8_t *lds) {
    const int nb = P.k >> 5;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nthreads = blockDim.x, waves = nthreads >> 6;
    uint8_t *slab = lds + (size_t)wave * TILE_BYTES;
    uint32_t *s_x = reinterpret_cast<uint32_t *>(lds + (size_t)waves * TILE_BYTES);
    const int tok_dwords = (int)(x_lds_bytes(nb) / 4);

    const int C = P.C, rpw = P.rpw;
    const int my_r = small_div(lane, P.c_mul), my_c = lane - my_r * C;
    const int colx = my_r < rpw ? my_c : 0;

    // 1. The activation rows' loads, before any weight tile's.
    XRaw<X_ENGINE> xr[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int i = tid + p * nthreads;
        const int t = small_div(i, P.nb_mul), b = i - t * nb;
        const bool live = t < P.m;
        x_load<X_ENGINE>(P.x + (size_t)(live ? t : 0) * P.x_stride, P.k, b, live, xr[p]);
    }

    int tile = block * waves + wave;
    const int tstride = nblocks * waves;
    // Tiles of this wave; the division only where a wave has two or more.
    const int n_my = tile >= P.tiles ? 0 : tile + tstride >= P.tiles ? 1 : (P.tiles - 1 - tile) / tstride + 1;

    auto stage_x = [&]() {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int i = tid + p * nthreads;
            const int t = small_div(i, P.nb_mul), b = i - t * nb;
            if (t < P.m) x_stage<X_ENGINE, true>(xr[p], b, s_x + t * tok_dwords);
        }
        __syncthreads();
    };

    const int acc_r = lane >> 3, acc_a = lane & 7;
    const __amdgpu_buffer_rsrc_t y_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(P.y, 0, 4 * P.rows * P.m, BUFFER_DWORD3);

    // One tile: buffer -> slab -> chunk -> blocks; then per token: terms ->
    // slab -> ordered lane sums -> tree -> y[t][row]. With refill the buffer
    // then receives the tile two strides ahead.
    auto step = [&](MtTile &bt, bool refill) {
        u32x4 *wslab = reinterpret_cast<u32x4 *>(slab);
#pragma unroll
        for (int p = 0; p < CHUNK_PIECES; ++p) wslab[64 * p + lane] = bt.p[p];
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
        if (refill) mt_load_tile(P, tile + 2 * tstride, lane, bt);
        uint32_t qs[8][4], dw[8];
#define W4A8_BLK(J) chunk_block<J>(w, dw[J], qs[J]);
        W4A8_BLK(0) W4A8_BLK(1) W4A8_BLK(2) W4A8_BLK(3) W4A8_BLK(4) W4A8_BLK(5) W4A8_BLK(6) W4A8_BLK(7)
#undef W4A8_BLK
        float *s_t = reinterpret_cast<float *>(slab);
        const int row = tile * rpw + acc_r;
        const bool mine = acc_r < rpw && acc_a == 0 && row < P.rows;
        // Tokens in groups of TG (2 or 4): their terms take TG x 64 lanes x 9
        // floats of the slab (all of it at TG = 4), so each group takes one
        // pair of syncs.
        for (int t0 = 0; t0 < P.m; t0 += TG) {
            float term[TG][8];
            mt_terms<TG>(qs, dw, s_x, tok_dwords, colx, t0, P.m, term);
            wave_sync_lds();
#pragma unroll
            for (int u = 0; u < TG; ++u)
#pragma unroll
                for (int j = 0; j < 8; ++j) s_t[u * 576 + 9 * lane + j] = term[u][j];
            wave_sync_lds();
            // Ordered sums. A tile's rows take 8 rpw lanes per token: all 64
            // at K = 2048, one token at a time; 16 at K = 8192, where lane
            // (u, r, a) takes accumulator a of row r of token u0 + u and one
            // pass serves four tokens, their dependent adds side by side
            // (down at M = 3, 4: 6.8-7.0 us against 7.5-7.6 one token at a
            // time).
            if constexpr (!SHARED_SUMS) {
#pragma unroll
                for (int u = 0; u < TG; ++u) {
                    const float yv = tree8_dpp(ordered_lane_sum(s_t + u * 576, acc_r, rpw, C, acc_a));
                    const bool store = mine && t0 + u < P.m;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv), y_rsrc,
                                                          store ? 4 * ((t0 + u) * P.rows + row) : OUT_OF_RANGE, 0, 0);
                }
            } else {
                const int per_tok = 8 * rpw, tok_pass = small_div(64, P.tok_mul);
                const int sum_u = small_div(lane, P.tok_mul), sum_r = (lane - sum_u * per_tok) >> 3;
                const int srow = tile * rpw + sum_r;
                for (int u0 = 0; u0 < TG; u0 += tok_pass) {
                    const int u = u0 + sum_u;
                    const bool live = sum_u < tok_pass && u < TG;
                    const float yv = tree8_dpp(ordered_lane_sum(s_t + (live ? u : u0) * 576, sum_r, rpw, C, acc_a));
                    const bool store = live && acc_a == 0 && sum_r < rpw && srow < P.rows && t0 + u < P.m;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv), y_rsrc,
                                                          store ? 4 * ((t0 + u) * P.rows + srow) : OUT_OF_RANGE, 0, 0);
                }
            }
        }
        wave_sync_lds();
        tile += tstride;
    };

    // 2. Straight-line paths per wave (no tile, one tile, or the two-deep
    // pipeline), so that every wait on the loads in flight is exact.
    if (n_my >= 2) {
        MtTile buf[2];
        mt_load_tile(P, tile, lane, buf[0]);
        mt_load_tile(P, tile + tstride, lane, buf[1]);
        stage_x();
        int done = 0;
        for (; done + 2 <= n_my; done += 2) {
            step(buf[0], true);
            step(buf[1], true);
        }
        if (done < n_my) step(buf[0], false);
    } else if (n_my == 1) {
        MtTile b;
        mt_load_tile(P, tile, lane, b);
        stage_x();
        step(b, false);
    } else {
        stage_x();
    }
}

// Few tiles per CU (at most four: down at K = 8192): one tile per pair of
// waves, each wave computing half the tokens, so that a SIMD holds two waves
// whose LDS reads and dependent adds interleave, where one wave per SIMD
// left them exposed. The pair loads the tile together (pieces 0-4 and 5-8),
// stages it in the pair's slab, and after a workgroup barrier each wave
// pulls its chunk. The pair's second buffer takes wave 1's terms, and the
// slab, once both chunks are pulled, wave 0's. Every wave has exactly one
// tile (the grid is sized so); past the last tile its loads read nothing and
// it stores nothing. TG: tokens per wave, ceil(m / 2).
template <int PASSES, int TG>
__device__ void gemv_mt_split_body(const MtParams &P, int block, uint8_t *lds) {
    const int nb = P.k >> 5;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nthreads = blockDim.x, waves = nthreads >> 6, pairs = waves >> 1;
    const int slot = wave >> 1, half = wave & 1;
    uint8_t *slab = lds + (size_t)slot * 2 * TILE_BYTES;
    float *s_t = reinterpret_cast<float *>(slab + (size_t)half * TILE_BYTES);
    uint32_t *s_x = reinterpret_cast<uint32_t *>(lds + (size_t)waves * TILE_BYTES);
    const int tok_dwords = (int)(x_lds_bytes(nb) / 4);

    const int C = P.C, rpw = P.rpw;
    const int my_r = small_div(lane, P.c_mul), my_c = lane - my_r * C;
    const int colx = my_r < rpw ? my_c : 0;

    // 1. The activation rows' loads, then this wave's pieces of the tile.
    XRaw<X_ENGINE> xr[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int i = tid + p * nthreads;
        const int t = small_div(i, P.nb_mul), b = i - t * nb;
        const bool live = t < P.m;
        x_load<X_ENGINE>(P.x + (size_t)(live ? t : 0) * P.x_stride, P.k, b, live, xr[p]);
    }
    const int tile = block * pairs + slot;
    u32x4 pc[5];
    {
        const size_t tile_bytes = (size_t)rpw * (size_t)C * CHUNK_BYTES;
        const size_t total = (size_t)P.rows * (size_t)C * CHUNK_BYTES;
        const size_t off0 = (size_t)__builtin_amdgcn_readfirstlane(tile) * tile_bytes;
        const bool in = off0 < total;
        const uint32_t n = in ? (uint32_t)(total - off0 < (size_t)TILE_BYTES ? total - off0 : (size_t)TILE_BYTES) : 0u;
        const __amdgpu_buffer_rsrc_t tb = buffer_of(P.w + (in ? off0 : 0), n);
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const int p = 5 * half + q;      // wave 1's fifth slot (p = 9) reads out of range
            pc[q] = __builtin_amdgcn_raw_buffer_load_b128(tb, p < CHUNK_PIECES ? 1024 * p + 16 * lane : OUT_OF_RANGE,
                                                          0, CACHE_NT);
        }
    }
    // 2. Stage the activation; the tile into the slab; each wave's chunk.
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int i = tid + p * nthreads;
        const int t = small_div(i, P.nb_mul), b = i - t * nb;
        if (t < P.m) x_stage<X_ENGINE, true>(xr[p], b, s_x + t * tok_dwords);
    }
    {
        u32x4 *wslab = reinterpret_cast<u32x4 *>(slab);
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const int p = 5 * half + q;
            if (p < CHUNK_PIECES) wslab[64 * p + lane] = pc[q];
        }
    }
    __syncthreads();
    uint32_t w[CHUNK_DWORDS];
    {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(slab + CHUNK_BYTES * lane);
#pragma unroll
        for (int q = 0; q < CHUNK_PIECES; ++q) {
            const u32x4 v = src[q];
            w[4 * q] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
        }
    }
    __syncthreads();   // both chunks pulled: the slab takes wave 0's terms
    uint32_t qs[8][4], dw[8];
#define W4A8_BLK(J) chunk_block<J>(w, dw[J], qs[J]);
    W4A8_BLK(0) W4A8_BLK(1) W4A8_BLK(2) W4A8_BLK(3) W4A8_BLK(4) W4A8_BLK(5) W4A8_BLK(6) W4A8_BLK(7)
#undef W4A8_BLK

    // 3. This wave's tokens t0 .. t0 + TG - 1: terms, then their ordered sums
    // in as few passes as the lanes allow (8 rpw lanes per token).
    const int t0 = half * TG;
    float term[TG][8];
    mt_terms<TG>(qs, dw, s_x, tok_dwords, colx, t0, P.m, term, 0);
#pragma unroll
    for (int u = 0; u < TG; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) s_t[u * 576 + 9 * lane + j] = term[u][j];
    wave_sync_lds();
    const int acc_a = lane & 7;
    const __amdgpu_buffer_rsrc_t y_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(P.y, 0, 4 * P.rows * P.m, BUFFER_DWORD3);
    const int per_tok = 8 * rpw, tok_pass = small_div(64, P.tok_mul);
    const int sum_u = small_div(lane, P.tok_mul), sum_r = (lane - sum_u * per_tok) >> 3;
    const int srow = tile * rpw + sum_r;
    for (int u0 = 0; u0 < TG; u0 += tok_pass) {
        const int u = u0 + sum_u;
        const bool live = sum_u < tok_pass && u < TG;
        const float yv = tree8_dpp(ordered_lane_sum(s_t + (live ? u : u0) * 576, sum_r, rpw, C, acc_a));
        const bool store = live && acc_a == 0 && sum_r < rpw && srow < P.rows && t0 + u < P.m;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv), y_rsrc,
                                              store ? 4 * ((t0 + u) * P.rows + srow) : OUT_OF_RANGE, 0, 0);
    }
}

template <int PASSES, int TG>
__global__ __launch_bounds__(MT_THREADS) void gemv_mt_split_kernel(MtParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    gemv_mt_split_body<PASSES, TG>(P, blockIdx.x, lds);
}

template <int PASSES, int TG, bool SHARED_SUMS>
__global__ __launch_bounds__(MT_THREADS) void gemv_mt_kernel(MtParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    gemv_mt_body<PASSES, TG, SHARED_SUMS>(P, blockIdx.x, gridDim.x, lds);
}

template <int PASSES>
hipError_t launch_mt_pass(const MtParams &P, int grid, int threads, size_t lds, bool split, hipStream_t stream) {
    auto go = [&](const void *fn, auto kernel) {
        const hipError_t e = allow_dynamic_lds(fn, MT_LDS_BUDGET);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), lds, stream, P);
        return hipGetLastError();
    };
    if (split) {
        const int tg = (P.m + 1) / 2;
        if (tg <= 1) return go(reinterpret_cast<const void *>(&gemv_mt_split_kernel<PASSES, 1>), gemv_mt_split_kernel<PASSES, 1>);
        if (tg <= 2) return go(reinterpret_cast<const void *>(&gemv_mt_split_kernel<PASSES, 2>), gemv_mt_split_kernel<PASSES, 2>);
        if (tg <= 3) return go(reinterpret_cast<const void *>(&gemv_mt_split_kernel<PASSES, 3>), gemv_mt_split_kernel<PASSES, 3>);
        return go(reinterpret_cast<const void *>(&gemv_mt_split_kernel<PASSES, 4>), gemv_mt_split_kernel<PASSES, 4>);
    }
    if (P.rpw <= 4) {
        if (P.m <= 2)
            return go(reinterpret_cast<const void *>(&gemv_mt_kernel<PASSES, 2, true>), gemv_mt_kernel<PASSES, 2, true>);
        return go(reinterpret_cast<const void *>(&gemv_mt_kernel<PASSES, 4, true>), gemv_mt_kernel<PASSES, 4, true>);
    }
    if (P.m <= 2) return go(reinterpret_cast<const void *>(&gemv_mt_kernel<PASSES, 2, false>), gemv_mt_kernel<PASSES, 2, false>);
    return go(reinterpret_cast<const void *>(&gemv_mt_kernel<PASSES, 4, false>), gemv_mt_kernel<PASSES, 4, false>);
}

}  // namespace

bool gemv_mt_fits(int m, int rows, int k) {
    return m >= 2 && m <= MT_MAX && k >= 2048 && k <= 8192 && k % 256 == 0 &&
           (size_t)rows * (size_t)(k / QK * Q4_0_BYTES) < 0x7fff0000u && (size_t)m * rows * 4 < 0x7fff0000u;
}

int gemv_mt_max_m(int rows, int k) {
    // Measured on MI355X against the MFMA kernels (rotated weights, us, with
    // the v_dot4 block dots):
    //  * m = 2 on every shape (q|k|v 4.3 against 4.9, o 4.2 against 4.8,
    //    gate|up 6.6 against 8.4, down 5.5 against 9.5);
    //  * m = 3, 4 from K = 4096 or 8,192 rows on (4096 x 4096 5.8-5.9
    //    against 6.9, gate|up 8.0-8.1 against 8.3-8.4, 8192 x 2048 5.6-5.7
    //    against 6.4, down 6.5-6.6 against 9.3-9.4); below that slower
    //    (q|k|v 5.0-5.1 against 4.9);
    //  * where a tile's tokens are split over two waves (at most four tiles
    //    per CU): m <= 8 at K = 8192 (down 7.6 at m = 5, 6 and 8.2-8.3 at
    //    m = 7, 8, against 9.3-9.4), m <= 6 at K = 2048 (8192 x 2048 6.5
    //    against 6.9 at m = 5, 6; 7.2 against 7.0 at m = 7, 8); 4096 x 4096
    //    even at m = 5, 6.
    const int rpw = 64 / (k / 256 > 0 ? k / 256 : 1);
    const int tiles = (rows + rpw - 1) / rpw;
    if (tiles <= 4 * device_cu_count()) {
        if (k >= 8192) return 8;
        if (k == 2048 && rows >= 8192) return 6;
    }
    if (rows >= 8192 || k >= 4096) return 4;
    return 2;
}

hipError_t launch_gemv_mt(const uint8_t *w, const uint8_t *x, int m, float *y, int rows, int k, hipStream_t stream) {
    if (!gemv_mt_fits(m, rows, k)) return hipErrorInvalidValue;
    MtParams P{};
    P.w = w;
    P.x = x;
    P.y = y;
    P.m = m;
    P.rows = rows;
    P.k = k;
    P.C = k / 256;
    P.rpw = 64 / P.C;
    P.tiles = (rows + P.rpw - 1) / P.rpw;
    P.nb_mul = div_mul((uint32_t)(k / QK));
    P.c_mul = div_mul((uint32_t)P.C);
    P.tok_mul = div_mul((uint32_t)(8 * P.rpw));
    P.x_stride = k + k / 8;
    const int nb = k / QK;
    const int cus = device_cu_count();
    // Launch shapes as for M = 1 (gemv_m1.hip), with workgroups of at least
    // four waves, so that the m activation rows are staged by enough threads:
    //  * up to eight tiles per CU (every layer matrix): one workgroup per CU
    //    at most, one tile per wave, every tile in flight at once;
    //  * more (the LM head): four-wave workgroups striding over the matrix,
    //    two per CU.
    int waves, grid;
    const bool split = P.tiles <= 4 * cus;
    if (split) {
        // One tile per pair of waves, four pairs per workgroup.
        waves = 8;
        grid = (P.tiles + 3) / 4;
    } else if (P.tiles <= 8 * cus) {
        const int per_cu = (P.tiles + cus - 1) / cus;
        waves = per_cu < 4 ? 4 : per_cu;
        grid = (P.tiles + waves - 1) / waves;
    } else {
        waves = 4;
        grid = (P.tiles + waves - 1) / waves;
        if (grid > 2 * cus) grid = 2 * cus;
    }
    const int threads = 64 * waves;
    const int passes = (m * nb + threads - 1) / threads;
    const size_t lds = (size_t)waves * TILE_BYTES + (size_t)m * x_lds_bytes(nb);
    if (lds > MT_LDS_BUDGET) return hipErrorInvalidValue;
    if (passes <= 1) return launch_mt_pass<1>(P, grid, threads, lds, split, stream);
    if (passes <= 2) return launch_mt_pass<2>(P, grid, threads, lds, split, stream);
    if (passes <= 4) return launch_mt_pass<4>(P, grid, threads, lds, split, stream);
    return launch_mt_pass<8>(P, grid, threads, lds, split, stream);
}

}  // namespace w4a8
