// Batched W4A8 (M > 1, prefill): Y[m][n] = sum over blocks of W[n] . X[m], for
// every (token m, row n) in the contract's order (src/llm_kv260/q4_0.py:170-182)
// exactly as the M = 1 kernel computes it.
//
// Here the work is a dense contraction, so the integer part runs on CDNA4 int8
// MFMA: v_mfma_i32_16x16x32_i8 multiplies a 16 (tokens) x 32 by a 32 x 16
// (rows) int8 tile. K = 32 is exactly one block, so each MFMA result is one
// block's exact int32 sum for 16 x 16 (token, row) pairs, never mixed across
// blocks. The weight operand is 16 (n - 8) as a signed byte: each nibble n
// moved to its byte's high half (the high nibbles are already there) and its
// top bit flipped, (n << 4) ^ 0x80, two operations a dword like the unsigned
// nibble's. The registers then hold 16 sum((n - 8) * x) exactly, and the
// block's scale is taken as d_w / 16 (exact: a power of two on an fp16
// value, never subnormal in fp32), so f32(16 sumi) * (d_w / 16) is the
// contract's f32(sumi) * d_w, the same real product rounded once.
//
// Operand layout of the 16x16x32 i8 MFMA (64 lanes, 8 int8 per lane):
//   A: lane l holds A[i = l % 16][k = 8 (l / 16) .. + 7]      (token i)
//   B: lane l holds B[k = 8 (l / 16) .. + 7][j = l % 16]      (row j)
//   D: lane l holds D[i = 4 (l / 16) + r][j = l % 16], r = 0..3
// Within a block, k-group g = 0..3 pairs x[8g .. 8g+7] with weights 8g .. 8g+7:
// the low nibbles of block bytes 0..7 (g = 0) and 8..15 (g = 1), then the high
// nibbles of bytes 0..7 (g = 2) and 8..15 (g = 3).
//
// Order. The contract's accumulator a (0..7) of an output adds the terms of
// blocks a, a + 8, a + 16, ... in that order, and never sees another block. A
// workgroup's eight waves share an item (16 rows x 16 MT tokens over all of
// K), and wave w owns accumulator a = w: it computes the terms of blocks
// 8c + w for c = 0, 1, ... in increasing order and adds each to its
// accumulator as it goes, from +0.0f. At the item's end the eight waves'
// accumulators of an output meet once, in the adjacent-pair tree.
//
// Data. What bounds this path is the bytes in flight and how many cache lines
// each load instruction touches, so every global load is a 16-byte piece of a
// contiguous run, 1 KB per wave instruction:
//  * A round is D consecutive chunks (8 D blocks, 256 D values of K) of one
//    item: the 16 rows' D * 144 weight bytes, each a contiguous run in the
//    ggml row, and the item's tokens' 256 D activation bytes and 8 D scales.
//  * All 512 threads load a round's pieces into registers P rounds ahead of
//    its use, and write it into one of two LDS round buffers once the round
//    before has been computed. One barrier per round separates the writes of
//    round q + 1 from the reads of round q - 1 in the same buffer.
//  * Each wave then reads its MFMA operands from LDS: the weight dwords of
//    block 8c + w of its row (realigned: a block starts every 18 bytes), one
//    8-byte activation piece per token tile, and the four token scales of its
//    output lanes as one 16-byte read (scales are stored block-major).
//  * Loads and the output stores are raw buffer accesses issued by every
//    thread in every round: lanes with nothing to move (rows past N, tokens
//    past M, rounds past the workgroup's last) are out of the buffer's range
//    and touch no memory. The number of memory operations in flight never
//    depends on data, so the wait before each round's LDS write is exact: it
//    waits for that round's loads only, with the next P - 1 rounds in flight.
// Workgroups are persistent over items; a workgroup's rounds form one stream
// that runs on across its items.
//
// Matrices of 8,192 rows and more go to gemm_rows.hip instead, which cuts the
// work along rows (two or four waves per 16-row group for the whole of K):
// with that many rows it fills the GPU without splitting K, and is faster.
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GW = 8;                  // waves per workgroup; wave w owns accumulator w
constexpr int GTHREADS = 64 * GW;
constexpr int NR = 16;                 // rows per item: the MFMA's 16 row columns
constexpr int OUT_OF_RANGE = 0x7ffffff0;
constexpr uint32_t BUFFER_DWORD3 = 0x00020000;
constexpr int CACHE_NT = 2;
constexpr int LDS_MAX = 160 * 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, BUFFER_DWORD3);
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// DPP quad broadcast of lane R of each quad (quad_perm [R, R, R, R]). With
// bound_ctrl set the compiler folds it into the consuming multiply as a DPP
// source (v_mul_f32_dpp), so it costs no instruction of its own.
template <int R>
__device__ __forceinline__ float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), R * 0x55, 0xF, 0xF, true));
}

struct GemmParams {
    const uint8_t *w;
    const uint8_t *x;      // m rows, engine layout
    float *y;              // [m][rows]
    int rows;
    int k;
    int m;
    int x_stride;          // bytes per activation row, k + k / 8
};

// Geometry of one instance: MT token tiles per item, D chunks per round, P
// rounds in flight, OCC workgroups per CU (the LDS of one is then at most
// LDS_MAX / OCC; with two, each SIMD runs four waves), NRL live rows per item
// (16, or 8 where 16-row items would leave CUs idle: the MFMA's row columns
// 8..15 then compute on whatever their LDS rows hold and are never stored).
template <int MT, int D, int P, int OCC, int NRL>
struct Geo {
    static constexpr int TT = 16 * MT;                      // tokens per item
    static constexpr int WP = D * CHUNK_BYTES + 16;         // LDS bytes per weight row (padded: bank spread)
    static constexpr int AP = D * 256 + 16;                 // LDS bytes per token's int8 slice
    static constexpr int W_OFF = 0;
    static constexpr int X_OFF = NR * WP;
    // fp32 scales [8 D blocks][XDP], tokens along a row. The pitch makes the
    // transposing writes (64 / TT pieces of consecutive tokens per wave
    // instruction, four rows apart) fall in distinct banks.
    static constexpr int XDP = TT < 64 ? TT + TT / 4 : TT;
    static constexpr int XD_OFF = X_OFF + TT * AP;
    static constexpr int BUF = XD_OFF + 8 * D * XDP * 4;    // one round
    // Exchange of the eight accumulators: [8][TT][EXP] fp32. Two of them
    // (consecutive items alternate) and a padded row pitch when they fit;
    // with one, the workgroup meets once more after each item's reduction.
    static constexpr int BUDGET = LDS_MAX / OCC;
    static constexpr int ex_bytes(int pitch) { return GW * TT * pitch * 4; }
    static constexpr int EXN = 2 * BUF + 2 * ex_bytes(NR) <= BUDGET ? 2 : 1;
    static constexpr int EXP = 2 * BUF + EXN * ex_bytes(NR + 4) <= BUDGET ? NR + 4 : NR;
    static constexpr int EX_BYTES = ex_bytes(EXP);
    static constexpr int EX_OFF = 2 * BUF;
    static constexpr int LDS = 2 * BUF + EXN * EX_BYTES;
    static_assert(LDS <= BUDGET, "round buffers exceed the LDS budget");
    static_assert(BUF < 65536, "a round buffer offset must fit an LDS instruction's immediate");
    // 16-byte pieces of a round and the load slots per thread that carry them.
    static_assert(NRL == 16 || NRL == 8, "an item is 16 or 8 rows");
    static constexpr int W_PIECES = NRL * D * 9;
    static constexpr int X_PIECES = TT * D * 16;
    static constexpr int XD_PIECES = TT * D * 2;
    static constexpr int SW = (W_PIECES + GTHREADS - 1) / GTHREADS;
    static constexpr int SX = (X_PIECES + GTHREADS - 1) / GTHREADS;
    static constexpr int SD = (XD_PIECES + GTHREADS - 1) / GTHREADS;
    static constexpr int OUTS = (TT * NR + GTHREADS - 1) / GTHREADS;   // outputs per thread per item
};

// One round's pieces in one thread's registers.
template <int SW, int SX, int SD>
struct Regs {
    u32x4 w[SW];
    u32x4 x[SX];
    u32x4 d[SD];
};

template <int MT, int D, int P, int OCC, int NRL, bool ODD>
struct Kernel {
    using G = Geo<MT, D, P, OCC, NRL>;
    using R = Regs<G::SW, G::SX, G::SD>;

    // Per-thread offsets of its load slots and outputs, fixed for the whole
    // launch. A round's loads go through buffer resources based at the
    // round's first row / token and chunk, whose size is the bytes the round
    // may read (zero for a dead round), so a lane's offset never changes and
    // the resource alone bounds every access: a row past N or a token past M
    // lies beyond the size. A slot with no piece has an offset beyond any size.
    struct Slots {
        uint32_t w_go[G::SW];
        int w_lo[G::SW];       // LDS byte offset in a round buffer; -1 when the slot carries no piece
        uint32_t x_go[G::SX];
        int x_lo[G::SX];
        uint32_t d_go[G::SD];
        int d_lo[G::SD];       // LDS float index of the first of the piece's four scales
        int o_ex[G::OUTS];     // exchange index of output o (accumulator 0)
        int o_tok[G::OUTS];    // its token and row in the item; INT_MAX when none
        int o_row[G::OUTS];
        uint32_t o_y[G::OUTS]; // its byte offset from the item's first output
    };

    static __device__ __forceinline__ void slots(const GemmParams &Pm, int row_bytes, Slots &s) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < G::SW; ++i) {
            const int q = i * GTHREADS + tid;
            const int r = q / (9 * D), p = q - r * (9 * D);
            const bool has = q < G::W_PIECES;
            s.w_go[i] = has ? (uint32_t)r * (uint32_t)row_bytes + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.w_lo[i] = has ? G::W_OFF + r * G::WP + 16 * p : -1;
        }
#pragma unroll
        for (int i = 0; i < G::SX; ++i) {
            const int q = i * GTHREADS + tid;
            const int t = q / (16 * D), p = q - t * (16 * D);
            const bool has = q < G::X_PIECES;
            s.x_go[i] = has ? (uint32_t)t * (uint32_t)Pm.x_stride + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.x_lo[i] = has ? G::X_OFF + t * G::AP + 16 * p : -1;
        }
#pragma unroll
        for (int i = 0; i < G::SD; ++i) {
            // Tokens fastest, so that the transposing LDS writes hit distinct banks.
            const int q = i * GTHREADS + tid;
            const int p = q / G::TT, t = q - p * G::TT;
            const bool has = q < G::XD_PIECES;
            s.d_go[i] = has ? (uint32_t)t * (uint32_t)Pm.x_stride + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.d_lo[i] = has ? G::XD_OFF / 4 + 4 * p * G::XDP + t : -1;
        }
#pragma unroll
        for (int o = 0; o < G::OUTS; ++o) {
            const int idx = o * GTHREADS + tid;
            const int tok = idx / NR, row = idx - tok * NR;
            const bool has = idx < G::TT * NR && row < NRL;
            s.o_ex[o] = tok * G::EXP + row;
            s.o_tok[o] = has ? tok : 0x7fffffff;
            s.o_row[o] = row;
            s.o_y[o] = ((uint32_t)tok * (uint32_t)Pm.rows + (uint32_t)row) * 4u;
        }
    }

    // Issue the loads of one round: rows n0.. (rows_left of them before the
    // end of W), tokens m0.. (toks_left), chunks c0 .. c0 + D - 1. The last
    // row a round may read ends at byte (rows_left - 1) row_bytes + 144 (c0 + D)
    // <= rows_left row_bytes - 144 c0 from the round's base, the next row
    // starts past that; likewise for the tokens' int8 (256 D of each
    // x_stride = K + K/8 bytes) and scales (32 D, after K).
    static __device__ __forceinline__ void load(const GemmParams &Pm, const Slots &s, int row_bytes, int n0, int m0,
                                                int c0, bool live, R &rg) {
        const uint32_t rows_left = (uint32_t)(Pm.rows - n0), toks_left = (uint32_t)(Pm.m - m0);
        const uint8_t *wbase = Pm.w + (size_t)n0 * row_bytes + (size_t)c0 * CHUNK_BYTES;
        const uint8_t *xrow = Pm.x + (size_t)m0 * Pm.x_stride;
        const __amdgpu_buffer_rsrc_t wb =
            buffer_of(wbase, live ? rows_left * (uint32_t)row_bytes - (uint32_t)c0 * CHUNK_BYTES : 0u);
        const __amdgpu_buffer_rsrc_t xb =
            buffer_of(xrow + (size_t)c0 * 256, live ? toks_left * (uint32_t)Pm.x_stride - (uint32_t)c0 * 256u : 0u);
        const __amdgpu_buffer_rsrc_t db =
            buffer_of(xrow + Pm.k + (size_t)c0 * 32,
                      live ? toks_left * (uint32_t)Pm.x_stride - (uint32_t)Pm.k - (uint32_t)c0 * 32u : 0u);
#pragma unroll
        for (int i = 0; i < G::SW; ++i) rg.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wb, (int)s.w_go[i], 0, CACHE_NT);
#pragma unroll
        for (int i = 0; i < G::SX; ++i) rg.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xb, (int)s.x_go[i], 0, 0);
#pragma unroll
        for (int i = 0; i < G::SD; ++i) rg.d[i] = __builtin_amdgcn_raw_buffer_load_b128(db, (int)s.d_go[i], 0, 0);
    }

    // Write one round from registers into an LDS round buffer.
    static __device__ __forceinline__ void stage(uint8_t *buf, const Slots &s, const R &rg) {
#pragma unroll
        for (int i = 0; i < G::SW; ++i)
            if ((i + 1) * GTHREADS <= G::W_PIECES || s.w_lo[i] >= 0)
                *reinterpret_cast<u32x4 *>(buf + s.w_lo[i]) = rg.w[i];
#pragma unroll
        for (int i = 0; i < G::SX; ++i)
            if ((i + 1) * GTHREADS <= G::X_PIECES || s.x_lo[i] >= 0)
                *reinterpret_cast<u32x4 *>(buf + s.x_lo[i]) = rg.x[i];
#pragma unroll
        for (int i = 0; i < G::SD; ++i)
            if ((i + 1) * GTHREADS <= G::XD_PIECES || s.d_lo[i] >= 0) {
                uint32_t *xd = reinterpret_cast<uint32_t *>(buf) + s.d_lo[i];
                const u32x4 v = rg.d[i];
                xd[0] = v.x;
                xd[G::XDP] = v.y;
                xd[2 * G::XDP] = v.z;
                xd[3 * G::XDP] = v.w;
            }
    }

    // The terms of blocks 8c + w (c = 0..D-1) of one round, added in order to
    // the wave's accumulators.
    static __device__ __forceinline__ void compute(const uint8_t *buf, float acc[MT][4]) {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        const int j = lane & 15, g = lane >> 4;
        const int h = g & 1;
        const int up = 4 - (g >> 1) * 4;         // 4: low nibbles, 0: high nibbles
        // Block 8c + w of row j starts at byte 18 w of its chunk: an even w at
        // a dword boundary (scale in the low half, the nibble run two bytes
        // in), an odd w two bytes into a dword (scale in the high half of the
        // dword before, the run dword-aligned). This lane's run is nibble
        // bytes 8h .. 8h + 7. Every address below is one dword-aligned base
        // plus constant offsets.
        const uint8_t *wrow = buf + G::W_OFF + j * G::WP + 18 * w;
        const uint32_t *run = reinterpret_cast<const uint32_t *>(wrow + (ODD ? 2 : 0) + 8 * h);
        const uint32_t *scl = reinterpret_cast<const uint32_t *>(wrow - (ODD ? 2 : 0));
        const uint8_t *xa = buf + G::X_OFF + j * G::AP + 32 * w + 8 * g;
        // The lane reads the scale of token 4g + (j & 3) of its tile; the
        // four lanes of a quad then hold the scales of the four tokens of the
        // lane's outputs, and a DPP quad broadcast hands scale r to output r.
        const float *xs = reinterpret_cast<const float *>(buf + G::XD_OFF) + w * G::XDP + 4 * g + (j & 3);
        // Phase 1: the integer block sums of the whole round (independent, so
        // the MFMAs issue back to back while the next operands are read).
        v4i v[D][MT];
        float dw[D], dx[D][MT];
#pragma unroll
        for (int c = 0; c < D; ++c) {
            uint32_t lo, hi, d_bits;
            if constexpr (!ODD) {
                const uint32_t v0 = run[36 * c], v1 = run[36 * c + 1], v2 = run[36 * c + 2];
                lo = __builtin_amdgcn_alignbyte(v1, v0, 2);
                hi = __builtin_amdgcn_alignbyte(v2, v1, 2);
                d_bits = scl[36 * c] & 0xFFFFu;
            } else {
                lo = run[36 * c];
                hi = run[36 * c + 1];
                d_bits = scl[36 * c] >> 16;
            }
            const long bw = as_long(((lo << up) & 0xF0F0F0F0u) ^ 0x80808080u, ((hi << up) & 0xF0F0F0F0u) ^ 0x80808080u);
            dw[c] = half_bits_to_float(d_bits) * 0.0625f;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const long ax = *reinterpret_cast<const long *>(xa + 16 * t * G::AP + 256 * c);
                dx[c][t] = xs[8 * c * G::XDP + 16 * t];
                v4i z = {0, 0, 0, 0};
                v[c][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
            }
        }
        // Phase 2: the fp32 terms, added to each accumulator in block order.
#pragma unroll
        for (int c = 0; c < D; ++c)
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float dxs[4] = {quad_bcast<0>(dx[c][t]), quad_bcast<1>(dx[c][t]), quad_bcast<2>(dx[c][t]),
                                      quad_bcast<3>(dx[c][t])};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = (float)v[c][t][r] * dw[c];
                    acc[t][r] = acc[t][r] + a * dxs[r];
                }
            }
    }

    // The workgroup's rounds form one stream over its items (row tiles
    // blockIdx.x, blockIdx.x + gridDim.x, ...; a launch covers one group of at
    // most TT tokens): round q is round q % RPI of item q / RPI. Two positions
    // walk the stream, the round being computed and the round being loaded
    // (P + 1 ahead), each advanced by one per round without a division.
    static __device__ __forceinline__ void run(const GemmParams &Pm, uint8_t *lds) {
        const int tid = threadIdx.x;
        const int lane = tid & 63, w = tid >> 6;
        const int j = lane & 15, g = lane >> 4;
        const int C = Pm.k >> 8;
        const int RPI = C / D;                                  // rounds per item (D divides C)
        const int row_bytes = C * CHUNK_BYTES;
        // Items are (row group, token group) pairs, row groups fastest.
        const int row_groups = (Pm.rows + NRL - 1) / NRL;
        const int items = row_groups * ((Pm.m + G::TT - 1) / G::TT);
        const int GD = gridDim.x;
        const int my_items = (int)blockIdx.x < items ? (items - 1 - (int)blockIdx.x) / GD + 1 : 0;
        const int QP = (my_items * RPI + P - 1) / P * P;        // rounds, padded to whole groups of P

        Slots s;
        slots(Pm, row_bytes, s);

        // A position in the workgroup's stream: round ss of its item kk, whose
        // row group and token group are rg_i and tg_i. Items kk and kk + 1
        // are GD apart, so moving to the next item adds GD to the row group
        // and carries into the token group (a few steps: GD <= items).
        struct Pos {
            int kk, ss, rg_i, tg_i;
        };
        auto advance = [&](Pos &p) {
            if (++p.ss == RPI) {
                p.ss = 0;
                ++p.kk;
                p.rg_i += GD;
                while (p.rg_i >= row_groups) {
                    p.rg_i -= row_groups;
                    ++p.tg_i;
                }
            }
        };
        auto load_at = [&](const Pos &p, R &rg) {
            load(Pm, s, row_bytes, p.rg_i * NRL, p.tg_i * G::TT, p.ss * D, p.kk < my_items, rg);
        };
        const Pos first{0, 0, (int)blockIdx.x % row_groups, (int)blockIdx.x / row_groups};
        const uint32_t y_total = (uint32_t)((size_t)Pm.m * Pm.rows * 4);

        R rg[P];
        Pos lp = first;                                         // the load position
#pragma unroll
        for (int d = 0; d < P; ++d) {
            load_at(lp, rg[d]);
            advance(lp);
        }
        stage(lds, s, rg[0]);
        load_at(lp, rg[0]);                                     // round P
        advance(lp);
        __syncthreads();

        float acc[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;

        Pos cp = first;                                         // the compute position: round q
        for (int q0 = 0; q0 < QP; q0 += P) {
#pragma unroll
            for (int d = 0; d < P; ++d) {
                const int q = q0 + d;
                const bool live = cp.kk < my_items;
                const bool item_end = live && cp.ss == RPI - 1;
                const int n0 = cp.rg_i * NRL, m0 = cp.tg_i * G::TT;
                float *ex = reinterpret_cast<float *>(lds + G::EX_OFF + (G::EXN == 2 ? (cp.kk & 1) * G::EX_BYTES : 0));
                if (live) compute(lds + (q & 1) * G::BUF, acc);
                if (item_end) {
#pragma unroll
                    for (int t = 0; t < MT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            ex[(w * G::TT + 16 * t + 4 * g + r) * G::EXP + j] = acc[t][r];
                            acc[t][r] = 0.0f;
                        }
                }
                // Round q + 1 into the other buffer (last read by round q - 1,
                // before the previous barrier), then its registers take round
                // q + 1 + P.
                stage(lds + ((q + 1) & 1) * G::BUF, s, rg[(d + 1) % P]);
                load_at(lp, rg[(d + 1) % P]);
                advance(lp);
                __syncthreads();
                // At an item's end: the eight accumulators of each output meet
                // in the adjacent-pair tree. Every thread issues its stores in
                // every round; the resource is empty when there is nothing to
                // store, and a lane past M or N stores out of range.
                const uint32_t y0 = ((uint32_t)m0 * (uint32_t)Pm.rows + (uint32_t)n0) * 4u;
                const __amdgpu_buffer_rsrc_t yb =
                    buffer_of(reinterpret_cast<uint8_t *>(Pm.y) + y0, item_end ? y_total - y0 : 0u);
#pragma unroll
                for (int o = 0; o < G::OUTS; ++o) {
                    float yv = 0.0f;
                    if (item_end && s.o_tok[o] < G::TT) {
                        float l[8];
#pragma unroll
                        for (int a = 0; a < 8; ++a) l[a] = ex[a * G::TT * G::EXP + s.o_ex[o]];
                        yv = ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
                    }
                    const bool ok = s.o_tok[o] < Pm.m - m0 && s.o_row[o] < Pm.rows - n0;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv), yb, ok ? (int)s.o_y[o] : OUT_OF_RANGE,
                                                          0, 0);
                }
                if (G::EXN == 1 && item_end) __syncthreads();   // the exchange is read before it is written again
                advance(cp);
            }
        }
    }
};

template <int MT, int D, int P, int OCC, int NRL>
__global__ __launch_bounds__(GTHREADS) __attribute__((amdgpu_waves_per_eu(2 * OCC, 2 * OCC)))
void gemm_mfma_kernel(GemmParams Pm) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if ((threadIdx.x >> 6) & 1)
        Kernel<MT, D, P, OCC, NRL, true>::run(Pm, lds);
    else
        Kernel<MT, D, P, OCC, NRL, false>::run(Pm, lds);
}

constexpr int DEPTH = 2;

template <int MT, int D, int OCC, int NRL = 16>
hipError_t launch_geo(const GemmParams &Pm, hipStream_t stream) {
    using G = Geo<MT, D, DEPTH, OCC, NRL>;
    const void *fn = reinterpret_cast<const void *>(&gemm_mfma_kernel<MT, D, DEPTH, OCC, NRL>);
    hipError_t e = allow_dynamic_lds(fn, LDS_MAX);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, GTHREADS, G::LDS);
    if (e != hipSuccess) return e;
    if (per_cu < 1) per_cu = 1;
    const long items = (long)((Pm.rows + NRL - 1) / NRL) * ((Pm.m + G::TT - 1) / G::TT);
    long grid = (long)device_cu_count() * per_cu;
    if (grid > items) grid = items;
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, D, DEPTH, OCC, NRL>), dim3((unsigned)grid), dim3(GTHREADS), G::LDS, stream,
                       Pm);
    return hipGetLastError();
}

// Chunks per round: the largest power of two up to DMAX that divides the
// K / 256 chunks of a row, so that every item is whole rounds.
template <int MT, int DMAX, int OCC, int NRL = 16>
hipError_t launch_mt(const GemmParams &Pm, hipStream_t stream) {
    const int C = Pm.k / 256;
    if constexpr (DMAX >= 8) {
        if (C % 8 == 0) return launch_geo<MT, 8, OCC, NRL>(Pm, stream);
    }
    if constexpr (DMAX >= 4) {
        if (C % 4 == 0) return launch_geo<MT, 4, OCC, NRL>(Pm, stream);
    }
    if constexpr (DMAX >= 2) {
        if (C % 2 == 0) return launch_geo<MT, 2, OCC, NRL>(Pm, stream);
    }
    return launch_geo<MT, 1, OCC, NRL>(Pm, stream);
}

// Workgroups per CU, and the item count under which wide token tiles split
// into 16-token items (below).
constexpr int GEMM_OCC = 2;
constexpr long GEMM_SPLIT_ITEMS = 160;

hipError_t launch_tokens(const GemmParams &Pm, hipStream_t stream) {
    // 16, 32 or 64 tokens per item. The widest tile that covers M streams the
    // weights once. With few row groups (2,048 rows: o, down) that leaves
    // most CUs idle, and 16-token items, one per (row group, token group),
    // are faster: down at M = 64 in 16.9 us against 28.3, at M = 24 in 11.4
    // against 16.2 (the weights are read once per token group, the later reads
    // mostly from the caches). At 3,072 rows (192 row groups) 16-token items
    // win at M > 32 only (8.8 against 9.5 us at M = 64; at M = 24 the 32-token
    // tile is faster). A round holds 128 (or, at two workgroups per CU, 64)
    // token-chunks of activations.
    constexpr int OCC = GEMM_OCC;
    const long row_groups = (Pm.rows + NR - 1) / NR;
    int mt = Pm.m <= 16 ? 1 : Pm.m <= 32 ? 2 : 4;
    const long wide_items = row_groups * ((Pm.m + 16 * mt - 1) / (16 * mt));
    if (mt > 1 && (wide_items < GEMM_SPLIT_ITEMS || (mt == 4 && wide_items < 2 * GEMM_SPLIT_ITEMS))) mt = 1;
    // One token group over long rows (K >= 8192: down) with fewer 16-row
    // groups than CUs: 8-row items, eight chunks per round, one workgroup per
    // CU. Down at M = 5..16 takes 9.2-10.1 us against 10.4-10.6 with 16-row
    // items (MI355X, rotated weights). With several token groups (M > 16) a
    // workgroup then runs its items one after another, 1.5-1.8x slower, and at
    // K = 2048 (o, q|k|v) 8-row items were slower too.
    if (mt == 1 && Pm.m <= 16 && Pm.k >= 8192 && row_groups < device_cu_count())
        return launch_mt<1, 8, 1, 8>(Pm, stream);
    if (mt == 1) return launch_mt<1, 8 / OCC, OCC>(Pm, stream);
    if (mt == 2) return launch_mt<2, 4 / OCC, OCC>(Pm, stream);
    return launch_mt<4, 2 / OCC, OCC>(Pm, stream);
}

}  // namespace

// From this many rows on, the row-split kernel: at gate|up (16,384 rows) it is
// 8-26% faster; at 3,072 rows it was twice as slow (48 workgroups).
constexpr int ROWS_MIN = 8192;

hipError_t launch_gemm(const MatrixRef &w, const uint8_t *x, int m, float *y, hipStream_t stream) {
    // One token is the M = 1 GEMV, byte for byte by the contract, and faster.
    // A few tokens are its weight stream with the arithmetic per token
    // (gemv_mt.hip), up to the m where that is the faster (gemv_mt_max_m:
    // 2 to 6 by shape), where the MFMA kernels' rounds cost more than the
    // per-token arithmetic; past that the arithmetic (0.8 us per token on
    // gate|up) loses to the MFMA kernels.
    if (m == 1) return launch_gemv_m1(w, x, X_ENGINE, y, stream);
    if (w.nseg == 1 && !w.paired && m <= gemv_mt_max_m(w.rows, w.k) && gemv_mt_fits(m, w.rows, w.k))
        return launch_gemv_mt(w.seg[0], x, m, y, w.rows, w.k, stream);
    GemmParams P{};
    P.w = w.seg[0];
    P.rows = w.rows;
    P.k = w.k;
    P.x_stride = w.k + w.k / 8;
    // Buffer ranges are 32-bit byte counts: the weights must fit one. Tokens
    // go in launches of at most 64 (one item's tokens, so the weights stream
    // once per launch), whose activations and outputs then fit one too.
    if ((size_t)P.rows * (size_t)(P.k / QK * Q4_0_BYTES) >= 0x7fff0000u ||
        (size_t)64 * P.rows * 4 >= 0x7fff0000u)
        return hipErrorInvalidValue;
    const bool by_rows = P.rows >= ROWS_MIN && gemm_rows_fits(P.rows, P.k);
    for (int m0 = 0; m0 < m; m0 += 64) {
        P.x = x + (size_t)m0 * P.x_stride;
        P.y = y + (size_t)m0 * P.rows;
        P.m = m - m0 < 64 ? m - m0 : 64;
        const hipError_t e = by_rows ? launch_gemm_rows(P.w, P.x, P.m, P.y, P.rows, P.k, stream) : launch_tokens(P, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace w4a8
