// Batched W4A8 (M > 1) for matrices with many rows: the same results as
// gemm_mfma.hip (the contract's order, src/llm_kv260/q4_0.py:170-182, applied
// row by row), with the work cut along rows instead of along the blocks of K.
//
// A 16-row group belongs to a pair of waves for the whole of K. Wave h of the
// pair owns the contract's accumulators 4h .. 4h + 3: it takes the blocks b
// with b % 8 in that range, in increasing b, and adds each term to accumulator
// b % 8 from +0.0f. At the end the pair meets once: wave 0's
// (a0 + a1) + (a2 + a3) plus wave 1's (a4 + a5) + (a6 + a7) is the
// adjacent-pair tree's last add. A workgroup holds two or four pairs (32 or
// 64 rows, pairs_of), so every wave has the same work. From 5 tokens the
// group has four waves instead (QuadKernel), each owning two accumulators.
//
// K goes by segments of 512 values (16 blocks). Per segment a pair stages its
// 16 rows' 288-byte runs in a slab of its own, and the workgroup stages the
// tokens' 512 activation bytes and 16 scales once for all four pairs: one
// barrier per segment, with the loads of the next two segments in flight.
//
// The integer part is v_mfma_i32_16x16x32_i8 as in gemm_mfma.hip (K = 32 is
// one block; unsigned nibbles, then a second MFMA against a constant -8
// operand; at four token tiles the weights made signed once instead,
// signed_nibbles). Operand layout of the 16x16x32 i8 MFMA (64 lanes):
//   A: lane l holds A[i = l % 16][k = 8 (l / 16) .. + 7]      (token i)
//   B: lane l holds B[k = 8 (l / 16) .. + 7][j = l % 16]      (row j)
//   D: lane l holds D[i = 4 (l / 16) + r][j = l % 16], r = 0..3
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-row groups (pairs of waves) per workgroup: two at one token tile (two
// workgroups then share a CU, each running while the other waits at its
// segment barrier: the LM head at M = 9..16 in 51-53 us against 67-70 with
// four), four at two or four token tiles (whose workgroups fill the CU's
// registers alone; two pairs were 1.1-1.6x slower there).
template <int MT>
constexpr int pairs_of() { return MT == 1 ? 2 : 4; }
constexpr int SEG = 512;                          // activation values per segment
constexpr int SEG_BLOCKS = SEG / QK;              // 16
constexpr int SEG_ROW_BYTES = SEG_BLOCKS * Q4_0_BYTES;   // 288
constexpr int W_PIECES = 16 * SEG_ROW_BYTES / 16;        // 288 pieces of 16 B per pair and segment
constexpr int SW = (W_PIECES + 127) / 128;                // 3 load slots per thread of a pair
constexpr int WPITCH = SEG_ROW_BYTES + 16;                // slab row pitch (16-byte aligned)
constexpr int SLAB = 16 * WPITCH;                         // 4,864 B
constexpr int OUT_OF_RANGE = 0x7ffffff0;
constexpr uint32_t BUFFER_DWORD3 = 0x00020000;
constexpr int CACHE_NT = 2;
constexpr int LDS_MAX = 160 * 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, BUFFER_DWORD3);
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// DPP quad broadcast of lane R of each quad; folds into the consuming multiply.
template <int R>
__device__ __forceinline__ float bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), R * 0x55, 0xF, 0xF, true));
}

// Four nibble values n (one a byte, 0..15) as the signed bytes n - 8: n ^ 8
// is n - 8 as a 4-bit two's-complement number, and its sign (bit 3) spread
// over the byte's high nibble makes it the 8-bit one. The spread is a
// multiply by 30 (8 * 30 = 240 = 0xF0) in two 16-bit halves, whose high
// bytes never carry into each other.
__device__ __forceinline__ uint32_t signed_nibbles(uint32_t n) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const uint32_t x = n ^ 0x08080808u;
    const uint32_t s = x & 0x08080808u;
    const u16x2 r = __builtin_bit_cast(u16x2, s) * (u16x2){30, 30} + __builtin_bit_cast(u16x2, x);
    return __builtin_bit_cast(uint32_t, r);
}

struct RowsParams {
    const uint8_t *w;
    const uint8_t *x;      // m rows, engine layout
    float *y;              // [m][rows]
    int rows;
    int k;
    int m;
    int x_stride;          // k + k / 8
};

template <int MT>
struct RGeo {
    static constexpr int TT = 16 * MT;                       // tokens
    static constexpr int APITCH = SEG + 16;                  // int8 bytes per token and segment, padded
    static constexpr int XDP = TT + 4;                       // scale rows: [16 blocks][XDP]
    static constexpr int XD_OFF = TT * APITCH;
    static constexpr int XBUF = XD_OFF + SEG_BLOCKS * XDP * 4;
    static constexpr int PAIRS = pairs_of<MT>();
    static constexpr int THREADS = 64 * 2 * PAIRS;
    static constexpr int SLAB_OFF = 2 * XBUF;                // [2][PAIRS] slabs
    static constexpr int EX_OFF = SLAB_OFF + 2 * PAIRS * SLAB;   // pair exchange [PAIRS][TT][16] floats
    static constexpr int LDS = EX_OFF + PAIRS * TT * 16 * 4;
    static_assert(LDS <= LDS_MAX, "LDS budget");
    static constexpr int X_PIECES = TT * (SEG / 16);         // int8 pieces per segment
    static constexpr int D_PIECES = TT * (SEG_BLOCKS / 4);   // scale pieces (4 scales each)
    static constexpr int SX = (X_PIECES + THREADS - 1) / THREADS;
    static constexpr int SD = (D_PIECES + THREADS - 1) / THREADS;
};

// PK > 1 (one token tile, M <= 16 / PK): PK blocks share one MFMA result
// tile (packed_group), so that the fp32 epilogue touches only live outputs.
template <int MT, int PK = 1>
struct RowsKernel {
    using G = RGeo<MT>;
    static_assert(PK == 1 || (MT == 1 && (PK == 2 || PK == 4)), "blocks per tile: 2 or 4, one token tile");

    struct Regs {
        u32x4 w[SW];
        u32x4 x[G::SX];
        u32x4 d[G::SD];
    };

    // Fixed per-thread offsets: weight pieces of the pair's rows, activation
    // and scale pieces of the workgroup's tokens.
    struct Slots {
        uint32_t w_go[SW];
        int w_lo[SW];          // slab byte offset, -1 for no piece
        uint32_t x_go[G::SX];
        int x_lo[G::SX];
        uint32_t d_go[G::SD];
        int d_lo[G::SD];       // float index of the piece's first scale in a buffer
    };

    static __device__ __forceinline__ void slots(const RowsParams &P, int row_bytes, Slots &s) {
        const int tid = threadIdx.x;
        const int tp = tid & 127;                // thread within the pair
#pragma unroll
        for (int i = 0; i < SW; ++i) {
            const int n = tp + 128 * i;
            const int r = n / 18, q = n - 18 * (n / 18);
            const bool has = n < W_PIECES;
            s.w_go[i] = has ? (uint32_t)r * (uint32_t)row_bytes + 16u * (uint32_t)q : (uint32_t)OUT_OF_RANGE;
            s.w_lo[i] = has ? r * WPITCH + 16 * q : -1;
        }
#pragma unroll
        for (int i = 0; i < G::SX; ++i) {
            const int n = tid + G::THREADS * i;
            const int t = n / 32, p = n - 32 * t;
            const bool has = n < G::X_PIECES;
            s.x_go[i] = has ? (uint32_t)t * (uint32_t)P.x_stride + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.x_lo[i] = has ? t * G::APITCH + 16 * p : -1;
        }
#pragma unroll
        for (int i = 0; i < G::SD; ++i) {
            const int n = tid + G::THREADS * i;
            const int p = n / G::TT, t = n - G::TT * p;   // tokens fastest: the transposing writes spread over banks
            const bool has = n < G::D_PIECES;
            s.d_go[i] = has ? (uint32_t)t * (uint32_t)P.x_stride + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.d_lo[i] = has ? G::XD_OFF / 4 + 4 * p * G::XDP + t : -1;
        }
    }

    // Loads of segment sg (sg >= nseg: nothing; the resources are then empty).
    static __device__ __forceinline__ void load(const RowsParams &P, const Slots &s, int row_bytes, int n0, int sg,
                                                int nseg, Regs &rg) {
        const bool live = sg < nseg;
        const uint32_t rows_left = n0 < P.rows ? (uint32_t)(P.rows - n0) : 0u;
        const uint32_t w_skip = (uint32_t)sg * SEG_ROW_BYTES;
        const __amdgpu_buffer_rsrc_t wb =
            rsrc(P.w + (size_t)n0 * row_bytes + (live ? w_skip : 0u),
                 live && rows_left ? rows_left * (uint32_t)row_bytes - w_skip : 0u);
        const uint32_t xs = (uint32_t)P.m * (uint32_t)P.x_stride;
        const __amdgpu_buffer_rsrc_t xb = rsrc(P.x + (live ? sg * SEG : 0), live ? xs - (uint32_t)(sg * SEG) : 0u);
        const uint32_t d0 = (uint32_t)P.k + (uint32_t)sg * SEG_BLOCKS * 4u;
        const __amdgpu_buffer_rsrc_t db = rsrc(P.x + (live ? d0 : 0u), live ? xs - d0 : 0u);
#pragma unroll
        for (int i = 0; i < SW; ++i) rg.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wb, (int)s.w_go[i], 0, CACHE_NT);
#pragma unroll
        for (int i = 0; i < G::SX; ++i) rg.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xb, (int)s.x_go[i], 0, 0);
#pragma unroll
        for (int i = 0; i < G::SD; ++i) rg.d[i] = __builtin_amdgcn_raw_buffer_load_b128(db, (int)s.d_go[i], 0, 0);
    }

    static __device__ __forceinline__ void stage(uint8_t *xbuf, uint8_t *slab, const Slots &s, const Regs &rg) {
#pragma unroll
        for (int i = 0; i < SW; ++i)
            if (s.w_lo[i] >= 0) *reinterpret_cast<u32x4 *>(slab + s.w_lo[i]) = rg.w[i];
#pragma unroll
        for (int i = 0; i < G::SX; ++i)
            if ((i + 1) * G::THREADS <= G::X_PIECES || s.x_lo[i] >= 0)
                *reinterpret_cast<u32x4 *>(xbuf + s.x_lo[i]) = rg.x[i];
#pragma unroll
        for (int i = 0; i < G::SD; ++i)
            if ((i + 1) * G::THREADS <= G::D_PIECES || s.d_lo[i] >= 0) {
                uint32_t *xd = reinterpret_cast<uint32_t *>(xbuf) + s.d_lo[i];
                const u32x4 v = rg.d[i];
                xd[0] = v.x;
                xd[G::XDP] = v.y;
                xd[2 * G::XDP] = v.z;
                xd[3 * G::XDP] = v.w;
            }
    }

    // Block B (0..15) of the segment, row j of the pair's group: the MFMA
    // weight operand of lane group g (the nibbles of weights 8g .. 8g + 7:
    // the low nibbles of bytes 0..7, g = 0, and 8..15, g = 1, then the high
    // nibbles, g = 2, 3) and the block's scale.
    template <int B>
    static __device__ __forceinline__ void weights_of(const uint8_t *slab, int j, int g, long &bw, float &dw) {
        const int h = g & 1;
        const int shift = (g >> 1) * 4;
        const uint8_t *wrow = slab + j * WPITCH + 18 * B;
        uint32_t lo, hi, d_bits;
        if constexpr ((B & 1) == 0) {
            // Dword-aligned block: scale in the low half, the nibble run two bytes in.
            const uint32_t *run = reinterpret_cast<const uint32_t *>(wrow + 8 * h);
            const uint32_t v0 = run[0], v1 = run[1], v2 = run[2];
            lo = __builtin_amdgcn_alignbyte(v1, v0, 2);
            hi = __builtin_amdgcn_alignbyte(v2, v1, 2);
            d_bits = *reinterpret_cast<const uint32_t *>(wrow) & 0xFFFFu;
        } else {
            // Two bytes into a dword: scale in the high half of the dword before, the run aligned.
            const uint32_t *run = reinterpret_cast<const uint32_t *>(wrow + 2 + 8 * h);
            lo = run[0];
            hi = run[1];
            d_bits = *reinterpret_cast<const uint32_t *>(wrow - 2) >> 16;
        }
        bw = as_long((lo >> shift) & 0x0F0F0F0Fu, (hi >> shift) & 0x0F0F0F0Fu);
        dw = half_bits_to_float(d_bits);
    }

    // Block B (0..15) of the segment: its MFMA sums for every token tile.
    template <int B>
    static __device__ __forceinline__ void block_sums(const uint8_t *slab, const uint8_t *xbuf, int j, int g, v4i v[MT],
                                                      float &dw, float dx[MT]) {
        long bw;
        weights_of<B>(slab, j, g, bw, dw);
        const long minus8 = as_long(0xF8F8F8F8u, 0xF8F8F8F8u);
        const uint8_t *xa = xbuf + j * G::APITCH + 32 * B + 8 * g;
        const float *xs = reinterpret_cast<const float *>(xbuf + G::XD_OFF) + B * G::XDP + 4 * g + (j & 3);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const long ax = *reinterpret_cast<const long *>(xa + 16 * t * G::APITCH);
            dx[t] = xs[16 * t];
            v4i z = {0, 0, 0, 0};
            z = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
            v[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, minus8, z, 0, 0, 0);
        }
    }

    // The terms of NB consecutive blocks B0 .. B0 + NB - 1 (accumulators
    // B0 % 4 ..), in block order: their MFMAs first, then the fp32 terms.
    template <int B0, int NB>
    static __device__ __forceinline__ void blocks(const uint8_t *slab, const uint8_t *xbuf, int j, int g,
                                                  float acc[4][MT][4]) {
        v4i v[NB][MT];
        float dw[NB], dx[NB][MT];
        block_sums<B0>(slab, xbuf, j, g, v[0], dw[0], dx[0]);
        block_sums<B0 + 1>(slab, xbuf, j, g, v[1], dw[1], dx[1]);
        if constexpr (NB == 4) {
            block_sums<B0 + 2>(slab, xbuf, j, g, v[2], dw[2], dx[2]);
            block_sums<B0 + 3>(slab, xbuf, j, g, v[3], dw[3], dx[3]);
        }
#pragma unroll
        for (int c = 0; c < NB; ++c)
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float dxs[4] = {bcast<0>(dx[c][t]), bcast<1>(dx[c][t]), bcast<2>(dx[c][t]), bcast<3>(dx[c][t])};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = (float)v[c][t][r] * dw[c];
                    acc[(B0 + c) & 3][t][r] = acc[(B0 + c) & 3][t][r] + a * dxs[r];
                }
            }
    }

    // Packed tiles (PK blocks of at most TPB = 16 / PK tokens each): the A
    // operand's 16 rows are (block c, token t) = (i / TPB, i % TPB). Block c's
    // MFMA sees zeros in every other block's rows, so the PK MFMAs put each
    // block's exact int32 sums in its own rows of one tile; one more MFMA
    // against -8 adds -8 sum(x) to every row. The result's lane l then holds
    // block c = 4 (l / 16) / TPB of the group, tokens 4 (l / 16) % TPB + r
    // (r = 0..3), row l % 16: every lane live, one fp32 term per value.
    template <int B0, int C>
    static __device__ __forceinline__ void packed_mfma(const uint8_t *slab, int j, int g, int ablk, int dblk, long ax,
                                                       v4i &d, float &dw) {
        long bw;
        float dwc;
        weights_of<B0 + C>(slab, j, g, bw, dwc);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ablk == C ? ax : 0L, bw, d, 0, 0, 0);
        dw = dblk == C ? dwc : dw;
        if constexpr (C + 1 < PK) packed_mfma<B0, C + 1>(slab, j, g, ablk, dblk, ax, d, dw);
    }

    // Blocks B0 .. B0 + PK - 1: their terms, added to the lane's accumulator
    // (that of its block, B0 % 8 + c) in block order.
    template <int B0>
    static __device__ __forceinline__ void packed_group(const uint8_t *slab, const uint8_t *xbuf, int j, int g,
                                                        float acc[4]) {
        constexpr int TPB = 16 / PK;
        const int ablk = j / TPB, atok = j - ablk * TPB;          // this lane's A row (block, token)
        const int dblk = 4 * g / TPB, dtok = 4 * g - dblk * TPB;  // its result rows
        const long ax = *reinterpret_cast<const long *>(xbuf + atok * G::APITCH + 32 * (B0 + ablk) + 8 * g);
        v4i d = {0, 0, 0, 0};
        float dw = 0.0f;
        packed_mfma<B0, 0>(slab, j, g, ablk, dblk, ax, d, dw);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, as_long(0xF8F8F8F8u, 0xF8F8F8F8u), d, 0, 0, 0);
        // The four tokens' scales of the lane's block: one 16-byte read (a
        // block's scales are a row of XDP floats, tokens along it).
        const float *xs = reinterpret_cast<const float *>(xbuf + G::XD_OFF) + (B0 + dblk) * G::XDP + dtok;
        const float4 dx = *reinterpret_cast<const float4 *>(xs);
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float a = (float)d[r] * dw;
            acc[r] = acc[r] + a * dxs[r];
        }
    }

    // The wave's eight blocks of a segment: its four accumulators' blocks
    // 4 half + c, then 8 + 4 half + c, in order. Two blocks per phase at four
    // token tiles keeps the MFMA results within the register budget.
    template <int H>
    static __device__ __forceinline__ void segment(const uint8_t *slab, const uint8_t *xbuf, int j, int g,
                                                   float acc[4][MT][4]) {
        if constexpr (PK == 4) {
            packed_group<4 * H>(slab, xbuf, j, g, acc[0][0]);
            packed_group<8 + 4 * H>(slab, xbuf, j, g, acc[0][0]);
        } else if constexpr (PK == 2) {
            packed_group<4 * H>(slab, xbuf, j, g, acc[0][0]);
            packed_group<4 * H + 2>(slab, xbuf, j, g, acc[1][0]);
            packed_group<8 + 4 * H>(slab, xbuf, j, g, acc[0][0]);
            packed_group<8 + 4 * H + 2>(slab, xbuf, j, g, acc[1][0]);
        } else if constexpr (MT <= 2) {
            blocks<4 * H, 4>(slab, xbuf, j, g, acc);
            blocks<8 + 4 * H, 4>(slab, xbuf, j, g, acc);
        } else {
            blocks<4 * H, 2>(slab, xbuf, j, g, acc);
            blocks<4 * H + 2, 2>(slab, xbuf, j, g, acc);
            blocks<8 + 4 * H, 2>(slab, xbuf, j, g, acc);
            blocks<8 + 4 * H + 2, 2>(slab, xbuf, j, g, acc);
        }
    }

    static __device__ __forceinline__ void run(const RowsParams &P, uint8_t *lds) {
        const int tid = threadIdx.x;
        // The wave index is uniform: as a scalar, the pair's resources and the
        // choice of accumulators are scalar too (no per-lane resource loop).
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int pair = wave >> 1, half = wave & 1;
        const int j = lane & 15, g = lane >> 4;
        const int row_bytes = P.k / QK * Q4_0_BYTES;
        const int nseg = P.k / SEG;
        const int n0 = ((int)blockIdx.x * G::PAIRS + pair) * 16;   // the pair's first row

        Slots s;
        slots(P, row_bytes, s);
        // Segments in flight: two; one at four token tiles, whose segment
        // takes long enough to cover the loads of the next and whose
        // registers are needed for the MFMA results.
        constexpr int DEPTH = MT >= 4 ? 1 : 2;
        Regs rg[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(P, s, row_bytes, n0, d, nseg, rg[d]);
        stage(lds, lds + G::SLAB_OFF + pair * SLAB, s, rg[0]);
        load(P, s, row_bytes, n0, DEPTH, nseg, rg[0]);
        __syncthreads();

        float acc[4][MT][4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[c][t][r] = 0.0f;

        for (int sg0 = 0; sg0 < nseg; sg0 += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                const int sg = sg0 + d;
                if (sg < nseg) {
                    const uint8_t *xbuf = lds + (sg & 1) * G::XBUF;
                    const uint8_t *slab = lds + G::SLAB_OFF + ((sg & 1) * G::PAIRS + pair) * SLAB;
                    if (half == 0)
                        segment<0>(slab, xbuf, j, g, acc);
                    else
                        segment<1>(slab, xbuf, j, g, acc);
                }
                // Segment sg + 1 into the other buffers (last read for
                // segment sg - 1, before the previous barrier); its registers
                // then take segment sg + 1 + DEPTH.
                const int nx = sg + 1;
                stage(lds + (nx & 1) * G::XBUF, lds + G::SLAB_OFF + ((nx & 1) * G::PAIRS + pair) * SLAB, s,
                      rg[(d + 1) % DEPTH]);
                load(P, s, row_bytes, n0, nx + DEPTH, nseg, rg[(d + 1) % DEPTH]);
                __syncthreads();
            }
        }

        float *ex = reinterpret_cast<float *>(lds + G::EX_OFF) + pair * G::TT * 16;
        if constexpr (PK > 1) {
            // The wave's four accumulators of an output sit in lanes 16 apart
            // (PK = 4: acc[0] of lane groups 0..3 hold a0..a3) or 32 apart in
            // two arrays (PK = 2: acc[0] holds a0 / a1, acc[1] a2 / a3): the
            // tree's (a0 + a1) + (a2 + a3), then the pair's last add through
            // LDS as below. Lanes of result block 0 hold the sums.
            constexpr int TPB = 16 / PK;
            const int dblk = 4 * g / TPB, dtok = 4 * g - dblk * TPB;
            float part[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (PK == 4) {
                    const float s = acc[0][0][r] + __shfl_xor(acc[0][0][r], 16);
                    part[r] = s + __shfl_xor(s, 32);
                } else {
                    const float s01 = acc[0][0][r] + __shfl_xor(acc[0][0][r], 32);
                    const float s23 = acc[1][0][r] + __shfl_xor(acc[1][0][r], 32);
                    part[r] = s01 + s23;
                }
            }
            if (half == 1 && dblk == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) ex[(dtok + r) * 16 + j] = part[r];
            }
            __syncthreads();
            if (half == 0) {
                const uint32_t y_bytes = (uint32_t)P.m * (uint32_t)P.rows * 4u;
                const __amdgpu_buffer_rsrc_t yb = rsrc(P.y, y_bytes);
                const bool row_ok = n0 + j < P.rows && dblk == 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = dtok + r;
                    const float yv = part[r] + ex[tok * 16 + j];
                    const bool ok = row_ok && tok < P.m;
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __float_as_uint(yv), yb, ok ? (int)(((uint32_t)tok * (uint32_t)P.rows + (uint32_t)(n0 + j)) * 4u) : OUT_OF_RANGE,
                        0, 0);
                }
            }
            return;
        }
        // The pair meets: wave 1 hands (a4 + a5) + (a6 + a7) to wave 0.
        float part[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[t][r] = (acc[0][t][r] + acc[1][t][r]) + (acc[2][t][r] + acc[3][t][r]);
        if (half == 1) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) ex[(16 * t + 4 * g + r) * 16 + j] = part[t][r];
        }
        __syncthreads();
        if (half == 0) {
            const uint32_t y_bytes = (uint32_t)P.m * (uint32_t)P.rows * 4u;
            const __amdgpu_buffer_rsrc_t yb = rsrc(P.y, y_bytes);
            const bool row_ok = n0 + j < P.rows;
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = 16 * t + 4 * g + r;
                    const float yv = part[t][r] + ex[tok * 16 + j];
                    const bool ok = row_ok && tok < P.m;
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __float_as_uint(yv), yb, ok ? (int)(((uint32_t)tok * (uint32_t)P.rows + (uint32_t)(n0 + j)) * 4u) : OUT_OF_RANGE,
                        0, 0);
                }
        }
    }
};

// Four waves per 16-row group (a quad): wave q owns the contract's
// accumulators 2q and 2q + 1, so it takes the blocks b with b % 8 in
// {2q, 2q + 1}, in increasing b. A workgroup holds GROUPS groups (64 rows
// at four: 16 waves), sharing the staged activation as the pairs do, and a
// SIMD then runs four waves instead of two: one wave's LDS reads, MFMA
// latency and waits are covered by the others' fp32 terms. At the end wave
// 0 of the group adds the tree: (p0 + p1) + (p2 + p3), p_q = a_2q + a_2q+1,
// the other waves' parts through LDS (over the activation buffers, which
// every wave has finished reading by then).
template <int MT, int GROUPS>
struct QuadGeo {
    static constexpr int TT = 16 * MT;
    static constexpr int APITCH = SEG + 16;
    static constexpr int XDP = TT + 4;
    static constexpr int XD_OFF = TT * APITCH;
    static constexpr int XBUF = XD_OFF + SEG_BLOCKS * XDP * 4;
    static constexpr int THREADS = 64 * 4 * GROUPS;
    static constexpr int SLAB_OFF = 2 * XBUF;                       // [2][GROUPS] slabs
    static constexpr int LDS = SLAB_OFF + 2 * GROUPS * SLAB;
    static constexpr int EX_FLOATS = GROUPS * 3 * TT * 16;         // the parts of waves 1..3
    static_assert(EX_FLOATS * 4 <= LDS, "exchange within the buffers");
    static_assert(LDS <= LDS_MAX, "LDS budget");
    static constexpr int X_PIECES = TT * (SEG / 16);
    static constexpr int D_PIECES = TT * (SEG_BLOCKS / 4);
    static constexpr int SX = (X_PIECES + THREADS - 1) / THREADS;
    static constexpr int SD = (D_PIECES + THREADS - 1) / THREADS;
    static constexpr int SWQ = (W_PIECES + 255) / 256;               // weight pieces per thread of a group
};

template <int MT, int GROUPS, int PK = 1>
struct QuadKernel {
    using G = QuadGeo<MT, GROUPS>;
    static_assert(PK == 1 || (PK == 2 && MT == 1), "packed quads: two blocks of at most 8 tokens a tile");

    struct Regs {
        u32x4 w[G::SWQ];
        u32x4 x[G::SX];
        u32x4 d[G::SD];
    };
    struct Slots {
        uint32_t w_go[G::SWQ];
        int w_lo[G::SWQ];
        uint32_t x_go[G::SX];
        int x_lo[G::SX];
        uint32_t d_go[G::SD];
        int d_lo[G::SD];
    };

    static __device__ __forceinline__ void slots(const RowsParams &P, int row_bytes, Slots &s) {
        const int tid = threadIdx.x;
        const int tp = tid & 255;                // thread within the group
#pragma unroll
        for (int i = 0; i < G::SWQ; ++i) {
            const int n = tp + 256 * i;
            const int r = n / 18, q = n - 18 * (n / 18);
            const bool has = n < W_PIECES;
            s.w_go[i] = has ? (uint32_t)r * (uint32_t)row_bytes + 16u * (uint32_t)q : (uint32_t)OUT_OF_RANGE;
            s.w_lo[i] = has ? r * WPITCH + 16 * q : -1;
        }
#pragma unroll
        for (int i = 0; i < G::SX; ++i) {
            const int n = tid + G::THREADS * i;
            const int t = n / 32, p = n - 32 * t;
            const bool has = n < G::X_PIECES;
            s.x_go[i] = has ? (uint32_t)t * (uint32_t)P.x_stride + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.x_lo[i] = has ? t * G::APITCH + 16 * p : -1;
        }
#pragma unroll
        for (int i = 0; i < G::SD; ++i) {
            const int n = tid + G::THREADS * i;
            const int p = n / G::TT, t = n - G::TT * p;
            const bool has = n < G::D_PIECES;
            s.d_go[i] = has ? (uint32_t)t * (uint32_t)P.x_stride + 16u * (uint32_t)p : (uint32_t)OUT_OF_RANGE;
            s.d_lo[i] = has ? G::XD_OFF / 4 + 4 * p * G::XDP + t : -1;
        }
    }

    static __device__ __forceinline__ void load(const RowsParams &P, const Slots &s, int row_bytes, int n0, int sg,
                                                int nseg, Regs &rg) {
        const bool live = sg < nseg;
        const uint32_t rows_left = n0 < P.rows ? (uint32_t)(P.rows - n0) : 0u;
        const uint32_t w_skip = (uint32_t)sg * SEG_ROW_BYTES;
        const __amdgpu_buffer_rsrc_t wb =
            rsrc(P.w + (size_t)n0 * row_bytes + (live ? w_skip : 0u),
                 live && rows_left ? rows_left * (uint32_t)row_bytes - w_skip : 0u);
        const uint32_t xs = (uint32_t)P.m * (uint32_t)P.x_stride;
        const __amdgpu_buffer_rsrc_t xb = rsrc(P.x + (live ? sg * SEG : 0), live ? xs - (uint32_t)(sg * SEG) : 0u);
        const uint32_t d0 = (uint32_t)P.k + (uint32_t)sg * SEG_BLOCKS * 4u;
        const __amdgpu_buffer_rsrc_t db = rsrc(P.x + (live ? d0 : 0u), live ? xs - d0 : 0u);
#pragma unroll
        for (int i = 0; i < G::SWQ; ++i) rg.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wb, (int)s.w_go[i], 0, CACHE_NT);
#pragma unroll
        for (int i = 0; i < G::SX; ++i) rg.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xb, (int)s.x_go[i], 0, 0);
#pragma unroll
        for (int i = 0; i < G::SD; ++i) rg.d[i] = __builtin_amdgcn_raw_buffer_load_b128(db, (int)s.d_go[i], 0, 0);
    }

    static __device__ __forceinline__ void stage(uint8_t *xbuf, uint8_t *slab, const Slots &s, const Regs &rg) {
#pragma unroll
        for (int i = 0; i < G::SWQ; ++i)
            if (s.w_lo[i] >= 0) *reinterpret_cast<u32x4 *>(slab + s.w_lo[i]) = rg.w[i];
#pragma unroll
        for (int i = 0; i < G::SX; ++i)
            if ((i + 1) * G::THREADS <= G::X_PIECES || s.x_lo[i] >= 0)
                *reinterpret_cast<u32x4 *>(xbuf + s.x_lo[i]) = rg.x[i];
#pragma unroll
        for (int i = 0; i < G::SD; ++i)
            if ((i + 1) * G::THREADS <= G::D_PIECES || s.d_lo[i] >= 0) {
                uint32_t *xd = reinterpret_cast<uint32_t *>(xbuf) + s.d_lo[i];
                const u32x4 v = rg.d[i];
                xd[0] = v.x;
                xd[G::XDP] = v.y;
                xd[2 * G::XDP] = v.z;
                xd[3 * G::XDP] = v.w;
            }
    }

    // Block B of the wave's view of the segment (the wave's blocks start at
    // 2q, folded into the pointers; B keeps the parity, which fixes where the
    // block's scale and nibbles sit in its dwords): its MFMA sums for every
    // token tile, the weight scale and the tokens' scales.
    template <int B>
    static __device__ __forceinline__ void block_sums(const uint8_t *slab, const uint8_t *xq, const float *xd, int j,
                                                      int g, v4i v[MT], float &dw, float dx[MT]) {
        long bw;
        RowsKernel<MT>::template weights_of<B>(slab, j, g, bw, dw);
        const uint8_t *xa = xq + j * G::APITCH + 32 * B + 8 * g;
        const float *xs = xd + B * G::XDP + 4 * g + (j & 3);
        if constexpr (MT >= 4) {
            // Four token tiles share the weight operand: make it the signed
            // weights n - 8 once (three integer ops a dword) instead of a
            // second MFMA per tile against -8.
            const long sw = as_long(signed_nibbles((uint32_t)bw), signed_nibbles((uint32_t)((unsigned long)bw >> 32)));
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const long ax = *reinterpret_cast<const long *>(xa + 16 * t * G::APITCH);
                dx[t] = xs[16 * t];
                v4i z = {0, 0, 0, 0};
                v[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, sw, z, 0, 0, 0);
            }
        } else {
            const long minus8 = as_long(0xF8F8F8F8u, 0xF8F8F8F8u);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const long ax = *reinterpret_cast<const long *>(xa + 16 * t * G::APITCH);
                dx[t] = xs[16 * t];
                v4i z = {0, 0, 0, 0};
                z = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
                v[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, minus8, z, 0, 0, 0);
            }
        }
    }

    // Block B (accumulator c of the wave's two): MFMAs first, then the fp32
    // terms.
    template <int B, int C>
    static __device__ __forceinline__ void one_block(const uint8_t *slab, const uint8_t *xq, const float *xd, int j,
                                                     int g, float acc[2][MT][4]) {
        v4i v[MT];
        float dw, dx[MT];
        block_sums<B>(slab, xq, xd, j, g, v, dw, dx);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float dxs[4] = {bcast<0>(dx[t]), bcast<1>(dx[t]), bcast<2>(dx[t]), bcast<3>(dx[t])};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a = (float)v[t][r] * dw;
                acc[C][t][r] = acc[C][t][r] + a * dxs[r];
            }
        }
    }
    // Blocks B0 (accumulator 2q) and B0 + 1 (accumulator 2q + 1), in order.
    template <int B0>
    static __device__ __forceinline__ void two_blocks(const uint8_t *slab, const uint8_t *xq, const float *xd, int j,
                                                      int g, float acc[2][MT][4]) {
        one_block<B0, 0>(slab, xq, xd, j, g, acc);
        // Keep each block's MFMAs beside its terms: hoisted together, the
        // four blocks' results would not fit the 128 registers a wave has
        // at four waves per SIMD.
        __builtin_amdgcn_sched_barrier(0);
        one_block<B0 + 1, 1>(slab, xq, xd, j, g, acc);
        __builtin_amdgcn_sched_barrier(0);
    }

    // PK = 2 (at most 8 tokens): blocks B0 and B0 + 1 share one MFMA result
    // tile, as in the pair kernel's packed_group: the A operand's row i is
    // (block i / 8, token i % 8), each block's MFMA sees zeros in the other
    // block's rows, and one MFMA against -8 serves both. Lane l then holds
    // block B0 + (l / 32) of its row l % 16 for tokens 4 ((l / 16) % 2) + r,
    // every value live: its accumulator is that block's (2q or 2q + 1).
    template <int B0>
    static __device__ __forceinline__ void packed_two(const uint8_t *slab, const uint8_t *xq, const float *xd, int j,
                                                      int g, float pacc[4]) {
        const int ablk = j >> 3, atok = j & 7;           // this lane's A row
        const int dblk = g >> 1, dtok = 4 * (g & 1);     // its result rows
        const long ax = *reinterpret_cast<const long *>(xq + atok * G::APITCH + 32 * (B0 + ablk) + 8 * g);
        long bw0, bw1;
        float dw0, dw1;
        RowsKernel<MT>::template weights_of<B0>(slab, j, g, bw0, dw0);
        RowsKernel<MT>::template weights_of<B0 + 1>(slab, j, g, bw1, dw1);
        v4i d = {0, 0, 0, 0};
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ablk == 0 ? ax : 0L, bw0, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ablk == 1 ? ax : 0L, bw1, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, as_long(0xF8F8F8F8u, 0xF8F8F8F8u), d, 0, 0, 0);
        const float dw = dblk == 0 ? dw0 : dw1;
        const float4 dx = *reinterpret_cast<const float4 *>(xd + (B0 + dblk) * G::XDP + dtok);
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float a = (float)d[r] * dw;
            pacc[r] = pacc[r] + a * dxs[r];
        }
    }

    static __device__ __forceinline__ void run(const RowsParams &P, uint8_t *lds) {
        if constexpr (PK == 2)
            run_packed(P, lds);
        else
            run_tiles(P, lds);
    }

    static __device__ __forceinline__ void run_packed(const RowsParams &P, uint8_t *lds) {
        const int tid = threadIdx.x;
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int grp = wave >> 2, q = wave & 3;
        const int j = lane & 15, g = lane >> 4;
        const int row_bytes = P.k / QK * Q4_0_BYTES;
        const int nseg = P.k / SEG;
        const int n0 = ((int)blockIdx.x * GROUPS + grp) * 16;

        Slots s;
        slots(P, row_bytes, s);
        Regs rg;
        load(P, s, row_bytes, n0, 0, nseg, rg);
        stage(lds, lds + G::SLAB_OFF + grp * SLAB, s, rg);
        load(P, s, row_bytes, n0, 1, nseg, rg);
        __syncthreads();

        float pacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int sg = 0; sg < nseg; ++sg) {
            const uint8_t *xbuf = lds + (sg & 1) * G::XBUF;
            const uint8_t *slab = lds + G::SLAB_OFF + ((sg & 1) * GROUPS + grp) * SLAB + 36 * q;
            const uint8_t *xq = xbuf + 64 * q;
            const float *xd = reinterpret_cast<const float *>(xbuf + G::XD_OFF) + 2 * q * G::XDP;
            packed_two<0>(slab, xq, xd, j, g, pacc);
            packed_two<8>(slab, xq, xd, j, g, pacc);
#pragma unroll
            for (int r = 0; r < 4; ++r) __asm__ volatile("" : "+v"(pacc[r]));
            const int nx = sg + 1;
            stage(lds + (nx & 1) * G::XBUF, lds + G::SLAB_OFF + ((nx & 1) * GROUPS + grp) * SLAB, s, rg);
            load(P, s, row_bytes, n0, nx + 1, nseg, rg);
            __syncthreads();
        }

        // a_2q + a_2q+1 meet across the lane halves; then the waves as below.
        const int dtok = 4 * (g & 1);
        const bool holder = g < 2;
        float part[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) part[r] = pacc[r] + __shfl_xor(pacc[r], 32);
        float *ex = reinterpret_cast<float *>(lds) + grp * 3 * G::TT * 16;
        if (q != 0 && holder) {
#pragma unroll
            for (int r = 0; r < 4; ++r) ex[((q - 1) * G::TT + dtok + r) * 16 + j] = part[r];
        }
        __syncthreads();
        if (q == 0) {
            const uint32_t y_bytes = (uint32_t)P.m * (uint32_t)P.rows * 4u;
            const __amdgpu_buffer_rsrc_t yb = rsrc(P.y, y_bytes);
            const bool row_ok = holder && n0 + j < P.rows;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = dtok + r;
                const float p1 = ex[(0 * G::TT + tok) * 16 + j];
                const float p2 = ex[(1 * G::TT + tok) * 16 + j];
                const float p3 = ex[(2 * G::TT + tok) * 16 + j];
                const float yv = (part[r] + p1) + (p2 + p3);
                const bool ok = row_ok && tok < P.m;
                __builtin_amdgcn_raw_buffer_store_b32(
                    __float_as_uint(yv), yb, ok ? (int)(((uint32_t)tok * (uint32_t)P.rows + (uint32_t)(n0 + j)) * 4u) : OUT_OF_RANGE,
                    0, 0);
            }
        }
    }

    static __device__ __forceinline__ void run_tiles(const RowsParams &P, uint8_t *lds) {
        const int tid = threadIdx.x;
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int grp = wave >> 2, q = wave & 3;
        const int j = lane & 15, g = lane >> 4;
        const int row_bytes = P.k / QK * Q4_0_BYTES;
        const int nseg = P.k / SEG;
        const int n0 = ((int)blockIdx.x * GROUPS + grp) * 16;

        Slots s;
        slots(P, row_bytes, s);
        Regs rg;
        load(P, s, row_bytes, n0, 0, nseg, rg);
        stage(lds, lds + G::SLAB_OFF + grp * SLAB, s, rg);
        load(P, s, row_bytes, n0, 1, nseg, rg);
        __syncthreads();

        float acc[2][MT][4];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[c][t][r] = 0.0f;

        for (int sg = 0; sg < nseg; ++sg) {
            const uint8_t *xbuf = lds + (sg & 1) * G::XBUF;
            const uint8_t *slab = lds + G::SLAB_OFF + ((sg & 1) * GROUPS + grp) * SLAB + 36 * q;
            const uint8_t *xq = xbuf + 64 * q;
            const float *xd = reinterpret_cast<const float *>(xbuf + G::XD_OFF) + 2 * q * G::XDP;
            two_blocks<0>(slab, xq, xd, j, g, acc);
            two_blocks<8>(slab, xq, xd, j, g, acc);
            // The terms are complete here: left alone, the compiler sinks
            // them below the staging's divergent stores, and the DPP
            // broadcasts of the scales then no longer fold into their
            // multiplies.
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) __asm__ volatile("" : "+v"(acc[c][t][r]));
            // Segment sg + 1 into the other buffers (last read for segment
            // sg - 1, before the previous barrier); the registers then take
            // segment sg + 2.
            const int nx = sg + 1;
            stage(lds + (nx & 1) * G::XBUF, lds + G::SLAB_OFF + ((nx & 1) * GROUPS + grp) * SLAB, s, rg);
            load(P, s, row_bytes, n0, nx + 1, nseg, rg);
            __syncthreads();
        }

        // The tree: waves 1..3 hand their parts to wave 0.
        float part[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[t][r] = acc[0][t][r] + acc[1][t][r];
        float *ex = reinterpret_cast<float *>(lds) + grp * 3 * G::TT * 16;
        if (q != 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) ex[((q - 1) * G::TT + 16 * t + 4 * g + r) * 16 + j] = part[t][r];
        }
        __syncthreads();
        if (q == 0) {
            const uint32_t y_bytes = (uint32_t)P.m * (uint32_t)P.rows * 4u;
            const __amdgpu_buffer_rsrc_t yb = rsrc(P.y, y_bytes);
            const bool row_ok = n0 + j < P.rows;
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = 16 * t + 4 * g + r;
                    const float p1 = ex[(0 * G::TT + tok) * 16 + j];
                    const float p2 = ex[(1 * G::TT + tok) * 16 + j];
                    const float p3 = ex[(2 * G::TT + tok) * 16 + j];
                    const float yv = (part[t][r] + p1) + (p2 + p3);
                    const bool ok = row_ok && tok < P.m;
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __float_as_uint(yv), yb, ok ? (int)(((uint32_t)tok * (uint32_t)P.rows + (uint32_t)(n0 + j)) * 4u) : OUT_OF_RANGE,
                        0, 0);
                }
        }
    }
};

template <int MT, int GROUPS, int PK>
__global__ __launch_bounds__(64 * 4 * GROUPS) void gemm_rows_quad_kernel(RowsParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    QuadKernel<MT, GROUPS, PK>::run(P, lds);
}

template <int MT, int GROUPS, int PK = 1>
hipError_t launch_rows_quad(const RowsParams &P, hipStream_t stream) {
    const void *fn = reinterpret_cast<const void *>(&gemm_rows_quad_kernel<MT, GROUPS, PK>);
    const hipError_t e = allow_dynamic_lds(fn, LDS_MAX);
    if (e != hipSuccess) return e;
    using G = QuadGeo<MT, GROUPS>;
    const int grid = (P.rows + 16 * GROUPS - 1) / (16 * GROUPS);
    hipLaunchKernelGGL((gemm_rows_quad_kernel<MT, GROUPS, PK>), dim3((unsigned)grid), dim3(G::THREADS), G::LDS, stream,
                       P);
    return hipGetLastError();
}

template <int MT, int PK>
__global__ __launch_bounds__(64 * 2 * pairs_of<MT>()) void gemm_rows_kernel(RowsParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    RowsKernel<MT, PK>::run(P, lds);
}

template <int MT, int PK = 1>
hipError_t launch_rows_mt(const RowsParams &P, hipStream_t stream) {
    const void *fn = reinterpret_cast<const void *>(&gemm_rows_kernel<MT, PK>);
    const hipError_t e = allow_dynamic_lds(fn, LDS_MAX);
    if (e != hipSuccess) return e;
    using G = RGeo<MT>;
    const int grid = (P.rows + 16 * G::PAIRS - 1) / (16 * G::PAIRS);
    hipLaunchKernelGGL((gemm_rows_kernel<MT, PK>), dim3((unsigned)grid), dim3(G::THREADS), G::LDS, stream, P);
    return hipGetLastError();
}

}  // namespace

bool gemm_rows_fits(int rows, int k) {
    return k % SEG == 0 && (size_t)rows * (size_t)(k / QK * Q4_0_BYTES) < 0x7fff0000u;
}

// m <= 64 tokens; y is [m][rows].
hipError_t launch_gemm_rows(const uint8_t *w, const uint8_t *x, int m, float *y, int rows, int k, hipStream_t stream) {
    if (m < 1 || m > 64 || !gemm_rows_fits(rows, k)) return hipErrorInvalidValue;
    RowsParams P{};
    P.w = w;
    P.x = x;
    P.y = y;
    P.rows = rows;
    P.k = k;
    P.m = m;
    P.x_stride = k + k / 8;
    if (m <= 4) return launch_rows_mt<1, 4>(P, stream);
    // One token tile: two 16-row groups a workgroup, two workgroups a CU
    // (four groups a workgroup were slower: gate|up at 8 / 16 tokens 8.8
    // against 8.3 / 8.4 us, the LM head 48.2 / 51.7 against 43.6 / 49.5).
    if (m <= 8) return launch_rows_quad<1, 2, 2>(P, stream);
    if (m <= 16) return launch_rows_quad<1, 2>(P, stream);
    if (m <= 32) return launch_rows_quad<2, 4>(P, stream);
    return launch_rows_quad<4, 4>(P, stream);
}

}  // namespace w4a8
