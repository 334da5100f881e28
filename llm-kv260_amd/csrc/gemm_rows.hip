// Batched W4A8 (M > 1) for matrices with many rows: the same results as
// gemm_mfma.hip (the contract's order, src/llm_kv260/q4_0.py:170-182, applied
// row by row), with the work cut along rows instead of along the blocks of K.
//
// A 16-row group belongs to WPG waves for the whole of K, and wave w of the
// group owns A = 8 / WPG of the contract's eight accumulators: it takes the
// blocks b with b % 8 in [A w, A w + A), in increasing b, and adds each term
// to accumulator b % 8 from +0.0f. At the end the group's waves meet once
// through LDS for the adjacent-pair tree's last adds.
//  - From 5 tokens a group has four waves (QuadKernel, two accumulators a
//    wave): a SIMD then runs four waves, so one wave's LDS reads, MFMA
//    latency and waits are covered by the others' fp32 terms.
//  - Up to 4 tokens it has two (PairKernel, four accumulators a wave), and
//    four blocks share one MFMA result tile (packed tiles, below).
// A workgroup holds GROUPS groups, which share the staged activation.
//
// K goes by segments of 512 values (16 blocks). Per segment a group stages its
// 16 rows' 288-byte runs in a slab of its own, and the workgroup stages the
// tokens' 512 activation bytes and 16 scales once for all its groups: one
// barrier per segment, with the loads of the next segments in flight.
//
// The integer part is v_mfma_i32_16x16x32_i8 (K = 32 is one block), one MFMA
// per block and token tile on the weights as 16 (n - 8) (block_weights).
// Operand layout of the 16x16x32 i8 MFMA (64 lanes):
//   A: lane l holds A[i = l % 16][k = 8 (l / 16) .. + 7]      (token i)
//   B: lane l holds B[k = 8 (l / 16) .. + 7][j = l % 16]      (row j)
//   D: lane l holds D[i = 4 (l / 16) + r][j = l % 16], r = 0..3
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int SEG = 512;                          // activation values per segment
constexpr int SEG_BLOCKS = SEG / QK;              // 16
constexpr int SEG_ROW_BYTES = SEG_BLOCKS * Q4_0_BYTES;   // 288
constexpr int W_PIECES = 16 * SEG_ROW_BYTES / 16;        // 288 pieces of 16 B per group and segment
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

// Block B (0..15) of a staged segment, row j of the group: the MFMA weight
// operand of lane group g (weights 8g .. 8g + 7: the low nibbles of bytes
// 0..7, g = 0, and 8..15, g = 1, then the high nibbles, g = 2, 3) and the
// block's scale. The operand is 16 (n - 8) as signed bytes: each nibble n
// moved to its byte's high half (where the high nibbles already are) and its
// top bit flipped, (n << 4) ^ 0x80 = 16 (n - 8) as int8 -- as cheap as the
// unsigned nibble, and it needs no second MFMA against -8. The MFMA sums are
// then 16 sumi exactly, and the scale comes back as d_w / 16 (exact: a
// power of two on an fp16 value, never subnormal in fp32), so the term
// f32(16 sumi) * (d_w / 16) is the same product as f32(sumi) * d_w,
// rounded once: every later operation sees the contract's value.
template <int B>
__device__ __forceinline__ void block_weights(const uint8_t *slab, int j, int g, long &bw, float &dw16) {
    const int h = g & 1;
    const int up = 4 - (g >> 1) * 4;            // 4: low nibbles, 0: high nibbles
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
    bw = as_long(((lo << up) & 0xF0F0F0F0u) ^ 0x80808080u, ((hi << up) & 0xF0F0F0F0u) ^ 0x80808080u);
    dw16 = half_bits_to_float(d_bits) * 0.0625f;
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

// A workgroup: GROUPS 16-row groups of WPG waves, MT token tiles of 16.
// LDS: two segment buffers of the activation ([TT][APITCH] int8 values, then
// the scales [16 blocks][XDP]), then two slabs per group. The waves' parts
// for the tree's last adds go over the activation buffers at the end, which
// every wave has finished reading by then.
template <int MT, int GROUPS, int WPG>
struct Geo {
    static constexpr int TT = 16 * MT;                       // tokens
    static constexpr int APITCH = SEG + 16;                  // int8 bytes per token and segment, padded
    static constexpr int XDP = TT + 4;                       // scale rows: [16 blocks][XDP]
    static constexpr int XD_OFF = TT * APITCH;
    static constexpr int XBUF = XD_OFF + SEG_BLOCKS * XDP * 4;
    static constexpr int GT = 64 * WPG;                      // threads per group
    static constexpr int THREADS = GT * GROUPS;
    static constexpr int SLAB_OFF = 2 * XBUF;                // [2][GROUPS] slabs
    static constexpr int LDS = SLAB_OFF + 2 * GROUPS * SLAB;
    static constexpr int EX_FLOATS = GROUPS * (WPG - 1) * TT * 16;
    static_assert(EX_FLOATS * 4 <= LDS, "the exchange within the buffers");
    static_assert(LDS <= LDS_MAX, "LDS budget");
    static constexpr int X_PIECES = TT * (SEG / 16);         // int8 pieces per segment
    static constexpr int D_PIECES = TT * (SEG_BLOCKS / 4);   // scale pieces (4 scales each)
    static constexpr int SW = (W_PIECES + GT - 1) / GT;      // weight pieces per thread of a group
    static constexpr int SX = (X_PIECES + THREADS - 1) / THREADS;
    static constexpr int SD = (D_PIECES + THREADS - 1) / THREADS;
};

// A segment's loads into registers, and their staging into LDS.
template <class G>
struct Stager {
    struct Regs {
        u32x4 w[G::SW];
        u32x4 x[G::SX];
        u32x4 d[G::SD];
    };

    // Fixed per-thread offsets: weight pieces of the group's rows, activation
    // and scale pieces of the workgroup's tokens.
    struct Slots {
        uint32_t w_go[G::SW];
        int w_lo[G::SW];       // slab byte offset, -1 for no piece
        uint32_t x_go[G::SX];
        int x_lo[G::SX];
        uint32_t d_go[G::SD];
        int d_lo[G::SD];       // float index of the piece's first scale in a buffer
    };

    static __device__ __forceinline__ void slots(const RowsParams &P, int row_bytes, Slots &s) {
        const int tid = threadIdx.x;
        const int tp = tid & (G::GT - 1);        // thread within the group
#pragma unroll
        for (int i = 0; i < G::SW; ++i) {
            const int n = tp + G::GT * i;
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
        for (int i = 0; i < G::SW; ++i) rg.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wb, (int)s.w_go[i], 0, CACHE_NT);
#pragma unroll
        for (int i = 0; i < G::SX; ++i) rg.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xb, (int)s.x_go[i], 0, 0);
#pragma unroll
        for (int i = 0; i < G::SD; ++i) rg.d[i] = __builtin_amdgcn_raw_buffer_load_b128(db, (int)s.d_go[i], 0, 0);
    }

    static __device__ __forceinline__ void stage(uint8_t *xbuf, uint8_t *slab, const Slots &s, const Regs &rg) {
#pragma unroll
        for (int i = 0; i < G::SW; ++i)
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
};

__device__ __forceinline__ void store_y(const RowsParams &P, bool ok, int tok, int row, float v) {
    const __amdgpu_buffer_rsrc_t yb = rsrc(P.y, (uint32_t)P.m * (uint32_t)P.rows * 4u);
    __builtin_amdgcn_raw_buffer_store_b32(
        __float_as_uint(v), yb, ok ? (int)(((uint32_t)tok * (uint32_t)P.rows + (uint32_t)row) * 4u) : OUT_OF_RANGE, 0,
        0);
}

// Up to 4 tokens: pairs of waves, wave h owning accumulators 4h .. 4h + 3,
// two groups a workgroup (two workgroups share a CU, each running while the
// other waits at its segment barrier). Packed tiles: four blocks of at most
// four tokens share one MFMA result tile, so that the fp32 epilogue touches
// only live outputs. The A operand's 16 rows are (block c, token t) =
// (i / 4, i % 4); block c's MFMA sees zeros in every other block's rows, so
// the four MFMAs put each block's exact int32 sums in its own rows of one
// tile. The result's lane l then holds block c = l / 16 of the four, tokens
// r = 0..3, row l % 16: every lane live, one fp32 term per value, and the
// lane's accumulator is its block's.
struct PairKernel {
    static constexpr int GROUPS = 2;
    using G = Geo<1, GROUPS, 2>;
    using S = Stager<G>;

    template <int B0, int C>
    static __device__ __forceinline__ void packed_mfma(const uint8_t *slab, int j, int g, int ablk, long ax, v4i &d,
                                                       float &dw) {
        long bw;
        float dwc;
        block_weights<B0 + C>(slab, j, g, bw, dwc);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ablk == C ? ax : 0L, bw, d, 0, 0, 0);
        dw = g == C ? dwc : dw;
        if constexpr (C + 1 < 4) packed_mfma<B0, C + 1>(slab, j, g, ablk, ax, d, dw);
    }

    // Blocks B0 .. B0 + 3: their terms, added to the lane's accumulator
    // (that of its block, B0 % 8 + l / 16) in block order.
    template <int B0>
    static __device__ __forceinline__ void packed_group(const uint8_t *slab, const uint8_t *xbuf, int j, int g,
                                                        float acc[4]) {
        const int ablk = j >> 2, atok = j & 3;            // this lane's A row (block, token)
        const long ax = *reinterpret_cast<const long *>(xbuf + atok * G::APITCH + 32 * (B0 + ablk) + 8 * g);
        v4i d = {0, 0, 0, 0};
        float dw = 0.0f;
        packed_mfma<B0, 0>(slab, j, g, ablk, ax, d, dw);
        // The four tokens' scales of the lane's block: one 16-byte read (a
        // block's scales are a row of XDP floats, tokens along it).
        const float4 dx =
            *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(xbuf + G::XD_OFF) + (B0 + g) * G::XDP);
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float a = (float)d[r] * dw;
            acc[r] = acc[r] + a * dxs[r];
        }
    }

    static __device__ __forceinline__ void run(const RowsParams &P, uint8_t *lds) {
        const int tid = threadIdx.x;
        // The wave index is uniform: as a scalar, the group's resources and
        // the choice of accumulators are scalar too (no per-lane resource loop).
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int pair = wave >> 1, half = wave & 1;
        const int j = lane & 15, g = lane >> 4;
        const int row_bytes = P.k / QK * Q4_0_BYTES;
        const int nseg = P.k / SEG;
        const int n0 = ((int)blockIdx.x * GROUPS + pair) * 16;   // the pair's first row

        typename S::Slots s;
        S::slots(P, row_bytes, s);
        // Two segments in flight.
        typename S::Regs rg[2];
        S::load(P, s, row_bytes, n0, 0, nseg, rg[0]);
        S::load(P, s, row_bytes, n0, 1, nseg, rg[1]);
        S::stage(lds, lds + G::SLAB_OFF + pair * SLAB, s, rg[0]);
        S::load(P, s, row_bytes, n0, 2, nseg, rg[0]);
        __syncthreads();

        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int sg0 = 0; sg0 < nseg; sg0 += 2) {
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const int sg = sg0 + d;
                if (sg < nseg) {
                    const uint8_t *xbuf = lds + (sg & 1) * G::XBUF;
                    const uint8_t *slab = lds + G::SLAB_OFF + ((sg & 1) * GROUPS + pair) * SLAB;
                    // The wave's eight blocks of the segment: 4 half + c, then
                    // 8 + 4 half + c, in order.
                    if (half == 0) {
                        packed_group<0>(slab, xbuf, j, g, acc);
                        packed_group<8>(slab, xbuf, j, g, acc);
                    } else {
                        packed_group<4>(slab, xbuf, j, g, acc);
                        packed_group<12>(slab, xbuf, j, g, acc);
                    }
                }
                // Segment sg + 1 into the other buffers (last read for
                // segment sg - 1, before the previous barrier); its registers
                // then take segment sg + 3.
                const int nx = sg + 1;
                S::stage(lds + (nx & 1) * G::XBUF, lds + G::SLAB_OFF + ((nx & 1) * GROUPS + pair) * SLAB, s,
                         rg[(d + 1) & 1]);
                S::load(P, s, row_bytes, n0, nx + 2, nseg, rg[(d + 1) & 1]);
                __syncthreads();
            }
        }

        // The wave's four accumulators of an output sit in lanes 16 apart
        // (lane group c holds a_4half+c): the tree's (a0 + a1) + (a2 + a3),
        // then wave 1's part goes to wave 0 through LDS. Lane group 0 holds
        // the sums.
        float part[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float s01 = acc[r] + __shfl_xor(acc[r], 16);
            part[r] = s01 + __shfl_xor(s01, 32);
        }
        float *ex = reinterpret_cast<float *>(lds) + pair * G::TT * 16;
        if (half == 1 && g == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) ex[r * 16 + j] = part[r];
        }
        __syncthreads();
        if (half == 0) {
            const bool row_ok = n0 + j < P.rows && g == 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) store_y(P, row_ok && r < P.m, r, n0 + j, part[r] + ex[r * 16 + j]);
        }
    }
};

// From 5 tokens: four waves per 16-row group (a quad), wave q owning the
// accumulators 2q and 2q + 1, so it takes the blocks b with b % 8 in
// {2q, 2q + 1}. At the end the tree's last adds, (p0 + p1) + (p2 + p3) with
// p_q = a_2q + a_2q+1, meet through LDS: wave 0 of the group adds them, or
// at four token tiles wave q adds tile q's. PK = 2 (at most 8 tokens):
// packed tiles of two blocks.
template <int MT, int GROUPS, int PK = 1>
struct QuadKernel {
    using G = Geo<MT, GROUPS, 4>;
    using S = Stager<G>;
    static_assert(PK == 1 || (PK == 2 && MT == 1), "packed quads: two blocks of at most 8 tokens a tile");

    // Block B of the wave's view of the segment (the wave's blocks start at
    // 2q, folded into the pointers; B keeps the parity): its MFMA sums for
    // every token tile, the weight scale and the tokens' scales.
    template <int B>
    static __device__ __forceinline__ void block_sums(const uint8_t *slab, const uint8_t *xq, const float *xd, int j,
                                                      int g, v4i v[MT], float &dw, float dx[MT]) {
        long bw;
        block_weights<B>(slab, j, g, bw, dw);
        const uint8_t *xa = xq + j * G::APITCH + 32 * B + 8 * g;
        const float *xs = xd + B * G::XDP + 4 * g + (j & 3);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const long ax = *reinterpret_cast<const long *>(xa + 16 * t * G::APITCH);
            dx[t] = xs[16 * t];
            v4i z = {0, 0, 0, 0};
            v[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
        }
    }

    // Block B (accumulator C of the wave's two): MFMAs first, then the fp32
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

    // PK = 2: blocks B0 and B0 + 1 share one MFMA result tile, as in
    // PairKernel: the A operand's row i is (block i / 8, token i % 8). Lane
    // l then holds block B0 + (l / 32) of its row l % 16 for tokens
    // 4 ((l / 16) % 2) + r, and its accumulator is that block's.
    template <int B0>
    static __device__ __forceinline__ void packed_two(const uint8_t *slab, const uint8_t *xq, const float *xd, int j,
                                                      int g, float pacc[4]) {
        const int ablk = j >> 3, atok = j & 7;           // this lane's A row
        const int dblk = g >> 1, dtok = 4 * (g & 1);     // its result rows
        const long ax = *reinterpret_cast<const long *>(xq + atok * G::APITCH + 32 * (B0 + ablk) + 8 * g);
        long bw0, bw1;
        float dw0, dw1;
        block_weights<B0>(slab, j, g, bw0, dw0);
        block_weights<B0 + 1>(slab, j, g, bw1, dw1);
        v4i d = {0, 0, 0, 0};
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ablk == 0 ? ax : 0L, bw0, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ablk == 1 ? ax : 0L, bw1, d, 0, 0, 0);
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
        const int tid = threadIdx.x;
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int grp = wave >> 2, q = wave & 3;
        const int j = lane & 15, g = lane >> 4;
        const int row_bytes = P.k / QK * Q4_0_BYTES;
        const int nseg = P.k / SEG;
        const int n0 = ((int)blockIdx.x * GROUPS + grp) * 16;

        typename S::Slots s;
        S::slots(P, row_bytes, s);
        typename S::Regs rg;
        S::load(P, s, row_bytes, n0, 0, nseg, rg);
        S::stage(lds, lds + G::SLAB_OFF + grp * SLAB, s, rg);
        S::load(P, s, row_bytes, n0, 1, nseg, rg);
        __syncthreads();

        // PK = 1: acc[c][t][r], accumulator 2q + c, tile t, token 16 t + 4 g + r.
        // PK = 2: acc[0][0][r], the lane's block's accumulator, token 4 (g % 2) + r.
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
            if constexpr (PK == 2) {
                packed_two<0>(slab, xq, xd, j, g, acc[0][0]);
                packed_two<8>(slab, xq, xd, j, g, acc[0][0]);
            } else {
                two_blocks<0>(slab, xq, xd, j, g, acc);
                two_blocks<8>(slab, xq, xd, j, g, acc);
            }
            // The terms are complete here: left alone, the compiler sinks
            // them below the staging's divergent stores, and the DPP
            // broadcasts of the scales then no longer fold into their
            // multiplies.
#pragma unroll
            for (int c = 0; c < (PK == 2 ? 1 : 2); ++c)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) __asm__ volatile("" : "+v"(acc[c][t][r]));
            // Segment sg + 1 into the other buffers (last read for segment
            // sg - 1, before the previous barrier); the registers then take
            // segment sg + 2.
            const int nx = sg + 1;
            S::stage(lds + (nx & 1) * G::XBUF, lds + G::SLAB_OFF + ((nx & 1) * GROUPS + grp) * SLAB, s, rg);
            S::load(P, s, row_bytes, n0, nx + 1, nseg, rg);
            __syncthreads();
        }

        if constexpr (MT == 4) {
            // Every wave hands its four tiles' parts over, and wave q adds
            // tile q's: the final adds and the stores spread over the group.
            static_assert(GROUPS * 4 * G::TT * 16 * 4 <= G::LDS, "the exchange within the buffers");
            float *ex4 = reinterpret_cast<float *>(lds) + grp * 4 * G::TT * 16;
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ex4[(q * G::TT + 16 * t + 4 * g + r) * 16 + j] = acc[0][t][r] + acc[1][t][r];
            __syncthreads();
            const bool row_ok = n0 + j < P.rows;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = 16 * q + 4 * g + r;
                const float p0 = ex4[(0 * G::TT + tok) * 16 + j];
                const float p1 = ex4[(1 * G::TT + tok) * 16 + j];
                const float p2 = ex4[(2 * G::TT + tok) * 16 + j];
                const float p3 = ex4[(3 * G::TT + tok) * 16 + j];
                store_y(P, row_ok && tok < P.m, tok, n0 + j, (p0 + p1) + (p2 + p3));
            }
            return;
        }
        // The tree: p_q = a_2q + a_2q+1 (PK = 2: across the lane halves),
        // then waves 1..3 hand their parts to wave 0.
        constexpr int NT = PK == 2 ? 1 : MT;
        float part[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                part[t][r] = PK == 2 ? acc[0][0][r] + __shfl_xor(acc[0][0][r], 32) : acc[0][t][r] + acc[1][t][r];
        // The lane's tokens: 16 t + 4 g + r; PK = 2, 4 (g % 2) + r, the
        // lanes of block 0 (g < 2) holding the sums.
        const bool holder = PK == 1 || g < 2;
        const int tok0 = PK == 2 ? 4 * (g & 1) : 4 * g;
        float *ex = reinterpret_cast<float *>(lds) + grp * 3 * G::TT * 16;
        if (q != 0 && holder) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) ex[((q - 1) * G::TT + 16 * t + tok0 + r) * 16 + j] = part[t][r];
        }
        __syncthreads();
        if (q == 0) {
            const bool row_ok = holder && n0 + j < P.rows;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = 16 * t + tok0 + r;
                    const float p1 = ex[(0 * G::TT + tok) * 16 + j];
                    const float p2 = ex[(1 * G::TT + tok) * 16 + j];
                    const float p3 = ex[(2 * G::TT + tok) * 16 + j];
                    store_y(P, row_ok && tok < P.m, tok, n0 + j, (part[t][r] + p1) + (p2 + p3));
                }
        }
    }
};

__global__ __launch_bounds__(PairKernel::G::THREADS) void gemm_rows_pair_kernel(RowsParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    PairKernel::run(P, lds);
}

template <int MT, int GROUPS, int PK>
__global__ __launch_bounds__(64 * 4 * GROUPS) void gemm_rows_quad_kernel(RowsParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    QuadKernel<MT, GROUPS, PK>::run(P, lds);
}

template <class G>
hipError_t launch_rows(void (*kernel)(RowsParams), const RowsParams &P, hipStream_t stream, int groups) {
    const hipError_t e = allow_dynamic_lds(reinterpret_cast<const void *>(kernel), LDS_MAX);
    if (e != hipSuccess) return e;
    const int grid = (P.rows + 16 * groups - 1) / (16 * groups);
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(G::THREADS), G::LDS, stream, P);
    return hipGetLastError();
}

template <int MT, int GROUPS, int PK = 1>
hipError_t launch_rows_quad(const RowsParams &P, hipStream_t stream) {
    return launch_rows<typename QuadKernel<MT, GROUPS, PK>::G>(&gemm_rows_quad_kernel<MT, GROUPS, PK>, P, stream,
                                                               GROUPS);
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
    if (m <= 4) return launch_rows<PairKernel::G>(&gemm_rows_pair_kernel, P, stream, PairKernel::GROUPS);
    // One token tile: two 16-row groups a workgroup, two workgroups a CU
    // (four groups a workgroup were slower: gate|up at 8 / 16 tokens 8.8
    // against 8.3 / 8.4 us, the LM head 48.2 / 51.7 against 43.6 / 49.5).
    if (m <= 8) return launch_rows_quad<1, 2, 2>(P, stream);
    if (m <= 16) return launch_rows_quad<1, 2>(P, stream);
    if (m <= 32) return launch_rows_quad<2, 4>(P, stream);
    return launch_rows_quad<4, 4>(P, stream);
}

}  // namespace w4a8
