// Batched W4A8 (M > 1, prefill): Y[m][n] = sum over blocks of W[n] . X[m], for
// every (token m, row n) in the contract's order (src/llm_kv260/q4_0.py:170-182)
// exactly as the M = 1 kernel computes it.
//
// Here the work is a dense contraction, so the integer part runs on CDNA4 int8
// MFMA: v_mfma_i32_16x16x32_i8 multiplies a 16 (tokens) x 32 by a 32 x 16
// (rows) int8 tile. K = 32 is exactly one block, so each MFMA result is one
// block's exact int32 sum for 16 x 16 (token, row) pairs, never mixed across
// blocks. The weight operand is the unsigned nibble n (0..15); a second MFMA
// against a constant -8 operand adds -8 * sum(x) into the same accumulator, so
// the registers end up holding sum((n - 8) * x) with no VALU work.
//
// Operand layout of the 16x16x32 i8 MFMA (64 lanes, 8 int8 per lane):
//   A: lane l holds A[i = l % 16][k = 8 (l / 16) .. + 7]      (token i)
//   B: lane l holds B[k = 8 (l / 16) .. + 7][j = l % 16]      (row j)
//   D: lane l holds D[i = 4 (l / 16) + r][j = l % 16], r = 0..3
// Within a block, k-group g = 0..3 pairs x[8g .. 8g+7] with weights 8g .. 8g+7:
// the low nibbles of block bytes 0..7 (g = 0) and 8..15 (g = 1), then the high
// nibbles of bytes 0..7 (g = 2) and 8..15 (g = 3).
//
// Order without serialising K: the contract's accumulator a (0..7) of an
// output adds the terms of blocks a, a + 8, a + 16, ... in that order, and
// never sees another block. A workgroup owns 16 rows x 16 MT tokens over all
// of K with eight waves, and wave w owns accumulator a = w: it computes the
// terms of blocks 8c + w for c = 0, 1, ... in increasing order and adds each
// to its accumulator as it goes, from +0.0f. The eight waves' accumulators of
// an output then meet once, in the adjacent-pair tree.
//
// Data: the K dimension goes in rounds of four chunks (32 blocks). A round's
// weights (16 rows x 4 chunks x 144 bytes, as 16-byte pieces spread over all
// threads), activations (int8, 16 MT tokens x 32 blocks) and activation
// scales are loaded into registers four rounds ahead, then written to LDS as
// they came: the MFMA lanes read their 8-byte nibble runs and fp16 scales out
// of the raw 18-byte blocks there. A workgroup is persistent: it takes
// several (row tile, token tile) items and its rounds form one sequence
// across them. Every load is a raw buffer load, issued by every thread on
// every path: lanes with nothing to load (rows past N, tokens past M, blocks
// past K, rounds past the workgroup's last) are out of the buffer's range and
// read nothing, so the waits on the loads in flight are exact.
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GW = 8;                  // waves per workgroup; wave w owns accumulator w
constexpr int GTHREADS = 64 * GW;
constexpr int NR = 16;                 // rows per workgroup (the MFMA's 16 columns)
constexpr int RC = 4;                  // chunks per round
constexpr int RB = RC * CHUNK_BLOCKS;  // blocks per round (32)
constexpr int OUT_OF_RANGE = 0x7ffffff0;
constexpr uint32_t BUFFER_DWORD3 = 0x00020000;
constexpr int CACHE_NT = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, BUFFER_DWORD3);
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

// LDS layout of one round (bytes), for MT token tiles.
template <int MT>
struct Lds {
    static constexpr int WS = 0;                                 // [NR][RC] x 144 B raw weight chunks
    static constexpr int XQ = WS + NR * RC * CHUNK_BYTES;        // [16 MT][RB] x 32 B activations
    static constexpr int XD = XQ + 16 * MT * RB * 32;            // [RB][16 MT] fp32 activation scales
    static constexpr int BYTES = XD + 16 * MT * RB * 4;
    // The accumulators of the eight waves, [8][16 MT][NR] fp32, reuse XQ at the end.
    static_assert(8 * 16 * MT * NR * 4 <= 16 * MT * RB * 32, "accumulator exchange must fit");
};

constexpr int W_PIECES = NR * RC * CHUNK_PIECES;                          // 576 per round
constexpr int W_PER_THREAD = (W_PIECES + GTHREADS - 1) / GTHREADS;       // 2

// One round in registers.
template <int MT>
struct Stage {
    u32x4 w[W_PER_THREAD];   // raw weight pieces t, t + GTHREADS of the round
    u32x4 xq[2 * MT];        // 16-byte activation pieces
    u32x4 xd;                // four activation scales: threads < 128 MT
};

// Round `round` of the item whose first row is n0 and first token m0
// (live_round == false: a round past the workgroup's last, which reads nothing).
template <int MT, int NRW>
__device__ __forceinline__ void load_round(const GemmParams &P, int n0, int m0, int round, bool live_round, int nb,
                                           Stage<MT> &s) {
    const int t = threadIdx.x;
    const int row_bytes = nb * Q4_0_BYTES;
    const int b0 = round * RB;
    // Weights: piece p of the round is row p / 36, chunk p % 36 / 9, piece p % 9.
    const __amdgpu_buffer_rsrc_t wb = buffer_of(P.w, (uint32_t)((size_t)P.rows * row_bytes));
#pragma unroll
    for (int i = 0; i < W_PER_THREAD; ++i) {
        const int p = t + GTHREADS * i;
        const int j = p / (RC * CHUNK_PIECES), within = p - j * (RC * CHUNK_PIECES);
        const int cc = within / CHUNK_PIECES, q = within - cc * CHUNK_PIECES;
        const int n = n0 + j, c = b0 / CHUNK_BLOCKS + cc;
        const bool live = live_round && p < W_PIECES && j < NRW && n < P.rows && c < nb / CHUNK_BLOCKS;
        s.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wb, live ? n * row_bytes + c * CHUNK_BYTES + 16 * q : OUT_OF_RANGE,
                                                       0, CACHE_NT);
    }
    const __amdgpu_buffer_rsrc_t xb = buffer_of(P.x, (uint32_t)((size_t)P.m * P.x_stride));
    // Activations: piece p = t + GTHREADS i of 64 per token: block p % 64 / 2, half p % 2.
#pragma unroll
    for (int i = 0; i < 2 * MT; ++i) {
        const int p = t + GTHREADS * i;
        const int tok = p >> 6, bb = (p & 63) >> 1, h = p & 1;
        const int m = m0 + tok, b = b0 + bb;
        const bool live = live_round && m < P.m && b < nb;
        s.xq[i] = __builtin_amdgcn_raw_buffer_load_b128(xb, live ? m * P.x_stride + 32 * b + 16 * h : OUT_OF_RANGE, 0, 0);
    }
    // Activation scales: thread t < 128 MT loads blocks 4 (t % 8) .. + 3 of token t / 8.
    {
        const int tok = t >> 3, q = t & 7;
        const int m = m0 + tok, b = b0 + 4 * q;
        const bool live = live_round && t < 128 * MT && m < P.m && b < nb;
        s.xd = __builtin_amdgcn_raw_buffer_load_b128(xb, live ? m * P.x_stride + P.k + 4 * b : OUT_OF_RANGE, 0, 0);
    }
}

template <int MT>
__device__ __forceinline__ void store_round(uint8_t *lds, const Stage<MT> &s) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < W_PER_THREAD; ++i) {
        const int p = t + GTHREADS * i;
        if (p < W_PIECES) *reinterpret_cast<u32x4 *>(lds + Lds<MT>::WS + p * 16) = s.w[i];
    }
#pragma unroll
    for (int i = 0; i < 2 * MT; ++i) {
        const int p = t + GTHREADS * i;
        *reinterpret_cast<u32x4 *>(lds + Lds<MT>::XQ + p * 16) = s.xq[i];   // token p / 64, block, half: in order
    }
    // Scales of token t / 8, blocks 4 (t % 8) .. + 3, stored block-major so
    // that the four tokens one MFMA lane needs are one 16-byte read.
    if (t < 128 * MT) {
        const int tok = t >> 3, b4 = 4 * (t & 7);
        float *xd = reinterpret_cast<float *>(lds + Lds<MT>::XD);
        xd[(b4 + 0) * 16 * MT + tok] = __uint_as_float(s.xd.x);
        xd[(b4 + 1) * 16 * MT + tok] = __uint_as_float(s.xd.y);
        xd[(b4 + 2) * 16 * MT + tok] = __uint_as_float(s.xd.z);
        xd[(b4 + 3) * 16 * MT + tok] = __uint_as_float(s.xd.w);
    }
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// Wave w's terms of the round's blocks 8 c + w, added to its accumulators in
// block order. Chunks of a round past K hold zeros in LDS (their loads were
// out of range): weight scale +0, activation +0, so their terms are +0.0 and
// leave the accumulators unchanged (an accumulator starts at +0.0 and is
// never -0.0). ODD: w is odd (its block starts two bytes into a dword).
template <int MT, bool ODD>
__device__ __forceinline__ void compute_round(const uint8_t *lds, float acc[MT][4]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const long minus8 = as_long(0xF8F8F8F8u, 0xF8F8F8F8u);
    const int shift = (g >> 1) * 4;
#pragma unroll
    for (int cc = 0; cc < RC; ++cc) {
        const int bb = cc * 8 + w;                                  // block within the round
        // Block w of chunk cc of row j starts 18 w bytes into the chunk: an
        // even w at a dword boundary (scale in the low half, nibbles two
        // bytes in), an odd w two bytes into a dword (scale in the high half,
        // nibbles dword-aligned).
        const int blk = Lds<MT>::WS + (j * RC + cc) * CHUNK_BYTES + 18 * w;
        uint32_t lo, hi, d_bits;
        if constexpr (!ODD) {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(lds + blk + 8 * (g & 1));
            const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
            lo = __builtin_amdgcn_alignbyte(d1, d0, 2);
            hi = __builtin_amdgcn_alignbyte(d2, d1, 2);
            d_bits = *reinterpret_cast<const uint32_t *>(lds + blk) & 0xFFFFu;
        } else {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(lds + blk + 2 + 8 * (g & 1));
            lo = p[0];
            hi = p[1];
            d_bits = *reinterpret_cast<const uint32_t *>(lds + blk - 2) >> 16;
        }
        const long bw = as_long((lo >> shift) & 0x0F0F0F0Fu, (hi >> shift) & 0x0F0F0F0Fu);
        const float dw = half_bits_to_float(d_bits);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint32_t *xa = reinterpret_cast<const uint32_t *>(lds + Lds<MT>::XQ + ((16 * t + j) * RB + bb) * 32 + 8 * g);
            const long ax = as_long(xa[0], xa[1]);
            v4i c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, minus8, c, 0, 0, 0);
            const float4 dx = *reinterpret_cast<const float4 *>(lds + Lds<MT>::XD + (bb * 16 * MT + 16 * t + 4 * g) * 4);
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a = (float)c[r] * dw;
                acc[t][r] = acc[t][r] + a * dxs[r];
            }
        }
    }
}

// The eight accumulators of each output of the item (n0, m0) meet in the
// adjacent-pair tree; the registers then restart from +0.0f.
template <int MT, int NRW>
__device__ __forceinline__ void finish_item(const GemmParams &P, uint8_t *lds, int n0, int m0, float acc[MT][4]) {
    __syncthreads();
    {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        const int j = lane & 15, g = lane >> 4;
        float *ex = reinterpret_cast<float *>(lds + Lds<MT>::XQ);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ex[(w * 16 * MT + 16 * t + 4 * g + r) * NR + j] = acc[t][r];
                acc[t][r] = 0.0f;
            }
    }
    __syncthreads();
    const float *ex = reinterpret_cast<const float *>(lds + Lds<MT>::XQ);
    for (int o = threadIdx.x; o < 16 * MT * NRW; o += GTHREADS) {
        const int tok = o / NRW, j = o % NRW;
        float l[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) l[a] = ex[(a * 16 * MT + tok) * NR + j];
        const float yv = ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
        const int m = m0 + tok, n = n0 + j;
        if (m < P.m && n < P.rows) P.y[(size_t)m * P.rows + n] = yv;
    }
}

// Persistent: workgroup g takes items g, g + G, ... (an item = NRW rows x
// 16 MT tokens over all of K), and its rounds form one sequence across its
// items, so the loads of the next item's first rounds are in flight while
// the current item finishes. NRW = 8 leaves the MFMA's columns 8..15 unused
// (their outputs are discarded) and doubles the number of items for matrices
// with few rows.
template <int MT, int NRW>
__global__ __launch_bounds__(GTHREADS) void gemm_mfma_kernel(GemmParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int nb = P.k >> 5;
    const int R = (nb + RB - 1) / RB;                      // rounds per item
    const int n_rt = (P.rows + NRW - 1) / NRW;
    const int items = n_rt * ((P.m + 16 * MT - 1) / (16 * MT));
    const int G = gridDim.x;
    const int my_items = (int)blockIdx.x < items ? (items - 1 - (int)blockIdx.x) / G + 1 : 0;
    const int S = my_items * R;                            // rounds in this workgroup's sequence

    // Sequence index s -> item (n0, m0) and round r.
    auto coords = [&](int s, int &n0, int &m0, int &r) {
        const int k = s / R;
        r = s - k * R;
        const int it = (int)blockIdx.x + k * G;
        const int tg = it / n_rt;
        n0 = (it - tg * n_rt) * NRW;
        m0 = tg * 16 * MT;
    };
    auto load = [&](int s, Stage<MT> &st) {
        int n0, m0, r;
        coords(s < S ? s : 0, n0, m0, r);
        load_round<MT, NRW>(P, n0, m0, r, s < S, nb, st);
    };

    float acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;

    // DEPTH rounds in flight: while round s is written to LDS and computed,
    // the next DEPTH - 1 are outstanding and round s + DEPTH is issued (four,
    // or three for 64-token tiles, whose stages are larger). The loads and
    // LDS writes of a round past the end still happen (they read nothing);
    // only its compute is skipped, so the body is the same on every pass.
    constexpr int DEPTH = MT >= 4 ? 3 : 4;
    Stage<MT> st[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(d, st[d]);
    auto step = [&](int s, Stage<MT> &stage) {
        __syncthreads();
        store_round<MT>(lds, stage);
        __syncthreads();
        load(s + DEPTH, stage);
        if (s < S) {
            int n0, m0, r;
            coords(s, n0, m0, r);
            if ((threadIdx.x >> 6) & 1)
                compute_round<MT, true>(lds, acc);
            else
                compute_round<MT, false>(lds, acc);
            if (r == R - 1) finish_item<MT, NRW>(P, lds, n0, m0, acc);
        }
    };
    for (int s = 0; s < S; s += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) step(s + d, st[d]);
    }
}

template <int MT, int NRW>
hipError_t launch_mt(const GemmParams &P, hipStream_t stream) {
    const void *fn = reinterpret_cast<const void *>(&gemm_mfma_kernel<MT, NRW>);
    static bool lds_allowed = false;
    if (!lds_allowed) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, Lds<MT>::BYTES);
        if (e != hipSuccess) return e;
        lds_allowed = true;
    }
    static int per_cu[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!per_cu[dev]) {
        int n = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, GTHREADS, Lds<MT>::BYTES);
        if (e != hipSuccess) return e;
        per_cu[dev] = n > 0 ? n : 1;
    }
    const long items = (long)((P.rows + NRW - 1) / NRW) * ((P.m + 16 * MT - 1) / (16 * MT));
    long grid = (long)device_cu_count() * per_cu[dev];
    if (grid > items) grid = items;
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, NRW>), dim3((unsigned)grid), dim3(GTHREADS), Lds<MT>::BYTES, stream, P);
    return hipGetLastError();
}

template <int MT>
hipError_t launch_rows(const GemmParams &P, hipStream_t stream) {
    // 16-row items unless that leaves fewer items than two per CU.
    const long items16 = (long)((P.rows + 15) / 16) * ((P.m + 16 * MT - 1) / (16 * MT));
    return items16 >= 2L * device_cu_count() ? launch_mt<MT, 16>(P, stream) : launch_mt<MT, 8>(P, stream);
}

}  // namespace

hipError_t launch_gemm(const MatrixRef &w, const uint8_t *x, int m, float *y, hipStream_t stream) {
    GemmParams P{};
    P.w = w.seg[0];
    P.x = x;
    P.y = y;
    P.rows = w.rows;
    P.k = w.k;
    P.m = m;
    P.x_stride = w.k + w.k / 8;
    // Buffer ranges are 32-bit byte counts.
    if ((size_t)P.rows * (size_t)(P.k / QK * Q4_0_BYTES) >= 0x7fff0000u ||
        (size_t)P.m * (size_t)P.x_stride >= 0x7fff0000u)
        return hipErrorInvalidValue;
    // Token tiles per workgroup: all of M up to 64 tokens, so the weights
    // stream once; beyond that, 64-token groups.
    if (m <= 16) return launch_rows<1>(P, stream);
    if (m <= 32) return launch_rows<2>(P, stream);
    return launch_rows<4>(P, stream);
}

}  // namespace w4a8
