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
// never sees another block. A workgroup's eight waves share an item (16 or 8
// rows x 16 MT tokens over all of K), and wave w owns accumulator a = w: it
// computes the terms of blocks 8c + w for c = 0, 1, ... in increasing order
// and adds each to its accumulator as it goes, from +0.0f. The eight waves'
// accumulators of an output then meet once, in the adjacent-pair tree.
//
// Data: each wave streams exactly the bytes it uses, straight from memory
// into registers, D chunks ahead (D = 8 -- 4 for 64-token tiles -- or the
// largest of 4, 2, 1 dividing the K / 256 chunks of a row, so that an item is
// whole groups of D chunks
// processed without a branch): per chunk, lane (row j, k-group g) loads the
// dwords holding its 8-byte nibble run and scale of block 8c + w of row j
// (the eight waves together read each 144-byte chunk once), and one 8-byte
// piece of each token tile's activations. The activation scales of the
// workgroup's tokens are staged in LDS once, block-major, so that the four
// tokens an MFMA lane needs are one 16-byte read. Nothing else is shared, so
// the waves meet only at item boundaries. Every load is a raw buffer load,
// issued by every lane on every path: lanes with nothing to load (rows past
// N, tokens past M, chunks past the workgroup's last item) are out of the
// buffer's range and read nothing, so the waits on the loads in flight are
// exact. Workgroups are persistent over items, and each wave's chunk stream
// runs on across items.
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GW = 8;                  // waves per workgroup; wave w owns accumulator w
constexpr int GTHREADS = 64 * GW;
constexpr int NR = 16;                 // the MFMA's 16 row columns
constexpr int OUT_OF_RANGE = 0x7ffffff0;
constexpr uint32_t BUFFER_DWORD3 = 0x00020000;
constexpr int CACHE_NT = 2;
constexpr int LDS_MAX = 160 * 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, BUFFER_DWORD3);
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

struct GemmParams {
    const uint8_t *w;
    const uint8_t *x;      // m rows, engine layout
    float *y;              // [m][rows]
    int rows;
    int k;
    int m;
    int x_stride;          // bytes per activation row, k + k / 8
};

// LDS: activation scales [nb][16 MT] fp32, then two exchange buffers
// [8][16 MT][NR] fp32 (consecutive items alternate between them).
template <int MT>
struct Lds {
    static constexpr int EX_BYTES = GW * 16 * MT * NR * 4;
    __host__ __device__ static int xd_bytes(int nb) { return nb * 16 * MT * 4; }
    __host__ __device__ static int bytes(int nb) { return xd_bytes(nb) + 2 * EX_BYTES; }
};

// One chunk of one wave in registers.
template <int MT>
struct Chunk {
    uint32_t w[4];           // the dwords holding the lane's nibble run, and its scale
    uint32_t x[MT][2];       // the lane's 8 activation bytes of each token tile
};

template <int MT, int NRW, int D, bool ODD>
struct Kernel {
    // Chunk c (block 8c + w of every row) of the item (n0, m0); live == false
    // reads nothing.
    static __device__ __forceinline__ void load(const GemmParams &P, int n0, int m0, int c, bool live, int row_bytes,
                                                Chunk<MT> &ch) {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        const int j = lane & 15, g = lane >> 4;
        const int n = n0 + j;
        const bool row_live = live && j < NRW && n < P.rows;
        // Block 8c + w of row n starts at o = n * row_bytes + 18 (8c + w):
        // even w at a dword boundary (the nibble run two bytes past it), odd
        // w two bytes into a dword (the run dword-aligned, the scale in the
        // high half of the dword before).
        const int o = n * row_bytes + 18 * (8 * c + w);
        const __amdgpu_buffer_rsrc_t wb = buffer_of(P.w, (uint32_t)((size_t)P.rows * row_bytes));
        if constexpr (!ODD) {
            const int base = row_live ? o + 8 * (g & 1) : OUT_OF_RANGE;
            ch.w[0] = __builtin_amdgcn_raw_buffer_load_b32(wb, base, 0, CACHE_NT);
            ch.w[1] = __builtin_amdgcn_raw_buffer_load_b32(wb, base + 4, 0, CACHE_NT);
            ch.w[2] = __builtin_amdgcn_raw_buffer_load_b32(wb, base + 8, 0, CACHE_NT);
            ch.w[3] = __builtin_amdgcn_raw_buffer_load_b32(wb, row_live ? o : OUT_OF_RANGE, 0, CACHE_NT);
        } else {
            const int base = row_live ? o + 2 + 8 * (g & 1) : OUT_OF_RANGE;
            ch.w[0] = __builtin_amdgcn_raw_buffer_load_b32(wb, base, 0, CACHE_NT);
            ch.w[1] = __builtin_amdgcn_raw_buffer_load_b32(wb, base + 4, 0, CACHE_NT);
            ch.w[3] = __builtin_amdgcn_raw_buffer_load_b32(wb, row_live ? o - 2 : OUT_OF_RANGE, 0, CACHE_NT);
        }
        const __amdgpu_buffer_rsrc_t xb = buffer_of(P.x, (uint32_t)((size_t)P.m * P.x_stride));
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int m = m0 + 16 * t + j;
            const int off = live && m < P.m ? m * P.x_stride + 32 * (8 * c + w) + 8 * g : OUT_OF_RANGE;
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(xb, off, 0, 0);
            ch.x[t][0] = (uint32_t)v[0];
            ch.x[t][1] = (uint32_t)v[1];
        }
    }

    // The terms of block 8c + w, added to the wave's accumulators.
    static __device__ __forceinline__ void compute(const Chunk<MT> &ch, const float *xd, int c, float acc[MT][4]) {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        const int g = lane >> 4;
        const int shift = (g >> 1) * 4;
        uint32_t lo, hi, d_bits;
        if constexpr (!ODD) {
            lo = __builtin_amdgcn_alignbyte(ch.w[1], ch.w[0], 2);
            hi = __builtin_amdgcn_alignbyte(ch.w[2], ch.w[1], 2);
            d_bits = ch.w[3] & 0xFFFFu;                    // the low half of the block's first dword
        } else {
            lo = ch.w[0];
            hi = ch.w[1];
            d_bits = ch.w[3] >> 16;                        // the high half of the dword before the run
        }
        const long bw = as_long((lo >> shift) & 0x0F0F0F0Fu, (hi >> shift) & 0x0F0F0F0Fu);
        const long minus8 = as_long(0xF8F8F8F8u, 0xF8F8F8F8u);
        const float dw = half_bits_to_float(d_bits);
        const int b = 8 * c + w;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            v4i v = {0, 0, 0, 0};
            const long ax = as_long(ch.x[t][0], ch.x[t][1]);
            v = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, v, 0, 0, 0);
            v = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, minus8, v, 0, 0, 0);
            const float4 dx = *reinterpret_cast<const float4 *>(xd + b * 16 * MT + 16 * t + 4 * g);
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a = (float)v[r] * dw;
                acc[t][r] = acc[t][r] + a * dxs[r];
            }
        }
    }

    // Activation scales of tokens m0 .. m0 + 16 MT - 1, block-major, into LDS.
    static __device__ __forceinline__ void stage_scales(const GemmParams &P, int m0, int nb, float *xd) {
        const __amdgpu_buffer_rsrc_t xb = buffer_of(P.x, (uint32_t)((size_t)P.m * P.x_stride));
        const int per_tok = nb / 4;                          // four blocks of one token per piece
        for (int p = threadIdx.x; p < 16 * MT * per_tok; p += GTHREADS) {
            const int tok = p / per_tok, b4 = 4 * (p - tok * per_tok);
            const int m = m0 + tok;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(
                xb, m < P.m ? m * P.x_stride + P.k + 4 * b4 : OUT_OF_RANGE, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) xd[(b4 + e) * 16 * MT + tok] = __uint_as_float((uint32_t)v[e]);
        }
    }

    // The eight accumulators of each output of the item (n0, m0) meet in the
    // adjacent-pair tree; the registers then restart from +0.0f.
    static __device__ __forceinline__ void finish(const GemmParams &P, float *ex, int n0, int m0, float acc[MT][4]) {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        const int j = lane & 15, g = lane >> 4;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ex[(w * 16 * MT + 16 * t + 4 * g + r) * NR + j] = acc[t][r];
                acc[t][r] = 0.0f;
            }
        __syncthreads();
        for (int o = threadIdx.x; o < 16 * MT * NRW; o += GTHREADS) {
            const int tok = o / NRW, j2 = o - tok * NRW;
            float l[8];
#pragma unroll
            for (int a = 0; a < 8; ++a) l[a] = ex[(a * 16 * MT + tok) * NR + j2];
            const float yv = ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
            const int m = m0 + tok, n = n0 + j2;
            if (m < P.m && n < P.rows) P.y[(size_t)m * P.rows + n] = yv;
        }
    }

    static __device__ __forceinline__ void run(const GemmParams &P, uint8_t *lds) {
        const int nb = P.k >> 5;
        const int C = nb >> 3;                                  // chunks per row = blocks per wave per item
        const int row_bytes = nb * Q4_0_BYTES;
        const int n_rt = (P.rows + NRW - 1) / NRW;
        const int items = n_rt * ((P.m + 16 * MT - 1) / (16 * MT));
        const int G = gridDim.x;
        const int my_items = (int)blockIdx.x < items ? (items - 1 - (int)blockIdx.x) / G + 1 : 0;
        const int S = my_items * C;                             // chunks in each wave's stream
        float *xd = reinterpret_cast<float *>(lds);
        float *ex0 = reinterpret_cast<float *>(lds + Lds<MT>::xd_bytes(nb));
        float *ex1 = ex0 + Lds<MT>::EX_BYTES / 4;

        auto item_of = [&](int k, int &n0, int &m0) {
            const int it = (int)blockIdx.x + k * G;
            const int tg = it / n_rt;
            n0 = (it - tg * n_rt) * NRW;
            m0 = tg * 16 * MT;
        };
        auto load_q = [&](int q, Chunk<MT> &ch) {
            const bool live = q < S;
            const int k = live ? q / C : 0;
            int n0, m0;
            item_of(k, n0, m0);
            load(P, n0, m0, live ? q - k * C : 0, live, row_bytes, ch);
        };

        // The first item's token group: scales staged before anything else.
        int cur_m0 = 0;
        {
            int n0;
            item_of(0, n0, cur_m0);
            if (my_items > 0) stage_scales(P, cur_m0, nb, xd);
        }
        Chunk<MT> st[D];
#pragma unroll
        for (int d = 0; d < D; ++d) load_q(d, st[d]);
        __syncthreads();

        float acc[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;

        // Each item is C / D groups of D chunks; stage d holds chunk q0 + d
        // of the stream and is refilled with chunk q0 + D + d after the
        // group, so the loads run one group ahead and a group is straight-
        // line code.
        int q0 = 0;
        for (int k = 0; k < my_items; ++k) {
            int n0, m0;
            item_of(k, n0, m0);
            if (m0 != cur_m0) {                                 // a new token group (M > 16 MT)
                __syncthreads();
                stage_scales(P, m0, nb, xd);
                __syncthreads();
                cur_m0 = m0;
            }
            for (int c0 = 0; c0 < C; c0 += D, q0 += D) {
#pragma unroll
                for (int d = 0; d < D; ++d) compute(st[d], xd, c0 + d, acc);
#pragma unroll
                for (int d = 0; d < D; ++d) load_q(q0 + D + d, st[d]);
            }
            finish(P, (k & 1) ? ex1 : ex0, n0, m0, acc);
        }
    }
};

template <int MT, int NRW, int D>
__global__ __launch_bounds__(GTHREADS) void gemm_mfma_kernel(GemmParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if ((threadIdx.x >> 6) & 1)
        Kernel<MT, NRW, D, true>::run(P, lds);
    else
        Kernel<MT, NRW, D, false>::run(P, lds);
}

template <int MT, int NRW, int D>
hipError_t launch_mt(const GemmParams &P, hipStream_t stream) {
    const void *fn = reinterpret_cast<const void *>(&gemm_mfma_kernel<MT, NRW, D>);
    const int lds = Lds<MT>::bytes(P.k / QK);
    static bool lds_allowed = false;
    if (!lds_allowed) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_MAX);
        if (e != hipSuccess) return e;
        lds_allowed = true;
    }
    int per_cu = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, GTHREADS, lds);
    if (e != hipSuccess) return e;
    if (per_cu < 1) per_cu = 1;
    const long items = (long)((P.rows + NRW - 1) / NRW) * ((P.m + 16 * MT - 1) / (16 * MT));
    long grid = (long)device_cu_count() * per_cu;
    if (grid > items) grid = items;
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, NRW, D>), dim3((unsigned)grid), dim3(GTHREADS), lds, stream, P);
    return hipGetLastError();
}

template <int MT, int NRW>
hipError_t launch_depth(const GemmParams &P, hipStream_t stream) {
    const int C = P.k / 256;
    if constexpr (MT < 4) {                 // a 64-token tile's stages only fit four deep
        if (C % 8 == 0) return launch_mt<MT, NRW, 8>(P, stream);
    }
    if (C % 4 == 0) return launch_mt<MT, NRW, 4>(P, stream);
    if (C % 2 == 0) return launch_mt<MT, NRW, 2>(P, stream);
    return launch_mt<MT, NRW, 1>(P, stream);
}

template <int MT>
hipError_t launch_rows(const GemmParams &P, hipStream_t stream) {
    // 16-row items unless that leaves fewer items than two per CU.
    const long items16 = (long)((P.rows + 15) / 16) * ((P.m + 16 * MT - 1) / (16 * MT));
    return items16 >= 2L * device_cu_count() ? launch_depth<MT, 16>(P, stream) : launch_depth<MT, 8>(P, stream);
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
    // stream once; beyond that, groups of 64 (32 when K is so long that a
    // group's activation scales would not fit in LDS).
    const int nb = P.k / QK;
    if (m <= 16) return launch_rows<1>(P, stream);
    if (m <= 32 || Lds<4>::bytes(nb) > LDS_MAX) return launch_rows<2>(P, stream);
    return launch_rows<4>(P, stream);
}

}  // namespace w4a8
