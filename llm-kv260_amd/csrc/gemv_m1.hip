// M = 1 W4A8 GEMV for gfx950: y[N] = W[N, K] x, W in ggml Q4_0, x in Q8_0.
//
// A bandwidth problem with a latency tail, so no MFMA and no barriers in the
// row loop. The unit of work is a row and the unit of parallelism a wave64:
//
//  * Lane j of a wave owns block j of the row (and j + 64, j + 128, ... when
//    K/32 > 64; several rows share a wave when K/32 < 64). Consecutive lanes
//    own consecutive 18-byte blocks, so the wave's five dword loads per block
//    cover the row's bytes contiguously: coalesced without any staging. An
//    18-byte block starts 0 or 2 bytes into a dword (even / odd block), so one
//    v_perm_b32 per nibble dword, with a per-lane selector, realigns it.
//  * The activation is staged once per workgroup in LDS (quantized there from
//    fp32 for the fused entry point) with each block's int8 sum, then every
//    lane keeps its own blocks' 32 int8 values, scale and sum in registers for
//    all the rows the wave visits.
//  * Each block's dot is exact in int32: eight v_dot4_i32_i8 on the unsigned
//    nibbles minus 8 * sum(x). Then t = (f32(sumi) * d_w) * d_x.
//  * The contract's order (src/llm_kv260/q4_0.py:170-182): lane l of a row
//    adds the terms of blocks l, l + 8, l + 16, ... in that order. Those terms
//    sit in lanes l, l + 8, ... of the wave (blocks j + 64m follow m-major),
//    so each lane gathers them with ds_bpermute in block order and adds them
//    one by one from +0.0f; the eight lane sums of a row then meet in a DPP
//    adjacent-pair tree.
//  * Weight loads for the wave's next row are issued before the current row is
//    reduced, so each wave keeps two rows of loads in flight.
#include "../../include/w4a8.h"
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / 64;
constexpr int MAX_NB = MAX_K_M1 / QK;            // 512 blocks
constexpr int MAX_NBPL = MAX_NB / 64;            // blocks per lane

struct GemvParams {
    const uint8_t *seg[4];
    const void *x;
    float *y;
    int seg_rows;     // rows per segment
    int nseg;
    int k;
    int lpr;          // lanes per row: min(K/32, 64)
    int rpw;          // rows per wave: 64 / lpr
    int groups;       // row groups (of rpw rows) in the whole matrix
    int paired;       // v2 port layout
};

// Stage block b of the activation into LDS: int8 values, fp32 scale, int8 sum.
template <int XF>
__device__ __forceinline__ void stage_x_block(const void *x, int k, int b, uint32_t *s_q, float *s_d, int32_t *s_s) {
    uint32_t q[8];
    float dx;
    if constexpr (XF == X_ENGINE) {
        const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(x) + 32 * b);
        const uint4 a = src[0], c = src[1];
        q[0] = a.x; q[1] = a.y; q[2] = a.z; q[3] = a.w;
        q[4] = c.x; q[5] = c.y; q[6] = c.z; q[7] = c.w;
        dx = reinterpret_cast<const float *>(static_cast<const uint8_t *>(x) + k)[b];
    } else if constexpr (XF == X_Q8_0) {
        const uint16_t *src = reinterpret_cast<const uint16_t *>(static_cast<const uint8_t *>(x) + Q8_0_BYTES * b);
        dx = half_bits_to_float(src[0]);
#pragma unroll
        for (int m = 0; m < 8; ++m) q[m] = (uint32_t)src[1 + 2 * m] | ((uint32_t)src[2 + 2 * m] << 16);
    } else {
        const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + 32 * b);
        float v[32];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const float4 f = src[m];
            v[4 * m] = f.x; v[4 * m + 1] = f.y; v[4 * m + 2] = f.z; v[4 * m + 3] = f.w;
        }
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
        const float d = q8_scale(amax);
        const float inv = safe_recip(d);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            uint32_t w = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) w |= ((uint32_t)(uint8_t)q8_round(v[4 * m + e], inv)) << (8 * e);
            q[m] = w;
        }
        dx = half_bits_to_float(float_to_half_bits(d));
    }
    int32_t sum = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) sum = __builtin_amdgcn_sdot4((int)q[m], 0x01010101, sum, false);
    uint4 *dst = reinterpret_cast<uint4 *>(s_q + 8 * b);
    dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
    dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
    s_d[b] = dx;
    s_s[b] = sum;
}

// Byte address of block b of row r (r counted over the whole matrix).
__device__ __forceinline__ const uint8_t *block_addr(const GemvParams &P, int r, int b) {
    const int nch = P.k >> 8;
    const int seg = r / P.seg_rows, local = r - seg * P.seg_rows;
    const uint8_t *base = P.seg[seg];
    if (P.paired) {
        // v2 port region: row i pairs with row i + R/2; their 144-byte chunks alternate.
        const int half = P.seg_rows >> 1;
        const int which = local >= half, i = local - which * half;
        return base + ((size_t)(i * nch + (b >> 3)) * 2 + which) * CHUNK_BYTES + Q4_0_BYTES * (b & 7);
    }
    return base + (size_t)local * (size_t)(nch * CHUNK_BYTES) + (size_t)Q4_0_BYTES * b;
}

// The five dwords covering an 18-byte block (4-byte aligned start, 0 or 2 bytes early).
struct BlockWords {
    uint32_t w[5];
};

__device__ __forceinline__ BlockWords load_block(const uint8_t *p) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(reinterpret_cast<uintptr_t>(p) & ~(uintptr_t)3);
    BlockWords r;
#pragma unroll
    for (int i = 0; i < 5; ++i) r.w[i] = __builtin_nontemporal_load(q + i);
    return r;
}

// Term t of one block: odd = the block starts 2 bytes into its first dword.
// The nibble bytes start 2 (even) or 4 (odd) bytes into the five dwords;
// v_perm_b32 picks the four bytes of each nibble dword from the pair
// {w[m+1], w[m]} with a per-lane selector (bytes 0-3 = w[m], 4-7 = w[m+1]).
__device__ __forceinline__ float block_term_words(const BlockWords &bw, bool odd, const uint32_t xv[8], int32_t xsum,
                                                  float dx) {
    const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
    uint32_t qs[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) qs[m] = __builtin_amdgcn_perm(bw.w[m + 1], bw.w[m], sel);
    const uint32_t d_bits = odd ? (bw.w[0] >> 16) : (bw.w[0] & 0xFFFFu);
    const int32_t sumi = block_dot_raw(qs, xv) - 8 * xsum;
    return block_term(sumi, d_bits, dx);
}

__device__ __forceinline__ float bpermute_f(int src_lane, float v) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}

template <int XF, int NBPL>
__global__ __launch_bounds__(THREADS) void gemv_m1_kernel(GemvParams P) {
    __shared__ __attribute__((aligned(16))) uint32_t s_q[MAX_NB * 8];
    __shared__ float s_d[MAX_NB];
    __shared__ int32_t s_s[MAX_NB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int nb = P.k >> 5;
    const int total_rows = P.seg_rows * P.nseg;

    for (int b = tid; b < nb; b += THREADS) stage_x_block<XF>(P.x, P.k, b, s_q, s_d, s_s);
    __syncthreads();

    // This lane's place: row slot within the wave's row group, block column.
    const int lpr = P.lpr;
    const int slot = lane / lpr;
    const int col = lane - slot * lpr;
    const bool lane_live = slot < P.rpw;
    const int row_lane0 = slot * lpr;        // first lane of this lane's row
    const int l8 = lane & 7;

    // The lane's activation blocks, kept in registers for every row.
    uint32_t xv[NBPL][8];
    float xd[NBPL];
    int32_t xs[NBPL];
    bool has[NBPL];
#pragma unroll
    for (int m = 0; m < NBPL; ++m) {
        const int b = col + 64 * m;
        has[m] = lane_live && b < nb;
        const int bb = has[m] ? b : 0;
        const uint4 *src = reinterpret_cast<const uint4 *>(s_q + 8 * bb);
        const uint4 a = src[0], c = src[1];
        xv[m][0] = a.x; xv[m][1] = a.y; xv[m][2] = a.z; xv[m][3] = a.w;
        xv[m][4] = c.x; xv[m][5] = c.y; xv[m][6] = c.z; xv[m][7] = c.w;
        xd[m] = s_d[bb];
        xs[m] = s_s[bb];
    }

    const int wave_id = blockIdx.x * WAVES + (tid >> 6);
    const int nwaves = gridDim.x * WAVES;
    int g = wave_id;
    if (g >= P.groups) return;

    BlockWords cur[NBPL];
    {
        int r = g * P.rpw + slot;
        r = r < total_rows ? r : total_rows - 1;
#pragma unroll
        for (int m = 0; m < NBPL; ++m) cur[m] = load_block(block_addr(P, r, has[m] ? col + 64 * m : 0));
    }

    const int groups8 = lpr >> 3;
    for (; g < P.groups; g += nwaves) {
        const int r = g * P.rpw + slot;
        const int gn = g + nwaves;
        BlockWords nxt[NBPL];
        if (gn < P.groups) {
            int rn = gn * P.rpw + slot;
            rn = rn < total_rows ? rn : total_rows - 1;
#pragma unroll
            for (int m = 0; m < NBPL; ++m) nxt[m] = load_block(block_addr(P, rn, has[m] ? col + 64 * m : 0));
        }

        float t[NBPL];
#pragma unroll
        for (int m = 0; m < NBPL; ++m)
            t[m] = has[m] ? block_term_words(cur[m], (col & 1) != 0, xv[m], xs[m], xd[m]) : 0.0f;

        // Lane l8 of the row: terms of blocks l8, l8 + 8, ... in block order.
        // Blocks beyond K/32 contribute +0.0f at the end of the order, which
        // leaves a sum that started from +0.0f unchanged.
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < NBPL; ++m) {
            for (int c8 = 0; c8 < groups8; ++c8) acc = acc + bpermute_f(row_lane0 + 8 * c8 + l8, t[m]);
        }
        const float yv = tree8_dpp(acc);
        if (lane_live && col == 0 && r < total_rows) P.y[r] = yv;

#pragma unroll
        for (int m = 0; m < NBPL; ++m) cur[m] = nxt[m];
    }
}

template <int XF>
hipError_t launch_xf(const GemvParams &P, int nbpl, int grid, hipStream_t stream) {
    const dim3 g(grid), b(THREADS);
    switch (nbpl) {
        case 1: hipLaunchKernelGGL((gemv_m1_kernel<XF, 1>), g, b, 0, stream, P); break;
        case 2: hipLaunchKernelGGL((gemv_m1_kernel<XF, 2>), g, b, 0, stream, P); break;
        case 3: hipLaunchKernelGGL((gemv_m1_kernel<XF, 3>), g, b, 0, stream, P); break;
        case 4: hipLaunchKernelGGL((gemv_m1_kernel<XF, 4>), g, b, 0, stream, P); break;
        case 5: hipLaunchKernelGGL((gemv_m1_kernel<XF, 5>), g, b, 0, stream, P); break;
        case 6: hipLaunchKernelGGL((gemv_m1_kernel<XF, 6>), g, b, 0, stream, P); break;
        case 7: hipLaunchKernelGGL((gemv_m1_kernel<XF, 7>), g, b, 0, stream, P); break;
        case 8: hipLaunchKernelGGL((gemv_m1_kernel<XF, 8>), g, b, 0, stream, P); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

hipError_t launch_gemv_m1(const MatrixRef &w, const void *x, XFormat xf, float *y, hipStream_t stream) {
    GemvParams P{};
    for (int s = 0; s < 4; ++s) P.seg[s] = s < w.nseg ? w.seg[s] : w.seg[0];
    P.x = x;
    P.y = y;
    P.seg_rows = w.seg_rows;
    P.nseg = w.nseg;
    P.k = w.k;
    P.paired = w.paired ? 1 : 0;
    const int nb = w.k / QK;
    P.lpr = nb < 64 ? nb : 64;
    P.rpw = 64 / P.lpr;
    const int rows = w.seg_rows * w.nseg;
    P.groups = (rows + P.rpw - 1) / P.rpw;
    const int nbpl = (nb + 63) / 64;
    if (nbpl > MAX_NBPL) return hipErrorInvalidValue;
    // Enough waves for every row group up to a few workgroups per CU; beyond
    // that each wave walks several row groups.
    const int cus = device_cu_count();
    const int per_cu = nbpl <= 2 ? 8 : 4;
    int grid = (P.groups + WAVES - 1) / WAVES;
    if (grid > cus * per_cu) grid = cus * per_cu;
    if (grid < 1) return hipSuccess;
    switch (xf) {
        case X_ENGINE: return launch_xf<X_ENGINE>(P, nbpl, grid, stream);
        case X_Q8_0: return launch_xf<X_Q8_0>(P, nbpl, grid, stream);
        case X_F32: return launch_xf<X_F32>(P, nbpl, grid, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_chain(const w4a8_chain_step *steps, int n, hipStream_t stream) {
    // One fused quantize + GEMV kernel per step; stream order carries the
    // step-to-step dependency.
    for (int i = 0; i < n; ++i) {
        MatrixRef m{};
        m.seg[0] = static_cast<const uint8_t *>(steps[i].w);
        m.nseg = 1;
        m.seg_rows = steps[i].rows;
        m.rows = steps[i].rows;
        m.k = steps[i].k;
        const hipError_t e = launch_gemv_m1(m, steps[i].x, X_F32, steps[i].y, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace w4a8
