// Batched W4A8 (M > 1, prefill): Y[m][n] = sum over blocks of W[n] . X[m], for
// every (token m, row n) the contract's order (src/llm_kv260/q4_0.py:170-182)
// exactly as the M = 1 kernel computes it.
//
// Here the work is a dense contraction, so the integer part runs on CDNA4
// int8 MFMA: v_mfma_i32_16x16x32_i8 multiplies a 16 (tokens) x 32 by a 32 x 16
// (rows) int8 tile. K = 32 is exactly one block, so each MFMA result is one
// block's exact int32 sum for 16 x 16 (token, row) pairs, never mixed across
// blocks. The weight operand is the unsigned nibble n (0..15); a second MFMA
// against a constant -8 matrix adds -8 * sum(x) into the same accumulator, so
// the registers end up holding sum((n - 8) * x) with no VALU work.
//
// Operand layout of the 16x16x32 i8 MFMA (64 lanes, 8 int8 per lane):
//   A: lane l holds A[i = l % 16][k = 8 (l / 16) .. + 7]
//   B: lane l holds B[k = 8 (l / 16) .. + 7][j = l % 16]
//   D: lane l holds D[i = 4 (l / 16) + r][j = l % 16], r = 0..3 (4 VGPRs)
// Within a block, k-group g = 0..3 pairs x[8g .. 8g+7] with weights 8g .. 8g+7:
// the low nibbles of block bytes 0..7 (g = 0) and 8..15 (g = 1), then the high
// nibbles of bytes 0..7 (g = 2) and 8..15 (g = 3).
//
// The fp32 epilogue then runs per (token, row) on the VALU: t = (f32(sumi) *
// d_w) * d_x, lane b % 8 accumulation in registers, the adjacent-pair tree at
// the end. Each wave owns 16 rows of W and MT x 16 tokens.
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int WAVES = 4;

struct GemmParams {
    const uint8_t *w;
    const uint8_t *x;      // m rows, engine layout
    float *y;              // [m][rows]
    int rows;
    int k;
    int m;
    int x_stride;          // bytes per activation row
};

__device__ __forceinline__ long pack8(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

template <int MT>
__global__ __launch_bounds__(64 * WAVES) void gemm_mfma_kernel(GemmParams P) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * WAVES + wave) * 16;
    if (n0 >= P.rows) return;
    const int m_base = blockIdx.y * (MT * 16);
    const int nb = P.k >> 5;
    const int row_bytes = nb * Q4_0_BYTES;
    const int j = lane & 15;           // row within the tile (B column, D column)
    const int g = lane >> 4;           // k-group (A, B) / D row group
    const int n = n0 + j;
    const bool n_ok = n < P.rows;
    const uint8_t *wrow = P.w + (size_t)(n_ok ? n : n0) * row_bytes;
    const int half = g & 1, hi_nib = g >> 1;

    // Activation rows this lane feeds (A) and receives (D) per m-tile.
    const uint8_t *xa[MT];
    const uint8_t *xd_rows[MT][4];
    bool m_ok[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int ma = m_base + t * 16 + j;
        xa[t] = P.x + (size_t)(ma < P.m ? ma : 0) * P.x_stride;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int md = m_base + t * 16 + 4 * g + r;
            m_ok[t][r] = md < P.m;
            xd_rows[t][r] = P.x + (size_t)(md < P.m ? md : 0) * P.x_stride + P.k;
        }
    }

    float acc[MT][4][LANES];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int l = 0; l < LANES; ++l) acc[t][r][l] = 0.0f;

    const long minus8 = pack8(0xF8F8F8F8u, 0xF8F8F8F8u);

    for (int b0 = 0; b0 < nb; b0 += LANES) {
#pragma unroll
        for (int l = 0; l < LANES; ++l) {
            const int b = b0 + l;
            const uint8_t *blk = wrow + (size_t)b * Q4_0_BYTES;
            uint16_t dbits;
            __builtin_memcpy(&dbits, blk, 2);
            uint32_t q[2];
            __builtin_memcpy(q, blk + 2 + 8 * half, 8);
            const uint32_t s = hi_nib ? 4u : 0u;
            const long bw = pack8((q[0] >> s) & 0x0F0F0F0Fu, (q[1] >> s) & 0x0F0F0F0Fu);
            const float dw = half_bits_to_float(dbits);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                long ax;
                __builtin_memcpy(&ax, xa[t] + 32 * b + 8 * g, 8);
                v4i c = {0, 0, 0, 0};
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, minus8, c, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float dx = reinterpret_cast<const float *>(xd_rows[t][r])[b];
                    const float a = (float)c[r] * dw;
                    acc[t][r][l] = acc[t][r][l] + a * dx;
                }
            }
        }
    }

#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float *L = acc[t][r];
            const float yv = ((L[0] + L[1]) + (L[2] + L[3])) + ((L[4] + L[5]) + (L[6] + L[7]));
            const int md = m_base + t * 16 + 4 * g + r;
            if (n_ok && m_ok[t][r]) P.y[(size_t)md * P.rows + n] = yv;
        }
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
    const int ntiles = (w.rows + 15) / 16;
    const int gx = (ntiles + WAVES - 1) / WAVES;
    // Few tokens: one 16-token tile per wave. More: two, so each weight block
    // loaded feeds two MFMA pairs.
    if (m <= 16) {
        hipLaunchKernelGGL(gemm_mfma_kernel<1>, dim3(gx, (m + 15) / 16), dim3(64 * WAVES), 0, stream, P);
    } else {
        hipLaunchKernelGGL(gemm_mfma_kernel<2>, dim3(gx, (m + 31) / 32), dim3(64 * WAVES), 0, stream, P);
    }
    return hipGetLastError();
}

}  // namespace w4a8
