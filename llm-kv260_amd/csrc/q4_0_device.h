// Device-side building blocks of the W4A8 engine for gfx950 (CDNA4).
//
// The arithmetic is the contract's, src/llm_kv260/q4_0.py:151-182, step for step:
//   1. sumi[b] = sum_j (n_j - 8) * x_j in int32 (exact, so any order),
//   2. t[b]    = (f32(sumi) * f32(d_w)) * f32(d_x), two fp32 multiplies left to right,
//   3. lane b % 8 accumulates t[b] in increasing b starting from +0.0f,
//   4. the eight lanes are summed by the adjacent-pair tree.
// Everything here is compiled with -ffp-contract=off and without fast-math, so
// every fp32 expression below is exactly the IEEE operations written.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a8 {

constexpr int QK = 32;            // weights per block (q4_0.py:59)
constexpr int Q4_0_BYTES = 18;    // fp16 d + 16 nibble bytes (q4_0.py:60)
constexpr int Q8_0_BYTES = 34;    // fp16 d + 32 int8 (q4_0.py:61)
constexpr int LANES = 8;          // fp32 accumulation lanes (q4_0.py:62)
// Eight consecutive blocks are 144 bytes = nine 16-byte pieces: the unit a
// thread owns (the same 9-beat chunk hls/int4_core/q4_0.h:21-25 streams).
constexpr int CHUNK_BLOCKS = 8;
constexpr int CHUNK_BYTES = CHUNK_BLOCKS * Q4_0_BYTES;   // 144
constexpr int CHUNK_DWORDS = CHUNK_BYTES / 4;            // 36
constexpr int CHUNK_PIECES = CHUNK_BYTES / 16;           // 9

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    // v_cvt_f32_f16: exact for every binary16 value, subnormals included.
    return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFFu)));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    // v_cvt_f16_f32 under the default MODE (round to nearest even, fp16 denormals
    // kept). The empty asm pins f as an fp32 value first: without it the
    // compiler folds a preceding multiply into v_fma_mixlo_f16(a, b, +0), which
    // rounds the product once to fp16 instead of through fp32 and turns a -0
    // product into +0 (the contract's d = extreme / -8 is -0 for a zero block).
    __asm__ volatile("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}

// Exact int32 dot of one Q4_0 block's 16 nibble bytes (four little-endian
// dwords) with the block's 32 int8 activations, on v_dot8_u32_u4 and no
// unpacking. Byte j of the block carries weight j in its low nibble and
// weight j + 16 in its high one (q4_0.py:22-24), so nibble 2e of dword k is
// weight 4k + e and nibble 2e + 1 is weight 4k + e + 16. The activation comes
// pre-split to match (x_nibbles): with x' = x + 128 (1..255, unsigned),
// xn[k] holds the high nibbles of x'[4k + e] / x'[4k + e + 16] in nibbles
// 2e / 2e + 1, and xn[4 + k] the low nibbles. Then, n being the unsigned
// weight nibbles,
//   sum((n - 8) x) = 16 sum(n a) + sum(n b) - 128 sum(n) - 8 sum(x)
// with a, b the high and low nibbles of x'; every term is an exact unsigned
// 4-bit dot, accumulated modulo 2^32, and c8 = -8 sum(x) seeds the b chain.
// 12 dots and 2 integer ops per block, where splitting the nibbles for
// v_dot4 took 21.
__device__ __forceinline__ int32_t block_dot_nib(const uint32_t qs[4], const uint32_t xn[8], int32_t c8) {
    uint32_t a = 0, b = (uint32_t)c8, n = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        a = __builtin_amdgcn_udot8(qs[k], xn[k], a, false);
        b = __builtin_amdgcn_udot8(qs[k], xn[4 + k], b, false);
        n = __builtin_amdgcn_udot8(qs[k], 0x11111111u, n, false);
    }
    return (int32_t)(16u * a + b) - 128 * (int32_t)n;
}

// The same exact int32 for a block whose activation is given as its int8
// values (xr[m]: x[4m .. 4m + 3]) and whose weights are unpacked to bytes
// (unpack_nibbles: lo[k] = weights 4k .. 4k + 3, the low nibbles of dword k;
// hi[k] = weights 16 + 4k .., its high nibbles), each an unsigned byte 0..15
// that v_dot4_i32_i8 multiplies by the signed x; c8 = -8 sum(x) makes the sum
// that of (n - 8) x. Eight dots per block and activation, against
// block_dot_nib's twelve dots and two integer ops on a nibble-split x: the
// cheaper form where one unpacked block meets several activations.
__device__ __forceinline__ void unpack_nibbles(const uint32_t qs[4], uint32_t lo[4], uint32_t hi[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        lo[k] = qs[k] & 0x0F0F0F0Fu;
        hi[k] = (qs[k] >> 4) & 0x0F0F0F0Fu;
    }
}

__device__ __forceinline__ int32_t block_dot_raw(const uint32_t lo[4], const uint32_t hi[4], const uint32_t xr[8],
                                                 int32_t c8) {
    int32_t acc = c8;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        acc = __builtin_amdgcn_sdot4((int)lo[k], (int)xr[k], acc, false);
        acc = __builtin_amdgcn_sdot4((int)hi[k], (int)xr[4 + k], acc, false);
    }
    return acc;
}

// The activation of one block as block_dot_nib takes it, from its eight
// dwords of int8 values (byte e of q[m] is x[4m + e]).
__device__ __forceinline__ void x_nibbles(const uint32_t q[8], uint32_t xn[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = q[k] ^ 0x80808080u, hi = q[4 + k] ^ 0x80808080u;   // x + 128, bytewise
        xn[k] = ((lo >> 4) & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u);
        xn[4 + k] = (lo & 0x0F0F0F0Fu) | ((hi << 4) & 0xF0F0F0F0u);
    }
}

// The fp32 epilogue of one block, step 2 of the contract.
__device__ __forceinline__ float block_term(int32_t sumi, uint32_t dw_bits, float dx) {
    const float a = (float)sumi * half_bits_to_float(dw_bits);
    return a * dx;
}

// Pull block j (0..7) of a 144-byte chunk held as 36 dwords: the fp16 scale
// bits and the 16 nibble bytes realigned to dword boundaries. Block j starts
// at byte 18j: an even j at a dword boundary (scale in the low half, nibbles
// two bytes in), an odd j two bytes into a dword (scale in the high half,
// nibbles dword-aligned).
template <int J>
__device__ __forceinline__ void chunk_block(const uint32_t w[CHUNK_DWORDS], uint32_t &d_bits, uint32_t qs[4]) {
    if constexpr ((J & 1) == 0) {
        constexpr int base = (J / 2) * 9;
        d_bits = w[base] & 0xFFFFu;
#pragma unroll
        for (int m = 0; m < 4; ++m) qs[m] = __builtin_amdgcn_alignbyte(w[base + m + 1], w[base + m], 2);
    } else {
        constexpr int base = (J / 2) * 9 + 4;
        d_bits = w[base] >> 16;
#pragma unroll
        for (int m = 0; m < 4; ++m) qs[m] = w[base + 1 + m];
    }
}

// Q8_0 quantization of one 32-element block, q4_0.py:83-97:
// amax = max|x|, d = amax / 127, inv = d == 0 ? 0 : 1 / d (both correctly
// rounded fp32 divisions), q = sign(s) * floor(|s| + 0.5) with s = x * inv.
// The sign goes on before the conversion: |s| + 0.5 is computed (and
// rounded) exactly as the contract writes it, copysign moves s's sign onto
// it, and the conversion truncates toward zero, which is floor for the
// magnitude in both signs. So the result is sign(s) * floor(|s| + 0.5) with
// no compare (-0 and NaN give 0, as the compare-and-negate form does).
__device__ __forceinline__ int8_t q8_round(float x, float inv) {
    const float s = x * inv;
    return (int8_t)(int)copysignf(fabsf(s) + 0.5f, s);
}

__device__ __forceinline__ float q8_scale(float amax) { return amax / 127.0f; }

__device__ __forceinline__ float safe_recip(float d) { return d == 0.0f ? 0.0f : 1.0f / d; }

// Adjacent-pair tree over the eight lanes held by eight consecutive threads
// (lane l in thread l of an aligned group of eight), with DPP moves:
// quad_perm [1,0,3,2] pairs (0,1)(2,3)..., quad_perm [2,3,0,1] pairs the pair
// sums, and row_half_mirror brings the other half of the eight. IEEE addition
// is commutative, so both partners of a pair hold the same bits, and every
// thread of the group ends with ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float tree8_dpp(float lane_sum) {
    float v = lane_sum;
    v = v + dpp_mov<0xB1>(v);     // quad_perm(1,0,3,2)
    v = v + dpp_mov<0x4E>(v);     // quad_perm(2,3,0,1)
    v = v + dpp_mov<0x141>(v);    // row_half_mirror: lane l <- lane 7 - l within eight
    return v;
}

}  // namespace w4a8

// ----------------------------------------------------------------------------
// Producers of the activation, from the reference's decode loop
// (board/tp/tp_llama.cpp): computed exactly as it does, so that the fused
// kernels see the same float32 activation its CPU code would hand the engine.
// Every operation is an IEEE one (fp64 adds, correctly rounded fp32 divide and
// square root, fused multiply-adds where the reference fuses), with
// -ffp-contract=off keeping everything else unfused.
namespace w4a8 {

// ggml's vector float32 exp (tp_llama.cpp:530-553, itself Arm's optimized-
// routines expf, MIT): n = round(x / ln 2) by the 1.5 * 2^23 shift, the
// remainder b = x - n ln 2 in two fused steps, a degree-5 polynomial in b
// evaluated with fused multiply-adds, and 2^n built in the exponent bits, with
// the two scalings that keep |n| > 126 and |n| > 192 in range. Same constants,
// same operation order, same fused steps, one element at a time.
__device__ __forceinline__ float ggml_vec_expf(float x) {
    const float shift = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, shift);
    const float n = z - shift;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = __float_as_uint(z) << 23;
    const float k = __uint_as_float(e + 0x3f800000u);
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u, fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)), u,
                         0x1.ffffecp-1f * b);
    if (!(fabsf(n) > 126.0f)) return fmaf(k, j, k);
    const uint32_t d = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = __uint_as_float(d + 0x7f000000u), s2 = __uint_as_float(e - d);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

// silu(g) * u (silu_mul, tp_llama.cpp:612-619): g / (1 + exp(-g)), then * u.
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sg = g / (1.0f + ggml_vec_expf(-g));
    return sg * u;
}

// rmsnorm's scale (tp_llama.cpp:557-569) from the float64 squares of x
// (exact: a float32 square fits a float64), n % 128 == 0: the sum of squares
// accumulates in float64 in four chains, element i in chain i % 4 in
// increasing i (the reference's fused multiply-add of an exact square is this
// add); the chains meet as (c0 + c2) + (c1 + c3); then
// 1 / sqrtf((float)(ss / n) + eps).
//
// Layout: chain c's squares lie contiguously, square i at rms_sq_index(i, n),
// each chain n / 4 + 2 doubles after the last; rms_sq_doubles(n) doubles in
// all, 16-byte aligned. The squares are written by the whole workgroup
// beforehand, so the chains carry the adds and nothing else.
//
// One wave runs the four chains, chain c in row c (lanes 16c .. 16c + 15):
// lane 16c + i holds chain c's squares 16g + i, g = 0, 1, ..., one 8-byte LDS
// read per lane per sixteen steps, four reads ahead. Each step is one
// v_fmac_f64 whose first operand comes through DPP row_newbcast:i (lane i of
// the row, to every lane of it): acc = sq * 1.0 + acc, the chain's add
// exactly (the product is exact, the fma rounds once). So a step costs one
// dependent float64 instruction (about 5.4 clocks at n = 2048: 2,764 for 512
// steps, where a chain lane reading its own squares from LDS took 4,900-6,300).
// The whole wave must be active. The result is returned in every lane.
__host__ __device__ constexpr size_t rms_sq_doubles(int n) { return (size_t)n + 8; }
__device__ __forceinline__ int rms_sq_index(int i, int n) { return (i & 3) * (n / 4 + 2) + (i >> 2); }

// Sixteen steps of the lane's chain from one read (lane i of the row holds
// step i). The leading s_nop keeps the DPP source clear of a VALU write in
// the two instructions before it, the trailing one keeps acc clear of a
// read right after.
__device__ __forceinline__ double rms_row_steps(double acc, double sq, double one) {
    __asm__(
        "s_nop 1\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f64_dpp %0, %1, %2 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1"
        : "+v"(acc)
        : "v"(sq), "v"(one));
    return acc;
}

template <int N>
__device__ __forceinline__ double rms_chain(const double *sq, int n, int lane) {
    constexpr int AHEAD = 4;                   // reads in flight
    const int len = N ? N : n;
    const int groups = len / 64;               // sixteen steps each
    const double *src = sq + (lane >> 4) * (len / 4 + 2) + (lane & 15);
    const double one = 1.0;
    double acc = 0.0;
    double buf[AHEAD];
#pragma unroll
    for (int t = 0; t < AHEAD; ++t) buf[t] = t < groups ? src[16 * t] : 0.0;
    auto round = [&](int g) {
#pragma unroll
        for (int t = 0; t < AHEAD; ++t) {
            if (g + t < groups) {
                const double v = buf[t];
                if (g + t + AHEAD < groups) buf[t] = src[16 * (g + t + AHEAD)];
                acc = rms_row_steps(acc, v, one);
            }
        }
    };
    if constexpr (N != 0) {
#pragma unroll
        for (int g = 0; g < N / 64; g += AHEAD) round(g);
    } else {
        for (int g = 0; g < groups; g += AHEAD) round(g);
    }
    return acc;
}

__device__ __forceinline__ float rms_scale_wave(const double *sq, int n, float eps) {
    const int lane = threadIdx.x & 63;
    // The hidden size of the decode shapes with its trip count known (the
    // compiler then unrolls the chain); any other n in a loop.
    const double acc = n == 2048 ? rms_chain<2048>(sq, n, lane) : rms_chain<0>(sq, n, lane);
    const double l0 = __shfl(acc, 0), l1 = __shfl(acc, 16), l2 = __shfl(acc, 32), l3 = __shfl(acc, 48);
    const double ss = (l0 + l2) + (l1 + l3);
    return 1.0f / sqrtf((float)(ss / (double)n) + eps);
}

}  // namespace w4a8
