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
// dwords) with the block's 32 int8 activations (eight dwords). Byte j of the
// block carries weight j in its low nibble and weight j + 16 in its high one
// (q4_0.py:22-24). Nibbles 0..15 are non-negative int8 values, so v_dot4
// gives sum(n * x) exactly and the -8 offset comes back as -8 * sum(x).
__device__ __forceinline__ int32_t block_dot_raw(const uint32_t qs[4], const uint32_t xv[8]) {
    int32_t acc = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t lo = qs[m] & 0x0F0F0F0Fu;
        const uint32_t hi = (qs[m] >> 4) & 0x0F0F0F0Fu;
        acc = __builtin_amdgcn_sdot4((int)lo, (int)xv[m], acc, false);
        acc = __builtin_amdgcn_sdot4((int)hi, (int)xv[4 + m], acc, false);
    }
    return acc;
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
__device__ __forceinline__ int8_t q8_round(float x, float inv) {
    const float s = x * inv;
    const float mag = floorf(fabsf(s) + 0.5f);
    return (int8_t)(int)(s < 0.0f ? -mag : mag);
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
