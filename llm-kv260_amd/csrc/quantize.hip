// Quantizer kernels: the fused Q8_0 activation quantizer (the engine caller's
// quantize_x, board/tp/tp_llama.cpp:330-352, with the contract's rounding,
// src/llm_kv260/q4_0.py:83-97) and a Q4_0 weight quantizer
// (src/llm_kv260/q4_0.py:100-121) for building matrices on the device.
//
// Both are element-wise over 32-element blocks. The activation quantizers
// give each block eight threads (one 16-byte load, four values each) and
// meet for the block's max through DPP: a launch of them is latency, and a
// thread that quantized a whole block alone spent ~250 instructions on it.
// The weight quantizer keeps one thread per block (weights are quantized
// once).
#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

namespace {

__device__ __forceinline__ void load_block(const float *src, float v[32]) {
    const float4 *p = reinterpret_cast<const float4 *>(src);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const float4 f = p[m];
        v[4 * m] = f.x; v[4 * m + 1] = f.y; v[4 * m + 2] = f.z; v[4 * m + 3] = f.w;
    }
}

// Q8_0 of one 32-element block (q4_0.py:83-97), stored as block b of row `row`
// of the engine layout (int8[k] | float32[k/32]) or of ggml Q8_0 blocks.
template <int OUT>
__device__ __forceinline__ void quantize_store(const float v[32], int row, int b, int k, uint8_t *__restrict__ out) {
    const int nb = k >> 5;
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
    const float d = q8_scale(amax);
    const float inv = safe_recip(d);
    uint32_t q[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) word |= ((uint32_t)(uint8_t)q8_round(v[4 * w + e], inv)) << (8 * e);
        q[w] = word;
    }
    const uint16_t dh = float_to_half_bits(d);
    if constexpr (OUT == X_ENGINE) {
        uint8_t *rowp = out + (size_t)row * (k + 4 * nb);
        uint4 *dst = reinterpret_cast<uint4 *>(rowp + 32 * b);
        dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
        dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
        reinterpret_cast<float *>(rowp + k)[b] = half_bits_to_float(dh);
    } else {
        uint16_t *dst = reinterpret_cast<uint16_t *>(out + ((size_t)row * nb + b) * Q8_0_BYTES);
        dst[0] = dh;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            dst[1 + 2 * w] = (uint16_t)(q[w] & 0xFFFFu);
            dst[2 + 2 * w] = (uint16_t)(q[w] >> 16);
        }
    }
}

// Q8_0 of values 4g .. 4g + 3 of a 32-element block, thread g (0..7) of an
// aligned group of eight: amax is the group's max (DPP quad_perm [1,0,3,2],
// [2,3,0,1], then row_half_mirror), so every thread computes the same d and
// inv as a thread holding the whole block, and its four bytes are the ones
// quantize_store would write there.
template <int OUT>
__device__ __forceinline__ void quantize_store8(const float4 v, int row, int b, int g, int k, uint8_t *__restrict__ out) {
    const int nb = k >> 5;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, dpp_mov<0xB1>(amax));
    amax = fmaxf(amax, dpp_mov<0x4E>(amax));
    amax = fmaxf(amax, dpp_mov<0x141>(amax));
    const float d = q8_scale(amax);
    const float inv = safe_recip(d);
    const uint32_t word = (uint32_t)(uint8_t)q8_round(v.x, inv) | ((uint32_t)(uint8_t)q8_round(v.y, inv) << 8) |
                          ((uint32_t)(uint8_t)q8_round(v.z, inv) << 16) | ((uint32_t)(uint8_t)q8_round(v.w, inv) << 24);
    const uint16_t dh = float_to_half_bits(d);
    if constexpr (OUT == X_ENGINE) {
        uint8_t *rowp = out + (size_t)row * (k + 4 * nb);
        reinterpret_cast<uint32_t *>(rowp + 32 * b)[g] = word;
        if (g == 0) reinterpret_cast<float *>(rowp + k)[b] = half_bits_to_float(dh);
    } else {
        uint16_t *dst = reinterpret_cast<uint16_t *>(out + ((size_t)row * nb + b) * Q8_0_BYTES);
        if (g == 0) dst[0] = dh;
        dst[1 + 2 * g] = (uint16_t)(word & 0xFFFFu);
        dst[2 + 2 * g] = (uint16_t)(word >> 16);
    }
}

template <int OUT>
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x, int k, int m,
                                                            uint8_t *__restrict__ out) {
    const int nb = k >> 5;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)nb * m * 8) return;           // whole groups of eight leave together
    const long blk = gid >> 3;
    const int g = (int)(gid & 7);
    const int row = (int)(blk / nb), b = (int)(blk - (long)row * nb);
    const float4 v = reinterpret_cast<const float4 *>(x + (size_t)row * k + 32 * b)[g];
    quantize_store8<OUT>(v, row, b, g, k, out);
}

// act = silu(gate) * up (tp_llama.cpp:612-619) of m rows gate | up
// (float32[2k] each, the gate|up GEMV's output), quantized to the engine layout.
__global__ __launch_bounds__(256) void silu_mul_q8_0_kernel(const float *__restrict__ gate_up, int k, int m,
                                                            uint8_t *__restrict__ out) {
    const int nb = k >> 5;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)nb * m * 8) return;           // whole groups of eight leave together
    const long blk = gid >> 3;
    const int t = (int)(gid & 7);
    const int row = (int)(blk / nb), b = (int)(blk - (long)row * nb);
    const float *src = gate_up + (size_t)row * 2 * k + 32 * b;
    const float4 g = reinterpret_cast<const float4 *>(src)[t];
    const float4 u = reinterpret_cast<const float4 *>(src + k)[t];
    const float4 v = make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
    quantize_store8<X_ENGINE>(v, row, b, t, k, out);
}

// h = rmsnorm(x) * norm_w (tp_llama.cpp:557-569) of m rows of float32[k],
// quantized to the engine layout: one workgroup per row (the sum of squares
// runs over the whole row); the squares in LDS as float64 for wave 0's four
// chains, x read again (from L2) for the normalization.
__global__ __launch_bounds__(256) void rmsnorm_q8_0_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                           float eps, int k, uint8_t *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) double sq[];
    __shared__ float scale;
    const int row = blockIdx.x, nb = k >> 5;
    const float *xr = x + (size_t)row * k;
    const int cs = k / 4 + 2;     // chain stride (rms_sq_index)
    for (int i = threadIdx.x; i < k / 4; i += blockDim.x) {
        const float4 v = reinterpret_cast<const float4 *>(xr)[i];
        const double a = v.x, b = v.y, c = v.z, d = v.w;
        sq[i] = a * a;
        sq[cs + i] = b * b;
        sq[2 * cs + i] = c * c;
        sq[3 * cs + i] = d * d;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const float sc = rms_scale_wave(sq, k, eps);
        if (threadIdx.x == 0) scale = sc;
    }
    __syncthreads();
    const float sc = scale;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        float xv[32], wv[32], v[32];
        load_block(xr + 32 * b, xv);
        load_block(w + 32 * b, wv);
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float a = xv[e] * sc;
            v[e] = a * wv[e];
        }
        quantize_store<X_ENGINE>(v, row, b, k, out);
    }
}

__global__ __launch_bounds__(256) void quantize_q4_0_kernel(const float *__restrict__ w, int rows, int k,
                                                            uint8_t *__restrict__ out) {
    const int nb = k >> 5;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)nb * rows) return;
    float v[32];
    load_block(w + gid * 32, v);   // rows are contiguous: block gid starts at float 32 * gid
    // The signed element of largest magnitude, first index on ties.
    float extreme = v[0], amax = fabsf(v[0]);
#pragma unroll
    for (int e = 1; e < 32; ++e) {
        const float a = fabsf(v[e]);
        if (a > amax) { amax = a; extreme = v[e]; }
    }
    const float d = extreme / -8.0f;
    const float inv = safe_recip(d);
    uint32_t nib[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const float s = v[e] * inv;
        const float u = s + 8.5f;
        const int n = (int)truncf(u);   // u >= 0.5 for every finite block; clamp keeps nibbles 4-bit
        nib[e] = (uint32_t)(n > 15 ? 15 : (n < 0 ? 0 : n));
    }
    uint16_t *dst = reinterpret_cast<uint16_t *>(out + gid * Q4_0_BYTES);
    dst[0] = float_to_half_bits(d);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t b0 = nib[2 * j] | (nib[2 * j + 16] << 4);
        const uint32_t b1 = nib[2 * j + 1] | (nib[2 * j + 17] << 4);
        dst[1 + j] = (uint16_t)(b0 | (b1 << 8));
    }
}

}  // namespace

hipError_t launch_quantize_q8_0(const float *x, int k, int m, uint8_t *out, XFormat out_fmt, hipStream_t stream) {
    const long blocks = (long)(k / 32) * m;
    if (blocks == 0) return hipSuccess;
    const long grid = (8 * blocks + 255) / 256;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    if (out_fmt == X_ENGINE)
        hipLaunchKernelGGL(quantize_q8_0_kernel<X_ENGINE>, dim3((unsigned)grid), dim3(256), 0, stream, x, k, m, out);
    else if (out_fmt == X_Q8_0)
        hipLaunchKernelGGL(quantize_q8_0_kernel<X_Q8_0>, dim3((unsigned)grid), dim3(256), 0, stream, x, k, m, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_silu_mul_q8_0(const float *gate_up, int k, int m, uint8_t *out, hipStream_t stream) {
    const long blocks = (long)(k / 32) * m;
    if (blocks == 0) return hipSuccess;
    const long grid = (8 * blocks + 255) / 256;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(silu_mul_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, stream, gate_up, k, m, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_q8_0(const float *x, const float *w, float eps, int k, int m, uint8_t *out,
                               hipStream_t stream) {
    if (m <= 0) return hipSuccess;
    const size_t lds = rms_sq_doubles(k) * 8;               // float64 squares: 128 KB at k = 16384
    const hipError_t e = allow_dynamic_lds(reinterpret_cast<const void *>(&rmsnorm_q8_0_kernel), 160 * 1024);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(rmsnorm_q8_0_kernel, dim3((unsigned)m), dim3(256), lds, stream, x, w, eps, k, out);
    return hipGetLastError();
}

hipError_t launch_quantize_q4_0(const float *w, int rows, int k, uint8_t *out, hipStream_t stream) {
    const long blocks = (long)(k / 32) * rows;
    if (blocks == 0) return hipSuccess;
    const long grid = (blocks + 255) / 256;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize_q4_0_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, rows, k, out);
    return hipGetLastError();
}

}  // namespace w4a8
