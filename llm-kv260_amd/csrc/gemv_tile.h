// Device pieces shared by the M = 1 kernels (gemv_m1.hip, chain.hip): raw
// buffer access, the activation formats and their LDS staging, the terms of
// one chunk, and the contract's ordered lane sums.
#pragma once

#include "kernels.h"
#include "q4_0_device.h"

namespace w4a8 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer accesses: the buffer unit range-checks every lane against the
// resource's size, so a lane whose offset is out of range touches no memory
// (a load returns zeros, a store is dropped). Loads and stores are then
// issued by every lane on every path -- the number of memory operations a
// wave has in flight never depends on data, and each wait is exact -- while
// the lanes with nothing to do cost no traffic.
constexpr int OUT_OF_RANGE = 0x7ffffff0;
constexpr uint32_t BUFFER_DWORD3 = 0x00020000;   // raw dword access on gfx9-family parts
constexpr int CACHE_NT = 2;                       // non-temporal (streamed once)
constexpr int SC1 = 16;                           // device-scope coherent access (sc1)

// n / d for 0 <= n < 64 and 1 <= d <= 64 (a lane's row in its tile) as
// floor((n + 0.5) * rcp(d)), four VALU operations in place of the division
// sequence the compiler emits for a run-time divisor. Exact: n + 0.5 lies at
// least 0.5 from a multiple of d, a margin of 0.5 / 64 in the quotient, far
// above v_rcp_f32's one-ulp error (checked for every n, d and rcp result
// within one ulp).
__device__ __forceinline__ int lane_quot(int n, int d) {
    return (int)(((float)n + 0.5f) * __builtin_amdgcn_rcpf((float)d));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, BUFFER_DWORD3);
}

// Raw activation block as the global loads deliver it, before staging.
template <int XF>
struct XRaw;
template <>
struct XRaw<X_ENGINE> {
    u32x4 q0, q1;
    float d;
};
template <>
struct XRaw<X_Q8_0> {
    uint16_t h[17];
};
template <>
struct XRaw<X_F32> {
    float4 v[8];
};
template <>
struct XRaw<X_RMS> {
    float4 v[8];   // x
    float4 w[8];   // norm weight
};
template <>
struct XRaw<X_SILU> {
    float4 g[8];   // gate
    float4 u[8];   // up
};

template <int AUX = 0>
__device__ __forceinline__ void load_f32_block(__amdgpu_buffer_rsrc_t rb, int off, float4 v[8]) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rb, off == OUT_OF_RANGE ? OUT_OF_RANGE : off + 16 * m, 0, AUX);
        v[m] = make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
    }
}

// An fp32 x read by whole lines: wave w takes blocks 64 w .. 64 w + 63, and
// its instruction m gives lane l the 16 bytes at 8192 w + 1024 m + 16 l
// (block 64 w + 8 m + l / 8, piece l % 8), so that every instruction reads 1
// KB of consecutive bytes. Loaded one block per lane (128 bytes apart), each
// instruction touched 64 lines and the memory pipeline took about 64 clocks
// for it, so that a wave's weight loads queued behind its activation's.
// Bytes past x read zeros.
struct XLines {
    u32x4 v[8];
};

template <int AUX = 0>
__device__ __forceinline__ void x_load_lines(const void *x, int k, int wave, int lane, XLines &r) {
    const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)(4 * k));
    const int base = 8192 * wave + 16 * lane;
#pragma unroll
    for (int m = 0; m < 8; ++m) r.v[m] = __builtin_amdgcn_raw_buffer_load_b128(xb, base + 1024 * m, 0, AUX);
}

// The lines regrouped one block per lane through `tmp`, 9,216 bytes of LDS
// that only this wave uses (144 bytes per block: both the writes and the
// reads spread over the banks): lane l then holds block 64 w + l as x_load
// delivers it.
__device__ __forceinline__ void x_lines_to_block(const XLines &r, int lane, uint8_t *tmp, XRaw<X_F32> &out) {
#pragma unroll
    for (int m = 0; m < 8; ++m)
        *reinterpret_cast<u32x4 *>(tmp + 144 * (8 * m + (lane >> 3)) + 16 * (lane & 7)) = r.v[m];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const u32x4 t = *reinterpret_cast<const u32x4 *>(tmp + 144 * lane + 16 * j);
        out.v[j] = make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
    }
}

// Block b of the activation; a lane with live == false reads nothing. AUX:
// the cache policy of the fp32 x's loads (SC1: from the device's coherence
// point, for an x that an earlier dispatch with no fence after it wrote).
template <int XF, int AUX = 0>
__device__ __forceinline__ void x_load(const void *x, int k, int b, bool live, XRaw<XF> &r,
                                       const float *norm_w = nullptr) {
    if constexpr (XF == X_RMS) {
        load_f32_block<AUX>(buffer_of(x, (uint32_t)(4 * k)), live ? 128 * b : OUT_OF_RANGE, r.v);
        load_f32_block(buffer_of(norm_w, (uint32_t)(4 * k)), live ? 128 * b : OUT_OF_RANGE, r.w);
    } else if constexpr (XF == X_SILU) {
        const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)(8 * k));
        load_f32_block(xb, live ? 128 * b : OUT_OF_RANGE, r.g);
        load_f32_block(xb, live ? 4 * k + 128 * b : OUT_OF_RANGE, r.u);
    } else if constexpr (XF == X_ENGINE) {
        const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)(k + k / 8));
        const int q_off = live ? 32 * b : OUT_OF_RANGE, d_off = live ? k + 4 * b : OUT_OF_RANGE;
        r.q0 = __builtin_amdgcn_raw_buffer_load_b128(xb, q_off, 0, AUX);
        r.q1 = __builtin_amdgcn_raw_buffer_load_b128(xb, q_off + 16, 0, AUX);
        r.d = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xb, d_off, 0, AUX));
    } else if constexpr (XF == X_Q8_0) {
        const uint16_t *src = reinterpret_cast<const uint16_t *>(static_cast<const uint8_t *>(x) +
                                                                 Q8_0_BYTES * (live ? b : 0));
#pragma unroll
        for (int i = 0; i < 17; ++i) r.h[i] = src[i];
    } else {
        const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)(4 * k));
        const int off = live ? 128 * b : OUT_OF_RANGE;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xb, off + 16 * m, 0, AUX);
            r.v[m] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
        }
    }
}

// The staged activation in LDS, one column per eight blocks (a chunk's
// width): 64 dwords of activation nibbles (x_nibbles of block j of the column
// at dword 8 j), the eight fp32 scales, the eight int32 corrections
// -8 * sum(x), then 4 dwords of padding, 84 dwords in all. Lane l of a wave reads column l % C, so the lanes of one
// LDS pass read eight different columns: at a stride of 84 dwords their
// 16-byte reads fall on distinct banks, where a stride of 64 sent all of them
// to the same ones (8-way conflicts at K = 2048, 32-way at K = 8192).
constexpr int XCOL_DWORDS = 84;
constexpr int XCOL_D = 64;     // the scales' offset in a column
constexpr int XCOL_S = 72;     // the corrections'
__host__ __device__ constexpr size_t x_lds_bytes(int nb) { return (size_t)(nb / 8) * XCOL_DWORDS * 4; }

// A quarter of an fp32 block for the rmsnorm staging spread over four
// threads: thread q of block b holds its elements 4q .. 4q + 3 (a) and
// 16 + 4q .. 16 + 4q + 3 (b), exactly the int8 values of dwords q and 4 + q
// of the staged block, which x_nibbles pairs into nibble dwords q and 4 + q.
struct XQuarter {
    float4 xa, xb, wa, wb;
};

template <int AUX = 0>
__device__ __forceinline__ void x_load_quarter(const void *x, const float *norm_w, int k, int b, int q, bool live,
                                               XQuarter &r) {
    const __amdgpu_buffer_rsrc_t xr = buffer_of(x, (uint32_t)(4 * k));
    const __amdgpu_buffer_rsrc_t wr = buffer_of(norm_w, (uint32_t)(4 * k));
    const int off = live ? 128 * b + 16 * q : OUT_OF_RANGE;
    const int off2 = live ? off + 64 : OUT_OF_RANGE;
    auto f4 = [](u32x4 t) { return make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w)); };
    r.xa = f4(__builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, AUX));
    r.xb = f4(__builtin_amdgcn_raw_buffer_load_b128(xr, off2, 0, AUX));
    r.wa = f4(__builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
    r.wb = f4(__builtin_amdgcn_raw_buffer_load_b128(wr, off2, 0, 0));
}

// The rmsnorm block's staging by its four threads (lanes 4b' .. 4b' + 3 of a
// wave, an aligned quad): out = (x * scale) * w for their eight elements, the
// block's amax met over the quad by DPP, the contract's Q8_0 rounding of each
// element, and -8 * sum(x) summed over the quad; each thread stores its two
// nibble dwords, thread 0 the scale and the correction. The same bytes as
// x_stage<X_RMS> on the whole block in one thread.
__device__ __forceinline__ void x_stage_quarter(const XQuarter &r, int b, int q, uint32_t *s_x, float rms_scale) {
    const float xv[8] = {r.xa.x, r.xa.y, r.xa.z, r.xa.w, r.xb.x, r.xb.y, r.xb.z, r.xb.w};
    const float wv[8] = {r.wa.x, r.wa.y, r.wa.z, r.wa.w, r.wb.x, r.wb.y, r.wb.z, r.wb.w};
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float a = xv[e] * rms_scale;
        v[e] = a * wv[e];
        amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = fmaxf(amax, dpp_mov<0xB1>(amax));   // quad_perm(1,0,3,2)
    amax = fmaxf(amax, dpp_mov<0x4E>(amax));   // quad_perm(2,3,0,1)
    const float d = q8_scale(amax);
    const float inv = safe_recip(d);
    uint32_t wlo = 0, whi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        wlo |= ((uint32_t)(uint8_t)q8_round(v[e], inv)) << (8 * e);
        whi |= ((uint32_t)(uint8_t)q8_round(v[4 + e], inv)) << (8 * e);
    }
    int32_t sum = __builtin_amdgcn_sdot4((int)wlo, 0x01010101, 0, false);
    sum = __builtin_amdgcn_sdot4((int)whi, 0x01010101, sum, false);
    sum += __builtin_amdgcn_mov_dpp(sum, 0xB1, 0xF, 0xF, false);
    sum += __builtin_amdgcn_mov_dpp(sum, 0x4E, 0xF, 0xF, false);
    const uint32_t lo = wlo ^ 0x80808080u, hi = whi ^ 0x80808080u;   // x + 128, bytewise (x_nibbles)
    uint32_t *col = s_x + (b >> 3) * XCOL_DWORDS;
    const int j = b & 7;
    col[8 * j + q] = ((lo >> 4) & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u);
    col[8 * j + 4 + q] = (lo & 0x0F0F0F0Fu) | ((hi << 4) & 0xF0F0F0F0u);
    if (q == 0) {
        col[XCOL_D + j] = __float_as_uint(half_bits_to_float(float_to_half_bits(d)));
        col[XCOL_S + j] = (uint32_t)(-8 * sum);
    }
}

// Quantize (if fp32) and store block b into LDS: its values as nibbles (RAW:
// as the int8 values themselves, for block_dot_raw), its fp32 scale, and -8
// times the sum of its int8 values.
template <int XF, bool RAW = false>
__device__ __forceinline__ void x_stage(const XRaw<XF> &r, int b, uint32_t *s_x, float rms_scale = 0.0f) {
    uint32_t q[8];
    float dx;
    if constexpr (XF == X_ENGINE) {
        q[0] = r.q0.x; q[1] = r.q0.y; q[2] = r.q0.z; q[3] = r.q0.w;
        q[4] = r.q1.x; q[5] = r.q1.y; q[6] = r.q1.z; q[7] = r.q1.w;
        dx = r.d;
    } else if constexpr (XF == X_Q8_0) {
        dx = half_bits_to_float(r.h[0]);
#pragma unroll
        for (int m = 0; m < 8; ++m) q[m] = (uint32_t)r.h[1 + 2 * m] | ((uint32_t)r.h[2 + 2 * m] << 16);
    } else {
        float v[32];
        if constexpr (XF == X_F32) {
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                v[4 * m] = r.v[m].x; v[4 * m + 1] = r.v[m].y; v[4 * m + 2] = r.v[m].z; v[4 * m + 3] = r.v[m].w;
            }
        } else if constexpr (XF == X_RMS) {
            // out = (x * scale) * w, rmsnorm's last step (tp_llama.cpp:568).
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const float xv[4] = {r.v[m].x, r.v[m].y, r.v[m].z, r.v[m].w};
                const float wv[4] = {r.w[m].x, r.w[m].y, r.w[m].z, r.w[m].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = xv[e] * rms_scale;
                    v[4 * m + e] = a * wv[e];
                }
            }
        } else {
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const float gv[4] = {r.g[m].x, r.g[m].y, r.g[m].z, r.g[m].w};
                const float uv[4] = {r.u[m].x, r.u[m].y, r.u[m].z, r.u[m].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * m + e] = silu_mul(gv[e], uv[e]);
            }
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
    uint32_t xn[8];
    if constexpr (RAW) {
#pragma unroll
        for (int m = 0; m < 8; ++m) xn[m] = q[m];
    } else {
        x_nibbles(q, xn);
    }
    uint32_t *col = s_x + (b >> 3) * XCOL_DWORDS;
    const int j = b & 7;
    u32x4 *dst = reinterpret_cast<u32x4 *>(col + 8 * j);
    dst[0] = (u32x4){xn[0], xn[1], xn[2], xn[3]};
    dst[1] = (u32x4){xn[4], xn[5], xn[6], xn[7]};
    col[XCOL_D + j] = __float_as_uint(dx);
    col[XCOL_S + j] = (uint32_t)(-8 * sum);
}

// The eight terms of one chunk.
__device__ __forceinline__ void chunk_terms(const uint32_t w[CHUNK_DWORDS], const uint32_t xv[8][8], const float xd[8],
                                            const int32_t xs[8], float t[8]) {
#define W4A8_TERM(J)                                                             \
    {                                                                            \
        uint32_t d_bits, qs[4];                                                  \
        chunk_block<J>(w, d_bits, qs);                                           \
        const int32_t sumi = block_dot_nib(qs, xv[J], xs[J]);                    \
        t[J] = block_term(sumi, d_bits, xd[J]);                                  \
    }
    W4A8_TERM(0) W4A8_TERM(1) W4A8_TERM(2) W4A8_TERM(3)
    W4A8_TERM(4) W4A8_TERM(5) W4A8_TERM(6) W4A8_TERM(7)
#undef W4A8_TERM
}

constexpr int TILE_BYTES = 64 * CHUNK_BYTES;   // 9,216
__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Raw buffer store of one fp32 to y[row]; a lane whose offset is past the end
// of y stores nothing (the buffer unit drops out-of-range writes). Every lane
// issues the instruction, so the number of memory operations a wave has in
// flight never depends on data, and the waits for the prefetched tiles stay
// exact.
template <int AUX = 0>
__device__ __forceinline__ void store_y(__amdgpu_buffer_rsrc_t y, int byte_off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), y, byte_off, 0, AUX);
}


// Accumulator a of row r of a tile whose terms sit in s_t at a stride of
// nine floats per lane (lane l, term j at 9 l + j): term a of chunks
// 0 .. C-1 of the row, in order, from +0.0f (src/llm_kv260/q4_0.py:178-179).
// Rows at or past rpw give +0.0f. The reads go eight at a time; a column past
// C contributes +0.0f, which leaves the sum unchanged (it started at +0.0f,
// so it is never -0.0f, and x + 0 = x for every other x).
__device__ __forceinline__ float ordered_lane_sum(const float *s_t, int r, int rpw, int C, int acc_a) {
    float acc = 0.0f;
    if (r < rpw) {
        const float *src = s_t + r * C * 9 + acc_a;
        if ((C & 7) == 0) {
            // Whole groups of eight (K a multiple of 2048): no guards,
            // and each group's reads go out before the previous
            // group's adds. The adds keep the chunk order.
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = src[9 * j];
            for (int c0 = 8; c0 < C; c0 += 8) {
                float nv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) nv[j] = src[9 * (c0 + j)];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = acc + v[j];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = nv[j];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = acc + v[j];
        } else {
            for (int c0 = 0; c0 < C; c0 += 8) {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = c0 + j < C ? src[9 * (c0 + j)] : 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = acc + v[j];
            }
        }
    }
    return acc;
}

// The same with the row's chunks at positions start + cstride c of the
// slab (a v2 tile's rows: their chunks alternate with the paired row's).
__device__ __forceinline__ float ordered_lane_sum_at(const float *s_t, int start, int cstride, bool live, int C,
                                                     int acc_a) {
    float acc = 0.0f;
    if (live) {
        const float *src = s_t + start * 9 + acc_a;
        const int step = 9 * cstride;
        for (int c0 = 0; c0 < C; c0 += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = c0 + j < C ? src[step * (c0 + j)] : 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = acc + v[j];
        }
    }
    return acc;
}

}  // namespace w4a8
