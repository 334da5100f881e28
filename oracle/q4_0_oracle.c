/*
 * CPU oracle (scalar C) for the W4A8 Q4_0 x Q8_0 GEMV contract.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, to compare the library against. The product library never links
 * it.
 *
 * A second, independent restatement of src/llm_kv260/q4_0.py (the first is
 * q4_0_oracle.py); the tests require the two to agree byte for byte, and both
 * to reproduce the reference-held golden SHA-256 of
 * tests/test_q4_0_contract.py:181-191. Built with -ffp-contract=off and no
 * fast-math so every fp32 operation is one IEEE round-to-nearest-even op, as
 * in NumPy.
 *
 * Rows are independent, so the GEMV is parallelised over rows with OpenMP
 * without changing a single bit of any output.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define Q4_0_BYTES 18
#define LANES 8

/* ------------------------------------------------------------------ fp16 */

/* Exact widening: every binary16 value is a binary32 value.
 * Follows the intent of half_to_float, hls/int4_core/gemv_core.h:51-81. */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, m = h & 1023u, bits;
    if (e == 31u) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0u) {
        bits = sign;
    } else {
        /* subnormal: m * 2^-24, renormalise so the leading one is implicit */
        int shift = 0;
        while (!(m & 1024u)) { m <<= 1; ++shift; }
        bits = sign | ((uint32_t)(113 - shift) << 23) | ((m & 1023u) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even narrowing (NumPy's astype(float16)). Written from the
 * IEEE 754 definition: keep 11 significant bits (fewer for subnormals), round
 * the discarded tail half-to-even, overflow to infinity. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t e = (x >> 23) & 255u, m = x & 0x7fffffu;
    if (e == 255u) {                                   /* inf or nan */
        if (m == 0u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)(m >> 13);   /* nan stays nan (quiet bit set) */
    }
    int exp = (int)e - 127;                             /* unbiased */
    if (e == 0u) return sign;                           /* f32 subnormals are < 2^-126: to 0 */
    uint32_t sig = m | 0x800000u;                       /* 24-bit significand, value sig*2^(exp-23) */
    int hexp = exp + 15;                                /* biased half exponent if normal */
    int drop;                                           /* bits of sig to discard */
    if (hexp >= 1) drop = 13;                           /* normal half: keep 11 bits */
    else drop = 13 + (1 - hexp);                        /* subnormal half: fewer bits */
    if (drop > 25) return sign;                         /* below half the smallest subnormal */
    uint32_t keep = sig >> drop;
    uint32_t rem = sig & ((1u << drop) - 1u);
    uint32_t half = 1u << (drop - 1);
    if (rem > half || (rem == half && (keep & 1u))) keep += 1u;
    if (hexp >= 1) {
        /* keep is 11 bits (1.xxx) or 12 after a carry */
        uint32_t he = (uint32_t)hexp;
        if (keep & 0x800u) { keep >>= 1; he += 1u; }
        if (he >= 31u) return sign | 0x7c00u;
        return sign | (uint16_t)(he << 10) | (uint16_t)(keep & 1023u);
    }
    /* subnormal result; a carry into bit 10 yields the smallest normal, which
     * the same encoding expresses */
    return sign | (uint16_t)keep;
}

/* ------------------------------------------------------------- quantizers */

/* Q8_0, src/llm_kv260/q4_0.py:83-97. q: int8[k]; d: fp16 bits [k/32]. */
void oracle_quantize_q8_0(const float *x, int8_t *q, uint16_t *d, int64_t k) {
    for (int64_t b = 0; b < k / QK; ++b) {
        const float *xb = x + b * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float db = amax / 127.0f;
        float inv = db == 0.0f ? 0.0f : 1.0f / db;
        for (int j = 0; j < QK; ++j) {
            float s = xb[j] * inv;
            float mag = floorf(fabsf(s) + 0.5f);
            q[b * QK + j] = (int8_t)(int)(s < 0.0f ? -mag : mag);
        }
        d[b] = oracle_f32_to_f16(db);
    }
}

/* Q4_0, src/llm_kv260/q4_0.py:100-121. blocks: uint8[rows][k/32*18]. */
void oracle_quantize_q4_0(const float *w, uint8_t *blocks, int64_t rows, int64_t k, int threads) {
    const int64_t nb = k / QK;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const float *wb = w + r * k + b * QK;
            uint8_t *out = blocks + (r * nb + b) * Q4_0_BYTES;
            /* first index of the largest magnitude, as argmax picks it */
            float extreme = wb[0], amax = fabsf(wb[0]);
            for (int j = 1; j < QK; ++j) {
                float a = fabsf(wb[j]);
                if (a > amax) { amax = a; extreme = wb[j]; }
            }
            float db = extreme / -8.0f;
            float inv = db == 0.0f ? 0.0f : 1.0f / db;
            uint8_t nib[QK];
            for (int j = 0; j < QK; ++j) {
                float v = wb[j] * inv;
                v = v + 8.5f;
                int n = (int)truncf(v);
                nib[j] = (uint8_t)(n > 15 ? 15 : n);
            }
            uint16_t h = oracle_f32_to_f16(db);
            out[0] = (uint8_t)(h & 255u);
            out[1] = (uint8_t)(h >> 8);
            for (int j = 0; j < 16; ++j) out[2 + j] = (uint8_t)(nib[j] | (nib[j + 16] << 4));
        }
    }
}

/* ------------------------------------------------------------------- gemv */

static float tree8(const float *l) {
    return ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
}

/* One row, the contract's order (q4_0.py:151-182): exact int32 block dot,
 * t = (f32(sumi) * dw) * dx, lane b % 8 accumulates in increasing b from +0,
 * then the adjacent-pair tree. xd is already widened to fp32. */
static float row_dot(const uint8_t *row, const int8_t *xq, const float *xd, int64_t nb) {
    float lanes[LANES] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t *blk = row + b * Q4_0_BYTES;
        const int8_t *xb = xq + b * QK;
        int32_t sumi = 0;
        for (int j = 0; j < 16; ++j) {
            int lo = (blk[2 + j] & 15) - 8, hi = (blk[2 + j] >> 4) - 8;
            sumi += lo * xb[j] + hi * xb[j + 16];
        }
        float dw = oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        float t = (float)sumi * dw;
        t = t * xd[b];
        lanes[b % LANES] = lanes[b % LANES] + t;
    }
    return tree8(lanes);
}

/* y[rows] = W x with x as (int8[k], fp16 bits [k/32]). */
void oracle_gemv_q4_0(const uint8_t *blocks, const int8_t *xq, const uint16_t *xd16, float *y,
                      int64_t rows, int64_t k, int threads) {
    const int64_t nb = k / QK;
    float *xd = (float *)malloc((size_t)nb * sizeof(float));
    if (!xd) abort();
    for (int64_t b = 0; b < nb; ++b) xd[b] = oracle_f16_to_f32(xd16[b]);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) y[r] = row_dot(blocks + r * nb * Q4_0_BYTES, xq, xd, nb);
    free(xd);
}

/* y[m][rows] for m activation rows; each row is the contract applied alone. */
void oracle_gemm_q4_0(const uint8_t *blocks, const int8_t *xq, const uint16_t *xd16, float *y,
                      int64_t m, int64_t rows, int64_t k, int threads) {
    for (int64_t i = 0; i < m; ++i)
        oracle_gemv_q4_0(blocks, xq + i * k, xd16 + i * (k / QK), y + i * rows, rows, k, threads);
}

/* Engine activation layout int8[k] then f32[k/32] (q4_0.py:193-200). */
void oracle_pack_x_for_engine(const int8_t *xq, const uint16_t *xd16, uint8_t *out, int64_t k) {
    memcpy(out, xq, (size_t)k);
    for (int64_t b = 0; b < k / QK; ++b) {
        float f = oracle_f16_to_f32(xd16[b]);
        memcpy(out + k + 4 * b, &f, 4);
    }
}

/* ----------------------------------------------- producers of the activation
 *
 * The reference's decode loop computes the GEMV inputs with these
 * (board/tp/tp_llama.cpp); restated in scalar C, one element at a time, in the
 * same operation order and with the same fused steps. */

/* rmsnorm, tp_llama.cpp:557-569: the sum of squares in float64 in four lanes
 * (element i in lane i % 4, increasing i; float products are exact in
 * float64, so the NEON fused multiply-add is the add), met as
 * (l0 + l2) + (l1 + l3); scale = 1 / sqrtf((float)(ss / n) + eps); out =
 * (x * scale) * w. n % 4 == 0. */
void oracle_rmsnorm(const float *x, const float *w, int64_t n, float eps, float *out) {
    double lane[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t i = 0; i < n; ++i) {
        const double v = (double)x[i];
        lane[i & 3] = lane[i & 3] + v * v;
    }
    const double ss = (lane[0] + lane[2]) + (lane[1] + lane[3]);
    const float scale = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (int64_t i = 0; i < n; ++i) {
        const float a = x[i] * scale;
        out[i] = a * w[i];
    }
}

/* ggml's vector expf (tp_llama.cpp:530-553; Arm optimized-routines, MIT) for
 * one element: the same constants, order and fused steps (fmaf = the NEON
 * vfma / vfms). */
float oracle_ggml_expf(float x) {
    const float shift = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, shift);
    const float n = z - shift;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    uint32_t zb;
    memcpy(&zb, &z, 4);
    const uint32_t e = zb << 23;
    const uint32_t kb = e + 0x3f800000u;
    float k;
    memcpy(&k, &kb, 4);
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u, fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                         u, 0x1.ffffecp-1f * b);
    if (!(fabsf(n) > 126.0f)) return fmaf(k, j, k);
    const uint32_t d = n <= 0.0f ? 0x82000000u : 0u;
    const uint32_t s1b = d + 0x7f000000u, s2b = e - d;
    float s1, s2;
    memcpy(&s1, &s1b, 4);
    memcpy(&s2, &s2b, 4);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

/* silu_mul, tp_llama.cpp:612-619: a = (g / (1 + exp(-g))) * u. */
void oracle_silu_mul(const float *g, const float *u, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i) {
        const float sg = g[i] / (1.0f + oracle_ggml_expf(-g[i]));
        out[i] = sg * u[i];
    }
}

/* The sampler's per-shard candidates, tp_llama.cpp:894-909, restated: k
 * slots start as {-1e30, 0}; each y[i] in increasing i is skipped when
 * y[i] <= the last slot's value, else inserted after every held value that is
 * not less than it (the shift loop stops at an equal value), the last slot
 * falling out. The reference's loop exactly, NaN included. */
void oracle_topk(const float *y, int64_t n, int k, float *vals, int32_t *idx) {
    for (int j = 0; j < k; ++j) {
        vals[j] = -1e30f;
        idx[j] = 0;
    }
    for (int64_t i = 0; i < n; ++i) {
        const float v = y[i];
        if (v <= vals[k - 1]) continue;
        int pos = k - 1;
        while (pos > 0 && vals[pos - 1] < v) {
            vals[pos] = vals[pos - 1];
            idx[pos] = idx[pos - 1];
            --pos;
        }
        vals[pos] = v;
        idx[pos] = (int32_t)i;
    }
}

const char *oracle_contract_version(void) { return "llm-kv260/w4a8-q4_0-v2"; }
