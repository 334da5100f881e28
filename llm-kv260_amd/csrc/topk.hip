// Top-k candidates of the LM head's logits: the per-shard selection of the
// reference's sampler (board/tp/tp_llama.cpp:894-909), whose insertion sort
// keeps the k largest y[i] in descending order, an equal value after the
// ones already held (so the smaller index first), and never admits a value
// at or below its initial sentinel -1e30 (slots it never fills stay
// {-1e30, 0}). On one GPU the shard is the whole vocabulary.
//
// Each logit becomes a 64-bit key: the float's order-preserving bits (with
// -0 taken as +0, which the reference's comparisons treat as equal) above
// the complemented index, so that the largest key is the largest value and,
// among equal values, the smallest index. A value that the reference would
// never admit (v <= -1e30, and NaN, which this version excludes as well)
// gets key 0. The k largest keys are then exactly the reference's k
// candidates, in its order, for every input without NaN.
//
// Stage 1: one 256-thread workgroup per 1024 logits. Each wave holds 256
// keys, four per lane as four lists of 64 (one key per lane each), sorts the
// four across its lanes (bitonic, register compare-exchanges with the lane
// `stride` apart), and merges them two by two; the four waves' best 64 then
// merge through LDS, and the workgroup writes its 64 best. Stage 2: one
// workgroup merges those lists pairwise, level by level. A merge of two
// descending lists A and B keeps, in lane l, max(A[l], B[63 - l]): a bitonic
// sequence holding their 64 best, which six compare-exchange steps sort.
#include "kernels.h"

namespace w4a8 {

namespace {

constexpr int TOPK_SLICE = 1024;      // logits per stage-1 workgroup
constexpr int TOPK_LIST = 64;         // candidates each list keeps (k <= 64)
constexpr int TOPK_MAX_LISTS = 256;   // stage 2's LDS: 256 x 64 keys = 128 KB
static_assert(TOPK_LIST == 64, "the index arithmetic below takes lists of 64");

__device__ __forceinline__ unsigned long long topk_key(float v, int i) {
    if (!(v > -1e30f)) return 0ull;                                  // never admitted (and NaN)
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }
__device__ __forceinline__ unsigned long long min_u64(unsigned long long a, unsigned long long b) { return a < b ? a : b; }

// One compare-exchange step of a bitonic network over the wave's 64 lanes:
// the pair (l, l ^ stride) ends ordered descending when `desc`, with the
// larger key in the lower lane.
__device__ __forceinline__ unsigned long long cx(unsigned long long v, int lane, int stride, bool desc) {
    const unsigned long long o = __shfl_xor(v, stride);
    const bool lower = (lane & stride) == 0;
    return lower == desc ? max_u64(v, o) : min_u64(v, o);
}

// Sort one key per lane into descending order across the wave.
__device__ __forceinline__ unsigned long long sort64(unsigned long long v, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) v = cx(v, lane, stride, (lane & size) == 0 || size == 64);
    return v;
}

// The 64 best of two descending lists, one key per lane: lane l keeps
// max(a[l], b[63 - l]), then the bitonic merge sorts it descending.
__device__ __forceinline__ unsigned long long merge64(unsigned long long a, unsigned long long b_rev, int lane) {
    unsigned long long v = max_u64(a, b_rev);
#pragma unroll
    for (int stride = 32; stride > 0; stride >>= 1) v = cx(v, lane, stride, true);
    return v;
}

__global__ __launch_bounds__(256) void topk_stage1(const float *__restrict__ y, int n,
                                                   unsigned long long *__restrict__ lists) {
    __shared__ unsigned long long wl[4][TOPK_LIST];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int base = blockIdx.x * TOPK_SLICE + wave * 256;
    // All four loads go out before any is used.
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = base + 64 * r + lane;
        v[r] = y[i < n ? i : n - 1];
    }
    unsigned long long k[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = base + 64 * r + lane;
        k[r] = sort64(i < n ? topk_key(v[r], i) : 0ull, lane);
    }
    const unsigned long long m01 = merge64(k[0], __shfl(k[1], 63 - lane), lane);
    const unsigned long long m23 = merge64(k[2], __shfl(k[3], 63 - lane), lane);
    wl[wave][lane] = merge64(m01, __shfl(m23, 63 - lane), lane);
    __syncthreads();
    if (wave == 0) {
        const unsigned long long a = merge64(wl[0][lane], wl[1][63 - lane], lane);
        const unsigned long long b = merge64(wl[2][lane], wl[3][63 - lane], lane);
        lists[(size_t)blockIdx.x * TOPK_LIST + lane] = merge64(a, __shfl(b, 63 - lane), lane);
    }
}

__global__ __launch_bounds__(1024) void topk_stage2(const float *__restrict__ y, const unsigned long long *lists,
                                                    int nlists, int k, float *__restrict__ vals,
                                                    int32_t *__restrict__ idx) {
    extern __shared__ __attribute__((aligned(16))) unsigned long long lk[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    int np = 1;
    while (np < nlists) np <<= 1;
    {
        // Up to 16 keys per thread (256 lists of 64), all loaded before any
        // is stored; missing lists are empty (key 0).
        const int have = nlists * TOPK_LIST;
        unsigned long long kv[TOPK_MAX_LISTS * TOPK_LIST / 1024];
#pragma unroll
        for (int j = 0; j < TOPK_MAX_LISTS * TOPK_LIST / 1024; ++j) {
            const int i = t + 1024 * j;
            kv[j] = lists[i < have ? i : have - 1];
        }
#pragma unroll
        for (int j = 0; j < TOPK_MAX_LISTS * TOPK_LIST / 1024; ++j) {
            const int i = t + 1024 * j;
            if (i < np * TOPK_LIST) lk[i] = i < have ? kv[j] : 0ull;
        }
    }
    // Level by level: lists a = 2 g s and b = a + s meet into a, a wave per pair.
    for (int s = 1; s < np; s <<= 1) {
        __syncthreads();
        const int pairs = np / (2 * s);
        for (int g = wave; g < pairs; g += 16) {
            unsigned long long *a = lk + (size_t)(2 * g * s) * TOPK_LIST;
            const unsigned long long *b = a + (size_t)s * TOPK_LIST;
            const unsigned long long m = merge64(a[lane], b[63 - lane], lane);
            a[lane] = m;
        }
    }
    __syncthreads();
    if (t < k) {
        const unsigned long long key = lk[t];
        if (key == 0ull) {
            vals[t] = -1e30f;
            idx[t] = 0;
        } else {
            const int i = (int)(0xFFFFFFFFu - (uint32_t)key);
            vals[t] = y[i];
            idx[t] = i;
        }
    }
}

}  // namespace

size_t topk_workspace_bytes(int n) {
    return n <= 0 ? 0 : (size_t)((n + TOPK_SLICE - 1) / TOPK_SLICE) * TOPK_LIST * sizeof(unsigned long long);
}

int topk_max_n() { return TOPK_SLICE * TOPK_MAX_LISTS; }

hipError_t launch_topk(const float *y, int n, int k, float *vals, int32_t *idx, void *workspace,
                       hipStream_t stream) {
    const int nlists = (n + TOPK_SLICE - 1) / TOPK_SLICE;
    if (n < 1 || nlists > TOPK_MAX_LISTS || k < 1 || k > TOPK_LIST) return hipErrorInvalidValue;
    auto *lists = static_cast<unsigned long long *>(workspace);
    hipLaunchKernelGGL(topk_stage1, dim3((unsigned)nlists), dim3(256), 0, stream, y, n, lists);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int np = 1;
    while (np < nlists) np <<= 1;
    const size_t lds = (size_t)np * TOPK_LIST * sizeof(unsigned long long);
    static bool lds_allowed = false;
    if (!lds_allowed) {
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&topk_stage2), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)((size_t)TOPK_MAX_LISTS * TOPK_LIST * sizeof(unsigned long long)));
        if (e != hipSuccess) return e;
        lds_allowed = true;
    }
    hipLaunchKernelGGL(topk_stage2, dim3(1), dim3(1024), lds, stream, y, lists, nlists, k, vals, idx);
    return hipGetLastError();
}

}  // namespace w4a8
