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
// never admit (v <= -1e30) gets key 0. The k largest keys are then exactly
// the reference's k candidates, in its order, for every input without NaN.
//
// Stage 1: one 256-thread workgroup per 1024 logits. Each wave holds 256
// keys, four per lane as four lists of 64 (one key per lane each), sorts the
// four across its lanes (bitonic, register compare-exchanges with the lane
// `stride` apart), and merges them two by two; the four waves' best 64 then
// merge through LDS, and the workgroup writes its 64 best. Stage 2: one
// workgroup merges those lists pairwise, level by level. A merge of two
// descending lists A and B keeps, in lane l, max(A[l], B[63 - l]): a bitonic
// sequence holding their 64 best, which six compare-exchange steps sort.
//
// A NaN logit has no place in that order: the reference's loop admits it
// (v <= NaN is false) into the last slot, evicting the k-th candidate it
// held at that point, and then admits the next logit whatever its value,
// so the result depends on where the NaN stands. A stage-1 workgroup that
// sees a NaN marks its list (first key all ones, which no value's key can
// be: NaN is the only float whose order bits are all ones), and stage 2,
// finding a mark, runs the reference's loop itself, in order, in one wave
// (topk_in_order): the same candidates, bit for bit, at the cost of one
// pass over y by a single wave.
#include "kernels.h"

#include <atomic>
#include <mutex>

namespace w4a8 {

namespace {

constexpr int TOPK_SLICE = 1024;      // logits per stage-1 workgroup
constexpr int TOPK_LIST = 64;         // candidates each list keeps (k <= 64)
constexpr int TOPK_MAX_LISTS = 256;   // stage 2's LDS: 256 x 64 keys = 128 KB
static_assert(TOPK_LIST == 64, "the index arithmetic below takes lists of 64");

constexpr unsigned long long NAN_MARK = ~0ull;   // a stage-1 list whose slice holds a NaN

__device__ __forceinline__ unsigned long long topk_key(float v, int i) {
    if (!(v > -1e30f)) return 0ull;                                  // never admitted (NaN: see NAN_MARK)
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

// The value of lane l ^ S for one 32-bit word: DPP for S = 1, 2, 8 (quad
// permutations, a rotation by 8 within a row of 16), an LDS swizzle in
// bit mode for S = 4, 16, ds_bpermute for S = 32.
template <int S>
__device__ __forceinline__ int xor_lane(int v, int lane) {
    if constexpr (S == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    else if constexpr (S == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    else if constexpr (S == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);  // row_ror:8
    else if constexpr (S == 4 || S == 16) return __builtin_amdgcn_ds_swizzle(v, (S << 10) | 0x1F);
    else return __builtin_amdgcn_ds_bpermute((lane ^ S) << 2, v);
}

// One compare-exchange step of a bitonic network over the wave's 64 lanes:
// the pair (l, l ^ S) ends ordered descending when `desc`, with the larger
// key in the lower lane.
template <int S>
__device__ __forceinline__ unsigned long long cx(unsigned long long v, int lane, bool desc) {
    const int lo = xor_lane<S>((int)(uint32_t)v, lane), hi = xor_lane<S>((int)(uint32_t)(v >> 32), lane);
    const unsigned long long o = ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
    const bool lower = (lane & S) == 0;
    return (o > v) == (lower == desc) ? o : v;
}

template <int SIZE, int S>
__device__ __forceinline__ unsigned long long sort_steps(unsigned long long v, int lane) {
    v = cx<S>(v, lane, SIZE == 64 || (lane & SIZE) == 0);
    if constexpr (S > 1) v = sort_steps<SIZE, S / 2>(v, lane);
    return v;
}

// Sort one key per lane into descending order across the wave.
__device__ __forceinline__ unsigned long long sort64(unsigned long long v, int lane) {
    v = sort_steps<2, 1>(v, lane);
    v = sort_steps<4, 2>(v, lane);
    v = sort_steps<8, 4>(v, lane);
    v = sort_steps<16, 8>(v, lane);
    v = sort_steps<32, 16>(v, lane);
    return sort_steps<64, 32>(v, lane);
}

// The 64 best of two descending lists, one key per lane: lane l keeps
// max(a[l], b[63 - l]), then the bitonic merge sorts it descending.
__device__ __forceinline__ unsigned long long merge64(unsigned long long a, unsigned long long b_rev, int lane) {
    return sort_steps<64, 32>(max_u64(a, b_rev), lane);
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
    bool nan = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) nan = nan || (base + 64 * r + lane < n && v[r] != v[r]);
    const unsigned long long m01 = merge64(k[0], __shfl(k[1], 63 - lane), lane);
    const unsigned long long m23 = merge64(k[2], __shfl(k[3], 63 - lane), lane);
    wl[wave][lane] = merge64(m01, __shfl(m23, 63 - lane), lane);
    const bool slice_has_nan = __syncthreads_or(nan);
    if (wave == 0) {
        const unsigned long long a = merge64(wl[0][lane], wl[1][63 - lane], lane);
        const unsigned long long b = merge64(wl[2][lane], wl[3][63 - lane], lane);
        const unsigned long long best = merge64(a, __shfl(b, 63 - lane), lane);
        lists[(size_t)blockIdx.x * TOPK_LIST + lane] = slice_has_nan && lane == 0 ? NAN_MARK : best;
    }
}

// The reference's loop (tp_llama.cpp:902-908) as written, over y[0..n) in
// order, in one wave: lane j holds slot j (value bits and index). A logit is
// taken when !(v <= last slot's value); each chunk of 64 logits is scanned
// for the next such lane after the one just taken, with the last slot read
// again after every insertion, so a logit is skipped exactly when the loop
// would skip it. The insertion point is one past the highest slot below k-1
// that is not less than v (the while loop's stop), 0 if there is none; the
// slots from there to k-2 move down by one and slot k-1 falls off.
__device__ void topk_in_order(const float *__restrict__ y, int n, int k, float *__restrict__ vals,
                              int32_t *__restrict__ idx, int lane) {
    uint32_t sv = __float_as_uint(-1e30f);
    int si = 0;
    constexpr int U = 8;                      // chunks of 64 loaded at once
    for (int c0 = 0; c0 < n; c0 += 64 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = c0 + 64 * u + lane;
            v[u] = y[i < n ? i : n - 1];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int base = c0 + 64 * u;
            if (base >= n) break;
            const bool in = base + lane < n;
            int last = -1;
            for (;;) {
                const float thr = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)sv, k - 1));
                const unsigned long long m = __ballot(in && lane > last && !(v[u] <= thr));
                if (!m) break;
                const int b = __builtin_ctzll(m);
                const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[u]), b));
                const unsigned long long stop = __ballot(lane < k - 1 && !(__uint_as_float(sv) < x));
                const int pos = stop ? 64 - __builtin_clzll(stop) : 0;
                const uint32_t above = (uint32_t)__shfl((int)sv, lane - 1);
                const int above_i = __shfl(si, lane - 1);
                if (lane == pos) {
                    sv = __float_as_uint(x);
                    si = base + b;
                } else if (lane > pos && lane < k) {
                    sv = above;
                    si = above_i;
                }
                last = b;
            }
        }
    }
    if (lane < k) {
        vals[lane] = __uint_as_float(sv);
        idx[lane] = si;
    }
}

__global__ __launch_bounds__(1024) void topk_stage2(const float *__restrict__ y, int n,
                                                    const unsigned long long *lists, int nlists, int k,
                                                    float *__restrict__ vals,
                                                    int32_t *__restrict__ idx) {
    extern __shared__ __attribute__((aligned(16))) unsigned long long lk[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (__syncthreads_or(t < nlists && lists[(size_t)t * TOPK_LIST] == NAN_MARK)) {
        if (wave == 0) topk_in_order(y, n, k, vals, idx, lane);
        return;
    }
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

// The stage-1 lists of the largest input (TOPK_MAX_LISTS lists of 64 keys,
// 128 KiB) for launch_topk_no_alloc: one copy per device, held until the
// process ends. Host code never passes the name itself to a kernel (on the
// host it is a stand-in, not a device address): it passes the address
// hipGetSymbolAddress gives for the current device.
static __device__ __align__(256) unsigned long long scratch[TOPK_MAX_LISTS * TOPK_LIST];

constexpr int SCRATCH_MAX_DEVICES = 64;
std::atomic<void *> g_scratch[SCRATCH_MAX_DEVICES];
std::mutex g_scratch_mu;

// The device address of `scratch` on the current device, looked up once per
// device (the first call on it) and kept. The lookup is no stream work, but
// it may load the library's code object on that device; under a stream
// capture in global mode such a call could invalidate the capture, so this
// thread's capture mode is relaxed around it (and restored), which lets the
// first call on a device itself be captured.
hipError_t scratch_of_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
            e = hipThreadExchangeStreamCaptureMode(&mode);
            if (e != hipSuccess) return e;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            const hipError_t back = hipThreadExchangeStreamCaptureMode(&mode);
            if (e == hipSuccess) e = back;
            if (e != hipSuccess) return e;
            if (!p) return hipErrorInvalidSymbol;
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
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
    hipError_t e = allow_dynamic_lds(reinterpret_cast<const void *>(&topk_stage2),
                                     (size_t)TOPK_MAX_LISTS * TOPK_LIST * sizeof(unsigned long long));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(topk_stage1, dim3((unsigned)nlists), dim3(256), 0, stream, y, n, lists);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    int np = 1;
    while (np < nlists) np <<= 1;
    const size_t lds = (size_t)np * TOPK_LIST * sizeof(unsigned long long);
    hipLaunchKernelGGL(topk_stage2, dim3(1), dim3(1024), lds, stream, y, n, lists, nlists, k, vals, idx);
    return hipGetLastError();
}

static_assert(sizeof(unsigned long long) * TOPK_MAX_LISTS * TOPK_LIST == 131072,
              "scratch holds the lists of the largest input launch_topk takes");

hipError_t launch_topk_no_alloc(const float *y, int n, int k, float *vals, int32_t *idx, hipStream_t stream) {
    if (n < 1 || n > topk_max_n() || k < 1 || k > TOPK_LIST) return hipErrorInvalidValue;
    void *lists = nullptr;
    const hipError_t e = scratch_of_current_device(&lists);
    if (e != hipSuccess) return e;
    return launch_topk(y, n, k, vals, idx, lists, stream);
}

}  // namespace w4a8
