// The chain plan's code object (chain_plan.hip dispatches these kernels as
// raw AQL packets): the M = 1 GEMV with its fp32 activation quantized in its
// staging (gemv_m1_dev.h, the same body, byte for byte), with or without the
// rmsnorm before it, or on an engine-layout activation, as a plain GEMV, as
// gate|up with silu * up as its epilogue (act as fp32 or quantized) and as
// the LM head with its greedy pick, each in four coherence variants and
// under plain C names. A plan's dispatches carry no cache fences
// between them, so a step whose x an earlier step wrote reads it from the
// device's coherence point (_xc), and a step whose y a later step reads
// writes it through (_yc); the others use the caches as usual.
// Built as a device-only code object and embedded in the library
// (chain_plan_co.S); not linked as a HIP module.
#include "gemv_m1_dev.h"

namespace w4a8 {
namespace {

template <int XF, bool ARGMAX, int PAIR, int COH, bool STREAM = false>
__device__ __forceinline__ void plan_step(const uint8_t *w0, const void *x, int rows, int k, int C, int rpw, int tiles,
                                          int nblocks, int nthreads, GemvParams &P, const StreamSync *S = nullptr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    P.seg[0] = w0;
    P.x = x;
    P.rows = rows;
    P.k = k;
    P.C = C;
    P.rpw = rpw;
    P.tiles = tiles;
    gemv_m1_body<XF, true, true, ARGMAX, PAIR, COH, STREAM>(P, blockIdx.x, nblocks, nthreads, lds, S);
}

// The timed twins' stamps: each workgroup's start (its wave 0's first
// instruction) and end (every wave of it done, its stores landed), in ticks
// of the device's constant-rate clock (s_memrealtime), stored by thread 0 as
// two words at stamp[2 g], g the workgroup. Plain vector stores to a slot of
// its own: no two workgroups touch one word, so stamping adds no contention.
__device__ __forceinline__ void stamp_workgroup(unsigned long long *stamp, unsigned long long t0) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
        stamp[2 * blockIdx.x] = t0;
        stamp[2 * blockIdx.x + 1] = t1;
    }
}

}  // namespace
}  // namespace w4a8

// The argument list is the one gemv_m1_kernel takes (its leading scalars are
// preloaded into SGPRs the same way); chain_plan.hip writes it.
#define W4A8_PLAN_ARGS                                                                                       \
    const uint8_t *w0, const void *x, int rows, int k, int C, int rpw, int tiles, int nblocks, int nthreads, \
        w4a8::GemvParams P
#define W4A8_PLAN_PASS w0, x, rows, k, C, rpw, tiles, nblocks, nthreads, P

// One kernel per (step kind, activation format, coherence variant), named
// w4a8_plan_<kind>_<format><variant>; chain_plan.hip builds the same names.
// Each has a timed twin, <name>_t, for w4a8_chain_plan_launch_timed: the
// same body, its workgroups' spans stamped through one more argument (the
// plain kernels are untouched by it).
#define W4A8_PLAN_KERNEL(NAME, XF, ARGMAX, PAIR, COH)                                                     \
    extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void NAME(W4A8_PLAN_ARGS) {            \
        w4a8::plan_step<XF, ARGMAX, PAIR, COH>(W4A8_PLAN_PASS);                                           \
    }                                                                                                     \
    extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void NAME##_t(W4A8_PLAN_ARGS,          \
                                                                             unsigned long long *stamp) { \
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();                                   \
        w4a8::plan_step<XF, ARGMAX, PAIR, COH>(W4A8_PLAN_PASS);                                           \
        w4a8::stamp_workgroup(stamp, t0);                                                                 \
    }
// The overlapped plan's kernels (the plain GEMV only): w4a8_plan_gemv_<format>
// <variant>_s, the step-to-step wait through one more argument.
#define W4A8_PLAN_STREAM_KERNEL(NAME, XF, COH)                                                       \
    extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void NAME##_s(W4A8_PLAN_ARGS,      \
                                                                             w4a8::StreamSync S) { \
        w4a8::plan_step<XF, false, 0, COH, true>(W4A8_PLAN_PASS, &S);                                \
    }
#define W4A8_PLAN_STREAM_KIND(FMT, XF)                                                   \
    W4A8_PLAN_STREAM_KERNEL(w4a8_plan_gemv_##FMT, XF, 0)                                 \
    W4A8_PLAN_STREAM_KERNEL(w4a8_plan_gemv_##FMT##_xc, XF, w4a8::COH_X)                  \
    W4A8_PLAN_STREAM_KERNEL(w4a8_plan_gemv_##FMT##_yc, XF, w4a8::COH_Y)                  \
    W4A8_PLAN_STREAM_KERNEL(w4a8_plan_gemv_##FMT##_xyc, XF, w4a8::COH_X | w4a8::COH_Y)

#define W4A8_PLAN_KIND(KIND, FMT, XF, ARGMAX, PAIR)                                            \
    W4A8_PLAN_KERNEL(w4a8_plan_##KIND##_##FMT, XF, ARGMAX, PAIR, 0)                            \
    W4A8_PLAN_KERNEL(w4a8_plan_##KIND##_##FMT##_xc, XF, ARGMAX, PAIR, w4a8::COH_X)             \
    W4A8_PLAN_KERNEL(w4a8_plan_##KIND##_##FMT##_yc, XF, ARGMAX, PAIR, w4a8::COH_Y)             \
    W4A8_PLAN_KERNEL(w4a8_plan_##KIND##_##FMT##_xyc, XF, ARGMAX, PAIR, w4a8::COH_X | w4a8::COH_Y)

// The GEMV (w4a8_gemv_f32, w4a8_gemv_rmsnorm, and w4a8_gemv on an
// engine-layout x), gate|up with silu * up as its epilogue
// (w4a8_gemv_gate_up_silu, and w4a8_gemv_gate_up_silu_q8_0 quantizing it),
// the LM head with its greedy pick (w4a8_gemv_f32_argmax,
// w4a8_gemv_rmsnorm_argmax).
W4A8_PLAN_KIND(gemv, f32, w4a8::X_F32, false, 0)
W4A8_PLAN_KIND(gemv, rms, w4a8::X_RMS, false, 0)
W4A8_PLAN_KIND(gemv, eng, w4a8::X_ENGINE, false, 0)
W4A8_PLAN_KIND(pair, f32, w4a8::X_F32, false, w4a8::PAIR_F32)
W4A8_PLAN_KIND(pair, rms, w4a8::X_RMS, false, w4a8::PAIR_F32)
W4A8_PLAN_KIND(pairq, f32, w4a8::X_F32, false, w4a8::PAIR_Q8)
W4A8_PLAN_KIND(pairq, rms, w4a8::X_RMS, false, w4a8::PAIR_Q8)
W4A8_PLAN_KIND(argmax, f32, w4a8::X_F32, true, 0)
W4A8_PLAN_KIND(argmax, rms, w4a8::X_RMS, true, 0)
W4A8_PLAN_STREAM_KIND(f32, w4a8::X_F32)
W4A8_PLAN_STREAM_KIND(eng, w4a8::X_ENGINE)
