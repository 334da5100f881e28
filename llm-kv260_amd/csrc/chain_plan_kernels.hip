// The chain plan's code object (chain_plan.hip dispatches these kernels as
// raw AQL packets): the per-step chain's M = 1 GEMV with the fp32 activation
// quantized in its staging (gemv_m1_dev.h, the same body, byte for byte), in
// four coherence variants and under plain C names. A plan's dispatches carry
// no cache fences between them, so a step whose x an earlier step wrote reads
// it from the device's coherence point (_xc), and a step whose y a later step
// reads writes it through (_yc); the others use the caches as usual.
// Built as a device-only code object and embedded in the library
// (chain_plan_co.S); not linked as a HIP module.
#include "gemv_m1_dev.h"

namespace w4a8 {
namespace {

template <int COH>
__device__ __forceinline__ void plan_step(const uint8_t *w0, const void *x, int rows, int k, int C, int rpw, int tiles,
                                          int nblocks, int nthreads, GemvParams &P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    P.seg[0] = w0;
    P.x = x;
    P.rows = rows;
    P.k = k;
    P.C = C;
    P.rpw = rpw;
    P.tiles = tiles;
    gemv_m1_body<X_F32, true, true, false, false, COH>(P, blockIdx.x, nblocks, nthreads, lds);
}

}  // namespace
}  // namespace w4a8

// The argument list is the one gemv_m1_kernel takes (its leading scalars are
// preloaded into SGPRs the same way); chain_plan.hip writes it.
#define W4A8_PLAN_ARGS                                                                                       \
    const uint8_t *w0, const void *x, int rows, int k, int C, int rpw, int tiles, int nblocks, int nthreads, \
        w4a8::GemvParams P
#define W4A8_PLAN_PASS w0, x, rows, k, C, rpw, tiles, nblocks, nthreads, P

extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void w4a8_plan_gemv_f32(W4A8_PLAN_ARGS) {
    w4a8::plan_step<0>(W4A8_PLAN_PASS);
}
extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void w4a8_plan_gemv_f32_xc(W4A8_PLAN_ARGS) {
    w4a8::plan_step<w4a8::COH_X>(W4A8_PLAN_PASS);
}
extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void w4a8_plan_gemv_f32_yc(W4A8_PLAN_ARGS) {
    w4a8::plan_step<w4a8::COH_Y>(W4A8_PLAN_PASS);
}
extern "C" __global__ __launch_bounds__(w4a8::MAX_THREADS) void w4a8_plan_gemv_f32_xyc(W4A8_PLAN_ARGS) {
    w4a8::plan_step<w4a8::COH_X | w4a8::COH_Y>(W4A8_PLAN_PASS);
}
