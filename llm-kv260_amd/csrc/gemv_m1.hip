// M = 1 W4A8 GEMV for gfx950: the host launchers (launch shapes, entry
// points, the batch and the per-step chain). The kernels and their design are
// in gemv_m1_dev.h.
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "gemv_m1_dev.h"

namespace w4a8 {

namespace {

template <int XF, bool PLAIN, bool ONE_PASS, bool ARGMAX, int PAIR = 0>
hipError_t launch_pass(const GemvParams &P, int grid, int threads, size_t lds, hipStream_t stream) {
    const hipError_t e =
        allow_dynamic_lds(reinterpret_cast<const void *>(&gemv_m1_kernel<XF, PLAIN, ONE_PASS, ARGMAX, PAIR>), LDS_BUDGET);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemv_m1_kernel<XF, PLAIN, ONE_PASS, ARGMAX, PAIR>), dim3(grid), dim3(threads), lds, stream,
                       P.seg[0], P.x, P.rows, P.k, P.C, P.rpw, P.tiles, grid, threads, P);
    return hipGetLastError();
}

template <int XF, bool PLAIN, bool ARGMAX>
hipError_t launch_xf(const GemvParams &P, int grid, int threads, size_t lds, hipStream_t stream) {
    return P.rpw <= 8 ? launch_pass<XF, PLAIN, true, ARGMAX>(P, grid, threads, lds, stream)
                      : launch_pass<XF, PLAIN, false, ARGMAX>(P, grid, threads, lds, stream);
}

template <int XF, bool ARGMAX = false>
hipError_t launch_layout(const GemvParams &P, bool plain, int grid, int threads, size_t lds, hipStream_t stream) {
    return plain ? launch_xf<XF, true, ARGMAX>(P, grid, threads, lds, stream)
                 : launch_xf<XF, false, ARGMAX>(P, grid, threads, lds, stream);
}

}  // namespace

int device_cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

hipError_t allow_dynamic_lds(const void *fn, size_t budget) {
    static std::mutex mu;
    static std::vector<std::pair<const void *, int>> done;   // (kernel, device) pairs already allowed
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> g(mu);
    for (const auto &d : done)
        if (d.first == fn && d.second == dev) return hipSuccess;
    // What the kernel's static LDS leaves of the budget.
    hipFuncAttributes attr{};
    e = hipFuncGetAttributes(&attr, fn);
    if (e != hipSuccess) return e;
    if (attr.sharedSizeBytes > budget) return hipErrorInvalidValue;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(budget - attr.sharedSizeBytes));
    if (e != hipSuccess) return e;
    done.emplace_back(fn, dev);
    return hipSuccess;
}

size_t argmax_workspace_bytes() { return ARGMAX_KEY_OFFSET + 64; }

M1Shape gemv_m1_shape(int tiles, int k, XFormat xf, bool /*argmax*/, int cus) {
    const int nb = k / QK;
    // Staged activation: int8 values, fp32 scale and int32 sum per block; for
    // X_RMS also the squares of x as float64 and the rmsnorm scale.
    const size_t x_lds = x_lds_bytes(nb) + (xf == X_RMS ? rms_sq_doubles(k) * 8 + 16 : 0);
    // Launch shape, from what bounds each size:
    //  * Small matrices (at most two tiles per CU): latency. One tile per
    //    wave, two-wave workgroups spread over the CUs (each stages its own
    //    copy of x in parallel). In the decode chain two waves per workgroup
    //    ran 234.3-235.0 us per step against 235.7-236.0 with one and 244.5
    //    with four (alone, q|k|v and o are within 0.04 us either way).
    //  * Mid-size (up to eight tiles per CU): one workgroup per CU whose waves
    //    walk MID_TILES_PER_WAVE tiles each. One per wave, every tile in
    //    flight at once: gate|up 5.8 us, against 6.0 at four per wave and
    //    6.4 at two. (Before the staged activation was padded against bank
    //    conflicts, four per wave had been the faster.)
    //  * Large: bandwidth. Four-wave workgroups, every wave walking tiles
    //    with a stride of the whole grid, at most eight resident waves per CU
    //    (two tiles and the activation column take about 208 VGPRs, two
    //    waves per SIMD); two workgroups per CU (below).
    // Every workgroup has at least one thread per activation block, so x is
    // staged in one pass. (Spreading an fp32 x's quantization over 2-8
    // threads per block, in helper waves or in the spare threads of the
    // larger workgroups, made no launch faster: the down GEMV lost 0.9 us.)
    int min_waves = nb > 64 ? (nb + 63) / 64 : 1;           // <= 8 for K <= 16384
    // The rmsnorm forms stage their x with four threads per block where a
    // workgroup can hold them (K = 2048: four waves).
    if (xf == X_RMS && nb / 16 <= MAX_THREADS / 64 && nb / 16 > min_waves) min_waves = nb / 16;
    int waves = min_waves > 2 ? min_waves : 2;
    int grid = (tiles + waves - 1) / waves;
    if (tiles > 2 * cus) {
        if (tiles > 8 * cus) {
            // Exactly the resident workgroups: two per CU. A third per CU
            // (taking over as one finishes) made the LM head slower with
            // every activation form: 25.8 against 24.4-25.0 us with engine x,
            // 26.4 against 24.4 with fp32 x, and the decode chain 237.2
            // against 235.1 us per step.
            waves = 4 > min_waves ? 4 : min_waves;
            grid = (tiles + waves - 1) / waves;
            if (grid > 2 * cus) grid = 2 * cus;
        } else {
            const int per_cu = (tiles + cus - 1) / cus;
            waves = (per_cu + MID_TILES_PER_WAVE - 1) / MID_TILES_PER_WAVE;
            if (waves < min_waves) waves = min_waves;
            grid = (tiles + waves - 1) / waves;
            if (grid > cus) grid = cus;
        }
    }
    return M1Shape{grid, 64 * waves, (size_t)waves * TILE_BYTES + x_lds};
}

hipError_t launch_gemv_m1(const MatrixRef &w, const void *x, XFormat xf, float *y, hipStream_t stream,
                          int32_t *argmax, void *workspace, XAux aux) {
    GemvParams P{};
    P.norm_w = aux.norm_w;
    P.eps = aux.eps;
    if (argmax) {
        P.argmax = argmax;
        P.ticket = static_cast<unsigned int *>(workspace);
        P.key = reinterpret_cast<unsigned long long *>(static_cast<uint8_t *>(workspace) + ARGMAX_KEY_OFFSET);
    }
    for (int s = 0; s < 4; ++s) P.seg[s] = s < w.nseg ? w.seg[s] : w.seg[0];
    P.x = x;
    P.y = y;
    P.seg_rows = w.seg_rows;
    P.nseg = w.nseg;
    P.k = w.k;
    P.rows = w.seg_rows * w.nseg;
    P.paired = w.paired ? 1 : 0;
    P.C = w.k / 256;
    if (P.C < 1 || P.C > 64 || w.k % 256) return hipErrorInvalidValue;
    P.rpw = 64 / P.C;
    P.tiles = (P.rows + P.rpw - 1) / P.rpw;
    const bool plain = w.nseg == 1 && !w.paired;
    if (!plain) {
        // Board layouts: whole tiles per segment (v2: whole row pairs).
        if (w.paired) {
            if (w.seg_rows % 2 || P.rpw < 2) return hipErrorInvalidValue;
            P.prw = P.rpw / 2;
            P.tps = (w.seg_rows / 2 + P.prw - 1) / P.prw;
        } else {
            P.tps = (w.seg_rows + P.rpw - 1) / P.rpw;
        }
        P.tiles = w.nseg * P.tps;
    }
    if (P.tiles < 1) return hipSuccess;
    if (xf == X_RMS && w.k > 8192) return hipErrorInvalidValue;
    const M1Shape sh = gemv_m1_shape(P.tiles, w.k, xf, argmax != nullptr, device_cu_count());
    const int grid = sh.grid, threads = sh.threads;
    const size_t lds = sh.lds;
    if (argmax) {
        if (xf == X_F32) return launch_layout<X_F32, true>(P, plain, grid, threads, lds, stream);
        if (xf == X_RMS) return launch_layout<X_RMS, true>(P, plain, grid, threads, lds, stream);
        return hipErrorInvalidValue;
    }
    switch (xf) {
        case X_ENGINE: return launch_layout<X_ENGINE>(P, plain, grid, threads, lds, stream);
        case X_Q8_0: return launch_layout<X_Q8_0>(P, plain, grid, threads, lds, stream);
        case X_F32: return launch_layout<X_F32>(P, plain, grid, threads, lds, stream);
        case X_RMS: return launch_layout<X_RMS>(P, plain, grid, threads, lds, stream);
        case X_SILU: return launch_layout<X_SILU>(P, plain, grid, threads, lds, stream);
        default: return hipErrorInvalidValue;
    }
}

template <bool ONE_PASS>
hipError_t launch_batch_pass(const BatchParams &B, int max_k, hipStream_t stream) {
    long blocks = 0;
    for (int i = 0; i < B.n; ++i) blocks += batch_blocks(B.e[i].rows, B.e[i].k, B.tiles_per_block);
    if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
    const size_t lds = (size_t)(BATCH_THREADS / 64) * TILE_BYTES + x_lds_bytes(max_k / QK);
    const hipError_t e = allow_dynamic_lds(reinterpret_cast<const void *>(&gemv_batch_kernel<ONE_PASS>), LDS_BUDGET);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gemv_batch_kernel<ONE_PASS>, dim3((unsigned)blocks), dim3(BATCH_THREADS), lds, stream, B);
    return hipGetLastError();
}

// Waves per workgroup of the gate|up + silu launch: V gate waves and their V
// up partners, one tile each, so V must divide tiles / 2 (the grid is
// tiles / 2 / V workgroups) and the 2V waves must hold one thread per
// activation block. V = 4 where it fits (eight waves, as the plain gate|up
// GEMV runs); 0 when no V does (or the shape is outside 2048 <= k <= 8192,
// whole tiles in each half).
int gate_up_silu_waves(int rows, int k) {
    if (k % 256 || k < 2048 || k > 8192 || rows < 2 || rows % 2) return 0;
    const int rpw = 64 / (k / 256);
    if ((rows / 2) % rpw) return 0;   // tiles may not straddle the two halves
    const int half = rows / 2 / rpw;
    const int nb = k / QK;
    const int min_waves = nb > 64 ? (nb + 63) / 64 : 1;
    for (int v = 4; 2 * v >= min_waves && v >= 1; v >>= 1)
        if (half % v == 0) return 2 * v;
    return 0;
}

bool gate_up_silu_q8_fits(int rows, int k) { return k == 2048 && gate_up_silu_waves(rows, k) == 8; }

hipError_t launch_gemv_gate_up_silu(const uint8_t *w, const float *x, XFormat xf, void *act, int rows, int k,
                                    hipStream_t stream, XAux aux, bool q8) {
    const int waves = gate_up_silu_waves(rows, k);
    if ((xf != X_F32 && xf != X_RMS) || waves == 0 || (q8 && !gate_up_silu_q8_fits(rows, k)))
        return hipErrorInvalidValue;
    GemvParams P{};
    derive_plain(P, w, x, static_cast<float *>(act), rows, k);
    P.norm_w = aux.norm_w;
    P.eps = aux.eps;
    const int half = P.tiles / 2;
    const int nb = k / QK;
    const int grid = half / (waves / 2);
    const size_t x_lds = x_lds_bytes(nb) + (xf == X_RMS ? rms_sq_doubles(k) * 8 + 16 : 0);
    const size_t lds = (size_t)waves * TILE_BYTES + x_lds;
    if (q8) {
        if (xf == X_RMS) return launch_pass<X_RMS, true, true, false, PAIR_Q8>(P, grid, 64 * waves, lds, stream);
        return launch_pass<X_F32, true, true, false, PAIR_Q8>(P, grid, 64 * waves, lds, stream);
    }
    if (xf == X_RMS) return launch_pass<X_RMS, true, true, false, PAIR_F32>(P, grid, 64 * waves, lds, stream);
    return launch_pass<X_F32, true, true, false, PAIR_F32>(P, grid, 64 * waves, lds, stream);
}

hipError_t launch_gemv_batch(const w4a8_chain_step *steps, int n, hipStream_t stream) {
    if (n < 1 || n > W4A8_CHAIN_MAX_STEPS) return hipErrorInvalidValue;
    // Entries with K >= 2048 (one pass of ordered sums per tile) and the rest
    // go to the two instances of the kernel: one launch when all are alike.
    BatchParams B[2] = {};
    int max_k[2] = {0, 0};
    for (int i = 0; i < n; ++i) {
        const int k = steps[i].k;
        if (k < 256 || k % 256 || k > MAX_K_M1 || steps[i].rows < 1) return hipErrorInvalidValue;
        const int s = k >= 2048 ? 0 : 1;
        B[s].e[B[s].n++] = BatchEntry{static_cast<const uint8_t *>(steps[i].w), steps[i].x, steps[i].y, steps[i].rows, k};
        if (k > max_k[s]) max_k[s] = k;
    }
    for (int s = 0; s < 2; ++s) B[s].tiles_per_block = BATCH_TILES_PER_WAVE * (BATCH_THREADS / 64);
    if (B[0].n) {
        const hipError_t e = launch_batch_pass<true>(B[0], max_k[0], stream);
        if (e != hipSuccess) return e;
    }
    if (B[1].n) return launch_batch_pass<false>(B[1], max_k[1], stream);
    return hipSuccess;
}

hipError_t launch_chain(const w4a8_chain_step *steps, int n, hipStream_t stream) {
    if (chain_one_launch_fits(steps, n)) {
        const hipError_t e = launch_chain_one(steps, n, stream);
        // Too few CUs free for every workgroup to be resident: per step below.
        if (e != hipErrorCooperativeLaunchTooLarge) return e;
        (void)hipGetLastError();
    }
    // One fused quantize + GEMV kernel per step; stream order carries the
    // step-to-step dependency.
    for (int i = 0; i < n; ++i) {
        MatrixRef m{};
        m.seg[0] = static_cast<const uint8_t *>(steps[i].w);
        m.nseg = 1;
        m.seg_rows = steps[i].rows;
        m.rows = steps[i].rows;
        m.k = steps[i].k;
        const hipError_t e = launch_gemv_m1(m, steps[i].x, X_F32, steps[i].y, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace w4a8
