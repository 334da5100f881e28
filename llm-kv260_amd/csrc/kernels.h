// Host-side launchers of the engine's HIP kernels (internal to the library).
// Argument checking happens in the C ABI layer (api.cpp); these assume valid,
// already-checked shapes and pointers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a8 {

// Activation formats the GEMV kernels can stage.
enum XFormat : int {
    X_ENGINE = 0,   // int8[K] then float32[K/32]  (pack_x_for_engine, q4_0.py:193-200)
    X_Q8_0 = 1,     // ggml Q8_0 blocks: fp16 d then 32 int8, 34 bytes each
    X_F32 = 2,      // float32[K], quantized to Q8_0 inside the kernel (fused)
    X_RMS = 3,      // float32[K] x and float32[K] norm weight: rmsnorm, then Q8_0, inside the kernel
    X_SILU = 4,     // float32[2K] gate | up: silu(gate) * up, then Q8_0, inside the kernel
};

// Extra inputs of the fused producer formats.
struct XAux {
    const float *norm_w = nullptr;   // X_RMS
    float eps = 0.0f;
};

// Up to four row segments of one matrix: rows [s*seg_rows, (s+1)*seg_rows) live
// contiguously (row-major, K/32*18 bytes per row) from seg[s]. One segment is a
// plain ggml matrix; four are the reference v1 engine's per-engine quarters.
// Output rows are contiguous: y[s*seg_rows + r].
// paired: the v2 engine's port layout instead -- in a segment of R rows, row i
// and row i + R/2 form a pair whose 144-byte chunks alternate
// (board/kv260gemv/gemv2_dev.h:46-49, 66-72); R must be even.
struct MatrixRef {
    const uint8_t *seg[4];
    int nseg;
    int seg_rows;
    int rows;
    int k;
    bool paired;
};

constexpr int MAX_K_M1 = 16384;   // LDS-staged activation limit of the M=1 kernel
constexpr int MAX_K_GEMM = 16384;

int device_cu_count();            // of the current device (cached per device)
// Lets kernel `fn` launch with up to `budget` bytes of LDS in all (its static
// LDS included) on the current device. The runtime needs this once per
// kernel and device for dynamic LDS above 64 KB; later calls only look it up.
// Thread-safe.
hipError_t allow_dynamic_lds(const void *fn, size_t budget);

// The M = 1 GEMV's launch shape for a matrix of `tiles` wave tiles (64 / (k /
// 256) rows each): workgroups, threads per workgroup, dynamic LDS bytes.
struct M1Shape {
    int grid, threads;
    size_t lds;
};
M1Shape gemv_m1_shape(int tiles, int k, XFormat xf, bool argmax, int cus);

// argmax != null: also *argmax = the first row of the largest y, reduced in the
// same launch through `workspace` (argmax_workspace_bytes(), zero between
// calls); x must then be X_F32 or X_RMS.
hipError_t launch_gemv_m1(const MatrixRef &w, const void *x, XFormat xf, float *y, hipStream_t stream,
                          int32_t *argmax = nullptr, void *workspace = nullptr, XAux aux = XAux{});
size_t argmax_workspace_bytes();   // of the current device

// The k (1..64) best of y[0..n) as the reference's sampler selects them
// (values descending, the smaller index first among equals, never a value at
// or below -1e30): two launches, the candidate lists of 1024-logit slices in
// `workspace` (topk_workspace_bytes(n)). n <= topk_max_n().
hipError_t launch_topk(const float *y, int n, int k, float *vals, int32_t *idx, void *workspace,
                       hipStream_t stream);
size_t topk_workspace_bytes(int n);
int topk_max_n();
// Same, the lists in the library's own device array (one per device, no
// allocation): calls that overlap on one device race on it.
hipError_t launch_topk_no_alloc(const float *y, int n, int k, float *vals, int32_t *idx, hipStream_t stream);

// y[m][rows] for m activation rows in engine layout (row stride K + K/8 bytes).
hipError_t launch_gemm(const MatrixRef &w, const uint8_t *x_engine_rows, int m, float *y, hipStream_t stream);
// The few-token GEMV (gemv_mt.hip): 2 <= m <= 8 engine-layout rows, k in
// 2048..8192, the M = 1 kernel's weight stream with the arithmetic per token.
bool gemv_mt_fits(int m, int rows, int k);
// The largest m for which it is the faster kernel on this shape.
int gemv_mt_max_m(int rows, int k);
hipError_t launch_gemv_mt(const uint8_t *w, const uint8_t *x, int m, float *y, int rows, int k, hipStream_t stream);
// The row-split M > 1 kernel (gemm_rows.hip): m <= 64, k % 512 == 0.
bool gemm_rows_fits(int rows, int k);
hipError_t launch_gemm_rows(const uint8_t *w, const uint8_t *x, int m, float *y, int rows, int k, hipStream_t stream);

// x: float32[m][K] -> engine layout rows, or ggml Q8_0 block rows.
hipError_t launch_quantize_q8_0(const float *x, int k, int m, uint8_t *out, XFormat out_fmt, hipStream_t stream);
// Producers of the activation, then Q8_0, to engine layout rows (K <= 16384):
// rmsnorm (m rows of float32[K], norm weight float32[K]); silu(gate) * up
// (m rows of float32[2K] gate | up).
hipError_t launch_rmsnorm_q8_0(const float *x, const float *w, float eps, int k, int m, uint8_t *out,
                               hipStream_t stream);
hipError_t launch_silu_mul_q8_0(const float *gate_up, int k, int m, uint8_t *out, hipStream_t stream);

}  // namespace w4a8

struct w4a8_chain_step;   // include/w4a8.h
struct w4a8_chain_plan;   // chain_plan.hip
struct w4a8_plan_step;    // include/w4a8.h

namespace w4a8 {

// The decode chain: one GEMV per step, in order, x quantized inside. One
// launch per step, or, in the one-launch mode when chain_one_launch_fits
// (every k in 2048 .. 8192), one cooperative launch for the whole chain.
hipError_t launch_chain(const w4a8_chain_step *steps, int n, hipStream_t stream);
bool chain_one_launch_fits(const w4a8_chain_step *steps, int n);
hipError_t launch_chain_one(const w4a8_chain_step *steps, int n, hipStream_t stream);
// The chain plan (chain_plan.hip): statuses as the C ABI's; a HIP error of
// create comes back in `he` with W4A8_ERR_HIP.
int plan_check_ranges(const w4a8_plan_step *steps, int n);   // before any device work
int chain_plan_create(const w4a8_plan_step *steps, int n, bool overlapped, w4a8_chain_plan **out, hipError_t &he);
int chain_plan_launch(w4a8_chain_plan *p, int passes);
int chain_plan_launch_timed(w4a8_chain_plan *p, int passes, unsigned long long *stamps, hipError_t &he);
int chain_plan_steps(const w4a8_chain_plan *p);
long chain_plan_workgroups(const w4a8_chain_plan *p, int step);
int chain_plan_wait(w4a8_chain_plan *p, int timeout_ms);
int chain_plan_destroy(w4a8_chain_plan *p);
// The one-launch chain's bounded waits: polls before a wait gives up
// (<= 0 restores the default), and the count of launches on the current
// device that gave up since the last call (read and cleared; synchronous).
void chain_set_spin_limit(int polls);
hipError_t chain_take_timeouts(int *out);
// 0: one launch when the chain fits; 1: one launch per step (the default).
void chain_set_mode(int mode);
int chain_mode();

// The same GEMVs with no order between them, in one launch.
hipError_t launch_gemv_batch(const w4a8_chain_step *steps, int n, hipStream_t stream);
// gate|up (rows = 2 n) with silu(gate) * up as the epilogue: act[n] from
// x as X_F32 or X_RMS (aux), 2048 <= k <= 8192, n a multiple of 64 / (k / 256).
// q8: act quantized in the epilogue, `act` then the engine layout of n values
// (gate_up_silu_q8_fits).
hipError_t launch_gemv_gate_up_silu(const uint8_t *w, const float *x, XFormat xf, void *act, int rows, int k,
                                    hipStream_t stream, XAux aux = XAux{}, bool q8 = false);
// Its workgroup size in waves for a shape, 0 when the shape does not fit.
int gate_up_silu_waves(int rows, int k);
// The quantizing form needs a workgroup's 32 outputs to be one Q8_0 block:
// k = 2048 and eight waves.
bool gate_up_silu_q8_fits(int rows, int k);

// w: float32[rows][K] -> Q4_0 rows.
hipError_t launch_quantize_q4_0(const float *w, int rows, int k, uint8_t *out, hipStream_t stream);

}  // namespace w4a8
