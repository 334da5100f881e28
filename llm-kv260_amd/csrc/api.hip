// The native C ABI (include/w4a8.h): argument checks, then one enqueue.
#include <stdint.h>

#include "../../include/w4a8.h"
#include "../../include/w4a8_gguf.h"
#include "kernels.h"

using namespace w4a8;

namespace {

thread_local int g_last_hip_error = 0;

int hip_status(hipError_t e) {
    if (e == hipSuccess) return W4A8_OK;
    g_last_hip_error = (int)e;
    return W4A8_ERR_HIP;
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int check_k(int k) {
    if (k < 256 || k > W4A8_MAX_K || k % 256) return W4A8_ERR_SHAPE;
    return W4A8_OK;
}

int check_gemv(const void *w, const void *x, const float *y, int rows, int k, uintptr_t x_align) {
    if (!w || !x || !y) return W4A8_ERR_NULL;
    if (check_k(k) || rows < 1) return W4A8_ERR_SHAPE;
    if (!aligned(w, 16) || !aligned(x, x_align) || !aligned(y, 4)) return W4A8_ERR_ALIGN;
    return W4A8_OK;
}

bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
    return pa < pb + nb && pb < pa + na;
}

// A GEMV whose y overlaps its own x (or weights) races: its workgroups read x
// while others already write y.
bool step_in_place(const w4a8_chain_step &s) {
    const size_t wb = (size_t)s.rows * (size_t)(s.k / 32) * 18;
    return overlaps(s.x, 4 * (size_t)s.k, s.y, 4 * (size_t)s.rows) || overlaps(s.w, wb, s.y, 4 * (size_t)s.rows);
}

MatrixRef plain_matrix(const void *w, int rows, int k) {
    MatrixRef m{};
    m.seg[0] = static_cast<const uint8_t *>(w);
    m.nseg = 1;
    m.seg_rows = rows;
    m.rows = rows;
    m.k = k;
    return m;
}

}  // namespace

extern "C" {

const char *w4a8_contract_version(void) { return "llm-kv260/w4a8-q4_0-v2"; }

const char *w4a8_strerror(int status) {
    switch (status) {
        case W4A8_OK: return "ok";
        case W4A8_ERR_NULL: return "a required pointer is NULL";
        case W4A8_ERR_SHAPE: return "shape outside the engine's rules (k % 256 == 0, 256 <= k <= 16384, rows >= 1)";
        case W4A8_ERR_ALIGN: return "pointer not aligned (weights and activations 16 B, output 4 B)";
        case W4A8_ERR_HIP: return "HIP runtime error";
        case W4A8_ERR_NODEV: return "no usable gfx950 device";
        case W4A8_ERR_FORMAT: return "not a GGUF file, or a malformed one";
        case W4A8_ERR_TIMEOUT: return "a bounded wait ran out";
        case W4A8_ERR_HSA: return "HSA runtime error (queue, code object or signal)";
        default: return "unknown status";
    }
}

int w4a8_last_hip_error(void) { return g_last_hip_error; }

size_t w4a8_q4_0_row_bytes(int k) { return k > 0 ? (size_t)k / 32 * 18 : 0; }
size_t w4a8_engine_x_bytes(int k) { return k > 0 ? (size_t)k + (size_t)k / 32 * 4 : 0; }
size_t w4a8_q8_0_row_bytes(int k) { return k > 0 ? (size_t)k / 32 * 34 : 0; }

int w4a8_gemv(const void *w, const void *x, float *y, int rows, int k, void *stream) {
    if (int s = check_gemv(w, x, y, rows, k, 16)) return s;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), x, X_ENGINE, y, (hipStream_t)stream));
}

int w4a8_gemv_q8_0(const void *w, const void *x_blocks, float *y, int rows, int k, void *stream) {
    if (int s = check_gemv(w, x_blocks, y, rows, k, 2)) return s;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), x_blocks, X_Q8_0, y, (hipStream_t)stream));
}

int w4a8_gemv_f32(const void *w, const float *x, float *y, int rows, int k, void *stream) {
    if (int s = check_gemv(w, x, y, rows, k, 16)) return s;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), x, X_F32, y, (hipStream_t)stream));
}

size_t w4a8_argmax_workspace_bytes(void) { return argmax_workspace_bytes(); }

int w4a8_gemv_f32_argmax(const void *w, const float *x, float *y, int rows, int k, int32_t *argmax,
                         void *workspace, size_t workspace_bytes, void *stream) {
    if (int s = check_gemv(w, x, y, rows, k, 16)) return s;
    if (!argmax || !workspace) return W4A8_ERR_NULL;
    if (!aligned(argmax, 4) || !aligned(workspace, 16)) return W4A8_ERR_ALIGN;
    if (workspace_bytes < argmax_workspace_bytes()) return W4A8_ERR_SHAPE;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), x, X_F32, y, (hipStream_t)stream, argmax, workspace));
}

int w4a8_gemv_gate_up_silu(const void *w, const float *x, const float *norm_w, float eps, float *act, int rows,
                           int k, void *stream) {
    if (int s = check_gemv(w, x, act, rows, k, 16)) return s;
    if (gate_up_silu_waves(rows, k) == 0) return W4A8_ERR_SHAPE;
    if (norm_w && !aligned(norm_w, 16)) return W4A8_ERR_ALIGN;
    XAux aux;
    aux.norm_w = norm_w;
    aux.eps = eps;
    return hip_status(launch_gemv_gate_up_silu(static_cast<const uint8_t *>(w), x, norm_w ? X_RMS : X_F32, act, rows,
                                               k, (hipStream_t)stream, aux));
}

int w4a8_gemv_gate_up_silu_q8_0(const void *w, const float *x, const float *norm_w, float eps, void *act_engine,
                                int rows, int k, void *stream) {
    if (int s = check_gemv(w, x, static_cast<const float *>(act_engine), rows, k, 16)) return s;
    if (!gate_up_silu_q8_fits(rows, k)) return W4A8_ERR_SHAPE;
    if (!aligned(act_engine, 16) || (norm_w && !aligned(norm_w, 16))) return W4A8_ERR_ALIGN;
    XAux aux;
    aux.norm_w = norm_w;
    aux.eps = eps;
    return hip_status(launch_gemv_gate_up_silu(static_cast<const uint8_t *>(w), x, norm_w ? X_RMS : X_F32, act_engine,
                                               rows, k, (hipStream_t)stream, aux, true));
}

size_t w4a8_topk_workspace_bytes(int n) { return topk_workspace_bytes(n); }

int w4a8_topk(const float *y, int n, int k, float *vals, int32_t *idx, void *workspace, size_t workspace_bytes,
              void *stream) {
    if (!y || !vals || !idx || !workspace) return W4A8_ERR_NULL;
    if (n < 1 || n > topk_max_n() || k < 1 || k > 64) return W4A8_ERR_SHAPE;
    if (!aligned(y, 4) || !aligned(vals, 4) || !aligned(idx, 4) || !aligned(workspace, 8)) return W4A8_ERR_ALIGN;
    if (workspace_bytes < topk_workspace_bytes(n)) return W4A8_ERR_SHAPE;
    return hip_status(launch_topk(y, n, k, vals, idx, workspace, (hipStream_t)stream));
}

int w4a8_topk_no_alloc(const float *y, int n, int k, float *vals, int32_t *idx, void *stream) {
    if (!y || !vals || !idx) return W4A8_ERR_NULL;
    if (n < 1 || n > W4A8_TOPK_NO_ALLOC_MAX_N || k < 1 || k > 64) return W4A8_ERR_SHAPE;
    if (!aligned(y, 4) || !aligned(vals, 4) || !aligned(idx, 4)) return W4A8_ERR_ALIGN;
    return hip_status(launch_topk_no_alloc(y, n, k, vals, idx, (hipStream_t)stream));
}

// The fused rmsnorm stages x's float64 squares in LDS: k <= 8192.
constexpr int RMS_FUSED_MAX_K = 8192;

int w4a8_gemv_rmsnorm(const void *w, const float *x, const float *norm_w, float eps, float *y, int rows, int k,
                      void *stream) {
    if (int s = check_gemv(w, x, y, rows, k, 16)) return s;
    if (k > RMS_FUSED_MAX_K) return W4A8_ERR_SHAPE;
    if (!norm_w) return W4A8_ERR_NULL;
    if (!aligned(norm_w, 16)) return W4A8_ERR_ALIGN;
    XAux aux;
    aux.norm_w = norm_w;
    aux.eps = eps;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), x, X_RMS, y, (hipStream_t)stream, nullptr, nullptr, aux));
}

int w4a8_gemv_rmsnorm_argmax(const void *w, const float *x, const float *norm_w, float eps, float *y, int rows, int k,
                             int32_t *argmax, void *workspace, size_t workspace_bytes, void *stream) {
    if (int s = check_gemv(w, x, y, rows, k, 16)) return s;
    if (k > RMS_FUSED_MAX_K) return W4A8_ERR_SHAPE;
    if (!norm_w || !argmax || !workspace) return W4A8_ERR_NULL;
    if (!aligned(norm_w, 16) || !aligned(argmax, 4) || !aligned(workspace, 16)) return W4A8_ERR_ALIGN;
    if (workspace_bytes < argmax_workspace_bytes()) return W4A8_ERR_SHAPE;
    XAux aux;
    aux.norm_w = norm_w;
    aux.eps = eps;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), x, X_RMS, y, (hipStream_t)stream, argmax, workspace, aux));
}

int w4a8_gemv_silu_mul(const void *w, const float *gate_up, float *y, int rows, int k, void *stream) {
    if (int s = check_gemv(w, gate_up, y, rows, k, 16)) return s;
    return hip_status(launch_gemv_m1(plain_matrix(w, rows, k), gate_up, X_SILU, y, (hipStream_t)stream));
}

int w4a8_rmsnorm_q8_0(const float *x, const float *norm_w, float eps, void *out_engine, int k, int m, void *stream) {
    if (!x || !norm_w || !out_engine) return W4A8_ERR_NULL;
    if (check_k(k) || m < 1) return W4A8_ERR_SHAPE;
    if (!aligned(x, 16) || !aligned(norm_w, 16) || !aligned(out_engine, 16)) return W4A8_ERR_ALIGN;
    return hip_status(launch_rmsnorm_q8_0(x, norm_w, eps, k, m, static_cast<uint8_t *>(out_engine), (hipStream_t)stream));
}

int w4a8_silu_mul_q8_0(const float *gate_up, void *out_engine, int k, int m, void *stream) {
    if (!gate_up || !out_engine) return W4A8_ERR_NULL;
    if (check_k(k) || m < 1) return W4A8_ERR_SHAPE;
    if (!aligned(gate_up, 16) || !aligned(out_engine, 16)) return W4A8_ERR_ALIGN;
    return hip_status(launch_silu_mul_q8_0(gate_up, k, m, static_cast<uint8_t *>(out_engine), (hipStream_t)stream));
}

int w4a8_gemv_quarters(const void *const w[4], const void *x, float *y, int rows, int k, void *stream) {
    if (!w) return W4A8_ERR_NULL;
    for (int q = 0; q < 4; ++q) {
        if (!w[q]) return W4A8_ERR_NULL;
        if (!aligned(w[q], 16)) return W4A8_ERR_ALIGN;
    }
    if (rows % 4) return W4A8_ERR_SHAPE;
    if (int s = check_gemv(w[0], x, y, rows, k, 16)) return s;
    MatrixRef m{};
    for (int q = 0; q < 4; ++q) m.seg[q] = static_cast<const uint8_t *>(w[q]);
    m.nseg = 4;
    m.seg_rows = rows / 4;
    m.rows = rows;
    m.k = k;
    return hip_status(launch_gemv_m1(m, x, X_ENGINE, y, (hipStream_t)stream));
}

int w4a8_quantize_q8_0(const float *x, void *out_engine, int k, int m, void *stream) {
    if (!x || !out_engine) return W4A8_ERR_NULL;
    if (check_k(k) || m < 1) return W4A8_ERR_SHAPE;
    if (!aligned(x, 16) || !aligned(out_engine, 16)) return W4A8_ERR_ALIGN;
    return hip_status(launch_quantize_q8_0(x, k, m, static_cast<uint8_t *>(out_engine), X_ENGINE, (hipStream_t)stream));
}

int w4a8_quantize_q8_0_blocks(const float *x, void *out_blocks, int k, int m, void *stream) {
    if (!x || !out_blocks) return W4A8_ERR_NULL;
    if (check_k(k) || m < 1) return W4A8_ERR_SHAPE;
    if (!aligned(x, 16) || !aligned(out_blocks, 2)) return W4A8_ERR_ALIGN;
    return hip_status(launch_quantize_q8_0(x, k, m, static_cast<uint8_t *>(out_blocks), X_Q8_0, (hipStream_t)stream));
}

int w4a8_quantize_q4_0(const float *w, void *out_blocks, int rows, int k, void *stream) {
    if (!w || !out_blocks) return W4A8_ERR_NULL;
    if (k < 32 || k % 32 || rows < 1) return W4A8_ERR_SHAPE;
    if (!aligned(w, 16) || !aligned(out_blocks, 2)) return W4A8_ERR_ALIGN;
    return hip_status(launch_quantize_q4_0(w, rows, k, static_cast<uint8_t *>(out_blocks), (hipStream_t)stream));
}

int w4a8_gemm(const void *w, const void *x_rows, float *y, int m, int rows, int k, void *stream) {
    if (int s = check_gemv(w, x_rows, y, rows, k, 16)) return s;
    if (m < 1 || m > 4096) return W4A8_ERR_SHAPE;
    return hip_status(launch_gemm(plain_matrix(w, rows, k), static_cast<const uint8_t *>(x_rows), m, y,
                                  (hipStream_t)stream));
}

int w4a8_chain_gemv(const w4a8_chain_step *steps, int n, void *stream) {
    if (!steps) return W4A8_ERR_NULL;
    if (n < 1 || n > W4A8_CHAIN_MAX_STEPS) return W4A8_ERR_SHAPE;
    for (int i = 0; i < n; ++i) {
        if (int s = check_gemv(steps[i].w, steps[i].x, steps[i].y, steps[i].rows, steps[i].k, 16)) return s;
        if (step_in_place(steps[i])) return W4A8_ERR_SHAPE;
    }
    return hip_status(launch_chain(steps, n, (hipStream_t)stream));
}

int w4a8_chain_plan_create_steps(const w4a8_plan_step *steps, int n, w4a8_chain_plan **plan) {
    if (!steps || !plan) return W4A8_ERR_NULL;
    *plan = nullptr;
    if (n < 1 || n > W4A8_CHAIN_MAX_STEPS) return W4A8_ERR_SHAPE;
    // The checks of the stream entry point each step stands for.
    for (int i = 0; i < n; ++i) {
        const w4a8_plan_step &s = steps[i];
        if (int st = check_gemv(s.w, s.x, static_cast<const float *>(s.y), s.rows, s.k, 16)) return st;
        if (s.k < 2048 || s.kind < W4A8_PLAN_GEMV || s.kind > W4A8_PLAN_GEMV_ENGINE) return W4A8_ERR_SHAPE;
        if (s.norm_w) {
            if (s.k > RMS_FUSED_MAX_K || s.kind == W4A8_PLAN_GEMV_ENGINE) return W4A8_ERR_SHAPE;
            if (!aligned(s.norm_w, 16)) return W4A8_ERR_ALIGN;
        }
        if (s.kind == W4A8_PLAN_GATE_UP_SILU && gate_up_silu_waves(s.rows, s.k) == 0) return W4A8_ERR_SHAPE;
        if (s.kind == W4A8_PLAN_GATE_UP_SILU_Q8) {
            if (!gate_up_silu_q8_fits(s.rows, s.k)) return W4A8_ERR_SHAPE;
            if (!aligned(s.y, 16)) return W4A8_ERR_ALIGN;
        }
        if (s.kind == W4A8_PLAN_ARGMAX) {
            if (!s.argmax || !s.workspace) return W4A8_ERR_NULL;
            if (!aligned(s.argmax, 4) || !aligned(s.workspace, 16)) return W4A8_ERR_ALIGN;
        }
    }
    if (int st = plan_check_ranges(steps, n)) return st;
    hipError_t he = hipSuccess;
    const int st = chain_plan_create(steps, n, false, plan, he);
    return st == W4A8_ERR_HIP ? hip_status(he) : st;
}

int w4a8_chain_plan_create_overlapped(const w4a8_chain_step *steps, int n, w4a8_chain_plan **plan) {
    if (!steps || !plan) return W4A8_ERR_NULL;
    *plan = nullptr;
    if (n < 1 || n > W4A8_CHAIN_MAX_STEPS) return W4A8_ERR_SHAPE;
    w4a8_plan_step ps[W4A8_CHAIN_MAX_STEPS] = {};
    for (int i = 0; i < n; ++i) {
        if (int s = check_gemv(steps[i].w, steps[i].x, steps[i].y, steps[i].rows, steps[i].k, 16)) return s;
        if (steps[i].k < 2048) return W4A8_ERR_SHAPE;
        ps[i] = w4a8_plan_step{W4A8_PLAN_GEMV, steps[i].w, steps[i].x, steps[i].y, steps[i].rows, steps[i].k,
                               nullptr, 0.0f, nullptr, nullptr};
    }
    if (int st = plan_check_ranges(ps, n)) return st;
    hipError_t he = hipSuccess;
    const int st = chain_plan_create(ps, n, true, plan, he);
    return st == W4A8_ERR_HIP ? hip_status(he) : st;
}

int w4a8_chain_plan_create(const w4a8_chain_step *steps, int n, w4a8_chain_plan **plan) {
    if (!steps || !plan) return W4A8_ERR_NULL;
    *plan = nullptr;
    if (n < 1 || n > W4A8_CHAIN_MAX_STEPS) return W4A8_ERR_SHAPE;
    w4a8_plan_step ps[W4A8_CHAIN_MAX_STEPS] = {};
    for (int i = 0; i < n; ++i)
        ps[i] = w4a8_plan_step{W4A8_PLAN_GEMV, steps[i].w, steps[i].x, steps[i].y, steps[i].rows, steps[i].k,
                               nullptr, 0.0f, nullptr, nullptr};
    return w4a8_chain_plan_create_steps(ps, n, plan);
}

int w4a8_chain_plan_launch(w4a8_chain_plan *plan, int passes) {
    if (!plan) return W4A8_ERR_NULL;
    if (passes < 1 || passes > (1 << 20)) return W4A8_ERR_SHAPE;
    return chain_plan_launch(plan, passes);
}

long w4a8_chain_plan_workgroups(const w4a8_chain_plan *plan, int step) {
    if (!plan) return W4A8_ERR_NULL;
    if (step < -1 || step >= chain_plan_steps(plan)) return W4A8_ERR_SHAPE;
    return chain_plan_workgroups(plan, step);
}

int w4a8_chain_plan_launch_timed(w4a8_chain_plan *plan, int passes, uint64_t *stamps) {
    if (!plan || !stamps) return W4A8_ERR_NULL;
    if (passes < 1 || (long long)passes * chain_plan_workgroups(plan, -1) > W4A8_PLAN_TIMED_MAX_SLOTS)
        return W4A8_ERR_SHAPE;
    if (!aligned(stamps, 16)) return W4A8_ERR_ALIGN;
    hipError_t he = hipSuccess;
    const int st = chain_plan_launch_timed(plan, passes, reinterpret_cast<unsigned long long *>(stamps), he);
    return st == W4A8_ERR_HIP ? hip_status(he) : st;
}

int w4a8_wall_clock_hz(int64_t *hz) {
    if (!hz) return W4A8_ERR_NULL;
    *hz = 0;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess) return W4A8_ERR_NODEV;
    if (int s = hip_status(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev))) return s;
    if (khz <= 0) return W4A8_ERR_NODEV;
    *hz = (int64_t)khz * 1000;
    return W4A8_OK;
}

int w4a8_chain_plan_wait(w4a8_chain_plan *plan, int timeout_ms) {
    if (!plan) return W4A8_ERR_NULL;
    return chain_plan_wait(plan, timeout_ms < 0 ? 0 : timeout_ms);
}

int w4a8_chain_plan_destroy(w4a8_chain_plan *plan) {
    if (!plan) return W4A8_OK;
    return chain_plan_destroy(plan);
}

int w4a8_chain_set_mode(int mode) {
    if (mode != W4A8_CHAIN_ONE_LAUNCH && mode != W4A8_CHAIN_PER_STEP) return W4A8_ERR_SHAPE;
    chain_set_mode(mode);
    return W4A8_OK;
}

int w4a8_chain_set_spin_limit(int polls) {
    chain_set_spin_limit(polls);
    return W4A8_OK;
}

int w4a8_chain_timeouts(void) {
    int n = 0;
    if (int s = hip_status(chain_take_timeouts(&n))) return s;
    return n;
}

int w4a8_gemv_batch(const w4a8_chain_step *steps, int n, void *stream) {
    if (!steps) return W4A8_ERR_NULL;
    if (n < 1 || n > W4A8_CHAIN_MAX_STEPS) return W4A8_ERR_SHAPE;
    for (int i = 0; i < n; ++i)
        if (int s = check_gemv(steps[i].w, steps[i].x, steps[i].y, steps[i].rows, steps[i].k, 16)) return s;
    // Every entry runs at once: no output may overlap any entry's input or
    // another entry's output.
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
            const w4a8_chain_step &a = steps[i], &b = steps[j];
            const size_t ya = 4 * (size_t)a.rows;
            const size_t wb = (size_t)b.rows * (size_t)(b.k / 32) * 18;
            if (overlaps(a.y, ya, b.x, 4 * (size_t)b.k) || overlaps(a.y, ya, b.w, wb) ||
                (i != j && overlaps(a.y, ya, b.y, 4 * (size_t)b.rows)))
                return W4A8_ERR_SHAPE;
        }
    return hip_status(launch_gemv_batch(steps, n, (hipStream_t)stream));
}

}  // extern "C"
