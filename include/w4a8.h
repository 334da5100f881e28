/*
 * w4a8.h -- native C ABI of the MI355X W4A8 engine (libkv260gemv.so).
 *
 * y = W x with W in ggml Q4_0 (18-byte blocks: fp16 scale d little-endian,
 * then 16 bytes whose byte j holds weight j in the low nibble and weight j+16
 * in the high nibble, value (n - 8) * d) and x in Q8_0, computed byte-for-byte
 * in the order src/llm_kv260/q4_0.py:151-182 fixes: exact int32 block dots,
 * t = (f32(sumi) * f32(d_w)) * f32(d_x), eight fp32 lanes accumulated in block
 * order, adjacent-pair tree.
 *
 * Every pointer argument is a device address (HBM; hipMalloc, torch, or the
 * udmabuf pools of udmabuf.h). `stream` is a hipStream_t (NULL = the null
 * stream of the current device). Calls enqueue work and return; nothing is
 * allocated per call. Shapes and alignment are checked before anything is
 * enqueued; a failed check returns a negative status and enqueues nothing.
 *
 * Shape rules: k % 256 == 0 (whole 8-block lane groups, q4_0.py:166-167),
 * 256 <= k <= 16384, rows >= 1. Alignment: W and x 16 bytes (the engine's
 * 16-byte vector loads; ggml and GGUF align tensor data to 32), y 4 bytes.
 */
#ifndef W4A8_H
#define W4A8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A8_QK 32
#define W4A8_Q4_0_BYTES 18
#define W4A8_Q8_0_BYTES 34
#define W4A8_LANES 8
#define W4A8_MAX_K 16384

enum w4a8_status {
    W4A8_OK = 0,
    W4A8_ERR_NULL = -1,    /* a required pointer is NULL */
    W4A8_ERR_SHAPE = -2,   /* k or rows (or m) outside the rules above */
    W4A8_ERR_ALIGN = -3,   /* a pointer is not aligned as required */
    W4A8_ERR_HIP = -4,     /* the HIP runtime reported an error (w4a8_last_hip_error) */
    W4A8_ERR_NODEV = -5,   /* no usable gfx950 device */
    /* -6: W4A8_ERR_FORMAT (w4a8_gguf.h) */
    W4A8_ERR_TIMEOUT = -7, /* a bounded wait ran out (w4a8_chain_plan_wait) */
    W4A8_ERR_HSA = -8,     /* the HSA runtime refused a queue, code object or signal */
};

/* "llm-kv260/w4a8-q4_0-v2": the contract these kernels are held to
 * (replaces CONTRACT_VERSION, src/llm_kv260/q4_0.py:64). */
const char *w4a8_contract_version(void);
const char *w4a8_strerror(int status);
/* The hipError_t value behind the last W4A8_ERR_HIP of this thread. */
int w4a8_last_hip_error(void);

/* Bytes of one Q4_0 row, of one engine-layout activation (int8[k] then
 * float32[k/32]) and of one row of Q8_0 blocks. */
size_t w4a8_q4_0_row_bytes(int k);
size_t w4a8_engine_x_bytes(int k);
size_t w4a8_q8_0_row_bytes(int k);

/* y[rows] = W[rows, k] x, x in the engine layout int8[k] | float32[k/32]
 * (pack_x_for_engine, src/llm_kv260/q4_0.py:193-200). The call the v1 engine
 * made with gemv_dev_run (board/kv260gemv/gemv_dev.h:19-23), now with the
 * drop-in argument order gemv(weights, activation, out, rows, cols). */
int w4a8_gemv(const void *w, const void *x, float *y, int rows, int k, void *stream);

/* Same, x as ggml Q8_0 blocks (34 bytes each: fp16 d then 32 int8). x needs
 * only 2-byte alignment. */
int w4a8_gemv_q8_0(const void *w, const void *x_blocks, float *y, int rows, int k, void *stream);

/* Same, x as float32[k], quantized to Q8_0 inside the GEMV kernel
 * (gemv_q4_0_f32, src/llm_kv260/q4_0.py:185-188). */
int w4a8_gemv_f32(const void *w, const float *x, float *y, int rows, int k, void *stream);

/* The LM head with its greedy pick in one launch: y = W x as w4a8_gemv_f32,
 * and *argmax (device int32) = the first row of the largest y, the reference's
 * "if (y[i] > y[best]) best = i" scan (board/tp/tp_llama.cpp:879-880): ties go
 * to the smaller row, -0 equals +0, a NaN is never picked, and a NaN at row 0
 * gives 0 as the scan does. Each workgroup reduces its rows and the last one
 * to finish reduces the workgroups' results, through `workspace`: device
 * memory of w4a8_argmax_workspace_bytes() bytes, 16-byte aligned, zero-filled
 * once before its first use (every call leaves it zero again). Calls that
 * share a workspace must not run concurrently. */
size_t w4a8_argmax_workspace_bytes(void);
int w4a8_gemv_f32_argmax(const void *w, const float *x, float *y, int rows, int k, int32_t *argmax,
                         void *workspace, size_t workspace_bytes, void *stream);

/* The sampler's candidates (board/tp/tp_llama.cpp:894-909): the k best
 * logits of y[0..n), 1 <= k <= 64, as vals[k] / idx[k] in the order the
 * reference's insertion sort leaves them: values descending, among equal
 * values (-0 equal to +0) the smaller index first, and a value at or below
 * -1e30 never admitted; slots left over hold {-1e30, 0} as there. vals are
 * y's own values (bit for bit). NaN logits are handled as the reference's
 * loop handles them: a NaN takes the last slot (v <= NaN is false), evicting
 * the k-th candidate held at that point, and the next logit then enters
 * whatever its value, so a NaN can be a candidate and can cost one. When y
 * holds a NaN the second launch runs that loop itself, in order, in one
 * wave (slower: a sequential pass over y). Two launches
 * through `workspace`: w4a8_topk_workspace_bytes(n) bytes of device memory,
 * 8-byte aligned, overwritten by each call. 1 <= n <= 262144. */
size_t w4a8_topk_workspace_bytes(int n);
int w4a8_topk(const float *y, int n, int k, float *vals, int32_t *idx, void *workspace, size_t workspace_bytes,
              void *stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc): w4a8_topk with its workspace in the library's own device
 * array, one per device (128 KiB, held until the process ends), so the call
 * allocates nothing. Same candidates, bit for bit, as w4a8_topk.
 * 1 <= n <= W4A8_TOPK_NO_ALLOC_MAX_N (larger n: W4A8_ERR_SHAPE), 1 <= k <= 64.
 * The array belongs to the device current at the call; every call on that
 * device shares it, so calls that overlap on one device (two streams, two
 * threads) race and may return wrong candidates: serialize them (replays of
 * a graph that captured the call share it too). The call may be captured
 * into a HIP graph, the first call on a device included: that call looks up
 * the array's address with this thread's capture mode relaxed for the
 * lookup. */
#define W4A8_TOPK_NO_ALLOC_MAX_N 262144
int w4a8_topk_no_alloc(const float *y, int n, int k, float *vals, int32_t *idx, void *stream);

/* The reference's producers of the GEMV input, fused into the GEMV's own
 * activation staging (board/tp/tp_llama.cpp, computed as it does):
 *   rmsnorm (:557-569): h = x * (1 / sqrtf((float)(ss / k) + eps)) * norm_w,
 *     ss the float64 sum of x_i^2 in four lanes (i % 4, increasing i), met as
 *     (l0 + l2) + (l1 + l3); the input of q|k|v, gate|up and the LM head
 *     (:828-830, :854-856, :878-879). y = W Q8_0(h).
 *   silu_mul (:612-619): a = silu(gate) * up with gate_up = gate | up,
 *     float32[2k] (the gate|up GEMV's output), silu(g) = g / (1 + expf(-g))
 *     through ggml's vector expf; the input of down (:858-860). y = W Q8_0(a).
 * Each is byte-identical to the standalone producer below followed by
 * w4a8_gemv. x, norm_w and gate_up 16-byte aligned; the fused rmsnorm takes
 * k <= 8192 (its float64 squares are staged in LDS), the standalone one any k.
 * The float64 sum is n / 4 dependent adds whatever the hardware: about 8 ns
 * each here, the latency the reference's summation order costs. */
int w4a8_gemv_rmsnorm(const void *w, const float *x, const float *norm_w, float eps, float *y, int rows, int k,
                      void *stream);
int w4a8_gemv_rmsnorm_argmax(const void *w, const float *x, const float *norm_w, float eps, float *y, int rows, int k,
                             int32_t *argmax, void *workspace, size_t workspace_bytes, void *stream);
/* silu(gate) * up in down's own staging: the same bytes as w4a8_silu_mul_q8_0
 * then w4a8_gemv, but slower than that pair and than w4a8_gemv_gate_up_silu
 * (each workgroup recomputes all k exponentials); prefer those. */
int w4a8_gemv_silu_mul(const void *w, const float *gate_up, float *y, int rows, int k, void *stream);

/* The gate|up GEMV with silu as its epilogue: y = W Q8_0(h) over rows = 2n
 * (gate rows, then up rows, as the reference fuses them, tp_llama.cpp:258-268)
 * with h = rmsnorm(x) * norm_w as w4a8_gemv_rmsnorm (norm_w != NULL) or
 * h = x (norm_w NULL), and act[i] = silu(y[i]) * y[n + i] (tp_llama.cpp:612-
 * 619, ggml's vector expf) written in place of y: float32[n], the activation
 * of down. Byte-identical to that GEMV followed by silu_mul, with silu
 * computed once per output instead of by every workgroup of down.
 * 2048 <= k <= 8192, n a multiple of r = 64 / (k / 256) rows (whole tiles of
 * r rows in each half), and the n / r tiles of each half a multiple of 2 when
 * k > 4096 (a workgroup pairs V gate tiles with their V up tiles, one per
 * wave, V dividing the half, and holds one thread per activation block);
 * other shapes return W4A8_ERR_SHAPE. */
int w4a8_gemv_gate_up_silu(const void *w, const float *x, const float *norm_w, float eps, float *act, int rows, int k,
                           void *stream);

/* The same with act quantized to Q8_0 in the epilogue: act_engine receives
 * the engine layout of the n values (int8[n] | float32[n / 32], 16-byte
 * aligned; n + n / 8 bytes), byte-identical to w4a8_gemv_gate_up_silu then
 * w4a8_quantize_q8_0 -- the input of w4a8_gemv for down, as the
 * reference's caller quantizes x before each engine call
 * (tp_llama.cpp:330-352). Down then reads n + n / 8 bytes instead of 4n.
 * k = 2048 only, and the n / 8 tiles of each half a multiple of 4 (a
 * workgroup's 32 outputs are one Q8_0 block); other shapes return
 * W4A8_ERR_SHAPE. No counterpart in the reference (its host quantizes). */
int w4a8_gemv_gate_up_silu_q8_0(const void *w, const float *x, const float *norm_w, float eps, void *act_engine,
                                int rows, int k, void *stream);

/* The same producers on their own, m rows, quantized to the engine layout
 * (row stride w4a8_engine_x_bytes(k)): the input of w4a8_gemv / w4a8_gemm. */
int w4a8_rmsnorm_q8_0(const float *x, const float *norm_w, float eps, void *out_engine, int k, int m, void *stream);
int w4a8_silu_mul_q8_0(const float *gate_up, void *out_engine, int k, int m, void *stream);

/* Four row quarters at their own addresses, rows/4 contiguous rows each,
 * y contiguous (gemv_dev_start4, board/kv260gemv/gemv_dev.h:29-35). rows % 4 == 0. */
int w4a8_gemv_quarters(const void *const w[4], const void *x, float *y, int rows, int k, void *stream);

/* Fused Q8_0 activation quantizer (q4_0.py:83-97; the caller's quantize_x,
 * board/tp/tp_llama.cpp:330-352): m rows of float32[k] -> m rows of the engine
 * layout (row stride w4a8_engine_x_bytes(k)). x and out 16-byte aligned. */
int w4a8_quantize_q8_0(const float *x, void *out_engine, int k, int m, void *stream);

/* Same quantizer, output as ggml Q8_0 blocks (row stride w4a8_q8_0_row_bytes(k)). */
int w4a8_quantize_q8_0_blocks(const float *x, void *out_blocks, int k, int m, void *stream);

/* Q4_0 weight quantizer (quantize_q4_0, src/llm_kv260/q4_0.py:100-121):
 * float32[rows][k] -> Q4_0 rows. For building matrices on the device. */
int w4a8_quantize_q4_0(const float *w, void *out_blocks, int rows, int k, void *stream);

/* Batched M > 1 (prefill): y[m][rows] = W x_i for m activation rows, each
 * byte-identical to w4a8_gemv on that row alone. x rows in the engine layout,
 * stride w4a8_engine_x_bytes(k). 1 <= m <= 4096. Int8 MFMA with exact
 * per-block int32 sums, then the same fp32 epilogue per (row, token). */
int w4a8_gemm(const void *w, const void *x_rows, float *y, int m, int rows, int k, void *stream);

/* One matrix of a decode step's GEMV chain: y = W x with x given as
 * float32[k] and quantized to Q8_0 inside the engine right before the GEMV. */
typedef struct w4a8_chain_step {
    const void *w;     /* Q4_0 rows, 16-byte aligned */
    const float *x;    /* float32[k], 16-byte aligned */
    float *y;          /* float32[rows] */
    int rows;
    int k;
} w4a8_chain_step;

#define W4A8_CHAIN_MAX_STEPS 96

/* A token's matrices in order (board/tp/tp_llama.cpp:822-883: per layer
 * q|k|v, o, gate|up, down, then the LM head; 65 engine calls per token).
 * Step j reads its activation only after every row of step j-1's output is
 * written, so x_j may be (or be computed from) an earlier y; each step
 * equals w4a8_gemv_f32 on its own, byte for byte. 1 <= n <=
 * W4A8_CHAIN_MAX_STEPS. A step whose y overlaps its own x or weights is
 * refused (W4A8_ERR_SHAPE): its workgroups would race. Steps may share
 * output bytes; the later step's win.
 *
 * By default (W4A8_CHAIN_PER_STEP) each step is one kernel, in stream order.
 * In W4A8_CHAIN_ONE_LAUNCH mode, a chain whose every k is in 2048..8192 is
 * one cooperative launch instead: a workgroup per CU whose fetch waves
 * stream the weights of the following matrices into LDS while its MAC
 * waves compute the current one (the gemv2 engine's fetch / MAC split and
 * the caller's prefetch of the next matrix, board/kv260gemv/gemv2_dev.h:
 * 40-44, board/tp/tp_llama.cpp:364-368), with a grid barrier between steps.
 * On MI355X that barrier, the activation staging it exposes and the skew
 * between workgroups cost more per step than a kernel boundary, so the
 * one-launch form is the slower one for the Llama-3.2-1B chain (its LM head
 * alone is faster, its weights streamed during the last layer). One-launch
 * chains on one device share that device's barrier state: they must not
 * run concurrently (one stream per device, as the reference's single
 * in-flight engine call), and the first one on a device allocates the state
 * (64 KB), so it must not be inside a stream capture (such a call runs per
 * step instead). */
int w4a8_chain_gemv(const w4a8_chain_step *steps, int n, void *stream);

/* How w4a8_chain_gemv runs, for every later call in this process:
 * W4A8_CHAIN_PER_STEP (the default) or W4A8_CHAIN_ONE_LAUNCH. */
#define W4A8_CHAIN_ONE_LAUNCH 0
#define W4A8_CHAIN_PER_STEP 1
int w4a8_chain_set_mode(int mode);

/* The one-launch chain's waits are bounded: a workgroup that polls the
 * barrier this many times (~0.5 us each; default 4,194,304) gives up, every
 * workgroup then skips the rest of the launch (its outputs are not valid)
 * and the last one out restores the barrier state. w4a8_chain_timeouts
 * returns how many launches on the current device gave up since its last
 * call and clears the count (synchronous: waits for the device); it is 0
 * whenever every launch completed. A limit <= 0 restores the default. */
int w4a8_chain_set_spin_limit(int polls);
int w4a8_chain_timeouts(void);

/* The same chain as a plan: made once, then launched any number of times.
 * Each launch runs `passes` passes over the n steps, step j + 1 of a pass
 * after step j, pass after pass, with the kernel of the per-step chain (every
 * y byte-identical to w4a8_chain_gemv's). The steps are dispatched as raw
 * AQL packets on a queue of the library's own (one per device), with no
 * cache fences between consecutive steps: an output that a step of the plan
 * reads is written through to the device's coherence point and read from
 * there, found by comparing the steps' ranges when the plan is made. That
 * saves the two fences the HIP runtime puts around every kernel of a stream
 * or graph. It is not ordered with HIP streams, as the reference's engine is
 * driven by start and wait calls (board/kv260gemv/gemv2_dev.h:40-44):
 *   - create: steps as for w4a8_chain_gemv, every k in 2048..W4A8_MAX_K; the
 *     plan belongs to the current device and keeps the pointers (the
 *     buffers must stay allocated, their contents may change between
 *     launches); 1 <= n <= W4A8_CHAIN_MAX_STEPS;
 *   - launch: returns once the packets are written; whatever writes the
 *     plan's x or weights must be complete before it (e.g.
 *     hipStreamSynchronize); 1 <= passes <= 1 << 20;
 *   - wait: until every launch of the plan so far is done, at most
 *     timeout_ms (W4A8_ERR_TIMEOUT); after W4A8_OK the outputs are visible
 *     to the host and to any later HIP work;
 *   - destroy: waits (at most 10 s) and frees the plan.
 * Launches of plans on one device go to that device's queue in call order.
 * A launch that finds the queue full waits for the device to take packets;
 * if the device takes none for 10 s it is stalled: the launch returns
 * W4A8_ERR_TIMEOUT, the plan's wait and destroy keep reporting the timeout
 * (its argument blocks stay allocated, since queued packets point at them),
 * and every later launch on that device fails at once.
 * Outputs: a step's y may be another step's x (in the same pass or the
 * next) and may share bytes with other steps' y (the later step's bytes
 * win, as in a stream); create refuses (W4A8_ERR_SHAPE) a step whose x
 * overlaps its own y, and any step's weights, norm_w, argmax or workspace
 * that overlap a step's y. */
typedef struct w4a8_chain_plan w4a8_chain_plan;
int w4a8_chain_plan_create(const w4a8_chain_step *steps, int n, w4a8_chain_plan **plan);

/* A plan whose steps may carry the producers either side of the GEMV, each
 * step byte-identical to the stream entry point it names:
 *   W4A8_PLAN_GEMV            w4a8_gemv_f32, or w4a8_gemv_rmsnorm when
 *                             norm_w is set (k <= 8192);
 *   W4A8_PLAN_GATE_UP_SILU    w4a8_gemv_gate_up_silu: y = silu(gate) * up,
 *                             float32[rows / 2] (its shape rules);
 *   W4A8_PLAN_ARGMAX          w4a8_gemv_f32_argmax, or w4a8_gemv_rmsnorm_argmax
 *                             when norm_w is set: *argmax = the row picked,
 *                             through `workspace` (w4a8_argmax_workspace_bytes(),
 *                             zero before the first launch; the step leaves
 *                             it zero);
 *   W4A8_PLAN_GATE_UP_SILU_Q8 w4a8_gemv_gate_up_silu_q8_0: y = the engine
 *                             layout of silu(gate) * up, rows / 2 values
 *                             (k = 2048, its shape rules);
 *   W4A8_PLAN_GEMV_ENGINE     w4a8_gemv: x in the engine layout
 *                             (int8[k] | float32[k / 32]), norm_w NULL --
 *                             down after W4A8_PLAN_GATE_UP_SILU_Q8.
 * Every k in 2048..W4A8_MAX_K; the rest as w4a8_chain_plan_create (which is
 * this with every step a W4A8_PLAN_GEMV without norm_w), with the same
 * rules for outputs: a step may read an earlier (or, over passes, a later)
 * step's y; weights, norm_w, argmax and the workspace must not overlap any
 * step's y (W4A8_ERR_SHAPE). */
#define W4A8_PLAN_GEMV 0
#define W4A8_PLAN_GATE_UP_SILU 1
#define W4A8_PLAN_ARGMAX 2
#define W4A8_PLAN_GATE_UP_SILU_Q8 3
#define W4A8_PLAN_GEMV_ENGINE 4
typedef struct w4a8_plan_step {
    int kind;
    const void *w;          /* Q4_0 rows, 16-byte aligned */
    const void *x;          /* float32[k] (GEMV_ENGINE: the engine layout), 16-byte aligned */
    void *y;                /* float32[rows] (gate|up: [rows / 2]; _Q8: its engine layout) */
    int rows;
    int k;
    const float *norm_w;    /* float32[k], 16-byte aligned, or NULL */
    float eps;
    int32_t *argmax;        /* W4A8_PLAN_ARGMAX only */
    void *workspace;        /* W4A8_PLAN_ARGMAX only, 16-byte aligned */
} w4a8_plan_step;
int w4a8_chain_plan_create_steps(const w4a8_plan_step *steps, int n, w4a8_chain_plan **plan);
int w4a8_chain_plan_launch(w4a8_chain_plan *plan, int passes);
int w4a8_chain_plan_wait(w4a8_chain_plan *plan, int timeout_ms);
int w4a8_chain_plan_destroy(w4a8_chain_plan *plan);

/* The same chain as a plan whose steps overlap: step j + 1's dispatch goes
 * out without the barrier bit, so its workgroups start while step j still
 * runs and issue their weight loads at once (weights never depend on the
 * chain); each then waits, inside the kernel, until every workgroup of step
 * j has stored its outputs and its flag (device-coherent flag bytes, one
 * per workgroup), and only then reads x. The first step of each pass keeps
 * the barrier bit, so passes never overlap. This is the GPU form of the
 * reference engine fetching the next matrix during the current MAC
 * (hls/gemv2/gemv2.h:1-3, board/tp/tp_llama.cpp:364-368). Every step is a
 * plain GEMV (w4a8_chain_step; k in 2048..W4A8_MAX_K), outputs byte-identical
 * to w4a8_chain_plan_create's; launch, wait and destroy as for any plan.
 * Every in-kernel wait is bounded: one that gives up ends every other wait
 * of the launch, the launch's outputs are then not valid, and
 * w4a8_chain_plan_wait returns W4A8_ERR_TIMEOUT once for it. A timed launch
 * of such a plan runs its steps with the barrier bit (no overlap). */
int w4a8_chain_plan_create_overlapped(const w4a8_chain_step *steps, int n, w4a8_chain_plan **plan);

/* A launch of the plan that also times each dispatch, from inside the
 * kernels (no tool intercepts the queue): the same kernels with the same
 * outputs, each workgroup reading the device's constant-rate clock when its
 * first wave starts and when all its waves are done (their stores landed),
 * and storing the two readings in a slot of its own (no atomics). Dispatch
 * i of the launch (pass i / n, step j = i % n) has
 * w4a8_chain_plan_workgroups(plan, j) workgroups; workgroup g of it writes
 * stamps[2 s] (start) and stamps[2 s + 1] (end), s = g plus the workgroup
 * counts of the dispatches before i. A dispatch's span is the latest end
 * minus the earliest start of its workgroups, in ticks of
 * w4a8_wall_clock_hz. stamps: device memory, 16-byte aligned, 2 * passes *
 * w4a8_chain_plan_workgroups(plan, -1) words; passes times that count at
 * most W4A8_PLAN_TIMED_MAX_SLOTS. The call waits for the plan's earlier
 * launches first (it rewrites the timed argument blocks), and the stamps are
 * valid once w4a8_chain_plan_wait returns W4A8_OK. A measurement aid: the
 * plain launch stays the one to use. */
#define W4A8_PLAN_TIMED_MAX_SLOTS (1L << 22)
int w4a8_chain_plan_launch_timed(w4a8_chain_plan *plan, int passes, uint64_t *stamps);
/* Workgroups of step `step` of the plan's dispatches (step -1: the sum over
 * all steps, one pass), or a negative status. */
long w4a8_chain_plan_workgroups(const w4a8_chain_plan *plan, int step);
/* Ticks per second of the clock the timed launch stamps with (current device). */
int w4a8_wall_clock_hz(int64_t *hz);

/* The same n GEMVs with no order between them, in one launch: every matrix
 * streams at once, so small matrices no longer pay a launch and a latency
 * tail each. Each y equals w4a8_gemv_f32 on its own, byte for byte. For
 * matrices that share an activation or are consumed together -- the
 * reference fuses q|k|v and gate|up into single matrices for this reason
 * (board/tp/tp_llama.cpp:258-268) -- or for a batch of independent
 * requests. No output may overlap any entry's x or weights, or another
 * entry's output (W4A8_ERR_SHAPE). 1 <= n <= W4A8_CHAIN_MAX_STEPS. */
int w4a8_gemv_batch(const w4a8_chain_step *steps, int n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A8_H */
