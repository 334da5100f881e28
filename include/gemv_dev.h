/*
 * gemv_dev.h -- the v1 engine ABI, served by the MI355X library.
 *
 * Drop-in for board/kv260gemv/gemv_dev.h:10-35 (same type, names, signatures
 * and argument meaning), so board/tp's engine_t (board/tp/tp_llama.cpp:295-375)
 * links against libkv260gemv.so unchanged.
 *
 * What the fields and addresses mean here:
 *   - gemv_dev_t.fd is the HIP device ordinal, .regs an opaque pointer to the
 *     library's per-device context (stream, pending state). The struct keeps
 *     the reference's size and layout.
 *   - Every uint64_t address is a device virtual address, as udmabuf_phys()
 *     (udmabuf.h) returns for pool memory.
 *   - start enqueues the GEMV on the context's HIP stream and returns; wait
 *     blocks until it has finished.
 *
 * Constraints, as the reference states them (board/kv260gemv/gemv_dev.h:22):
 * k % 256 == 0, k <= 8192, rows % 16 == 0. A call that breaks them is a
 * caller bug: the library prints what was wrong and aborts, rather than
 * computing anything (the reference's start/run are void too).
 */
#ifndef KV260GEMV_GEMV_DEV_H
#define KV260GEMV_GEMV_DEV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int fd;
    volatile uint32_t *regs;
} gemv_dev_t;

/* Opens the engine "gemv_q4_0" on the GPU (KV260GEMV_DEVICE selects the HIP
 * device, default 0). 0 on success, -1 with a message on stderr otherwise.
 * Replaces gemv_dev_open, board/kv260gemv/gemv_dev.c:48. */
int gemv_dev_open(gemv_dev_t *d);

/* Any of the reference's engine names: "gemv_q4_0", "gemv_fetch", "gemv_mac".
 * quiet suppresses the message when the name is unknown or no GPU is usable.
 * Replaces board/kv260gemv/gemv_dev.c:35-46. */
int gemv_dev_open_named(gemv_dev_t *d, const char *name, int quiet);

/* Waits for outstanding work, releases the context. gemv_dev.c:50-55. */
void gemv_dev_close(gemv_dev_t *d);

/* y[rows] = W[rows, k] x. w: the Q4_0 rows, ggml layout; x: int8[k] then
 * float32[k/32]; y: rows float32. Blocks until done. gemv_dev.h:19-23. */
void gemv_dev_run(gemv_dev_t *d, uint64_t w, uint64_t x, uint64_t y, int k, int rows);

/* Split form: enqueue, then wait. gemv_dev.h:25-27. */
void gemv_dev_start(gemv_dev_t *d, uint64_t w, uint64_t x, uint64_t y, int k, int rows);
void gemv_dev_wait(gemv_dev_t *d);

/* Quarter m of the rows (rows/4 contiguous rows) at w[m]; y contiguous.
 * gemv_dev.h:29-35. */
void gemv_dev_start4(gemv_dev_t *d, const uint64_t w[4], uint64_t x, uint64_t y, int k, int rows);

#ifdef __cplusplus
}
#endif

#endif /* KV260GEMV_GEMV_DEV_H */
