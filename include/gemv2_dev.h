/*
 * gemv2_dev.h -- the v2 (fetch + MAC) engine ABI, served by the MI355X library.
 *
 * Drop-in for board/kv260gemv/gemv2_dev.h:22-45: same type, names, signatures,
 * call discipline and matrix layout, so board/tp's gemv2 path and
 * bench_gemv2.c link unchanged.
 *
 * Call discipline (as on the fabric): gemv2_fetch_start(W) names the matrix as
 * soon as it is known; gemv2_mac_start(x, y) then computes y = W x with that
 * matrix. The two must be issued for the same matrix, in order, with nothing
 * in between. Here the fetch records W (and lets the MAC kernel find it); the
 * MAC start enqueues one GEMV kernel that reads the chunk-interleaved layout
 * directly, with no reformatting pass.
 *
 * Layout (board/kv260gemv/gemv2_dev.h:46-49): a [rows, k] matrix is four port
 * regions of rows/4 rows at w[0..3]. Inside a region, row i pairs with row
 * i + rows/8 and their 144-byte chunks (8 blocks) alternate. rows % 32 == 0,
 * k % 256 == 0, k <= 8192.
 */
#ifndef KV260GEMV_GEMV2_DEV_H
#define KV260GEMV_GEMV2_DEV_H

#include <stddef.h>
#include <stdint.h>

#include "gemv_dev.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    gemv_dev_t fetch, mac;
} gemv2_dev_t;

#define GEMV2_CHUNK_BYTES 144

/* 0 on success; -1 (quietly) when no usable GPU. gemv2_dev.c:19-23. */
int gemv2_dev_open(gemv2_dev_t *d);
void gemv2_dev_close(gemv2_dev_t *d);

/* Byte offset of chunk c of row r inside its port's region; *port receives
 * the port. Port p holds rows [p R, (p+1) R), R = rows / 4; row p R + i pairs
 * with row p R + i + H, H = R / 2, and chunk c of the pair's rows sit side by
 * side: the pair's chunks run (i, c=0, first), (i, c=0, second), (i, c=1,
 * first), ... The layout is the interface (gemv2_dev.h:66-72 of the reference),
 * so the formula is the same. */
static inline size_t gemv2_chunk_offset(int r, int c, int rows, int k, int *port) {
    const int per_port = rows / 4, half = per_port / 2, chunks = k / 256;
    const int local = r % per_port;
    const int pair = local % half, second = local / half;
    *port = r / per_port;
    return (((size_t)pair * (size_t)chunks + (size_t)c) * 2u + (size_t)second) * GEMV2_CHUNK_BYTES;
}

/* Names the matrix the next gemv2_mac_start computes with (its four port
 * region addresses). Waits for nothing: no FIFO can fill here. */
void gemv2_fetch_start(gemv2_dev_t *d, const uint64_t w[4], int k, int rows);
void gemv2_fetch_wait(gemv2_dev_t *d);
/* y[rows] = W x with the fetched W; x int8[k] then float32[k/32]. Enqueues. */
void gemv2_mac_start(gemv2_dev_t *d, uint64_t x, uint64_t y, int k, int rows);
void gemv2_mac_wait(gemv2_dev_t *d);
/* 1 when no MAC work is outstanding. */
int gemv2_mac_idle(gemv2_dev_t *d);
/* Forgets a fetched matrix that was never computed (a previous caller's). */
void gemv2_drain(gemv2_dev_t *d);

#ifdef __cplusplus
}
#endif

#endif /* KV260GEMV_GEMV2_DEV_H */
