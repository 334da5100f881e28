/*
 * udmabuf.h -- the engine-memory ABI, served by the MI355X library.
 *
 * Drop-in for board/kv260gemv/udmabuf.h:15-36. On the board a pool is CMA
 * memory the CPU and the fabric share, and clean/invalidate are cache
 * maintenance. On the GPU a pool is two allocations of the same size: device
 * memory in HBM (what the engine reads; `phys` is its device address) and a
 * pinned host copy (`base`, what the CPU code touches), mapped for the GPU and
 * coherent. The library tracks which copy of each range is current:
 *   - udmabuf_clean(p, len): the CPU wrote [p, p+len). Under 1 MiB nothing is
 *     copied yet: the range is marked host-current, and the next engine call
 *     that reads it (as x or as weights) copies it to the device first, on
 *     the engine's stream, ahead of the GEMV. From 1 MiB on (weights after
 *     loading) it is copied host -> device at once, synchronously.
 *   - an engine call writes its y straight into the host copy (the GPU's
 *     stores cross PCIe as the GEMV makes them), so y's range is
 *     host-current once the call's wait returns.
 *   - udmabuf_invalidate(p, len): the CPU will read [p, p+len). The parts
 *     not host-current are copied device -> host, synchronously (the device
 *     copy may hold writes made outside the engine calls); host-current parts
 *     need nothing. A write into the device copy of a host-current range by
 *     anything but an engine call (a kernel of the caller's own at the pool's
 *     device address) is therefore not seen by the host; clean such a range
 *     with 1 MiB or more first (copied at once, it leaves nothing
 *     host-current), or keep those writes to ranges the host never cleaned.
 * So the reference's discipline ("clean before the engine reads what the CPU
 * wrote, invalidate before the CPU reads what the engine wrote") still carries
 * the data exactly where it did on the board, and its per-call clean of x and
 * invalidates of y cost no copy of their own. Pointers outside every open pool
 * are ignored, as cache maintenance on them would be.
 *
 * Pool sizes: KV260GEMV_UDMABUF_SIZES, e.g. "udmabuf0=1G,udmabuf1=256M"
 * (K/M/G suffixes); default udmabuf0 = 1 GiB and no other pool, so
 * udmabuf_open("udmabuf1") fails as it does on a board without that pool.
 */
#ifndef KV260GEMV_UDMABUF_H
#define KV260GEMV_UDMABUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int fd;          /* HIP device ordinal of the pool */
    uint8_t *base;   /* host mirror */
    uint64_t phys;   /* device address of the pool's first byte */
    size_t size;
    size_t used;     /* bump allocator watermark */
} udmabuf_t;

/* 0, or -1 with a message when the pool is not configured or memory is short.
 * Replaces board/kv260gemv/udmabuf.c:25-40. */
int udmabuf_open(udmabuf_t *b, const char *name);
void udmabuf_close(udmabuf_t *b);

/* Bump-allocate `size` bytes aligned to `align` (a power of two); NULL when
 * full. No free: a model is loaded once. udmabuf.c:47-52. */
void *udmabuf_alloc(udmabuf_t *b, size_t size, size_t align);

static inline uint64_t udmabuf_phys(const udmabuf_t *b, const void *p) {
    return b->phys + (uint64_t)((const uint8_t *)p - b->base);
}

void udmabuf_clean(const void *p, size_t len);        /* CPU wrote, device will read */
void udmabuf_invalidate(const void *p, size_t len);   /* device wrote, CPU will read */

#ifdef __cplusplus
}
#endif

#endif /* KV260GEMV_UDMABUF_H */
