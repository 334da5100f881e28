// The reference's engine ABI (gemv_dev.h, gemv2_dev.h, udmabuf.h of
// board/kv260gemv) on the MI355X. Board code written against those headers
// links against this library unchanged; see the headers under include/ for
// what each call means on the GPU.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "../../include/gemv2_dev.h"
#include "../../include/gemv_dev.h"
#include "../../include/udmabuf.h"
#include "kernels.h"
#include "pool_ranges.h"
#include "q4_0_device.h"

using namespace w4a8;

namespace {

constexpr int REF_MAX_K = 8192;   // the engine's MAX_K, hls/int4_core/q4_0.h:17

struct EngineCtx {
    int device;
    hipStream_t stream;
    // v2: the matrix named by gemv2_fetch_start, consumed by gemv2_mac_start
    bool pending;
    uint64_t pending_w[4];
    int pending_k, pending_rows;
};

[[noreturn]] void die(const char *what, const char *detail) {
    fprintf(stderr, "kv260gemv: %s%s%s\n", what, detail ? ": " : "", detail ? detail : "");
    fflush(stderr);
    abort();
}

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) die(what, hipGetErrorString(e));
}

int env_device() {
    const char *s = getenv("KV260GEMV_DEVICE");
    return s ? atoi(s) : 0;
}

EngineCtx *ctx_of(gemv_dev_t *d) {
    if (!d || !d->regs) die("engine not open", nullptr);
    return (EngineCtx *)(uintptr_t)d->regs;
}

int open_ctx(gemv_dev_t *d, int quiet) {
    d->fd = -1;
    d->regs = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        if (!quiet) fprintf(stderr, "kv260gemv: no HIP device visible\n");
        return -1;
    }
    const int dev = env_device();
    if (dev < 0 || dev >= n) {
        if (!quiet) fprintf(stderr, "kv260gemv: KV260GEMV_DEVICE=%d but %d device(s)\n", dev, n);
        return -1;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (!quiet) fprintf(stderr, "kv260gemv: device %d is not gfx950\n", dev);
        return -1;
    }
    if (hipSetDevice(dev) != hipSuccess) return -1;
    EngineCtx *c = (EngineCtx *)calloc(1, sizeof(EngineCtx));
    if (!c) return -1;
    c->device = dev;
    if (hipStreamCreate(&c->stream) != hipSuccess) {
        free(c);
        if (!quiet) fprintf(stderr, "kv260gemv: cannot create a stream\n");
        return -1;
    }
    d->fd = dev;
    d->regs = (volatile uint32_t *)(uintptr_t)c;
    return 0;
}

void close_ctx(gemv_dev_t *d) {
    if (!d) return;
    if (d->regs) {
        EngineCtx *c = (EngineCtx *)(uintptr_t)d->regs;
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamDestroy(c->stream);
        free(c);
    }
    d->regs = nullptr;
    d->fd = -1;
}

// The reference's constraints (board/kv260gemv/gemv_dev.h:22, gemv2_dev.h:14)
// plus the GPU's alignment; a violation is a caller bug, reported and fatal.
void check_call(uint64_t x, uint64_t y, int k, int rows, int row_multiple, const char *who) {
    char msg[160];
    if (k < 256 || k > REF_MAX_K || k % 256) {
        snprintf(msg, sizeof msg, "k=%d (need k %% 256 == 0, 256 <= k <= %d)", k, REF_MAX_K);
        die(who, msg);
    }
    if (rows <= 0 || rows % row_multiple) {
        snprintf(msg, sizeof msg, "rows=%d (need a positive multiple of %d)", rows, row_multiple);
        die(who, msg);
    }
    if (!x || (x & 15) || !y || (y & 3)) {
        snprintf(msg, sizeof msg, "x=0x%llx y=0x%llx (x 16-byte, y 4-byte aligned, non-null)",
                 (unsigned long long)x, (unsigned long long)y);
        die(who, msg);
    }
}

void check_w(const uint64_t *w, int n, const char *who) {
    for (int i = 0; i < n; ++i)
        if (!w[i] || (w[i] & 15)) die(who, "weight address NULL or not 16-byte aligned");
}

// ------------------------------------------------------------------ pools
//
// A pool is device memory (what the engine reads; its addresses are the
// "physical" ones handed to the engine) and pinned host memory of the same
// size (what the CPU touches), mapped for the GPU and coherent. Which copy of
// a range is current:
//  * udmabuf_clean of a range under EAGER_CLEAN bytes copies nothing: the
//    range joins the pool's host-current set (a larger clean, such as the
//    weights once after loading, is copied at once);
//  * an engine call first copies the host-current parts of what it reads
//    (its weights and x) to the device, on its own stream, ahead of the
//    GEMV, and writes its y straight into the host copy, so that y's range
//    is host-current afterwards;
//  * udmabuf_invalidate copies to the host only the parts that are not
//    host-current (the device copy of those may hold writes made outside
//    the engine calls).
// The reference caller's per-call clean of x and its invalidates of y before
// and after the call then cost no copy of their own; x's copy rides on the
// engine's stream ahead of the GEMV, and y's bytes go to the host as the
// GEMV writes them.

constexpr size_t EAGER_CLEAN = (size_t)1 << 20;

struct Pool {
    uint8_t *host;
    uint8_t *dev;
    size_t size;
    int device;
    uint8_t *host_dev;                          // the host memory's address on the GPU
    pool_ranges::Set *host_cur;                 // the host-current ranges (offsets)
};
constexpr int MAX_POOLS = 16;
Pool g_pools[MAX_POOLS];
std::mutex g_pool_mu;

// Bytes [a, b) of src to dst (the same offsets in both): 16-byte pieces, the
// unaligned head and tail byte by byte.
__global__ void copy_range_kernel(uint8_t *dst, const uint8_t *src, size_t a, size_t b) {
    const size_t a16 = (a + 15) & ~(size_t)15, b16 = b & ~(size_t)15;
    const size_t i = a16 + 16 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (a16 < b16 && i < b16) *reinterpret_cast<uint4 *>(dst + i) = *reinterpret_cast<const uint4 *>(src + i);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const size_t head = a16 < b ? a16 : b;
        for (size_t j = a; j < head; ++j) dst[j] = src[j];
        for (size_t j = (b16 > head ? b16 : head); j < b; ++j) dst[j] = src[j];
    }
}

// The pool whose device memory holds [phys, phys + len), or null.
Pool *pool_of_dev(uint64_t phys, size_t len, size_t *off) {
    const uint8_t *a = (const uint8_t *)(uintptr_t)phys;
    for (auto &pl : g_pools) {
        if (!pl.host || a < pl.dev || a >= pl.dev + pl.size) continue;
        *off = (size_t)(a - pl.dev);
        if (len > pl.size - *off) return nullptr;
        return &pl;
    }
    return nullptr;
}

// Before an engine call on `stream`: the host-current parts of a range it reads go to the device.
void flush_reads(uint64_t phys, size_t len, hipStream_t stream, const char *who) {
    std::lock_guard<std::mutex> g(g_pool_mu);
    size_t off;
    Pool *pl = pool_of_dev(phys, len, &off);
    if (!pl || pl->host_cur->empty()) return;
    for (const auto &r : pool_ranges::parts(*pl->host_cur, off, off + len, true)) {
        const size_t n = r.second - r.first;
        if (n >= EAGER_CLEAN) {
            check_hip(hipMemcpyAsync(pl->dev + r.first, pl->host + r.first, n, hipMemcpyHostToDevice, stream), who);
        } else {
            const size_t units = (n + 15) / 16 + 1;
            const unsigned grid = (unsigned)((units + 255) / 256);
            hipLaunchKernelGGL(copy_range_kernel, dim3(grid), dim3(256), 0, stream, pl->dev, pl->host_dev, r.first,
                               r.second);
            check_hip(hipGetLastError(), who);
        }
    }
    pool_ranges::remove(*pl->host_cur, off, off + len);
}

// y of an engine call: its address in the host copy when it lies in a pool
// (the range is host-current from then on), else y itself.
float *route_y(uint64_t y, int rows) {
    std::lock_guard<std::mutex> g(g_pool_mu);
    size_t off;
    const size_t len = (size_t)rows * 4;
    Pool *pl = pool_of_dev(y, len, &off);
    if (!pl) return (float *)(uintptr_t)y;
    pool_ranges::add(*pl->host_cur, off, off + len);
    return reinterpret_cast<float *>(pl->host_dev + off);
}

void start(EngineCtx *c, const MatrixRef &m, uint64_t x, uint64_t y, const char *who) {
    check_hip(hipSetDevice(c->device), who);
    const size_t seg_bytes = (size_t)m.seg_rows * (size_t)(m.k / QK) * Q4_0_BYTES;
    for (int q = 0; q < m.nseg; ++q) flush_reads((uint64_t)(uintptr_t)m.seg[q], seg_bytes, c->stream, who);
    flush_reads(x, (size_t)m.k + (size_t)m.k / 8, c->stream, who);
    float *yp = route_y(y, m.rows);
    check_hip(launch_gemv_m1(m, (const void *)(uintptr_t)x, X_ENGINE, yp, c->stream), who);
}

size_t parse_size(const char *s, const char *end) {
    char *e = nullptr;
    unsigned long long v = strtoull(s, &e, 10);
    if (e && e < end) {
        if (*e == 'K' || *e == 'k') v <<= 10;
        else if (*e == 'M' || *e == 'm') v <<= 20;
        else if (*e == 'G' || *e == 'g') v <<= 30;
    }
    return (size_t)v;
}

// Size configured for pool `name`: KV260GEMV_UDMABUF_SIZES="name=SIZE,...",
// default udmabuf0 = 1 GiB and nothing else.
size_t pool_size(const char *name) {
    const char *spec = getenv("KV260GEMV_UDMABUF_SIZES");
    if (!spec) return strcmp(name, "udmabuf0") == 0 ? (size_t)1 << 30 : 0;
    const size_t nl = strlen(name);
    const char *p = spec;
    while (*p) {
        const char *end = strchr(p, ',');
        if (!end) end = p + strlen(p);
        const char *eq = (const char *)memchr(p, '=', (size_t)(end - p));
        if (eq && (size_t)(eq - p) == nl && strncmp(p, name, nl) == 0) return parse_size(eq + 1, end);
        p = *end ? end + 1 : end;
    }
    return 0;
}

// The pool holding host address p, clamped range [off, off + len); called
// with g_pool_mu held.
Pool *find_pool(const void *p, size_t len, size_t *off, size_t *n) {
    const uint8_t *a = (const uint8_t *)p;
    for (auto &pl : g_pools) {
        if (!pl.host || a < pl.host || a >= pl.host + pl.size) continue;
        *off = (size_t)(a - pl.host);
        *n = len < pl.size - *off ? len : pl.size - *off;
        return &pl;
    }
    return nullptr;
}

}  // namespace

extern "C" {

// ------------------------------------------------------------------ v1 ABI

int gemv_dev_open_named(gemv_dev_t *d, const char *name, int quiet) {
    if (!d) return -1;
    if (!name || (strcmp(name, "gemv_q4_0") && strcmp(name, "gemv_fetch") && strcmp(name, "gemv_mac"))) {
        if (!quiet) fprintf(stderr, "kv260gemv: no engine named %s\n", name ? name : "(null)");
        d->fd = -1;
        d->regs = nullptr;
        return -1;
    }
    return open_ctx(d, quiet);
}

int gemv_dev_open(gemv_dev_t *d) { return gemv_dev_open_named(d, "gemv_q4_0", 0); }

void gemv_dev_close(gemv_dev_t *d) { close_ctx(d); }

void gemv_dev_start4(gemv_dev_t *d, const uint64_t w[4], uint64_t x, uint64_t y, int k, int rows) {
    EngineCtx *c = ctx_of(d);
    check_call(x, y, k, rows, 16, "gemv_dev_start4");
    check_w(w, 4, "gemv_dev_start4");
    MatrixRef m{};
    for (int q = 0; q < 4; ++q) m.seg[q] = (const uint8_t *)(uintptr_t)w[q];
    m.nseg = 4;
    m.seg_rows = rows / 4;
    m.rows = rows;
    m.k = k;
    start(c, m, x, y, "gemv_dev_start4");
}

void gemv_dev_start(gemv_dev_t *d, uint64_t w, uint64_t x, uint64_t y, int k, int rows) {
    EngineCtx *c = ctx_of(d);
    check_call(x, y, k, rows, 16, "gemv_dev_start");
    check_w(&w, 1, "gemv_dev_start");
    // The four quarters back to back are the plain row-major matrix.
    MatrixRef m{};
    m.seg[0] = (const uint8_t *)(uintptr_t)w;
    m.nseg = 1;
    m.seg_rows = rows;
    m.rows = rows;
    m.k = k;
    start(c, m, x, y, "gemv_dev_start");
}

void gemv_dev_wait(gemv_dev_t *d) {
    EngineCtx *c = ctx_of(d);
    check_hip(hipSetDevice(c->device), "gemv_dev_wait");
    check_hip(hipStreamSynchronize(c->stream), "gemv_dev_wait");
}

void gemv_dev_run(gemv_dev_t *d, uint64_t w, uint64_t x, uint64_t y, int k, int rows) {
    gemv_dev_start(d, w, x, y, k, rows);
    gemv_dev_wait(d);
}

// ------------------------------------------------------------------ v2 ABI

int gemv2_dev_open(gemv2_dev_t *d) {
    if (!d) return -1;
    if (open_ctx(&d->mac, 1)) {
        d->fetch.fd = -1;
        d->fetch.regs = nullptr;
        return -1;
    }
    // One context serves both "kernels"; fetch carries it too, so a call on
    // either half finds it.
    d->fetch = d->mac;
    return 0;
}

void gemv2_dev_close(gemv2_dev_t *d) {
    if (!d) return;
    close_ctx(&d->mac);
    d->fetch.regs = nullptr;
    d->fetch.fd = -1;
}

void gemv2_fetch_wait(gemv2_dev_t *d) { (void)ctx_of(&d->mac); }

void gemv2_fetch_start(gemv2_dev_t *d, const uint64_t w[4], int k, int rows) {
    EngineCtx *c = ctx_of(&d->mac);
    check_w(w, 4, "gemv2_fetch_start");
    if (c->pending) die("gemv2_fetch_start", "a fetched matrix was never consumed by gemv2_mac_start");
    for (int q = 0; q < 4; ++q) c->pending_w[q] = w[q];
    c->pending_k = k;
    c->pending_rows = rows;
    c->pending = true;
}

void gemv2_mac_start(gemv2_dev_t *d, uint64_t x, uint64_t y, int k, int rows) {
    EngineCtx *c = ctx_of(&d->mac);
    check_call(x, y, k, rows, 32, "gemv2_mac_start");
    if (!c->pending) die("gemv2_mac_start", "no matrix fetched (call gemv2_fetch_start first)");
    if (c->pending_k != k || c->pending_rows != rows)
        die("gemv2_mac_start", "k/rows differ from the fetched matrix's");
    MatrixRef m{};
    for (int q = 0; q < 4; ++q) m.seg[q] = (const uint8_t *)(uintptr_t)c->pending_w[q];
    m.nseg = 4;
    m.seg_rows = rows / 4;
    m.rows = rows;
    m.k = k;
    m.paired = true;
    c->pending = false;
    start(c, m, x, y, "gemv2_mac_start");
}

void gemv2_mac_wait(gemv2_dev_t *d) {
    EngineCtx *c = ctx_of(&d->mac);
    check_hip(hipSetDevice(c->device), "gemv2_mac_wait");
    check_hip(hipStreamSynchronize(c->stream), "gemv2_mac_wait");
}

int gemv2_mac_idle(gemv2_dev_t *d) {
    EngineCtx *c = ctx_of(&d->mac);
    (void)hipSetDevice(c->device);
    return hipStreamQuery(c->stream) == hipSuccess ? 1 : 0;
}

void gemv2_drain(gemv2_dev_t *d) {
    EngineCtx *c = ctx_of(&d->mac);
    c->pending = false;
    check_hip(hipSetDevice(c->device), "gemv2_drain");
    check_hip(hipStreamSynchronize(c->stream), "gemv2_drain");
}

// ---------------------------------------------------------------- udmabuf

int udmabuf_open(udmabuf_t *b, const char *name) {
    if (!b) return -1;
    memset(b, 0, sizeof *b);
    b->fd = -1;
    const size_t size = name ? pool_size(name) : 0;
    if (!size) {
        fprintf(stderr, "udmabuf: no pool %s (KV260GEMV_UDMABUF_SIZES)\n", name ? name : "(null)");
        return -1;
    }
    const int dev = env_device();
    void *host = nullptr, *devp = nullptr;
    if (hipSetDevice(dev) != hipSuccess || hipMalloc(&devp, size) != hipSuccess) {
        fprintf(stderr, "udmabuf: cannot allocate %zu MB of device memory for %s\n", size >> 20, name);
        return -1;
    }
    if (hipHostMalloc(&host, size, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
        (void)hipFree(devp);
        fprintf(stderr, "udmabuf: cannot allocate %zu MB of pinned host memory for %s\n", size >> 20, name);
        return -1;
    }
    void *host_dev = nullptr;
    auto *cur = new (std::nothrow) pool_ranges::Set();
    if (!cur || hipHostGetDevicePointer(&host_dev, host, 0) != hipSuccess) {
        delete cur;
        (void)hipHostFree(host);
        (void)hipFree(devp);
        fprintf(stderr, "udmabuf: cannot map the host memory of %s for the device\n", name);
        return -1;
    }
    {
        std::lock_guard<std::mutex> g(g_pool_mu);
        int slot = -1;
        for (int i = 0; i < MAX_POOLS; ++i)
            if (!g_pools[i].host) { slot = i; break; }
        if (slot < 0) {
            delete cur;
            (void)hipHostFree(host);
            (void)hipFree(devp);
            fprintf(stderr, "udmabuf: more than %d pools open\n", MAX_POOLS);
            return -1;
        }
        g_pools[slot] = Pool{(uint8_t *)host, (uint8_t *)devp, size, dev, (uint8_t *)host_dev, cur};
    }
    b->fd = dev;
    b->base = (uint8_t *)host;
    b->phys = (uint64_t)(uintptr_t)devp;
    b->size = size;
    b->used = 0;
    return 0;
}

void udmabuf_close(udmabuf_t *b) {
    if (!b) return;
    if (b->base) {
        Pool found{};
        {
            std::lock_guard<std::mutex> g(g_pool_mu);
            for (auto &pl : g_pools)
                if (pl.host == b->base) { found = pl; pl = Pool{}; break; }
        }
        if (found.host) {
            (void)hipSetDevice(found.device);
            (void)hipDeviceSynchronize();
            (void)hipHostFree(found.host);
            (void)hipFree(found.dev);
            delete found.host_cur;
        }
    }
    memset(b, 0, sizeof *b);
    b->fd = -1;
}

void *udmabuf_alloc(udmabuf_t *b, size_t size, size_t align) {
    if (!b || !b->base || !align || (align & (align - 1))) return NULL;
    const size_t start = (b->used + align - 1) & ~(align - 1);
    if (start > b->size || size > b->size - start) return NULL;
    b->used = start + size;
    return b->base + start;
}

void udmabuf_clean(const void *p, size_t len) {
    std::lock_guard<std::mutex> g(g_pool_mu);
    size_t off, n;
    Pool *pl = len ? find_pool(p, len, &off, &n) : nullptr;
    if (!pl) return;
    if (n < EAGER_CLEAN) {
        pool_ranges::add(*pl->host_cur, off, off + n);
        return;
    }
    check_hip(hipSetDevice(pl->device), "udmabuf_clean");
    check_hip(hipMemcpy(pl->dev + off, pl->host + off, n, hipMemcpyHostToDevice), "udmabuf_clean");
    pool_ranges::remove(*pl->host_cur, off, off + n);
}

void udmabuf_invalidate(const void *p, size_t len) {
    std::lock_guard<std::mutex> g(g_pool_mu);
    size_t off, n;
    Pool *pl = len ? find_pool(p, len, &off, &n) : nullptr;
    if (!pl) return;
    const auto parts = pool_ranges::parts(*pl->host_cur, off, off + n, false);
    if (parts.empty()) return;
    check_hip(hipSetDevice(pl->device), "udmabuf_invalidate");
    for (const auto &r : parts)
        check_hip(hipMemcpy(pl->host + r.first, pl->dev + r.first, r.second - r.first, hipMemcpyDeviceToHost),
                  "udmabuf_invalidate");
}

}  // extern "C"
