// The decode step's GEMV chain as a plan: the M = 1 GEMV's kernels
// (gemv_m1_dev.h, fp32 x quantized in their staging; with the rmsnorm, the
// silu * up epilogue or the greedy pick fused as the stream entry points
// have them), dispatched as raw AQL packets on an HSA queue of the library's
// own (one per device) instead of through HIP launches.
//
// Why: between two kernels of a HIP stream or graph the packet processor
// runs a release fence (every XCD's L2 written back) and an acquire fence
// (every L2 and the scalar caches invalidated). The chain's kernels are
// small and dependent, so those fences sit on the critical path 65 times
// per token. A plan's packets carry no fences between steps (acquire at
// system scope on a launch's first packet, release at system scope on its
// last) and keep only the barrier bit, which orders step j + 1 after step j.
// What the fences did for the chain's own data is done per step instead:
// an output that a later step reads is written through to the device's
// coherence point and waited for before its waves end, and that step reads
// it from there (the kernels' _yc / _xc variants); everything else goes
// through the caches as before. The kernel arguments sit in device memory,
// written once when the plan is made (w4a8_chain_plan says why not in host
// memory).
//
// This mirrors how the reference drives its engine: the host starts the
// work and later waits for it (board/kv260gemv/gemv2_dev.h:40-44,
// board/tp/tp_llama.cpp:318-323), not through a stream.
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <chrono>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "gemv_m1_dev.h"
#include "plan_ring.h"

extern "C" const char w4a8_chain_plan_co_begin[];
extern "C" const char w4a8_chain_plan_co_end[];

struct w4a8_chain_plan {
    int device = 0;
    int n = 0;
    std::vector<int> kind;                 // kernel variant per step
    std::vector<uint32_t> grid, threads, group;
    // The steps' argument blocks, ARG_STRIDE bytes each: in device memory
    // (what the packets point at) and a host copy (the timed launch builds
    // its blocks from it). In pinned coherent host memory instead, every
    // launch paid about 50 us more: its first packet's acquire drops the
    // blocks from the caches, and each of the first pass's 65 dispatches then
    // fetched its block across PCIe (one pass 296 us against 244-248; the
    // steady state the same, 233-234 us per pass).
    char *kargs = nullptr;
    std::vector<char> kargs_host;
    hsa_signal_t done{};                   // launches in flight
    char *timed_kargs = nullptr;           // the timed launch's, device memory: one block per dispatch
    size_t timed_bytes = 0;
    // Overlapped plans: steps after the first of a pass go out without the
    // barrier bit and wait in the kernel (gemv_m1_dev.h, StreamSync).
    bool overlapped = false;
    uint8_t *flags = nullptr;              // device memory: per-step flag bytes, then the abort word
    uint32_t *abort_word = nullptr;
};

namespace w4a8 {

namespace {

// The kernels' argument block (their kernarg segment is exactly this).
struct PlanArgs {
    const uint8_t *w0;
    const void *x;
    int rows, k, C, rpw, tiles, nblocks, nthreads, pad;
    GemvParams P;
};
static_assert(sizeof(PlanArgs) == 176, "argument block of the plan's kernels");
// The timed twins take one more argument after the block: the dispatch's
// two stamp words.
constexpr size_t TIMED_ARGS_BYTES = sizeof(PlanArgs) + sizeof(unsigned long long *);
// The overlapped plan's kernels take the step-to-step wait's arguments after
// the block.
constexpr size_t STREAM_ARGS_BYTES = sizeof(PlanArgs) + sizeof(StreamSync);
static_assert(STREAM_ARGS_BYTES <= 256, "argument slot");
constexpr int STREAM_SPIN_LIMIT = 1 << 20;   // polls (each a device-coherent read) before a wait gives up
constexpr size_t ARG_STRIDE = 256;
constexpr uint32_t QUEUE_PACKETS = 16384;
// Kernel variants: (kernel kind) x (x format) x (coherence), in
// chain_plan_kernels.hip, w4a8_plan_<kind>_<format><coherence>. Not every
// kind has every format (HAS_FORMAT); the slots of the others stay empty.
constexpr int N_KKINDS = 4, N_FORMATS = 3, N_KERNELS = N_KKINDS * N_FORMATS * 4;
constexpr int KK_GEMV = 0, KK_PAIR = 1, KK_ARGMAX = 2, KK_PAIR_Q8 = 3;
constexpr int FMT_F32 = 0, FMT_RMS = 1, FMT_ENG = 2;
constexpr const char *KIND_NAMES[N_KKINDS] = {"gemv", "pair", "argmax", "pairq"};
constexpr const char *FORMAT_NAMES[N_FORMATS] = {"f32", "rms", "eng"};
constexpr const char *COH_NAMES[4] = {"", "_xc", "_yc", "_xyc"};
constexpr bool HAS_FORMAT[N_KKINDS][N_FORMATS] = {{true, true, true}, {true, true, false}, {true, true, false},
                                                  {true, true, false}};
constexpr int kernel_index(int kk, int fmt, int coh) { return (kk * N_FORMATS + fmt) * 4 + coh; }

// A plan step's kernel kind and x format.
int kernel_kind(const w4a8_plan_step &s) {
    switch (s.kind) {
        case W4A8_PLAN_GATE_UP_SILU: return KK_PAIR;
        case W4A8_PLAN_ARGMAX: return KK_ARGMAX;
        case W4A8_PLAN_GATE_UP_SILU_Q8: return KK_PAIR_Q8;
        default: return KK_GEMV;
    }
}
int x_format(const w4a8_plan_step &s) {
    if (s.kind == W4A8_PLAN_GEMV_ENGINE) return FMT_ENG;
    return s.norm_w ? FMT_RMS : FMT_F32;
}
// The bytes a step reads as x and writes as y.
size_t x_bytes(const w4a8_plan_step &s) {
    return s.kind == W4A8_PLAN_GEMV_ENGINE ? (size_t)s.k + (size_t)s.k / 8 : 4 * (size_t)s.k;
}
size_t y_bytes(const w4a8_plan_step &s) {
    if (s.kind == W4A8_PLAN_GATE_UP_SILU) return 4 * (size_t)(s.rows / 2);
    if (s.kind == W4A8_PLAN_GATE_UP_SILU_Q8) return (size_t)(s.rows / 2) + (size_t)(s.rows / 16);
    return 4 * (size_t)s.rows;
}
// A launch waiting for free packet slots gives up once the device has taken
// no packet for this long: the device is then stalled, not merely busy.
constexpr double QUEUE_STALL_S = 10.0;

struct DeviceRuntime {
    std::mutex m;                  // one producer on the queue at a time
    bool tried = false;
    int status = W4A8_OK;
    bool stalled = false;          // a launch found the queue stalled: every later launch fails
    hsa_agent_t agent{};
    hsa_queue_t *queue = nullptr;
    hsa_executable_t exe{};
    // [0]: the kernels, [1]: their timed twins.
    uint64_t kobj[2][N_KERNELS]{};
    uint32_t group[2][N_KERNELS]{}, priv[2][N_KERNELS]{};
    // The overlapped plan's GEMV kernels: [x format f32 / eng][coherence variant].
    uint64_t kobj_s[2][4]{};
    uint32_t group_s[2][4]{}, priv_s[2][4]{};
};
constexpr int MAX_DEVICES = 16;
DeviceRuntime g_rt[MAX_DEVICES];

struct AgentMatch {
    uint32_t domain, bdf;
    hsa_agent_t agent;
    bool found;
};

hsa_status_t match_agent(hsa_agent_t a, void *data) {
    auto *m = static_cast<AgentMatch *>(data);
    hsa_device_type_t t;
    if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS || t != HSA_DEVICE_TYPE_GPU)
        return HSA_STATUS_SUCCESS;
    uint32_t bdf = 0, domain = 0;
    if (hsa_agent_get_info(a, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_BDFID, &bdf) != HSA_STATUS_SUCCESS ||
        hsa_agent_get_info(a, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_DOMAIN, &domain) != HSA_STATUS_SUCCESS)
        return HSA_STATUS_SUCCESS;
    if (bdf == m->bdf && domain == m->domain) {
        m->agent = a;
        m->found = true;
        return HSA_STATUS_INFO_BREAK;
    }
    return HSA_STATUS_SUCCESS;
}

// The HSA agent of HIP device `dev`, the plan kernels loaded for it and its
// queue; made once per device.
int runtime_of(int dev, DeviceRuntime *&out) {
    if (dev < 0 || dev >= MAX_DEVICES) return W4A8_ERR_NODEV;
    DeviceRuntime &rt = g_rt[dev];
    std::lock_guard<std::mutex> lk(rt.m);
    out = &rt;
    if (rt.tried) return rt.status;
    rt.tried = true;
    rt.status = W4A8_ERR_HSA;
    int bus = 0, devid = 0, domain = 0;
    if (hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, dev) != hipSuccess ||
        hipDeviceGetAttribute(&devid, hipDeviceAttributePciDeviceId, dev) != hipSuccess ||
        hipDeviceGetAttribute(&domain, hipDeviceAttributePciDomainID, dev) != hipSuccess)
        return rt.status = W4A8_ERR_NODEV;
    if (hsa_init() != HSA_STATUS_SUCCESS) return rt.status;
    AgentMatch m{(uint32_t)domain, ((uint32_t)bus << 8) | ((uint32_t)devid << 3), {}, false};
    const hsa_status_t it = hsa_iterate_agents(match_agent, &m);
    if ((it != HSA_STATUS_SUCCESS && it != HSA_STATUS_INFO_BREAK) || !m.found) return rt.status = W4A8_ERR_NODEV;
    rt.agent = m.agent;
    hsa_code_object_reader_t rd;
    const size_t co_bytes = (size_t)(w4a8_chain_plan_co_end - w4a8_chain_plan_co_begin);
    if (hsa_code_object_reader_create_from_memory(w4a8_chain_plan_co_begin, co_bytes, &rd) != HSA_STATUS_SUCCESS)
        return rt.status;
    if (hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, nullptr, &rt.exe) !=
            HSA_STATUS_SUCCESS ||
        hsa_executable_load_agent_code_object(rt.exe, rt.agent, rd, nullptr, nullptr) != HSA_STATUS_SUCCESS ||
        hsa_executable_freeze(rt.exe, nullptr) != HSA_STATUS_SUCCESS)
        return rt.status;
    for (int t = 0; t < 2; ++t)
        for (int v = 0; v < N_KERNELS; ++v) {
            const int kk = v / (4 * N_FORMATS), fmt = (v / 4) % N_FORMATS;
            if (!HAS_FORMAT[kk][fmt]) continue;
            hsa_executable_symbol_t sym;
            char name[64];
            std::snprintf(name, sizeof name, "w4a8_plan_%s_%s%s%s.kd", KIND_NAMES[kk], FORMAT_NAMES[fmt],
                          COH_NAMES[v % 4], t ? "_t" : "");
            uint32_t kargs = 0;
            if (hsa_executable_get_symbol_by_name(rt.exe, name, &rt.agent, &sym) != HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &rt.kobj[t][v]) !=
                    HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE,
                                               &rt.group[t][v]) != HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE,
                                               &rt.priv[t][v]) != HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, &kargs) !=
                    HSA_STATUS_SUCCESS)
                return rt.status;
            // The argument block written per step is all a kernel may read: one
            // that also read hidden arguments (grid sizes, code-object v5's
            // implicit block) would find zeros there, so refuse the code object.
            if (kargs != (t ? TIMED_ARGS_BYTES : sizeof(PlanArgs))) return rt.status;
        }
    for (int f = 0; f < 2; ++f)
        for (int c = 0; c < 4; ++c) {
            hsa_executable_symbol_t sym;
            char name[64];
            std::snprintf(name, sizeof name, "w4a8_plan_gemv_%s%s_s.kd", f ? "eng" : "f32", COH_NAMES[c]);
            uint32_t kargs = 0;
            if (hsa_executable_get_symbol_by_name(rt.exe, name, &rt.agent, &sym) != HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &rt.kobj_s[f][c]) !=
                    HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE,
                                               &rt.group_s[f][c]) != HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE,
                                               &rt.priv_s[f][c]) != HSA_STATUS_SUCCESS ||
                hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, &kargs) !=
                    HSA_STATUS_SUCCESS ||
                kargs != STREAM_ARGS_BYTES)
                return rt.status;
        }
    if (hsa_queue_create(rt.agent, QUEUE_PACKETS, HSA_QUEUE_TYPE_SINGLE, nullptr, nullptr, UINT32_MAX, UINT32_MAX,
                         &rt.queue) != HSA_STATUS_SUCCESS)
        return rt.status;
    return rt.status = W4A8_OK;
}

bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

}  // namespace

// A plan has no cache fences between its steps, so what a step writes may
// only be read back where the plan knows to read it from the coherence point:
// as another step's x. Everything else a step reads (its weights, norm_w) or
// writes besides y (the argmax row and workspace) must not lie in any step's
// y, and no step may read its own output as its x (its workgroups would race
// with each other).
int plan_check_ranges(const w4a8_plan_step *steps, int n) {
    for (int i = 0; i < n; ++i) {
        const w4a8_plan_step &s = steps[i];
        if (overlaps(s.x, x_bytes(s), s.y, y_bytes(s))) return W4A8_ERR_SHAPE;
        for (int j = 0; j < n; ++j) {
            const w4a8_plan_step &o = steps[j];
            const size_t w_bytes = (size_t)o.rows * (size_t)(o.k / QK) * Q4_0_BYTES;
            if (overlaps(o.w, w_bytes, s.y, y_bytes(s))) return W4A8_ERR_SHAPE;
            if (o.norm_w && overlaps(o.norm_w, 4 * (size_t)o.k, s.y, y_bytes(s))) return W4A8_ERR_SHAPE;
            if (o.kind == W4A8_PLAN_ARGMAX &&
                (overlaps(o.argmax, sizeof(int32_t), s.y, y_bytes(s)) ||
                 overlaps(o.workspace, argmax_workspace_bytes(), s.y, y_bytes(s))))
                return W4A8_ERR_SHAPE;
        }
    }
    return W4A8_OK;
}

int chain_plan_create(const w4a8_plan_step *steps, int n, bool overlapped, w4a8_chain_plan **out, hipError_t &he) {
    if (overlapped)
        for (int j = 0; j < n; ++j)
            if ((steps[j].kind != W4A8_PLAN_GEMV && steps[j].kind != W4A8_PLAN_GEMV_ENGINE) || steps[j].norm_w)
                return W4A8_ERR_SHAPE;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return W4A8_ERR_NODEV;
    DeviceRuntime *rt = nullptr;
    if (const int s = runtime_of(dev, rt)) return s;
    auto *p = new w4a8_chain_plan();
    p->device = dev;
    p->n = n;
    p->overlapped = overlapped;
    p->kind.assign(n, 0);
    // Which outputs another step reads, in this pass or the next: written
    // through, and read from the coherence point. Outputs that share bytes
    // with another step's output are written through as well: each step's
    // shape maps its rows to other workgroups, and so to other XCDs' L2s, so
    // the shared lines could otherwise sit dirty in two L2s at once, and the
    // launch's closing release would write both back in no defined order.
    std::vector<int> coh(n, 0);
    for (int j = 0; j < n; ++j)
        for (int i = 0; i < n; ++i) {
            if (overlaps(steps[j].x, x_bytes(steps[j]), steps[i].y, y_bytes(steps[i]))) {
                coh[j] |= COH_X;
                coh[i] |= COH_Y;
            }
            if (i != j && overlaps(steps[j].y, y_bytes(steps[j]), steps[i].y, y_bytes(steps[i]))) {
                coh[j] |= COH_Y;
                coh[i] |= COH_Y;
            }
        }
    const int cus = device_cu_count();
    std::vector<PlanArgs> args(n);
    for (int j = 0; j < n; ++j) {
        const w4a8_plan_step &s = steps[j];
        const bool rms = s.norm_w != nullptr;
        const int fmt = x_format(s);
        const XFormat xf = fmt == FMT_ENG ? X_ENGINE : (rms ? X_RMS : X_F32);
        p->kind[j] = kernel_index(kernel_kind(s), fmt, coh[j]);
        const int C = s.k / 256, rpw = 64 / C, tiles = (s.rows + rpw - 1) / rpw;
        M1Shape sh = gemv_m1_shape(tiles, s.k, xf, s.kind == W4A8_PLAN_ARGMAX, cus);
        if (s.kind == W4A8_PLAN_GATE_UP_SILU || s.kind == W4A8_PLAN_GATE_UP_SILU_Q8) {
            // gate|up's shape (launch_gemv_gate_up_silu): workgroups of waves / 2
            // gate waves and their up partners, one tile each.
            const int waves = gate_up_silu_waves(s.rows, s.k);
            sh.grid = tiles / 2 / (waves / 2);
            sh.threads = 64 * waves;
            sh.lds = (size_t)waves * TILE_BYTES + x_lds_bytes(s.k / QK) + (rms ? rms_sq_doubles(s.k) * 8 + 16 : 0);
        }
        PlanArgs a;
        std::memset(&a, 0, sizeof a);
        a.w0 = static_cast<const uint8_t *>(s.w);
        a.x = s.x;
        a.rows = s.rows;
        a.k = s.k;
        a.C = C;
        a.rpw = rpw;
        a.tiles = tiles;
        a.nblocks = sh.grid;
        a.nthreads = sh.threads;
        for (int g = 0; g < 4; ++g) a.P.seg[g] = a.w0;
        a.P.x = s.x;
        a.P.y = static_cast<float *>(s.y);
        a.P.seg_rows = s.rows;
        a.P.nseg = 1;
        a.P.k = s.k;
        a.P.rows = s.rows;
        a.P.C = C;
        a.P.rpw = rpw;
        a.P.tiles = tiles;
        a.P.norm_w = s.norm_w;
        a.P.eps = s.eps;
        if (s.kind == W4A8_PLAN_ARGMAX) {
            a.P.argmax = s.argmax;
            a.P.ticket = static_cast<unsigned int *>(s.workspace);
            a.P.key = reinterpret_cast<unsigned long long *>(static_cast<uint8_t *>(s.workspace) + ARGMAX_KEY_OFFSET);
        }
        args[j] = a;
        p->grid.push_back((uint32_t)sh.grid);
        p->threads.push_back((uint32_t)sh.threads);
        p->group.push_back((uint32_t)sh.lds);
    }
    std::vector<char> host((size_t)n * ARG_STRIDE, 0);
    for (int j = 0; j < n; ++j) std::memcpy(host.data() + (size_t)j * ARG_STRIDE, &args[j], sizeof(PlanArgs));
    if (overlapped) {
        // Flag bytes: each step's run 256-byte aligned, then the abort word;
        // all zero (no instance finished yet).
        std::vector<size_t> off(n);
        size_t total = 0;
        for (int j = 0; j < n; ++j) {
            off[j] = total;
            total += ((size_t)p->grid[j] + 255) / 256 * 256;
        }
        hipError_t fe = hipMalloc(&p->flags, total + 256);
        if (fe == hipSuccess) fe = hipMemset(p->flags, 0, total + 256);
        if (fe == hipSuccess) fe = hipDeviceSynchronize();
        if (fe != hipSuccess) {
            if (p->flags) (void)hipFree(p->flags);
            delete p;
            he = fe;
            return W4A8_ERR_HIP;
        }
        p->abort_word = reinterpret_cast<uint32_t *>(p->flags + total);
        for (int j = 0; j < n; ++j) {
            StreamSync S{};
            S.prev = j > 0 ? p->flags + off[j - 1] : nullptr;
            S.mine = p->flags + off[j];
            S.abort = p->abort_word;
            S.prev_groups = j > 0 ? (int)p->grid[j - 1] : 0;
            S.spin_limit = STREAM_SPIN_LIMIT;
            std::memcpy(host.data() + (size_t)j * ARG_STRIDE + sizeof(PlanArgs), &S, sizeof S);
        }
    }
    hipError_t e = hipMalloc(&p->kargs, host.size());
    if (e == hipSuccess) e = hipMemcpy(p->kargs, host.data(), host.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (p->kargs) (void)hipFree(p->kargs);
        if (p->flags) (void)hipFree(p->flags);
        delete p;
        he = e;
        return W4A8_ERR_HIP;
    }
    p->kargs_host = std::move(host);
    if (hsa_signal_create(0, 0, nullptr, &p->done) != HSA_STATUS_SUCCESS) {
        (void)hipFree(p->kargs);
        if (p->flags) (void)hipFree(p->flags);
        delete p;
        return W4A8_ERR_HSA;
    }
    *out = p;
    return W4A8_OK;
}

namespace {

// Writes `passes` passes of the plan's dispatches to its device's queue:
// every packet with the barrier bit (step j + 1 starts after step j ends),
// fence scope none except an acquire at system scope on the first packet and
// a release at system scope on the last, which carries the plan's completion
// signal. `kargs_of(i)` is dispatch i's argument block; TIMED selects the
// timed twins.
template <bool TIMED, class KArgs>
int issue(w4a8_chain_plan *p, int passes, KArgs kargs_of) {
    DeviceRuntime *rt = nullptr;
    if (const int s = runtime_of(p->device, rt)) return s;
    std::lock_guard<std::mutex> lk(rt->m);
    if (rt->stalled) return W4A8_ERR_TIMEOUT;
    hsa_queue_t *q = rt->queue;
    const long total = (long)passes * p->n;
    hsa_signal_add_relaxed(p->done, 1);
    uint64_t idx = hsa_queue_load_write_index_relaxed(q);
    for (long i = 0; i < total; ++i, ++idx) {
        const int j = (int)(i % p->n);
        const plan_ring::Room room = plan_ring::wait_for_room(
            idx, q->size, [q] { return hsa_queue_load_read_index_scacquire(q); },
            [q](uint64_t last) { hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)last); },
            QUEUE_STALL_S);
        if (room != plan_ring::Room::OK) {
            // The device has taken no packet for QUEUE_STALL_S: it is stalled.
            // No slot is claimed past the packets written (the queue stays
            // well formed), but this launch's last packet, the one carrying
            // the completion signal, is not among them: the plan's wait and
            // destroy report the timeout rather than free argument blocks
            // that queued packets still point at, and every later launch on
            // the device fails at once.
            rt->stalled = true;
            return W4A8_ERR_TIMEOUT;
        }
        auto *pk = reinterpret_cast<hsa_kernel_dispatch_packet_t *>(q->base_address) + (idx & (q->size - 1));
        std::memset(reinterpret_cast<char *>(pk) + 4, 0, sizeof(*pk) - 4);
        const int v = p->kind[j];
        // Overlapped plans (not the timed launch): every step but the first
        // of a pass without the barrier bit; its kernel waits for the step
        // before. The plain GEMV's variant index is (format) * 4 + coherence.
        const bool stream = p->overlapped && !TIMED;
        const int sf = (v / 4) % N_FORMATS == FMT_ENG ? 1 : 0, sc = v % 4;
        pk->workgroup_size_x = (uint16_t)p->threads[j];
        pk->workgroup_size_y = 1;
        pk->workgroup_size_z = 1;
        pk->grid_size_x = p->grid[j] * p->threads[j];
        pk->grid_size_y = 1;
        pk->grid_size_z = 1;
        pk->private_segment_size = stream ? rt->priv_s[sf][sc] : rt->priv[TIMED][v];
        pk->group_segment_size = (stream ? rt->group_s[sf][sc] : rt->group[TIMED][v]) + p->group[j];
        pk->kernel_object = stream ? rt->kobj_s[sf][sc] : rt->kobj[TIMED][v];
        pk->kernarg_address = kargs_of(i);
        const bool first = i == 0, last = i == total - 1;
        if (last) pk->completion_signal = p->done;
        const bool barrier = !stream || j == 0;
        const uint16_t header =
            (uint16_t)((HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) | ((barrier ? 1 : 0) << HSA_PACKET_HEADER_BARRIER) |
                       ((first ? HSA_FENCE_SCOPE_SYSTEM : HSA_FENCE_SCOPE_NONE) << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                       ((last ? HSA_FENCE_SCOPE_SYSTEM : HSA_FENCE_SCOPE_NONE) << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE));
        const uint32_t setup = 1u << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS;
        __atomic_store_n(&pk->full_header, (uint32_t)header | (setup << 16), __ATOMIC_RELEASE);
        hsa_queue_store_write_index_relaxed(q, idx + 1);
        if (plan_ring::ring_after(idx, q->size, j, p->n))
            hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
    }
    return W4A8_OK;
}

}  // namespace

int chain_plan_steps(const w4a8_chain_plan *p) { return p->n; }

int chain_plan_launch(w4a8_chain_plan *p, int passes) {
    return issue<false>(p, passes, [p](long i) { return p->kargs + (size_t)(i % p->n) * ARG_STRIDE; });
}

long chain_plan_workgroups(const w4a8_chain_plan *p, int step) {
    if (step >= 0) return step < p->n ? (long)p->grid[step] : -1;
    long w = 0;
    for (int j = 0; j < p->n; ++j) w += p->grid[j];
    return w;
}

int chain_plan_launch_timed(w4a8_chain_plan *p, int passes, unsigned long long *stamps, hipError_t &he) {
    // The argument blocks of an earlier timed launch may be rewritten below.
    if (const int s = chain_plan_wait(p, 10000)) return s;
    const size_t total = (size_t)passes * (size_t)p->n;
    const size_t bytes = total * ARG_STRIDE;
    // Every dispatch gets its own argument block (its stamp slots differ).
    // They go to device memory: blocks the packet processor has not read
    // before are then one device read each, as the plain launch's are.
    if (p->timed_bytes < bytes) {
        if (p->timed_kargs) (void)hipFree(p->timed_kargs);
        p->timed_kargs = nullptr;
        p->timed_bytes = 0;
        if ((he = hipMalloc(&p->timed_kargs, bytes)) != hipSuccess) {
            p->timed_kargs = nullptr;
            return W4A8_ERR_HIP;
        }
        p->timed_bytes = bytes;
    }
    // Dispatch i: step i % n's argument block, then the address of its
    // workgroups' slots (two words each, after those of the dispatches before).
    std::vector<char> host(bytes, 0);
    size_t slot = 0;
    for (size_t i = 0; i < total; ++i) {
        char *a = host.data() + i * ARG_STRIDE;
        const size_t j = i % (size_t)p->n;
        std::memcpy(a, p->kargs_host.data() + j * ARG_STRIDE, sizeof(PlanArgs));
        unsigned long long *st = stamps + 2 * slot;
        std::memcpy(a + sizeof(PlanArgs), &st, sizeof st);
        slot += p->grid[j];
    }
    if ((he = hipMemcpy(p->timed_kargs, host.data(), bytes, hipMemcpyHostToDevice)) != hipSuccess)
        return W4A8_ERR_HIP;
    return issue<true>(p, passes, [p](long i) { return p->timed_kargs + (size_t)i * ARG_STRIDE; });
}

int chain_plan_wait(w4a8_chain_plan *p, int timeout_ms) {
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        const hsa_signal_value_t v =
            hsa_signal_wait_scacquire(p->done, HSA_SIGNAL_CONDITION_LT, 1, 1000000, HSA_WAIT_STATE_ACTIVE);
        if (v < 1) break;
        if (std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() > timeout_ms)
            return W4A8_ERR_TIMEOUT;
    }
    if (p->overlapped) {
        // A step-to-step wait that gave up: the launch's outputs are not
        // valid. Reported once, the word cleared for the next launch.
        uint32_t aborted = 0;
        if (hipMemcpy(&aborted, p->abort_word, sizeof aborted, hipMemcpyDeviceToHost) != hipSuccess)
            return W4A8_ERR_HIP;
        if (aborted) {
            const uint32_t zero = 0;
            if (hipMemcpy(p->abort_word, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess) return W4A8_ERR_HIP;
            return W4A8_ERR_TIMEOUT;
        }
    }
    return W4A8_OK;
}

int chain_plan_destroy(w4a8_chain_plan *p) {
    const int s = chain_plan_wait(p, 10000);
    if (s != W4A8_OK) return s;   // work in flight: the plan stays valid
    hsa_signal_destroy(p->done);
    (void)hipFree(p->kargs);
    if (p->timed_kargs) (void)hipFree(p->timed_kargs);
    if (p->flags) (void)hipFree(p->flags);
    delete p;
    return W4A8_OK;
}

}  // namespace w4a8
