// What one engine call costs on the MI355X, column for column against the
// reference's per-call table (board/kv260gemv/bench_calls.c, printed in
// docs/buildlog/evidence/0012-bench-calls.txt):
//
//   raw       gemv_dev_run alone through the reference ABI (gemv_dev.h): the
//             host-visible time of one synchronous call, best and mean of N
//   clean     udmabuf_clean of x (k + k/8 bytes host -> device), best
//   inval_y   udmabuf_invalidate of y (4 rows bytes device -> host), best
//   graph     the device-side time per call: N w4a8_gemv launches captured in
//             one HIP graph, replayed, HIP events around the replay, / N
//             (the kernel plus the launch boundary, no host in the loop)
//   start, wait  raw's two halves: gemv_dev_start (the enqueue) and gemv_dev_wait
//   launch_poll  w4a8_gemv on a stream, waited for by polling hipStreamQuery
//   q8        the standalone Q8_0 quantize of a float32 x (w4a8_quantize_q8_0,
//             the reference's q8ref / q8neon columns run on the CPU): host-
//             visible launch + stream sync, best and mean, and device-side
//             per launch from a graph
//
// Shapes: the reference's tiny / x2048 / x8192 rows (16 output rows), then
// the unsplit single-GPU shapes of the Llama-3.2-1B decode (one GPU holds
// the whole model, so no shard of four). Weights are valid Q4_0 blocks with
// seeded nibbles (timing does not depend on the values); each call is on the
// same buffers, as in the reference's table.
//
// Then the gemv2 table of board/kv260gemv/bench_gemv2.c:92-129 (evidence
// 0013-bench-gemv2.txt:14-20) at the same five model shapes: "cold" is
// gemv2_fetch_start + gemv2_mac_start + gemv2_mac_wait back to back, and
// the reference's "prefetched" protocol, the MAC alone 1 ms after the fetch
// was started (on the GPU the fetch only names the matrix, so this measures
// a call after 1 ms of host idle); beside them the v1 engine's gemv_dev_run
// back to back and after 1 ms of idle. Each call takes the next of several
// copies of the matrix (together more than the 256 MB Infinity Cache), so a
// call reads HBM. Last, a token's 65 calls with the next
// matrix fetched right after each MAC, with no gap and with a 300 us gap
// after each call (bench_gemv2.c:132-153), over 65 distinct matrices
// (695 MB).
//
// Usage: call_costs [--reps N]. Needs a pool of 1 GB
// (KV260GEMV_UDMABUF_SIZES=udmabuf0=1G). Prints one JSON line.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

extern "C" {
#include "gemv2_dev.h"
#include "gemv_dev.h"
#include "udmabuf.h"
#include "w4a8.h"
}

#define DIE(...)                                     \
    do {                                             \
        fprintf(stderr, "call_costs: " __VA_ARGS__); \
        fprintf(stderr, "\n");                       \
        exit(1);                                     \
    } while (0)

#define HIP_OK(e)                                                              \
    do {                                                                       \
        hipError_t err_ = (e);                                                 \
        if (err_ != hipSuccess) DIE("%s: %s", #e, hipGetErrorString(err_));    \
    } while (0)

static double now() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

struct Stat {
    double best = 1e30, sum = 0;
    int n = 0;
    void add(double s) {
        best = std::min(best, s);
        sum += s;
        ++n;
    }
    double best_us() const { return best * 1e6; }
    double mean_us() const { return n ? sum / n * 1e6 : 0; }
};

struct Shape {
    const char *name;
    int k, rows;
};

static uint64_t mix(uint64_t &s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1Dull;
}

int main(int argc, char **argv) {
    int reps = 200;
    for (int i = 1; i < argc; ++i) {
        if (!strcmp(argv[i], "--reps") && i + 1 < argc) reps = atoi(argv[++i]);
        else DIE("usage: call_costs [--reps N]");
    }
    if (reps < 1) DIE("--reps must be positive");
    const Shape shapes[] = {{"tiny", 256, 16},      {"x2048", 2048, 16},       {"x8192", 8192, 16},
                            {"qkv", 2048, 3072},    {"o", 2048, 2048},         {"gate_up", 2048, 16384},
                            {"down", 8192, 2048},   {"lm_head", 2048, 128256}};

    udmabuf_t pool;
    if (udmabuf_open(&pool, "udmabuf0")) DIE("no pool udmabuf0 (KV260GEMV_UDMABUF_SIZES)");
    gemv_dev_t dev;
    if (gemv_dev_open(&dev)) DIE("gemv_q4_0 engine not available");
    hipStream_t s;
    HIP_OK(hipStreamCreate(&s));
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));

    std::string out = "{\"reps\": " + std::to_string(reps) + ", \"shapes\": [";
    uint64_t seed = 12345;
    for (size_t si = 0; si < sizeof shapes / sizeof shapes[0]; ++si) {
        const Shape &sh = shapes[si];
        const size_t wbytes = (size_t)sh.rows * sh.k / 32 * 18, xbytes = sh.k + sh.k / 8, ybytes = 4ull * sh.rows;
        pool.used = 0;
        uint8_t *w = (uint8_t *)udmabuf_alloc(&pool, wbytes, 64 << 10);
        uint8_t *x = (uint8_t *)udmabuf_alloc(&pool, xbytes + 64, 4096);
        uint8_t *y = (uint8_t *)udmabuf_alloc(&pool, ybytes, 4096);
        float *xf = (float *)udmabuf_alloc(&pool, 4ull * sh.k, 4096);
        uint8_t *xq = (uint8_t *)udmabuf_alloc(&pool, xbytes, 4096);
        if (!w || !x || !y || !xf || !xq) DIE("pool too small for %s", sh.name);
        for (size_t b = 0; b < wbytes; b += 18) {          // scale 2^-10 (fp16 0x1400), seeded nibbles
            w[b] = 0x00;
            w[b + 1] = 0x14;
            for (int j = 2; j < 18; ++j) w[b + j] = (uint8_t)mix(seed);
        }
        for (int i = 0; i < sh.k; ++i) x[i] = (uint8_t)(mix(seed) % 255 + 129);   // int8 in -127..127
        for (int b = 0; b < sh.k / 32; ++b) {
            const float d = 1.0f / 64;
            memcpy(x + sh.k + 4 * b, &d, 4);
        }
        for (int i = 0; i < sh.k; ++i) xf[i] = (float)((int)(mix(seed) % 2001) - 1000) / 500.0f;
        udmabuf_clean(w, wbytes);
        udmabuf_clean(x, xbytes);
        udmabuf_clean(xf, 4ull * sh.k);
        const uint64_t wp = udmabuf_phys(&pool, w), xp = udmabuf_phys(&pool, x), yp = udmabuf_phys(&pool, y);
        const uint64_t xfp = udmabuf_phys(&pool, xf), xqp = udmabuf_phys(&pool, xq);

        // raw: one synchronous call through the reference ABI.
        Stat raw, clean, inval, q8host;
        for (int r = 0; r < 5; ++r) gemv_dev_run(&dev, wp, xp, yp, sh.k, sh.rows);
        for (int r = 0; r < reps; ++r) {
            const double a = now();
            gemv_dev_run(&dev, wp, xp, yp, sh.k, sh.rows);
            raw.add(now() - a);
        }
        for (int r = 0; r < reps; ++r) {
            double a = now();
            udmabuf_clean(x, xbytes);
            clean.add(now() - a);
            a = now();
            udmabuf_invalidate(y, ybytes);
            inval.add(now() - a);
        }
        // The parts of raw: the enqueue alone (gemv_dev_start), then the wait;
        // and the same launch waited for by polling the stream instead.
        Stat enq, wait, poll;
        for (int r = 0; r < reps; ++r) {
            double a = now();
            gemv_dev_start(&dev, wp, xp, yp, sh.k, sh.rows);
            const double b = now();
            gemv_dev_wait(&dev);
            enq.add(b - a);
            wait.add(now() - b);
        }
        for (int r = 0; r < reps; ++r) {
            const double a = now();
            if (w4a8_gemv((const void *)wp, (const void *)xp, (float *)yp, sh.rows, sh.k, s)) DIE("w4a8_gemv");
            hipError_t q;
            while ((q = hipStreamQuery(s)) == hipErrorNotReady) {
            }
            HIP_OK(q);
            poll.add(now() - a);
        }
        // q8: the standalone quantize, launch + sync, host-visible.
        for (int r = 0; r < 5; ++r)
            if (w4a8_quantize_q8_0((const float *)xfp, (void *)xqp, sh.k, 1, s)) DIE("quantize %s", sh.name);
        HIP_OK(hipStreamSynchronize(s));
        for (int r = 0; r < reps; ++r) {
            const double a = now();
            w4a8_quantize_q8_0((const float *)xfp, (void *)xqp, sh.k, 1, s);
            HIP_OK(hipStreamSynchronize(s));
            q8host.add(now() - a);
        }

        // graph: device-side per call, for the GEMV and for the quantize.
        auto graph_us = [&](bool quantize) {
            const int n = 50;
            hipGraph_t g;
            hipGraphExec_t ge;
            HIP_OK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < n; ++i) {
                const int rc = quantize ? w4a8_quantize_q8_0((const float *)xfp, (void *)xqp, sh.k, 1, s)
                                        : w4a8_gemv((const void *)wp, (const void *)xp, (float *)yp, sh.rows, sh.k, s);
                if (rc) DIE("launch under capture (%s): %d", sh.name, rc);
            }
            HIP_OK(hipStreamEndCapture(s, &g));
            HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            const int replays = std::max(2, std::min(20, reps / 10));
            HIP_OK(hipGraphLaunch(ge, s));
            HIP_OK(hipStreamSynchronize(s));
            HIP_OK(hipEventRecord(e0, s));
            for (int i = 0; i < replays; ++i) HIP_OK(hipGraphLaunch(ge, s));
            HIP_OK(hipEventRecord(e1, s));
            HIP_OK(hipEventSynchronize(e1));
            float ms = 0;
            HIP_OK(hipEventElapsedTime(&ms, e0, e1));
            HIP_OK(hipGraphExecDestroy(ge));
            HIP_OK(hipGraphDestroy(g));
            return ms * 1e3 / (replays * n);
        };
        const double gemv_graph = graph_us(false), q8_graph = graph_us(true);

        char buf[1024];
        snprintf(buf, sizeof buf,
                 "%s{\"shape\": \"%s\", \"k\": %d, \"rows\": %d, \"weight_mb\": %.3f, \"raw_best_us\": %.2f, "
                 "\"raw_mean_us\": %.2f, \"raw_gbps\": %.2f, \"graph_us\": %.3f, \"clean_x_us\": %.2f, "
                 "\"inval_y_us\": %.2f, \"q8_host_best_us\": %.2f, \"q8_host_mean_us\": %.2f, \"q8_graph_us\": %.3f, "
                 "\"start_us\": %.2f, \"wait_us\": %.2f, \"launch_poll_us\": %.2f}",
                 si ? ", " : "", sh.name, sh.k, sh.rows, wbytes / 1e6, raw.best_us(), raw.mean_us(),
                 wbytes / raw.best / 1e9, gemv_graph, clean.best_us(), inval.best_us(), q8host.best_us(),
                 q8host.mean_us(), q8_graph, enq.best_us(), wait.best_us(), poll.best_us());
        out += buf;
        fprintf(stderr, "call_costs: %-8s raw %.2f us (mean %.2f), graph %.3f us, q8 %.2f us host / %.3f us graph\n",
                sh.name, raw.best_us(), raw.mean_us(), gemv_graph, q8host.best_us(), q8_graph);
    }
    out += "]";

    // ------------------------------------------------------------- gemv2
    gemv2_dev_t dev2;
    if (gemv2_dev_open(&dev2)) DIE("gemv2 engine not available");
    struct Mat {
        uint64_t port[4];
        uint64_t plain;
    };
    // Four 64 KB-aligned port regions, ports 1 and 3 from 16 KB in
    // (bench_gemv2.c:29-40), plus the same bytes as one plain matrix for v1.
    auto new_mat = [&](int rows, int k, bool plain) {
        Mat m{};
        const size_t quarter = (size_t)rows / 4 * k / 32 * 18;
        for (int p = 0; p < 4; ++p) {
            const size_t off = (p & 1) * (16 << 10);
            uint8_t *b = (uint8_t *)udmabuf_alloc(&pool, quarter + off, 64 << 10);
            if (!b) DIE("pool too small for the gemv2 matrices (rows %d)", rows);
            m.port[p] = udmabuf_phys(&pool, b) + off;
        }
        if (plain) {
            uint8_t *b = (uint8_t *)udmabuf_alloc(&pool, 4 * quarter, 64 << 10);
            if (!b) DIE("pool too small for the gemv2 matrices (rows %d)", rows);
            m.plain = udmabuf_phys(&pool, b);
        }
        return m;
    };
    const Shape model[] = {{"qkv", 2048, 3072}, {"o", 2048, 2048}, {"gate_up", 2048, 16384},
                           {"down", 8192, 2048}, {"lm_head", 2048, 128256}};
    out += ", \"gemv2\": [";
    for (size_t si = 0; si < sizeof model / sizeof model[0]; ++si) {
        const Shape &sh = model[si];
        pool.used = 0;
        uint8_t *x = (uint8_t *)udmabuf_alloc(&pool, sh.k + sh.k / 8 + 64, 4096);
        uint8_t *y = (uint8_t *)udmabuf_alloc(&pool, 4ull * sh.rows, 4096);
        if (!x || !y) DIE("pool");
        memset(x, 0, sh.k + sh.k / 8);
        udmabuf_clean(x, sh.k + sh.k / 8);
        const uint64_t xp = udmabuf_phys(&pool, x), yp = udmabuf_phys(&pool, y);
        const size_t wbytes = (size_t)sh.rows * sh.k / 32 * 18;
        // Copies of the port regions together well past the 256 MB cache (and
        // the plain copies likewise), within a 1 GB pool.
        const int copies = (int)std::min<size_t>((900ull << 20) / (2 * wbytes),
                                                 std::max<size_t>(2, ((600ull << 20) + wbytes - 1) / wbytes));
        std::vector<Mat> mats;
        for (int c = 0; c < copies; ++c) mats.push_back(new_mat(sh.rows, sh.k, true));
        const int n = wbytes > (100u << 20) ? 12 : 60;
        Stat cold, pre, v1, v1_idle;
        for (int r = 0; r < n + 2; ++r) {
            const Mat &m = mats[r % copies];
            double a = now();
            gemv2_fetch_start(&dev2, m.port, sh.k, sh.rows);
            gemv2_mac_start(&dev2, xp, yp, sh.k, sh.rows);
            gemv2_mac_wait(&dev2);
            if (r >= 2) cold.add(now() - a);
        }
        for (int r = 0; r < n + 2; ++r) {
            const Mat &m = mats[r % copies];
            gemv2_fetch_start(&dev2, m.port, sh.k, sh.rows);
            usleep(1000);
            double a = now();
            gemv2_mac_start(&dev2, xp, yp, sh.k, sh.rows);
            gemv2_mac_wait(&dev2);
            if (r >= 2) pre.add(now() - a);
        }
        for (int r = 0; r < n + 2; ++r) {
            const Mat &m = mats[r % copies];
            double a = now();
            gemv_dev_run(&dev, m.plain, xp, yp, sh.k, sh.rows);
            if (r >= 2) v1.add(now() - a);
        }
        for (int r = 0; r < n + 2; ++r) {     // the same after 1 ms of host idle, as the prefetched MAC
            const Mat &m = mats[r % copies];
            usleep(1000);
            double a = now();
            gemv_dev_run(&dev, m.plain, xp, yp, sh.k, sh.rows);
            if (r >= 2) v1_idle.add(now() - a);
        }
        char buf[512];
        snprintf(buf, sizeof buf,
                 "%s{\"shape\": \"%s\", \"k\": %d, \"rows\": %d, \"weight_mb\": %.3f, \"copies\": %d, "
                 "\"cold_best_us\": %.2f, \"cold_gbps\": %.1f, \"after_1ms_best_us\": %.2f, \"after_1ms_gbps\": %.1f, "
                 "\"v1_cold_best_us\": %.2f, \"v1_after_idle_best_us\": %.2f}",
                 si ? ", " : "", sh.name, sh.k, sh.rows, wbytes / 1e6, copies, cold.best_us(), wbytes / cold.best / 1e9,
                 pre.best_us(), wbytes / pre.best / 1e9, v1.best_us(), v1_idle.best_us());
        out += buf;
        fprintf(stderr, "call_costs: gemv2 %-8s cold %.2f us, 1 ms after the fetch %.2f us, v1 %.2f us, v1 after 1 ms idle %.2f us\n",
                sh.name, cold.best_us(), pre.best_us(), v1.best_us(), v1_idle.best_us());
    }
    out += "]";

    // A token: 16 x (q|k|v, o, gate|up, down) + LM head, 65 distinct matrices,
    // the next one fetched right after each MAC.
    {
        pool.used = 0;
        uint8_t *x = (uint8_t *)udmabuf_alloc(&pool, 8192 + 1024 + 64, 4096);
        uint8_t *y = (uint8_t *)udmabuf_alloc(&pool, 4 * 128256, 4096);
        if (!x || !y) DIE("pool");
        const uint64_t xp = udmabuf_phys(&pool, x), yp = udmabuf_phys(&pool, y);
        std::vector<Mat> seq;
        std::vector<int> si;
        for (int l = 0; l < 16; ++l)
            for (int j = 0; j < 4; ++j) {
                seq.push_back(new_mat(model[j].rows, model[j].k, false));
                si.push_back(j);
            }
        seq.push_back(new_mat(model[4].rows, model[4].k, false));
        si.push_back(4);
        out += ", \"token\": [";
        for (int gi = 0; gi < 2; ++gi) {
            const int gap = gi ? 300 : 0;
            double best_mac = 1e30, best_wall = 1e30;
            for (int rep = 0; rep < 4; ++rep) {
                double mac = 0;
                const double w0 = now();
                gemv2_fetch_start(&dev2, seq[0].port, model[si[0]].k, model[si[0]].rows);
                for (int c = 0; c < 65; ++c) {
                    const Shape &sh = model[si[c]];
                    const double a = now();
                    gemv2_mac_start(&dev2, xp, yp, sh.k, sh.rows);
                    gemv2_mac_wait(&dev2);
                    mac += now() - a;
                    if (c + 1 < 65) gemv2_fetch_start(&dev2, seq[c + 1].port, model[si[c + 1]].k, model[si[c + 1]].rows);
                    if (gap) usleep(gap);
                }
                best_mac = std::min(best_mac, mac);
                best_wall = std::min(best_wall, now() - w0);
            }
            char buf[256];
            snprintf(buf, sizeof buf, "%s{\"gap_us\": %d, \"mac_ms\": %.3f, \"wall_ms\": %.3f}", gi ? ", " : "", gap,
                     best_mac * 1e3, best_wall * 1e3);
            out += buf;
            fprintf(stderr, "call_costs: token, %d us gap: MAC time %.3f ms, wall %.3f ms\n", gap, best_mac * 1e3,
                    best_wall * 1e3);
        }
        out += "]";
        gemv2_drain(&dev2);
    }
    gemv2_dev_close(&dev2);
    out += "}";
    printf("%s\n", out.c_str());
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    HIP_OK(hipStreamDestroy(s));
    gemv_dev_close(&dev);
    udmabuf_close(&pool);
    return 0;
}
