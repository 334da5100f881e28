// The reference's decode-side caller of the engine, on one GPU, written only
// against the reference driver's headers (gemv_dev.h, gemv2_dev.h, udmabuf.h)
// and linked against libkv260gemv.so: the evidence that board/tp's engine
// code runs unchanged on the MI355X, and the measurement of what a call costs
// as the board code sees it.
//
// What it reproduces, piece for piece (board/tp/tp_llama.cpp):
//   pools_t         :78-95    three udmabuf pools, largest first, one bump allocator
//   qmat, new_mat   :105-119, 210-224
//                             four quarters per matrix, 64 KB aligned, quarters 1
//                             and 3 used from 16 KB in; v2 stores rows through
//                             gemv2_chunk_offset, chunk by chunk
//   copy_rows       :190-197  q|k|v and gate|up fused into one matrix each (:258-268)
//   engine_t        :296-374  probe (gemv2 if present, else v1), open, prefetch of
//                             the next matrix, gemv = quantize x, clean x,
//                             invalidate y, start, wait, invalidate y
//   forward()       :822-883  the call order of one token: per layer q|k|v, o,
//                             gate|up, down, then the LM head and its argmax, each
//                             call naming the matrix that comes next
// with nranks = 1: every matrix unsplit, no exchange. The weights are synthetic
// Q4_0 blocks (seeded), written the way load_model writes GGUF tensors, and each
// call's activation is a fresh seeded float32 vector standing in for what
// rmsnorm / attention / silu would have produced.
//
// The activation quantizer is the contract's, src/llm_kv260/q4_0.py:83-97:
// d = amax / 127, inv = 1 / d (0 for d = 0), q = sign(s) floor(|s| + 0.5)
// with s = x inv, d stored through float16 (round to nearest even). It is the
// one the GPU engine is held to, so the outputs can be checked byte for byte.
// (tp_llama's NEON quantize_x rounds with vcvta; the two agree except where
// |s| + 0.5 rounds up in fp32.)
//
// With --gguf PATH the model comes from a GGUF file instead, as load_model
// reads it (:226-287): hyperparameters from the llama.* keys, and every Q4_0
// tensor's rows copied from the mapped file into the pools as they lie
// (q|k|v and gate|up fused, token_embd as the LM head). The file is read
// with the library's GGUF reader (include/w4a8_gguf.h), which stands where
// the reference uses llama.cpp's gguf API.
//
// Usage: engine_caller [--v1] [--tokens N] [--layers L] [--gguf PATH] [--dump DIR]
// Prints one JSON line with the per-call and per-token times. --dump DIR writes
// the first token's inputs and outputs of layer 0's q|k|v, o and down, and of
// the LM head, for an outside check.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <string>
#include <vector>

extern "C" {
#include "gemv2_dev.h"
#include "gemv_dev.h"
#include "udmabuf.h"
#include "w4a8_gguf.h"
}

#define DIE(...)                                       \
    do {                                               \
        fprintf(stderr, "engine_caller: " __VA_ARGS__); \
        fprintf(stderr, "\n");                         \
        exit(1);                                       \
    } while (0)

static double now() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

// ------------------------------------------------------------------ numbers

// xorshift64*: the seeded stream behind the synthetic weights and activations.
struct rng_t {
    uint64_t s;
    explicit rng_t(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    uint64_t next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 0x2545F4914F6CDD1Dull;
    }
    float uniform() { return (float)((next() >> 40) * (1.0 / 16777216.0)); }   // [0, 1)
    float normal() {                                                             // Box-Muller
        const float u = 1.0f - uniform(), v = uniform();
        return sqrtf(-2.0f * logf(u)) * cosf(6.2831853f * v);
    }
};

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// float -> binary16, round to nearest even, subnormals and overflow included.
static uint16_t f32_to_f16(float f) {
    const uint32_t u = f32_bits(f), sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);               // rounds past 65504
    if (a < 0x38800000u) {                                                  // below 2^-14: subnormal or 0
        // value = a_float; the half subnormal unit is 2^-24. Round a / 2^-24.
        const float q = bits_f32(a) * 16777216.0f;                          // exact: a power-of-two scale
        float r = nearbyintf(q);                                            // default mode: ties to even
        return (uint16_t)(sign | (uint32_t)r);
    }
    const uint32_t e = (a >> 23) - 127 + 15, m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;              // may carry into the exponent
    return (uint16_t)(sign | h);
}

static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0) return bits_f32(sign) + (sign ? -1.0f : 1.0f) * (float)m * 5.9604644775390625e-08f;
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

// ------------------------------------------------------------------ memory

// The three u-dma-buf pools, largest first, as one allocator.
struct pools_t {
    std::vector<udmabuf_t> p;
    void open() {
        for (const char *name : {"udmabuf0", "udmabuf1", "udmabuf2"}) {
            udmabuf_t b;
            if (udmabuf_open(&b, name) == 0) p.push_back(b);
        }
        if (p.empty()) DIE("no udmabuf pools (KV260GEMV_UDMABUF_SIZES)");
    }
    void *alloc(size_t size, uint64_t *phys, size_t align = 4096) {
        for (auto &b : p) {
            void *v = udmabuf_alloc(&b, size, align);
            if (v) {
                *phys = udmabuf_phys(&b, v);
                return v;
            }
        }
        DIE("out of pool memory allocating %zu MB", size >> 20);
    }
    void close() {
        for (auto &b : p) udmabuf_close(&b);
        p.clear();
    }
};

// A Q4_0 matrix in engine memory: four quarters of its rows, one per v1
// engine (or v2 port), each in its own 64 KB-aligned allocation, quarters 1
// and 3 used from 16 KB in.
struct qmat {
    uint8_t *q[4] = {};
    uint64_t qphys[4] = {};
    int rows = 0, k = 0;
    bool v2 = false;
    size_t bytes() const { return (size_t)rows * k / 32 * 18; }
    size_t row_bytes() const { return (size_t)k / 32 * 18; }
    uint8_t *chunk(int r, int c) const {
        const int R = rows / 4;
        if (!v2) return q[r / R] + (size_t)(r % R) * row_bytes() + (size_t)c * GEMV2_CHUNK_BYTES;
        int p;
        const size_t o = gemv2_chunk_offset(r, c, rows, k, &p);
        return q[p] + o;
    }
};

static qmat new_mat(pools_t &pools, int rows, int k, bool v2) {
    qmat m;
    m.rows = rows;
    m.k = k;
    m.v2 = v2;
    const size_t quarter = m.bytes() / 4, stagger = 16 << 10;
    for (int e = 0; e < 4; ++e) {
        const size_t off = (e & 1) * stagger;
        uint64_t phys;
        uint8_t *base = (uint8_t *)pools.alloc(quarter + off, &phys, 64 << 10);
        m.q[e] = base + off;
        m.qphys[e] = phys + off;
    }
    return m;
}

// Rows [r0, r0 + rows) of a row-major Q4_0 [N, K] tensor into rows dst_row.. of m.
static void copy_rows(qmat &m, const uint8_t *src, int k, int r0, int rows, int dst_row) {
    const size_t rb = (size_t)k / 32 * 18;
    const int nch = k / 256;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < nch; ++c)
            memcpy(m.chunk(dst_row + r, c), src + (size_t)(r0 + r) * rb + (size_t)c * GEMV2_CHUNK_BYTES,
                   GEMV2_CHUNK_BYTES);
}

// A synthetic Q4_0 tensor as GGUF would hold it: row-major 18-byte blocks,
// fp16 scales of N(0, 0.02) weights' size (d = max|w| / 8, about 0.005), random nibbles.
static std::vector<uint8_t> synth_tensor(int rows, int k, uint64_t seed) {
    std::vector<uint8_t> t((size_t)rows * k / 32 * 18);
    rng_t g(seed);
    for (size_t b = 0; b < t.size(); b += 18) {
        const uint16_t d = f32_to_f16((g.uniform() < 0.5f ? -1.0f : 1.0f) * (0.003f + 0.004f * g.uniform()));
        t[b] = (uint8_t)(d & 0xff);
        t[b + 1] = (uint8_t)(d >> 8);
        uint64_t lo = g.next(), hi = g.next();
        memcpy(&t[b + 2], &lo, 8);
        memcpy(&t[b + 10], &hi, 8);
    }
    return t;
}

// ------------------------------------------------------------------ engine

struct timing_t {
    double quant = 0, clean = 0, inv_before = 0, run = 0, inv_after = 0;
    long calls = 0;
};

struct engine_t {
    bool v2 = false;
    gemv_dev_t dev;
    gemv2_dev_t dev2;
    const qmat *pending = nullptr;     // gemv2: the matrix whose fetch has been started
    uint8_t *x;
    uint64_t x_phys;                   // int8[K] + float[K/32]
    float *y;
    uint64_t y_phys;                   // up to the LM head's rows
    timing_t t;

    void probe(bool want_v2) {
        if (want_v2 && gemv2_dev_open(&dev2) == 0) {
            v2 = true;
            if (!gemv2_mac_idle(&dev2)) DIE("gemv2 MAC kernel is busy");
            gemv2_drain(&dev2);
        } else if (gemv_dev_open(&dev)) {
            DIE("engine not available");
        }
    }
    void open(pools_t &pools, size_t y_floats) {
        x = (uint8_t *)pools.alloc(8192 + 256 * 4, &x_phys);
        y = (float *)pools.alloc(y_floats * 4, &y_phys);
    }
    void close() {
        if (v2) gemv2_dev_close(&dev2);
        else gemv_dev_close(&dev);
    }
    void prefetch(const qmat &W) {
        if (!v2 || pending == &W) return;
        if (pending) DIE("a prefetch of another matrix is pending");
        gemv2_fetch_start(&dev2, W.qphys, W.k, W.rows);
        pending = &W;
    }
    // Q8_0 of x into the engine layout int8[k] | float32[k/32] (q4_0.py:83-97).
    static void quantize_x(const float *xin, int8_t *qs, float *xd, int k) {
        for (int b = 0; b < k / 32; ++b) {
            const float *xb = xin + 32 * b;
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xb[j]));
            const float d = amax / 127.0f;
            const float inv = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < 32; ++j) {
                const float s = xb[j] * inv;
                const float mag = floorf(fabsf(s) + 0.5f);
                qs[32 * b + j] = (int8_t)(int)(s < 0.0f ? -mag : mag);
            }
            xd[b] = f16_to_f32(f32_to_f16(d));
        }
    }
    // y = W x, as engine_t::gemv: the result is left in this->y.
    void gemv(const qmat &W, const float *xin, const qmat *next) {
        const int k = W.k, nb = k / 32;
        double t0 = now();
        quantize_x(xin, (int8_t *)x, (float *)(x + k), k);
        double t1 = now();
        udmabuf_clean(x, (size_t)k + 4 * nb);
        double t2 = now();
        udmabuf_invalidate(y, (size_t)W.rows * 4);
        double t3 = now();
        if (v2) {
            prefetch(W);
            pending = nullptr;
            gemv2_mac_start(&dev2, x_phys, y_phys, k, W.rows);
            gemv2_mac_wait(&dev2);
            if (next) prefetch(*next);
        } else {
            gemv_dev_start4(&dev, W.qphys, x_phys, y_phys, k, W.rows);
            gemv_dev_wait(&dev);
        }
        double t4 = now();
        udmabuf_invalidate(y, (size_t)W.rows * 4);
        double t5 = now();
        t.quant += t1 - t0;
        t.clean += t2 - t1;
        t.inv_before += t3 - t2;
        t.run += t4 - t3;
        t.inv_after += t5 - t4;
        ++t.calls;
    }
};

// ------------------------------------------------------------------ model

// The model's shape at one rank (board/tp/tp_llama.cpp:231-243 with nranks = 1):
// Llama-3.2-1B unless a GGUF file says otherwise.
struct hparams {
    int n_layer = 16, n_embd = 2048, n_ff = 8192, n_head = 32, n_head_kv = 8, n_vocab = 128256;
    int head_dim() const { return n_embd / n_head; }
    int kv_rows() const { return n_head_kv * head_dim(); }
};

struct layer_w {
    qmat qkv, o, gateup, down;
};

// A GGUF file as load_model reads it (gguf_file, tp_llama.cpp:149-188).
struct gguf_file {
    w4a8_gguf *g = nullptr;
    void open(const char *path) {
        if (w4a8_gguf_open(path, &g) != 0) DIE("cannot read %s", path);
    }
    void close() { w4a8_gguf_close(g); }
    const uint8_t *data(const char *name, int rows, int k) const {
        const int64_t i = w4a8_gguf_find_tensor(g, name);
        if (i < 0) DIE("tensor %s missing", name);
        w4a8_gguf_tensor t;
        w4a8_gguf_tensor_info(g, i, &t);
        if (t.type != W4A8_GGML_TYPE_Q4_0 || t.n_dims != 2 || t.ne[0] != (uint64_t)k || t.ne[1] != (uint64_t)rows)
            DIE("tensor %s is not Q4_0 [%d, %d]", name, k, rows);
        return (const uint8_t *)w4a8_gguf_tensor_data(g, i);
    }
    uint32_t u32(const char *key) const {
        uint32_t v;
        if (w4a8_gguf_get_u32(g, key, &v) != 0) DIE("key %s missing", key);
        return v;
    }
};

static void write_file(const std::string &path, const void *p, size_t n) {
    FILE *f = fopen(path.c_str(), "wb");
    if (!f || fwrite(p, 1, n, f) != n) DIE("cannot write %s", path.c_str());
    fclose(f);
}

// Plain row-major bytes of m (undoing the quarters or the port layout).
static std::vector<uint8_t> plain_bytes(const qmat &m) {
    std::vector<uint8_t> out(m.bytes());
    const int nch = m.k / 256;
    for (int r = 0; r < m.rows; ++r)
        for (int c = 0; c < nch; ++c)
            memcpy(&out[(size_t)r * m.row_bytes() + (size_t)c * GEMV2_CHUNK_BYTES], m.chunk(r, c), GEMV2_CHUNK_BYTES);
    return out;
}

int main(int argc, char **argv) {
    bool want_v2 = true;
    int tokens = 8, layers_arg = 0;
    std::string dump, gguf;
    for (int i = 1; i < argc; ++i) {
        if (!strcmp(argv[i], "--v1")) want_v2 = false;
        else if (!strcmp(argv[i], "--tokens") && i + 1 < argc) tokens = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--layers") && i + 1 < argc) layers_arg = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--dump") && i + 1 < argc) dump = argv[++i];
        else if (!strcmp(argv[i], "--gguf") && i + 1 < argc) gguf = argv[++i];
        else DIE("usage: engine_caller [--v1] [--tokens N] [--layers L] [--gguf PATH] [--dump DIR]");
    }
    if (tokens < 1 || layers_arg < 0) DIE("need tokens >= 1 and layers >= 1");

    engine_t E;
    E.probe(want_v2);
    pools_t pools;
    pools.open();
    const double t_load0 = now();
    hparams h;
    gguf_file f;
    if (!gguf.empty()) {
        f.open(gguf.c_str());
        h.n_layer = (int)f.u32("llama.block_count");
        h.n_embd = (int)f.u32("llama.embedding_length");
        h.n_ff = (int)f.u32("llama.feed_forward_length");
        h.n_head = (int)f.u32("llama.attention.head_count");
        h.n_head_kv = (int)f.u32("llama.attention.head_count_kv");
        h.n_vocab = (int)f.u32("llama.vocab_size");
    }
    if (layers_arg > 0) h.n_layer = layers_arg < h.n_layer ? layers_arg : h.n_layer;
    const int Q_ROWS = h.n_embd, KV_ROWS = h.kv_rows();
    for (int v : {Q_ROWS + 2 * KV_ROWS, h.n_embd, 2 * h.n_ff, h.n_vocab})
        if (v % 32) DIE("rows %d not a multiple of 32", v);
    for (int v : {h.n_embd, h.n_ff})
        if (v % 256 || v > 8192) DIE("width %d unusable by the engine", v);

    // Row-major Q4_0 of one tensor: from the file, or synthetic and seeded.
    std::vector<uint8_t> scratch;
    uint64_t seed = 1000;
    char name[96];
    auto tensor = [&](int l, const char *what, int rows, int k) -> const uint8_t * {
        if (l >= 0) snprintf(name, sizeof name, "blk.%d.%s.weight", l, what);
        else snprintf(name, sizeof name, "%s.weight", what);
        if (f.g) return f.data(name, rows, k);
        scratch = synth_tensor(rows, k, seed++);
        return scratch.data();
    };
    std::vector<layer_w> layers(h.n_layer);
    size_t total = 0;
    for (int l = 0; l < h.n_layer; ++l) {
        layer_w &L = layers[l];
        L.qkv = new_mat(pools, Q_ROWS + 2 * KV_ROWS, h.n_embd, E.v2);
        copy_rows(L.qkv, tensor(l, "attn_q", Q_ROWS, h.n_embd), h.n_embd, 0, Q_ROWS, 0);
        copy_rows(L.qkv, tensor(l, "attn_k", KV_ROWS, h.n_embd), h.n_embd, 0, KV_ROWS, Q_ROWS);
        copy_rows(L.qkv, tensor(l, "attn_v", KV_ROWS, h.n_embd), h.n_embd, 0, KV_ROWS, Q_ROWS + KV_ROWS);
        L.o = new_mat(pools, h.n_embd, h.n_embd, E.v2);
        copy_rows(L.o, tensor(l, "attn_output", h.n_embd, h.n_embd), h.n_embd, 0, h.n_embd, 0);
        L.gateup = new_mat(pools, 2 * h.n_ff, h.n_embd, E.v2);
        copy_rows(L.gateup, tensor(l, "ffn_gate", h.n_ff, h.n_embd), h.n_embd, 0, h.n_ff, 0);
        copy_rows(L.gateup, tensor(l, "ffn_up", h.n_ff, h.n_embd), h.n_embd, 0, h.n_ff, h.n_ff);
        L.down = new_mat(pools, h.n_embd, h.n_ff, E.v2);
        copy_rows(L.down, tensor(l, "ffn_down", h.n_embd, h.n_ff), h.n_ff, 0, h.n_embd, 0);
        total += L.qkv.bytes() + L.o.bytes() + L.gateup.bytes() + L.down.bytes();
    }
    // The LM head is token_embd's rows (tp_llama.cpp:273-275).
    qmat lm_head = new_mat(pools, h.n_vocab, h.n_embd, E.v2);
    copy_rows(lm_head, tensor(-1, "token_embd", h.n_vocab, h.n_embd), h.n_embd, 0, h.n_vocab, 0);
    total += lm_head.bytes();
    scratch.clear();
    scratch.shrink_to_fit();
    if (f.g) f.close();
    E.open(pools, (size_t)h.n_vocab);
    // Everything the engine reads was written by the CPU: clean once.
    for (auto &p : pools.p) udmabuf_clean(p.base, p.used);
    const double t_load = now() - t_load0;
    const int n_layer = h.n_layer, N_EMBD = h.n_embd, N_FF = h.n_ff, N_VOCAB = h.n_vocab;

    std::vector<float> x(N_FF);
    rng_t gx(7);
    auto fresh_x = [&](int k) {
        for (int i = 0; i < k; ++i) x[i] = gx.normal();
        return x.data();
    };
    auto dump_call = [&](const char *name, const qmat &W, const float *xin) {
        if (dump.empty()) return;
        write_file(dump + "/" + name + ".x.f32", xin, (size_t)W.k * 4);
        write_file(dump + "/" + name + ".y.f32", E.y, (size_t)W.rows * 4);
        const std::vector<uint8_t> w = plain_bytes(W);
        write_file(dump + "/" + name + ".w.q4_0", w.data(), w.size());
        FILE *f = fopen((dump + "/" + name + ".shape").c_str(), "w");
        if (!f) DIE("cannot write the shape of %s", name);
        fprintf(f, "%d %d\n", W.rows, W.k);
        fclose(f);
    };

    std::vector<double> token_s;
    int argmax = -1;
    timing_t warm{};
    for (int tok = 0; tok < tokens + 1; ++tok) {            // token 0 warms up and is not timed
        const double t0 = now();
        for (int l = 0; l < n_layer; ++l) {
            layer_w &L = layers[l];
            const float *xi = fresh_x(N_EMBD);
            E.gemv(L.qkv, xi, &L.o);
            if (tok == 0 && l == 0) dump_call("qkv", L.qkv, xi);
            xi = fresh_x(N_EMBD);
            E.gemv(L.o, xi, &L.gateup);
            if (tok == 0 && l == 0) dump_call("o", L.o, xi);
            xi = fresh_x(N_EMBD);
            E.gemv(L.gateup, xi, &L.down);
            xi = fresh_x(N_FF);
            E.gemv(L.down, xi, l + 1 < n_layer ? &layers[l + 1].qkv : &lm_head);
            if (tok == 0 && l == 0) dump_call("down", L.down, xi);
        }
        const float *xi = fresh_x(N_EMBD);
        E.gemv(lm_head, xi, &layers[0].qkv);
        int best = 0;
        for (int i = 1; i < N_VOCAB; ++i)
            if (E.y[i] > E.y[best]) best = i;
        if (tok == 0) {
            argmax = best;
            dump_call("lm_head", lm_head, xi);
            warm = E.t;
        }
        if (tok > 0) token_s.push_back(now() - t0);
    }
    if (E.v2) gemv2_drain(&E.dev2);

    const timing_t &T = E.t;
    const double calls = (double)(T.calls - warm.calls);
    auto per_call_us = [&](double a, double b) { return (a - b) / calls * 1e6; };
    double sum = 0;
    for (double s : token_s) sum += s;
    const double tok_ms = sum / token_s.size() * 1e3;
    printf("{\"engine\": \"%s\", \"layers\": %d, \"tokens_timed\": %zu, \"calls_per_token\": %d, "
           "\"weight_bytes\": %zu, \"load_s\": %.3f, \"ms_per_token\": %.4f, \"tokens_per_s\": %.2f, "
           "\"us_per_call\": {\"quantize\": %.3f, \"clean_x\": %.3f, \"invalidate_y_before\": %.3f, "
           "\"start_wait\": %.3f, \"invalidate_y_after\": %.3f, \"total\": %.3f}, \"first_token_argmax\": %d}\n",
           E.v2 ? "gemv2" : "gemv_q4_0", n_layer, token_s.size(), 4 * n_layer + 1, total, t_load, tok_ms,
           1e3 / tok_ms, per_call_us(T.quant, warm.quant), per_call_us(T.clean, warm.clean),
           per_call_us(T.inv_before, warm.inv_before), per_call_us(T.run, warm.run),
           per_call_us(T.inv_after, warm.inv_after),
           per_call_us(T.quant + T.clean + T.inv_before + T.run + T.inv_after,
                       warm.quant + warm.clean + warm.inv_before + warm.run + warm.inv_after),
           argmax);
    E.close();
    pools.close();
    return 0;
}
