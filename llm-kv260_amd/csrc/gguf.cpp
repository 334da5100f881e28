// GGUF v2/v3 reader and in-place tensor upload (include/w4a8_gguf.h): the
// model-file surface the reference takes from llama.cpp's gguf API
// (board/tp/tp_llama.cpp:149-188). The file is mapped read-only and parsed
// with every read bounds-checked against the map, so a truncated or
// malformed file is an error status, never a read past the end.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <unordered_set>
#include <vector>

#include "../../include/w4a8.h"
#include "../../include/w4a8_gguf.h"

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;   // "GGUF" read as a little-endian u32
constexpr uint32_t DEFAULT_ALIGNMENT = 32;
constexpr int MAX_ARRAY_DEPTH = 8;

struct Kv {
    std::string key;
    uint32_t type = 0, elem_type = 0;
    uint64_t count = 0;
    const uint8_t *val = nullptr;   // the value's bytes in the map (after the type word)
};

struct Tensor {
    std::string name;
    uint32_t type = 0, n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
};

// Cursor over the map; any read past the end sets `bad` and yields zeros.
struct Reader {
    const uint8_t *p, *end;
    bool bad = false;
    bool take(void *dst, size_t n) {
        if (bad || (size_t)(end - p) < n) {
            bad = true;
            if (dst) memset(dst, 0, n);
            return false;
        }
        if (dst) memcpy(dst, p, n);
        p += n;
        return true;
    }
    uint32_t u32() {
        uint32_t v;
        take(&v, 4);
        return v;
    }
    uint64_t u64() {
        uint64_t v;
        take(&v, 8);
        return v;
    }
    bool str(std::string *out) {
        const uint64_t n = u64();
        if (bad || n > (uint64_t)(end - p)) return bad = true, false;
        if (out) out->assign(reinterpret_cast<const char *>(p), (size_t)n);
        p += n;
        return true;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case W4A8_GGUF_UINT8: case W4A8_GGUF_INT8: case W4A8_GGUF_BOOL: return 1;
        case W4A8_GGUF_UINT16: case W4A8_GGUF_INT16: return 2;
        case W4A8_GGUF_UINT32: case W4A8_GGUF_INT32: case W4A8_GGUF_FLOAT32: return 4;
        case W4A8_GGUF_UINT64: case W4A8_GGUF_INT64: case W4A8_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

// Step over one value of type t (arrays recursively).
bool skip_value(Reader &r, uint32_t t, int depth) {
    if (const size_t n = scalar_size(t)) return r.take(nullptr, n);
    if (t == W4A8_GGUF_STRING) return r.str(nullptr);
    if (t != W4A8_GGUF_ARRAY || depth >= MAX_ARRAY_DEPTH) return r.bad = true, false;
    const uint32_t et = r.u32();
    const uint64_t count = r.u64();
    if (r.bad) return false;
    if (const size_t n = scalar_size(et)) {
        if (count > (uint64_t)(r.end - r.p) / n) return r.bad = true, false;
        return r.take(nullptr, (size_t)(count * n));
    }
    for (uint64_t i = 0; i < count; ++i)
        if (!skip_value(r, et, depth + 1)) return false;
    return true;
}

// Data bytes of a tensor of a type the engine uses, 0 for other types, and
// UINT64_MAX when a used type's element or byte count overflows 64 bits (no
// file holds that many bytes, so the range check refuses the tensor).
uint64_t tensor_bytes(uint32_t type, const uint64_t ne[4]) {
    uint64_t per = 0, unit = 1;   // bytes per `unit` elements
    switch (type) {
        case W4A8_GGML_TYPE_F32: per = 4; break;
        case W4A8_GGML_TYPE_F16: per = 2; break;
        case W4A8_GGML_TYPE_Q4_0: per = 18, unit = 32; break;
        case W4A8_GGML_TYPE_Q8_0: per = 34, unit = 32; break;
        default: return 0;
    }
    if (ne[0] % unit) return 0;
    uint64_t n = 1;
    for (int d = 0; d < 4; ++d) {
        if (ne[d] && n > UINT64_MAX / ne[d]) return UINT64_MAX;
        n *= ne[d];
    }
    n /= unit;
    return n > UINT64_MAX / per ? UINT64_MAX : n * per;
}

}  // namespace

struct w4a8_gguf {
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = DEFAULT_ALIGNMENT;
    uint64_t data_offset = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
};

namespace {

int parse(w4a8_gguf &g) {
    Reader r{g.map, g.map + g.size};
    if (r.u32() != GGUF_MAGIC) return W4A8_ERR_FORMAT;
    g.version = r.u32();
    if (g.version != 2 && g.version != 3) return W4A8_ERR_FORMAT;   // v1 counted in u32
    const uint64_t n_tensors = r.u64(), n_kv = r.u64();
    // Each key/value takes at least 13 bytes of the file (key length, one
    // byte of value, type) and each tensor info at least 32, so larger counts
    // cannot fit: refuse them before reserving anything.
    if (r.bad || n_kv > g.size / 13 || n_tensors > g.size / 32) return W4A8_ERR_FORMAT;
    g.kv.reserve((size_t)n_kv);
    std::unordered_set<std::string> keys, names;
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv e;
        // A name with a NUL byte could not be asked for through the C API.
        if (!r.str(&e.key) || e.key.find('\0') != std::string::npos) return W4A8_ERR_FORMAT;
        e.type = r.u32();
        e.val = r.p;
        if (e.type == W4A8_GGUF_ARRAY) {
            Reader peek = r;
            e.elem_type = peek.u32();
            e.count = peek.u64();
        }
        if (!skip_value(r, e.type, 0)) return W4A8_ERR_FORMAT;
        if (!keys.insert(e.key).second) return W4A8_ERR_FORMAT;   // a key twice, as llama.cpp refuses too
        if (e.key == "general.alignment") {
            if (e.type != W4A8_GGUF_UINT32) return W4A8_ERR_FORMAT;
            memcpy(&g.alignment, e.val, 4);
            if (!g.alignment || (g.alignment & (g.alignment - 1))) return W4A8_ERR_FORMAT;
        }
        g.kv.push_back(std::move(e));
    }
    g.tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        if (!r.str(&t.name) || t.name.find('\0') != std::string::npos) return W4A8_ERR_FORMAT;
        if (!names.insert(t.name).second) return W4A8_ERR_FORMAT;   // a tensor name twice
        t.n_dims = r.u32();
        if (t.n_dims < 1 || t.n_dims > 4) return W4A8_ERR_FORMAT;
        for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = r.u64();
        t.type = r.u32();
        t.offset = r.u64();
        if (r.bad) return W4A8_ERR_FORMAT;
        t.nbytes = tensor_bytes(t.type, t.ne);
        if (t.offset % g.alignment) return W4A8_ERR_FORMAT;
        g.tensors.push_back(std::move(t));
    }
    const uint64_t header_end = (uint64_t)(r.p - g.map);
    g.data_offset = (header_end + g.alignment - 1) / g.alignment * g.alignment;
    if (g.data_offset > g.size) return W4A8_ERR_FORMAT;
    for (const Tensor &t : g.tensors)
        if (t.offset > g.size - g.data_offset || t.nbytes > g.size - g.data_offset - t.offset) return W4A8_ERR_FORMAT;
    return W4A8_OK;
}

const Kv *kv_of(const w4a8_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    for (const Kv &e : g->kv)
        if (e.key == key) return &e;
    return nullptr;
}

template <typename T>
int get_scalar(const w4a8_gguf *g, const char *key, uint32_t type, T *v) {
    if (!v) return W4A8_ERR_NULL;
    const Kv *e = kv_of(g, key);
    if (!e) return W4A8_ERR_SHAPE;
    if (e->type != type) return W4A8_ERR_FORMAT;
    memcpy(v, e->val, sizeof(T));
    return W4A8_OK;
}

}  // namespace

extern "C" {

int w4a8_gguf_open(const char *path, w4a8_gguf **out) {
    if (!path || !out) return W4A8_ERR_NULL;
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return W4A8_ERR_FORMAT;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return W4A8_ERR_FORMAT;
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return W4A8_ERR_FORMAT;
    w4a8_gguf *g = new (std::nothrow) w4a8_gguf;
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return W4A8_ERR_NULL;
    }
    g->map = static_cast<const uint8_t *>(m);
    g->size = (size_t)st.st_size;
    int s;
    try {
        s = parse(*g);
    } catch (const std::bad_alloc &) {   // names or tables too large for memory: no exception crosses the C ABI
        s = W4A8_ERR_FORMAT;
    }
    if (s != W4A8_OK) {
        w4a8_gguf_close(g);
        return s;
    }
    *out = g;
    return W4A8_OK;
}

void w4a8_gguf_close(w4a8_gguf *g) {
    if (!g) return;
    if (g->map) munmap(const_cast<uint8_t *>(g->map), g->size);
    delete g;
}

uint32_t w4a8_gguf_version(const w4a8_gguf *g) { return g ? g->version : 0; }
int64_t w4a8_gguf_n_tensors(const w4a8_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }
int64_t w4a8_gguf_n_kv(const w4a8_gguf *g) { return g ? (int64_t)g->kv.size() : 0; }
uint64_t w4a8_gguf_data_offset(const w4a8_gguf *g) { return g ? g->data_offset : 0; }

int64_t w4a8_gguf_find_key(const w4a8_gguf *g, const char *key) {
    if (!g || !key) return -1;
    for (size_t i = 0; i < g->kv.size(); ++i)
        if (g->kv[i].key == key) return (int64_t)i;
    return -1;
}

int64_t w4a8_gguf_find_tensor(const w4a8_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); ++i)
        if (g->tensors[i].name == name) return (int64_t)i;
    return -1;
}

const char *w4a8_gguf_key(const w4a8_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->kv.size()) return nullptr;
    return g->kv[(size_t)i].key.c_str();
}

int w4a8_gguf_kv_type(const w4a8_gguf *g, int64_t i, uint32_t *type, uint32_t *elem_type, uint64_t *count) {
    if (!g || !type) return W4A8_ERR_NULL;
    if (i < 0 || i >= (int64_t)g->kv.size()) return W4A8_ERR_SHAPE;
    const Kv &e = g->kv[(size_t)i];
    *type = e.type;
    if (elem_type) *elem_type = e.elem_type;
    if (count) *count = e.count;
    return W4A8_OK;
}

int w4a8_gguf_get_u32(const w4a8_gguf *g, const char *key, uint32_t *v) { return get_scalar(g, key, W4A8_GGUF_UINT32, v); }
int w4a8_gguf_get_i32(const w4a8_gguf *g, const char *key, int32_t *v) { return get_scalar(g, key, W4A8_GGUF_INT32, v); }
int w4a8_gguf_get_u64(const w4a8_gguf *g, const char *key, uint64_t *v) { return get_scalar(g, key, W4A8_GGUF_UINT64, v); }
int w4a8_gguf_get_f32(const w4a8_gguf *g, const char *key, float *v) { return get_scalar(g, key, W4A8_GGUF_FLOAT32, v); }

int w4a8_gguf_get_str(const w4a8_gguf *g, const char *key, const char **s, uint64_t *len) {
    if (!s || !len) return W4A8_ERR_NULL;
    const Kv *e = kv_of(g, key);
    if (!e) return W4A8_ERR_SHAPE;
    if (e->type != W4A8_GGUF_STRING) return W4A8_ERR_FORMAT;
    memcpy(len, e->val, 8);
    *s = reinterpret_cast<const char *>(e->val + 8);
    return W4A8_OK;
}

int w4a8_gguf_tensor_info(const w4a8_gguf *g, int64_t i, w4a8_gguf_tensor *info) {
    if (!g || !info) return W4A8_ERR_NULL;
    if (i < 0 || i >= (int64_t)g->tensors.size()) return W4A8_ERR_SHAPE;
    const Tensor &t = g->tensors[(size_t)i];
    info->name = t.name.c_str();
    info->type = t.type;
    info->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) info->ne[d] = t.ne[d];
    info->offset = t.offset;
    info->nbytes = t.nbytes;
    return W4A8_OK;
}

const void *w4a8_gguf_tensor_data(const w4a8_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
    return g->map + g->data_offset + g->tensors[(size_t)i].offset;
}

int w4a8_gguf_upload(const w4a8_gguf *g, int64_t i, void *dst, size_t cap, void *stream) {
    if (!g || !dst) return W4A8_ERR_NULL;
    if (i < 0 || i >= (int64_t)g->tensors.size()) return W4A8_ERR_SHAPE;
    const Tensor &t = g->tensors[(size_t)i];
    if (!t.nbytes || t.nbytes > cap) return W4A8_ERR_SHAPE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(dst, g->map + g->data_offset + t.offset, (size_t)t.nbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? W4A8_OK : W4A8_ERR_HIP;
}

}  // extern "C"
