/*
 * w4a8_gguf.h -- GGUF model files for the MI355X W4A8 engine (libkv260gemv.so).
 *
 * The reference loads its weights from GGUF through llama.cpp's gguf API
 * (board/tp/tp_llama.cpp:149-188: gguf_init_from_file, gguf_find_key,
 * gguf_get_val_u32 / _f32, gguf_find_tensor, gguf_get_data_offset +
 * gguf_get_tensor_offset into an mmap of the file), then copies each Q4_0
 * tensor's rows into engine memory as they lie (copy_rows / copy_cols,
 * :190-208). These calls are that surface: a GGUF v2/v3 reader over a
 * read-only mmap of the file, and an upload that copies a tensor's bytes into
 * device memory unchanged -- ggml's Q4_0 rows are the engine's weight layout,
 * so w4a8_gemv reads the uploaded bytes in place.
 *
 * Format (the GGUF specification of ggml): "GGUF", u32 version, u64 tensor
 * count, u64 key/value count, the key/value pairs, the tensor infos (name,
 * u32 n_dims, u64 ne[n_dims] with ne[0] the row length, u32 type, u64 offset
 * from the data section), then the data section at the next multiple of
 * general.alignment (default 32). Strings are u64 length + bytes.
 *
 * Errors: negative status codes of w4a8.h (W4A8_ERR_*) plus W4A8_ERR_FORMAT;
 * lookups that find nothing return -1, as gguf_find_key / gguf_find_tensor do.
 */
#ifndef W4A8_GGUF_H
#define W4A8_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A8_ERR_FORMAT (-6)   /* not a GGUF file, or malformed / truncated */

/* ggml tensor types used by the engine (ggml.h's GGML_TYPE_* values). */
#define W4A8_GGML_TYPE_F32 0
#define W4A8_GGML_TYPE_F16 1
#define W4A8_GGML_TYPE_Q4_0 2
#define W4A8_GGML_TYPE_Q8_0 8

/* GGUF value types (gguf.h's GGUF_TYPE_* values). */
enum w4a8_gguf_type {
    W4A8_GGUF_UINT8 = 0, W4A8_GGUF_INT8 = 1, W4A8_GGUF_UINT16 = 2, W4A8_GGUF_INT16 = 3,
    W4A8_GGUF_UINT32 = 4, W4A8_GGUF_INT32 = 5, W4A8_GGUF_FLOAT32 = 6, W4A8_GGUF_BOOL = 7,
    W4A8_GGUF_STRING = 8, W4A8_GGUF_ARRAY = 9, W4A8_GGUF_UINT64 = 10, W4A8_GGUF_INT64 = 11,
    W4A8_GGUF_FLOAT64 = 12,
};

typedef struct w4a8_gguf w4a8_gguf;

typedef struct {
    const char *name;     /* NUL-terminated, owned by the handle */
    uint32_t type;        /* ggml tensor type */
    uint32_t n_dims;
    uint64_t ne[4];       /* ne[0] = elements per row; unused dims are 1 */
    uint64_t offset;      /* from the start of the data section */
    uint64_t nbytes;      /* bytes of the tensor's data (0 for a type this reader does not size) */
} w4a8_gguf_tensor;

/* Parse `path` (replaces gguf_init_from_file + the reference's mmap). */
int w4a8_gguf_open(const char *path, w4a8_gguf **out);
void w4a8_gguf_close(w4a8_gguf *g);

uint32_t w4a8_gguf_version(const w4a8_gguf *g);
int64_t w4a8_gguf_n_tensors(const w4a8_gguf *g);
int64_t w4a8_gguf_n_kv(const w4a8_gguf *g);
/* Byte offset of the data section in the file (gguf_get_data_offset). */
uint64_t w4a8_gguf_data_offset(const w4a8_gguf *g);

/* Index of key / tensor `name`, or -1 (gguf_find_key / gguf_find_tensor). */
int64_t w4a8_gguf_find_key(const w4a8_gguf *g, const char *key);
int64_t w4a8_gguf_find_tensor(const w4a8_gguf *g, const char *name);

/* Key i's name and value type (for arrays, *elem_type and *count too). */
const char *w4a8_gguf_key(const w4a8_gguf *g, int64_t i);
int w4a8_gguf_kv_type(const w4a8_gguf *g, int64_t i, uint32_t *type, uint32_t *elem_type, uint64_t *count);

/* Scalar values of key `key` (gguf_get_val_u32 / _f32 ...): W4A8_ERR_SHAPE
 * when the key is missing, W4A8_ERR_FORMAT when it has another type. */
int w4a8_gguf_get_u32(const w4a8_gguf *g, const char *key, uint32_t *v);
int w4a8_gguf_get_i32(const w4a8_gguf *g, const char *key, int32_t *v);
int w4a8_gguf_get_u64(const w4a8_gguf *g, const char *key, uint64_t *v);
int w4a8_gguf_get_f32(const w4a8_gguf *g, const char *key, float *v);
/* A string value: pointer into the file and its length (not NUL-terminated). */
int w4a8_gguf_get_str(const w4a8_gguf *g, const char *key, const char **s, uint64_t *len);

int w4a8_gguf_tensor_info(const w4a8_gguf *g, int64_t i, w4a8_gguf_tensor *info);
/* Host pointer to tensor i's bytes inside the read-only map
 * (map + gguf_get_data_offset + gguf_get_tensor_offset). */
const void *w4a8_gguf_tensor_data(const w4a8_gguf *g, int64_t i);

/* Copy tensor i's bytes, unchanged, to device memory `dst` (capacity `cap`
 * bytes) on `stream` (hipStream_t or NULL) and wait for the copy. For a Q4_0
 * tensor of ne = [k, rows] the device bytes are then the `rows x k` weight
 * matrix w4a8_gemv takes. W4A8_ERR_SHAPE when cap is too small. */
int w4a8_gguf_upload(const w4a8_gguf *g, int64_t i, void *dst, size_t cap, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A8_GGUF_H */
