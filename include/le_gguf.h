/*
 * le_gguf.h -- GGUF reader of the C ABI (host code in lible_qmm.so; touches no device).
 *
 * Replaces the reference's Gguf::open (src/gguf.rs:95-122: GGUF v2/v3 header, kv pairs, tensor
 * infos, data start aligned to general.alignment, default 32) and the tensor addressing that
 * cpu_ref::Model builds on it (src/cpu_ref.rs:56-58 absolute offsets; :70-85 expert slabs of the
 * 3D ffn_{gate,up,down}_exps tensors). A caller reads tensor bytes with le_gguf_read (or maps the
 * file itself) and uploads them; the bytes are exactly what le_matvec, le_gemm and le_moe_layer
 * take (dims[0] = cols, dims[1] = rows, dims[2] = experts).
 *
 * Status codes are those of le_qmm.h: LE_OK, LE_ERR_ARG (null / unknown name / out of range),
 * LE_ERR_TYPE (key missing or of another type, unknown ggml type), LE_ERR_SHAPE (malformed or
 * truncated file; le_gguf_open_error() gives the reason, like the reference's io::Error text).
 */
#ifndef LE_GGUF_H
#define LE_GGUF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct le_gguf le_gguf;

/* Parse the header, kv pairs and tensor infos of `path` (src/gguf.rs:95-122). */
int le_gguf_open(const char *path, le_gguf **out);
/* Reason of the last failed le_gguf_open on this thread. */
const char *le_gguf_open_error(void);
void le_gguf_close(le_gguf *g);

int le_gguf_version(const le_gguf *g);
/* Absolute file offset where tensor data begins (Gguf::data_start). */
uint64_t le_gguf_data_start(const le_gguf *g);
int le_gguf_tensor_count(const le_gguf *g);
int le_gguf_kv_count(const le_gguf *g);

/* Index of the tensor called `name`, or -1. */
int le_gguf_find(const le_gguf *g, const char *name);
/* Tensor i: name (owned by g), ggml type, number of dims, dims[8] (unused dims = 1), absolute
 * file offset of its data, and its byte size (0 for a type this build does not know). Any output
 * pointer may be NULL. */
int le_gguf_tensor_info(const le_gguf *g, int i, const char **name, int *ggml_type, int *n_dims, uint64_t *dims,
                        uint64_t *offset, uint64_t *nbytes);
/* Expert e's slab of a 3D tensor [cols, rows, n_expert]: absolute offset and bytes
 * (rows * row_bytes(type, cols)), as cpu_ref::expert_parts (src/cpu_ref.rs:78-85). */
int le_gguf_expert_slab(const le_gguf *g, const char *name, int expert, uint64_t *offset, uint64_t *bytes);

/* GGUF value type of `key` (0 u8 .. 12 f64), or -1 when absent. */
int le_gguf_kv_type(const le_gguf *g, const char *key);
/* Value::as_u64 (src/gguf.rs:14-22): unsigned integers and bool, signed integers when >= 0. */
int le_gguf_kv_u64(const le_gguf *g, const char *key, uint64_t *out);
/* Any integer or bool as int64 (u64 above INT64_MAX: LE_ERR_TYPE). */
int le_gguf_kv_i64(const le_gguf *g, const char *key, int64_t *out);
/* Value::as_f32 (src/gguf.rs:24): f32, or f64 narrowed. */
int le_gguf_kv_f32(const le_gguf *g, const char *key, float *out);
/* Value::as_str (src/gguf.rs:23): the string, owned by g. */
int le_gguf_kv_str(const le_gguf *g, const char *key, const char **out);
/* An array's element type and length (its elements are skipped, not kept). */
int le_gguf_kv_array(const le_gguf *g, const char *key, int *elem_type, uint64_t *count);

/* Copy `bytes` file bytes at absolute `offset` into host memory dst. */
int le_gguf_read(const le_gguf *g, uint64_t offset, uint64_t bytes, void *dst);

#ifdef __cplusplus
}
#endif

#endif /* LE_GGUF_H */
