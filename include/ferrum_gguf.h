/*
 * ferrum_gguf.h — GGUF reader and device weight upload of libferrum_kv.so.
 *
 * The model's weights reach the decode layer's GEMVs (include/ferrum_q8.h) through this:
 * fkv_gguf_open is Ferrum's gguf::load (crates/gguf/src/parse.rs:53-64) — memory-map a
 * little-endian GGUF v2/v3 file and decode its header, metadata and tensor directory with
 * the same checks, in the same order, with the same messages (parse.rs:100-258,
 * layout.rs:57-72, crates/core-types/src/source.rs:25-56, dtype.rs:87-129) — and
 * fkv_gguf_upload copies the tensor data section into device memory through pinned
 * staging buffers, keeping every tensor at its data_offset (so each keeps the file's
 * alignment). A tensor's device bytes are then dev_base + data_offset: the same bytes
 * GgufModel::tensor_bytes (parse.rs:483-501) borrows from the map.
 *
 * Errors: FKV_ERR_GGUF with Display "gguf: <msg>" (FerrumError::Gguf,
 * crates/core-types/src/error.rs:32-33), the reference's message text; FKV_ERR_INVALID for
 * null arguments and buffer sizes at this boundary; FKV_ERR_INTERNAL for HIP failures.
 */
#ifndef FERRUM_GGUF_H
#define FERRUM_GGUF_H

#include <stdint.h>

#include "ferrum_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FKV_ERR_GGUF 6 /* "gguf: <msg>" (FerrumError::Gguf) */

/* Metadata value types: the GGUF ids of MetadataType (crates/core-types/src/metadata.rs:30-47). */
#define FKV_GGUF_UINT8 0
#define FKV_GGUF_INT8 1
#define FKV_GGUF_UINT16 2
#define FKV_GGUF_INT16 3
#define FKV_GGUF_UINT32 4
#define FKV_GGUF_INT32 5
#define FKV_GGUF_FLOAT32 6
#define FKV_GGUF_BOOL 7
#define FKV_GGUF_STRING 8
#define FKV_GGUF_ARRAY 9
#define FKV_GGUF_UINT64 10
#define FKV_GGUF_INT64 11
#define FKV_GGUF_FLOAT64 12

typedef struct fkv_gguf fkv_gguf;

/* One tensor of the directory (TensorDesc, source.rs:13-22). name points into the
 * handle and lives as long as it. shape has n_dims entries, shape[0] contiguous. */
typedef struct fkv_gguf_tensor_info {
  const char* name;
  uint64_t name_len;
  uint32_t n_dims;
  uint32_t ggml_type;
  uint64_t shape[4];
  uint64_t data_offset; /* from the start of the data section */
  uint64_t nbytes;
} fkv_gguf_tensor_info;

/* A metadata value. Scalars: the integer types widen into u (unsigned) or i (signed),
 * FLOAT32/FLOAT64 into f, BOOL into u (0/1). STRING: str/str_len point into the handle.
 * ARRAY: elem_type and count; read elements with fkv_gguf_meta_array_*. */
typedef struct fkv_gguf_value {
  uint32_t type;
  uint32_t elem_type;
  uint64_t count;
  uint64_t u;
  int64_t i;
  double f;
  const char* str;
  uint64_t str_len;
} fkv_gguf_value;

/* gguf::load(path) (parse.rs:53-64): open read-only, map, decode. */
int32_t fkv_gguf_open(const char* path, fkv_gguf** out);
int32_t fkv_gguf_close(fkv_gguf* g);

/* GgufModel::version, alignment, metadata_len, tensors().len(); data_start and the data
 * section's byte length (file length - data_start). */
int32_t fkv_gguf_info(const fkv_gguf* g, uint32_t* version, uint64_t* alignment,
                      uint64_t* n_metadata, uint64_t* n_tensors, uint64_t* data_start,
                      uint64_t* data_bytes);

/* The index-th tensor in file order. */
int32_t fkv_gguf_tensor(const fkv_gguf* g, uint64_t index, fkv_gguf_tensor_info* out);

/* GgufModel::tensor(name) (parse.rs:476-481): its index, or "gguf: missing tensor <name>".
 * Names and keys are passed with their byte length: GGUF strings may hold NUL bytes. */
int32_t fkv_gguf_find(const fkv_gguf* g, const char* name, uint64_t name_len, uint64_t* index);

/* GgufModel::metadata(key): FKV_OK and the value, or FKV_ERR_INVALID "missing metadata key
 * <key>" (the reference returns None). */
int32_t fkv_gguf_meta(const fkv_gguf* g, const char* key, uint64_t key_len, fkv_gguf_value* out);

/* Element i of an array value: scalars and strings as fkv_gguf_meta gives them; a nested
 * array reports its elem_type and count only. */
int32_t fkv_gguf_meta_array_elem(const fkv_gguf* g, const char* key, uint64_t key_len,
                                 uint64_t i, fkv_gguf_value* out);

/* GgufModel::dump (format_gguf_dump, source.rs:70-92) into buf (cap bytes); *len gets the
 * full length (call with cap 0 to size it). The text is NUL-terminated when it fits. */
int32_t fkv_gguf_dump(const fkv_gguf* g, char* buf, uint64_t cap, uint64_t* len);

/* Copy the data section (data_bytes bytes) into device memory at dst (dst_bytes >=
 * data_bytes) on the calling thread's current device. `threads` host threads (0: 4, fewer
 * when the process may run on fewer CPUs) each own one pinned buffer of chunk_bytes (0:
 * 8 MiB) and one stream, and move every threads-th chunk: pread from the file, then
 * hipMemcpyAsync, reusing the buffer once that copy is done. Returns when every copy is
 * done. Tensor t's device bytes are then dst + info(t).data_offset. A read failure is
 * FKV_ERR_GGUF "failed to read tensor data: ..."; a HIP failure FKV_ERR_INTERNAL. */
int32_t fkv_gguf_upload(const fkv_gguf* g, void* dst, uint64_t dst_bytes, uint64_t chunk_bytes,
                        uint32_t threads);

#ifdef __cplusplus
}
#endif

#endif /* FERRUM_GGUF_H */
