/* ggq_gguf.h -- GGUF (version 3) reader over mmap, and upload of its raw
 * tensors to HBM for the quantized matmul in ggq.h.
 *
 * Replaces the reference's GgufLoader (include/ggnpu/gguf.h,
 * src/gguf/gguf.cpp:108-398) for the purpose the matmul path needs: tensor
 * infos (name, ggml type, dims, offset) and their raw bytes, read in place
 * from the mapped file, plus the typed metadata key/values.  Behaviour kept
 * from the reference:
 *   - magic "GGUF", version 3 only (gguf.cpp:148-165); anything else is
 *     GGQ_INVALID_PARAM;
 *   - keys and tensor names at most 1024 bytes, strings at most 64 MiB
 *     (gguf.cpp:174, 297, 190);
 *   - tensor data starts after the tensor infos, rounded up to
 *     general.alignment (default 32), and tensor offsets are relative to it
 *     (gguf.cpp:342-372);
 *   - a tensor's size is elements / block size * block bytes
 *     (gguf.cpp:328-331, tensor.h:64-66).
 * Unlike the reference, every read is bounds-checked against the file size,
 * and integer metadata keeps its declared width and sign.
 *
 * Pointers returned by these functions (names, strings, tensor data) point
 * into the mapping or into the handle and stay valid until ggq_gguf_close.
 * Status values are those of ggq.h.  No function here needs a GPU except
 * ggq_gguf_upload. */
#ifndef GGQ_GGUF_H
#define GGQ_GGUF_H

#include <stdint.h>

#include "ggq.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggq_gguf ggq_gguf;

/* Metadata value types (include/ggnpu/gguf.h GgufType). */
#define GGQ_GGUF_UINT8 0
#define GGQ_GGUF_INT8 1
#define GGQ_GGUF_UINT16 2
#define GGQ_GGUF_INT16 3
#define GGQ_GGUF_UINT32 4
#define GGQ_GGUF_INT32 5
#define GGQ_GGUF_FLOAT32 6
#define GGQ_GGUF_BOOL 7
#define GGQ_GGUF_STRING 8
#define GGQ_GGUF_ARRAY 9
#define GGQ_GGUF_UINT64 10
#define GGQ_GGUF_INT64 11
#define GGQ_GGUF_FLOAT64 12

/* Opens and maps `path`.  GGQ_NOT_FOUND if it cannot be opened, GGQ_INVALID_PARAM
 * if it is not a well-formed GGUF v3 file (the message says why). */
int ggq_gguf_open(const char* path, ggq_gguf** out);
void ggq_gguf_close(ggq_gguf* g);
/* Why the last ggq_gguf_open on this thread failed ("" after a success). */
const char* ggq_gguf_last_error(void);

uint32_t ggq_gguf_version(const ggq_gguf* g);
uint64_t ggq_gguf_alignment(const ggq_gguf* g);
/* File offset of the tensor data section. */
uint64_t ggq_gguf_data_offset(const ggq_gguf* g);
uint64_t ggq_gguf_file_size(const ggq_gguf* g);

typedef struct {
    const char* name;  /* NUL-terminated copy held by the handle */
    uint32_t type;     /* ggml type id */
    int32_t n_dims;
    int64_t dims[4];   /* dims[0] = K (fastest), dims[1] = N, dims[2] = experts ... (1 past n_dims) */
    uint64_t offset;   /* relative to the data section */
    uint64_t nbytes;   /* elements / block size * block bytes */
    const void* data;  /* in the mapping: data section + offset */
} ggq_gguf_tensor;

int64_t ggq_gguf_n_tensors(const ggq_gguf* g);
int ggq_gguf_tensor_at(const ggq_gguf* g, int64_t i, ggq_gguf_tensor* out);
/* Index of the tensor called `name`, or -1. */
int64_t ggq_gguf_find_tensor(const ggq_gguf* g, const char* name);

int64_t ggq_gguf_n_kv(const ggq_gguf* g);
const char* ggq_gguf_kv_key(const ggq_gguf* g, int64_t i);
/* Index of metadata key `key`, or -1. */
int64_t ggq_gguf_find_kv(const ggq_gguf* g, const char* key);
uint32_t ggq_gguf_kv_type(const ggq_gguf* g, int64_t i);
/* Integer (UINT8..INT64, BOOL) value; GGQ_INVALID_PARAM for other types. */
int ggq_gguf_kv_int(const ggq_gguf* g, int64_t i, int64_t* out);
/* Unsigned 64-bit value (UINT64 values above INT64_MAX). */
int ggq_gguf_kv_uint(const ggq_gguf* g, int64_t i, uint64_t* out);
/* FLOAT32 / FLOAT64 value. */
int ggq_gguf_kv_float(const ggq_gguf* g, int64_t i, double* out);
/* STRING value: NUL-terminated copy and its length (GGUF strings may hold
 * NUL bytes; `len` is authoritative). */
int ggq_gguf_kv_str(const ggq_gguf* g, int64_t i, const char** s, uint64_t* len);
/* ARRAY: element type and count; for numeric element types `data` points at
 * the little-endian elements in the mapping (null for string arrays). */
int ggq_gguf_kv_array(const ggq_gguf* g, int64_t i, uint32_t* elem_type, uint64_t* n, const void** data);
/* Element j of a string ARRAY (not NUL-terminated; `len` bytes at `s`, in
 * the mapping). */
int ggq_gguf_kv_array_str(const ggq_gguf* g, int64_t i, uint64_t j, const char** s, uint64_t* len);

/* Uploads tensor `name` unchanged to HBM as a matmul weight: K = dims[0] and
 * N = dims[1] * dims[2] * ... (an expert tensor [K][N][E] becomes E matrices
 * back to back, the layout ggq_moe_ffn_dev reads).  Same checks and errors
 * as ggq_weight_upload; GGQ_NOT_FOUND if there is no such tensor.  Replaces
 * the reference's upload of mmap'd tensor bytes on first use
 * (amd_xdna.cpp:279-310; main.cpp:1430-1432 hands the mmap pointer as B). */
int ggq_gguf_upload(ggq_ctx* ctx, const ggq_gguf* g, const char* name, ggq_weight** out);

#ifdef __cplusplus
}
#endif

#endif /* GGQ_GGUF_H */
