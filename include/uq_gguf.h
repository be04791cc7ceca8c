/*
 * uq_gguf.h -- GGUF reader and GGUF -> HBM loader of libuq.so.
 *
 * Replaces the reference's weight loader for the quantized linear layer:
 * the header parser gguf::parse (crates/unltd-model-loader/src/gguf.rs:353-520),
 * the memory-mapped tensor access MappedWeights (weights.rs:23-96) and the
 * per-tensor validation of Qwen35Forward::open (qwen35_forward.rs:109-128),
 * plus the upload of a tensor's bytes, unchanged, into a uq_weights handle.
 *
 * The reader validates the whole header before serving a byte and refuses,
 * in the reference's order:
 *   magic "GGUF" (UQ_ERR_MAGIC), version 2 or 3 (UQ_ERR_VERSION);
 *   n_kv > file_size/8 or n_tensors > file_size/16, any read past the end of
 *   the file, a string longer than the file, an unknown metadata value type,
 *   an array larger than the file or nested, general.alignment != 32, a
 *   tensor with n_dims 0 or > 64, zero elements or an element count that
 *   overflows 64 bits (UQ_ERR_FILE);
 *   then, over the tensors sorted by absolute offset, an offset that is not a
 *   multiple of 32 (UQ_ERR_TENSOR_ALIGN), data past the end of the file
 *   (UQ_ERR_TENSOR_BOUNDS) and overlapping data (UQ_ERR_TENSOR_OVERLAP).
 * Tensor offsets in the file are relative to the data section, which starts
 * at the first multiple of 32 after the last tensor info; every offset
 * reported here is absolute. A tensor of an unknown ggml type is kept with
 * has_nbytes = 0 and skips the range checks, as in the reference.
 * uq_last_error() carries the message (names, offsets and sizes).
 *
 * A uq_gguf is read-only after open and may be shared between threads.
 */
#ifndef UQ_GGUF_H
#define UQ_GGUF_H

#include "uq.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct uq_gguf_s *uq_gguf;

/* GGUF metadata value type ids (GgufValueType::from_id, gguf.rs:56-72). */
typedef enum uq_gguf_type {
    UQ_GGUF_U8 = 0, UQ_GGUF_I8 = 1, UQ_GGUF_U16 = 2, UQ_GGUF_I16 = 3,
    UQ_GGUF_U32 = 4, UQ_GGUF_I32 = 5, UQ_GGUF_F32 = 6, UQ_GGUF_BOOL = 7,
    UQ_GGUF_STRING = 8, UQ_GGUF_ARRAY = 9, UQ_GGUF_U64 = 10, UQ_GGUF_I64 = 11,
    UQ_GGUF_F64 = 12
} uq_gguf_type;

/* One entry of the tensor table (TensorMeta, unltd-model-loader/src/lib.rs:24-38). */
typedef struct uq_gguf_tensor {
    const char *name;       /* not NUL-terminated in general: use name_len */
    size_t name_len;
    uint64_t offset;        /* absolute file offset */
    uint64_t nbytes;        /* ceil(n_elements / block_elems) * block_bytes */
    int has_nbytes;         /* 0: unknown ggml type (nbytes None) */
    uint32_t ggml_type;
    uint32_t n_dims;
    const uint64_t *shape;  /* n_dims entries, GGUF order: shape[0] is contiguous */
    uint64_t n_elements;
} uq_gguf_tensor;

/* One metadata pair. Scalars and numeric arrays: data points at the values
 * as the file stores them (little-endian; bool as one byte, nonzero = true),
 * count = 1 for a scalar. Strings (and arrays of strings) are read with
 * uq_gguf_kv_string; their data is NULL. */
typedef struct uq_gguf_kv {
    const char *key;
    size_t key_len;
    uint32_t type;       /* uq_gguf_type */
    uint32_t elem_type;  /* arrays: element type; otherwise equal to type */
    uint64_t count;
    const void *data;
} uq_gguf_kv;

/* MappedWeights::open (weights.rs:32-41) over GgufReader::open
 * (gguf.rs:298-303): map the file read-only and validate its header. */
uq_status uq_gguf_open(const char *path, uq_gguf *out);

/* gguf::parse (gguf.rs:353-520) over an in-memory file of len bytes (the
 * bytes are copied). */
uq_status uq_gguf_parse(const void *bytes, size_t len, uq_gguf *out);

uq_status uq_gguf_close(uq_gguf g);

/* GgufReader's version, file_size and data_start, plus the table sizes. */
uq_status uq_gguf_header(uq_gguf g, uint32_t *version, uint64_t *file_size, uint64_t *data_start,
                         uint64_t *n_kv, uint64_t *n_tensors);

/* GgufReader::tensors()[i]. The pointers stay valid until uq_gguf_close. */
uq_status uq_gguf_tensor_at(uq_gguf g, uint64_t i, uq_gguf_tensor *out);

/* WeightIndex::find (gguf.rs:341-344): index of the tensor called name (the
 * last one, when a name repeats). UQ_ERR_MISSING_TENSOR when absent. */
uq_status uq_gguf_find(uq_gguf g, const char *name, uint64_t *index);

/* MappedWeights::tensor (weights.rs:55-61): the tensor's bytes in the
 * mapping. UQ_ERR_MISSING_TENSOR when absent, UQ_ERR_GGML_TYPE when its
 * ggml type is unknown (the reference's None). */
uq_status uq_gguf_tensor_bytes(uq_gguf g, const char *name, const uint8_t **bytes, uint64_t *nbytes);

/* MappedWeights::tensor_checked (weights.rs:67-96): as uq_gguf_tensor_bytes,
 * and UQ_ERR_ELEMENT_COUNT when the element count is not n_elements. The
 * checks run in the reference's order: missing, count, type. */
uq_status uq_gguf_tensor_checked(uq_gguf g, const char *name, uint64_t n_elements, const uint8_t **bytes,
                                 uint64_t *nbytes);

/* check (qwen35_forward.rs:109-128): present (UQ_ERR_MISSING_TENSOR), exactly
 * n_elements elements (UQ_ERR_ELEMENT_COUNT), a ggml type dtype_of knows
 * (min_forward.rs:39-48; UQ_ERR_GGML_TYPE) and one of the allowed dtypes
 * (UQ_ERR_FILE, the reference's LoadError::corrupt). allowed is a bit mask:
 * bit d allows uq_dtype d, e.g.
 * (1u << UQ_Q4_K) | (1u << UQ_Q6_K). *dtype (may be NULL) receives the
 * tensor's dtype. */
uq_status uq_gguf_check(uq_gguf g, const char *name, uint64_t n_elements, uint64_t allowed, uq_dtype *dtype);

/* Load one tensor into HBM: uq_weights_upload of its bytes, unchanged, with
 * dim_in = shape[0], dim_out = n_elements / shape[0] and the dtype of its
 * ggml type (a 1-D tensor is one row). Fails as uq_gguf_tensor_bytes, then
 * as uq_weights_upload (e.g. UQ_ERR_DTYPE for F16). */
uq_status uq_gguf_upload(uq_gguf g, const char *name, uq_weights *out);

/* GgufReader::metadata[i]. */
uq_status uq_gguf_kv_at(uq_gguf g, uint64_t i, uq_gguf_kv *out);

/* GgufReader::get (gguf.rs:306-308): index of the first pair with this key.
 * UQ_ERR_ARG (message "no key") when absent. */
uq_status uq_gguf_kv_find(uq_gguf g, const char *key, uint64_t *index);

/* The bytes of a string value (elem ignored) or of element elem of an array
 * of strings, as stored (the reference decodes them as lossy UTF-8). */
uq_status uq_gguf_kv_string(uq_gguf g, uint64_t i, uint64_t elem, const char **s, size_t *len);

/* ggml_type_blocksize (gguf.rs:193-234): bytes and elements per block.
 * UQ_ERR_GGML_TYPE for ids the table leaves unknown or retired. */
uq_status uq_gguf_type_blocksize(uint32_t ggml_type, uint64_t *block_bytes, uint64_t *block_elems);

/* ggml_type_name (gguf.rs:237-278), NUL-terminated into buf. */
uq_status uq_gguf_type_name(uint32_t ggml_type, char *buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* UQ_GGUF_H */
