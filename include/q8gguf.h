/*
 * q8gguf.h -- read-only GGUF reader of libq8mi.so: the ingestion side of the
 * Q8_0 path.  A model file is memory-mapped and every tensor is handed back
 * as a pointer into that map, so a weight goes from disk to the device
 * residency cache (q8_weight_resident, include/q8mi.h) with no host copy,
 * keyed by the same (address, length) identity the reference uses.
 *
 * Replaces the reference's GgufFile (apps/engine/src/gguf.rs:95-311, with its
 * Reader 313-402, read_typed_value 404-442 and skip_array 444-468) and the
 * shape-checked weight lookup of the model loader (apps/engine/src/model.rs:
 * 1670-1684).  Same file format rules, same checks, same error kinds:
 *   magic 0x46554747, version 2 or 3, u64 tensor and key counts;
 *   metadata value types 0..12 (9 = array, recorded by offset, decoded on
 *   request); tensor types F32 (0), F16 (1), Q8_0 (8), anything else is
 *   Q8_ERR_UNSUPPORTED; every string is checked to be UTF-8;
 *   alignment = `general.alignment` when stored as an unsigned integer, else
 *   32; data start = end of the tensor table rounded up to the alignment;
 *   every tensor must lie inside the file.
 * Where the reference would panic or wrap (a zero alignment, u64 overflow of
 * an element count or an end offset, arrays nested without limit) this reader
 * returns Q8_ERR_FORMAT instead.
 *
 * Status codes are those of q8mi.h; the reader adds three EngineError kinds:
 * Q8_ERR_FORMAT (EngineError::Format, "malformed gguf: ..."), Q8_ERR_MISSING
 * (EngineError::MissingTensor / MissingMetadata) and Q8_ERR_IO
 * (EngineError::Io).  q8_last_error() holds the message.
 */
#ifndef Q8GGUF_H
#define Q8GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "q8mi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q8_gguf q8_gguf;

/* Tensor element types (DType::from_id, gguf.rs:27-34). */
enum { Q8_GGUF_F32 = 0, Q8_GGUF_F16 = 1, Q8_GGUF_Q8_0 = 8 };

/* Metadata value types (read_typed_value, gguf.rs:404-442). */
enum {
    Q8_GGUF_TYPE_U8 = 0, Q8_GGUF_TYPE_I8 = 1, Q8_GGUF_TYPE_U16 = 2, Q8_GGUF_TYPE_I16 = 3,
    Q8_GGUF_TYPE_U32 = 4, Q8_GGUF_TYPE_I32 = 5, Q8_GGUF_TYPE_F32 = 6, Q8_GGUF_TYPE_BOOL = 7,
    Q8_GGUF_TYPE_STRING = 8, Q8_GGUF_TYPE_ARRAY = 9, Q8_GGUF_TYPE_U64 = 10, Q8_GGUF_TYPE_I64 = 11,
    Q8_GGUF_TYPE_F64 = 12,
};

/* TensorInfo (gguf.rs:58-65) plus its place in the map.  Pointers are owned by
 * the file handle and stay valid until q8_gguf_close. */
typedef struct {
    const char *name;     /* NUL-terminated */
    uint64_t name_len;    /* bytes, NUL excluded */
    uint32_t n_dims;
    const uint64_t *dims; /* GGUF order: dims[0] is the row length (k) */
    uint32_t dtype;       /* Q8_GGUF_* */
    uint64_t offset;      /* from the start of the data section */
    uint64_t byte_len;    /* DType::byte_len(elements), gguf.rs:53-55 */
    uint64_t elements;    /* product of dims */
    const uint8_t *data;  /* byte_len bytes inside the map (gguf.rs:185-191) */
} q8_gguf_tensor_info;

/* GgufFile::open (gguf.rs:95-175): map the file read-only and parse the header,
 * metadata and tensor table. */
int q8_gguf_open(const char *path, q8_gguf **out);
/* Unmap.  Tensor data pointers (and weights made resident from them, whose
 * identity is their address) must not be used afterwards. */
void q8_gguf_close(q8_gguf *g);
/* Header facts: format version, alignment in force, data section start and
 * file size in bytes. */
int q8_gguf_layout(const q8_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_start,
                   uint64_t *file_bytes);

/* GgufFile::tensors (gguf.rs:177-179), in file order. */
int q8_gguf_tensor_count(const q8_gguf *g, uint64_t *count);
int q8_gguf_tensor_at(const q8_gguf *g, uint64_t index, q8_gguf_tensor_info *out);
/* GgufFile::tensor / data (gguf.rs:181-191): the first tensor of that name;
 * Q8_ERR_MISSING ("missing tensor: NAME") if there is none. */
int q8_gguf_tensor(const q8_gguf *g, const char *name, q8_gguf_tensor_info *out);

/* Metadata keys in the order the file first defines them (a repeated key
 * keeps its first place and its last value, as the reference's map insert
 * does).  `type` is Q8_GGUF_TYPE_*; for arrays `elem_type` and `len` describe
 * the payload (else 0). */
int q8_gguf_meta_count(const q8_gguf *g, uint64_t *count);
int q8_gguf_meta_key_at(const q8_gguf *g, uint64_t index, const char **key);
int q8_gguf_meta_type(const q8_gguf *g, const char *key, uint32_t *type, uint32_t *elem_type, uint64_t *len);

/* Typed getters (gguf.rs:193-311).  A missing key is Q8_ERR_MISSING ("missing
 * metadata key: KEY"); a value of another kind is Q8_ERR_FORMAT.
 * meta_u64 takes any unsigned value and any signed value >= 0; meta_f32 takes
 * f32 and f64 values (an f64 is rounded to f32); meta_bool only bools. */
int q8_gguf_meta_u64(const q8_gguf *g, const char *key, uint64_t *out);
int q8_gguf_meta_f32(const q8_gguf *g, const char *key, float *out);
int q8_gguf_meta_bool(const q8_gguf *g, const char *key, int *out);
/* A string value: `*str` is NUL-terminated, `*len` its byte length. */
int q8_gguf_meta_str(const q8_gguf *g, const char *key, const char **str, uint64_t *len);
/* GgufFile::has_key_prefix (gguf.rs:238-240): 1 if any key starts with prefix. */
int q8_gguf_has_key_prefix(const q8_gguf *g, const char *prefix);

/* Arrays, decoded from the map on request (gguf.rs:250-311).  `*len` is always
 * set to the array's length; min(cap, len) entries are written.
 * i32: element type I32 or U32 (read as 32 bits, reinterpreted);
 * f32: element type F32; str: element type STRING, `ptrs[i]`/`lens[i]` point
 * into the map (not NUL-terminated). */
int q8_gguf_meta_i32_array(const q8_gguf *g, const char *key, int32_t *out, uint64_t cap, uint64_t *len);
int q8_gguf_meta_f32_array(const q8_gguf *g, const char *key, float *out, uint64_t cap, uint64_t *len);
int q8_gguf_meta_str_array(const q8_gguf *g, const char *key, const char **ptrs, uint64_t *lens, uint64_t cap,
                           uint64_t *len);

/* The loader's `weight()` (model.rs:1670-1684) followed by the device upload
 * (Gpu::quantized, apps/engine/src/cuda/mod.rs:1769-1790): the tensor must be
 * Q8_0 with dims exactly [k, out] (else Q8_ERR_FORMAT "NAME has shape [..],
 * expected [k, out]"); its bytes in the map are made resident by identity. */
int q8_gguf_weight(q8_ctx *c, const q8_gguf *g, const char *name, int k, int out, const q8_weight **weight);

#ifdef __cplusplus
}
#endif

#endif /* Q8GGUF_H */
