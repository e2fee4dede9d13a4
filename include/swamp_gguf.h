/*
 * swamp_gguf.h -- GGUF reader and device upload of libswamp_gpu.so: the data
 * format on the input side of the quantized-matmul path.
 *
 * Replaces GgufFile (swamp-gguf/src/mmap.rs:16-151) and TensorInfo
 * (swamp-gguf/src/tensor_info.rs:8-62) for the path's needs: open a file
 * read-only by mmap, parse header / metadata / tensor infos exactly like
 * GgufFile::parse (mmap.rs:34-94), and hand out a tensor's raw block bytes
 * (tensor_raw_bytes, mmap.rs:110-117) zero-copy on the host or copied to a
 * device buffer, where swamp_qgemv / swamp_qgemm read them as they are.
 *
 * Parsing rules (as in the reference):
 *  - magic "GGUF", version 1..3; version 1 has u32 tensor/kv counts and
 *    u32 dims, versions 2 and 3 u64 (mmap.rs:41-49, 64-67);
 *  - metadata value types 0..12 (metadata.rs:202-243); an unknown value
 *    or array element type is SWAMP_EDTYPE (the reference's UnknownDType);
 *  - tensor dtype codes must be GGML codes (dtype.rs:43-75) -> SWAMP_EDTYPE;
 *  - the data section starts at the end of the tensor infos rounded up to
 *    32 bytes; general.alignment is NOT consulted (mmap.rs:13, 76-79);
 *  - tensor offsets are relative to the data section; nbytes =
 *    nbytes_for(dtype, product(shape)) (tensor_info.rs:19-27);
 *  - a read past the end of the file while parsing is SWAMP_EIO (the
 *    reader's UnexpectedEof, metadata.rs:129-197).
 * The strings returned point into the handle and live until close.
 */
#ifndef SWAMP_GGUF_H
#define SWAMP_GGUF_H

#ifndef SWAMP_API
#define SWAMP_API __attribute__((visibility("default")))
#endif

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SWAMP_EIO = -7,        /* open / mmap failed, or the file ends inside the header (Io) */
  SWAMP_EMAGIC = -8,     /* not "GGUF" (InvalidMagic) */
  SWAMP_EVERSION = -9,   /* version outside 1..3 (UnsupportedVersion) */
  SWAMP_ENOTFOUND = -10, /* tensor or metadata key absent, or of another type
                            (TensorNotFound, MetadataKeyNotFound) */
  SWAMP_ETENSOR = -11    /* tensor bytes outside the file (InvalidTensor) */
};

/* Metadata value types (metadata.rs:202-218). */
enum {
  SWAMP_GGUF_U8 = 0, SWAMP_GGUF_I8 = 1, SWAMP_GGUF_U16 = 2, SWAMP_GGUF_I16 = 3,
  SWAMP_GGUF_U32 = 4, SWAMP_GGUF_I32 = 5, SWAMP_GGUF_F32 = 6, SWAMP_GGUF_BOOL = 7,
  SWAMP_GGUF_STRING = 8, SWAMP_GGUF_ARRAY = 9, SWAMP_GGUF_U64 = 10, SWAMP_GGUF_I64 = 11,
  SWAMP_GGUF_F64 = 12
};

typedef struct swamp_gguf swamp_gguf;

/* GgufFile::open (mmap.rs:27-31) + parse.  On success *out is a handle to
 * close with swamp_gguf_close. */
SWAMP_API int swamp_gguf_open(const char *path, swamp_gguf **out);
SWAMP_API void swamp_gguf_close(swamp_gguf *g);

/* Header facts: version, tensor count (n_tensors, mmap.rs:119-121), the
 * data-section offset (data_offset) and the file size (file_size). */
SWAMP_API uint32_t swamp_gguf_version(const swamp_gguf *g);
SWAMP_API int64_t swamp_gguf_n_tensors(const swamp_gguf *g);
SWAMP_API int64_t swamp_gguf_n_kv(const swamp_gguf *g);
SWAMP_API uint64_t swamp_gguf_data_offset(const swamp_gguf *g);
SWAMP_API uint64_t swamp_gguf_file_size(const swamp_gguf *g);

/* Tensor i (file order): name (NUL-terminated), dtype, number of dims and
 * up to 4 dims (shape[0] = n_cols), the ABSOLUTE byte offset in the file
 * (the reference adds data_offset, mmap.rs:81-86) and nbytes.  Any output
 * pointer may be NULL.  i out of range -> SWAMP_EINVAL; more than 4 dims
 * fill the first 4. */
SWAMP_API int swamp_gguf_tensor_info(const swamp_gguf *g, int64_t i, const char **name, uint32_t *dtype,
                           int *n_dims, uint64_t dims[4], uint64_t *offset, uint64_t *nbytes);

/* GgufFile::tensor (mmap.rs:96-99): index of the first tensor named
 * `name`, or SWAMP_ENOTFOUND (tensor_or_err, :101-105). */
SWAMP_API int64_t swamp_gguf_find(const swamp_gguf *g, const char *name);

/* GgufFile::tensor_raw_bytes (mmap.rs:110-117): host pointer into the
 * mapping and length; SWAMP_ETENSOR when the range passes the end. */
SWAMP_API int swamp_gguf_tensor_raw(const swamp_gguf *g, int64_t i, const void **ptr, size_t *len);

/* Copy tensor i's raw bytes into the device buffer d_dst (dst_len bytes
 * available) on `stream` (hipStream_t as void*, NULL = default).  The copy
 * is complete when the call returns (the source is pageable mapped memory).
 * dst_len < nbytes -> SWAMP_ESHAPE; copy failure -> SWAMP_ELAUNCH. */
SWAMP_API int swamp_gguf_upload(const swamp_gguf *g, int64_t i, void *d_dst, size_t dst_len, void *stream);

/* Metadata lookup (Metadata::get_u32 / get_u64 / get_f32 / get_str,
 * metadata.rs:263-292).  Conversions follow MetadataValue::as_u32 /
 * as_u64 / as_f32 (metadata.rs:60-90); a key that is absent or does not
 * convert -> SWAMP_ENOTFOUND.  The string is not NUL-terminated: use len. */
SWAMP_API int swamp_gguf_meta_type(const swamp_gguf *g, const char *key, uint32_t *type);
SWAMP_API int swamp_gguf_meta_u32(const swamp_gguf *g, const char *key, uint32_t *out);
SWAMP_API int swamp_gguf_meta_u64(const swamp_gguf *g, const char *key, uint64_t *out);
SWAMP_API int swamp_gguf_meta_f32(const swamp_gguf *g, const char *key, float *out);
SWAMP_API int swamp_gguf_meta_str(const swamp_gguf *g, const char *key, const char **str, size_t *len);

#ifdef __cplusplus
}
#endif

#endif /* SWAMP_GGUF_H */
