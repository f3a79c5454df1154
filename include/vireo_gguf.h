/* GGUF types and the GGUF reader of vireo-hip.
 *
 * The first block states everything the reference's src/gguf.h declares - the
 * wire enums, gguf_str, gguf_kv, gguf_tensor, gguf_ctx (src/gguf.h:15-55) and
 * the prototypes of its reader (src/gguf.h:57-72, defined by src/gguf.c when a
 * program links it) - under the same include guard. So either header may come
 * first: after src/gguf.h this block is skipped and its definitions are the
 * ones seen; included first, it defines the same names and src/gguf.h is then
 * skipped with nothing of it missing. At the compute ABI only two fields of
 * gguf_tensor are read, as in the reference's gguf_matmul: `data` (there a
 * device pointer) and `ggml_type`.
 *
 * The second block (its own guard, so it is seen whichever header defined the
 * types) declares this library's reader, vireo_gguf_*: the reference's
 * gguf_open / gguf_find / gguf_get_* / gguf_tensor_by_name
 * (src/gguf.c:79-190) under its own names, so both can be linked into one
 * program. */
#ifndef VIREO_GGUF_H
#define VIREO_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF metadata value types (wire enum, src/gguf.h:16-18). */
enum { GGUF_U8=0, GGUF_I8=1, GGUF_U16=2, GGUF_I16=3, GGUF_U32=4, GGUF_I32=5,
       GGUF_F32=6, GGUF_BOOL=7, GGUF_STRING=8, GGUF_ARRAY=9, GGUF_U64=10,
       GGUF_I64=11, GGUF_F64=12 };

/* ggml tensor types (wire enum subset, src/gguf.h:21-23). */
enum { GGML_F32=0, GGML_F16=1, GGML_Q4_0=2, GGML_Q4_1=3, GGML_Q5_0=6,
       GGML_Q5_1=7, GGML_Q8_0=8, GGML_Q8_1=9, GGML_Q2_K=10, GGML_Q3_K=11,
       GGML_Q4_K=12, GGML_Q5_K=13, GGML_Q6_K=14, GGML_Q8_K=15 };

typedef struct { const char *ptr; uint64_t len; } gguf_str;

typedef struct {
    gguf_str key;
    uint32_t type;
    union { uint64_t u; int64_t i; double f; } val;  /* scalars           */
    gguf_str str;                                    /* if GGUF_STRING    */
    uint32_t arr_type; uint64_t arr_len;             /* if GGUF_ARRAY     */
    const uint8_t *arr_data;                         /* first array item  */
} gguf_kv;

typedef struct {
    gguf_str name;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t ggml_type;
    uint64_t offset;       /* from data section start */
    const void *data;      /* from the reader: into the file mapping; at the compute ABI: a device pointer */
    uint64_t n_elems;
    uint64_t nbytes;
} gguf_tensor;

typedef struct {
    int fd; void *map; size_t size;
    uint32_t version;
    uint64_t n_tensors, n_kv;
    gguf_kv *kv;
    gguf_tensor *tensors;
    const uint8_t *data;   /* tensor data section start */
    uint64_t alignment;
} gguf_ctx;

/* The reference's reader (src/gguf.h:57-72), for programs that link src/gguf.c;
 * this library's own reader is vireo_gguf_* below. */
gguf_ctx *gguf_open(const char *path);
void gguf_close(gguf_ctx *g);
const gguf_kv *gguf_find(const gguf_ctx *g, const char *key);
int gguf_get_u64(const gguf_ctx *g, const char *key, uint64_t *out);
int gguf_get_f32(const gguf_ctx *g, const char *key, float *out);
const char *gguf_get_str(const gguf_ctx *g, const char *key, uint64_t *len);
const gguf_tensor *gguf_tensor_by_name(const gguf_ctx *g, const char *name);
int gguf_type_block(uint32_t ggml_type, int *block_elems, int *block_bytes);
void gguf_dump(const gguf_ctx *g);

#ifdef __cplusplus
}
#endif
#endif /* VIREO_GGUF_H */

#ifndef VIREO_GGUF_READER_H
#define VIREO_GGUF_READER_H

#ifdef __cplusplus
extern "C" {
#endif

/* src/gguf.c:79-131: map a GGUF v2/v3 file read-only and parse its metadata
 * and tensor table; tensor `data` pointers point into the mapping. Returns
 * NULL on failure with errno set (EINVAL for a malformed file). Beyond the
 * reference's checks it rejects a zero alignment, tensors whose bytes reach
 * past the end of the file, element counts that overflow, and counts larger
 * than the file could hold; it accepts nested arrays (the reference rejects
 * them). Scalars keep the reference's convention: integer values are their raw
 * little-endian bits, zero-extended (a negative I32 reads back as 2^32 - |v|). */
gguf_ctx *vireo_gguf_open(const char *path);
/* src/gguf.c:133-138 */
void vireo_gguf_close(gguf_ctx *g);
/* src/gguf.c:143-146: the first entry with this key, or NULL */
const gguf_kv *vireo_gguf_find(const gguf_ctx *g, const char *key);
/* src/gguf.c:147-160: 0 on success, -1 if absent or of another type
 * (u64: any integer type or BOOL; f32: F32 or F64) */
int vireo_gguf_get_u64(const gguf_ctx *g, const char *key, uint64_t *out);
int vireo_gguf_get_f32(const gguf_ctx *g, const char *key, float *out);
/* src/gguf.c:161-165: a STRING value (not NUL-terminated) and its length, or NULL */
const char *vireo_gguf_get_str(const gguf_ctx *g, const char *key, uint64_t *len);
/* src/gguf.c:166-171: the first tensor with this name, or NULL */
const gguf_tensor *vireo_gguf_tensor_by_name(const gguf_ctx *g, const char *name);

#ifdef __cplusplus
}
#endif
#endif /* VIREO_GGUF_READER_H */
