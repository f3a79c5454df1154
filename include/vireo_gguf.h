/* GGUF tensor types used at the vireo-hip C-ABI.
 *
 * Same layout as the reference's src/gguf.h:21-45 (ggml type ids, gguf_str,
 * gguf_tensor) and the same include guard, so a translation unit that already
 * includes src/gguf.h sees identical definitions and a standalone caller can
 * include this header instead. At the ABI only two fields of gguf_tensor are
 * read, as in the reference's gguf_matmul: `data` (here a device pointer) and
 * `ggml_type`. */
#ifndef VIREO_GGUF_H
#define VIREO_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types (wire enum subset, src/gguf.h:21-23). */
enum { GGML_F32=0, GGML_F16=1, GGML_Q4_0=2, GGML_Q4_1=3, GGML_Q5_0=6,
       GGML_Q5_1=7, GGML_Q8_0=8, GGML_Q8_1=9, GGML_Q2_K=10, GGML_Q3_K=11,
       GGML_Q4_K=12, GGML_Q5_K=13, GGML_Q6_K=14, GGML_Q8_K=15 };

typedef struct { const char *ptr; uint64_t len; } gguf_str;

typedef struct {
    gguf_str name;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t ggml_type;
    uint64_t offset;       /* from data section start */
    const void *data;      /* at the vireo-hip ABI: a device pointer */
    uint64_t n_elems;
    uint64_t nbytes;
} gguf_tensor;

#ifdef __cplusplus
}
#endif
#endif
