/* GGUF v2/v3 reader (host side): the file is mapped read-only, the metadata
 * and the tensor table are parsed in place, and tensor pointers point into the
 * mapping. Behaviour follows the reference's reader (src/gguf.c:11-171):
 * the same structures, the same 32-byte default alignment overridden by a U32
 * "general.alignment", the same scalar convention (raw little-endian bits,
 * zero-extended; F32 and F64 as double) and the same nbytes rule
 * (n_elems / block_elems * block_bytes for the types of vireo_type_block, 0
 * otherwise). Every read is bounded by the end of the file, and a file whose
 * tensors would be read past its end is rejected instead of handed back. */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "vireo_gguf.h"

int vireo_type_block(uint32_t ggml_type, int *block_elems, int *block_bytes); /* runtime.hip */

/* ---- bounded little-endian reads over the mapping ---- */
typedef struct {
    const uint8_t *p, *end;
} span;

static int get(span *s, void *dst, uint64_t n) {
    if ((uint64_t)(s->end - s->p) < n) return -1;
    memcpy(dst, s->p, n);
    s->p += n;
    return 0;
}
static int get_u32(span *s, uint32_t *v) { return get(s, v, 4); }
static int get_u64(span *s, uint64_t *v) { return get(s, v, 8); }
static int get_str(span *s, gguf_str *out) {
    uint64_t n;
    if (get_u64(s, &n) || (uint64_t)(s->end - s->p) < n) return -1;
    out->ptr = (const char *)s->p;
    out->len = n;
    s->p += n;
    return 0;
}

/* bytes of one scalar of metadata type t; 0 for strings, arrays and unknown types */
static unsigned scalar_bytes(uint32_t t) {
    switch (t) {
    case GGUF_U8: case GGUF_I8: case GGUF_BOOL: return 1;
    case GGUF_U16: case GGUF_I16: return 2;
    case GGUF_U32: case GGUF_I32: case GGUF_F32: return 4;
    case GGUF_U64: case GGUF_I64: case GGUF_F64: return 8;
    default: return 0;
    }
}

/* step over `count` values of type t (arrays may nest a few levels) */
static int skip_values(span *s, uint32_t t, uint64_t count, int depth) {
    const unsigned sz = scalar_bytes(t);
    if (sz) {
        if ((uint64_t)(s->end - s->p) / sz < count) return -1;
        s->p += count * sz;
        return 0;
    }
    for (uint64_t i = 0; i < count; i++) {
        if (t == GGUF_STRING) {
            gguf_str str;
            if (get_str(s, &str)) return -1;
        } else if (t == GGUF_ARRAY && depth < 8) {
            uint32_t at;
            uint64_t n;
            if (get_u32(s, &at) || get_u64(s, &n) || skip_values(s, at, n, depth + 1)) return -1;
        } else {
            return -1;
        }
    }
    return 0;
}

static int parse_value(span *s, gguf_kv *kv, uint32_t t) {
    kv->type = t;
    if (t == GGUF_STRING) return get_str(s, &kv->str);
    if (t == GGUF_ARRAY) {
        if (get_u32(s, &kv->arr_type) || get_u64(s, &kv->arr_len)) return -1;
        kv->arr_data = s->p;
        return skip_values(s, kv->arr_type, kv->arr_len, 1);
    }
    const unsigned sz = scalar_bytes(t);
    if (!sz) return -1;
    uint64_t raw = 0;
    if (get(s, &raw, sz)) return -1;
    if (t == GGUF_F32) {
        float f;
        memcpy(&f, &raw, 4);
        kv->val.f = f;
    } else if (t == GGUF_F64) {
        double f;
        memcpy(&f, &raw, 8);
        kv->val.f = f;
    } else {
        kv->val.u = raw;
    }
    return 0;
}

static int str_is(const gguf_str *s, const char *k) {
    const size_t n = strlen(k);
    return s->len == n && memcmp(s->ptr, k, n) == 0;
}

void vireo_gguf_close(gguf_ctx *g) {
    if (!g) return;
    if (g->map && g->map != MAP_FAILED) munmap(g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    free(g->kv);
    free(g->tensors);
    free(g);
}

static gguf_ctx *fail(gguf_ctx *g, int err) {
    vireo_gguf_close(g);
    errno = err;
    return NULL;
}

gguf_ctx *vireo_gguf_open(const char *path) {
    if (!path) { errno = EINVAL; return NULL; }
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st)) {
        const int e = errno;
        close(fd);
        errno = e;
        return NULL;
    }
    if (st.st_size < 24) {  /* magic, version and the two counts */
        close(fd);
        errno = EINVAL;
        return NULL;
    }
    gguf_ctx *g = calloc(1, sizeof *g);
    if (!g) { close(fd); errno = ENOMEM; return NULL; }
    g->fd = fd;
    g->size = (size_t)st.st_size;
    g->alignment = 32;
    g->map = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (g->map == MAP_FAILED) { const int e = errno; g->map = NULL; return fail(g, e); }
    const uint8_t *base = (const uint8_t *)g->map;
    span s = {base, base + g->size};

    char magic[4];
    if (get(&s, magic, 4) || memcmp(magic, "GGUF", 4)) return fail(g, EINVAL);
    if (get_u32(&s, &g->version) || (g->version != 2 && g->version != 3)) return fail(g, EINVAL);
    if (get_u64(&s, &g->n_tensors) || get_u64(&s, &g->n_kv)) return fail(g, EINVAL);
    /* a key-value pair takes at least 13 bytes, a tensor entry at least 24 */
    const uint64_t left = (uint64_t)(s.end - s.p);
    if (g->n_kv > left / 13 || g->n_tensors > left / 24) return fail(g, EINVAL);

    g->kv = calloc(g->n_kv ? g->n_kv : 1, sizeof(gguf_kv));
    g->tensors = calloc(g->n_tensors ? g->n_tensors : 1, sizeof(gguf_tensor));
    if (!g->kv || !g->tensors) return fail(g, ENOMEM);
    for (uint64_t i = 0; i < g->n_kv; i++) {
        uint32_t t;
        if (get_str(&s, &g->kv[i].key) || get_u32(&s, &t) || parse_value(&s, &g->kv[i], t))
            return fail(g, EINVAL);
    }
    const gguf_kv *al = vireo_gguf_find(g, "general.alignment");
    if (al && al->type == GGUF_U32) {
        if (al->val.u == 0) return fail(g, EINVAL);
        g->alignment = al->val.u;
    }
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        gguf_tensor *t = &g->tensors[i];
        if (get_str(&s, &t->name) || get_u32(&s, &t->n_dims) || t->n_dims > 4) return fail(g, EINVAL);
        t->n_elems = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            if (get_u64(&s, &t->dims[d])) return fail(g, EINVAL);
            if (t->dims[d] && t->n_elems > UINT64_MAX / t->dims[d]) return fail(g, EINVAL);
            t->n_elems *= t->dims[d];
        }
        if (get_u32(&s, &t->ggml_type) || get_u64(&s, &t->offset)) return fail(g, EINVAL);
        int be, bb;
        if (vireo_type_block(t->ggml_type, &be, &bb) == 0) t->nbytes = t->n_elems / (uint64_t)be * (uint64_t)bb;
    }
    /* the data section starts at the next multiple of the alignment */
    const uint64_t pos = (uint64_t)(s.p - base);
    const uint64_t start = pos + (g->alignment - pos % g->alignment) % g->alignment;
    if (start > g->size) return fail(g, EINVAL);
    g->data = base + start;
    const uint64_t avail = g->size - start;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        gguf_tensor *t = &g->tensors[i];
        if (t->offset > avail || t->nbytes > avail - t->offset) return fail(g, EINVAL);
        t->data = g->data + t->offset;
    }
    return g;
}

const gguf_kv *vireo_gguf_find(const gguf_ctx *g, const char *key) {
    if (!g || !key) return NULL;
    for (uint64_t i = 0; i < g->n_kv; i++)
        if (str_is(&g->kv[i].key, key)) return &g->kv[i];
    return NULL;
}

int vireo_gguf_get_u64(const gguf_ctx *g, const char *key, uint64_t *out) {
    const gguf_kv *k = vireo_gguf_find(g, key);
    if (!k || !out) return -1;
    switch (k->type) {
    case GGUF_U8: case GGUF_U16: case GGUF_U32: case GGUF_U64:
    case GGUF_I8: case GGUF_I16: case GGUF_I32: case GGUF_I64: case GGUF_BOOL:
        *out = k->val.u;
        return 0;
    default: return -1;
    }
}

int vireo_gguf_get_f32(const gguf_ctx *g, const char *key, float *out) {
    const gguf_kv *k = vireo_gguf_find(g, key);
    if (!k || !out || (k->type != GGUF_F32 && k->type != GGUF_F64)) return -1;
    *out = (float)k->val.f;
    return 0;
}

const char *vireo_gguf_get_str(const gguf_ctx *g, const char *key, uint64_t *len) {
    const gguf_kv *k = vireo_gguf_find(g, key);
    if (!k || k->type != GGUF_STRING) return NULL;
    if (len) *len = k->str.len;
    return k->str.ptr;
}

const gguf_tensor *vireo_gguf_tensor_by_name(const gguf_ctx *g, const char *name) {
    if (!g || !name) return NULL;
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (str_is(&g->tensors[i].name, name)) return &g->tensors[i];
    return NULL;
}
