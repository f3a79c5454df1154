/* Drives the library's GGUF reader (vireo_amd/csrc/gguf.c, compiled into this
 * program with AddressSanitizer and UndefinedBehaviorSanitizer by the CPU
 * tests) over the files named on the command line: opens each, reads every
 * metadata entry, string, array and tensor it reports, then closes it. Prints
 * one line per file, 1 if it opened and 0 if it was refused; a sanitizer
 * report ends the program with a failure. */
#include <stdio.h>
#include <string.h>
#include "vireo_gguf.h"

/* The ggml block table the reader sizes tensors with (src/gguf.c:27-38);
 * the library's copy lives in its HIP runtime file, which this program does
 * not link. */
int vireo_type_block(uint32_t t, int *be, int *bb) {
    switch (t) {
    case GGML_F32: *be = 1; *bb = 4; return 0;
    case GGML_F16: *be = 1; *bb = 2; return 0;
    case GGML_Q8_0: *be = 32; *bb = 34; return 0;
    case GGML_Q4_0: *be = 32; *bb = 18; return 0;
    case GGML_Q5_0: *be = 32; *bb = 22; return 0;
    case GGML_Q4_K: *be = 256; *bb = 144; return 0;
    case GGML_Q6_K: *be = 256; *bb = 210; return 0;
    default: return -22;
    }
}

static unsigned touch(const void *p, uint64_t n) {
    const unsigned char *b = (const unsigned char *)p;
    unsigned h = 0;
    for (uint64_t i = 0; i < n; i++) h = h * 31u + b[i];
    return h;
}

int main(int argc, char **argv) {
    unsigned sink = 0;
    for (int a = 1; a < argc; a++) {
        gguf_ctx *g = vireo_gguf_open(argv[a]);
        printf("%d\n", g != NULL);
        if (!g) continue;
        for (uint64_t i = 0; i < g->n_kv; i++) {
            const gguf_kv *kv = &g->kv[i];
            sink += touch(kv->key.ptr, kv->key.len);
            if (kv->type == GGUF_STRING) sink += touch(kv->str.ptr, kv->str.len);
            char key[256];
            uint64_t kl = kv->key.len < 255 ? kv->key.len : 255;
            memcpy(key, kv->key.ptr, kl);
            key[kl] = 0;
            uint64_t u, n;
            float f;
            sink += (unsigned)vireo_gguf_get_u64(g, key, &u) + (unsigned)vireo_gguf_get_f32(g, key, &f);
            if (vireo_gguf_get_str(g, key, &n)) sink += (unsigned)n;
            if (vireo_gguf_find(g, key) != kv && vireo_gguf_find(g, key) == NULL) return 3;
        }
        for (uint64_t i = 0; i < g->n_tensors; i++) {
            const gguf_tensor *t = &g->tensors[i];
            sink += touch(t->name.ptr, t->name.len);
            sink += touch(t->data, t->nbytes);
            char name[256];
            uint64_t nl = t->name.len < 255 ? t->name.len : 255;
            memcpy(name, t->name.ptr, nl);
            name[nl] = 0;
            if (!vireo_gguf_tensor_by_name(g, name)) return 4;
        }
        vireo_gguf_close(g);
    }
    fprintf(stderr, "checksum %u\n", sink);
    return 0;
}
