/* A C caller of libvireo_hip through the public headers only, as a runner that
 * replaces the reference's moe_ffn would be: load an MoE GGUF file, run every
 * layer's moe_ffn_forward on one hidden state, then one greedy stack step.
 *
 *   moe_caller MODEL.gguf X.bin XB.bin OUT.bin
 *
 * X.bin / XB.bin hold `dim` floats (the residual and its RMSNorm); OUT.bin
 * receives x after layer 0, x after the last layer, then the stack step's
 * token (as a float) - what the tests compare with the oracle. */
#include <stdio.h>
#include <stdlib.h>
#include <hip/hip_runtime_api.h>
#include "vireo_hip.h"

static int fail(const char *what, int rc) {
    fprintf(stderr, "%s: %s (%s)\n", what, vireo_hip_strerror(rc), vireo_gguf_moe_error());
    return 1;
}

static int read_floats(const char *path, float *dst, int n) {
    FILE *f = fopen(path, "rb");
    if (!f) return -1;
    size_t got = fread(dst, sizeof(float), (size_t)n, f);
    fclose(f);
    return got == (size_t)n ? 0 : -1;
}

int main(int argc, char **argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s MODEL.gguf X.bin XB.bin OUT.bin\n", argv[0]);
        return 2;
    }
    int rc = vireo_hip_init(0);
    if (rc) return fail("vireo_hip_init", rc);
    vireo_gguf_moe *m = NULL;
    rc = vireo_gguf_moe_load(argv[1], 0, 1, &m);
    if (rc) return fail("vireo_gguf_moe_load", rc);
    const int dim = m->model.dim, L = m->model.n_layers;
    float *hx = malloc(sizeof(float) * (size_t)dim * 2), *out = malloc(sizeof(float) * ((size_t)dim * 2 + 1));
    if (!hx || !out) return 1;
    if (read_floats(argv[2], hx, dim) || read_floats(argv[3], hx + dim, dim)) {
        fprintf(stderr, "cannot read %d floats from %s / %s\n", dim, argv[2], argv[3]);
        return 1;
    }
    float *d_x, *d_xb, *d_logits;
    int32_t *d_token;
    if (hipMalloc((void **)&d_x, sizeof(float) * dim) || hipMalloc((void **)&d_xb, sizeof(float) * dim) ||
        hipMalloc((void **)&d_logits, sizeof(float) * (size_t)(m->vocab > 0 ? m->vocab : 1)) ||
        hipMalloc((void **)&d_token, sizeof(int32_t)))
        return fail("hipMalloc", -12);
    hipMemcpy(d_x, hx, sizeof(float) * dim, hipMemcpyHostToDevice);
    hipMemcpy(d_xb, hx + dim, sizeof(float) * dim, hipMemcpyHostToDevice);
    /* x += moe_l(xb) for every layer, synchronously (stream NULL), as the
     * reference's forward() calls moe_ffn (src/gguf_run.c:239) */
    for (int l = 0; l < L; l++) {
        rc = moe_ffn_forward(&m->model, l, d_x, d_xb, 1, NULL, NULL, NULL);
        if (rc) return fail("moe_ffn_forward", rc);
        if (l == 0) hipMemcpy(out, d_x, sizeof(float) * dim, hipMemcpyDeviceToHost);
    }
    hipMemcpy(out + dim, d_x, sizeof(float) * dim, hipMemcpyDeviceToHost);
    /* one greedy step of the stack from token 3 */
    int32_t tok = 3;
    hipMemcpy(d_token, &tok, sizeof tok, hipMemcpyHostToDevice);
    if (m->stack.lm_head) {
        rc = moe_stack_step(&m->stack, d_token, d_x, d_xb, d_logits, NULL);
        if (rc) return fail("moe_stack_step", rc);
        hipMemcpy(&tok, d_token, sizeof tok, hipMemcpyDeviceToHost);
    }
    out[2 * dim] = (float)tok;
    ExpertStats st;
    expert_store_stats(m->model.es, &st);
    printf("requests=%llu hits=%llu misses=%llu resident=%llu\n", (unsigned long long)st.requests,
           (unsigned long long)st.hits, (unsigned long long)st.misses, (unsigned long long)st.resident_bytes);
    FILE *f = fopen(argv[4], "wb");
    if (!f || fwrite(out, sizeof(float), (size_t)dim * 2 + 1, f) != (size_t)dim * 2 + 1) return 1;
    fclose(f);
    hipFree(d_x);
    hipFree(d_xb);
    hipFree(d_logits);
    hipFree(d_token);
    vireo_gguf_moe_free(m);
    free(hx);
    free(out);
    return 0;
}
