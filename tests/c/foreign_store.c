/* A program that still links the reference's CPU src/expert_store.c (its
 * expert_store_create wins inside the executable) and hands that store to
 * moe_ffn_forward: the library must refuse it (-EINVAL) instead of reading
 * host pointers from a foreign struct layout. Runs without a GPU: the store
 * is checked before any device call. */
#include <errno.h>
#include <stdio.h>
#include "vireo_hip.h"

int main(void) {
    ExpertStore *es = expert_store_create(-1, 0, 1, 8); /* the executable's own (CPU) store */
    if (!es) return 3;
    gguf_tensor router = {0}, gate = {0}, up = {0}, down = {0};
    static float fake_router[8 * 256];
    router.ggml_type = GGML_F32;
    router.data = fake_router;
    gate.ggml_type = up.ggml_type = GGML_Q4_K;
    down.ggml_type = GGML_Q6_K;
    vireo_moe_layer ly = {&router, &gate, &up, &down, NULL};
    vireo_moe_model m = {256, 8, 2, 256, 1, 1, &ly, es};
    static float x[256], xb[256];
    int rc = moe_ffn_forward(&m, 0, x, xb, 1, NULL, NULL, NULL);
    const void *const *tab = NULL;
    int rc2 = expert_store_pin_layer(es, 0, &tab);
    printf("moe_ffn_forward=%d expert_store_pin_layer=%d\n", rc, rc2);
    expert_store_destroy(es);
    return (rc == -EINVAL && rc2 == -EINVAL) ? 0 : 1;
}
