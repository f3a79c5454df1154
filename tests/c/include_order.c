/* Both orders of the reference's headers and this library's must compile and
 * see every name of both (built with -DREF_FIRST or without). */
#ifdef REF_FIRST
#include "gguf.h"
#include "kvstore.h"
#include "expert_store.h"
#include "vireo_hip.h"
#include "vireo_kv.h"
#else
#include "vireo_hip.h"
#include "vireo_kv.h"
#include "gguf.h"
#include "kvstore.h"
#include "expert_store.h"
#endif

/* names only the reference's headers declare, and names only ours do */
int use_both(const char *path) {
    gguf_ctx *g = gguf_open(path);
    int be = 0, bb = 0;
    (void)gguf_type_block(GGML_Q4_K, &be, &bb);
    KVStoreOps ops = {0};
    KVConfig cfg = {1, 64, 32, 0, 0, 0};
    VireoKVConfig vcfg = {cfg.n_layers, cfg.kv_dim, cfg.block_tokens, cfg.sink_tokens, cfg.window_tokens,
                          cfg.capacity_bytes};
    float acc[4], q[4] = {1, 2, 3, 4};
    KVSoftmax sm;
    kv_softmax_init(&sm, acc, 4);
    (void)kv_dot(q, q, 4);
    gguf_tensor t = {0};
    vireo_moe_model m = {0};
    ExpertStats st = {0};
    (void)ops;
    (void)vcfg;
    (void)t;
    (void)m;
    (void)st;
    if (g) gguf_close(g);
    return be + bb + (int)sizeof(VireoKVStats) + (int)sizeof(KVStats);
}
