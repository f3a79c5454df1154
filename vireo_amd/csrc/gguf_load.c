/* MoE models from GGUF files into HBM (API: include/vireo_hip.h,
 * vireo_gguf_moe_load). The metadata keys, tensor names, defaults and expert
 * slice registration follow the reference's loader, src/gguf_run.c:266-333;
 * the file is read with this library's reader (gguf.c), the small tensors are
 * copied to the device, and the expert slices stay in the file until the
 * ExpertStore pages them into its HBM pool. Attention tensors are not read:
 * the MoE path does not use them. */
#define _POSIX_C_SOURCE 200809L
#define __HIP_PLATFORM_AMD__ 1
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <hip/hip_runtime_api.h>
#include "vireo_hip.h"

static _Thread_local char g_err[256];

static int fail_msg(int rc, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return rc;
}

const char *vireo_gguf_moe_error(void) { return g_err; }

/* everything the model owns besides the gguf context */
typedef struct {
    vireo_moe_layer *layers;   /* [n_layers] */
    gguf_tensor *dev;          /* [4 n_layers]: router (device copy), gate, up, down (types only) */
    const float **ffn_norm;    /* [n_layers] device pointers or NULL */
    gguf_tensor head, embd;    /* device copies */
    void **allocs;             /* device allocations to free */
    int n_allocs, cap_allocs;
} priv_t;

static int dev_copy(priv_t *p, const void *src, uint64_t bytes, void **out) {
    if (p->n_allocs == p->cap_allocs) {
        const int cap = p->cap_allocs ? 2 * p->cap_allocs : 16;
        void **a = realloc(p->allocs, sizeof(void *) * (size_t)cap);
        if (!a) return -ENOMEM;
        p->allocs = a;
        p->cap_allocs = cap;
    }
    void *d = NULL;
    if (hipMalloc(&d, bytes ? bytes : 1) != hipSuccess) return -ENOMEM;
    p->allocs[p->n_allocs++] = d;
    if (bytes && hipMemcpy(d, src, bytes, hipMemcpyHostToDevice) != hipSuccess) return -EIO;
    *out = d;
    return 0;
}

static const gguf_tensor *tensor_l(const gguf_ctx *g, const char *fmt, int l) {
    char name[96];
    snprintf(name, sizeof name, fmt, l);
    return vireo_gguf_tensor_by_name(g, name);
}

static int get_key(const gguf_ctx *g, const char *arch, const char *suffix, uint64_t *v) {
    char key[160];
    snprintf(key, sizeof key, "%s.%s", arch, suffix);
    return vireo_gguf_get_u64(g, key, v);
}

static int expert_type_ok(uint32_t t) { return t == GGML_Q8_0 || t == GGML_Q4_K || t == GGML_Q6_K; }

void vireo_gguf_moe_free(vireo_gguf_moe *m) {
    if (!m) return;
    if (m->model.es) expert_store_destroy(m->model.es);
    priv_t *p = (priv_t *)m->priv;
    if (p) {
        for (int i = 0; i < p->n_allocs; i++) hipFree(p->allocs[i]);
        free(p->allocs);
        free(p->layers);
        free(p->dev);
        free(p->ffn_norm);
        free(p);
    }
    vireo_gguf_close(m->gguf);
    free(m);
}

static int load(vireo_gguf_moe *m, const char *path, uint64_t cap, int load_head) {
    m->gguf = vireo_gguf_open(path);
    if (!m->gguf) return fail_msg(errno == EINVAL ? -EINVAL : -(errno ? errno : EIO), "cannot read %s as GGUF", path);
    const gguf_ctx *g = m->gguf;
    priv_t *p = calloc(1, sizeof *p);
    if (!p) return -ENOMEM;
    m->priv = p;

    /* metadata (src/gguf_run.c:274-293) */
    strcpy(m->arch, "qwen2");
    uint64_t alen = 0;
    const char *a = vireo_gguf_get_str(g, "general.architecture", &alen);
    if (a) {
        const size_t n = alen < sizeof m->arch - 1 ? (size_t)alen : sizeof m->arch - 1;
        memcpy(m->arch, a, n);
        m->arch[n] = 0;
    }
    uint64_t L = 0, d = 0, ffn = 0, E = 0, k = 8, fe = 0, renorm = strcmp(m->arch, "olmoe") != 0, u;
    if (get_key(g, m->arch, "block_count", &L) || L == 0 || L > 4096)
        return fail_msg(-EINVAL, "%s.block_count missing or out of range", m->arch);
    if (get_key(g, m->arch, "embedding_length", &d) || d == 0 || d > (1u << 20))
        return fail_msg(-EINVAL, "%s.embedding_length missing or out of range", m->arch);
    get_key(g, m->arch, "feed_forward_length", &ffn);
    if (get_key(g, m->arch, "expert_count", &E) || E == 0)
        return fail_msg(-EINVAL, "%s.expert_count missing: not a MoE model", m->arch);
    if (get_key(g, m->arch, "expert_used_count", &u) == 0) k = u;
    fe = ffn;
    if (get_key(g, m->arch, "expert_feed_forward_length", &u) == 0) fe = u;
    if (get_key(g, m->arch, "expert_weights_norm", &u) == 0) renorm = u;
    if (E > 256 || k < 1 || k > 64 || k > E || fe == 0 || fe > (1u << 20))
        return fail_msg(-EINVAL, "unsupported MoE shape: %llu experts, top-%llu, expert width %llu",
                        (unsigned long long)E, (unsigned long long)k, (unsigned long long)fe);
    char key[160];
    snprintf(key, sizeof key, "%s.attention.layer_norm_rms_epsilon", m->arch);
    m->eps = 0.0f;
    vireo_gguf_get_f32(g, key, &m->eps);

    /* per-layer MoE tensors (src/gguf_run.c:300-318) */
    p->layers = calloc((size_t)L, sizeof(vireo_moe_layer));
    p->dev = calloc((size_t)L * 4, sizeof(gguf_tensor));
    p->ffn_norm = calloc((size_t)L, sizeof(float *));
    if (!p->layers || !p->dev || !p->ffn_norm) return -ENOMEM;
    m->model.es = expert_store_create(g->fd, cap, (int)L, (int)E);
    if (!m->model.es) return fail_msg(-ENOMEM, "cannot create the expert store");
    const uint8_t *map = (const uint8_t *)g->map;
    for (int l = 0; l < (int)L; l++) {
        const gguf_tensor *r = tensor_l(g, "blk.%d.ffn_gate_inp.weight", l);
        const gguf_tensor *gt = tensor_l(g, "blk.%d.ffn_gate_exps.weight", l);
        const gguf_tensor *ut = tensor_l(g, "blk.%d.ffn_up_exps.weight", l);
        const gguf_tensor *dt = tensor_l(g, "blk.%d.ffn_down_exps.weight", l);
        const gguf_tensor *nt = tensor_l(g, "blk.%d.ffn_norm.weight", l);
        if (!r || !gt || !ut || !dt) return fail_msg(-EINVAL, "layer %d: missing an ffn_gate_inp/gate/up/down tensor", l);
        if (r->ggml_type != GGML_F32 || r->n_dims != 2 || r->dims[0] != d || r->dims[1] != E)
            return fail_msg(-EINVAL, "layer %d: ffn_gate_inp is not F32 [%llu x %llu]", l, (unsigned long long)E,
                            (unsigned long long)d);
        const gguf_tensor *ex[3] = {gt, ut, dt};
        const uint64_t rows[3] = {fe, fe, d}, cols[3] = {d, d, fe};
        for (int i = 0; i < 3; i++) {
            const gguf_tensor *t = ex[i];
            if (!expert_type_ok(t->ggml_type) || t->n_dims != 3 || t->dims[0] != cols[i] || t->dims[1] != rows[i] ||
                t->dims[2] != E || t->nbytes == 0 || t->nbytes % E || t->nbytes / E > UINT32_MAX)
                return fail_msg(-EINVAL, "layer %d: expert tensor %d has an unsupported type or shape", l, i);
        }
        if (gt->ggml_type != ut->ggml_type) return fail_msg(-EINVAL, "layer %d: gate and up types differ", l);
        if (nt && (nt->ggml_type != GGML_F32 || nt->n_elems != d))
            return fail_msg(-EINVAL, "layer %d: ffn_norm is not F32 [%llu]", l, (unsigned long long)d);

        gguf_tensor *dv = &p->dev[4 * l];
        void *dr;
        if (dev_copy(p, r->data, r->nbytes, &dr)) return fail_msg(-ENOMEM, "device copy of layer %d router", l);
        dv[0] = *r;
        dv[0].data = dr;
        for (int i = 0; i < 3; i++) {
            dv[1 + i] = *ex[i];
            dv[1 + i].data = NULL;  /* expert bytes come from the store */
        }
        if (nt) {
            void *dn;
            if (dev_copy(p, nt->data, nt->nbytes, &dn)) return fail_msg(-ENOMEM, "device copy of layer %d norm", l);
            p->ffn_norm[l] = (const float *)dn;
        }
        p->layers[l] = (vireo_moe_layer){&dv[0], &dv[1], &dv[2], &dv[3], NULL};
        /* expert e at offset + e * slice of each tensor (src/gguf_run.c:323-331) */
        const uint64_t bg = (uint64_t)((const uint8_t *)gt->data - map), bu = (uint64_t)((const uint8_t *)ut->data - map),
                       bd = (uint64_t)((const uint8_t *)dt->data - map);
        const uint64_t gs = gt->nbytes / E, us = ut->nbytes / E, ds = dt->nbytes / E;
        for (int e = 0; e < (int)E; e++) {
            const ExpertSlices sl = {bg + (uint64_t)e * gs, bu + (uint64_t)e * us, bd + (uint64_t)e * ds,
                                     (uint32_t)gs, (uint32_t)us, (uint32_t)ds};
            expert_store_register(m->model.es, l, e, &sl);
        }
    }
    m->model = (vireo_moe_model){(int)d, (int)E, (int)k, (int)fe, (int)renorm, (int)L, p->layers, m->model.es};

    /* stack: embeddings, output norm, LM head (src/gguf_run.c:294-299) */
    const gguf_tensor *te = vireo_gguf_tensor_by_name(g, "token_embd.weight");
    if (te && te->n_dims >= 2 && te->dims[0] == d && te->dims[1] <= INT32_MAX) m->vocab = (int)te->dims[1];
    m->stack = (vireo_moe_stack){&m->model, p->ffn_norm, NULL, NULL, m->vocab, m->eps, NULL};
    if (load_head) {
        const gguf_tensor *on = vireo_gguf_tensor_by_name(g, "output_norm.weight");
        const gguf_tensor *lm = vireo_gguf_tensor_by_name(g, "output.weight");
        if (!lm) lm = te;
        if (!te || !m->vocab) return fail_msg(-EINVAL, "no token_embd.weight [%llu x vocab]", (unsigned long long)d);
        if (!on || on->ggml_type != GGML_F32 || on->n_elems != d)
            return fail_msg(-EINVAL, "no F32 output_norm.weight [%llu]", (unsigned long long)d);
        if (lm->n_dims != 2 || lm->dims[0] != d || lm->dims[1] != (uint64_t)m->vocab || !lm->nbytes)
            return fail_msg(-EINVAL, "the LM head is not [%d x %llu]", m->vocab, (unsigned long long)d);
        void *dn, *dh;
        if (dev_copy(p, on->data, on->nbytes, &dn) || dev_copy(p, lm->data, lm->nbytes, &dh))
            return fail_msg(-ENOMEM, "device copy of the output norm or LM head");
        p->head = *lm;
        p->head.data = dh;
        m->stack.out_norm = (const float *)dn;
        m->stack.lm_head = &p->head;
        if (lm != te) {  /* an untied model: the embedding is its own tensor */
            void *de;
            if (dev_copy(p, te->data, te->nbytes, &de)) return fail_msg(-ENOMEM, "device copy of token_embd");
            p->embd = *te;
            p->embd.data = de;
            m->stack.tok_embd = &p->embd;
        }
    }
    g_err[0] = 0;
    return 0;
}

int vireo_gguf_moe_load(const char *path, uint64_t expert_capacity_bytes, int load_head, vireo_gguf_moe **out) {
    if (!path || !out) return fail_msg(-EINVAL, "null argument");
    *out = NULL;
    vireo_gguf_moe *m = calloc(1, sizeof *m);
    if (!m) return -ENOMEM;
    const int rc = load(m, path, expert_capacity_bytes, load_head);
    if (rc) {
        vireo_gguf_moe_free(m);
        return rc;
    }
    *out = m;
    return 0;
}
