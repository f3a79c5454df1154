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
#include <math.h>
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
    if (bytes && src && hipMemcpy(d, src, bytes, hipMemcpyHostToDevice) != hipSuccess) return -EIO;
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

static int expert_type_ok(uint32_t t) {
    return t == GGML_Q8_0 || t == GGML_Q4_K || t == GGML_Q6_K || t == GGML_Q5_0 || t == GGML_F16 || t == GGML_F32;
}

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

/* ---- whole models (vireo_gguf_model_load) --------------------------------- */

int vireo_rope_table(float base, int head_size, int max_pos, float *dev_out) {
    if (head_size <= 0 || head_size % 2 || max_pos <= 0 || !dev_out) return -EINVAL;
    const int half = head_size / 2;
    float *t = malloc(sizeof(float) * (size_t)max_pos * (size_t)head_size);
    if (!t) return -ENOMEM;
    for (int p = 0; p < max_pos; p++) {
        float *row = t + (size_t)p * (size_t)head_size;
        for (int j = 0; j < half; j++) {  /* the expressions of rope_neox, src/gguf_run.c:171 */
            const float freq = powf(base, -2.0f * j / head_size);
            const float a = p * freq;
            row[j] = cosf(a);
            row[half + j] = sinf(a);
        }
    }
    const hipError_t e = hipMemcpy(dev_out, t, sizeof(float) * (size_t)max_pos * (size_t)head_size,
                                   hipMemcpyHostToDevice);
    free(t);
    return e == hipSuccess ? 0 : -EIO;
}

typedef struct {
    vireo_gguf_moe *moe;   /* MoE files: routers, experts, FFN norms and head (owns the gguf context) */
    priv_t dev;            /* this loader's own device allocations */
    vireo_block *blocks;   /* [n_layers] */
    gguf_tensor *mats;     /* [n_layers x 7]: wq wk wv wo wg wu wd with device data */
    gguf_tensor embd, head;
} mpriv_t;

void vireo_gguf_model_free(vireo_gguf_model *m) {
    if (!m) return;
    mpriv_t *p = (mpriv_t *)m->priv;
    if (p) {
        for (int i = 0; i < p->dev.n_allocs; i++) hipFree(p->dev.allocs[i]);
        free(p->dev.allocs);
        free(p->blocks);
        free(p->mats);
        if (p->moe) {
            vireo_gguf_moe_free(p->moe); /* closes the file too */
            m->gguf = NULL;
        }
        free(p);
    }
    if (m->gguf) vireo_gguf_close(m->gguf);
    free(m);
}

static int mat_type_ok(uint32_t t) {
    return t == GGML_Q8_0 || t == GGML_Q4_K || t == GGML_Q6_K || t == GGML_Q5_0 || t == GGML_F16 || t == GGML_F32;
}

/* a [rows x cols] matrix (GGUF dims {cols, rows}) copied to the device */
static int dev_mat(priv_t *p, const gguf_tensor *t, uint64_t cols, uint64_t rows, gguf_tensor *out, const char *what,
                   int l) {
    if (!t) return fail_msg(-EINVAL, "layer %d: missing %s", l, what);
    if (!mat_type_ok(t->ggml_type) || t->n_dims != 2 || t->dims[0] != cols || t->dims[1] != rows)
        return fail_msg(-EINVAL, "layer %d: %s is not a supported [%llu x %llu] matrix", l, what,
                        (unsigned long long)rows, (unsigned long long)cols);
    void *d;
    if (dev_copy(p, t->data, t->nbytes, &d)) return fail_msg(-ENOMEM, "device copy of layer %d %s", l, what);
    *out = *t;
    out->data = d;
    return 0;
}

/* an n-element vector of any dequantizable type as F32 on the device (the
 * reference dequantizes norms and biases with gguf_dequant_row, src/gguf_run.c:163,166) */
static int dev_f32(priv_t *p, const gguf_tensor *t, uint64_t n, const float **out, const char *what, int l) {
    int be = 0, bb = 0;
    if (t->n_elems != n || vireo_type_block(t->ggml_type, &be, &bb) || n % (uint64_t)be || n > (1u << 24))
        return fail_msg(-EINVAL, "layer %d: %s has %llu elements of type %u, expected %llu", l, what,
                        (unsigned long long)t->n_elems, t->ggml_type, (unsigned long long)n);
    void *raw, *f;
    if (dev_copy(p, t->data, t->nbytes, &raw)) return fail_msg(-ENOMEM, "device copy of layer %d %s", l, what);
    if (t->ggml_type == GGML_F32) {
        *out = (const float *)raw;
        return 0;
    }
    if (dev_copy(p, NULL, n * sizeof(float), &f)) return fail_msg(-ENOMEM, "device copy of layer %d %s", l, what);
    if (qdequant_rows(t->ggml_type, raw, (float *)f, (int)n, 1, NULL))
        return fail_msg(-EINVAL, "layer %d: cannot dequantize %s", l, what);
    *out = (const float *)f;
    return 0;
}

static int load_model(vireo_gguf_model *m, const char *path, uint64_t cap, int max_pos) {
    mpriv_t *p = calloc(1, sizeof *p);
    if (!p) return -ENOMEM;
    m->priv = p;
    /* MoE files: the MoE loader binds routers, experts, FFN norms and the head */
    gguf_ctx *probe = vireo_gguf_open(path);
    if (!probe) return fail_msg(errno == EINVAL ? -EINVAL : -(errno ? errno : EIO), "cannot read %s as GGUF", path);
    strcpy(m->arch, "qwen2");
    uint64_t alen = 0;
    const char *a = vireo_gguf_get_str(probe, "general.architecture", &alen);
    if (a) {
        const size_t n = alen < sizeof m->arch - 1 ? (size_t)alen : sizeof m->arch - 1;
        memcpy(m->arch, a, n);
        m->arch[n] = 0;
    }
    uint64_t E = 0;
    const int is_moe = get_key(probe, m->arch, "expert_count", &E) == 0 && E > 0; /* src/gguf_run.c:288 */
    if (is_moe) {
        vireo_gguf_close(probe);
        int rc = vireo_gguf_moe_load(path, cap, 1, &p->moe);
        if (rc) return rc;
        m->gguf = p->moe->gguf;
        m->moe = p->moe->model;
    } else {
        m->gguf = probe;
    }
    const gguf_ctx *g = m->gguf;

    /* metadata (src/gguf_run.c:278-287) */
    uint64_t L = 0, d = 0, ffn = 0, nh = 0, nkv = 0, u;
    if (get_key(g, m->arch, "block_count", &L) || L == 0 || L > 4096)
        return fail_msg(-EINVAL, "%s.block_count missing or out of range", m->arch);
    if (get_key(g, m->arch, "embedding_length", &d) || d == 0 || d > (1u << 20))
        return fail_msg(-EINVAL, "%s.embedding_length missing or out of range", m->arch);
    get_key(g, m->arch, "feed_forward_length", &ffn);
    if (get_key(g, m->arch, "attention.head_count", &nh) || nh == 0 || nh > 1024)
        return fail_msg(-EINVAL, "%s.attention.head_count missing or out of range", m->arch);
    if (get_key(g, m->arch, "attention.head_count_kv", &nkv) || nkv == 0 || nh % nkv || nkv > 16)
        return fail_msg(-EINVAL, "%s.attention.head_count_kv missing or unsupported", m->arch);
    char key[160];
    float eps = 0.0f, base = 10000.0f;
    snprintf(key, sizeof key, "%s.attention.layer_norm_rms_epsilon", m->arch);
    vireo_gguf_get_f32(g, key, &eps);
    snprintf(key, sizeof key, "%s.rope.freq_base", m->arch);
    vireo_gguf_get_f32(g, key, &base);
    uint64_t hs = d / nh;
    if (get_key(g, m->arch, "attention.key_length", &u) == 0) hs = u;
    if (hs == 0 || hs % 2 || hs > 256) return fail_msg(-EINVAL, "unsupported head size %llu", (unsigned long long)hs);
    if (!is_moe && (ffn == 0 || ffn > (1u << 20)))
        return fail_msg(-EINVAL, "%s.feed_forward_length missing or out of range", m->arch);
    if (max_pos <= 0) return fail_msg(-EINVAL, "max_pos must be positive");

    /* per-block tensors (src/gguf_run.c:300-318) */
    p->blocks = calloc((size_t)L, sizeof(vireo_block));
    p->mats = calloc((size_t)L * 7, sizeof(gguf_tensor));
    if (!p->blocks || !p->mats) return -ENOMEM;
    const uint64_t nq = nh * hs, nk = nkv * hs;
    for (int l = 0; l < (int)L; l++) {
        vireo_block *b = &p->blocks[l];
        gguf_tensor *mt = &p->mats[7 * l];
        const gguf_tensor *t;
        int rc;
        if (!(t = tensor_l(g, "blk.%d.attn_norm.weight", l))) return fail_msg(-EINVAL, "layer %d: missing attn_norm", l);
        if ((rc = dev_f32(&p->dev, t, d, &b->attn_norm, "attn_norm", l))) return rc;
        if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.attn_q.weight", l), d, nq, &mt[0], "attn_q", l))) return rc;
        if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.attn_k.weight", l), d, nk, &mt[1], "attn_k", l))) return rc;
        if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.attn_v.weight", l), d, nk, &mt[2], "attn_v", l))) return rc;
        if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.attn_output.weight", l), nq, d, &mt[3], "attn_output", l)))
            return rc;
        b->wq = &mt[0], b->wk = &mt[1], b->wv = &mt[2], b->wo = &mt[3];
        if ((t = tensor_l(g, "blk.%d.attn_q.bias", l)) && (rc = dev_f32(&p->dev, t, nq, &b->bq, "attn_q.bias", l)))
            return rc;
        if ((t = tensor_l(g, "blk.%d.attn_k.bias", l)) && (rc = dev_f32(&p->dev, t, nk, &b->bk, "attn_k.bias", l)))
            return rc;
        if ((t = tensor_l(g, "blk.%d.attn_v.bias", l)) && (rc = dev_f32(&p->dev, t, nk, &b->bv, "attn_v.bias", l)))
            return rc;
        /* QK-norm: per head when dims[0] is the head size, else over the
         * whole vector (src/gguf_run.c:226-229) */
        if ((t = tensor_l(g, "blk.%d.attn_q_norm.weight", l))) {
            b->q_norm_len = t->dims[0] == hs ? (int)hs : (int)nq;
            if ((rc = dev_f32(&p->dev, t, (uint64_t)b->q_norm_len, &b->q_norm, "attn_q_norm", l))) return rc;
        }
        if ((t = tensor_l(g, "blk.%d.attn_k_norm.weight", l))) {
            b->k_norm_len = t->dims[0] == hs ? (int)hs : (int)nk;
            if ((rc = dev_f32(&p->dev, t, (uint64_t)b->k_norm_len, &b->k_norm, "attn_k_norm", l))) return rc;
        }
        if (is_moe) {
            b->ffn_norm = p->moe->stack.ffn_norm[l];
            if (!b->ffn_norm) return fail_msg(-EINVAL, "layer %d: missing ffn_norm", l);
        } else {
            if (!(t = tensor_l(g, "blk.%d.ffn_norm.weight", l))) return fail_msg(-EINVAL, "layer %d: missing ffn_norm", l);
            if ((rc = dev_f32(&p->dev, t, d, &b->ffn_norm, "ffn_norm", l))) return rc;
            if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.ffn_gate.weight", l), d, ffn, &mt[4], "ffn_gate", l)))
                return rc;
            if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.ffn_up.weight", l), d, ffn, &mt[5], "ffn_up", l))) return rc;
            if ((rc = dev_mat(&p->dev, tensor_l(g, "blk.%d.ffn_down.weight", l), ffn, d, &mt[6], "ffn_down", l)))
                return rc;
            b->wg = &mt[4], b->wu = &mt[5], b->wd = &mt[6];
        }
    }

    /* embedding, output norm, LM head (src/gguf_run.c:294-299) */
    vireo_model *md = &m->model;
    if (is_moe) {
        md->tok_embd = p->moe->stack.tok_embd ? p->moe->stack.tok_embd : p->moe->stack.lm_head;
        md->out_norm = p->moe->stack.out_norm;
        md->lm_head = p->moe->stack.lm_head;
        md->vocab = p->moe->vocab;
    } else {
        const gguf_tensor *te = vireo_gguf_tensor_by_name(g, "token_embd.weight");
        const gguf_tensor *on = vireo_gguf_tensor_by_name(g, "output_norm.weight");
        const gguf_tensor *lm = vireo_gguf_tensor_by_name(g, "output.weight");
        if (!te || te->n_dims != 2 || te->dims[0] != d || te->dims[1] == 0 || te->dims[1] > INT32_MAX)
            return fail_msg(-EINVAL, "no token_embd.weight [%llu x vocab]", (unsigned long long)d);
        if (!on) return fail_msg(-EINVAL, "no output_norm.weight");
        md->vocab = (int)te->dims[1];
        int rc;
        if ((rc = dev_mat(&p->dev, te, d, te->dims[1], &p->embd, "token_embd", -1))) return rc;
        if ((rc = dev_f32(&p->dev, on, d, &md->out_norm, "output_norm", -1))) return rc;
        md->tok_embd = &p->embd;
        md->lm_head = &p->embd;
        if (lm) {
            if ((rc = dev_mat(&p->dev, lm, d, te->dims[1], &p->head, "output", -1))) return rc;
            md->lm_head = &p->head;
        }
    }
    const uint32_t et = md->tok_embd->ggml_type;
    if (et != GGML_Q8_0 && et != GGML_F16 && et != GGML_F32)
        return fail_msg(-EINVAL, "token_embd type %u is not Q8_0, F16 or F32", et);
    void *rope;
    if (dev_copy(&p->dev, NULL, sizeof(float) * (uint64_t)max_pos * hs, &rope))
        return fail_msg(-ENOMEM, "device RoPE table");
    if (vireo_rope_table(base, (int)hs, max_pos, (float *)rope)) return fail_msg(-EIO, "RoPE table");
    md->n_layers = (int)L, md->dim = (int)d, md->n_heads = (int)nh, md->n_kv_heads = (int)nkv;
    md->head_size = (int)hs, md->ffn = (int)ffn, md->eps = eps, md->rope_base = base;
    md->blocks = p->blocks;
    md->moe = is_moe ? &m->moe : NULL;
    md->rope = (const float *)rope;
    md->max_pos = max_pos;
    g_err[0] = 0;
    return 0;
}

int vireo_gguf_model_load(const char *path, uint64_t expert_capacity_bytes, int max_pos, vireo_gguf_model **out) {
    if (!path || !out) return fail_msg(-EINVAL, "null argument");
    *out = NULL;
    vireo_gguf_model *m = calloc(1, sizeof *m);
    if (!m) return -ENOMEM;
    const int rc = load_model(m, path, expert_capacity_bytes, max_pos);
    if (rc) {
        vireo_gguf_model_free(m);
        return rc;
    }
    *out = m;
    return 0;
}
