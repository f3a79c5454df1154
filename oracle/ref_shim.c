/* Test infrastructure: exposes the reference's own MoE-FFN code for use as a
 * checker. This file is compiled together with the reference's unmodified
 * sources where they lie (see oracle/Makefile); nothing from the reference is
 * copied here.
 *
 * src/gguf_run.c keeps moe_ffn (src/gguf_run.c:185-214), rmsnorm (:161-165),
 * softmax_n (:181-182) and argmax (:254) `static`, so this translation unit
 * includes that file and wraps those functions with extern entry points.
 * `main` is renamed so the CLI does not clash, and every call that moe_ffn
 * makes to expert_store_lookup goes through ref_hook_lookup, which records the
 * selected expert ids in the order moe_ffn chose them before forwarding to the
 * reference ExpertStore (src/expert_store.c:72-92). That recording is the
 * reference's own top-k order, including its lowest-index tie-break. */
#define main vireo_gguf_main
#define expert_store_lookup ref_hook_lookup
#include "gguf_run.c"
#undef expert_store_lookup
#undef main

#include <unistd.h>

int expert_store_lookup(ExpertStore *s, int layer, int expert, ExpertView *view);

static int g_trace[64];
static int g_ntrace;

int ref_hook_lookup(ExpertStore *s, int layer, int expert, ExpertView *view) {
    if (g_ntrace < 64) g_trace[g_ntrace++] = expert;
    return expert_store_lookup(s, layer, expert, view);
}

/* gguf_matmul / gguf_dequant_row / gguf_f16_to_f32 are public in
 * src/gguf_compute.h and are exported by the reference object directly. */
int ref_type_block(uint32_t t, int *be, int *bb) { return gguf_type_block(t, be, bb); }

void ref_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    gguf_tensor tw = {0};
    tw.data = w; tw.ggml_type = GGML_F32;
    rmsnorm(o, x, &tw, n, eps);
}
void ref_softmax_n(float *v, int n) { softmax_n(v, n); }
int  ref_argmax(const float *v, int n) { return argmax(v, n); }

static int put_bytes(int fd, const void *p, uint64_t n, uint64_t off) {
    const uint8_t *b = (const uint8_t *)p;
    while (n) {
        ssize_t w = pwrite(fd, b, n, (off_t)off);
        if (w <= 0) return -1;
        b += w; n -= (uint64_t)w; off += (uint64_t)w;
    }
    return 0;
}

/* One MoE model (n_layers layers of ne experts) backed by an unlinked temp
 * file, so the reference ExpertStore pages expert slices with pread exactly
 * as it does from a GGUF file (src/gguf_run.c:320-333). */
typedef struct {
    int fd;
    gguf_ctx g;
    uint8_t anchor;
    gguf_tensor *tr, *tg, *tu, *tdn;
    Layer *L;
    Model m;
} RefMoE;

/* routers[l]: F32 [ne x d]; gate/up slices [fe x d], down slices [d x fe];
 * layer l, expert e slice lives at bytes_*[l] + e*slice. */
void *ref_moe_create(int n_layers, int d, int ne, int k, int fe, int renorm,
                     const float *const *routers, uint32_t gt, uint32_t ut, uint32_t dt,
                     const void *const *gate_all, const void *const *up_all, const void *const *down_all,
                     uint64_t gslice, uint64_t uslice, uint64_t dslice, uint64_t cap_bytes) {
    RefMoE *r = calloc(1, sizeof *r);
    if (!r) return NULL;
    char path[512];
    const char *td = getenv("TMPDIR");
    snprintf(path, sizeof path, "%s/vireo_ref_XXXXXX", (td && strlen(td) < 400) ? td : "/tmp");
    r->fd = mkstemp(path);
    if (r->fd < 0) { free(r); return NULL; }
    unlink(path);
    uint64_t G = gslice * (uint64_t)ne, U = uslice * (uint64_t)ne, D = dslice * (uint64_t)ne;
    uint64_t per_layer = G + U + D;
    for (int l = 0; l < n_layers; l++) {
        uint64_t base = per_layer * (uint64_t)l;
        if (put_bytes(r->fd, gate_all[l], G, base) || put_bytes(r->fd, up_all[l], U, base + G) ||
            put_bytes(r->fd, down_all[l], D, base + G + U)) { close(r->fd); free(r); return NULL; }
    }
    r->g.map = &r->anchor; r->g.fd = r->fd;
    r->tr = calloc((size_t)n_layers, sizeof(gguf_tensor));
    r->tg = calloc((size_t)n_layers, sizeof(gguf_tensor));
    r->tu = calloc((size_t)n_layers, sizeof(gguf_tensor));
    r->tdn = calloc((size_t)n_layers, sizeof(gguf_tensor));
    r->L = calloc((size_t)n_layers, sizeof(Layer));
    Model *m = &r->m;
    memset(m, 0, sizeof *m);
    m->g = &r->g; m->L = r->L; m->n_layers = n_layers; m->dim = d;
    m->is_moe = 1; m->n_experts = ne; m->n_used = k; m->ffn_exp = fe; m->topk_renorm = renorm;
    m->es = expert_store_create(r->fd, cap_bytes, n_layers, ne);
    for (int l = 0; l < n_layers; l++) {
        uint64_t base = per_layer * (uint64_t)l;
        r->tr[l].data = routers[l]; r->tr[l].ggml_type = GGML_F32;
        r->tg[l].data = &r->anchor; r->tg[l].ggml_type = gt; r->tg[l].nbytes = G;
        r->tu[l].data = &r->anchor; r->tu[l].ggml_type = ut; r->tu[l].nbytes = U;
        r->tdn[l].data = &r->anchor; r->tdn[l].ggml_type = dt; r->tdn[l].nbytes = D;
        r->L[l].router = &r->tr[l]; r->L[l].gate_exps = &r->tg[l];
        r->L[l].up_exps = &r->tu[l]; r->L[l].down_exps = &r->tdn[l];
        for (int e = 0; e < ne; e++) {
            ExpertSlices sl = { base + (uint64_t)e * gslice, base + G + (uint64_t)e * uslice,
                                base + G + U + (uint64_t)e * dslice,
                                (uint32_t)gslice, (uint32_t)uslice, (uint32_t)dslice };
            expert_store_register(m->es, l, e, &sl);
        }
    }
    m->rlog = malloc((size_t)ne * 4); m->gbuf = malloc((size_t)fe * 4); m->ubuf = malloc((size_t)fe * 4);
    m->dbuf = malloc((size_t)d * 4); m->moe_acc = malloc((size_t)d * 4);
    return r;
}

/* Run moe_ffn for layer `layer` over n_tokens tokens, one at a time, as
 * forward() does (src/gguf_run.c:239): x[t] += moe(hb[t]).
 * idx_out [n_tokens x k]: expert ids in the order moe_ffn looked them up.
 * prob_out [n_tokens x ne]: the softmax probabilities moe_ffn left in rlog. */
int ref_moe_run(void *h, int layer, float *x, const float *hb, int n_tokens, int *idx_out, float *prob_out) {
    RefMoE *r = (RefMoE *)h;
    Model *m = &r->m;
    int d = m->dim, ne = m->n_experts, kk = m->n_used < 64 ? m->n_used : 64;
    for (int t = 0; t < n_tokens; t++) {
        m->x = x + (size_t)t * d;
        g_ntrace = 0;
        moe_ffn(m, layer, (float *)(hb + (size_t)t * d));
        if (idx_out) for (int j = 0; j < kk; j++) idx_out[(size_t)t * kk + j] = j < g_ntrace ? g_trace[j] : -1;
        if (prob_out) memcpy(prob_out + (size_t)t * ne, m->rlog, (size_t)ne * 4);
    }
    return 0;
}

void ref_moe_stats(void *h, uint64_t out[7]) {
    ExpertStats st;
    expert_store_stats(((RefMoE *)h)->m.es, &st);
    out[0] = st.requests; out[1] = st.hits; out[2] = st.misses; out[3] = st.bytes_read;
    out[4] = st.resident_bytes; out[5] = st.capacity_bytes; out[6] = st.experts_resident;
}

void ref_moe_destroy(void *h) {
    RefMoE *r = (RefMoE *)h;
    if (!r) return;
    Model *m = &r->m;
    free(m->rlog); free(m->gbuf); free(m->ubuf); free(m->dbuf); free(m->moe_acc);
    expert_store_destroy(m->es);
    free(r->tr); free(r->tg); free(r->tu); free(r->tdn); free(r->L);
    close(r->fd);
    free(r);
}

/* ---- a whole model from a GGUF file, run through the reference's forward() ----
 * ref_model_open fills the reference's Model from a GGUF file with the
 * reference's reader (gguf_open), binding the fields that forward()
 * (src/gguf_run.c:216-251) reads under the names and defaults of the
 * reference's loader (src/gguf_run.c:276-333): metadata keys, per-layer
 * tensors, the MoE tensors with every expert slice registered in an
 * unbounded ExpertStore over the file, and an out-of-core KV store with the
 * "all" strategy, block_tokens per block and the loader's default sink (32)
 * and window (256). The tokenizer is not read. */
typedef struct {
    Model m;
    int block_tokens;
} RefModel;

static const gguf_tensor *tn(gguf_ctx *g, const char *fmt, int l) {
    char b[128];
    snprintf(b, sizeof b, fmt, l);
    return gguf_tensor_by_name(g, b);
}

void *ref_model_open(const char *path, int block_tokens) {
    gguf_ctx *g = gguf_open(path);
    if (!g) return NULL;
    RefModel *r = calloc(1, sizeof *r);
    Model *m = &r->m;
    m->g = g;
    char arch[64] = "qwen2", key[160];
    uint64_t al = 0, u = 0;
    const char *a = gguf_get_str(g, "general.architecture", &al);
    if (a) { int n = al < 63 ? (int)al : 63; memcpy(arch, a, (size_t)n); arch[n] = 0; }
#define KEYF(s) (snprintf(key, sizeof key, "%s.%s", arch, s), key)
    gguf_get_u64(g, KEYF("block_count"), &u); m->n_layers = (int)u;
    gguf_get_u64(g, KEYF("embedding_length"), &u); m->dim = (int)u;
    u = 0; gguf_get_u64(g, KEYF("feed_forward_length"), &u); m->ffn = (int)u;
    gguf_get_u64(g, KEYF("attention.head_count"), &u); m->n_heads = (int)u;
    gguf_get_u64(g, KEYF("attention.head_count_kv"), &u); m->n_kv_heads = (int)u;
    gguf_get_f32(g, KEYF("attention.layer_norm_rms_epsilon"), &m->eps);
    m->rope_base = 10000.0f;
    gguf_get_f32(g, KEYF("rope.freq_base"), &m->rope_base);
    m->head_size = m->dim / m->n_heads;
    if (gguf_get_u64(g, KEYF("attention.key_length"), &u) == 0) m->head_size = (int)u;
    if (gguf_get_u64(g, KEYF("expert_count"), &u) == 0 && u > 0) {
        m->is_moe = 1; m->n_experts = (int)u;
        m->n_used = 8; if (gguf_get_u64(g, KEYF("expert_used_count"), &u) == 0) m->n_used = (int)u;
        m->ffn_exp = m->ffn; if (gguf_get_u64(g, KEYF("expert_feed_forward_length"), &u) == 0) m->ffn_exp = (int)u;
        m->topk_renorm = strcmp(arch, "olmoe") != 0;
        if (gguf_get_u64(g, KEYF("expert_weights_norm"), &u) == 0) m->topk_renorm = (int)u;
    }
#undef KEYF
    m->tok_embd = gguf_tensor_by_name(g, "token_embd.weight");
    m->out_norm = gguf_tensor_by_name(g, "output_norm.weight");
    m->lm_head = gguf_tensor_by_name(g, "output.weight");
    if (!m->lm_head) m->lm_head = m->tok_embd;
    if (!m->tok_embd || !m->out_norm) { free(r); return NULL; }
    m->vocab = (int)m->tok_embd->dims[1];
    m->L = calloc((size_t)m->n_layers, sizeof(Layer));
    for (int l = 0; l < m->n_layers; l++) {
        Layer *ly = &m->L[l];
        ly->attn_norm = tn(g, "blk.%d.attn_norm.weight", l);
        ly->wq = tn(g, "blk.%d.attn_q.weight", l); ly->bq = tn(g, "blk.%d.attn_q.bias", l);
        ly->wk = tn(g, "blk.%d.attn_k.weight", l); ly->bk = tn(g, "blk.%d.attn_k.bias", l);
        ly->wv = tn(g, "blk.%d.attn_v.weight", l); ly->bv = tn(g, "blk.%d.attn_v.bias", l);
        ly->wo = tn(g, "blk.%d.attn_output.weight", l);
        ly->ffn_norm = tn(g, "blk.%d.ffn_norm.weight", l);
        ly->q_norm = tn(g, "blk.%d.attn_q_norm.weight", l);
        ly->k_norm = tn(g, "blk.%d.attn_k_norm.weight", l);
        if (m->is_moe) {
            ly->router = tn(g, "blk.%d.ffn_gate_inp.weight", l);
            ly->gate_exps = tn(g, "blk.%d.ffn_gate_exps.weight", l);
            ly->up_exps = tn(g, "blk.%d.ffn_up_exps.weight", l);
            ly->down_exps = tn(g, "blk.%d.ffn_down_exps.weight", l);
        } else {
            ly->wg = tn(g, "blk.%d.ffn_gate.weight", l);
            ly->wu = tn(g, "blk.%d.ffn_up.weight", l);
            ly->wd = tn(g, "blk.%d.ffn_down.weight", l);
        }
    }
    if (m->is_moe) {
        m->exp_type = m->L[0].gate_exps->ggml_type;
        m->es = expert_store_create(g->fd, 0, m->n_layers, m->n_experts);
        for (int l = 0; l < m->n_layers; l++) {
            const Layer *ly = &m->L[l];
            const uint8_t *map = (const uint8_t *)g->map;
            uint64_t bg = (uint64_t)((const uint8_t *)ly->gate_exps->data - map);
            uint64_t bu = (uint64_t)((const uint8_t *)ly->up_exps->data - map);
            uint64_t bd = (uint64_t)((const uint8_t *)ly->down_exps->data - map);
            uint32_t gs = (uint32_t)(ly->gate_exps->nbytes / m->n_experts);
            uint32_t us = (uint32_t)(ly->up_exps->nbytes / m->n_experts);
            uint32_t ds = (uint32_t)(ly->down_exps->nbytes / m->n_experts);
            for (int e = 0; e < m->n_experts; e++) {
                ExpertSlices sl = {bg + (uint64_t)e * gs, bu + (uint64_t)e * us, bd + (uint64_t)e * ds, gs, us, ds};
                expert_store_register(m->es, l, e, &sl);
            }
        }
    }
    KVConfig cfg = {0};
    cfg.n_layers = m->n_layers * m->n_kv_heads; cfg.kv_dim = m->head_size;
    cfg.block_tokens = block_tokens; cfg.sink_tokens = 32; cfg.window_tokens = 256;
    m->kv = kvstore_ooc_create(cfg, &VIREO_SELECT_ALL, NULL);
    int hs = m->head_size;
    m->x = malloc((size_t)m->dim * 4); m->xb = malloc((size_t)m->dim * 4);
    m->h1 = malloc((size_t)(m->ffn > 0 ? m->ffn : 1) * 4); m->h2 = malloc((size_t)(m->ffn > 0 ? m->ffn : 1) * 4);
    m->q = malloc((size_t)m->n_heads * hs * 4); m->k = malloc((size_t)m->n_kv_heads * hs * 4);
    m->v = malloc((size_t)m->n_kv_heads * hs * 4); m->att_out = malloc((size_t)m->n_heads * hs * 4);
    m->logits = malloc((size_t)m->vocab * 4);
    if (m->is_moe) {
        m->rlog = malloc((size_t)m->n_experts * 4); m->gbuf = malloc((size_t)m->ffn_exp * 4);
        m->ubuf = malloc((size_t)m->ffn_exp * 4); m->dbuf = malloc((size_t)m->dim * 4);
        m->moe_acc = malloc((size_t)m->dim * 4);
    }
    r->block_tokens = block_tokens;
    return r;
}

/* shape: dim, vocab, n_layers, n_heads, n_kv_heads, head_size, is_moe */
void ref_model_shape(void *h, int out[7]) {
    const Model *m = &((RefModel *)h)->m;
    out[0] = m->dim; out[1] = m->vocab; out[2] = m->n_layers; out[3] = m->n_heads;
    out[4] = m->n_kv_heads; out[5] = m->head_size; out[6] = m->is_moe;
}

/* forward(token, pos) (src/gguf_run.c:216); x_out [dim] receives the residual
 * stream after the last block, logits_out [vocab] the logits (want_logits). */
void ref_model_forward(void *h, int token, int pos, int want_logits, float *x_out, float *logits_out) {
    Model *m = &((RefModel *)h)->m;
    float *lg = forward(m, token, pos, want_logits);
    if (x_out) memcpy(x_out, m->x, (size_t)m->dim * 4);
    if (lg && logits_out) memcpy(logits_out, lg, (size_t)m->vocab * 4);
}

void ref_model_close(void *h) {
    RefModel *r = (RefModel *)h;
    if (!r) return;
    Model *m = &r->m;
    if (m->es) expert_store_destroy(m->es);
    if (m->kv) kv_destroy(m->kv);
    free(m->x); free(m->xb); free(m->h1); free(m->h2); free(m->q); free(m->k); free(m->v); free(m->att_out);
    free(m->logits); free(m->rlog); free(m->gbuf); free(m->ubuf); free(m->dbuf); free(m->moe_acc);
    free(m->L);
    gguf_close(m->g);
    free(r);
}
