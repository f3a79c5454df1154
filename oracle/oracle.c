/* CPU oracle for vireo's quantized MoE-FFN path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h for what each function restates and how it is pinned.
 *
 * Every floating-point expression below keeps the reference's operation order
 * and rounding points. The build uses -std=c11, which makes GCC keep separate
 * multiplies and adds (no contraction), exactly as the reference Makefile:2
 * does; fused multiply-adds appear only where the reference uses the AVX2
 * _mm256_fmadd_ps intrinsic, written here as fmaf on eight explicit lanes. */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include "oracle.h"

/* ---- scalars --------------------------------------------------------------
 * src/gguf_compute.c:17-36. binary16 -> binary32 is exact: normal values only
 * rebias the exponent (15 -> 127); a subnormal is mant * 2^-24, which fp32
 * holds exactly; exponent 31 maps to inf/NaN keeping the payload. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t ex = (h >> 10) & 31u, man = h & 1023u, bits;
    float f;
    if (ex == 31u) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (ex != 0u) {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    } else {
        f = (float)man * 0x1p-24f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    }
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/gguf.c:27-38 */
int or_type_block(uint32_t t, int *be, int *bb) {
    switch (t) {
    case OR_F32:  *be = 1;   *bb = 4;   return 0;
    case OR_F16:  *be = 1;   *bb = 2;   return 0;
    case OR_Q8_0: *be = 32;  *bb = 34;  return 0;
    case 2:       *be = 32;  *bb = 18;  return 0; /* Q4_0: sized but never dequantized */
    case OR_Q5_0: *be = 32;  *bb = 22;  return 0;
    case OR_Q4_K: *be = 256; *bb = 144; return 0;
    case OR_Q6_K: *be = 256; *bb = 210; return 0;
    default: return -1;
    }
}

/* ---- dequantization --------------------------------------------------------
 * Q4_K super-block (144 B): f16 d @0, f16 dmin @2, 12 packed scale bytes @4,
 * 128 nibble bytes @16. Sub-block j (32 elements) has a 6-bit scale and a
 * 6-bit min; j<4 read the low 6 bits of bytes j / j+4, j>=4 combine a nibble
 * of byte j+4 with the top two bits of bytes j-4 / j (src/gguf_compute.c:45-51). */
static void q4k_unpack(int j, const uint8_t *s, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* src/gguf_compute.c:52-66: element 64c + l (l < 32) is the low nibble of
 * qs[32c + l] under sub-block 2c, element 64c + 32 + l its high nibble under
 * sub-block 2c+1; y = (d*sc)*q - dmin*m. */
static void dq_q4k(const uint8_t *b, float *y, int n) {
    for (int sb = 0; sb < n / 256; sb++, b += 144, y += 256) {
        float d = or_f16_to_f32(rd16(b)), dmin = or_f16_to_f32(rd16(b + 2));
        const uint8_t *qs = b + 16;
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            q4k_unpack(j, b + 4, &sc, &mn);
            float d1 = d * sc, m1 = dmin * mn;
            const uint8_t *q = qs + 32 * (j / 2);
            int shift = (j & 1) ? 4 : 0;
            for (int l = 0; l < 32; l++) y[32 * j + l] = d1 * ((q[l] >> shift) & 15) - m1;
        }
    }
}

/* src/gguf_compute.c:83-103. Q6_K super-block (210 B): ql[128] @0, qh[64]
 * @128, int8 scales[16] @192, f16 d @208. Element 128h + 32g + l (h<2, g<4,
 * l<32) takes nibble (g>=2 ? high : low) of ql[64h + l + 32(g&1)], bits
 * 2g..2g+1 of qh[32h + l], minus 32, scaled by (d*scales[8h + l/16 + 2g]). */
static void dq_q6k(const uint8_t *b, float *y, int n) {
    for (int sb = 0; sb < n / 256; sb++, b += 210, y += 256) {
        float d = or_f16_to_f32(rd16(b + 208));
        const int8_t *sc = (const int8_t *)(b + 192);
        for (int i = 0; i < 256; i++) {
            int h = i >> 7, g = (i >> 5) & 3, l = i & 31;
            int qlb = b[64 * h + l + 32 * (g & 1)];
            int lo4 = (g >= 2) ? (qlb >> 4) : (qlb & 15);
            int hi2 = (b[128 + 32 * h + l] >> (2 * g)) & 3;
            int q = (lo4 | (hi2 << 4)) - 32;
            y[i] = d * sc[8 * h + l / 16 + 2 * g] * q;
        }
    }
}

/* src/gguf_compute.c:67-82. Q5_0 block (22 B): f16 d, 32 high bits, 16
 * nibble bytes; element j (j<16) = low nibble of qs[j] | bit j << 4, element
 * j+16 = high nibble | bit j+16 << 4, both minus 16, times d. */
static void dq_q5_0(const uint8_t *b, float *y, int n) {
    for (int blk = 0; blk < n / 32; blk++, b += 22, y += 32) {
        float d = or_f16_to_f32(rd16(b));
        uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        const uint8_t *qs = b + 6;
        for (int j = 0; j < 16; j++) {
            int x0 = ((qs[j] & 15) | (int)(((qh >> j) & 1u) << 4)) - 16;
            int x1 = ((qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4)) - 16;
            y[j] = x0 * d;
            y[j + 16] = x1 * d;
        }
    }
}

/* src/gguf_compute.c:105-124 */
void or_dequant_row(uint32_t type, const void *src, float *dst, int n) {
    const uint8_t *b = (const uint8_t *)src;
    switch (type) {
    case OR_F32: memcpy(dst, src, (size_t)n * 4); return;
    case OR_F16:
        for (int i = 0; i < n; i++) dst[i] = or_f16_to_f32(rd16(b + 2 * i));
        return;
    case OR_Q8_0:
        for (int blk = 0; blk < n / 32; blk++, b += 34) {
            float d = or_f16_to_f32(rd16(b));
            for (int i = 0; i < 32; i++) dst[32 * blk + i] = (int8_t)b[2 + i] * d;
        }
        return;
    case OR_Q5_0: dq_q5_0(b, dst, n); return;
    case OR_Q4_K: dq_q4k(b, dst, n); return;
    case OR_Q6_K: dq_q6k(b, dst, n); return;
    default: return; /* unknown types write nothing, as in the reference */
    }
}

/* ---- mat-vec -----------------------------------------------------------------
 * The reference's AVX2 helpers (src/gguf_compute.c:127-157) keep eight fp32
 * lanes, each a chain of fused multiply-adds, then fold them with a fixed
 * tree: ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)). */
static float fold8(const float a[8]) {
    return ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
}

/* one Q8_0 block: sum of 32 int8 * x, unscaled (src/gguf_compute.c:138-148) */
static float q8_block_dot(const int8_t *qs, const float *x) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < 4; k++)
        for (int l = 0; l < 8; l++) a[l] = fmaf((float)qs[8 * k + l], x[8 * k + l], a[l]);
    return fold8(a);
}

/* src/gguf_compute.c:149-156 */
static float f32_dot(const float *a, const float *b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float s = fold8(acc);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* src/gguf_compute.c:159-214. Each output row is computed by one thread in
 * block order, so the result does not depend on the thread count; OpenMP is
 * used only when n*d > 2^20, as in the reference. */
void or_matmul(float *y, const float *x, uint32_t type, const void *w, int n, int d) {
    const int par = (long)n * (long)d > (1L << 20);
    const uint8_t *base = (const uint8_t *)w;
    if (type == OR_Q8_0) {
        const int nb = n / 32;
#pragma omp parallel for schedule(static) if (par)
        for (int o = 0; o < d; o++) {
            const uint8_t *row = base + (size_t)o * nb * 34;
            float acc = 0.0f;
            for (int j = 0; j < nb; j++) {
                float scale = or_f16_to_f32(rd16(row + 34 * j));
                acc += q8_block_dot((const int8_t *)(row + 34 * j + 2), x + 32 * j) * scale;
            }
            y[o] = acc;
        }
        return;
    }
    int be, bb;
    if (type != OR_F32 && type != OR_F16 && or_type_block(type, &be, &bb) == 0) {
        const size_t row_bytes = (size_t)(n / be) * bb;
#pragma omp parallel if (par)
        {
            float *tmp = (float *)malloc((size_t)n * sizeof(float));
#pragma omp for schedule(static)
            for (int o = 0; o < d; o++) {
                or_dequant_row(type, base + (size_t)o * row_bytes, tmp, n);
                y[o] = f32_dot(tmp, x, n);
            }
            free(tmp);
        }
        return;
    }
    if (type == OR_F32) {
        const float *W = (const float *)w;
#pragma omp parallel for schedule(static) if (par)
        for (int o = 0; o < d; o++) {
            const float *r = W + (size_t)o * n;
            float a = 0.0f;
            for (int i = 0; i < n; i++) a += r[i] * x[i];
            y[o] = a;
        }
        return;
    }
    if (type == OR_F16) {
#pragma omp parallel for schedule(static) if (par)
        for (int o = 0; o < d; o++) {
            const uint8_t *r = base + (size_t)o * n * 2;
            float a = 0.0f;
            for (int i = 0; i < n; i++) a += or_f16_to_f32(rd16(r + 2 * i)) * x[i];
            y[o] = a;
        }
    }
}

/* ---- model glue ----------------------------------------------------------- */

/* src/gguf_run.c:161-165: o = (x * r) * w with r = 1/sqrt(mean(x^2) + eps) */
void or_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    float r = 1.0f / sqrtf(ss / n + eps);
    for (int i = 0; i < n; i++) o[i] = x[i] * r * w[i];
}

/* src/gguf_run.c:181-182 */
void or_softmax(float *v, int n) {
    float m = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > m) m = v[i];
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        v[i] = expf(v[i] - m);
        s += v[i];
    }
    for (int i = 0; i < n; i++) v[i] /= s;
}

/* src/gguf_run.c:189-192: k rounds, each taking the not-yet-chosen expert with
 * the largest probability (strict >, scanning ids upward, so the lowest id wins
 * a tie); optional renormalisation by the in-order sum of the chosen weights. */
void or_topk(const float *p, int ne, int k, int renorm, int *idx, float *w) {
    int kk = k < 64 ? k : 64;
    for (int t = 0; t < kk; t++) {
        int best = -1;
        float bv = -1.0f;
        for (int e = 0; e < ne; e++) {
            int taken = 0;
            for (int j = 0; j < t; j++)
                if (idx[j] == e) { taken = 1; break; }
            if (!taken && p[e] > bv) { bv = p[e]; best = e; }
        }
        idx[t] = best;
        w[t] = bv;
    }
    if (renorm) {
        float ws = 0.0f;
        for (int t = 0; t < kk; t++) ws += w[t];
        if (ws > 0.0f)
            for (int t = 0; t < kk; t++) w[t] /= ws;
    }
}

/* src/gguf_run.c:254 */
int or_argmax(const float *v, int n) {
    int bi = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; bi = i; }
    return bi;
}

/* src/gguf_run.c:185-214, one token at a time. */
void or_moe_ffn(const or_moe_cfg *c, const float *router, const float *logit_bias,
                const void *const *gate, const void *const *up, const void *const *down,
                float *x, const float *hb, int n_tokens,
                int *idx_out, float *w_out, float *prob_out) {
    const int d = c->d, ne = c->ne, fe = c->fe, kk = c->k < 64 ? c->k : 64;
    float *p = malloc((size_t)ne * 4), *g = malloc((size_t)fe * 4), *u = malloc((size_t)fe * 4);
    float *dv = malloc((size_t)d * 4), *acc = malloc((size_t)d * 4);
    int idx[64];
    float w[64];
    for (int t = 0; t < n_tokens; t++) {
        const float *h = hb + (size_t)t * d;
        float *xt = x + (size_t)t * d;
        or_matmul(p, h, OR_F32, router, d, ne);
        if (logit_bias)
            for (int e = 0; e < ne; e++) p[e] += logit_bias[e];
        or_softmax(p, ne);
        or_topk(p, ne, c->k, c->renorm, idx, w);
        if (prob_out) memcpy(prob_out + (size_t)t * ne, p, (size_t)ne * 4);
        if (idx_out) memcpy(idx_out + (size_t)t * kk, idx, (size_t)kk * sizeof(int));
        if (w_out) memcpy(w_out + (size_t)t * kk, w, (size_t)kk * 4);
        for (int i = 0; i < d; i++) acc[i] = 0.0f;
        for (int j = 0; j < kk; j++) {
            int e = idx[j];
            if (e < 0 || !gate[e] || !up[e] || !down[e]) continue; /* failed lookup: skipped */
            or_matmul(g, h, c->gate_type, gate[e], d, fe);
            or_matmul(u, h, c->up_type, up[e], d, fe);
            for (int i = 0; i < fe; i++) {
                float gv = g[i];
                g[i] = (gv / (1.0f + expf(-gv))) * u[i];
            }
            or_matmul(dv, g, c->down_type, down[e], fe, d);
            for (int i = 0; i < d; i++) acc[i] += w[j] * dv[i];
        }
        for (int i = 0; i < d; i++) xt[i] += acc[i];
    }
    free(p); free(g); free(u); free(dv); free(acc);
}

/* ---- expert pager (src/expert_store.c) ------------------------------------ */
typedef struct {
    uint64_t off[3];
    uint32_t len[3];
    void *buf[3];
    uint64_t bytes, last_used;
    int resident, lease, registered;
} or_slot;

struct or_store {
    int fd, n_layers, n_experts;
    or_slot *slots;
    uint64_t tick, resident_bytes, capacity;
    uint64_t requests, hits, misses, bytes_read, experts_resident;
};

or_store *or_store_create(int fd, uint64_t capacity_bytes, int n_layers, int n_experts) {
    or_store *s = calloc(1, sizeof *s);
    s->fd = fd;
    s->n_layers = n_layers;
    s->n_experts = n_experts;
    s->slots = calloc((size_t)n_layers * n_experts, sizeof(or_slot));
    s->capacity = capacity_bytes;
    return s;
}

void or_store_register(or_store *s, int layer, int expert, uint64_t gate_off, uint64_t up_off,
                       uint64_t down_off, uint32_t gate_bytes, uint32_t up_bytes, uint32_t down_bytes) {
    or_slot *sl = &s->slots[(size_t)layer * s->n_experts + expert];
    sl->off[0] = gate_off; sl->off[1] = up_off; sl->off[2] = down_off;
    sl->len[0] = gate_bytes; sl->len[1] = up_bytes; sl->len[2] = down_bytes;
    sl->bytes = (uint64_t)gate_bytes + up_bytes + down_bytes;
    sl->registered = 1;
}

/* Evict unleased residents, least recently used first, until `need` more
 * bytes fit; if every resident is leased the store stays over budget
 * (src/expert_store.c:52-63). */
static void or_make_room(or_store *s, uint64_t need) {
    if (!s->capacity) return;
    const int n = s->n_layers * s->n_experts;
    while (s->resident_bytes + need > s->capacity) {
        or_slot *victim = NULL;
        for (int i = 0; i < n; i++) {
            or_slot *c = &s->slots[i];
            if (c->resident && !c->lease && (!victim || c->last_used < victim->last_used)) victim = c;
        }
        if (!victim) break;
        for (int k = 0; k < 3; k++) { free(victim->buf[k]); victim->buf[k] = NULL; }
        victim->resident = 0;
        s->resident_bytes -= victim->bytes;
        s->experts_resident--;
    }
}

int or_store_lookup(or_store *s, int layer, int expert, or_view *v) {
    or_slot *sl = &s->slots[(size_t)layer * s->n_experts + expert];
    s->requests++;
    if (!sl->registered) { memset(v, 0, sizeof *v); return -1; }
    if (sl->resident) {
        s->hits++;
    } else {
        s->misses++;
        or_make_room(s, sl->bytes);
        for (int k = 0; k < 3; k++) {
            sl->buf[k] = malloc(sl->len[k]);
            if (sl->buf[k] && pread(s->fd, sl->buf[k], sl->len[k], (off_t)sl->off[k]) < 0) { /* as reference */ }
            s->bytes_read += sl->len[k];
        }
        sl->resident = 1;
        s->resident_bytes += sl->bytes;
        s->experts_resident++;
    }
    sl->last_used = ++s->tick;
    sl->lease++;
    v->gate = sl->buf[0]; v->up = sl->buf[1]; v->down = sl->buf[2]; v->slot = sl;
    return 0;
}

void or_store_release(or_store *s, or_view *v) {
    (void)s;
    if (v && v->slot) {
        or_slot *sl = (or_slot *)v->slot;
        if (sl->lease > 0) sl->lease--;
    }
    if (v) memset(v, 0, sizeof *v);
}

void or_store_stats(const or_store *s, uint64_t out[7]) {
    out[0] = s->requests; out[1] = s->hits; out[2] = s->misses; out[3] = s->bytes_read;
    out[4] = s->resident_bytes; out[5] = s->capacity; out[6] = s->experts_resident;
}

void or_store_destroy(or_store *s) {
    if (!s) return;
    const int n = s->n_layers * s->n_experts;
    for (int i = 0; i < n; i++)
        for (int k = 0; k < 3; k++) free(s->slots[i].buf[k]);
    free(s->slots);
    free(s);
}
