// Whole-model decode: forward() of the reference's GGUF runner
// (src/gguf_run.c:216-251) on the device, one launch sequence per token:
// embedding, per block RMSNorm -> q/k/v matvecs (+ biases) -> QK-norms ->
// NEOX RoPE -> KV append -> grouped-query attention over the KV store ->
// output projection -> residual -> RMSNorm -> MoE layer or dense SwiGLU FFN
// -> residual, then the output norm, LM head and argmax. The matvecs are
// qmatvec (the output and down projections add into the residual stream
// themselves), the attention is the KV store's kernel, the MoE layer is the
// decode plan of moe_ffn_forward; this file adds the small element-wise
// kernels (biases, per-head QK-norms and RoPE in one launch).
#include <hip/hip_runtime.h>
#include "common.h"
#include "vireo_hip.h"
#include "route_kernels.h"
#include "vireo_kv.h"
#include "kv_view.h"

namespace {

// NEOX rotation of q (nq heads) and k (nk heads) in place at one position
// (rope_neox, src/gguf_run.c:169-174): pair (j, j + hs/2) of every head turns
// by angle a_j; tab = [cos a_0 .. cos a_{hs/2-1}, sin a_0 ..]. Each product
// and sum is rounded on its own, as the reference's C (no contraction).
// The table row is that of position pos_dev ? *pos_dev : pos; a device
// position outside [0, max_pos) rotates nothing.
__global__ void __launch_bounds__(256) rope_kernel(float *__restrict__ q, int nq, float *__restrict__ k, int nk, int hs,
                                                   const float *__restrict__ rope, int pos,
                                                   const int32_t *__restrict__ pos_dev, int max_pos) {
    const int half = hs / 2;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (pos_dev) pos = *pos_dev;
    if (i >= (nq + nk) * half || pos < 0 || pos >= max_pos) return;
    const float *tab = rope + size_t(pos) * hs;
    const int h = i / half, j = i % half;
    float *p = h < nq ? q + size_t(h) * hs : k + size_t(h - nq) * hs;
    const float c = tab[j], s = tab[half + j];
    const float x0 = p[j], x1 = p[j + half];
    p[j] = sub_rn(mul_rn(x0, c), mul_rn(x1, s));
    p[j + half] = add_rn(mul_rn(x0, s), mul_rn(x1, c));
}

// The attention inputs of one token in one launch: workgroup h (one wave)
// takes query head h, then the key heads, then the value heads (value heads
// only when they have a bias). A head gets its bias (as add_kernel), its
// RMSNorm over the head (as rmsnorm_kernel over a row of hs <= 256 values:
// lane l squares values l + 64 c, each group c of 64 is summed by one wave
// reduction and the groups' sums are added as ((s0 + s1) + (s2 + s3)), so
// the result is that kernel's bit for bit) and then, for queries and keys,
// the rotation of rope_kernel. hs is a multiple of 64. With a contiguous
// store (kv.base) the key and value heads are also appended at the position,
// as kv_append_pos_kernel appends them (kv head h to store layer layer0 + h;
// nothing outside [0, max_blocks G)).
struct HeadJob {
    float *p;           // heads x hs values, updated in place
    const float *bias;  // heads x hs values, or null
    const float *norm;  // hs RMSNorm weights shared by the heads, or null: no norm
    int heads;
};
__global__ void __launch_bounds__(64) head_prologue_kernel(HeadJob q, HeadJob k, HeadJob v, int hs, float eps,
                                                           const float *__restrict__ rope, int pos,
                                                           const int32_t *__restrict__ pos_dev, int max_pos,
                                                           KvContigView kv, int layer0) {
    __shared__ float row[256];
    int h = blockIdx.x, kind = 0;  // 0 query, 1 key, 2 value
    HeadJob j = q;
    if (h >= q.heads) {
        h -= q.heads, j = k, kind = 1;
        if (h >= k.heads) h -= k.heads, j = v, kind = 2;
    }
    const int l = threadIdx.x, ng = hs >> 6, half = hs / 2;
    float *p = j.p + size_t(h) * hs;
    // 1. every load that needs no position, issued with the position's:
    //    the head's values, its bias and the norm weights (unconditional:
    //    slots past the head and absent operands read the head's values
    //    again, unused)
    if (pos_dev) pos = *pos_dev;
    const float *bp = j.bias ? j.bias + size_t(h) * hs : p, *np = j.norm ? j.norm : p;
    float val[4], bia[4], nrm[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int i = min(64 * c + l, hs - 1);
        val[c] = p[i];
        bia[c] = bp[i];
        nrm[c] = np[i];
    }
    // 2. the position's loads: the rotation's table entries and, for a key
    //    appended to the store, the block's mean-key entries this lane updates
    const bool rotate = kind < 2 && pos >= 0 && pos < max_pos;
    float *srow = nullptr, *ks = nullptr;
    float inv = 0.0f;
    int slot = 0;
    if (kv.base && kind > 0 && pos >= 0 && pos < kv.max_blocks * kv.G) {
        const int b = pos / kv.G;
        slot = pos % kv.G;
        const size_t li = size_t(layer0 + h) * kv.max_blocks + b;
        srow = kv.base + li * size_t(2 * kv.G * hs) + size_t(kind == 1 ? slot : kv.G + slot) * hs;
        if (kind == 1) ks = kv.ksum + li * size_t(hs);
        inv = 1.0f / float(slot + 1);
    }
    // the indices this lane emits: rotated, i and i + half for i = l, l + 64
    // (below half); else l + 64 c (below hs)
    int ei[4];
    bool eon[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        if (rotate) {
            const int i = l + 64 * (u & 1);
            ei[u] = u < 2 ? i : i + half;
            eon[u] = i < half;
        } else {
            ei[u] = l + 64 * u;
            eon[u] = ei[u] < hs;
        }
    }
    const float *tab = rope + size_t(rotate ? pos : 0) * hs;
    float cs[2], sn[2], kold[4];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int i = min(l + 64 * u, half - 1);
        cs[u] = tab[i];
        sn[u] = tab[half + i];
    }
    const float *kp = ks ? ks : p;
#pragma unroll
    for (int u = 0; u < 4; u++) kold[u] = kp[min(ei[u], hs - 1)];
    // 3. the arithmetic
#pragma unroll
    for (int c = 0; c < 4; c++)
        if (j.bias) val[c] = add_rn(val[c], bia[c]);
    if (j.norm) {
        double part[4];
#pragma unroll
        for (int c = 0; c < 4; c++) part[c] = c < ng ? wave_sum_d(double(mul_rn(val[c], val[c]))) : 0.0;
        const float ss = float((part[0] + part[1]) + (part[2] + part[3]));
        const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(ss, float(hs)), eps)));
#pragma unroll
        for (int c = 0; c < 4; c++) val[c] = mul_rn(mul_rn(val[c], r), nrm[c]);
    }
    // the head's final value u at index ei[u]: to its buffer, and to the store
    float outv[4];
    if (rotate) {
#pragma unroll
        for (int c = 0; c < 4; c++)
            if (c < ng) row[64 * c + l] = val[c];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int i = min(l + 64 * u, half - 1);
            const float x0 = row[i], x1 = row[i + half];
            outv[u] = sub_rn(mul_rn(x0, cs[u]), mul_rn(x1, sn[u]));
            outv[u + 2] = add_rn(mul_rn(x0, sn[u]), mul_rn(x1, cs[u]));
        }
    } else {
#pragma unroll
        for (int u = 0; u < 4; u++) outv[u] = val[u];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        if (!eon[u]) continue;
        const int i = ei[u];
        const float x = outv[u];
        p[i] = x;
        if (srow) {
            srow[i] = x;
            if (ks) {
                const float old = slot == 0 ? 0.0f : kold[u];  // a new block's mean starts at zero
                ks[i] = add_rn(old, mul_rn(sub_rn(x, old), inv));
            }
        }
    }
}

// y_i += b_i for up to three (y, b, n) vectors (add_bias, src/gguf_run.c:166,
// and the residual adds x += xb, :237 / :248); a null b is skipped
struct AddJob {
    float *y;
    const float *b;
    int n;
};
__global__ void __launch_bounds__(256) add_kernel(AddJob j0, AddJob j1, AddJob j2) {
    const AddJob &j = blockIdx.y == 0 ? j0 : blockIdx.y == 1 ? j1 : j2;
    if (!j.b) return;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < j.n; i += gridDim.x * 256) j.y[i] = add_rn(j.y[i], j.b[i]);
}

// *pos += 1 (the device position of a captured decode loop)
__global__ void advance_kernel(int32_t *pos) { *pos += 1; }

// h1_i = silu(h1_i) * h2_i (src/gguf_run.c:246)
__global__ void __launch_bounds__(256) swiglu_kernel(float *__restrict__ h1, const float *__restrict__ h2, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h1[i] = swiglu(h1[i], h2[i]);
}

int add3(AddJob a, AddJob b, AddJob c, hipStream_t s) {
    const int n = max(a.n, max(b.n, c.n));
    const unsigned gx = unsigned(min((n + 255) / 256, 64));
    hipLaunchKernelGGL(add_kernel, dim3(gx, 3), dim3(256), 0, s, a, b, c);
    return vh_check(hipGetLastError());
}

int64_t pad64(int64_t n) { return (n + 63) / 64 * 64; }

// the state's buffers, each 256-byte aligned
struct Bufs {
    float *xb, *q, *k, *v, *att, *h1, *h2;
};

Bufs carve(const vireo_model *m, void *state) {
    const int64_t nq = int64_t(m->n_heads) * m->head_size, nk = int64_t(m->n_kv_heads) * m->head_size;
    const int64_t nf = m->moe ? 0 : m->ffn;
    float *p = static_cast<float *>(state);
    Bufs b;
    b.xb = p, p += pad64(m->dim);
    b.q = p, p += pad64(nq);
    b.k = p, p += pad64(nk);
    b.v = p, p += pad64(nk);
    b.att = p, p += pad64(nq);
    b.h1 = p, p += pad64(nf);
    b.h2 = p;
    return b;
}

int check_model(const vireo_model *m) {
    if (!m || !m->blocks || !m->tok_embd || m->n_layers <= 0 || m->dim <= 0 || m->n_heads <= 0 ||
        m->n_kv_heads <= 0 || m->n_heads % m->n_kv_heads || m->head_size <= 0 || m->head_size % 2 || m->vocab <= 0 ||
        !m->rope || m->max_pos <= 0)
        return -EINVAL;
    if (m->moe ? (m->moe->n_layers != m->n_layers || m->moe->dim != m->dim) : m->ffn <= 0) return -EINVAL;
    for (int l = 0; l < m->n_layers; l++) {
        const vireo_block &b = m->blocks[l];
        if (!b.wq || !b.wk || !b.wv || !b.wo) return -EINVAL;
        if (!m->moe && (!b.wg || !b.wu || !b.wd)) return -EINVAL;
    }
    return 0;
}

}  // namespace

extern "C" int64_t vireo_model_state_bytes(const vireo_model *m) {
    if (int rc = check_model(m)) return rc;
    const int64_t nq = int64_t(m->n_heads) * m->head_size, nk = int64_t(m->n_kv_heads) * m->head_size;
    const int64_t nf = m->moe ? 0 : m->ffn;
    return 4 * (pad64(m->dim) + 2 * pad64(nq) + 2 * pad64(nk) + 2 * pad64(nf));
}

namespace {

// one token through the model at position pos (host) or *pos_dev (device)
int model_step(const vireo_model *m, VireoKV *kv, int32_t *token, int pos, int32_t *pos_dev, int want_logits,
               float *x, float *logits, void *state, hipStream_t s) {
    const Bufs b = carve(m, state);
    const int d = m->dim, hs = m->head_size, nh = m->n_heads, nkh = m->n_kv_heads;
    const int nq = nh * hs, nk = nkh * hs;
    const float eps = m->eps;

    // a contiguous store with rows of the head size takes the device-position
    // appends inside head_prologue_kernel
    KvContigView view{};
    const bool append_in_place = pos_dev && vh_kv_contig_view(kv, &view) == 0 && view.d == hs;

    int rc = vireo_embed(m->tok_embd->ggml_type, m->tok_embd->data, d, m->vocab, token, 1, x, s);
    for (int l = 0; l < m->n_layers && !rc; l++) {
        const vireo_block &B = m->blocks[l];
        bool appended = false;
        // attention (src/gguf_run.c:221-237): the RMSNorm and q, k and v in
        // one launch where the types allow, else the norm, then q, k and v in
        // one launch, else one per matrix
        rc = vh_qmatvec3_normed(x, B.attn_norm, eps, d, b.q, B.wq, nq, b.k, B.wk, nk, b.v, B.wv, nk, s);
        if (rc == -ENOTSUP) {
            rc = vireo_rmsnorm(b.xb, x, B.attn_norm, d, 1, eps, s);
            if (!rc) rc = vh_qmatvec3(b.xb, d, b.q, B.wq, nq, b.k, B.wk, nk, b.v, B.wv, nk, s);
            if (rc == -ENOTSUP) {
                rc = qmatvec_async(b.q, b.xb, B.wq, d, nq, s);
                if (!rc) rc = qmatvec_async(b.k, b.xb, B.wk, d, nk, s);
                if (!rc) rc = qmatvec_async(b.v, b.xb, B.wv, d, nk, s);
            }
        }
        if (!rc && hs % 64 == 0 && hs <= 256 && (!B.q_norm || B.q_norm_len == hs) &&
            (!B.k_norm || B.k_norm_len == hs)) {
            // per-head QK-norms (or none): biases, norms and RoPE in one launch,
            // which also appends to a contiguous store at a device position
            appended = append_in_place && (l + 1) * nkh <= view.layers;
            const unsigned heads = unsigned(nh + nkh + (B.bv || appended ? nkh : 0));
            hipLaunchKernelGGL(head_prologue_kernel, dim3(heads), dim3(64), 0, s, HeadJob{b.q, B.bq, B.q_norm, nh},
                               HeadJob{b.k, B.bk, B.k_norm, nkh}, HeadJob{b.v, B.bv, nullptr, nkh}, hs, eps, m->rope,
                               pos, pos_dev, m->max_pos, appended ? view : KvContigView{}, l * nkh);
            rc = vh_check(hipGetLastError());
        } else if (!rc) {
            // a norm over the whole q or k vector: separate launches
            if (B.bq || B.bk || B.bv)
                rc = add3(AddJob{b.q, B.bq, nq}, AddJob{b.k, B.bk, nk}, AddJob{b.v, B.bv, nk}, s);
            if (!rc && B.q_norm)
                rc = B.q_norm_len == hs ? vireo_rmsnorm(b.q, b.q, B.q_norm, hs, nh, eps, s)
                                        : vireo_rmsnorm(b.q, b.q, B.q_norm, nq, 1, eps, s);
            if (!rc && B.k_norm)
                rc = B.k_norm_len == hs ? vireo_rmsnorm(b.k, b.k, B.k_norm, hs, nkh, eps, s)
                                        : vireo_rmsnorm(b.k, b.k, B.k_norm, nk, 1, eps, s);
            if (!rc) {
                const int pairs = (nh + nkh) * (hs / 2);
                hipLaunchKernelGGL(rope_kernel, dim3((pairs + 255) / 256), dim3(256), 0, s, b.q, nh, b.k, nkh, hs,
                                   m->rope, pos, pos_dev, m->max_pos);
                rc = vh_check(hipGetLastError());
            }
        }
        if (!rc && !appended)
            rc = pos_dev ? vireo_kv_append_pos(kv, l * nkh, nkh, pos_dev, b.k, b.v, s)
                         : vireo_kv_append_n(kv, l * nkh, nkh, pos, b.k, b.v, s);
        if (!rc) rc = pos_dev ? vireo_kv_attend_gqa_pos(kv, l * nkh, nh, nkh, pos_dev, b.q, b.att, s)
                              : vireo_kv_attend_gqa(kv, l * nkh, nh, nkh, b.q, b.att, s);
        if (!rc) rc = vh_qmatvec_acc(x, b.att, B.wo, nq, d, s);  // x += wo att
        // FFN (src/gguf_run.c:238-249)
        if (rc) break;
        if (m->moe) {
            rc = vh_moe_layer_normed(m->moe, l, x, B.ffn_norm, eps, b.xb, s);
        } else {
            const int f = m->ffn;
            rc = vireo_rmsnorm(b.xb, x, B.ffn_norm, d, 1, eps, s);
            if (!rc) rc = qmatvec_async(b.h1, b.xb, B.wg, d, f, s);
            if (!rc) rc = qmatvec_async(b.h2, b.xb, B.wu, d, f, s);
            if (!rc) {
                hipLaunchKernelGGL(swiglu_kernel, dim3((f + 255) / 256), dim3(256), 0, s, b.h1, b.h2, f);
                rc = vh_check(hipGetLastError());
            }
            if (!rc) rc = vh_qmatvec_acc(x, b.h1, B.wd, f, d, s);  // x += wd h
        }
    }
    if (want_logits && !rc) {  // src/gguf_run.c:251-252, argmax :254
        rc = vireo_rmsnorm(b.xb, x, m->out_norm, d, 1, eps, s);
        if (!rc) rc = qmatvec_async(logits, b.xb, m->lm_head, d, m->vocab, s);
        if (!rc) rc = vireo_argmax(logits, m->vocab, token, s);
    }
    return rc;
}

}  // namespace

extern "C" int vireo_model_step(const vireo_model *m, VireoKV *kv, int32_t *token, int pos, int want_logits,
                                float *x, float *logits, void *state, void *stream) {
    if (int rc = check_model(m)) return rc;
    if (!kv || !token || !x || !state || (want_logits && (!logits || !m->lm_head)) || pos < 0 || pos >= m->max_pos)
        return -EINVAL;
    if (reinterpret_cast<uintptr_t>(state) & 255u) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = vh_finish(s, model_step(m, kv, token, pos, nullptr, want_logits, x, logits, state, s));
    if (!rc && !s && vh_plan_waits()) rc = vh_take_status(nullptr);  // a grid-wide wait that gave up
    return rc;
}

extern "C" int vireo_model_step_pos(const vireo_model *m, VireoKV *kv, int32_t *token, int32_t *pos,
                                    int want_logits, float *x, float *logits, void *state, void *stream) {
    if (int rc = check_model(m)) return rc;
    if (!kv || !token || !pos || !x || !state || (want_logits && (!logits || !m->lm_head))) return -EINVAL;
    if (reinterpret_cast<uintptr_t>(state) & 255u) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = model_step(m, kv, token, 0, pos, want_logits, x, logits, state, s);
    if (!rc) {
        hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, pos);
        rc = vh_check(hipGetLastError());
    }
    rc = vh_finish(s, rc);
    if (!rc && !s && vh_plan_waits()) rc = vh_take_status(nullptr);  // a grid-wide wait that gave up
    return rc;
}
