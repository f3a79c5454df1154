// Model glue around the MoE layers: rmsnorm (src/gguf_run.c:161-165), argmax
// (src/gguf_run.c:254), the embedding lookup (src/gguf_run.c:218) and the
// decode step of an MoE stack (src/gguf_run.c:216-251 without attention).
#include <hip/hip_runtime.h>
#include "common.h"
#include "route.h"
#include "route_kernels.h"
#include "qdecode.h"
#include "route_kernels.h"
#include "vireo_hip.h"

namespace {

// One workgroup per row. The sum of squares is reduced in fp64 and rounded
// once, so it is the correctly rounded value of the exact sum; the reference
// adds in fp32 sequentially, which is within n*2^-24 relative of it.
__global__ void __launch_bounds__(256) rmsnorm_kernel(float *o, const float *x,
                                                      const float *__restrict__ w, int n, float eps) {
    __shared__ double part[4];
    const size_t row = blockIdx.x;
    const float *xr = x + row * n;
    float *orow = o + row * n;
    double acc = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        acc += double(mul_rn(v, v));
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float ss = float((part[0] + part[1]) + (part[2] + part[3]));
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(ss, float(n)), eps)));
    // w == nullptr: unit weight (x * r * 1.0f is x * r)
    for (int i = threadIdx.x; i < n; i += 256) orow[i] = w ? mul_rn(mul_rn(xr[i], r), w[i]) : mul_rn(xr[i], r);
}

// argmax in two launches: workgroup g of argmax_part_kernel reduces the
// chunk [g * chunk, (g + 1) * chunk) to its first maximum (value, index);
// argmax_final_kernel reduces the partials in chunk order. A later index
// replaces the running best only when strictly greater, an earlier one also
// when equal, so the result is the first index of the maximum, as the
// reference's upward scan with a strict '>' from v[0] (src/gguf_run.c:254).
struct ArgBest {
    float v;
    int i;
};
VH_DEV void arg_merge(float &bv, int &bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}
VH_DEV void arg_block(float &bv, int &bi, float (&sv)[4], int (&si)[4]) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) arg_merge(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int w = 1; w < 4; w++) arg_merge(bv, bi, sv[w], si[w]);
}

__global__ void __launch_bounds__(256) argmax_part_kernel(const float *__restrict__ v, int n, int chunk,
                                                          ArgBest *__restrict__ part) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int lo = blockIdx.x * chunk, hi = min(n, lo + chunk);
    float bv = v[lo];
    int bi = lo;
#pragma unroll 4
    for (int i = lo + threadIdx.x; i < hi; i += 256) arg_merge(bv, bi, v[i], i);
    arg_block(bv, bi, sv, si);
    if (threadIdx.x == 0) part[blockIdx.x] = ArgBest{bv, bi};
}

__global__ void __launch_bounds__(256) argmax_final_kernel(const ArgBest *__restrict__ part, int np,
                                                           int32_t *__restrict__ out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float bv = part[0].v;
    int bi = part[0].i;
    for (int g = threadIdx.x; g < np; g += 256) arg_merge(bv, bi, part[g].v, part[g].i);
    arg_block(bv, bi, sv, si);
    if (threadIdx.x == 0) *out = bi;
}

// dst[i] = gguf_dequant_row(table row tokens[i]) for i < count, one
// workgroup per row (Q8_0: thread j of 256 writes elements j, j + 256, ...;
// the block scale of element c is that of block c / 32). A token outside
// [0, n_rows) gives a zero row.
template <int T>
__global__ void __launch_bounds__(256) embed_kernel(const uint8_t *__restrict__ table, int64_t row_bytes, int n,
                                                    int n_rows, const int32_t *__restrict__ tokens,
                                                    float *__restrict__ dst) {
    const int tok = tokens[blockIdx.x];
    float *o = dst + size_t(blockIdx.x) * n;
    if (tok < 0 || tok >= n_rows) {
        for (int c = threadIdx.x; c < n; c += 256) o[c] = 0.0f;
        return;
    }
    const uint8_t *r = table + int64_t(tok) * row_bytes;
    for (int c = threadIdx.x; c < n; c += 256) {
        if constexpr (T == VT_Q8_0) {  // src/gguf_compute.c:112-120: qs * d, exact
            const uint8_t *b = r + 34 * (c >> 5);
            o[c] = mul_rn(float(int8_t(ld_u8(b + 2 + (c & 31)))), h2f(ld_u16(b)));
        } else if constexpr (T == VT_F16) {
            o[c] = h2f(ld_u16(r + 2 * c));
        } else {
            o[c] = reinterpret_cast<const float *>(r)[c];
        }
    }
}

}  // namespace

extern "C" int vireo_embed(uint32_t type, const void *table, int n, int n_rows, const int32_t *tokens, int count,
                           float *dst, void *stream) {
    if (n <= 0 || n_rows <= 0 || count < 0 || (count && (!table || !tokens || !dst))) return -EINVAL;
    if ((type == VT_Q8_0 && n % 32) || (type != VT_Q8_0 && type != VT_F16 && type != VT_F32)) return -EINVAL;
    if (reinterpret_cast<uintptr_t>(table) & 3u) return -EINVAL;
    if (count == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *t = static_cast<const uint8_t *>(table);
    const int64_t rb = vh_row_bytes(type, n);
    switch (type) {
    case VT_Q8_0: hipLaunchKernelGGL(embed_kernel<VT_Q8_0>, dim3(count), dim3(256), 0, s, t, rb, n, n_rows, tokens, dst); break;
    case VT_F16: hipLaunchKernelGGL(embed_kernel<VT_F16>, dim3(count), dim3(256), 0, s, t, rb, n, n_rows, tokens, dst); break;
    default: hipLaunchKernelGGL(embed_kernel<VT_F32>, dim3(count), dim3(256), 0, s, t, rb, n, n_rows, tokens, dst); break;
    }
    return vh_finish(s, vh_check(hipGetLastError()));
}

namespace {
int stack_step(const vireo_moe_stack *st, int32_t *token, float *x, float *xb, float *logits, int32_t *idx,
               uint32_t *flags, void *stream) {
    if (!st || !st->moe || !st->lm_head || !token || !x || !xb || !logits || st->vocab <= 0) return -EINVAL;
    const vireo_moe_model *m = st->moe;
    const int d = m->dim;
    void *s = stream;
    const gguf_tensor *emb = st->tok_embd ? st->tok_embd : st->lm_head;
    int rc = vireo_embed(emb->ggml_type, emb->data, d, st->vocab, token, 1, x, s);
    for (int l = 0; l < m->n_layers && !rc; l++)
        rc = vh_moe_layer_normed(m, l, x, st->ffn_norm ? st->ffn_norm[l] : nullptr, st->eps, xb,
                                 static_cast<hipStream_t>(s), idx ? idx + size_t(l) * m->n_used : nullptr,
                                 flags ? flags + l : nullptr);
    if (!rc) rc = vireo_rmsnorm(xb, x, st->out_norm, d, 1, st->eps, s);
    if (!rc) rc = qmatvec_async(logits, xb, st->lm_head, d, st->vocab, s);
    if (!rc) rc = vireo_argmax(logits, st->vocab, token, s);
    rc = vh_finish(static_cast<hipStream_t>(s), rc);
    if (!rc && !s && vh_plan_waits()) rc = vh_take_status(nullptr);  // a grid-wide wait that gave up
    return rc;
}
}  // namespace

extern "C" int moe_stack_step(const vireo_moe_stack *st, int32_t *token, float *x, float *xb, float *logits,
                              void *stream) {
    return stack_step(st, token, x, xb, logits, nullptr, nullptr, stream);
}

extern "C" int moe_stack_step_trace(const vireo_moe_stack *st, int32_t *token, float *x, float *xb, float *logits,
                                    int32_t *idx, uint32_t *flags, void *stream) {
    if (!idx || !flags) return -EINVAL;
    return stack_step(st, token, x, xb, logits, idx, flags, stream);
}

// One row of the reference's RMSNorm, bit for bit (its in-order fp32 sum of
// squares: one thread adds them from LDS, the rest of the row is parallel).
constexpr int kRmsRefMaxLds = 16384;  // floats of squares kept in LDS (longer rows use the output row)
__global__ void __launch_bounds__(256) rmsnorm_ref_kernel(float *__restrict__ o, const float *__restrict__ x,
                                                          const float *__restrict__ w, int n, float eps) {
    extern __shared__ float4 sq4[];
    __shared__ float red;
    reference_rmsnorm_block(o, x, w, eps, n, &red, n <= kRmsRefMaxLds ? reinterpret_cast<float *>(sq4) : nullptr);
}

int vh_rmsnorm_ref(float *o, const float *x, const float *w, int n, float eps, hipStream_t s) {
    if (n <= 0 || !o || !x || o == x) return -EINVAL;
    const size_t lds = n <= kRmsRefMaxLds ? size_t(n + 3) / 4 * 16 : 0;
    hipLaunchKernelGGL(rmsnorm_ref_kernel, dim3(1), dim3(256), lds, s, o, x, w, n, eps);
    return vh_check(hipGetLastError());
}

extern "C" int vireo_rmsnorm_exact(float *o, const float *x, const float *w, int n, float eps, void *stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    return vh_finish(s, vh_rmsnorm_ref(o, x, w, n, eps, s));
}

extern "C" int vireo_rmsnorm(float *o, const float *x, const float *w, int n, int rows, float eps, void *stream) {
    if (n <= 0 || rows < 0 || (rows && (!o || !x))) return -EINVAL;
    if (rows == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, o, x, w, n, eps);
    return vh_finish(s, vh_check(hipGetLastError()));
}

extern "C" int vireo_argmax(const float *v, int n, int32_t *out, void *stream) {
    if (n <= 0 || !v || !out) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // about 1 K values per workgroup (four loads per thread in flight), at most 1 024 workgroups
    int np = (n + 1023) / 1024;
    if (np > 1024) np = 1024;
    const int chunk = (n + np - 1) / np;
    np = (n + chunk - 1) / chunk;
    void *part;
    if (int rc = vh_reduce_scratch(sizeof(ArgBest) * size_t(np), &part)) return rc;
    ArgBest *p = static_cast<ArgBest *>(part);
    hipLaunchKernelGGL(argmax_part_kernel, dim3(np), dim3(256), 0, s, v, n, chunk, p);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, p, np, out);
    return vh_finish(s, vh_check(hipGetLastError()));
}
