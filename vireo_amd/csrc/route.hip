// Routing kernels: router logits for n tokens, then the per-token top-k.
//
// Two ways to get the logits the reference would compute (src/gguf_run.c:187,
// an in-order fp32 sum per expert, src/gguf_compute.c:202-207):
//   route_parts_kernel  one wave per (expert, token): fp64 sum of the rounded
//                       products plus a bound on the reference's rounding; the
//                       top-k step certifies the ranking or recomputes the
//                       contenders exactly. Short latency: used for decode.
//   route_exact_kernel  every (token, expert) logit by the reference's own
//                       sequential fp32 recurrence. One chain is 2*d dependent
//                       operations, but a 64-token x 16-expert tile keeps 1024
//                       chains in flight per workgroup, so with many tokens the
//                       dependency is hidden and the result is exact: used for
//                       prefill.
#include <hip/hip_runtime.h>
#include "common.h"
#include "route.h"
#include "route_kernels.h"

namespace {

template <int C>
__global__ void __launch_bounds__(64) route_parts_kernel(const float *__restrict__ R, const float *__restrict__ hb,
                                                         const float *__restrict__ bias, int d, int E,
                                                         RoutePart *__restrict__ parts, uint32_t *__restrict__ zero,
                                                         int nzero) {
    const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int gid = (blockIdx.y * gridDim.x + blockIdx.x) * 64 + lane;
    if (gid < nzero) zero[gid] = 0u;
    RoutePart p = route_row_part<C>(R + size_t(e) * d, hb + size_t(t) * d, d, lane);
    if (lane == 0) {
        if (bias) p.c += double(bias[e]);
        parts[size_t(t) * E + e] = p;
    }
}

constexpr int kExTok = 64, kExExp = 16, kExChunk = 64;

// grid (ceil(T/64), ceil(E/16)), 256 threads: thread (token tid%64, experts
// 4*(tid/64) .. +3 of the tile). Router and token chunks go through LDS.
__global__ void __launch_bounds__(256) route_exact_kernel(const float *__restrict__ R, const float *__restrict__ hb,
                                                          const float *__restrict__ bias, int d, int E, int T,
                                                          RoutePart *__restrict__ parts) {
    __shared__ float xs[kExTok][kExChunk + 1];
    __shared__ float rs[kExExp][kExChunk];
    const int tid = threadIdx.x, tl = tid & 63, g = tid >> 6;
    const int t0 = blockIdx.x * kExTok, e0 = blockIdx.y * kExExp;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < d; c0 += kExChunk) {
        const int cn = min(kExChunk, d - c0);
        for (int i = tid; i < kExTok * kExChunk; i += 256) {
            const int tt = i / kExChunk, cc = i % kExChunk;
            xs[tt][cc] = (t0 + tt < T && cc < cn) ? hb[size_t(t0 + tt) * d + c0 + cc] : 0.0f;
        }
        for (int i = tid; i < kExExp * kExChunk; i += 256) {
            const int ee = i / kExChunk, cc = i % kExChunk;
            rs[ee][cc] = (e0 + ee < E && cc < cn) ? R[size_t(e0 + ee) * d + c0 + cc] : 0.0f;
        }
        __syncthreads();
        for (int i = 0; i < cn; i++) {
            const float xv = xs[tl][i];
#pragma unroll
            for (int q = 0; q < 4; q++) acc[q] = __fadd_rn(acc[q], __fmul_rn(rs[4 * g + q][i], xv));
        }
        __syncthreads();
    }
    const int t = t0 + tl;
    if (t < T) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = e0 + 4 * g + q;
            if (e < E) {
                float a = acc[q];
                if (bias) a = __fadd_rn(a, bias[e]);
                RoutePart p;
                p.c = double(a);
                p.beta = 0.0;
                parts[size_t(t) * E + e] = p;
            }
        }
    }
}

// one 256-thread workgroup per token
__global__ void __launch_bounds__(256) route_finish_kernel(const RoutePart *__restrict__ parts,
                                                           const float *__restrict__ R, const float *__restrict__ hb,
                                                           const float *__restrict__ bias, int d, int E, int k,
                                                           int renorm, int exact, int32_t *__restrict__ idx,
                                                           float *__restrict__ w, uint32_t *__restrict__ flags,
                                                           float *__restrict__ probs) {
    __shared__ TopKSmem sm;
    const int t = blockIdx.x, tid = threadIdx.x;
    route_topk_block(sm, parts + size_t(t) * E, R, hb + size_t(t) * d, bias, d, E, k, renorm, exact != 0,
                     probs ? probs + size_t(t) * E : nullptr);
    if (tid < k) {
        idx[size_t(t) * k + tid] = sm.sel[tid];
        w[size_t(t) * k + tid] = sm.sel_w[tid];
    }
    if (tid == 0 && flags) flags[t] = sm.flag;
}

}  // namespace

int vh_route_parts(const float *R, const float *hb, const float *bias, int d, int E, int T, bool exact,
                   RoutePart *parts, hipStream_t s, uint32_t *zero, int nzero) {
    if (nzero > E * T * 64) return -EINVAL;
    if (exact) {
        if (nzero) return -EINVAL;
        dim3 g((T + kExTok - 1) / kExTok, (E + kExExp - 1) / kExExp);
        hipLaunchKernelGGL(route_exact_kernel, g, dim3(256), 0, s, R, hb, bias, d, E, T, parts);
    } else {
        const bool fast = d == 2048 && (reinterpret_cast<uintptr_t>(R) & 15u) == 0 &&
                          (reinterpret_cast<uintptr_t>(hb) & 15u) == 0;
        dim3 g(E, T);
        if (fast) VH_LAUNCH(route_parts_kernel<32>, g, dim3(64), 0, s, R, hb, bias, d, E, parts, zero, nzero);
        else VH_LAUNCH(route_parts_kernel<0>, g, dim3(64), 0, s, R, hb, bias, d, E, parts, zero, nzero);
    }
    return vh_check(hipGetLastError());
}

int vh_route_finish(const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E, int k,
                    int renorm, bool exact, int T, int32_t *idx, float *w, uint32_t *flags, float *probs,
                    hipStream_t s) {
    hipLaunchKernelGGL(route_finish_kernel, dim3(T), dim3(256), 0, s, parts, R, hb, bias, d, E, k, renorm,
                       exact ? 1 : 0, idx, w, flags, probs);
    return vh_check(hipGetLastError());
}
