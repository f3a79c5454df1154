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
//                       operations, but a 64-token x 8-expert tile keeps 512
//                       chains in flight per workgroup, so with many tokens the
//                       dependency is hidden and the result is exact: used for
//                       prefill.
#include <hip/hip_runtime.h>
#include <type_traits>
#include "common.h"
#include "route.h"
#include "route_kernels.h"

namespace {

template <int C, bool ST>
__global__ void __launch_bounds__(64) route_parts_kernel(const float *__restrict__ R, const float *__restrict__ hb,
                                                         const float *__restrict__ bias, int d, int E,
                                                         RoutePart *__restrict__ parts, uint32_t *__restrict__ zero,
                                                         int nzero, uint64_t *__restrict__ stamps) {
    PhaseStamps<ST> ps(stamps);
    ps.now(0);
    const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int gid = (blockIdx.y * gridDim.x + blockIdx.x) * 64 + lane;
    if (gid < nzero) zero[gid] = 0u;
    RoutePart p = route_row_part<C>(R + size_t(e) * d, hb + size_t(t) * d, d, lane);
    ps.after(1, p.c);
    if (lane == 0) {
        if (bias) p.c += double(bias[e]);
        parts[size_t(t) * E + e] = p;
    }
    ps.store();
}

// route_parts_kernel on the RMSNorm of x (src/gguf_run.c:161-165) instead of a
// given hb: every wave reduces the sum of squares of its token's x in fp64
// (the same operations in every wave, so the same r), forms
// hb = (x * r) * w in registers and uses it for its row's part; the wave of
// expert 0 also writes hb for the later stages. d == 64 * C.
template <int C, bool ST>
__global__ void __launch_bounds__(64) route_parts_norm_kernel(const float *__restrict__ R, const float *__restrict__ x,
                                                              const float *__restrict__ nw, float eps,
                                                              float *__restrict__ hb_out, const float *__restrict__ bias,
                                                              int d, int E, RoutePart *__restrict__ parts,
                                                              uint32_t *__restrict__ zero, int nzero,
                                                              uint64_t *__restrict__ stamps) {
    PhaseStamps<ST> ps(stamps);
    ps.now(0);
    const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int gid = (blockIdx.y * gridDim.x + blockIdx.x) * 64 + lane;
    if (gid < nzero) zero[gid] = 0u;
    // every load first, together: this lane's x, its norm weights (without
    // them, x again, unused) and its router row piece; then the arithmetic
    float xv[C], wv[C], rv[C];
    const float4 *x4 = reinterpret_cast<const float4 *>(x + size_t(t) * d + lane * C);
    const float4 *w4 = reinterpret_cast<const float4 *>((nw ? nw : x + size_t(t) * d) + lane * C);
    const float4 *r4 = reinterpret_cast<const float4 *>(R + size_t(e) * d + lane * C);
#pragma unroll
    for (int i = 0; i < C / 4; i++) {
        const float4 v = x4[i], w = w4[i], a = r4[i];
        xv[4 * i + 0] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
        wv[4 * i + 0] = w.x;
        wv[4 * i + 1] = w.y;
        wv[4 * i + 2] = w.z;
        wv[4 * i + 3] = w.w;
        rv[4 * i + 0] = a.x;
        rv[4 * i + 1] = a.y;
        rv[4 * i + 2] = a.z;
        rv[4 * i + 3] = a.w;
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the arithmetic
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < C; i++) ss += double(mul_rn(xv[i], xv[i]));
    ss = wave_sum_d(ss);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(float(ss), float(d)), eps)));
#pragma unroll
    for (int i = 0; i < C; i++) xv[i] = nw ? mul_rn(mul_rn(xv[i], r), wv[i]) : mul_rn(xv[i], r);
    double abs_products;
    RoutePart p = route_row_part_vals<C>(rv, xv, lane, &abs_products);
    p = route_part_on_own_norm(p, abs_products, d, bias, e);  // certified against the reference's xb
    ps.after(1, p.c);
    if (lane == 0) parts[size_t(t) * E + e] = p;
    if (e == 0) {  // after the part: no wait in this wave counts these stores
        float4 *h4 = reinterpret_cast<float4 *>(hb_out + size_t(t) * d + lane * C);
#pragma unroll
        for (int i = 0; i < C / 4; i++) h4[i] = make_float4(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2], xv[4 * i + 3]);
    }
    ps.store();
}

constexpr int kExTok = 64, kExCpl = 2, kExExp = 4 * kExCpl;
constexpr int kExChunk = 64;  // columns per LDS chunk (128: 54.6 us against 53.9 below)

// grid (ceil(T/64), ceil(E/8)), 256 threads: lane = token t0 + lane, wave g
// = experts e0 + 2g, e0 + 2g + 1 (two independent in-order chains per lane;
// two workgroups per CU keep the dependent adds of more waves in flight).
// Each CH-column chunk of the tokens' inputs (token-major, xs[token][column],
// rows padded by 16 bytes so that a lane's 16-byte read of four columns and
// the staging writes are conflict-free) and of the 8 router rows (read four
// columns at a time, one address for the whole wave) goes through LDS; the
// next chunks are loaded into registers while the current one is summed.
// V4: 16-byte staging loads (d % 4 == 0, 16-byte aligned rows), each
// thread CH / 16 of the inputs and at most one of the router rows; else one
// float per load. Measured (2048 tokens x 128 experts, d = 2048): 70.0 us
// with column-major xs and one read per column, 58.6 token-major, 53.9 with
// 16-byte staging.
template <int CH, bool V4>
__global__ void __launch_bounds__(256) route_exact_kernel(const float *__restrict__ R, const float *__restrict__ hb,
                                                          const float *__restrict__ bias, int d, int E, int T,
                                                          RoutePart *__restrict__ parts) {
    static_assert(V4 || CH == 64, "one-float staging covers 64 columns");
    __shared__ __align__(16) float xs[kExTok][CH + 4];
    __shared__ float4 rs[kExExp][CH / 4];
    const int tid = threadIdx.x, tl = tid & 63, g = tid >> 6;
    const int t0 = blockIdx.x * kExTok, e0 = blockIdx.y * kExExp;
    // one-float staging: thread tid loads column tid & 63 of token rows
    // (tid >> 6) + 4j (j < 16) and of router rows (tid >> 6) + 4j (j < kExCpl);
    // 16-byte staging: piece tid % (CH / 4) of token rows tid / (CH / 4) +
    // (256 / (CH / 4)) j, and piece tid % (CH / 4) of router row tid / (CH / 4)
    // (threads below kExExp * CH / 4).
    constexpr int NX = V4 ? kExTok * CH / 4 / 256 : 16, NR = V4 ? 1 : kExCpl, PR = CH / 4;
    const int cc = V4 ? tid % PR : tid & 63, r0 = V4 ? tid / PR : tid >> 6;
    constexpr int RSTEP = V4 ? 256 / PR : 4;
    const bool rload = !V4 || tid < kExExp * PR;
    // two register sets, loaded two chunks ahead; every load unconditional
    // (rows and columns past the end repeat the last one, and their values are
    // never used), so the wait before a set's store counts only older loads
    typedef float vf4 __attribute__((ext_vector_type(4)));
    typedef typename std::conditional<V4, vf4, float>::type Item;
    Item xr2[2][NX], rr2[2][NR];
    auto load = [&](auto SET, int c0) {
        constexpr int set = decltype(SET)::value;
        if constexpr (V4) {
            const int c = min(c0 + 4 * cc, d - 4);
#pragma unroll
            for (int j = 0; j < NX; j++)
                xr2[set][j] = *reinterpret_cast<const vf4 *>(hb + size_t(min(t0 + r0 + RSTEP * j, T - 1)) * d + c);
            rr2[set][0] = *reinterpret_cast<const vf4 *>(R + size_t(min(e0 + (rload ? r0 : 0), E - 1)) * d + c);
        } else {
            const int c = min(c0 + cc, d - 1);
#pragma unroll
            for (int j = 0; j < NX; j++) xr2[set][j] = hb[size_t(min(t0 + r0 + 4 * j, T - 1)) * d + c];
#pragma unroll
            for (int j = 0; j < NR; j++) rr2[set][j] = R[size_t(min(e0 + r0 + 4 * j, E - 1)) * d + c];
        }
    };
    auto store = [&](auto SET) {
        constexpr int set = decltype(SET)::value;
        if constexpr (V4) {
#pragma unroll
            for (int j = 0; j < NX; j++) *reinterpret_cast<vf4 *>(&xs[r0 + RSTEP * j][4 * cc]) = xr2[set][j];
            if (rload) *reinterpret_cast<vf4 *>(&rs[r0][cc]) = rr2[set][0];
        } else {
#pragma unroll
            for (int j = 0; j < NX; j++) xs[r0 + 4 * j][cc] = xr2[set][j];
#pragma unroll
            for (int j = 0; j < NR; j++) reinterpret_cast<float *>(&rs[r0 + 4 * j][0])[cc] = rr2[set][j];
        }
    };
    float acc[kExCpl] = {};
    auto chunk = [&](auto SET, int c0) {
        store(SET);
        lds_barrier();  // LDS only: the loads in flight stay in flight
        load(SET, c0 + 2 * CH);
        if (d - c0 >= CH) {
            // operands of four columns, read one group ahead of their use
            float4 rn[kExCpl], xn;
#pragma unroll
            for (int q = 0; q < kExCpl; q++) rn[q] = rs[kExCpl * g + q][0];
            xn = *reinterpret_cast<const float4 *>(&xs[tl][0]);
#pragma unroll
            for (int i4 = 0; i4 < CH / 4; i4++) {
                float4 r[kExCpl];
#pragma unroll
                for (int q = 0; q < kExCpl; q++) r[q] = rn[q];
                const float4 x4 = xn;
                if (i4 + 1 < CH / 4) {
#pragma unroll
                    for (int q = 0; q < kExCpl; q++) rn[q] = rs[kExCpl * g + q][i4 + 1];
                    xn = *reinterpret_cast<const float4 *>(&xs[tl][4 * i4 + 4]);
                }
                // the four columns' products first, then the chains' adds in
                // column order: an add never waits for a product issued just
                // before it (the asm statement keeps the products ahead)
                float pr[4][kExCpl];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float xv = u == 0 ? x4.x : u == 1 ? x4.y : u == 2 ? x4.z : x4.w;
#pragma unroll
                    for (int q = 0; q < kExCpl; q++) {
                        const float rv = u == 0 ? r[q].x : u == 1 ? r[q].y : u == 2 ? r[q].z : r[q].w;
                        pr[u][q] = mul_rn(rv, xv);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int q = 0; q < kExCpl; q++) asm volatile("" : "+v"(pr[u][q]));
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int q = 0; q < kExCpl; q++) acc[q] = add_rn(acc[q], pr[u][q]);
                __builtin_amdgcn_sched_barrier(0);  // the next group's products stay behind these adds
            }
        } else {  // the last, partial chunk: only its d - c0 columns
            for (int i = 0; i < d - c0; i++) {
                const float xv = xs[tl][i];
#pragma unroll
                for (int q = 0; q < kExCpl; q++)
                    acc[q] = add_rn(acc[q], mul_rn(reinterpret_cast<const float *>(&rs[kExCpl * g + q][0])[i], xv));
            }
        }
        lds_barrier();
    };
    const std::integral_constant<int, 0> s0;
    const std::integral_constant<int, 1> s1;
    load(s0, 0);
    load(s1, CH);
    int c0 = 0;
    for (; c0 + CH < d; c0 += 2 * CH) {
        chunk(s0, c0);
        chunk(s1, c0 + CH);
    }
    if (c0 < d) chunk(s0, c0);
    const int t = t0 + tl;
    if (t < T) {
#pragma unroll
        for (int q = 0; q < kExCpl; q++) {
            const int e = e0 + kExCpl * g + q;
            if (e < E) {
                float a = acc[q];
                if (bias) a = add_rn(a, bias[e]);
                RoutePart p;
                p.c = double(a);
                p.beta = 0.0;
                parts[size_t(t) * E + e] = p;
            }
        }
    }
}

// One workgroup per token: 512 threads for certified parts (eight waves
// share an uncertified token's contenders), 256 for exact ones. Dynamic LDS
// (only where route_topk_block can stream the contenders' rows: d != 2048,
// parts not exact): the rows' buffers, then the token's inputs.
__global__ void __launch_bounds__(512) route_finish_kernel(const RoutePart *__restrict__ parts,
                                                           const float *__restrict__ R, const float *__restrict__ hb,
                                                           const float *__restrict__ bias, int d, int E, int k,
                                                           int renorm, int exact, int32_t *__restrict__ idx,
                                                           float *__restrict__ w, uint32_t *__restrict__ flags,
                                                           float *__restrict__ probs, int staged) {
    __shared__ TopKSmem sm;
    extern __shared__ float4 dyn[];
    float4 *stage = staged ? dyn : nullptr;                                            // the contenders' rows
    float *xbuf = staged ? reinterpret_cast<float *>(dyn + kStageScrF4) : nullptr;  // the token's inputs
    const int t = blockIdx.x, tid = threadIdx.x;
    route_topk_block(sm, parts + size_t(t) * E, R, hb + size_t(t) * d, bias, d, E, k, renorm, exact != 0,
                     probs ? probs + size_t(t) * E : nullptr, stage, xbuf);
    if (tid < k) {
        idx[size_t(t) * k + tid] = sm.sel[tid];
        w[size_t(t) * k + tid] = sm.sel_w[tid];
    }
    if (tid == 0 && flags) flags[t] = sm.flag;
}

// one 64-thread workgroup per (expert, token): the wave-split chain for
// d == 2048 with aligned rows, else lane 0's sequential chain
__global__ void __launch_bounds__(64) router_logits_kernel(const float *__restrict__ R, const float *__restrict__ hb,
                                                           int d, int E, float *__restrict__ out) {
    const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const float *r = R + size_t(e) * d, *x = hb + size_t(t) * d;
    float a;
    if (d == 2048 && ((reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0) {
        float xv[32];
        const float4 *x4 = reinterpret_cast<const float4 *>(x + lane * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = x4[i];
            xv[4 * i] = v.x;
            xv[4 * i + 1] = v.y;
            xv[4 * i + 2] = v.z;
            xv[4 * i + 3] = v.w;
        }
        a = exact_logit_wave(r, xv, lane);
    } else {
        a = lane == 0 ? exact_logit(r, x, d) : 0.0f;
    }
    if (lane == 0) out[size_t(t) * E + e] = a;
}

}  // namespace

extern "C" int vireo_router_logits(const float *R, const float *hb, int d, int E, int T, float *out, void *stream) {
    if (d <= 0 || E <= 0 || T < 0 || E > 65535 || T > 65535 || (T && (!R || !hb || !out))) return -EINVAL;
    if (T == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(router_logits_kernel, dim3(E, T), dim3(64), 0, s, R, hb, d, E, out);
    return vh_finish(s, vh_check(hipGetLastError()));
}

int vh_route_parts_norm(const float *R, const float *x, const float *nw, float eps, float *hb_out, const float *bias,
                        int d, int E, int T, RoutePart *parts, hipStream_t s, uint32_t *zero, int nzero) {
    if (d != 2048 || (reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(hb_out) & 15u) ||
        (reinterpret_cast<uintptr_t>(R) & 15u) || nzero > E * T * 64)
        return -EINVAL;
    if (uint64_t *st = vh_stamps_for(0))
        VH_LAUNCH((route_parts_norm_kernel<32, true>), dim3(E, T), dim3(64), 0, s, R, x, nw, eps, hb_out, bias, d, E,
                  parts, zero, nzero, st);
    else
        VH_LAUNCH((route_parts_norm_kernel<32, false>), dim3(E, T), dim3(64), 0, s, R, x, nw, eps, hb_out, bias, d, E,
                  parts, zero, nzero, nullptr);
    return vh_check(hipGetLastError());
}

int vh_route_parts(const float *R, const float *hb, const float *bias, int d, int E, int T, bool exact,
                   RoutePart *parts, hipStream_t s, uint32_t *zero, int nzero) {
    if (nzero > E * T * 64) return -EINVAL;
    if (!exact && T >= 8 && nzero == 0) {  // d == 2048: inputs shared by 4 x 4 tiles (fewer tokens: too few waves)
        const int rc = vh_route_parts_tiled(R, hb, bias, d, E, T, parts, nullptr, nullptr, s);
        if (rc != -EINVAL) return rc;
    }
    if (exact) {
        if (nzero) return -EINVAL;
        dim3 g((T + kExTok - 1) / kExTok, (E + kExExp - 1) / kExExp);
        const bool v4 = d % 4 == 0 && d >= 128 &&
                        ((reinterpret_cast<uintptr_t>(R) | reinterpret_cast<uintptr_t>(hb)) & 15u) == 0;
        if (v4)
            hipLaunchKernelGGL((route_exact_kernel<kExChunk, true>), g, dim3(256), 0, s, R, hb, bias, d, E, T, parts);
        else
            hipLaunchKernelGGL((route_exact_kernel<kExChunk, false>), g, dim3(256), 0, s, R, hb, bias, d, E, T, parts);
    } else {
        const bool fast = d == 2048 && (reinterpret_cast<uintptr_t>(R) & 15u) == 0 &&
                          (reinterpret_cast<uintptr_t>(hb) & 15u) == 0;
        dim3 g(E, T);
        uint64_t *st = vh_stamps_for(0);
        if (fast && st)  // the stamped build only where the phases are recorded (d == 2048)
            VH_LAUNCH((route_parts_kernel<32, true>), g, dim3(64), 0, s, R, hb, bias, d, E, parts, zero, nzero, st);
        else if (fast)
            VH_LAUNCH((route_parts_kernel<32, false>), g, dim3(64), 0, s, R, hb, bias, d, E, parts, zero, nzero, st);
        else
            VH_LAUNCH((route_parts_kernel<0, false>), g, dim3(64), 0, s, R, hb, bias, d, E, parts, zero, nzero, st);
    }
    return vh_check(hipGetLastError());
}

int vh_route_finish(const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E, int k,
                    int renorm, bool exact, int T, int32_t *idx, float *w, uint32_t *flags, float *probs,
                    hipStream_t s) {
    // a small LDS footprint where the rows are not streamed: prefill calls run thousands of these
    const bool staged = !exact && d != 2048 && d <= kXScrFloats;
    const size_t lds = staged ? size_t(kStageScrF4) * 16 + size_t(kXScrFloats) * 4 : 0;
    hipLaunchKernelGGL(route_finish_kernel, dim3(T), dim3(exact ? 256 : 512), lds, s, parts, R, hb, bias, d, E, k,
                       renorm, exact ? 1 : 0, idx, w, flags, probs, staged ? 1 : 0);
    return vh_check(hipGetLastError());
}
