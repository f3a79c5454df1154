// Routing device code shared by the routing kernels and the fused decode
// kernel: router logits (fast bounded fp64 sums, or exact in-order fp32 sums),
// and the top-k selection of one token by one 256-thread workgroup.
//
// Reference: moe_ffn computes logits with the F32 gguf_matmul, an in-order,
// uncontracted fp32 sum per expert (src/gguf_compute.c:202-207), softmaxes
// them (src/gguf_run.c:181-182), takes the top k probabilities with the lowest
// expert id winning ties (:189-191) and optionally renormalises (:192).
#pragma once
#include <math.h>
#include "common.h"
#include "vireo_hip.h"

// Per (token, expert): S = the fp64 sum of the fp32-rounded products r_i*x_i
// (plus the optional bias), beta = a rigorous bound on |s^ - S| where s^ is the
// reference's sequential fp32 sum. For recursive summation
//   |s^_n - S_n| <= (u/(1-u)) sum_{k>=2} |s^_k| <= 1.001 * u * sum_k |S_k|
// (u = 2^-24, n <= 2^17 so the second-order term is below 0.1%).
struct RoutePart {
    double c, beta;
};

constexpr double kRouteMargin = 2e-6;  // separation required beyond the bounds
constexpr float kNearTie = 1e-6f;      // exact-logit gap reported as an exception
constexpr int kMaxExperts = 256;

// One wave: router row r (d floats) against x. Lane l owns elements
// [l*C, l*C + C) so prefix sums follow element order. Returns the part on all lanes.
template <int C>
VH_DEV RoutePart route_row_part(const float *__restrict__ r, const float *__restrict__ x, int d, int lane) {
    double tot = 0.0, run, absum = 0.0;
    if constexpr (C > 0) {
        // fast path: d == 64*C, C a multiple of 4
        float p[C];
        const float4 *r4 = reinterpret_cast<const float4 *>(r + lane * C);
        const float4 *x4 = reinterpret_cast<const float4 *>(x + lane * C);
#pragma unroll
        for (int i = 0; i < C / 4; i++) {
            const float4 a = r4[i], b = x4[i];
            p[4 * i + 0] = __fmul_rn(a.x, b.x);
            p[4 * i + 1] = __fmul_rn(a.y, b.y);
            p[4 * i + 2] = __fmul_rn(a.z, b.z);
            p[4 * i + 3] = __fmul_rn(a.w, b.w);
        }
#pragma unroll
        for (int i = 0; i < C; i++) tot += double(p[i]);
        run = wave_incl_scan_d(tot) - tot;
#pragma unroll
        for (int i = 0; i < C; i++) {
            run += double(p[i]);
            absum += fabs(run);
        }
    } else {
        const int cpl = (d + 63) / 64, i0 = lane * cpl, i1 = min(d, i0 + cpl);
        for (int i = i0; i < i1; i++) tot += double(__fmul_rn(r[i], x[i]));
        run = wave_incl_scan_d(tot) - tot;
        for (int i = i0; i < i1; i++) {
            run += double(__fmul_rn(r[i], x[i]));
            absum += fabs(run);
        }
    }
    RoutePart out;
    out.c = wave_sum_d(tot);
    out.beta = 1.001 * 5.9604644775390625e-08 * wave_sum_d(absum) + 1e-30;
    return out;
}

// The reference logit exactly: a = 0; a += r[i]*x[i] for i in order, every
// product and sum rounded to fp32.
VH_DEV float exact_logit(const float *__restrict__ r, const float *__restrict__ x, int d) {
    float a = 0.0f;
    for (int i = 0; i < d; i++) a = __fadd_rn(a, __fmul_rn(r[i], x[i]));
    return a;
}

// Order-preserving 32-bit image of an fp32 value.
VH_DEV uint32_t ordered_u32(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Workspace of route_topk_block (LDS).
struct TopKSmem {
    uint32_t key[kMaxExperts];       // 32-bit rank keys
    uint64_t key64[kMaxExperts];     // full-precision keys (re-ranking)
    int sel[64];                     // chosen experts in order
    float sel_w[64];                 // their weights
    double sel_lo[65], sel_hi[64];   // their intervals; sel_lo[64]: best remaining
    float red[2][4];                 // per-wave partials
    float m;                         // max logit
    uint32_t flag;
    int uncertain;
};

// Top-k of one token by a 256-thread workgroup (all threads call it; E <= 256,
// k <= 64). Thread e owns expert e. Its rank is the number of experts with a
// larger key, so the k chosen experts and their order come out of one parallel
// pass. The ranking is certified with the fp64 intervals; when any gap that
// decides the set or its order is not wider than both bounds plus
// kRouteMargin, every expert that could still be among the k is recomputed
// exactly (in-order fp32, as the reference) and the experts are ranked again
// on full-precision keys. With exact_parts the parts already hold exact fp32
// logits (beta = 0) and only full-precision ranking and near-tie reporting
// are needed. On return (after a barrier) sm.sel / sm.sel_w / sm.flag hold the
// result; probs (optional, [E]) receives the softmax.
VH_DEV void route_topk_block(TopKSmem &sm, const RoutePart *__restrict__ part, const float *__restrict__ R,
                             const float *__restrict__ x, const float *__restrict__ bias, int d, int E, int k,
                             int renorm, bool exact_parts, float *__restrict__ probs) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool mine = tid < E;
    double lo = -INFINITY, hi = -INFINITY;
    float lg = -INFINITY;
    if (mine) {
        const RoutePart p = part[tid];
        lo = p.c - p.beta;
        hi = p.c + p.beta;
        lg = float(p.c);
    }
    // 8 mantissa bits give way to the id (lowest id wins a tie of the truncated
    // keys): values that close can never be certified, so a wrong truncated
    // order always reaches the full-precision re-ranking below.
    const uint32_t key = mine ? ((ordered_u32(lg) & 0xffffff00u) | uint32_t(255 - tid)) : 0u;
    sm.key[tid] = key;
    if (tid == 0) { sm.uncertain = 0; sm.flag = 0; }
    __syncthreads();
    int rank = 1 << 30;
    if (mine) {
        const uint4 *k4 = reinterpret_cast<const uint4 *>(sm.key);
        int r = 0;
        for (int j = 0; j < (E + 3) / 4; j++) {
            const uint4 v = k4[j];
            r += int(v.x > key) + int(v.y > key) + int(v.z > key) + int(v.w > key);
        }
        rank = r;
        if (rank < k) { sm.sel[rank] = tid; sm.sel_lo[rank] = lo; sm.sel_hi[rank] = hi; }
        if (rank == 0) sm.m = lg;
    }
    // the largest upper bound outside the chosen k, rounded up to fp32 (an
    // upper bound is all the certification needs)
    const float rest = (mine && rank >= k) ? __double2float_ru(hi) : -INFINITY;
    const float rw = wave_max_f(rest);
    if (lane == 0) sm.red[0][wv] = rw;
    __syncthreads();
    if (tid < k) {
        const float rh = fmaxf(fmaxf(sm.red[0][0], sm.red[0][1]), fmaxf(sm.red[0][2], sm.red[0][3]));
        const double next_hi = tid + 1 < k ? sm.sel_hi[tid + 1] : (k < E ? double(rh) : -INFINITY);
        if (!(sm.sel_lo[tid] - next_hi > (exact_parts ? 0.0 : kRouteMargin))) atomicOr(&sm.uncertain, 1);
        if (exact_parts && sm.sel_lo[tid] - next_hi < double(kNearTie)) atomicOr(&sm.flag, VIREO_ROUTE_NEAR_TIE);
    }
    __syncthreads();
    if (sm.uncertain) {
        // exact logits for every possible member of the top k
        double thr = INFINITY;
        for (int t = 0; t < k; t++) thr = fmin(thr, sm.sel_lo[t]);
        thr -= kRouteMargin;
        const bool cand = mine && hi >= thr;
        if (cand && !exact_parts) {
            float a = exact_logit(R + size_t(tid) * d, x, d);
            if (bias) a = __fadd_rn(a, bias[tid]);
            lg = a;
        }
        sm.key64[tid] = cand ? ((uint64_t(ordered_u32(lg)) << 8) | uint64_t(255 - tid)) : 0ull;
        if (tid == 0) {
            // the near-tie verdict is taken again on the full-precision ranking
            sm.flag = exact_parts ? 0u : VIREO_ROUTE_EXACT_FALLBACK;
            sm.sel_lo[64] = -INFINITY;
        }
        __syncthreads();
        rank = 1 << 30;
        if (cand) {
            const uint64_t k64 = sm.key64[tid];
            int r = 0;
            for (int j = 0; j < E; j++) r += int(sm.key64[j] > k64);
            rank = r;
            if (rank < k) { sm.sel[rank] = tid; sm.sel_lo[rank] = double(lg); }
            if (rank == k) sm.sel_lo[64] = double(lg);  // best contender left out
            if (rank == 0) sm.m = lg;
        }
        __syncthreads();
        if (tid < k) {
            const double nxt = tid + 1 < k ? sm.sel_lo[tid + 1] : sm.sel_lo[64];
            if (sm.sel_lo[tid] - nxt < double(kNearTie)) atomicOr(&sm.flag, VIREO_ROUTE_NEAR_TIE);
        }
        __syncthreads();
    }
    // softmax over all experts (src/gguf_run.c:181-182)
    const float ex = mine ? expf(lg - sm.m) : 0.0f;
    const float part_sum = wave_sum_f(ex);
    if (lane == 0) sm.red[1][wv] = part_sum;
    __syncthreads();
    const float s = (sm.red[1][0] + sm.red[1][1]) + (sm.red[1][2] + sm.red[1][3]);
    if (mine) {
        if (probs) probs[tid] = ex / s;
        if (rank < k) sm.sel_w[rank] = ex / s;
    }
    __syncthreads();
    if (tid == 0 && renorm) {
        float wsum = 0.0f;
        for (int t = 0; t < k; t++) wsum += sm.sel_w[t];  // in selection order
        if (wsum > 0.0f)
            for (int t = 0; t < k; t++) sm.sel_w[t] = sm.sel_w[t] / wsum;
    }
    __syncthreads();
}
