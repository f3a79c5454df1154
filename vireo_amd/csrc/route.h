// Routing device code shared by the routing kernels and the fused decode
// kernel: router logits (fast bounded fp64 sums, or exact in-order fp32 sums),
// and the top-k selection of one token by one wave.
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

VH_DEV double wave_excl_scan_d(double v, int lane) {
    double incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    return incl - v;
}

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
        run = wave_excl_scan_d(tot, lane);
#pragma unroll
        for (int i = 0; i < C; i++) {
            run += double(p[i]);
            absum += fabs(run);
        }
    } else {
        const int cpl = (d + 63) / 64, i0 = lane * cpl, i1 = min(d, i0 + cpl);
        for (int i = i0; i < i1; i++) tot += double(__fmul_rn(r[i], x[i]));
        run = wave_excl_scan_d(tot, lane);
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

// max of (value, id) with the lowest id first among equal values
VH_DEV void wave_argmax_d(double &v, int &i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const double ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
}
VH_DEV void wave_argmax_f(float &v, int &i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
}
VH_DEV double wave_max_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
    return v;
}
VH_DEV float wave_max_f(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
VH_DEV double wave_min_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmin(v, __shfl_xor(v, off, 64));
    return v;
}

struct TopK {
    int sel;       // on lane t < k: the t-th chosen expert
    float w;       // on lane t < k: its weight (renormalised if asked)
    uint32_t flag; // VIREO_ROUTE_* bits (uniform)
};

// Order-preserving 32-bit key of an fp32 value with the expert id packed in
// the low 8 bits (lowest id wins a tie). Dropping 8 mantissa bits only matters
// for values within 2^-15 relative of each other, and such pairs can never pass
// the certification (their intervals overlap), so they always reach the exact
// fallback, which ranks without truncation.
VH_DEV uint32_t rank_key(float v, int e) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (b & 0xffffff00u) | uint32_t(255 - e);
}

// Top-k of one token by one wave (all 64 lanes active, E <= 256).
// part: the token's E route parts. R, x, bias: for the exact fallback.
// When every gap that decides the chosen set and its order is wider than both
// bounds plus kRouteMargin, ranking by S is certainly the reference's ranking;
// otherwise every expert that could still be among the k is recomputed
// exactly and the ranking uses those logits. With exact_parts the parts already
// hold the exact fp32 logits (beta = 0): the ranking is taken as is and only
// near ties are reported. probs (optional, [E]) receives the softmax.
VH_DEV TopK route_topk(const RoutePart *__restrict__ part, const float *__restrict__ R,
                       const float *__restrict__ x, const float *__restrict__ bias, int d, int E, int k, int renorm,
                       bool exact_parts, float *__restrict__ probs) {
    const int lane = threadIdx.x & 63;
    double lo[4], hi[4];
    float lg[4];
    uint32_t key[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        if (e < E) {
            const RoutePart p = part[e];
            lo[j] = p.c - p.beta;
            hi[j] = p.c + p.beta;
            lg[j] = float(p.c);
            key[j] = rank_key(lg[j], e);
        } else {
            lo[j] = hi[j] = -INFINITY;
            lg[j] = -INFINITY;
            key[j] = 0u;
        }
    }
    int my_sel = -1;
    double my_lo = INFINITY, prev_lo = 0.0, min_gap = INFINITY;
    bool certain = true;
    for (int t = 0; t < k; t++) {
        const uint32_t best = wave_max_u(max(max(key[0], key[1]), max(key[2], key[3])));
        const int e = 255 - int(best & 0xffu), owner = e & 63, slot = e >> 6;
        double wl = slot == 0 ? lo[0] : slot == 1 ? lo[1] : slot == 2 ? lo[2] : lo[3];
        double wh = slot == 0 ? hi[0] : slot == 1 ? hi[1] : slot == 2 ? hi[2] : hi[3];
        wl = readlane_d(wl, owner);
        wh = readlane_d(wh, owner);
        if (lane == owner) key[slot] = 0u;  // taken
        if (t > 0) {
            if (!(prev_lo - wh > kRouteMargin)) certain = false;
            min_gap = fmin(min_gap, prev_lo - wh);
        }
        prev_lo = wl;
        if (lane == t) { my_sel = e; my_lo = wl; }
    }
    double rest_hi = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (key[j] != 0u) rest_hi = fmax(rest_hi, hi[j]);
    rest_hi = wave_max_d(rest_hi);
    if (k < E) {
        if (!(prev_lo - rest_hi > kRouteMargin)) certain = false;
        min_gap = fmin(min_gap, prev_lo - rest_hi);
    }
    uint32_t flag = 0;
    if (exact_parts) {
        // exact logits (beta = 0): a truncated-key tie can misorder two values
        // closer than 2^-15 relative; those are near ties and are re-ranked below
        if (min_gap < double(kNearTie)) flag |= VIREO_ROUTE_NEAR_TIE;
        certain = min_gap > 0.0 || k == 0;
    }
    if (!certain) {
        if (!exact_parts) flag |= VIREO_ROUTE_EXACT_FALLBACK;
        const double thr = wave_min_d(my_lo) - kRouteMargin;  // lowest lower bound among the k
        bool cand[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            cand[j] = e < E && hi[j] >= thr;
            if (cand[j] && !exact_parts) {
                float a = exact_logit(R + size_t(e) * d, x, d);
                if (bias) a = __fadd_rn(a, bias[e]);
                lg[j] = a;
            }
        }
        // full-precision ranking of the contenders (lowest id first on ties)
        bool tk[4] = {false, false, false, false};
        float prev = 0.0f, gap = INFINITY;
        for (int t = 0; t < k; t++) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = lane + 64 * j;
                if (cand[j] && !tk[j] && (lg[j] > bv || (lg[j] == bv && e < bi))) { bv = lg[j]; bi = e; }
            }
            wave_argmax_f(bv, bi);
#pragma unroll
            for (int j = 0; j < 4; j++) if (lane + 64 * j == bi) tk[j] = true;
            if (t > 0) gap = fminf(gap, prev - bv);
            prev = bv;
            if (lane == t) my_sel = bi;
        }
        float nb = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; j++) if (cand[j] && !tk[j]) nb = fmaxf(nb, lg[j]);
        nb = wave_max_f(nb);
        if (nb > -INFINITY) gap = fminf(gap, prev - nb);
        if (gap < kNearTie) flag |= VIREO_ROUTE_NEAR_TIE;
    }
    // softmax over all experts (src/gguf_run.c:181-182)
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) if (lane + 64 * j < E) m = fmaxf(m, lg[j]);
    m = wave_max_f(m);
    float ex[4], s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        ex[j] = lane + 64 * j < E ? expf(lg[j] - m) : 0.0f;
        s += ex[j];
    }
    s = wave_sum_f(s);
    if (probs) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j < E) probs[lane + 64 * j] = ex[j] / s;
    }
    // weight of the t-th choice on lane t: fetch ex[sel] from the owning lane
    const int src = my_sel >= 0 ? (my_sel & 63) : 0, slot = my_sel >= 0 ? (my_sel >> 6) : 0;
    const float v0 = __shfl(ex[0], src, 64), v1 = __shfl(ex[1], src, 64), v2 = __shfl(ex[2], src, 64),
                v3 = __shfl(ex[3], src, 64);
    float wt = (slot == 0 ? v0 : slot == 1 ? v1 : slot == 2 ? v2 : v3) / s;
    if (renorm) {
        float ws = 0.0f;
        for (int t = 0; t < k; t++) ws += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wt), t));
        if (ws > 0.0f) wt = wt / ws;
    }
    TopK out;
    out.sel = my_sel;
    out.w = wt;
    out.flag = flag;
    return out;
}
