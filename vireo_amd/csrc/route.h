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

// One wave: the part of a router row against x from the lane's C router
// values rv and inputs xv in registers (columns lane*C .. lane*C + C - 1;
// d == 64*C): lane l owns elements [l*C, l*C + C), so prefix sums follow
// element order. Returns the part on all lanes.
template <int C>
VH_DEV RoutePart route_row_part_vals(const float (&rv)[C], const float (&xv)[C], int lane,
                                     double *abs_products = nullptr) {
    float p[C];
#pragma unroll
    for (int i = 0; i < C; i++) p[i] = mul_rn(rv[i], xv[i]);
    double tot = 0.0, absum = 0.0, pabs = 0.0;
#pragma unroll
    for (int i = 0; i < C; i++) {
        tot += double(p[i]);
        pabs += fabs(double(p[i]));
    }
    double run = wave_incl_scan_d(tot) - tot;
#pragma unroll
    for (int i = 0; i < C; i++) {
        run += double(p[i]);
        absum += fabs(run);
    }
    RoutePart out;
    out.c = wave_sum_d(tot);
    out.beta = 1.001 * 5.9604644775390625e-08 * wave_sum_d(absum) + 1e-30;
    if (abs_products) *abs_products = wave_sum_d(pabs);
    return out;
}

// Certification of a router part computed on hb = our own RMSNorm of x
// (sum of squares in fp64, rounded once) instead of the reference's xb (an
// in-order fp32 sum, src/gguf_run.c:162). Both are fl(fl(x_i r) w_i) with a
// different scale r, so xb_i = s hb_i (1 + theta_i), |theta_i| <= 4u, with one
// s > 0 for all experts; the reference's products fl(R_i xb_i) are then
// s p_i (1 + phi_i), |phi_i| <= 6u, p_i = fl(R_i hb_i). The reference's logit
// divided by s therefore lies within beta' + 6.0003 u sum|p_i| of c (beta'
// slightly above beta: its prefix sums are ours scaled by s within 6u), and a
// ranking certified on these intervals is the reference's ranking - a common
// positive scale changes no order. (The reference's prefix sums carry the same
// 6u per product, which adds 1.001 n u * 6u sum|p_i| to beta': the second term
// of the widening.) A logit bias is not scaled with the rest;
// with one, the interval also covers |s - 1| <= sigma (the in-order fp32 sum of
// n squares is within 1.001 n u of the exact one, r moves by half of that plus
// the roundings of the scale).
VH_DEV RoutePart route_part_on_own_norm(RoutePart p, double abs_products, int n, const float *bias, int e) {
    constexpr double u = 5.9604644775390625e-08;
    p.beta = p.beta * 1.000001 + (6.0002 + 6.01 * double(n) * u) * u * abs_products;
    if (bias) {
        const double sigma = 0.5 * 1.001 * double(n) * u + 8.0 * u;
        p.beta += sigma * (fabs(p.c) + p.beta);
        p.c += double(bias[e]);
    }
    return p;
}

// The in-order fp32 sum of q[0 .. d) by one thread (the reference's
// sequence of roundings), 16 values per step with the next 16 read while
// these are added.
VH_DEV float inorder_sum(const float *q, int d) {
    float ss = 0.0f;
    int i = 0;
    if ((reinterpret_cast<uintptr_t>(q) & 15u) == 0 && d >= 16) {
        const float4 *q4 = reinterpret_cast<const float4 *>(q);
        float4 c0 = q4[0], c1 = q4[1], c2 = q4[2], c3 = q4[3];
        for (; i + 32 <= d; i += 16) {
            const int j = (i >> 2) + 4;
            const float4 n0 = q4[j], n1 = q4[j + 1], n2 = q4[j + 2], n3 = q4[j + 3];
            // the reads stay ahead of the adds: memory operations do not cross
            // this asm, and the chain passes through it (the compiler would sink them)
            asm volatile("" : "+v"(ss)::"memory");
            ss = add_rn(add_rn(add_rn(add_rn(ss, c0.x), c0.y), c0.z), c0.w);
            ss = add_rn(add_rn(add_rn(add_rn(ss, c1.x), c1.y), c1.z), c1.w);
            ss = add_rn(add_rn(add_rn(add_rn(ss, c2.x), c2.y), c2.z), c2.w);
            ss = add_rn(add_rn(add_rn(add_rn(ss, c3.x), c3.y), c3.z), c3.w);
            c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        }
        ss = add_rn(add_rn(add_rn(add_rn(ss, c0.x), c0.y), c0.z), c0.w);
        ss = add_rn(add_rn(add_rn(add_rn(ss, c1.x), c1.y), c1.z), c1.w);
        ss = add_rn(add_rn(add_rn(add_rn(ss, c2.x), c2.y), c2.z), c2.w);
        ss = add_rn(add_rn(add_rn(add_rn(ss, c3.x), c3.y), c3.z), c3.w);
        i += 16;
    }
    for (; i < d; i++) ss = add_rn(ss, q[i]);
    return ss;
}

// The reference's RMSNorm of x (src/gguf_run.c:161-165) into dst[0..d) by a
// whole workgroup, bit for bit: the squares in parallel, their in-order fp32
// sum by one thread (d dependent adds: used only where exactness needs it),
// r = 1/sqrtf(ss/n + eps), then (x_i r) w_i. dst: d floats (LDS or global),
// red: one float of LDS; sq (optional): d floats of LDS for the squares
// (each branch keeps its pointer's own address space, so the sum reads LDS
// with LDS loads), else they go to dst. All threads of the workgroup call it.
VH_DEV void reference_rmsnorm_block(float *dst, const float *__restrict__ x, const float *__restrict__ nw, float eps,
                                    int d, float *red, float *sq = nullptr) {
    if (sq) {
        for (int i = threadIdx.x; i < d; i += blockDim.x) sq[i] = mul_rn(x[i], x[i]);
        __syncthreads();
        if (threadIdx.x == 0)
            *red = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(inorder_sum(sq, d), float(d)), eps)));
    } else {
        for (int i = threadIdx.x; i < d; i += blockDim.x) dst[i] = mul_rn(x[i], x[i]);
        __syncthreads();
        if (threadIdx.x == 0)
            *red = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(inorder_sum(dst, d), float(d)), eps)));
    }
    __syncthreads();
    const float r = *red;
    for (int i = threadIdx.x; i < d; i += blockDim.x)
        dst[i] = nw ? mul_rn(mul_rn(x[i], r), nw[i]) : mul_rn(x[i], r);
    __syncthreads();
}

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
            p[4 * i + 0] = mul_rn(a.x, b.x);
            p[4 * i + 1] = mul_rn(a.y, b.y);
            p[4 * i + 2] = mul_rn(a.z, b.z);
            p[4 * i + 3] = mul_rn(a.w, b.w);
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
        for (int i = i0; i < i1; i++) tot += double(mul_rn(r[i], x[i]));
        run = wave_incl_scan_d(tot) - tot;
        for (int i = i0; i < i1; i++) {
            run += double(mul_rn(r[i], x[i]));
            absum += fabs(run);
        }
    }
    RoutePart out;
    out.c = wave_sum_d(tot);
    out.beta = 1.001 * 5.9604644775390625e-08 * wave_sum_d(absum) + 1e-30;
    return out;
}

// The reference logit exactly: a = 0; a += r[i]*x[i] for i in order, every
// product and sum rounded to fp32. The chain is sequential, so its speed is
// set by keeping the operands in registers ahead of it: with 16-byte aligned
// rows and d a multiple of 64, chunks of 64 elements are loaded one chunk
// ahead of the chunk being summed.
VH_DEV float exact_logit(const float *__restrict__ r, const float *__restrict__ x, int d) {
    float a = 0.0f;
    if (((reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0 && d % 64 == 0) {
        const float4 *r4 = reinterpret_cast<const float4 *>(r), *x4 = reinterpret_cast<const float4 *>(x);
        float4 rc[16], xc[16], rn[16], xn[16];
#pragma unroll
        for (int i = 0; i < 16; i++) { rc[i] = r4[i]; xc[i] = x4[i]; }
        for (int c = 0; c < d / 64; c++) {
            const int nxt = c + 1 < d / 64 ? c + 1 : c;
#pragma unroll
            for (int i = 0; i < 16; i++) { rn[i] = r4[16 * nxt + i]; xn[i] = x4[16 * nxt + i]; }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                a = add_rn(a, mul_rn(rc[i].x, xc[i].x));
                a = add_rn(a, mul_rn(rc[i].y, xc[i].y));
                a = add_rn(a, mul_rn(rc[i].z, xc[i].z));
                a = add_rn(a, mul_rn(rc[i].w, xc[i].w));
            }
#pragma unroll
            for (int i = 0; i < 16; i++) { rc[i] = rn[i]; xc[i] = xn[i]; }
        }
        return a;
    }
    for (int i = 0; i < d; i++) a = add_rn(a, mul_rn(r[i], x[i]));
    return a;
}

// Order-preserving 32-bit image of an fp32 value.
VH_DEV uint32_t ordered_u32(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The contenders' exact logits with their router rows streamed through LDS:
// wave 1 copies chunks of 256 columns of up to kStageRows rows by direct
// global-to-LDS loads (global_load_lds_dwordx4: lane i's 16 bytes land at the
// wave-uniform base + 16 i) into three buffers, two chunks ahead of the
// chains, and lane c (< n) of wave 0 runs contender c's chain
// a = fl(a + fl(r_i x_i)), i = 0 .. d-1, in order, exactly as exact_logit
// does, reading its row and the inputs (already in LDS: xs) four at a time.
// Rows are 16 bytes apart beyond their 1 KB, so the chains' reads of one
// column group fall in different banks. Every chunk issues kStageRows loads
// (rows past n repeat contender 0 into their own slots), so an explicit
// vmcnt wait leaves the two later chunks in flight; the barriers are bare
// s_barriers for the same reason. Needs d % 256 == 0, n <= kStageRows, R
// 16-byte aligned and at least two waves; every thread calls it. Returns lane
// c's logit on wave 0 (without the bias), 0 elsewhere.
constexpr int kStageRows = 16, kStageRowF4 = 65;  // a row chunk is 64 float4s, plus one of padding
constexpr int kStageBufF4 = kStageRows * kStageRowF4;
constexpr int kStageScrF4 = 3 * kStageBufF4;  // 49 920 bytes of LDS
VH_DEV bool exact_staged_ok(const float *R, int d, int n) {
    return n <= kStageRows && d % 256 == 0 && (reinterpret_cast<uintptr_t>(R) & 15u) == 0 && blockDim.x >= 128;
}
VH_DEV float exact_logits_staged(const float *__restrict__ R, const float *xs, int d, const int *cand, int n,
                                 float4 *scr) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nch = d / 256;
    auto issue = [&](int buf, int c) {  // wave 1: chunk c of every row into buffer buf
        const float *src = R + 256 * c + 4 * lane;
#pragma unroll
        for (int j = 0; j < kStageRows; j++) {
            const int e = cand[j < n ? j : 0];
            __builtin_amdgcn_global_load_lds((gvoid *)(src + size_t(e) * d),
                                             (lds_void *)(scr + buf * kStageBufF4 + j * kStageRowF4), 16, 0, 0);
        }
    };
    if (wv == 1) {
        issue(0, 0);
        issue(1, min(1, nch - 1));
    }
    float a = 0.0f;
    for (int c = 0; c < nch; c++) {
        if (wv == 1) {
            issue((c + 2) % 3, min(c + 2, nch - 1));  // past the last chunk: the last again, into a spent buffer
            VH_WAIT_VMCNT(2 * kStageRows);             // chunk c has landed; c + 1 and c + 2 stay in flight
        }
        dma_barrier();
        if (wv == 0 && lane < n) {
            // 16 columns per step, the next 16 read before these are added
            const float4 *row = scr + (c % 3) * kStageBufF4 + lane * kStageRowF4;
            const float4 *x4 = reinterpret_cast<const float4 *>(xs + 256 * c);
            float4 r0 = row[0], r1 = row[1], r2 = row[2], r3 = row[3];
            float4 x0 = x4[0], x1 = x4[1], x2 = x4[2], x3 = x4[3];
            auto step = [&](const float4 &r, const float4 &xv) {
                a = add_rn(a, mul_rn(r.x, xv.x));
                a = add_rn(a, mul_rn(r.y, xv.y));
                a = add_rn(a, mul_rn(r.z, xv.z));
                a = add_rn(a, mul_rn(r.w, xv.w));
            };
            for (int c4 = 0; c4 < 64; c4 += 4) {
                const int nx = c4 + 4 < 64 ? c4 + 4 : c4;
                const float4 q0 = row[nx], q1 = row[nx + 1], q2 = row[nx + 2], q3 = row[nx + 3];
                const float4 y0 = x4[nx], y1 = x4[nx + 1], y2 = x4[nx + 2], y3 = x4[nx + 3];
                asm volatile("" : "+v"(a)::"memory");  // the reads stay ahead of the chain
                step(r0, x0);
                step(r1, x1);
                step(r2, x2);
                step(r3, x3);
                r0 = q0; r1 = q1; r2 = q2; r3 = q3;
                x0 = y0; x1 = y1; x2 = y2; x3 = y3;
            }
        }
        dma_barrier();  // buffer c % 3 is read before chunk c + 3 goes into it
    }
    if (wv == 1) VH_WAIT_VMCNT(0);  // no load may land after the buffers are given back
    dma_barrier();
    return a;
}

// The reference logit exactly (exact_logit's in-order chain a = fl(a +
// fl(r_i x_i)), i = 0 .. 2047) by a whole wave, for d = 2048: lane l runs
// steps 32 l .. 32 l + 31 from a guess of the chain's value there and hands
// its end to lane l + 1, until every lane's start equals, bit for bit, the
// end of the lane before it (lane 0 starts at the reference's 0). Then every
// lane ran from the chain's true value, by induction from lane 0, and lane
// 63's end is the reference's sum. Each round fixes at least one more lane,
// so 64 rounds always suffice (the first guesses are the fp64 prefix sums of
// the products rounded to fp32). Chains from starts a few ulps apart rarely
// meet, so on router-like data most of the 64 rounds run and the chain takes
// about as long as one lane's; the gain is that a workgroup's waves each
// take a contender. r and xv: the lane's 32 elements of the row (16-byte
// aligned) and of the inputs. Every lane gets the result.
VH_DEV float exact_logit_wave(const float *__restrict__ r, const float (&xv)[32], int lane) {
    float p[32];
    const float4 *r4 = reinterpret_cast<const float4 *>(r + lane * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 a = r4[i];
        p[4 * i] = mul_rn(a.x, xv[4 * i]);
        p[4 * i + 1] = mul_rn(a.y, xv[4 * i + 1]);
        p[4 * i + 2] = mul_rn(a.z, xv[4 * i + 2]);
        p[4 * i + 3] = mul_rn(a.w, xv[4 * i + 3]);
    }
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < 32; i++) tot += double(p[i]);
    const double pre = wave_incl_scan_d(tot) - tot;
    float g = lane == 0 ? 0.0f : float(pre), e = 0.0f;
    for (int round = 0; round <= 64; round++) {
        e = g;
#pragma unroll
        for (int i = 0; i < 32; i++) e = add_rn(e, p[i]);
        const float from = __shfl_up(e, 1, 64);
        const float ng = lane == 0 ? 0.0f : from;
        if (__ballot(__float_as_uint(ng) != __float_as_uint(g)) == 0ull) break;
        g = ng;
    }
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), 63));
}

constexpr int kXScrFloats = 2048;  // inputs route_topk_block can copy into its caller's x_scr

// Workspace of route_topk_block (LDS).
struct TopKSmem {
    uint32_t key[kMaxExperts];       // 32-bit rank keys; then the exact path's exponentials
    uint64_t key64[kMaxExperts];     // full-precision keys (re-ranking)
    int sel[64];                     // chosen experts in order
    float sel_w[64];                 // their weights
    double sel_lo[65], sel_hi[64];   // their intervals; sel_lo[64]: best remaining
    float red[2][8];                 // per-wave partials (up to 8 waves)
    float m;                         // max logit
    float s, p_next;                 // exact path: the softmax's sum, the best probability left out
    uint32_t flag;
    int uncertain;
    // the contenders' exact logits (route_topk_block's first fallback)
    int cand[64], corder[64];
    float cl[64];
    double cut;
    int ncand, near;
};

// Fp32 spacing at |v| (the distance to the next float away from zero).
VH_DEV float ulp_f(float v) {
    const float a = fabsf(v);
    return __uint_as_float(__float_as_uint(a) + 1u) - a;
}

// Margin below the chosen experts' lowest lower bound within which an expert
// still contends for the top k when the ranking is not certified.
constexpr double kContend = 1e-4;

// Logit span of a certified top k: the k-th chosen expert's logit lies within
// kRouteSpan of the largest. The reference ranks probabilities
// p = expf(l - m) / s (src/gguf_run.c:180-191) and lets the lowest id win a
// tie; distinct logits can give equal probabilities only where l - m is
// rounded coarser than kRouteMargin (|l - m| >= 32, fp32 spacing 3.8e-6) or
// expf underflows, so within the span a certified logit order is the
// reference's probability order.
constexpr double kRouteSpan = 30.0;

// Top-k of one token by a workgroup of 256 to 512 threads (all threads call
// it; E <= 256, k <= 64). Thread e owns expert e. Its rank is the number of
// experts with a larger key, so the k chosen experts and their order come out
// of one parallel pass. The ranking is certified with the fp64 intervals:
// every gap that decides the set or its order wider than both bounds plus
// kRouteMargin, and the chosen within kRouteSpan of the top. Otherwise the
// contenders' exact logits decide (see below) or, when they are too close,
// the reference's softmax is formed exactly - every logit in-order fp32 (or
// exact_parts: the parts hold them, beta = 0), m, expf(l - m), their in-order
// fp32 sum s and p = e / s (src/gguf_run.c:180-182) - and the experts are
// ranked on p with the lowest id winning a tie (:189-191); the weights are
// those p. The device's expf can differ from the reference's C library by an
// ulp: it decides only exact ties of the exponentials, and a chosen
// probability equal to the next one, or exact logits closer than kNearTie, is
// reported (VIREO_ROUTE_NEAR_TIE). On return (after a barrier) sm.sel /
// sm.sel_w / sm.flag hold the result; probs (optional, [E]) receives the
// softmax. stage_scr (kStageScrF4 float4s) and x_scr (kXScrFloats floats), both
// LDS and optional, let the contenders' chains read their rows and inputs
// from LDS (exact_logits_staged).
VH_DEV void route_topk_block(TopKSmem &sm, const RoutePart *__restrict__ part, const float *__restrict__ R,
                             const float *__restrict__ x, const float *__restrict__ bias, int d, int E, int k,
                             int renorm, bool exact_parts, float *__restrict__ probs,
                             float4 *stage_scr = nullptr, float *x_scr = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nwaves = int(blockDim.x) >> 6;
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
    // order always reaches the exact ranking below.
    const uint32_t key = mine ? ((ordered_u32(lg) & 0xffffff00u) | uint32_t(255 - tid)) : 0u;
    if (tid < kMaxExperts) sm.key[tid] = key;
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
        float rh = sm.red[0][0];
        for (int i = 1; i < nwaves; i++) rh = fmaxf(rh, sm.red[0][i]);
        const double next_hi = tid + 1 < k ? sm.sel_hi[tid + 1] : (k < E ? double(rh) : -INFINITY);
        if (!(sm.sel_lo[tid] - next_hi > kRouteMargin)) atomicOr(&sm.uncertain, 1);
        if (!(sm.sel_lo[tid] > sm.sel_hi[0] - kRouteSpan)) atomicOr(&sm.uncertain, 1);
    }
    __syncthreads();
    // Not certified: first the exact in-order logits of the contenders only -
    // the k experts ranked first and every expert whose upper bound reaches
    // the lowest of their lower bounds less kContend (any other expert's
    // exact logit lies more than kContend below each of those k, so the
    // reference's top k is among the contenders). Ranked on those logits
    // (lowest id first on equal ones), the result is the reference's ranking
    // when every decision down to the k-th place is a gap wider than 2 ulp of
    // the larger |l - m| plus 1e-6: then the reference's rounded l - m,
    // its expf and the division by the common sum keep the order strictly, so
    // the probabilities rank the same and no tie rule applies. Otherwise (or
    // with more than 64 contenders) the whole softmax is formed exactly below.
    bool full = sm.uncertain != 0, resolved = false;
    if (full && !exact_parts) {
        if (tid == 0) {
            double L = sm.sel_lo[0];
            for (int t = 1; t < k; t++) L = fmin(L, sm.sel_lo[t]);
            sm.cut = L - kContend;
            sm.ncand = 0;
            sm.near = 0;
        }
        __syncthreads();
        if (mine && (rank < k || hi >= sm.cut)) {
            const int j = atomicAdd(&sm.ncand, 1);
            if (j < 64) sm.cand[j] = tid;
        }
        __syncthreads();
        const int n = sm.ncand;
        if (n <= 64) {
            // with LDS from the caller: the rows streamed through it (the inputs
            // copied there first unless they already are); else each
            // contender's lane reads its own row
            const bool staged = stage_scr && x_scr && d <= kXScrFloats && exact_staged_ok(R, d, n);
            const bool waves = d == 2048 && ((reinterpret_cast<uintptr_t>(R) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0;
            if (waves) {  // one contender per wave at a time, the chain split over its lanes
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
                for (int c = wv; c < n; c += nwaves) {
                    const int e = sm.cand[c];
                    const float a = exact_logit_wave(R + size_t(e) * d, xv, lane);
                    if (lane == 0) sm.cl[c] = bias ? add_rn(a, bias[e]) : a;
                }
            } else if (staged) {
                if (x != x_scr)
                    for (int i = tid; i < d; i += blockDim.x) x_scr[i] = x[i];
                __syncthreads();
                const float a = exact_logits_staged(R, x_scr, d, sm.cand, n, stage_scr);
                if (wv == 0 && lane < n) sm.cl[lane] = bias ? add_rn(a, bias[sm.cand[lane]]) : a;
            } else if (wv == 0 && lane < n) {
                const int e = sm.cand[lane];
                float a = exact_logit(R + size_t(e) * d, x, d);
                if (bias) a = add_rn(a, bias[e]);
                sm.cl[lane] = a;
            }
            __syncthreads();
            if (tid < n) {
                const float a = sm.cl[tid];
                const int e = sm.cand[tid];
                int r = 0;
                for (int i = 0; i < n; i++) {
                    const float b = sm.cl[i];
                    r += int(b > a || (b == a && sm.cand[i] < e));
                }
                sm.corder[r] = tid;
            }
            __syncthreads();
            if (tid < k) {
                // place tid against place tid + 1 (the best contender left
                // out, or below the cut everything outside the contenders)
                const float m = sm.cl[sm.corder[0]], a = sm.cl[sm.corder[tid]];
                const float b = tid + 1 < n ? sm.cl[sm.corder[tid + 1]] : float(sm.cut);
                const float span = fmaxf(fabsf(sub_rn(a, m)), fabsf(sub_rn(b, m)));
                const double gap = tid + 1 < n ? double(a) - double(b) : double(a) - sm.cut;
                if (!(gap > 2.0 * double(ulp_f(span)) + 1e-6)) atomicOr(&sm.near, 1);
                if (tid == k - 1) {  // the experts outside the contenders lie below the cut
                    const float sc = fabsf(sub_rn(float(sm.cut), m));
                    if (!(kContend > 2.0 * double(ulp_f(sc)) + 1e-6)) atomicOr(&sm.near, 1);
                }
            }
            __syncthreads();
            if (!sm.near) {
                full = false;
                resolved = true;
                if (tid < k) sm.sel[tid] = sm.cand[sm.corder[tid]];
                if (tid == 0) sm.flag = VIREO_ROUTE_EXACT_FALLBACK;
                __syncthreads();
            }
        }
    }
    if (full) {
        // the reference's softmax, exactly: every logit, their maximum, the
        // exponentials, their in-order sum (one thread), the probabilities
        if (mine && !exact_parts) {
            float a = exact_logit(R + size_t(tid) * d, x, d);
            if (bias) a = add_rn(a, bias[tid]);
            lg = a;
        }
        const float wm = wave_max_f(mine ? lg : -INFINITY);
        __syncthreads();  // every thread is done with the first ranking's LDS
        if (lane == 0) sm.red[0][wv] = wm;
        __syncthreads();
        float m = sm.red[0][0];
        for (int i = 1; i < nwaves; i++) m = fmaxf(m, sm.red[0][i]);
        const float ev = mine ? expf(sub_rn(lg, m)) : 0.0f;
        if (tid < kMaxExperts) sm.key[tid] = __float_as_uint(ev);
        if (tid == 0) {
            sm.flag = exact_parts ? 0u : VIREO_ROUTE_EXACT_FALLBACK;
            sm.p_next = -1.0f;
            sm.sel_lo[64] = -INFINITY;
        }
        __syncthreads();
        if (tid == 0) {
            float s = 0.0f;
            for (int i = 0; i < E; i++) s = add_rn(s, __uint_as_float(sm.key[i]));
            sm.s = s;
        }
        __syncthreads();
        const float pr = __fdiv_rn(ev, sm.s);
        if (tid < kMaxExperts) sm.key64[tid] = mine ? ((uint64_t(ordered_u32(pr)) << 8) | uint64_t(255 - tid)) : 0ull;
        __syncthreads();
        rank = 1 << 30;
        if (mine) {
            const uint64_t k64 = sm.key64[tid];
            int r = 0;
            for (int j = 0; j < E; j++) r += int(sm.key64[j] > k64);
            rank = r;
            if (probs) probs[tid] = pr;
            if (rank < k) { sm.sel[rank] = tid; sm.sel_w[rank] = pr; sm.sel_lo[rank] = double(lg); }
            if (rank == k) { sm.sel_lo[64] = double(lg); sm.p_next = pr; }  // best contender left out
        }
        __syncthreads();
        if (tid < k) {
            const double nxt = tid + 1 < k ? sm.sel_lo[tid + 1] : sm.sel_lo[64];
            const float pn = tid + 1 < k ? sm.sel_w[tid + 1] : sm.p_next;
            if (fabs(sm.sel_lo[tid] - nxt) < double(kNearTie) || sm.sel_w[tid] == pn)
                atomicOr(&sm.flag, VIREO_ROUTE_NEAR_TIE);
        }
        __syncthreads();
    } else {
        // softmax over all experts (src/gguf_run.c:181-182) on the certified
        // logits (also for a ranking the contenders' exact logits resolved:
        // only the order had to be exact)
        const float ex = mine ? expf(lg - sm.m) : 0.0f;
        const float part_sum = wave_sum_f(ex);
        if (lane == 0) sm.red[1][wv] = part_sum;
        __syncthreads();
        float s = sm.red[1][0];
        for (int i = 1; i < nwaves; i++) s += sm.red[1][i];
        if (mine) {
            if (probs) probs[tid] = ex / s;
            if (!resolved && rank < k) sm.sel_w[rank] = ex / s;
        }
        if (resolved && tid < k) sm.sel_w[tid] = expf(float(part[sm.sel[tid]].c) - sm.m) / s;
        __syncthreads();
    }
    if (tid == 0 && renorm) {
        float wsum = 0.0f;
        for (int t = 0; t < k; t++) wsum += sm.sel_w[t];  // in selection order
        if (wsum > 0.0f)
            for (int t = 0; t < k; t++) sm.sel_w[t] = sm.sel_w[t] / wsum;
    }
    __syncthreads();
}

// The chosen experts of one token by one wave, without a workgroup barrier,
// so that every wave of a workgroup can select on its own: Q parts per lane
// (expert lane + 64q, E <= 64Q); k rounds of a wave-wide max over the 32-bit
// keys (lower id wins a tie) find the winners, then the order is certified in
// one step as in route_topk_block: each winner's owner writes its interval to
// `cert` (64 entries of this wave's LDS) and lane t checks round t against
// round t+1 (the last round against the best upper bound left out). Returns
// whether it was certified (the same on every lane, and in every wave given
// the same parts). e_want / e_want2 receive the experts chosen in rounds want
// / want2; rank[q] the round in which this lane's slot q was chosen (-1 if not).
template <int Q>
VH_DEV bool route_select_wave(const RoutePart (&p)[Q], int E, int k, int want, int &e_want, int want2, int &e_want2,
                              int (&rank)[Q], double2 *cert) {
    const int lane = threadIdx.x & 63;
    uint32_t key[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int e = lane + 64 * q;
        key[q] = e < E ? ((ordered_u32(float(p[q].c)) & 0xffffff00u) | uint32_t(255 - e)) : 0u;
        rank[q] = -1;
    }
    e_want = 0;
    e_want2 = 0;
    for (int t = 0; t < k; t++) {
        uint32_t best = 0u;
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (rank[q] < 0 && key[q] > best) best = key[q];
        const uint32_t wb = wave_max_u(best);
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (key[q] == wb) rank[q] = t;  // keys are distinct: one slot of one lane
        if (t == want) e_want = 255 - int(wb & 0xffu);
        if (t == want2) e_want2 = 255 - int(wb & 0xffu);
    }
    float rest = -INFINITY;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        if (rank[q] >= 0) cert[rank[q]] = make_double2(p[q].c - p[q].beta, p[q].c + p[q].beta);
        else if (key[q] != 0u) rest = fmaxf(rest, __double2float_ru(p[q].c + p[q].beta));
    }
    rest = wave_max_f(rest);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bool good = true;
    if (lane < k) {
        const double lo = cert[lane].x;
        if (lane + 1 < k) good = lo - cert[lane + 1].y > kRouteMargin;
        else if (k < E) good = lo - double(rest) > kRouteMargin;
        good = good && lo > cert[0].y - kRouteSpan;  // no probability ties (route_topk_block)
    }
    return __builtin_amdgcn_read_exec() == __ballot(good);
}

// The two halves of route_select_wave, for callers that act on the ranking
// before it is certified (and redo the work when it is not): k rounds of the
// wave-wide max over the 32-bit keys (rank[q] = the round of slot q, -1 if not
// chosen; sel[t] (LDS, k entries) = the expert of round t, written by the lane
// that owns it), then the certification of that order as route_select_wave
// does it (cert: 64 entries of this wave's LDS; the same verdict on every
// lane, and in every wave or workgroup given the same parts).
template <int Q>
VH_DEV void route_rank_wave(const RoutePart (&p)[Q], int E, int k, int (&rank)[Q], int *sel) {
    const int lane = threadIdx.x & 63;
    uint32_t key[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int e = lane + 64 * q;
        key[q] = e < E ? ((ordered_u32(float(p[q].c)) & 0xffffff00u) | uint32_t(255 - e)) : 0u;
        rank[q] = -1;
    }
    for (int t = 0; t < k; t++) {
        uint32_t best = 0u;
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (rank[q] < 0 && key[q] > best) best = key[q];
        const uint32_t wb = wave_max_u(best);
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (key[q] == wb) {  // keys are distinct: one slot of one lane
                rank[q] = t;
                sel[t] = lane + 64 * q;
            }
    }
}

// The same ranking as route_rank_wave by a whole workgroup of 512 threads in
// one counting pass instead of k dependent wave-wide rounds: every wave holds
// the same parts; the keys go to LDS, thread t counts the keys above the key of
// expert t mod 64Q among one share of 64Q / (512 / 64Q) keys, and the shares'
// counts meet in LDS. The rank of an expert is its count (distinct keys: the
// same order as k rounds of the maximum). rank[q] is the rank of slot q when
// below k, else -1, in every wave; sel[t] (LDS, k entries) is the expert of
// rank t, written by wave 0 when sel is not null. Contains two LDS-only
// workgroup barriers (global loads in flight keep streaming); keys holds 64Q
// entries and cnt 512.
template <int Q>
VH_DEV void route_rank_block(const RoutePart (&p)[Q], int E, int k, uint32_t *keys, int *cnt, int (&rank)[Q],
                             int *sel) {
    constexpr int EP = 64 * Q, S = 512 / EP, N = EP / S;
    static_assert(S * EP == 512 && N % 4 == 0, "512 threads cover the experts in whole shares");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t key[Q], mine = 0u;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int e = lane + 64 * q;
        key[q] = e < E ? ((ordered_u32(float(p[q].c)) & 0xffffff00u) | uint32_t(255 - e)) : 0u;
        if (q == wv % Q) mine = key[q];
    }
    if (wv < Q) keys[tid] = mine;
    lds_barrier();
    const int s = wv / Q;  // this thread's share of keys
    const uint4 *kv = reinterpret_cast<const uint4 *>(keys + s * N);
    int c = 0;
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
        const uint4 v = kv[i];
        c += int(v.x > mine) + int(v.y > mine) + int(v.z > mine) + int(v.w > mine);
    }
    cnt[s * EP + (tid % EP)] = c;
    lds_barrier();
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int e = lane + 64 * q;
        int r = 0;
#pragma unroll
        for (int t = 0; t < S; t++) r += cnt[t * EP + e];
        rank[q] = e < E && r < k ? r : -1;
        if (sel && wv == 0 && rank[q] >= 0) sel[r] = e;
    }
}

// The expert of rank t (0 <= t < k) from rank[] as route_rank_block leaves
// it, on every lane of the wave.
template <int Q>
VH_DEV int rank_owner(const int (&rank)[Q], int t) {
    int e = 0;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const uint64_t m = __ballot(rank[q] == t);
        if (m) e = 64 * q + __builtin_ctzll(m);
    }
    return e;
}

template <int Q>
VH_DEV bool route_certify_wave(const RoutePart (&p)[Q], int E, int k, const int (&rank)[Q], double2 *cert) {
    const int lane = threadIdx.x & 63;
    float rest = -INFINITY;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        if (rank[q] >= 0) cert[rank[q]] = make_double2(p[q].c - p[q].beta, p[q].c + p[q].beta);
        else if (lane + 64 * q < E) rest = fmaxf(rest, __double2float_ru(p[q].c + p[q].beta));
    }
    rest = wave_max_f(rest);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bool good = true;
    if (lane < k) {
        const double lo = cert[lane].x;
        if (lane + 1 < k) good = lo - cert[lane + 1].y > kRouteMargin;
        else if (k < E) good = lo - double(rest) > kRouteMargin;
        good = good && lo > cert[0].y - kRouteSpan;  // no probability ties (route_topk_block)
    }
    return __builtin_amdgcn_read_exec() == __ballot(good);
}

// Softmax weights of the experts chosen by route_select_wave (src/gguf_run.c:
// 181-192), by one wave: lane t < k returns the expert of round t in e_out and
// its weight (renormalised over the k in selection order when renorm).
// `stage` is a 64-entry LDS scratch owned by this wave.
template <int Q>
VH_DEV void route_weights_wave(const RoutePart (&p)[Q], const int (&rank)[Q], int E, int k, int renorm,
                               float2 *stage, int &e_out, float &w_out) {
    const int lane = threadIdx.x & 63;
    float lg[Q], mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        lg[q] = lane + 64 * q < E ? float(p[q].c) : -INFINITY;
        mx = fmaxf(mx, lg[q]);
    }
    const float m = wave_max_f(mx);
    float ex[Q], part = 0.0f;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        ex[q] = lane + 64 * q < E ? expf(lg[q] - m) : 0.0f;
        part += ex[q];
    }
    const float s = wave_sum_f(part);
#pragma unroll
    for (int q = 0; q < Q; q++)
        if (rank[q] >= 0) stage[rank[q]] = make_float2(ex[q] / s, __int_as_float(lane + 64 * q));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float2 v = stage[lane < k ? lane : 0];
    float w = v.x;
    if (renorm) {
        float wsum = 0.0f;
        for (int t = 0; t < k; t++) wsum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), t));
        if (wsum > 0.0f) w = w / wsum;
    }
    e_out = __float_as_int(v.y);
    w_out = w;
}

// Entry idx of a table spread over a wave's registers as table_entry holds
// it, where idx may differ from lane to lane: every lane reads all TPL slots of
// lane idx / TPL across the wave (ds_bpermute; call it with every lane of the
// wave active) and keeps slot idx % TPL. No memory round trip, unlike a
// reload of the entry from the table.
template <int TPL>
VH_DEV const void *table_gather(const void *const (&tab)[TPL], int idx) {
    const int src = idx / TPL, slot = idx - src * TPL;
    uint64_t v = 0;
#pragma unroll
    for (int s = 0; s < TPL; s++) {
        const uint64_t t = reinterpret_cast<uint64_t>(tab[s]);
        const uint32_t lo = uint32_t(__builtin_amdgcn_ds_bpermute(src << 2, int(uint32_t(t))));
        const uint32_t hi = uint32_t(__builtin_amdgcn_ds_bpermute(src << 2, int(uint32_t(t >> 32))));
        if (s == slot) v = (uint64_t(hi) << 32) | lo;
    }
    return reinterpret_cast<const void *>(v);
}

// Entry idx of a table spread over a wave's registers (lane l holds entries
// [TPL*l, TPL*l + TPL)); idx must be the same on every lane.
template <int TPL>
VH_DEV const uint8_t *table_entry(const void *const (&tab)[TPL], int idx) {
    const int src = idx / TPL, slot = idx - src * TPL;
    uint64_t v = 0;
#pragma unroll
    for (int s = 0; s < TPL; s++)
        if (s == slot) v = reinterpret_cast<uint64_t>(tab[s]);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), src));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), src));
    return reinterpret_cast<const uint8_t *>((uint64_t(hi) << 32) | lo);
}

