// Grouped projections for groups of a few tokens (calls of a decode batch's
// size, fewer than kMfmaMinCall tokens), built like the one-token
// decode kernels: a lane owns fixed 32-weight items of every row its wave
// computes, the wave loads the raw words of its rows once, and the group's
// tokens stream through in chunks of NT whose inputs (and their run sums) sit
// in registers. A group's weights are therefore read from HBM once, whatever
// its token count, and no LDS staging or barrier is involved.
//
// gate/up: grid (ceil(fe / (8 RPW NB)), active slots), 512 threads; every
// wave computes NB batches of RPW rows of gate and up of expert active[s];
// lane l owns items l, l + 64, ... (IPL of them) of a row of d columns;
// h[pair][o] = silu(gate_o . hb) * (up_o . hb) (src/gguf_run.c:205-207).
//
// down: grid (ceil(d / (8 (64 / L) RPG NB)), active slots), 512 threads; lane
// groups of L lanes, each computing NB batches of RPG rows of down of expert
// active[s]; lane li owns items li, li + L, ... of a row of fe columns;
// y[pair][o] = down_o . h[pair] (src/gguf_run.c:208), combined afterwards in
// selection order by combine_kernel.
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route_kernels.h"

namespace {

// An item's raw words reduced to what every token's dot product needs: the
// token-independent work of Reg<T>::compute (scale unpacking, bit assembly,
// alignment) done once per row, the same arithmetic per token afterwards.
template <int T>
struct Prep;

template <>
struct Prep<VT_Q4_K> {  // d1·Σq·x − m1·Σx over the low and the high nibbles
    uint4 q;
    float d1, m1, d2, m2;
    VH_DEV void set(const Reg<VT_Q4_K>::Words &r, int it) {
        const int c = (it & 7) >> 1;
        const float d = h2f(r.hdr.x & 0xffffu), dmin = h2f(r.hdr.x >> 16);
        int sc0, mn0, sc1, mn1;
        q4k_scale_min(2 * c, r.hdr.y, r.hdr.z, r.hdr.w, sc0, mn0);
        q4k_scale_min(2 * c + 1, r.hdr.y, r.hdr.z, r.hdr.w, sc1, mn1);
        d1 = d * float(sc0);
        m1 = dmin * float(mn0);
        d2 = d * float(sc1);
        m2 = dmin * float(mn1);
        q = r.q;
    }
    VH_DEV float dot(const float (&x)[32], const float (&s)[2]) const {
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        float dl = 0.0f, dh = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t lo = qw[i] & 0x0f0f0f0fu, hi = (qw[i] >> 4) & 0x0f0f0f0fu;
            asm volatile("" : "+v"(lo), "+v"(hi));  // one v_cvt_f32_ubyte per quant
#pragma unroll
            for (int k = 0; k < 4; k++) {
                dl = fmaf(float((lo >> (8 * k)) & 0xffu), x[4 * i + k], dl);
                dh = fmaf(float((hi >> (8 * k)) & 0xffu), x[16 + 4 * i + k], dh);
            }
        }
        return d1 * dl - m1 * s[0] + d2 * dh - m2 * s[1];
    }
};

template <>
struct Prep<VT_Q6_K> {  // d·Σ_g sc_g (Σq·x − 32 Σx) over the four runs
    uint32_t t[4][2];
    float sc[4], d;
    VH_DEV void set(const Q6Raw &r, int) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t A = h ? r.a1 : r.a0, B = h ? r.b1 : r.b0, H = h ? r.h1 : r.h0;
            t[0][h] = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
            t[1][h] = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
            t[2][h] = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
            t[3][h] = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int g = 0; g < 4; g++) sc[g] = float(int(int8_t(r.sc >> (8 * g))));
        d = h2f(r.d);
    }
    VH_DEV float dot(const float (&x)[32], const float (&sx)[4]) const {
        float s = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t w0 = t[g][0], w1 = t[g][1];
            asm volatile("" : "+v"(w0), "+v"(w1));
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) acc = fmaf(float(((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xffu), x[8 * g + i], acc);
            s = fmaf(sc[g], fmaf(-32.0f, sx[g], acc), s);
        }
        return d * s;
    }
};

template <>
struct Prep<VT_Q8_0> {  // d·Σq·x over the block's 32 signed bytes
    uint32_t q[8];
    float d;
    VH_DEV void set(const Reg<VT_Q8_0>::Words &r, int) {
        d = h2f((r.w[0] >> (8 * r.s)) & 0xffffu);
        const uint32_t sh = 16 + 8 * r.s;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = uint32_t(((uint64_t(r.w[i + 1]) << 32) | r.w[i]) >> sh);
    }
    VH_DEV float dot(const float (&x)[32], const float (&)[1]) const {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int k = 0; k < 4; k++) acc = fmaf(float(int(int8_t(q[i] >> (8 * k)))), x[4 * i + k], acc);
        return acc * d;
    }
};

// gate/up: wave w of workgroup (b, s) owns rows ((8 b + w) NB + i) RPW + r
// (i < NB batches, r < RPW) of gate and up of expert active[s]. For each
// chunk of NT tokens it loads their inputs once and streams its batches of
// rows, the next batch's raw words in flight while the current one computes.
template <int T, int IPL, int RPW, int NT>
__global__ void __launch_bounds__(512) gdec_gateup_kernel(const int32_t *__restrict__ counts,
                                                          const int32_t *__restrict__ offs,
                                                          const int32_t *__restrict__ perm,
                                                          const int32_t *__restrict__ active,
                                                          const void *const *__restrict__ table,
                                                          const float *__restrict__ hb, int d, int fe, int k, int E,
                                                          int nb, int64_t row_bytes, float *__restrict__ h) {
    using F = Reg<T>;
    using Raw = typename F::Raw;
    constexpr int NS = F::NS;
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ow = (blockIdx.x * 8 + wv) * nb * RPW;  // the wave's first row
    if (ow >= fe) return;
    const int nbw = min(nb, (fe - ow + RPW - 1) / RPW);  // batches with rows inside fe
    gbyte *G = gmem(table[3 * e]);
    gbyte *U = gmem(table[3 * e + 1]);
    if (!G || !U) {  // an unregistered expert contributes nothing (src/gguf_run.c:201)
        const int nr = min(nb * RPW, fe - ow);
        for (int i = lane; i < cnt * nr; i += 64) h[size_t(perm[base + i / nr]) * fe + ow + i % nr] = 0.0f;
        return;
    }
    const int items = F::items(d);
    auto fetch = [&](Raw (&rg)[RPW][IPL], Raw (&ru)[RPW][IPL], int bi) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int64_t ro = int64_t(min(ow + bi * RPW + r, fe - 1)) * row_bytes;
#pragma unroll
            for (int m = 0; m < IPL; m++) {
                const int it = lane + 64 * m;
                if (it < items) {
                    rg[r][m] = F::fetch(G, ro, it);
                    ru[r][m] = F::fetch(U, ro, it);
                }
            }
        }
    };
    for (int t0 = 0; t0 < cnt; t0 += NT) {
        const int tn = min(NT, cnt - t0);
        int pr[NT];
        float xr[NT][IPL][32], xs[NT][IPL][NS];
#pragma unroll
        for (int j = 0; j < NT; j++) {
            pr[j] = j < tn ? perm[base + t0 + j] : 0;
            if (j < tn) {
                const float *row = hb + size_t(pr[j] / k) * d;
#pragma unroll
                for (int m = 0; m < IPL; m++) {
                    const int it = lane + 64 * m;
                    if (it < items) {
                        F::load_x(row, it, xr[j][m]);
                        F::sums(xr[j][m], xs[j][m]);
                    }
                }
            }
        }
        auto compute = [&](const Raw (&rg)[RPW][IPL], const Raw (&ru)[RPW][IPL], int bi) {
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const int o = ow + bi * RPW + r;
                Prep<T> pg[IPL], pu[IPL];
#pragma unroll
                for (int m = 0; m < IPL; m++) {
                    const int it = lane + 64 * m;
                    if (it < items) {
                        pg[m].set(F::resolve(rg[r][m], it), it);
                        pu[m].set(F::resolve(ru[r][m], it), it);
                    }
                }
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    if (j >= tn) break;  // the same for the whole wave
                    float g = 0.0f, u = 0.0f;
#pragma unroll
                    for (int m = 0; m < IPL; m++) {
                        const int it = lane + 64 * m;
                        if (it < items) {
                            g += pg[m].dot(xr[j][m], xs[j][m]);
                            u += pu[m].dot(xr[j][m], xs[j][m]);
                        }
                    }
                    g = group_sum<64>(g);
                    u = group_sum<64>(u);
                    if (lane == 63 && o < fe) h[size_t(pr[j]) * fe + o] = swiglu(g, u);
                }
            }
        };
        Raw ga[RPW][IPL], ua[RPW][IPL], gb[RPW][IPL], ub[RPW][IPL];
        fetch(ga, ua, 0);
        for (int bi = 0; bi < nbw; bi += 2) {
            if (bi + 1 < nbw) fetch(gb, ub, bi + 1);
            compute(ga, ua, bi);
            if (bi + 1 >= nbw) break;
            if (bi + 2 < nbw) fetch(ga, ua, bi + 2);
            compute(gb, ub, bi + 1);
        }
    }
}

// down: lane group g (L lanes) of wave w of workgroup (b, s) owns rows
// (((8 b + w) SUB + g) NB + i) RPG + r of down of expert active[s], streamed
// in NB batches as in gdec_gateup_kernel.
template <int T, int L, int IPL, int RPG, int NT>
__global__ void __launch_bounds__(512) gdec_down_kernel(const int32_t *__restrict__ counts,
                                                        const int32_t *__restrict__ offs,
                                                        const int32_t *__restrict__ perm,
                                                        const int32_t *__restrict__ active,
                                                        const void *const *__restrict__ table,
                                                        const float *__restrict__ h, int fe, int d, int E, int nb,
                                                        int64_t row_bytes, float *__restrict__ y) {
    using F = Reg<T>;
    using Raw = typename F::Raw;
    constexpr int NS = F::NS, SUB = 64 / L;
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e];
    gbyte *D = gmem(table[3 * e + 2]);
    if (!D) return;  // the combine skips an unregistered expert (src/gguf_run.c:201)
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, grp = lane / L, li = lane % L;
    const int wfirst = (blockIdx.x * 8 + wv) * SUB * nb * RPG;  // the wave's first row
    if (wfirst >= d) return;
    const int og = wfirst + grp * nb * RPG;  // the lane group's first row (rows past d are not stored)
    const int nbw = nb;
    const int items = F::items(fe);
    auto fetch = [&](Raw (&raw)[RPG][IPL], int bi) {
#pragma unroll
        for (int r = 0; r < RPG; r++) {
            const int64_t ro = int64_t(min(og + bi * RPG + r, d - 1)) * row_bytes;
#pragma unroll
            for (int m = 0; m < IPL; m++) {
                const int it = li + L * m;
                if (it < items) raw[r][m] = F::fetch(D, ro, it);
            }
        }
    };
    for (int t0 = 0; t0 < cnt; t0 += NT) {
        const int tn = min(NT, cnt - t0);
        int pr[NT];
        float xr[NT][IPL][32], xs[NT][IPL][NS];
#pragma unroll
        for (int j = 0; j < NT; j++) {
            pr[j] = j < tn ? perm[base + t0 + j] : 0;
            if (j < tn) {
                const float *row = h + size_t(pr[j]) * fe;
#pragma unroll
                for (int m = 0; m < IPL; m++) {
                    const int it = li + L * m;
                    if (it < items) {
                        F::load_x(row, it, xr[j][m]);
                        F::sums(xr[j][m], xs[j][m]);
                    }
                }
            }
        }
        auto compute = [&](const Raw (&raw)[RPG][IPL], int bi) {
#pragma unroll
            for (int r = 0; r < RPG; r++) {
                const int o = og + bi * RPG + r;
                Prep<T> pw[IPL];
#pragma unroll
                for (int m = 0; m < IPL; m++) {
                    const int it = li + L * m;
                    if (it < items) pw[m].set(F::resolve(raw[r][m], it), it);
                }
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    if (j >= tn) break;  // the same for the whole wave
                    float acc = 0.0f;
#pragma unroll
                    for (int m = 0; m < IPL; m++) {
                        const int it = li + L * m;
                        if (it < items) acc += pw[m].dot(xr[j][m], xs[j][m]);
                    }
                    acc = group_sum<L>(acc);
                    if (li == L - 1 && o < d) y[size_t(pr[j]) * d + o] = acc;
                }
            }
        };
        Raw ra[RPG][IPL], rb[RPG][IPL];
        fetch(ra, 0);
        for (int bi = 0; bi < nbw; bi += 2) {
            if (bi + 1 < nbw) fetch(rb, bi + 1);
            compute(ra, bi);
            if (bi + 1 >= nbw) break;
            if (bi + 2 < nbw) fetch(ra, bi + 2);
            compute(rb, bi + 1);
        }
    }
}

// ---- rows of 2048 inputs (64 items, lane = item): inputs in LDS, weights
// converted once per row
//
// gdec_gateup_wide_kernel: grid (ceil(fe / (4 rpw)), active slots, token
// chunks), 256 threads; wave w of workgroup (b, s, c) computes rows
// (4 b + w) rpw .. + rpw - 1 of gate and up of expert active[s] for tokens
// NT c .. NT c + NT - 1 of its group (so a workgroup's work does not grow
// with the group: a group of many tokens is spread over more workgroups,
// which read its rows again). The tokens' inputs go to LDS in item order (xs[j][c][it] holds inputs
// 4c .. 4c + 3 of item it of token j, so a wave's reads of one c are 64
// consecutive 16-byte words) with the item's run sums (ss[j][g][it]). For each
// row the lane converts its item's 32 quants of gate and of up to fp32 once
// (Hoist), then every token costs one FMA per weight, in four independent
// chains; the row's raw words for the next row are in flight meanwhile.

// An item's quants as floats, with the item's scales: dot(x, s) is the item's
// share of the row . x, as Reg<T>::compute (the same sums, reassociated).
template <int T>
struct Hoist;

template <>
struct Hoist<VT_Q4_K> {  // d1 * sum(q x) - m1 * sum(x) over each of the two runs
    float q[32];
    float d1, m1, d2, m2;
    VH_DEV void set(const Reg<VT_Q4_K>::Words &r, int it) {
        const int c = (it & 7) >> 1;
        const float d = h2f(r.hdr.x & 0xffffu), dmin = h2f(r.hdr.x >> 16);
        int sc0, mn0, sc1, mn1;
        q4k_scale_min(2 * c, r.hdr.y, r.hdr.z, r.hdr.w, sc0, mn0);
        q4k_scale_min(2 * c + 1, r.hdr.y, r.hdr.z, r.hdr.w, sc1, mn1);
        d1 = d * float(sc0);
        m1 = dmin * float(mn0);
        d2 = d * float(sc1);
        m2 = dmin * float(mn1);
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t lo = qw[i] & 0x0f0f0f0fu, hi = (qw[i] >> 4) & 0x0f0f0f0fu;
            asm volatile("" : "+v"(lo), "+v"(hi));  // one v_cvt_f32_ubyte per quant
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[4 * i + k] = float((lo >> (8 * k)) & 0xffu);
                q[16 + 4 * i + k] = float((hi >> (8 * k)) & 0xffu);
            }
        }
    }
    VH_DEV float dot(const float (&x)[32], const float (&s)[2]) const {
        float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a0 = fmaf(q[2 * i], x[2 * i], a0);
            a1 = fmaf(q[2 * i + 1], x[2 * i + 1], a1);
            b0 = fmaf(q[16 + 2 * i], x[16 + 2 * i], b0);
            b1 = fmaf(q[17 + 2 * i], x[17 + 2 * i], b1);
        }
        return d1 * (a0 + a1) - m1 * s[0] + d2 * (b0 + b1) - m2 * s[1];
    }
};

template <>
struct Hoist<VT_Q6_K> {  // d * sum_g sc_g (sum(q x) - 32 sum(x)) over the four runs of 8
    float q[32];
    float sc[4], d;
    VH_DEV void set(const Q6Raw &r, int) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t A = h ? r.a1 : r.a0, B = h ? r.b1 : r.b0, H = h ? r.h1 : r.h0;
            uint32_t t0 = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
            uint32_t t1 = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
            uint32_t t2 = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
            uint32_t t3 = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
            asm volatile("" : "+v"(t0), "+v"(t1), "+v"(t2), "+v"(t3));
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[4 * h + k] = float((t0 >> (8 * k)) & 0xffu);
                q[8 + 4 * h + k] = float((t1 >> (8 * k)) & 0xffu);
                q[16 + 4 * h + k] = float((t2 >> (8 * k)) & 0xffu);
                q[24 + 4 * h + k] = float((t3 >> (8 * k)) & 0xffu);
            }
        }
#pragma unroll
        for (int g = 0; g < 4; g++) sc[g] = float(int(int8_t(r.sc >> (8 * g))));
        d = h2f(r.d);
    }
    VH_DEV float dot(const float (&x)[32], const float (&s)[4]) const {
        float a[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float u = 0.0f, v = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                u = fmaf(q[8 * g + 2 * i], x[8 * g + 2 * i], u);
                v = fmaf(q[8 * g + 2 * i + 1], x[8 * g + 2 * i + 1], v);
            }
            a[g] = fmaf(-32.0f, s[g], u + v);
        }
        return d * fmaf(sc[0], a[0], fmaf(sc[1], a[1], fmaf(sc[2], a[2], sc[3] * a[3])));
    }
};

template <>
struct Hoist<VT_Q8_0> {  // d * sum(q x) over the block's 32 signed bytes
    float q[32];
    float d;
    VH_DEV void set(const Reg<VT_Q8_0>::Words &r, int) {
        d = h2f((r.w[0] >> (8 * r.s)) & 0xffffu);
        const uint32_t sh = 16 + 8 * r.s;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // q + 128 as an unsigned byte (one v_cvt_f32_ubyte each), then - 128: exact
            uint32_t u = uint32_t(((uint64_t(r.w[i + 1]) << 32) | r.w[i]) >> sh) ^ 0x80808080u;
            asm volatile("" : "+v"(u));
#pragma unroll
            for (int k = 0; k < 4; k++) q[4 * i + k] = float((u >> (8 * k)) & 0xffu) - 128.0f;
        }
    }
    VH_DEV float dot(const float (&x)[32], const float (&)[1]) const {
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a0 = fmaf(q[4 * i], x[4 * i], a0);
            a1 = fmaf(q[4 * i + 1], x[4 * i + 1], a1);
            a2 = fmaf(q[4 * i + 2], x[4 * i + 2], a2);
            a3 = fmaf(q[4 * i + 3], x[4 * i + 3], a3);
        }
        return d * ((a0 + a1) + (a2 + a3));
    }
};

constexpr int kWideThreads = 256;

// Inputs of tokens t0 .. t0 + tn - 1 of a group into LDS in item order:
// xs[j][c][it] = inputs 4c .. 4c + 3 of item it of token j (item order of
// Reg<T>), ss[j][g][it] = the item's run sums. Row j of the inputs starts at
// src + rowof(j) * n, n = 32 * items.
template <int T, int NT, int IT, class RowOf>
VH_DEV void stage_inputs(float4 (&xs)[NT][8][IT], float (&ss)[NT][Reg<T>::NS][IT], const float *__restrict__ src,
                         int items, int tn, RowOf rowof) {
    using F = Reg<T>;
    constexpr int NS = F::NS;
    const int n = 32 * items;
    for (int q = threadIdx.x; q < tn * items; q += kWideThreads) {
        const int j = q / items, it = q % items;
        float xv[32], sv[NS];
        F::load_x(src + size_t(rowof(j)) * n, it, xv);
        F::sums(xv, sv);
#pragma unroll
        for (int c = 0; c < 8; c++) xs[j][c][it] = make_float4(xv[4 * c], xv[4 * c + 1], xv[4 * c + 2], xv[4 * c + 3]);
#pragma unroll
        for (int g = 0; g < NS; g++) ss[j][g][it] = sv[g];
    }
}

// The 32 inputs and run sums of item it of token j from LDS
template <int T, int NT, int IT>
VH_DEV void lds_inputs(const float4 (&xs)[NT][8][IT], const float (&ss)[NT][Reg<T>::NS][IT], int j, int it,
                       float (&x)[32], float (&sv)[Reg<T>::NS]) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const float4 v = xs[j][c][it];
        x[4 * c] = v.x;
        x[4 * c + 1] = v.y;
        x[4 * c + 2] = v.z;
        x[4 * c + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < Reg<T>::NS; q++) sv[q] = ss[j][q][it];
}

// Weight words of rows in flight: a ring of PD sets, the loads of row r + PD
// issued right after row r is computed (and PD rows issued before the inputs
// are staged).
template <class Raw, int PD, class Fetch, class Compute>
VH_DEV void row_ring(Raw (&ring)[PD], int nrows, Fetch fetch, Compute compute) {
    for (int r0 = 0; r0 < nrows; r0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; j++) {
            const int r = r0 + j;
            if (r >= nrows) break;
            compute(ring[j], r);
            if (r + PD < nrows) fetch(ring[j], r + PD);
        }
    }
}

// gdec_gateup_wide_kernel (rows of 2048 inputs, lane = item): grid
// (ceil(fe / (4 rpw)), active slots, token chunks), 256 threads; wave w of
// workgroup (b, s, c) computes rows (4 b + w) rpw .. + rpw - 1 of gate and up
// of expert active[s] for tokens NT c .. NT c + NT - 1 of its group (a group
// of many tokens is spread over more workgroups, which read its rows again, so
// no workgroup's work grows with its group). For each row the lane converts
// its item's 32 quants to fp32 once (Hoist), then every token costs one FMA
// per weight, in four independent chains; gate's row sum goes through LDS to
// the up pass, which forms h = silu(gate) * up (src/gguf_run.c:205-207).
template <int T, int NT, int PD>
__global__ void __launch_bounds__(kWideThreads) gdec_gateup_wide_kernel(
    const int32_t *__restrict__ counts, const int32_t *__restrict__ offs, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ active, const void *const *__restrict__ table, const float *__restrict__ hb, int fe,
    int k, int E, int rpw, int64_t row_bytes, float *__restrict__ h) {
    using F = Reg<T>;
    using Raw = typename F::Raw;
    constexpr int NS = F::NS, IT = 64;
    __shared__ float4 xs[NT][8][IT];
    __shared__ float ss[NT][NS][IT];
    __shared__ float gsum[4][NT];
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e], t0 = blockIdx.z * NT;
    if (t0 >= cnt) return;
    const int tn = min(NT, cnt - t0);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ow = (blockIdx.x * 4 + wv) * rpw;  // the wave's first row
    const int nrows = max(0, min(rpw, fe - ow));
    gbyte *G = gmem(table[3 * e]);
    gbyte *U = gmem(table[3 * e + 1]);
    if (!G || !U) {  // an unregistered expert contributes nothing (src/gguf_run.c:201)
        for (int i = lane; i < tn * nrows; i += 64)
            h[size_t(perm[base + t0 + i / nrows]) * fe + ow + i % nrows] = 0.0f;
        return;
    }
    struct Pair {
        Raw g, u;
    };
    auto fetch = [&](Pair &p, int r) {
        const int64_t ro = int64_t(ow + r) * row_bytes;
        p.g = F::fetch(G, ro, lane);
        p.u = F::fetch(U, ro, lane);
    };
    Pair ring[PD];
#pragma unroll
    for (int j = 0; j < PD; j++)
        if (j < nrows) fetch(ring[j], j);
    stage_inputs<T, NT, IT>(xs, ss, hb, IT, tn, [&](int j) { return perm[base + t0 + j] / k; });
    __syncthreads();
    if (nrows == 0) return;
    auto pass = [&](const Raw &raw, int r, bool up) {
        Hoist<T> hq;
        hq.set(F::resolve(raw, lane), lane);
#pragma unroll 1
        for (int j = 0; j < tn; j++) {
            float x[32], sv[NS];
            lds_inputs<T, NT, IT>(xs, ss, j, lane, x, sv);
            const float t = group_sum<64>(hq.dot(x, sv));
            if (lane == 63) {
                if (!up) gsum[wv][j] = t;
                else h[size_t(perm[base + t0 + j]) * fe + ow + r] = swiglu(gsum[wv][j], t);
            }
        }
    };
    row_ring<Pair, PD>(ring, nrows, fetch, [&](const Pair &p, int r) {
        pass(p.g, r, false);
        pass(p.u, r, true);
    });
}

// gdec_down_wide_kernel (rows of at most 1024 inputs): the same scheme with
// half a wave per row (lane & 31 = item, lanes past the row's items idle), two
// rows per step: wave w of workgroup (b, s, c) computes rows
// (4 b + w) rpw .. + rpw - 1 of down of expert active[s] for its token chunk;
// y[pair][o] = down_o . h[pair] (src/gguf_run.c:208), combined afterwards in
// selection order by combine_kernel.
template <int T, int NT, int PD>
__global__ void __launch_bounds__(kWideThreads) gdec_down_wide_kernel(
    const int32_t *__restrict__ counts, const int32_t *__restrict__ offs, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ active, const void *const *__restrict__ table, const float *__restrict__ h, int fe,
    int d, int E, int rpw, int64_t row_bytes, float *__restrict__ y) {
    using F = Reg<T>;
    using Raw = typename F::Raw;
    constexpr int NS = F::NS, IT = 32;
    __shared__ float4 xs[NT][8][IT];
    __shared__ float ss[NT][NS][IT];
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e], t0 = blockIdx.z * NT;
    if (t0 >= cnt) return;
    gbyte *D = gmem(table[3 * e + 2]);
    if (!D) return;  // the combine skips an unregistered expert (src/gguf_run.c:201)
    const int tn = min(NT, cnt - t0), items = F::items(fe);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, half = lane >> 5, li = lane & 31;
    const int ow = (blockIdx.x * 4 + wv) * rpw;  // the wave's first row; rows ow + 2 i + half
    const int nsteps = max(0, (min(rpw, d - ow) + 1) / 2);
    const bool live = li < items;
    auto fetch = [&](Raw &raw, int i) {
        const int64_t ro = int64_t(min(ow + 2 * i + half, d - 1)) * row_bytes;
        if (live) raw = F::fetch(D, ro, li);
    };
    Raw ring[PD];
#pragma unroll
    for (int j = 0; j < PD; j++)
        if (j < nsteps) fetch(ring[j], j);
    stage_inputs<T, NT, IT>(xs, ss, h, items, tn, [&](int j) { return perm[base + t0 + j]; });
    __syncthreads();
    if (nsteps == 0) return;
    row_ring<Raw, PD>(ring, nsteps, fetch, [&](const Raw &raw, int i) {
        const int o = ow + 2 * i + half;
        Hoist<T> hq;
        if (live) hq.set(F::resolve(raw, li), li);
#pragma unroll 1
        for (int j = 0; j < tn; j++) {
            float x[32], sv[NS], v = 0.0f;
            if (live) {
                lds_inputs<T, NT, IT>(xs, ss, j, li, x, sv);
                v = hq.dot(x, sv);
            }
            v = group_sum<32>(v);
            if (li == 31 && o < d && o < ow + rpw) y[size_t(perm[base + t0 + j]) * d + o] = v;
        }
    });
}

constexpr int kWideNT = 4;

// rows per wave: about three workgroups per CU over the call's slots, even, 2..64
int wide_rpw(int rows, int slots) {
    const int64_t want = int64_t(3) * vh_num_cus();
    int64_t rpw = (int64_t(rows) * slots + 4 * want - 1) / (4 * want);
    rpw = (rpw + 1) & ~int64_t(1);
    return int(rpw < 2 ? 2 : rpw > 64 ? 64 : rpw);
}

// register sets of rows in flight (a Q6_K row's words are 13 registers per
// item, Q4_K 8, Q8_0 11): two keep every kernel at 4 waves per SIMD except
// the Q6_K gate/up (3); the Q6_K down kernel measured 104 -> 78 us at Qwen3
// B=32 going from 3 sets (3 waves per SIMD) to 2 (4 waves)
template <int T>
constexpr int wide_pd_gu() { return 2; }
template <int T>
constexpr int wide_pd_down() { return T == VT_Q6_K ? 2 : 4; }

constexpr int kGdecRPW = 2;
// down rows per lane group and batch: Q6_K's decoder needs more registers
template <int T>
constexpr int gdec_rpg() { return T == VT_Q6_K ? 2 : 4; }
// tokens per chunk: what fits the registers next to two batches of raw words
// with one (two) items per lane
template <int T, int IPL>
constexpr int gdec_nt() { return IPL == 1 ? (T == VT_Q4_K ? 4 : 3) : 1; }
// gate/up holds two matrices' rows: one token fewer
template <int T, int IPL>
constexpr int gdec_nt_gu() { return IPL == 1 ? (T == VT_Q4_K ? 3 : 2) : 1; }

// batches per wave: enough rows per workgroup that the expected number of
// workgroups (about min(E, pairs) active experts) is about two per CU
int gdec_batches(int rows, int rows_per_batch_wg, int est_experts) {
    const int64_t want = int64_t(rows) * est_experts / (int64_t(rows_per_batch_wg) * 2 * vh_num_cus());
    return int(want < 1 ? 1 : want > 8 ? 8 : want);
}

template <int T>
int gdec_gateup_t(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                  const void *const *table, const float *hb, int d, int fe, int k, int E, int max_slots, int max_count,
                  float *h, hipStream_t s) {
    if (d == 2048) {  // 64 items: lane = item
        const int rpw = wide_rpw(fe, max_slots);
        const dim3 g((fe + 4 * rpw - 1) / (4 * rpw), max_slots, (max_count + kWideNT - 1) / kWideNT);
        hipLaunchKernelGGL((gdec_gateup_wide_kernel<T, kWideNT, wide_pd_gu<T>()>), g, dim3(kWideThreads), 0, s, counts,
                           offs, perm,
                           active, table, hb, fe, k, E, rpw, vh_row_bytes(T, d), h);
        return vh_check(hipGetLastError());
    }
    const int nb = gdec_batches(fe, 8 * kGdecRPW, max_slots);
    const dim3 g((fe + 8 * kGdecRPW * nb - 1) / (8 * kGdecRPW * nb), max_slots);
    const int64_t rb = vh_row_bytes(T, d);
    hipLaunchKernelGGL((gdec_gateup_kernel<T, 1, kGdecRPW, gdec_nt_gu<T, 1>()>), g, dim3(512), 0, s, counts, offs,
                       perm, active, table, hb, d, fe, k, E, nb, rb, h);
    return vh_check(hipGetLastError());
}

template <int T>
int gdec_down_t(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                const void *const *table, const float *h, int d, int fe, int E, int max_slots, int max_count, float *y,
                hipStream_t s) {
    if (fe <= 1024) {  // at most 32 items per row: half a wave per row
        const int rpw = wide_rpw(d, max_slots);
        const dim3 g((d + 4 * rpw - 1) / (4 * rpw), max_slots, (max_count + kWideNT - 1) / kWideNT);
        hipLaunchKernelGGL((gdec_down_wide_kernel<T, kWideNT, wide_pd_down<T>()>), g, dim3(kWideThreads), 0, s, counts,
                           offs, perm, active, table, h, fe, d, E, rpw, vh_row_bytes(T, fe), y);
        return vh_check(hipGetLastError());
    }
    const int items = fe / 32;
    int L = 8;
    while (L < items && L < 64) L *= 2;
    const int rows_per_batch = 8 * (64 / L) * gdec_rpg<T>();
    const int nb = gdec_batches(d, rows_per_batch, max_slots);
    const dim3 g((d + rows_per_batch * nb - 1) / (rows_per_batch * nb), max_slots);
    const int64_t rb = vh_row_bytes(T, fe);
#define VH_GDEC_DOWN(LL, II)                                                                                    \
    hipLaunchKernelGGL((gdec_down_kernel<T, LL, II, gdec_rpg<T>(), gdec_nt<T, II>()>), g, dim3(512), 0, s,    \
                       counts,                                                                              \
                       offs, perm, active, table, h, fe, d, E, nb, rb, y)
    switch (L) {
    case 8: VH_GDEC_DOWN(8, 1); break;
    case 16: VH_GDEC_DOWN(16, 1); break;
    case 32: VH_GDEC_DOWN(32, 1); break;
    default: VH_GDEC_DOWN(64, 1); break;
    }
#undef VH_GDEC_DOWN
    return vh_check(hipGetLastError());
}

}  // namespace

bool vh_gdec_supported(uint32_t tg, uint32_t td, int d, int fe, const float *hb) {
    auto ok = [](uint32_t t, int n) {
        return (t == VT_Q8_0 && n % 32 == 0) || ((t == VT_Q4_K || t == VT_Q6_K) && n % 256 == 0);
    };
    // one item per lane: rows of at most 64 items (2048 weights)
    return ok(tg, d) && ok(td, fe) && d / 32 <= 64 && fe / 32 <= 64 && !(reinterpret_cast<uintptr_t>(hb) & 15u);
}

int vh_gdec_gateup(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                   const int32_t *active, const void *const *table, const float *hb, int d, int fe, int k, int E,
                   int max_slots, int max_count, float *h, hipStream_t s) {
    if (max_count < 1 || max_count > 65535 * kWideNT) return -EINVAL;
    switch (type) {
    case VT_Q8_0:
        return gdec_gateup_t<VT_Q8_0>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, max_count, h, s);
    case VT_Q4_K:
        return gdec_gateup_t<VT_Q4_K>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, max_count, h, s);
    case VT_Q6_K:
        return gdec_gateup_t<VT_Q6_K>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, max_count, h, s);
    default: return -EINVAL;
    }
}

int vh_gdec_down(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                 const int32_t *active, const void *const *table, const float *h, int d, int fe, int E, int max_slots,
                 int max_count, float *ybuf, hipStream_t s) {
    if (max_count < 1 || max_count > 65535 * kWideNT) return -EINVAL;
    switch (type) {
    case VT_Q8_0:
        return gdec_down_t<VT_Q8_0>(counts, offs, perm, active, table, h, d, fe, E, max_slots, max_count, ybuf, s);
    case VT_Q4_K:
        return gdec_down_t<VT_Q4_K>(counts, offs, perm, active, table, h, d, fe, E, max_slots, max_count, ybuf, s);
    case VT_Q6_K:
        return gdec_down_t<VT_Q6_K>(counts, offs, perm, active, table, h, d, fe, E, max_slots, max_count, ybuf, s);
    default: return -EINVAL;
    }
}
