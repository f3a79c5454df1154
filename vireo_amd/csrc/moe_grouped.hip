// Grouped expert path for many tokens (batched decode, prefill).
//
// dispatch   buckets the T*k (token, slot) pairs by expert: counts, offsets,
//            perm sorted by (expert, token), and the list of experts that got
//            at least one token. The reference has no counterpart: it runs
//            tokens one at a time (src/gguf_run.c:367-368).
// gateup     one workgroup per (active expert, row block): each weight item is
//            decoded once into registers and applied to every token of the
//            expert (token rows staged in LDS), so expert weights are read once
//            per call instead of once per token.
// down       the same for the down projection; writes y[pair][o].
// combine    x[t][o] += sum_j w[t][j] * y[t*k+j][o] in selection order
//            (src/gguf_run.c:209,213); one writer per element, no atomics.
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route_kernels.h"

namespace {

constexpr int kDispWaves = 16;

// One workgroup of 16 waves (see moe_dispatch in include/vireo_hip.h).
__global__ void __launch_bounds__(1024) dispatch_kernel(const int32_t *__restrict__ idx, int P, int E,
                                                        int32_t *__restrict__ counts, int32_t *__restrict__ offs,
                                                        int32_t *__restrict__ perm, int32_t *__restrict__ active) {
    __shared__ int hist[kMaxExperts][kDispWaves];
    __shared__ int tot[kMaxExperts + 1];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < kMaxExperts * kDispWaves; i += blockDim.x) hist[i / kDispWaves][i % kDispWaves] = 0;
    __syncthreads();
    const int seg = (P + kDispWaves - 1) / kDispWaves;
    const int p0 = min(P, wv * seg), p1 = min(P, p0 + seg);
    for (int p = p0 + lane; p < p1; p += 64) {
        const int e = idx[p];
        if (e >= 0 && e < E) atomicAdd(&hist[e][wv], 1);  // counts only: order-free
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0, na = 0;
        for (int e = 0; e < E; e++) {
            tot[e] = run;
            int ce = 0;
            for (int s = 0; s < kDispWaves; s++) { const int c = hist[e][s]; hist[e][s] = run + ce; ce += c; }
            run += ce;
            if (active && ce > 0) active[na++] = e;
        }
        tot[E] = run;
        if (active) active[E] = na;  // number of active experts
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        counts[e] = tot[e + 1] - tot[e];
        offs[e] = tot[e];
    }
    if (threadIdx.x == 0) offs[E] = tot[E];
    // hist[e][wv] is now this segment's first slot in bucket e; lanes that share
    // an expert take consecutive slots by their rank in the 64-pair chunk.
    for (int pb = p0; pb < p1; pb += 64) {
        const int p = pb + lane;
        int e = p < p1 ? idx[p] : -1;
        if (e < 0 || e >= E) e = -1;
        uint64_t pending = __ballot(e >= 0);
        while (pending) {
            const int leader = __ffsll((unsigned long long)pending) - 1;
            const int el = __shfl(e, leader, 64);
            const uint64_t grp = __ballot(e == el) & pending;
            if ((grp >> lane) & 1ull) perm[hist[el][wv] + __popcll(grp & ((1ull << lane) - 1ull))] = p;
            if (lane == leader) hist[el][wv] += __popcll(grp);
            pending &= ~grp;
        }
    }
}

// ------------------------------------------------------------ item dequant
// An item of a row dequantized to NW floats in natural column order; col0 is
// the column of the first one. Q4_K and Q6_K items cover two / four runs of
// columns (see qdecode.h); they are split into 16- / 8-column segments.
template <int T, bool PAIRED>
struct Items {
    static constexpr int NW = (T == VT_Q8_0 && PAIRED) ? 64 : 32;
    static constexpr int SEG = T == VT_Q4_K ? 16 : T == VT_Q6_K ? 8 : NW;  // columns per contiguous run
    static constexpr int STRIDE = T == VT_Q4_K ? 32 : T == VT_Q6_K ? 32 : 0;  // column step between runs
    static __host__ __device__ int items(int n) { return T == VT_Q8_0 && PAIRED ? n / 64 : n / 32; }
    static VH_DEV int col0(int it) {
        if constexpr (T == VT_Q4_K) { const int sb = it >> 3, r = it & 7; return 256 * sb + 64 * (r >> 1) + 16 * (r & 1); }
        else if constexpr (T == VT_Q6_K) { const int sb = it >> 3, r = it & 7; return 256 * sb + 128 * (r >> 2) + 8 * (r & 3); }
        else return NW * it;
    }
    // item `it` of the row at byte offset `row` of the 4-aligned tensor `base`
    static VH_DEV void deq(const uint8_t *base, int64_t row, int it, float *wv) {
        if constexpr (T == VT_Q8_0 && PAIRED) {
            const uint8_t *p = base + row + 68 * it;
            uint32_t w[17];
#pragma unroll
            for (int i = 0; i < 17; i++) w[i] = ld_u32(p + 4 * i);
            const float d0 = h2f(w[0] & 0xffffu), d1 = h2f(w[8] >> 16);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t q0 = align2(w[i + 1], w[i], 2), q1 = w[9 + i];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    wv[4 * i + k] = float(int(int8_t(q0 >> (8 * k)))) * d0;
                    wv[32 + 4 * i + k] = float(int(int8_t(q1 >> (8 * k)))) * d1;
                }
            }
        } else if constexpr (T == VT_Q8_0) {
            const uint8_t *b = base + row + 34 * it;  // even address
            const float d = h2f(ld_u16(b));
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t two = ld_u16(b + 2 + 2 * i);
                wv[2 * i] = float(int(int8_t(two))) * d;
                wv[2 * i + 1] = float(int(int8_t(two >> 8))) * d;
            }
        } else if constexpr (T == VT_Q4_K) {
            const int sbi = it >> 3, r = it & 7, c = r >> 1, h = r & 1;
            const uint8_t *sb = base + row + 144 * sbi;
            const uint4 hdr = *reinterpret_cast<const uint4 *>(sb);
            const uint4 q = *reinterpret_cast<const uint4 *>(sb + 16 + 32 * c + 16 * h);
            const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
            int sc0, m0, sc1, m1;
            q4k_scale_min(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
            q4k_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
            const float d1 = d * float(sc0), mm1 = dmin * float(m0), d2 = d * float(sc1), mm2 = dmin * float(m1);
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t b = (qw[i >> 2] >> (8 * (i & 3))) & 0xffu;
                wv[i] = d1 * float(b & 15u) - mm1;
                wv[16 + i] = d2 * float(b >> 4) - mm2;
            }
        } else if constexpr (T == VT_Q6_K) {
            const int sbi = it >> 3, r = it & 7;
            const Q6Raw q = q6k_fetch(base, row + 210 * sbi, r >> 2, r & 3);
            const float d = h2f(q.d);
            float ds[4];
#pragma unroll
            for (int g = 0; g < 4; g++) ds[g] = d * float(int(int8_t(q.sc >> (8 * g))));
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t qa = ((i < 4 ? q.a0 : q.a1) >> (8 * (i & 3))) & 0xffu;
                const uint32_t qb = ((i < 4 ? q.b0 : q.b1) >> (8 * (i & 3))) & 0xffu;
                const uint32_t qh = ((i < 4 ? q.h0 : q.h1) >> (8 * (i & 3))) & 0xffu;
                wv[i] = ds[0] * float(int((qa & 15u) | ((qh & 3u) << 4)) - 32);
                wv[8 + i] = ds[1] * float(int((qb & 15u) | (((qh >> 2) & 3u) << 4)) - 32);
                wv[16 + i] = ds[2] * float(int((qa >> 4) | (((qh >> 4) & 3u) << 4)) - 32);
                wv[24 + i] = ds[3] * float(int((qb >> 4) | (((qh >> 6) & 3u) << 4)) - 32);
            }
        } else {  // Q5_0
            const uint8_t *b = base + row + 22 * it;  // even address
            const float d = h2f(ld_u16(b));
            const uint32_t qh = ld_u16(b + 2) | (ld_u16(b + 4) << 16);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t qs = (ld_u16(b + 6 + 2 * (j / 2)) >> (8 * (j & 1))) & 0xffu;
                wv[j] = float(int((qs & 15u) | (((qh >> j) & 1u) << 4)) - 16) * d;
                wv[j + 16] = float(int((qs >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16) * d;
            }
        }
    }
    // dot of a dequantized item with a row x (LDS or global)
    static VH_DEV float dot(const float *wv, int c0, const float *x) {
        float acc = 0.0f;
        if constexpr (SEG == NW) {
#pragma unroll
            for (int i = 0; i < NW; i++) acc = fmaf(wv[i], x[c0 + i], acc);
        } else {
#pragma unroll
            for (int s = 0; s < NW / SEG; s++)
#pragma unroll
                for (int i = 0; i < SEG; i++) acc = fmaf(wv[s * SEG + i], x[c0 + s * STRIDE + i], acc);
        }
        return acc;
    }
};

int64_t rbytes(uint32_t t, int n) {
    switch (t) {
    case VT_Q8_0: return int64_t(n / 32) * 34;
    case VT_Q4_K: return int64_t(n / 256) * 144;
    case VT_Q6_K: return int64_t(n / 256) * 210;
    default: return int64_t(n / 32) * 22;  // Q5_0
    }
}

constexpr int kTokTile = 8;   // tokens staged per pass
constexpr int kGuRows = 16;   // gate/up rows per workgroup (4 per wave)

// grid (ceil(fe / kGuRows), max_slots), 256 threads. A row is split over L
// lanes (L = items per row rounded down to a power of two, <= 64).
template <int T, bool PAIRED, int L>
__global__ void __launch_bounds__(256) grouped_gateup_kernel(const int32_t *__restrict__ counts,
                                                             const int32_t *__restrict__ offs,
                                                             const int32_t *__restrict__ perm,
                                                             const int32_t *__restrict__ active,
                                                             const void *const *__restrict__ table,
                                                             const float *__restrict__ hb, int d, int fe, int k, int E,
                                                             int64_t row_bytes, float *__restrict__ h) {
    using I = Items<T, PAIRED>;
    extern __shared__ float xs[];  // [kTokTile][d]
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e];
    const uint8_t *G = static_cast<const uint8_t *>(table[3 * e]);
    const uint8_t *U = static_cast<const uint8_t *>(table[3 * e + 1]);
    constexpr int RPW = 64 / L;  // rows per wave per step
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, sub = lane / L, li = lane % L;
    const int items = I::items(d);
    for (int t0 = 0; t0 < cnt; t0 += kTokTile) {
        const int tn = min(kTokTile, cnt - t0);
        __syncthreads();
        for (int i = threadIdx.x; i < tn * d; i += 256) {
            const int tt = i / d, c = i % d;
            xs[i] = hb[size_t(perm[base + t0 + tt] / k) * d + c];
        }
        __syncthreads();
        for (int ob = blockIdx.x * kGuRows + wv * RPW; ob < min(fe, (blockIdx.x + 1) * kGuRows); ob += 4 * RPW) {
            const int o = ob + sub;
            const bool ok = o < fe && G && U;
            float ag[kTokTile], au[kTokTile];
#pragma unroll
            for (int tt = 0; tt < kTokTile; tt++) ag[tt] = au[tt] = 0.0f;
            if (ok) {
                for (int it = li; it < items; it += L) {
                    float wg[I::NW], wu[I::NW];
                    I::deq(G, int64_t(o) * row_bytes, it, wg);
                    I::deq(U, int64_t(o) * row_bytes, it, wu);
                    const int c0 = I::col0(it);
#pragma unroll
                    for (int tt = 0; tt < kTokTile; tt++) {
                        if (tt < tn) {
                            ag[tt] += I::dot(wg, c0, xs + tt * d);
                            au[tt] += I::dot(wu, c0, xs + tt * d);
                        }
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < kTokTile; tt++) {
                const float g = group_sum<L>(ag[tt]), u = group_sum<L>(au[tt]);
                if (li == L - 1 && o < fe && tt < tn) h[size_t(perm[base + t0 + tt]) * fe + o] = ok ? swiglu(g, u) : 0.0f;
            }
        }
    }
}

// grid (d / kDnRows, max_slots), 256 threads: rows of the down matrix of one
// expert against the activations of its tokens.
constexpr int kDnRows = 16;
template <int T, bool PAIRED, int L>
__global__ void __launch_bounds__(256) grouped_down_kernel(const int32_t *__restrict__ counts,
                                                           const int32_t *__restrict__ offs,
                                                           const int32_t *__restrict__ perm,
                                                           const int32_t *__restrict__ active,
                                                           const void *const *__restrict__ table,
                                                           const float *__restrict__ h, int d, int fe, int E,
                                                           int64_t row_bytes, float *__restrict__ ybuf) {
    using I = Items<T, PAIRED>;
    extern __shared__ float hs[];  // [kTokTile][fe]
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e];
    const uint8_t *D = static_cast<const uint8_t *>(table[3 * e + 2]);
    constexpr int RPW = 64 / L;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, sub = lane / L, li = lane % L;
    const int items = I::items(fe);
    for (int t0 = 0; t0 < cnt; t0 += kTokTile) {
        const int tn = min(kTokTile, cnt - t0);
        __syncthreads();
        for (int i = threadIdx.x; i < tn * fe; i += 256) {
            const int tt = i / fe, c = i % fe;
            hs[i] = h[size_t(perm[base + t0 + tt]) * fe + c];
        }
        __syncthreads();
        for (int ob = blockIdx.x * kDnRows + wv * RPW; ob < min(d, (blockIdx.x + 1) * kDnRows); ob += 4 * RPW) {
            const int o = ob + sub;
            const bool ok = o < d && D;
            float ay[kTokTile];
#pragma unroll
            for (int tt = 0; tt < kTokTile; tt++) ay[tt] = 0.0f;
            if (ok) {
                for (int it = li; it < items; it += L) {
                    float wd[I::NW];
                    I::deq(D, int64_t(o) * row_bytes, it, wd);
                    const int c0 = I::col0(it);
#pragma unroll
                    for (int tt = 0; tt < kTokTile; tt++)
                        if (tt < tn) ay[tt] += I::dot(wd, c0, hs + tt * fe);
                }
            }
#pragma unroll
            for (int tt = 0; tt < kTokTile; tt++) {
                const float y = group_sum<L>(ay[tt]);
                if (li == L - 1 && o < d && tt < tn) ybuf[size_t(perm[base + t0 + tt]) * d + o] = ok ? y : 0.0f;
            }
        }
    }
}

__global__ void __launch_bounds__(256) combine_kernel(const int32_t *__restrict__ idx, const float *__restrict__ w,
                                                      const void *const *__restrict__ table,
                                                      const float *__restrict__ ybuf, int d, int k,
                                                      float *__restrict__ x) {
    const int t = blockIdx.y;
    const int o = blockIdx.x * 256 + threadIdx.x;
    if (o >= d) return;
    float a = 0.0f;
    for (int j = 0; j < k; j++) {
        const int e = idx[size_t(t) * k + j];
        if (e < 0 || !table[3 * e + 2]) continue;  // failed lookup: skipped (src/gguf_run.c:201)
        a = __fadd_rn(a, __fmul_rn(w[size_t(t) * k + j], ybuf[(size_t(t) * k + j) * d + o]));
    }
    x[size_t(t) * d + o] = __fadd_rn(x[size_t(t) * d + o], a);
}

int lanes_for(int items) {
    int L = 64;
    while (L > 1 && L > items) L >>= 1;
    return L;
}

template <int T, bool PAIRED>
int gu_launch(int L, dim3 g, size_t lds, hipStream_t s, const int32_t *counts, const int32_t *offs,
              const int32_t *perm, const int32_t *active, const void *const *table, const float *hb, int d, int fe,
              int k, int E, int64_t rb, float *h) {
    switch (L) {
    case 64: hipLaunchKernelGGL((grouped_gateup_kernel<T, PAIRED, 64>), g, dim3(256), lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h); break;
    case 32: hipLaunchKernelGGL((grouped_gateup_kernel<T, PAIRED, 32>), g, dim3(256), lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h); break;
    case 16: hipLaunchKernelGGL((grouped_gateup_kernel<T, PAIRED, 16>), g, dim3(256), lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h); break;
    case 8: hipLaunchKernelGGL((grouped_gateup_kernel<T, PAIRED, 8>), g, dim3(256), lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h); break;
    default: hipLaunchKernelGGL((grouped_gateup_kernel<T, PAIRED, 4>), g, dim3(256), lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h); break;
    }
    return vh_check(hipGetLastError());
}

template <int T, bool PAIRED>
int dn_launch(int L, dim3 g, size_t lds, hipStream_t s, const int32_t *counts, const int32_t *offs,
              const int32_t *perm, const int32_t *active, const void *const *table, const float *h, int d, int fe,
              int E, int64_t rb, float *ybuf) {
    switch (L) {
    case 64: hipLaunchKernelGGL((grouped_down_kernel<T, PAIRED, 64>), g, dim3(256), lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf); break;
    case 32: hipLaunchKernelGGL((grouped_down_kernel<T, PAIRED, 32>), g, dim3(256), lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf); break;
    case 16: hipLaunchKernelGGL((grouped_down_kernel<T, PAIRED, 16>), g, dim3(256), lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf); break;
    case 8: hipLaunchKernelGGL((grouped_down_kernel<T, PAIRED, 8>), g, dim3(256), lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf); break;
    default: hipLaunchKernelGGL((grouped_down_kernel<T, PAIRED, 4>), g, dim3(256), lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf); break;
    }
    return vh_check(hipGetLastError());
}

}  // namespace

int vh_dispatch(const int32_t *idx, int P, int E, int32_t *counts, int32_t *offs, int32_t *perm, int32_t *active,
                hipStream_t s) {
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, idx, P, E, counts, offs, perm, active);
    return vh_check(hipGetLastError());
}

int vh_grouped_gateup(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                      const int32_t *active, const void *const *table, const float *hb, int d, int fe, int k, int E,
                      int max_slots, float *h, hipStream_t s) {
    const int64_t rb = rbytes(type, d);
    dim3 g((fe + kGuRows - 1) / kGuRows, max_slots);
    const size_t lds = size_t(kTokTile) * d * 4;
    switch (type) {
    case VT_Q8_0:
        if (d % 64 == 0) return gu_launch<VT_Q8_0, true>(lanes_for(d / 64), g, lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h);
        return gu_launch<VT_Q8_0, false>(lanes_for(d / 32), g, lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h);
    case VT_Q4_K: return gu_launch<VT_Q4_K, false>(lanes_for(d / 32), g, lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h);
    case VT_Q6_K: return gu_launch<VT_Q6_K, false>(lanes_for(d / 32), g, lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h);
    case VT_Q5_0: return gu_launch<VT_Q5_0, false>(lanes_for(d / 32), g, lds, s, counts, offs, perm, active, table, hb, d, fe, k, E, rb, h);
    default: return -EINVAL;
    }
}

int vh_grouped_down(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                    const int32_t *active, const void *const *table, const float *h, int d, int fe, int E,
                    int max_slots, float *ybuf, hipStream_t s) {
    const int64_t rb = rbytes(type, fe);
    dim3 g((d + kDnRows - 1) / kDnRows, max_slots);
    const size_t lds = size_t(kTokTile) * fe * 4;
    switch (type) {
    case VT_Q8_0:
        if (fe % 64 == 0) return dn_launch<VT_Q8_0, true>(lanes_for(fe / 64), g, lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf);
        return dn_launch<VT_Q8_0, false>(lanes_for(fe / 32), g, lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf);
    case VT_Q4_K: return dn_launch<VT_Q4_K, false>(lanes_for(fe / 32), g, lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf);
    case VT_Q6_K: return dn_launch<VT_Q6_K, false>(lanes_for(fe / 32), g, lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf);
    case VT_Q5_0: return dn_launch<VT_Q5_0, false>(lanes_for(fe / 32), g, lds, s, counts, offs, perm, active, table, h, d, fe, E, rb, ybuf);
    default: return -EINVAL;
    }
}

int vh_combine(const int32_t *idx, const float *w, const void *const *table, const float *ybuf, int d, int k, int T,
               float *x, hipStream_t s) {
    dim3 g((d + 255) / 256, T);
    hipLaunchKernelGGL(combine_kernel, g, dim3(256), 0, s, idx, w, table, ybuf, d, k, x);
    return vh_check(hipGetLastError());
}
