// Grouped expert path for many tokens (batched decode, prefill).
//
// dispatch   buckets the T*k (token, slot) pairs by expert: counts, offsets,
//            perm sorted by (expert, token), and the list of experts that got
//            at least one token. The reference has no counterpart: it runs
//            tokens one at a time (src/gguf_run.c:367-368).
// gateup     one workgroup per (active expert, row block): each weight item is
//            read once into registers, dequantized once per chunk of tokens
//            and applied to every token of the expert (token rows staged in
//            LDS), so expert weights are read once per call, not per token.
// down       the same for the down projection; writes y[pair][o].
// combine    x[t][o] += sum_j w[t][j] * y[t*k+j][o] in selection order
//            (src/gguf_run.c:209,213); one writer per element, no atomics.
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route_kernels.h"

namespace {

constexpr int kDispWaves = 16;
// up to this many pairs one workgroup dispatches (one launch, shorter); above,
// the two-kernel form with a workgroup per expert
constexpr int kDispatchOneBlock = 2048;

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
    // exclusive scan in (expert, segment) order: thread e < E turns its row of
    // segment counts into prefixes, then a block scan over the expert totals
    // (and over "has tokens", for the list of active experts) adds the offsets
    __shared__ int wsum[kDispWaves][2];
    const int t = threadIdx.x;
    int ce = 0;
    if (t < E) {
        for (int s = 0; s < kDispWaves; s++) {
            const int c = hist[t][s];
            hist[t][s] = ce;
            ce += c;
        }
    }
    const int a = (t < E && ce > 0) ? 1 : 0;
    int ic = ce, ia = a;  // inclusive wave scans (row_shr steps, then across rows)
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        const int oc = __shfl_up(ic, sh, 64), oa = __shfl_up(ia, sh, 64);
        if (lane >= sh) { ic += oc; ia += oa; }
    }
    if (lane == 63) { wsum[wv][0] = ic; wsum[wv][1] = ia; }
    __syncthreads();
    int bc = 0, ba = 0;
    for (int w2 = 0; w2 < wv; w2++) { bc += wsum[w2][0]; ba += wsum[w2][1]; }
    const int ex_c = bc + ic - ce, ex_a = ba + ia - a;
    if (t < E) {
        tot[t] = ex_c;
        for (int s = 0; s < kDispWaves; s++) hist[t][s] += ex_c;
        if (active && a) active[ex_a] = t;
    }
    if (t == E - 1) {
        tot[E] = ex_c + ce;
        if (active) active[E] = ex_a + a;  // number of active experts
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

int64_t rbytes(uint32_t t, int n) { return vh_row_bytes(t, n); }

// Large calls: one workgroup per expert, twice. dispatch_count_kernel counts
// the pairs of expert blockIdx.x; dispatch_place_kernel sums the counts of the
// experts before it (its bucket offset and its rank among the non-empty
// experts) and writes its pairs in pair order: blocks of 16 consecutive pairs
// per thread, a block scan of the per-thread matches giving each its slot.
constexpr int kPlacePer = 16;

VH_DEV int block_excl_scan(int v, int &total, int (&wsum)[4]) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        const int o = __shfl_up(inc, sh, 64);
        if (lane >= sh) inc += o;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        before += w < wv ? wsum[w] : 0;
        total += wsum[w];
    }
    __syncthreads();  // wsum is reused by the next call
    return before + inc - v;
}

__global__ void __launch_bounds__(256) dispatch_count_kernel(const int32_t *__restrict__ idx, int P,
                                                             int32_t *__restrict__ counts) {
    __shared__ int wsum[4];
    const int e = blockIdx.x;
    int c = 0;
#pragma unroll 16  // independent loads in flight together
    for (int p = threadIdx.x; p < P; p += 256) c += idx[p] == e ? 1 : 0;
    int total;
    block_excl_scan(c, total, wsum);
    if (threadIdx.x == 0) counts[e] = total;
}

__global__ void __launch_bounds__(256) dispatch_place_kernel(const int32_t *__restrict__ idx, int P, int E,
                                                             const int32_t *__restrict__ counts,
                                                             int32_t *__restrict__ offs, int32_t *__restrict__ perm,
                                                             int32_t *__restrict__ active) {
    __shared__ int wsum[4];
    const int e = blockIdx.x, tid = threadIdx.x;
    int o = 0, a = 0;
    for (int i = tid; i < e; i += 256) {
        const int c = counts[i];
        o += c;
        a += c > 0 ? 1 : 0;
    }
    int base, rank;
    block_excl_scan(o, base, wsum);
    block_excl_scan(a, rank, wsum);
    const int mine = counts[e];
    if (tid == 0) {
        offs[e] = base;
        if (active && mine > 0) active[rank] = e;
        if (e == E - 1) {
            offs[E] = base + mine;
            if (active) active[E] = rank + (mine > 0 ? 1 : 0);
        }
    }
    int run = base;
    const bool al16 = (reinterpret_cast<uintptr_t>(idx) & 15u) == 0;
    for (int p0 = 0; p0 < P; p0 += 256 * kPlacePer) {
        const int q0 = p0 + kPlacePer * tid;
        uint32_t hit = 0;
        if (q0 + kPlacePer <= P && al16) {  // four 16-byte loads (q0 is a multiple of 16)
            const int4 *q4 = reinterpret_cast<const int4 *>(idx + q0);
#pragma unroll
            for (int j = 0; j < kPlacePer / 4; j++) {
                const int4 v = q4[j];
                hit |= uint32_t(v.x == e) << (4 * j) | uint32_t(v.y == e) << (4 * j + 1) |
                       uint32_t(v.z == e) << (4 * j + 2) | uint32_t(v.w == e) << (4 * j + 3);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kPlacePer; j++)
                if (q0 + j < P && idx[q0 + j] == e) hit |= 1u << j;
        }
        int total;
        int pos = run + block_excl_scan(__popc(hit), total, wsum);
        while (hit) {
            const int j = __ffs(hit) - 1;
            perm[pos++] = q0 + j;
            hit &= hit - 1u;
        }
        run += total;
    }
}

// One launch for large calls (P % 4 == 0, idx 16-byte aligned, P at most
// kFusedChunks * kFusedChunk pairs): workgroup e reads every pair's expert
// once - a group of four 4096-pair chunks' loads issued before any is used -
// and counts the pairs of experts below e (its bucket offset) and its own
// (its count, and which of its 16 consecutive pairs per thread match, kept in
// LDS); with `active`, it also marks in LDS the experts seen (its rank among
// the non-empty experts). Then it writes its pairs in pair order as
// dispatch_place_kernel does, four chunks per block scan. The same counts,
// offsets, order and list as the two-kernel form.
constexpr int kFusedThreads = 256, kFusedChunk = kFusedThreads * kPlacePer, kFusedChunks = 32;

// Exclusive block scan (kFusedThreads threads) of N values at once: before[i]
// = the sum of v[i] over the threads below, total[i] = over all. Two barriers.
template <int N>
VH_DEV void block_excl_scan_n(const int (&v)[N], int (&before)[N], int (&total)[N],
                              int (&wsum)[kFusedThreads / 64][N]) {
    constexpr int W = kFusedThreads / 64;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int inc[N];
#pragma unroll
    for (int i = 0; i < N; i++) inc[i] = v[i];
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1)
#pragma unroll
        for (int i = 0; i < N; i++) {
            const int o = __shfl_up(inc[i], sh, 64);
            if (lane >= sh) inc[i] += o;
        }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < N; i++) wsum[wv][i] = inc[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; i++) {
        int b = 0, t = 0;
#pragma unroll
        for (int w = 0; w < W; w++) {
            b += w < wv ? wsum[w][i] : 0;
            t += wsum[w][i];
        }
        before[i] = b + inc[i] - v[i];
        total[i] = t;
    }
    __syncthreads();  // wsum is reused by the next call
}

__global__ void __launch_bounds__(kFusedThreads) dispatch_fused_kernel(const int32_t *__restrict__ idx, int P, int E,
                                                                       int32_t *__restrict__ counts,
                                                                       int32_t *__restrict__ offs,
                                                                       int32_t *__restrict__ perm,
                                                                       int32_t *__restrict__ active) {
    constexpr int W = kFusedThreads / 64;
    static_assert(kFusedThreads == kMaxExperts, "one thread per expert clears seen[]");
    __shared__ uint32_t hits[kFusedChunks][kFusedThreads];
    __shared__ int seen[kMaxExperts];
    __shared__ int wsum3[W][3], wsum[W][4];
    const int e = blockIdx.x, tid = threadIdx.x;
    const bool list = active != nullptr;
    if (list) seen[tid] = 0;  // kFusedThreads == kMaxExperts
    __syncthreads();
    const int nch = (P + kFusedChunk - 1) / kFusedChunk, P4 = P / 4;
    const int4 *idx4 = reinterpret_cast<const int4 *>(idx);
    int below = 0, mine = 0;
    for (int c0 = 0; c0 < nch; c0 += 4) {
        // four chunks' loads first (unconditional: past the end the last
        // pairs again, masked below)
        int4 v[4][kPlacePer / 4];
#pragma unroll
        for (int cc = 0; cc < 4; cc++)
#pragma unroll
            for (int j = 0; j < kPlacePer / 4; j++)
                v[cc][j] = idx4[min(((c0 + cc) * kFusedChunk + kPlacePer * tid) / 4 + j, P4 - 1)];
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const int q0 = (c0 + cc) * kFusedChunk + kPlacePer * tid;
            const bool whole = q0 + kPlacePer <= P;  // every pair of the thread's 16 exists
            uint32_t hit = 0;
#pragma unroll
            for (int j = 0; j < kPlacePer; j++) {
                const int4 w4 = v[cc][j / 4];
                const int x = (j & 3) == 0 ? w4.x : (j & 3) == 1 ? w4.y : (j & 3) == 2 ? w4.z : w4.w;
                const bool in = whole || q0 + j < P;
                // an expert id outside [0, E) belongs to no bucket: as unsigned it
                // is at least E, so neither below e nor e
                below += in && uint32_t(x) < uint32_t(e) ? 1 : 0;
                hit |= uint32_t(in && x == e) << j;
                if (list && in && uint32_t(x) < uint32_t(E)) seen[x] = 1;
            }
            mine += __popc(hit);
            if (c0 + cc < nch) hits[c0 + cc][tid] = hit;
        }
    }
    __syncthreads();  // seen[] and hits[] complete
    const int v3[3] = {below, mine, list && tid < e ? seen[tid] : 0};
    int b3[3], t3[3];
    block_excl_scan_n<3>(v3, b3, t3, wsum3);
    const int base = t3[0], count = t3[1], rank = t3[2];
    if (tid == 0) {
        counts[e] = count;
        offs[e] = base;
        if (list && count > 0) active[rank] = e;
        if (e == E - 1) {
            offs[E] = base + count;
            if (list) active[E] = rank + (count > 0 ? 1 : 0);
        }
    }
    int run = base;
    for (int c0 = 0; c0 < nch; c0 += 4) {
        uint32_t hit[4];
        int pc[4], before[4], total[4];
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            hit[cc] = c0 + cc < nch ? hits[c0 + cc][tid] : 0u;
            pc[cc] = __popc(hit[cc]);
        }
        block_excl_scan_n<4>(pc, before, total, wsum);
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            int pos = run + before[cc];
            const int q0 = (c0 + cc) * kFusedChunk + kPlacePer * tid;
            uint32_t h = hit[cc];
            while (h) {
                const int j = __ffs(h) - 1;
                perm[pos++] = q0 + j;
                h &= h - 1u;
            }
            run += total[cc];
        }
    }
}

// ------------------------------------------------------------ grouped projections
// An item's 32 weights dequantized from the resolved words of Reg<T>::fetch, in the
// item's own order (the order Reg<T>::load_x gives the inputs): every value is
// the reference's dequantized weight (src/gguf_compute.c:52-103, 112-120).
template <int T>
VH_DEV void deq_raw(const typename Reg<T>::Words &r, float (&w)[32]) {
    if constexpr (T == VT_Q4_K) {
        // the item's two sub-blocks: c = it/2 % 4 is not in the raw words, so
        // the caller passes the scale pair through deq_q4k below
    } else if constexpr (T == VT_Q6_K) {
        const float d = h2f(r.d);
        float ds[4];
#pragma unroll
        for (int g = 0; g < 4; g++) ds[g] = d * float(int(int8_t(r.sc >> (8 * g))));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t qa = ((i < 4 ? r.a0 : r.a1) >> (8 * (i & 3))) & 0xffu;
            const uint32_t qb = ((i < 4 ? r.b0 : r.b1) >> (8 * (i & 3))) & 0xffu;
            const uint32_t qh = ((i < 4 ? r.h0 : r.h1) >> (8 * (i & 3))) & 0xffu;
            w[i] = ds[0] * float(int((qa & 15u) | ((qh & 3u) << 4)) - 32);
            w[8 + i] = ds[1] * float(int((qb & 15u) | (((qh >> 2) & 3u) << 4)) - 32);
            w[16 + i] = ds[2] * float(int((qa >> 4) | (((qh >> 4) & 3u) << 4)) - 32);
            w[24 + i] = ds[3] * float(int((qb >> 4) | (((qh >> 6) & 3u) << 4)) - 32);
        }
    } else if constexpr (T == VT_Q5_0) {  // src/gguf_compute.c:68-82: ((q | h << 4) - 16) * d
        const float d = h2f(r.b[0] & 0xffffu);
        const uint32_t qh = (r.b[0] >> 16) | (r.b[1] << 16);
        const uint32_t qs[4] = {(r.b[1] >> 16) | (r.b[2] << 16), (r.b[2] >> 16) | (r.b[3] << 16),
                                (r.b[3] >> 16) | (r.b[4] << 16), (r.b[4] >> 16) | (r.b[5] << 16)};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t q = (qs[i >> 2] >> (8 * (i & 3))) & 0xffu;
            w[i] = float(int((q & 15u) | (((qh >> i) & 1u) << 4)) - 16) * d;
            w[16 + i] = float(int((q >> 4) | (((qh >> (i + 16)) & 1u) << 4)) - 16) * d;
        }
    } else if constexpr (T == VT_F16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q[4] = {r.q[i].x, r.q[i].y, r.q[i].z, r.q[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                w[8 * i + 2 * j] = h2f(q[j] & 0xffffu);
                w[8 * i + 2 * j + 1] = h2f(q[j] >> 16);
            }
        }
    } else if constexpr (T == VT_F32) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            w[4 * i] = __uint_as_float(r.q[i].x);
            w[4 * i + 1] = __uint_as_float(r.q[i].y);
            w[4 * i + 2] = __uint_as_float(r.q[i].z);
            w[4 * i + 3] = __uint_as_float(r.q[i].w);
        }
    } else {  // Q8_0
        const float d = h2f((r.w[0] >> (8 * r.s)) & 0xffffu);
        const uint32_t sh = 16 + 8 * r.s;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = uint32_t(((uint64_t(r.w[i + 1]) << 32) | r.w[i]) >> sh);
#pragma unroll
            for (int k = 0; k < 4; k++) w[4 * i + k] = float(int(int8_t(q >> (8 * k)))) * d;
        }
    }
}
VH_DEV void deq_q4k(const Reg<VT_Q4_K>::Raw &r, int it, float (&w)[32]) {
    const int c = (it & 7) >> 1;
    const float d = h2f(r.hdr.x & 0xffffu), dmin = h2f(r.hdr.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_scale_min(2 * c, r.hdr.y, r.hdr.z, r.hdr.w, sc0, m0);
    q4k_scale_min(2 * c + 1, r.hdr.y, r.hdr.z, r.hdr.w, sc1, m1);
    const float d1 = d * float(sc0), mm1 = dmin * float(m0), d2 = d * float(sc1), mm2 = dmin * float(m1);
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t b = (qw[i >> 2] >> (8 * (i & 3))) & 0xffu;
        w[i] = d1 * float(b & 15u) - mm1;
        w[16 + i] = d2 * float(b >> 4) - mm2;
    }
}
template <int T>
VH_DEV void deq_item(const typename Reg<T>::Raw &raw, int it, float (&w)[32]) {
    const typename Reg<T>::Words &r = Reg<T>::resolve(raw, it);
    if constexpr (T == VT_Q4_K) deq_q4k(r, it, w);
    else deq_raw<T>(r, w);
}

// Column of the item's i-th input (i a multiple of 4: runs never split a float4).
template <int T>
VH_DEV int item_col(int it, int i) {
    if constexpr (T == VT_Q4_K) return Split<VT_Q4_K>::col0(it) + (i < 16 ? i : i + 16);
    else if constexpr (T == VT_Q6_K) return Split<VT_Q6_K>::col0(it) + 32 * (i >> 3) + (i & 7);
    else return 32 * it + i;
}
// Rows staged in LDS keep 4 pad floats after every 32, so the float4 reads of
// the lanes of a wave (32 columns apart) fall in different banks.
VH_DEV int padc(int c) { return c + 4 * (c >> 5); }
__host__ __device__ inline int padded_k(int K) { return K + 4 * (K / 32); }

// grid (ceil(rows / RB), max_slots), 512 threads, RB = 8 * (64 / L) * RPL
// rows per workgroup. Workgroup (rb, s): rows [rb*RB, rb*RB + RB) of the
// weight matrix (or matrices) of active expert s, for every token routed to it,
// in chunks of NT tokens staged in LDS. Lane group g (L lanes) takes RPL
// consecutive rows, one after the other, loading the next row's raw words
// while the current one computes; lane li owns items li, li + L, ... (IPL at
// most) of each row. GATEUP: rows of gate and up (K = d) -> h[pair][o] =
// silu(g) * u; else rows of down (K = fe) -> y[pair][o].
template <int T, bool GATEUP, int L, int IPL, int NT, int RPL>
__global__ void __launch_bounds__(512) grouped_proj_kernel(const int32_t *__restrict__ counts,
                                                           const int32_t *__restrict__ offs,
                                                           const int32_t *__restrict__ perm,
                                                           const int32_t *__restrict__ active,
                                                           const void *const *__restrict__ table,
                                                           const float *__restrict__ src, int K, int rows, int k,
                                                           int E, int64_t row_bytes, float *__restrict__ out) {
    constexpr int SUB = 64 / L, RB = 8 * SUB * RPL, NM = GATEUP ? 2 : 1;
    using Raw = typename Reg<T>::Raw;
    extern __shared__ float xs[];  // [NT][padded_k(K)]
    const int s = blockIdx.y;
    if (s >= active[E]) return;
    const int e = active[s], cnt = counts[e], base = offs[e];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, grp = lane / L, li = lane % L;
    const uint8_t *M0 = static_cast<const uint8_t *>(table[3 * e + (GATEUP ? 0 : 2)]);
    const uint8_t *M1 = GATEUP ? static_cast<const uint8_t *>(table[3 * e + 1]) : nullptr;
    const bool ok = M0 && (!GATEUP || M1);
    const int items = K / 32, KP = padded_k(K);
    const int o_first = blockIdx.x * RB + (wv * SUB + grp) * RPL;
    auto fetch_row = [&](int o, Raw (&raw)[NM][IPL]) {
        const int64_t oo = min(o, rows - 1);
#pragma unroll
        for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
            for (int m = 0; m < IPL; m++) {
                const int it = li + L * m;
                if (it < items) raw[mtx][m] = Reg<T>::fetch(mtx ? M1 : M0, oo * row_bytes, it);
            }
    };
    for (int t0 = 0; t0 < cnt; t0 += NT) {
        const int tn = min(NT, cnt - t0);
        Raw cur[NM][IPL];
        if (ok) fetch_row(o_first, cur);
        __syncthreads();
        for (int i = tid; i < tn * (K / 4); i += 512) {
            const int tt = i / (K / 4), c = 4 * (i - tt * (K / 4));
            const int p = perm[base + t0 + tt];
            const float *row = GATEUP ? src + size_t(p / k) * K : src + size_t(p) * K;
            *reinterpret_cast<float4 *>(xs + tt * KP + padc(c)) = *reinterpret_cast<const float4 *>(row + c);
        }
        __syncthreads();
#pragma unroll 1
        for (int rr = 0; rr < RPL; rr++) {
            const int o = o_first + rr;
            Raw nxt[NM][IPL];
            if (ok && rr + 1 < RPL) fetch_row(o + 1, nxt);
            float acc[NM][NT];
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                for (int tt = 0; tt < NT; tt++) acc[mtx][tt] = 0.0f;
            if (ok) {
#pragma unroll
                for (int m = 0; m < IPL; m++) {
                    const int it = li + L * m;
                    if (it >= items) continue;
                    float w[NM][32];
#pragma unroll
                    for (int mtx = 0; mtx < NM; mtx++) deq_item<T>(cur[mtx][m], it, w[mtx]);
#pragma unroll
                    for (int tt = 0; tt < NT; tt++) {
                        if (tt >= tn) break;
                        const float *xt = xs + tt * KP;
#pragma unroll
                        for (int q = 0; q < 8; q++) {
                            const float4 v = *reinterpret_cast<const float4 *>(xt + padc(item_col<T>(it, 4 * q)));
#pragma unroll
                            for (int mtx = 0; mtx < NM; mtx++) {
                                float a = acc[mtx][tt];
                                a = fmaf(w[mtx][4 * q + 0], v.x, a);
                                a = fmaf(w[mtx][4 * q + 1], v.y, a);
                                a = fmaf(w[mtx][4 * q + 2], v.z, a);
                                a = fmaf(w[mtx][4 * q + 3], v.w, a);
                                acc[mtx][tt] = a;
                            }
                        }
                        // one token's inputs in registers at a time: keep the
                        // scheduler from hoisting the next token's reads
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                if (tt >= tn) break;  // the same for every lane of the workgroup
                const float g = group_sum<L>(acc[0][tt]);
                const float u = GATEUP ? group_sum<L>(acc[NM - 1][tt]) : 0.0f;
                if (li == L - 1 && o < rows) {
                    const int p = perm[base + t0 + tt];
                    // an unregistered expert contributes nothing (src/gguf_run.c:201)
                    out[size_t(p) * rows + o] = !ok ? 0.0f : GATEUP ? swiglu(g, u) : g;
                }
            }
            if (rr + 1 < RPL) {
#pragma unroll
                for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                    for (int m = 0; m < IPL; m++) cur[mtx][m] = nxt[mtx][m];
            }
        }
    }
}

// x[t][o] += sum_j w[t][j] y[t k + j][o] in selection order, fp32, each
// product and sum rounded (src/gguf_run.c:208-213). A thread owns four
// consecutive outputs (d % 4 == 0): the token's routing and the experts'
// presence are read first, then every y row's four values are loaded at
// once, then summed in order. K = k, a compile-time count.
template <int K>
__global__ void __launch_bounds__(256) combine_kernel(const int32_t *__restrict__ idx, const float *__restrict__ w,
                                                      const void *const *__restrict__ table,
                                                      const float *__restrict__ ybuf, int d,
                                                      float *__restrict__ x) {
    const int t = blockIdx.y;
    const int o = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (o >= d) return;
    float wt[K];
    bool use[K];
#pragma unroll
    for (int j = 0; j < K; j++) {
        const int e = idx[size_t(t) * K + j];
        wt[j] = w[size_t(t) * K + j];
        use[j] = e >= 0 && table[3 * e + 2] != nullptr;  // a failed lookup is skipped (src/gguf_run.c:201)
    }
    float4 yv[K];
#pragma unroll
    for (int j = 0; j < K; j++) yv[j] = *reinterpret_cast<const float4 *>(ybuf + (size_t(t) * K + j) * d + o);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < K; j++) {
        if (!use[j]) continue;
        a.x = add_rn(a.x, mul_rn(wt[j], yv[j].x));
        a.y = add_rn(a.y, mul_rn(wt[j], yv[j].y));
        a.z = add_rn(a.z, mul_rn(wt[j], yv[j].z));
        a.w = add_rn(a.w, mul_rn(wt[j], yv[j].w));
    }
    float4 *xp = reinterpret_cast<float4 *>(x + size_t(t) * d + o);
    float4 xv = *xp;
    xv.x = add_rn(xv.x, a.x);
    xv.y = add_rn(xv.y, a.y);
    xv.z = add_rn(xv.z, a.z);
    xv.w = add_rn(xv.w, a.w);
    *xp = xv;
}

// the general case (another k, or d not a multiple of 4, or unaligned
// rows): one output per thread
__global__ void __launch_bounds__(256) combine_any_kernel(const int32_t *__restrict__ idx,
                                                          const float *__restrict__ w,
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
        a = add_rn(a, mul_rn(w[size_t(t) * k + j], ybuf[(size_t(t) * k + j) * d + o]));
    }
    x[size_t(t) * d + o] = add_rn(x[size_t(t) * d + o], a);
}

// tokens staged per chunk: 4 (more would not fit the registers of 512-thread
// workgroups; 4 rows of d = 2048 inputs take 37 KB of LDS)
template <bool GATEUP>
constexpr int group_tokens() { return 4; }

// Lanes per row: the smallest of 8 / 16 / 32 / 64 with at most 3 items per
// lane; for the two matrices of gate/up, one item per lane where a row has at
// most 64 items (two matrices' raw words and weights must fit the registers).
int proj_lanes(int items, bool gateup) {
    if (gateup && items <= 64) {
        int L = 8;
        while (L < items) L *= 2;
        return L;
    }
    for (int L : {8, 16, 32, 64})
        if ((items + L - 1) / L <= 3) return L;
    return 0;
}

template <int T, bool GATEUP>
int proj_launch(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                const void *const *table, const float *src, int K, int rows, int k, int E, int max_slots, float *out,
                hipStream_t s) {
    const int items = K / 32, L = proj_lanes(items, GATEUP);
    if (!L || K % 32) return -EINVAL;
    // F16 / F32 items are 64 / 128 raw bytes: one row per lane group (no next
    // row's words in flight), more workgroups instead
    constexpr int RPL = (T == VT_F16 || T == VT_F32) ? 1 : GATEUP ? 8 : 4;
    const int ipl = (items + L - 1) / L, RB = 8 * (64 / L) * RPL;
    const dim3 g((rows + RB - 1) / RB, max_slots);
    constexpr int NT = group_tokens<GATEUP>();
    const size_t lds = size_t(NT) * padded_k(K) * 4;
    if (lds > 64 * 1024) return -E2BIG;
    const int64_t rb = rbytes(T, K);
#define VH_PROJ(LL, II) \
    hipLaunchKernelGGL((grouped_proj_kernel<T, GATEUP, LL, II, NT, RPL>), g, dim3(512), lds, s, counts, offs, \
                       perm, active, table, src, K, rows, k, E, rb, out)
    if constexpr (GATEUP) {  // L >= items: one item per lane
        switch (L) {
        case 8: VH_PROJ(8, 1); break;
        case 16: VH_PROJ(16, 1); break;
        case 32: VH_PROJ(32, 1); break;
        default: VH_PROJ(64, 1); break;
        }
    } else {
        switch (L * 4 + (ipl <= 2 ? 2 : 3)) {
        case 8 * 4 + 2: VH_PROJ(8, 2); break;
        case 8 * 4 + 3: VH_PROJ(8, 3); break;
        case 16 * 4 + 2: VH_PROJ(16, 2); break;
        case 16 * 4 + 3: VH_PROJ(16, 3); break;
        case 32 * 4 + 2: VH_PROJ(32, 2); break;
        case 32 * 4 + 3: VH_PROJ(32, 3); break;
        case 64 * 4 + 2: VH_PROJ(64, 2); break;
        default: VH_PROJ(64, 3); break;
        }
    }
#undef VH_PROJ
    return vh_check(hipGetLastError());
}

}  // namespace

int vh_dispatch(const int32_t *idx, int P, int E, int32_t *counts, int32_t *offs, int32_t *perm, int32_t *active,
                hipStream_t s) {
    if (P <= kDispatchOneBlock) {
        hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, idx, P, E, counts, offs, perm, active);
    } else if (P % 4 == 0 && (reinterpret_cast<uintptr_t>(idx) & 15u) == 0 && P <= kFusedChunks * kFusedChunk &&
               E <= kMaxExperts) {
        hipLaunchKernelGGL(dispatch_fused_kernel, dim3(E), dim3(kFusedThreads), 0, s, idx, P, E, counts, offs, perm,
                           active);
    } else {
        hipLaunchKernelGGL(dispatch_count_kernel, dim3(E), dim3(256), 0, s, idx, P, counts);
        hipLaunchKernelGGL(dispatch_place_kernel, dim3(E), dim3(256), 0, s, idx, P, E, counts, offs, perm, active);
    }
    return vh_check(hipGetLastError());
}

int vh_grouped_gateup(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                      const int32_t *active, const void *const *table, const float *hb, int d, int fe, int k, int E,
                      int max_slots, float *h, hipStream_t s) {
    switch (type) {
    case VT_Q8_0: return proj_launch<VT_Q8_0, true>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, h, s);
    case VT_Q4_K: return proj_launch<VT_Q4_K, true>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, h, s);
    case VT_Q6_K: return proj_launch<VT_Q6_K, true>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, h, s);
    case VT_Q5_0: return proj_launch<VT_Q5_0, true>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, h, s);
    case VT_F16: return proj_launch<VT_F16, true>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, h, s);
    case VT_F32: return proj_launch<VT_F32, true>(counts, offs, perm, active, table, hb, d, fe, k, E, max_slots, h, s);
    default: return -EINVAL;
    }
}

int vh_grouped_down(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                    const int32_t *active, const void *const *table, const float *h, int d, int fe, int E,
                    int max_slots, float *ybuf, hipStream_t s) {
    switch (type) {
    case VT_Q8_0: return proj_launch<VT_Q8_0, false>(counts, offs, perm, active, table, h, fe, d, 1, E, max_slots, ybuf, s);
    case VT_Q4_K: return proj_launch<VT_Q4_K, false>(counts, offs, perm, active, table, h, fe, d, 1, E, max_slots, ybuf, s);
    case VT_Q6_K: return proj_launch<VT_Q6_K, false>(counts, offs, perm, active, table, h, fe, d, 1, E, max_slots, ybuf, s);
    case VT_Q5_0: return proj_launch<VT_Q5_0, false>(counts, offs, perm, active, table, h, fe, d, 1, E, max_slots, ybuf, s);
    case VT_F16: return proj_launch<VT_F16, false>(counts, offs, perm, active, table, h, fe, d, 1, E, max_slots, ybuf, s);
    case VT_F32: return proj_launch<VT_F32, false>(counts, offs, perm, active, table, h, fe, d, 1, E, max_slots, ybuf, s);
    default: return -EINVAL;
    }
}

int vh_combine(const int32_t *idx, const float *w, const void *const *table, const float *ybuf, int d, int k, int T,
               float *x, hipStream_t s) {
    const bool vec = (k == 8 || k == 4 || k == 2) && d % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(ybuf) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0;
    if (vec) {
        dim3 g((d / 4 + 255) / 256, T);
        if (k == 8) hipLaunchKernelGGL(combine_kernel<8>, g, dim3(256), 0, s, idx, w, table, ybuf, d, x);
        else if (k == 4) hipLaunchKernelGGL(combine_kernel<4>, g, dim3(256), 0, s, idx, w, table, ybuf, d, x);
        else hipLaunchKernelGGL(combine_kernel<2>, g, dim3(256), 0, s, idx, w, table, ybuf, d, x);
    } else {
        dim3 g((d + 255) / 256, T);
        hipLaunchKernelGGL(combine_any_kernel, g, dim3(256), 0, s, idx, w, table, ybuf, d, k, x);
    }
    return vh_check(hipGetLastError());
}
