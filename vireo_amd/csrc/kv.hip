// KV cache on the GPU (API: include/vireo_kv.h): the reference's KVStore
// (src/kvstore.h, src/kvstore_dense.c, src/kvstore_ooc.c, src/select/*) with
// its blocks in HBM.
//
// Host side: per layer a list of blocks (device copy, host copy once
// spilled, token count, lease, recency) and the pager of kvstore_ooc: blocks
// start resident, the least recently used unpinned unleased block is spilled
// (a device-to-host copy into pinned memory) when a new one would exceed the
// capacity, and a query pages its selected blocks back (host to device),
// counting requests, hits, misses and bytes as the reference does. Device
// memory comes from slabs of kSlabBlocks blocks; a block is K (G x d) then V.
//
// Device side:
//   kv_append_kernel   copies n (k, v) rows into their blocks and updates each
//                      block's running mean key with the reference's fp32
//                      operations (src/kvstore_ooc.c:139-141), so the TOPK
//                      scores below are the reference's bits;
//   kv_score_kernel    q . mean key per candidate block, the reference's
//                      in-order fp32 sum (kv_dot, src/kvstore.h:75-79);
//   kv_attend_kernel   grid (chunks, heads), 256 threads: wave w of chunk c
//                      takes list entries c CB + w, c CB + w + 4, ... and runs
//                      an online softmax over their tokens (lane = token for
//                      the scores, lane = output dimension for the weighted
//                      sum), then the four waves merge in order into the
//                      chunk's partial (m, l, acc);
//   kv_merge_kernel    per head, the chunks' partials in order: out = acc / l.
// The work split depends only on the selected token sequence, so a block
// gives the same bits resident, spilled or paged back.
#include <hip/hip_runtime.h>
#include <errno.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <new>
#include <vector>
#include "common.h"
#include "vireo_kv.h"
#include "kv_view.h"

namespace {

constexpr int kSlabBlocks = 64;   // blocks per device allocation
constexpr int kMaxAppend = 16;    // rows per vireo_kv_append_n launch
constexpr int kChunkBlocks = 8;   // list entries per attention workgroup
constexpr int kStageRing = 8;     // pinned staging buffers in turn

struct KvBlock {
    float *dev = nullptr;   // K (G d) then V (G d), while resident
    float *host = nullptr;  // pinned copy, made at the first spill
    int ntok = 0;
    int resident = 0;
    int lease = 0;
    uint64_t last_used = 0;
};

struct KvLayer {
    std::vector<KvBlock> blocks;
    float *ksum = nullptr;  // device [cap x d]: running mean key per block
    int cap = 0;
};

struct KvDesc {
    const float *blk;
    int ntok;
    int pad;
};

struct AppendArgs {
    float *dst[kMaxAppend];  // the token's K row in its block (V at + G d)
    float *ks[kMaxAppend];   // the block's mean key
    float inv[kMaxAppend];   // 1 / (tokens in the block after this one)
};

// sum of v over the 64 lanes in lane order (the same on every lane)
VH_DEV float wave_sum_ordered(float v) {
    float s = 0.0f;
    for (int u = 0; u < 64; u++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), u));
    return s;
}

// grid n, 64 * DPL threads... (any multiple of 64): row i of k and v into its block
__global__ void __launch_bounds__(256) kv_append_kernel(AppendArgs a, const float *__restrict__ k,
                                                        const float *__restrict__ v, int d, int gd) {
    const int i = blockIdx.x;
    const float *ki = k + size_t(i) * d, *vi = v + size_t(i) * d;
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
        const float kj = ki[j];
        a.dst[i][j] = kj;
        a.dst[i][gd + j] = vi[j];
        // ks += (k - ks) * inv, three roundings as in the reference
        const float ks = a.ks[i][j];
        a.ks[i][j] = add_rn(ks, mul_rn(sub_rn(kj, ks), a.inv[i]));
    }
}

// scores[h * stride + c] = q_h . ksum[cand[h] + c] for c < ncand[h]
__global__ void __launch_bounds__(256) kv_score_kernel(const float *const *__restrict__ ksum,
                                                       const int *__restrict__ lo, const int *__restrict__ ncand,
                                                       const float *__restrict__ q, int d, int stride,
                                                       float *__restrict__ scores) {
    const int h = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= ncand[h]) return;
    const float *a = q + size_t(h) * d, *b = ksum[h] + size_t(lo[h] + c) * d;
    float s = 0.0f;
    for (int i = 0; i < d; i++) s = add_rn(s, mul_rn(a[i], b[i]));
    scores[size_t(h) * stride + c] = s;
}

// partial of chunk c of head h: part[(h * nchunk + c) * (2 + d)] = {m, l, acc[d]}
template <int DPL>
__global__ void __launch_bounds__(256) kv_attend_kernel(const KvDesc *__restrict__ desc, const int *__restrict__ off,
                                                        const int *__restrict__ cnt, const float *__restrict__ q,
                                                        int G, float scale, int nchunk, float *__restrict__ part) {
    constexpr int D = 64 * DPL;
    __shared__ float qs[D];
    __shared__ float wm[4], wl[4], wacc[4][D];
    const int h = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = cnt[h], e0 = c * kChunkBlocks, e1 = min(n, e0 + kChunkBlocks);
    float *pout = part + (size_t(h) * nchunk + c) * (2 + D);
    if (e0 >= n) {  // an empty chunk (heads with fewer entries than others)
        if (tid == 0) { pout[0] = -INFINITY; pout[1] = 0.0f; }
        return;
    }
    for (int j = tid; j < D; j += 256) qs[j] = q[size_t(h) * D + j];
    __syncthreads();
    float m = -INFINITY, l = 0.0f, acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; i++) acc[i] = 0.0f;
    const KvDesc *dl = desc + off[h];
    for (int e = e0 + wv; e < e1; e += 4) {
        // the entry is the same for the whole wave
        const int ntok = __builtin_amdgcn_readfirstlane(dl[e].ntok);
        const uint64_t bp = reinterpret_cast<uint64_t>(dl[e].blk);
        const float *K = reinterpret_cast<const float *>(
            (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(bp >> 32)))) << 32) |
            uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(bp)))));
        const float *V = K + size_t(G) * D;
        // scores: lane t < ntok takes token t
        float s = -INFINITY;
        if (lane < ntok) {
            const float4 *kr = reinterpret_cast<const float4 *>(K + size_t(lane) * D);
            const float4 *qv = reinterpret_cast<const float4 *>(qs);
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 8
            for (int j = 0; j < D / 4; j++) {
                const float4 kk = kr[j], qq = qv[j];
                a0 = fmaf(qq.x, kk.x, a0);
                a1 = fmaf(qq.y, kk.y, a1);
                a2 = fmaf(qq.z, kk.z, a2);
                a3 = fmaf(qq.w, kk.w, a3);
            }
            s = ((a0 + a1) + (a2 + a3)) * scale;
        }
        const float bm = wave_max_f(s);
        const float mn = fmaxf(m, bm);
        const float cr = expf(m - mn);  // 0 while m is -inf
        const float p = lane < ntok ? expf(s - mn) : 0.0f;
        l = l * cr + wave_sum_f(p);
#pragma unroll
        for (int i = 0; i < DPL; i++) acc[i] *= cr;
        for (int t = 0; t < ntok; t++) {
            const float pt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), t));
            const float *vr = V + size_t(t) * D;
#pragma unroll
            for (int i = 0; i < DPL; i++) acc[i] = fmaf(pt, vr[lane + 64 * i], acc[i]);
        }
        m = mn;
    }
    if (lane == 0) { wm[wv] = m; wl[wv] = l; }
#pragma unroll
    for (int i = 0; i < DPL; i++) wacc[wv][lane + 64 * i] = acc[i];
    __syncthreads();
    if (wv == 0) {  // the four waves' partials, in wave order
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w]);
        float L = 0.0f, A[DPL];
#pragma unroll
        for (int i = 0; i < DPL; i++) A[i] = 0.0f;
        for (int w = 0; w < 4; w++) {
            if (wl[w] == 0.0f) continue;  // a wave without tokens
            const float f = expf(wm[w] - M);
            L += wl[w] * f;
#pragma unroll
            for (int i = 0; i < DPL; i++) A[i] = fmaf(wacc[w][lane + 64 * i], f, A[i]);
        }
        if (lane == 0) { pout[0] = M; pout[1] = L; }
#pragma unroll
        for (int i = 0; i < DPL; i++) pout[2 + lane + 64 * i] = A[i];
    }
}

// out[h] = (sum_c acc_c e^(m_c - M)) / (sum_c l_c e^(m_c - M)), chunks in
// order: lane c takes chunk c's (m, l) for the maximum and the weights
// e^(m_c - M) (64 chunks at a time), then every lane adds its columns'
// accumulators over the chunks in order
// counts.count(h): the blocks query head h attended
struct HeadCounts {
    const int *cnt;
    VH_DEV int count(int h) const { return cnt[h]; }
};
template <int DPL, class Counts>
__global__ void __launch_bounds__(64) kv_merge_kernel(const float *__restrict__ part, Counts counts, int nchunk, int cb,
                                                      float *__restrict__ out) {
    constexpr int D = 64 * DPL;
    __shared__ float fs[64];
    const int h = blockIdx.x, lane = threadIdx.x;
    const int nc = (counts.count(h) + cb - 1) / cb;
    const float *p = part + size_t(h) * nchunk * (2 + D);
    float M = -INFINITY;
    for (int c = lane; c < nc; c += 64) M = fmaxf(M, p[size_t(c) * (2 + D)]);
    M = wave_max_f(M);
    float L = 0.0f, A[DPL];
#pragma unroll
    for (int i = 0; i < DPL; i++) A[i] = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 64) {
        const int c = c0 + lane;
        float f = 0.0f, lw = 0.0f;
        if (c < nc) {
            const float lc = p[size_t(c) * (2 + D) + 1];
            if (lc != 0.0f) {  // an empty chunk adds nothing
                f = expf(p[size_t(c) * (2 + D)] - M);
                lw = lc * f;
            }
        }
        fs[lane] = f;
        // l summed in chunk order: lane 0 adds the 64 weights in turn
        __syncthreads();
        const float lsum = wave_sum_ordered(lw);
        L += lsum;
        const int n = min(64, nc - c0);
        // 16 chunks' loads in flight: the loop is bound by their latency (the
        // accumulation order, and so the result, does not depend on it; 998 ->
        // 1 146 tok/s for 48 layers at context 4096 against 4 in flight)
#pragma unroll 16
        for (int u = 0; u < n; u++) {
            const float fu = fs[u];
            const float *pc = p + size_t(c0 + u) * (2 + D) + 2;
#pragma unroll
            for (int i = 0; i < DPL; i++) A[i] = fmaf(pc[lane + 64 * i], fu, A[i]);
        }
        __syncthreads();
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; i++) out[size_t(h) * D + lane + 64 * i] = A[i] * inv;
}

constexpr int kGroupBlocks = 2;  // list entries per workgroup of the grouped-query kernel

// Grouped-query attention when every query head of a group attends the same
// blocks (selections that do not depend on the query): grid (chunks, kv
// heads), 256 threads. Chunk c of kv head g covers entries c CB .. c CB + CB - 1
// of g's list; its keys and values are read once for the HPG query heads
// g HPG .. g HPG + HPG - 1, whose partials {m, l, acc} it writes as
// kv_attend_kernel does (chunk size CB). Phases: the scores of every token
// and head (a quad of lanes per token, a quarter of the dimensions each), the
// per-head softmax over the chunk (a wave per head), then the weighted sum of
// the values (a thread per column of 4 dimensions and group of tokens),
// reduced over the token groups in order.
// The blocks of kv head g's list: count(g), and entry(g, e) = (block, tokens).
struct ListedBlocks {  // lists uploaded by the host
    const KvDesc *desc;
    const int *off, *cnt;
    VH_DEV int count(int g) const { return cnt[g]; }
    VH_DEV KvDesc entry(int g, int e) const { return desc[off[g] + e]; }
};
struct ContiguousBlocks {  // a contiguous store at the position *pos (every block attended)
    const float *base;  // block b of layer l at base + (l * max_blocks + b) * 2 G D
    const int *pos;
    int layer0, max_blocks, G, D;
    VH_DEV int count(int) const {
        const int p = *pos;
        return p < 0 ? 0 : min(p / G + 1, max_blocks);
    }
    VH_DEV KvDesc entry(int g, int e) const {
        const int p = *pos, last = p / G;
        KvDesc k;
        k.blk = base + (size_t(layer0 + g) * max_blocks + e) * size_t(2 * G * D);
        k.ntok = e < last ? G : p % G + 1;
        k.pad = 0;
        return k;
    }
};

// a query head's count is its kv head's list's (the heads of a group attend
// the same blocks)
template <class Lists>
struct GroupCounts {
    Lists lists;
    int hpg;
    VH_DEV int count(int h) const { return lists.count(h / hpg); }
};

template <int D, int HPG, class Lists>
__global__ void __launch_bounds__(256) kv_attend_group_kernel(Lists lists, const float *__restrict__ q, int G,
                                                              float scale, int nchunk, float *__restrict__ part) {
    constexpr int CB = kGroupBlocks, TMAX = CB * 64, QD = D / 4, NDQ = D / 4, NTG = 256 / NDQ;
    __shared__ float4 qs[HPG][D / 4];
    __shared__ float ps[HPG][TMAX];
    __shared__ float hm[HPG], hl[HPG];
    __shared__ float4 red[NTG][HPG][NDQ];
    const int g = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = lists.count(g), e0 = c * CB, e1 = min(n, e0 + CB);
    if (e0 >= n) {  // an empty chunk: its heads' partials are empty
        if (tid < HPG) {
            float *po = part + (size_t(g * HPG + tid) * nchunk + c) * (2 + D);
            po[0] = -INFINITY;
            po[1] = 0.0f;
        }
        return;
    }
    for (int i = tid; i < HPG * (D / 4); i += 256)
        qs[i / (D / 4)][i % (D / 4)] = reinterpret_cast<const float4 *>(q + size_t(g) * HPG * D)[i];
    const KvDesc d0 = lists.entry(g, e0), d1 = e0 + 1 < e1 ? lists.entry(g, e0 + 1) : KvDesc{d0.blk, 0, 0};
    const float *B0 = d0.blk, *B1 = d1.blk;
    const int n0 = d0.ntok, T = n0 + d1.ntok;
    auto krow = [&](int t) { return t < n0 ? B0 + size_t(t) * D : B1 + size_t(t - n0) * D; };  // V at + G D
    // the values this thread weighs in the last phase, loaded before the scores
    // are formed (D <= 128: at most 16 float4 per thread)
    const int dq = tid % NDQ, tg = tid / NDQ;
    constexpr int MT = D <= 128 ? TMAX / NTG : 1;
    float4 vv[MT];
    if constexpr (D <= 128) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const int t = tg + NTG * m;
            vv[m] = t < T ? reinterpret_cast<const float4 *>(krow(t) + size_t(G) * D)[dq] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    __syncthreads();
    // scores: lanes 4m .. 4m + 3 take token t = tid / 4 (+ 64 j), quarter tid % 4
    const int qd = tid & 3;
#pragma unroll
    for (int t0 = 0; t0 < TMAX; t0 += 64) {
        const int t = t0 + (tid >> 2);
        float sc[HPG];
#pragma unroll
        for (int i = 0; i < HPG; i++) sc[i] = 0.0f;
        if (t < T) {
            const float4 *kr = reinterpret_cast<const float4 *>(krow(t) + qd * QD);
#pragma unroll
            for (int j = 0; j < QD / 4; j++) {
                const float4 kk = kr[j];
#pragma unroll
                for (int i = 0; i < HPG; i++) {
                    const float4 qq = qs[i][qd * (QD / 4) + j];
                    sc[i] = fmaf(qq.x, kk.x, fmaf(qq.y, kk.y, fmaf(qq.z, kk.z, fmaf(qq.w, kk.w, sc[i]))));
                }
            }
        }
#pragma unroll
        for (int i = 0; i < HPG; i++) {
            sc[i] += dpp_f<0xB1>(sc[i]);
            sc[i] += dpp_f<0x4E>(sc[i]);
        }
        if (qd == 0 && t < T)
#pragma unroll
            for (int i = 0; i < HPG; i++) ps[i][t] = sc[i] * scale;
    }
    __syncthreads();
    // softmax of each head over the chunk's tokens: wave w takes heads w, w + 4, ...
    for (int i = wv; i < HPG; i += 4) {
        const float a = lane < T ? ps[i][lane] : -INFINITY, b = lane + 64 < T ? ps[i][lane + 64] : -INFINITY;
        const float mx = wave_max_f(fmaxf(a, b));
        const float pa = lane < T ? expf(a - mx) : 0.0f, pb = lane + 64 < T ? expf(b - mx) : 0.0f;
        const float l = wave_sum_f(pa + pb);
        if (lane < T) ps[i][lane] = pa;
        if (lane + 64 < T) ps[i][lane + 64] = pb;
        if (lane == 0) {
            hm[i] = mx;
            hl[i] = l;
        }
    }
    __syncthreads();
    // weighted values: thread (token group tg, column dq) sums tokens tg, tg + NTG, ...
    float4 acc[HPG];
#pragma unroll
    for (int i = 0; i < HPG; i++) acc[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto weigh = [&](const float4 &v, int t) {
#pragma unroll
        for (int i = 0; i < HPG; i++) {
            const float pt = ps[i][t];
            acc[i].x = fmaf(pt, v.x, acc[i].x);
            acc[i].y = fmaf(pt, v.y, acc[i].y);
            acc[i].z = fmaf(pt, v.z, acc[i].z);
            acc[i].w = fmaf(pt, v.w, acc[i].w);
        }
    };
    if constexpr (D <= 128) {
#pragma unroll
        for (int m = 0; m < MT; m++)
            if (tg + NTG * m < T) weigh(vv[m], tg + NTG * m);
    } else {
        for (int t = tg; t < T; t += NTG) weigh(reinterpret_cast<const float4 *>(krow(t) + size_t(G) * D)[dq], t);
    }
#pragma unroll
    for (int i = 0; i < HPG; i++) red[tg][i][dq] = acc[i];
    __syncthreads();
    for (int x = tid; x < HPG * NDQ; x += 256) {
        const int i = x / NDQ, col = x % NDQ;
        float4 a = red[0][i][col];
        for (int u = 1; u < NTG; u++) {
            const float4 b = red[u][i][col];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        float *po = part + (size_t(g * HPG + i) * nchunk + c) * (2 + D);
        po[2 + 4 * col] = a.x;
        po[3 + 4 * col] = a.y;
        po[4 + 4 * col] = a.z;
        po[5 + 4 * col] = a.w;
        if (col == 0) {
            po[0] = hm[i];
            po[1] = hl[i];
        }
    }
}

template <int D, class Lists>
int launch_group(int hpg, Lists lists, const float *q, int G, float scale, int nchunk, int n_kv, int n_heads,
                 float *part, float *out, hipStream_t s) {
    const dim3 g(nchunk, n_kv);
    switch (hpg) {
    case 1: hipLaunchKernelGGL((kv_attend_group_kernel<D, 1, Lists>), g, dim3(256), 0, s, lists, q, G, scale, nchunk, part); break;
    case 2: hipLaunchKernelGGL((kv_attend_group_kernel<D, 2, Lists>), g, dim3(256), 0, s, lists, q, G, scale, nchunk, part); break;
    case 4: hipLaunchKernelGGL((kv_attend_group_kernel<D, 4, Lists>), g, dim3(256), 0, s, lists, q, G, scale, nchunk, part); break;
    default: hipLaunchKernelGGL((kv_attend_group_kernel<D, 8, Lists>), g, dim3(256), 0, s, lists, q, G, scale, nchunk, part); break;
    }
    hipLaunchKernelGGL((kv_merge_kernel<D / 64, GroupCounts<Lists>>), dim3(n_heads), dim3(64), 0, s, part,
                       GroupCounts<Lists>{lists, hpg}, nchunk, kGroupBlocks, out);
    return vh_check(hipGetLastError());
}

// contiguous stores: k and v rows for layers layer0 .. layer0 + n - 1 at the
// position *pos (no effect outside [0, max_tokens)), as kv_append_kernel
__global__ void __launch_bounds__(256) kv_append_pos_kernel(float *__restrict__ base, float *__restrict__ ksum,
                                                            int layer0, int max_blocks, int max_tokens,
                                                            const int *__restrict__ pos_p, const float *__restrict__ k,
                                                            const float *__restrict__ v, int d, int G) {
    const int pos = *pos_p;
    if (pos < 0 || pos >= max_tokens) return;
    const int i = blockIdx.x, b = pos / G, slot = pos % G;
    const size_t li = size_t(layer0 + i) * max_blocks + b;
    float *blk = base + li * size_t(2 * G * d);
    float *ks = ksum + li * size_t(d);
    const float inv = 1.0f / float(slot + 1);
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
        const float kj = k[size_t(i) * d + j];
        blk[size_t(slot) * d + j] = kj;
        blk[size_t(G + slot) * d + j] = v[size_t(i) * d + j];
        const float old = slot == 0 ? 0.0f : ks[j];  // a new block's mean starts at zero
        ks[j] = add_rn(old, mul_rn(sub_rn(kj, old), inv));
    }
}

int blocks_for(int tokens, int g) { return tokens > 0 ? (tokens + g - 1) / g : 0; }

int by_score_desc(const void *a, const void *b);

}  // namespace

struct VireoKV {
    VireoKVConfig cfg{};
    bool dense = false;  // kvstore_dense semantics for the statistics
    int strategy = VIREO_KV_SELECT_ALL, budget = 0;  // budget: the strategy's (0 = unbounded)
    int sink_blocks = 0, window_blocks = 0, d = 0, G = 0;
    uint64_t block_bytes = 0, resident_bytes = 0, tick = 0;
    VireoKVStats st{};
    std::vector<KvLayer> layers;
    std::vector<void *> slabs;
    std::vector<float *> free_blocks;
    // device scratch and its pinned staging
    void *dscratch = nullptr;
    size_t dscratch_bytes = 0;
    // pinned staging for uploads, a ring: slot i is reused once its last
    // upload has been read (staged[i]), so the host may run calls ahead
    void *hstage[kStageRing] = {};
    size_t hstage_bytes[kStageRing] = {};
    hipEvent_t staged[kStageRing] = {};
    int stage_next = 0;
    float *part = nullptr;
    size_t part_bytes = 0;
    // device buffers replaced by larger ones: HIP graphs captured earlier may
    // still point at them, so they are freed only with the store
    std::vector<void *> retired;
    std::vector<float> hscores;
    // contiguous stores (vireo_kv_create_contiguous): every layer's blocks in
    // one region, block b of layer l at cbase + (l * max_blocks + b) * 2 G d,
    // mean keys at cksum + (l * max_blocks + b) * d
    bool contig = false;
    int max_blocks = 0;
    float *cbase = nullptr, *cksum = nullptr;
};

namespace {

struct Scored {
    int id;
    float score;
};
// src/select/select_topk.c: descending score (the same comparator, for qsort)
int by_score_desc(const void *a, const void *b) {
    const float d = static_cast<const Scored *>(b)->score - static_cast<const Scored *>(a)->score;
    return (d > 0) - (d < 0);
}

bool is_pinned(const VireoKV *S, const KvLayer &L, int i) {
    const int nb = int(L.blocks.size());
    return i < S->sink_blocks || i >= nb - S->window_blocks || i == nb - 1;
}

int take_block(VireoKV *S, float **out) {
    if (S->free_blocks.empty()) {
        void *p = nullptr;
        if (hipMalloc(&p, S->block_bytes * kSlabBlocks) != hipSuccess) return -ENOMEM;
        S->slabs.push_back(p);
        for (int i = kSlabBlocks - 1; i >= 0; i--)
            S->free_blocks.push_back(reinterpret_cast<float *>(static_cast<char *>(p) + size_t(i) * S->block_bytes));
    }
    *out = S->free_blocks.back();
    S->free_blocks.pop_back();
    return 0;
}

// src/kvstore_ooc.c:63-72 (a copy in pinned host memory instead of a file)
int spill(VireoKV *S, KvBlock &b, hipStream_t s) {
    if (!b.host && hipHostMalloc(reinterpret_cast<void **>(&b.host), S->block_bytes, 0) != hipSuccess) {
        b.host = nullptr;
        return -ENOMEM;
    }
    if (hipMemcpyAsync(b.host, b.dev, S->block_bytes, hipMemcpyDeviceToHost, s) != hipSuccess) return -EIO;
    S->st.bytes_spilled += S->block_bytes;
    S->free_blocks.push_back(b.dev);  // reused only by work enqueued after this copy
    b.dev = nullptr;
    b.resident = 0;
    S->resident_bytes -= S->block_bytes;
    return 0;
}

// src/kvstore_ooc.c:74-91
int evict_until_room(VireoKV *S, hipStream_t s) {
    if (!S->cfg.capacity_bytes) return 0;
    while (S->resident_bytes + S->block_bytes > S->cfg.capacity_bytes) {
        KvBlock *victim = nullptr;
        uint64_t best = UINT64_MAX;
        for (auto &L : S->layers)
            for (int i = 0; i < int(L.blocks.size()); i++) {
                KvBlock &b = L.blocks[i];
                if (b.resident && !b.lease && !is_pinned(S, L, i) && b.last_used < best) {
                    best = b.last_used;
                    victim = &b;
                }
            }
        if (!victim) break;  // nothing evictable now: stay over budget
        if (int rc = spill(S, *victim, s)) return rc;
    }
    return 0;
}

// src/kvstore_ooc.c:93-110 (a lease is taken on the block)
int ensure_resident(VireoKV *S, KvBlock &b, hipStream_t s) {
    S->st.requests++;
    if (b.resident) {
        S->st.hits++;
        b.last_used = ++S->tick;
        b.lease++;
        return 0;
    }
    S->st.misses++;
    if (int rc = evict_until_room(S, s)) return rc;
    if (int rc = take_block(S, &b.dev)) return rc;
    if (hipMemcpyAsync(b.dev, b.host, S->block_bytes, hipMemcpyHostToDevice, s) != hipSuccess) return -EIO;
    b.resident = 1;
    S->resident_bytes += S->block_bytes;
    S->st.bytes_read += S->block_bytes;
    b.last_used = ++S->tick;
    b.lease++;
    return 0;
}

// src/kvstore_ooc.c:113-132
int start_block(VireoKV *S, KvLayer &L, hipStream_t s) {
    const int nb = int(L.blocks.size());
    if (S->contig) {
        if (nb >= S->max_blocks) return -ENOSPC;
        const size_t li = size_t(&L - S->layers.data()) * S->max_blocks + nb;
        KvBlock b;
        b.dev = S->cbase + li * size_t(2 * S->G * S->d);
        b.resident = 1;
        b.last_used = ++S->tick;
        L.blocks.push_back(b);
        S->resident_bytes += S->block_bytes;
        // the mean key starts at zero (the region is cleared at creation; the
        // row is cleared again in case a device-position call wrote it)
        return hipMemsetAsync(S->cksum + li * S->d, 0, size_t(S->d) * sizeof(float), s) == hipSuccess ? 0 : -EIO;
    }
    if (nb >= L.cap) {
        const int cap = L.cap ? 2 * L.cap : 64;
        float *ks = nullptr;
        if (hipMalloc(&ks, size_t(cap) * S->d * sizeof(float)) != hipSuccess) return -ENOMEM;
        if (L.ksum) {
            if (hipMemcpyAsync(ks, L.ksum, size_t(nb) * S->d * sizeof(float), hipMemcpyDeviceToDevice, s) !=
                    hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                return -EIO;
            (void)hipFree(L.ksum);
        }
        L.ksum = ks;
        L.cap = cap;
    }
    KvBlock b;
    if (int rc = take_block(S, &b.dev)) return rc;
    b.resident = 1;
    b.last_used = ++S->tick;
    if (hipMemsetAsync(L.ksum + size_t(nb) * S->d, 0, size_t(S->d) * sizeof(float), s) != hipSuccess) return -EIO;
    L.blocks.push_back(b);
    S->resident_bytes += S->block_bytes;
    return evict_until_room(S, s);
}

// device scratch of at least `bytes` (grown; the stream is idle when it grows)
// Replace *buf by an allocation of at least `need` bytes (twice that, so a
// store grows a few times at most). The old buffer is kept until the store is
// destroyed: enqueued work and captured graphs may still use it.
template <class T>
int grow(VireoKV *S, T **buf, size_t *bytes, size_t need) {
    if (need <= *bytes) return 0;
    const size_t nb = need < (size_t(1) << 16) ? (size_t(1) << 16) : 2 * need;
    void *p = nullptr;
    if (hipMalloc(&p, nb) != hipSuccess) return -ENOMEM;
    if (*buf) S->retired.push_back(static_cast<void *>(*buf));
    *buf = static_cast<T *>(p);
    *bytes = nb;
    return 0;
}

int scratch(VireoKV *S, size_t bytes, hipStream_t, void **out) {
    if (int rc = grow(S, &S->dscratch, &S->dscratch_bytes, bytes)) return rc;
    *out = S->dscratch;
    return 0;
}

// the next pinned staging buffer of the ring, of at least `bytes`, once its
// previous upload is done; record staged[*slot] after the upload from it
int staging(VireoKV *S, size_t bytes, void **out, int *slot) {
    const int i = S->stage_next;
    S->stage_next = (i + 1) % kStageRing;
    if (S->staged[i] && hipEventSynchronize(S->staged[i]) != hipSuccess) return -EIO;
    if (bytes > S->hstage_bytes[i]) {
        if (S->hstage[i]) (void)hipHostFree(S->hstage[i]);
        S->hstage[i] = nullptr;
        const size_t nb = bytes < (size_t(1) << 16) ? (size_t(1) << 16) : 2 * bytes;
        if (hipHostMalloc(&S->hstage[i], nb, 0) != hipSuccess) { S->hstage_bytes[i] = 0; return -ENOMEM; }
        S->hstage_bytes[i] = nb;
    }
    *out = S->hstage[i];
    *slot = i;
    return 0;
}

int append_n(VireoKV *S, int layer0, int n, const float *k, const float *v, hipStream_t s) {
    AppendArgs a;
    for (int i = 0; i < n; i++) {
        KvLayer &L = S->layers[layer0 + i];
        if (L.blocks.empty() || L.blocks.back().ntok == S->G)
            if (int rc = start_block(S, L, s)) return rc;
        const int bi = int(L.blocks.size()) - 1;
        KvBlock &b = L.blocks[bi];
        a.dst[i] = b.dev + size_t(b.ntok) * S->d;
        a.ks[i] = L.ksum + size_t(bi) * S->d;
        b.ntok++;
        a.inv[i] = 1.0f / float(b.ntok);
        b.last_used = ++S->tick;
    }
    hipLaunchKernelGGL(kv_append_kernel, dim3(n), dim3(S->d < 256 ? S->d : 256), 0, s, a, k, v, S->d, S->G * S->d);
    return vh_check(hipGetLastError());
}

// The blocks head h attends to (src/kvstore_ooc.c:163-176), as ids into
// seen[]; for TOPK the candidates' scores are in scores[0 .. ncand).
void select_blocks(const VireoKV *S, int nb, const float *scores, std::vector<unsigned char> &seen) {
    seen.assign(size_t(nb), 0);
    int budget = S->budget > 0 ? S->budget : nb;
    if (budget > nb) budget = nb;
    if (S->strategy == VIREO_KV_SELECT_ALL) {
        for (int i = 0; i < budget; i++) seen[i] = 1;
    } else if (S->strategy == VIREO_KV_SELECT_TOPK) {
        const int lo = S->sink_blocks, hi = nb - S->window_blocks;
        if (nb > 0 && hi > lo) {  // src/select/select_topk.c:19-40
            const int ncand = hi - lo;
            std::vector<Scored> sc(static_cast<size_t>(ncand));
            for (int i = 0; i < ncand; i++) sc[i] = Scored{lo + i, scores[i]};
            qsort(sc.data(), size_t(ncand), sizeof(Scored), by_score_desc);
            int take = S->budget < ncand ? S->budget : ncand;
            if (take > budget) take = budget;
            for (int i = 0; i < take; i++) seen[sc[i].id] = 1;
        }
    }
    for (int i = 0; i < S->sink_blocks && i < nb; i++) seen[i] = 1;
    for (int i = nb - S->window_blocks; i < nb; i++)
        if (i >= 0) seen[i] = 1;
}

template <int DPL>
void launch_attend(const KvDesc *desc, const int *off, const int *cnt, const float *q, int G, float scale,
                   int nchunk, int heads, float *part, float *out, hipStream_t s) {
    hipLaunchKernelGGL((kv_attend_kernel<DPL>), dim3(nchunk, heads), dim3(256), 0, s, desc, off, cnt, q, G, scale,
                       nchunk, part);
    hipLaunchKernelGGL((kv_merge_kernel<DPL, HeadCounts>), dim3(heads), dim3(64), 0, s, part, HeadCounts{cnt}, nchunk,
                       kChunkBlocks, out);
}

// heads h < n_heads attend layer layer0 + h / kv_mul with q_h
int attend(VireoKV *S, int layer0, int n_heads, int kv_mul, const float *q, float *out, hipStream_t s) {
    const int d = S->d;
    std::vector<std::vector<unsigned char>> seen(static_cast<size_t>(n_heads));
    // TOPK: every head's candidate scores in one launch, then on the host
    if (S->strategy == VIREO_KV_SELECT_TOPK) {
        int maxc = 0;
        std::vector<int> lo(static_cast<size_t>(n_heads)), nc(static_cast<size_t>(n_heads));
        std::vector<const float *> ks(static_cast<size_t>(n_heads));
        for (int h = 0; h < n_heads; h++) {
            const KvLayer &L = S->layers[layer0 + h / kv_mul];
            const int nb = int(L.blocks.size()), hi = nb - S->window_blocks;
            lo[h] = S->sink_blocks;
            nc[h] = hi > lo[h] ? hi - lo[h] : 0;
            ks[h] = L.ksum;
            maxc = nc[h] > maxc ? nc[h] : maxc;
        }
        if (maxc > 0) {
            const size_t tb = size_t(n_heads) * (sizeof(void *) + 2 * sizeof(int));
            const size_t sb = size_t(n_heads) * maxc * sizeof(float);
            void *dv, *hv;
            if (int rc = scratch(S, tb + sb, s, &dv)) return rc;
            int slot;
            if (int rc = staging(S, tb, &hv, &slot)) return rc;
            char *hc = static_cast<char *>(hv);
            memcpy(hc, ks.data(), size_t(n_heads) * sizeof(void *));
            memcpy(hc + size_t(n_heads) * sizeof(void *), lo.data(), size_t(n_heads) * sizeof(int));
            memcpy(hc + size_t(n_heads) * (sizeof(void *) + sizeof(int)), nc.data(), size_t(n_heads) * sizeof(int));
            char *dc = static_cast<char *>(dv);
            if (hipMemcpyAsync(dc, hc, tb, hipMemcpyHostToDevice, s) != hipSuccess ||
                hipEventRecord(S->staged[slot], s) != hipSuccess)
                return -EIO;
            float *dsc = reinterpret_cast<float *>(dc + tb);
            hipLaunchKernelGGL(kv_score_kernel, dim3((maxc + 255) / 256, n_heads), dim3(256), 0, s,
                               reinterpret_cast<const float *const *>(dc),
                               reinterpret_cast<const int *>(dc + size_t(n_heads) * sizeof(void *)),
                               reinterpret_cast<const int *>(dc + size_t(n_heads) * (sizeof(void *) + sizeof(int))), q,
                               d, maxc, dsc);
            if (int rc = vh_check(hipGetLastError())) return rc;
            S->hscores.resize(size_t(n_heads) * maxc);
            if (hipMemcpyAsync(S->hscores.data(), dsc, sb, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                return -EIO;
        }
        for (int h = 0; h < n_heads; h++)
            select_blocks(S, int(S->layers[layer0 + h / kv_mul].blocks.size()),
                          maxc > 0 ? S->hscores.data() + size_t(h) * maxc : nullptr, seen[h]);
    } else {
        for (int h = 0; h < n_heads; h++) select_blocks(S, int(S->layers[layer0 + h / kv_mul].blocks.size()), nullptr, seen[h]);
    }
    // page the selected blocks in, head by head and in ascending order, and
    // list them; every lease is held until the kernels are enqueued. When the
    // selection does not depend on the query and the group size has a
    // grouped-query kernel, the list is kept once per kv head (the heads of a
    // group select the same blocks) and the blocks are read once per group.
    const bool grouped = S->strategy != VIREO_KV_SELECT_TOPK &&
                         (kv_mul == 1 || kv_mul == 2 || kv_mul == 4 || kv_mul == 8) &&
                         !(reinterpret_cast<uintptr_t>(q) & 15u);
    const int n_lists = grouped ? n_heads / kv_mul : n_heads, cb = grouped ? kGroupBlocks : kChunkBlocks;
    std::vector<KvDesc> desc;
    std::vector<int> off(static_cast<size_t>(n_lists)), cnt(static_cast<size_t>(n_heads));
    std::vector<KvBlock *> leased;
    int rc = 0, nchunk = 1;
    for (int h = 0; h < n_heads && !rc; h++) {
        KvLayer &L = S->layers[layer0 + h / kv_mul];
        const bool lists = !grouped || h % kv_mul == 0;
        const int d0 = int(desc.size());
        if (lists) off[grouped ? h / kv_mul : h] = d0;
        int got = 0;
        for (int i = 0; i < int(L.blocks.size()) && !rc; i++) {
            if (!seen[h][i]) continue;
            KvBlock &b = L.blocks[i];
            if ((rc = ensure_resident(S, b, s))) break;
            leased.push_back(&b);
            if (lists) desc.push_back(KvDesc{b.dev, b.ntok, 0});
            got++;
        }
        cnt[h] = got;
        const int nc = (got + cb - 1) / cb;
        nchunk = nc > nchunk ? nc : nchunk;
    }
    if (!rc) {
        // device: desc, then off [n_lists], then (grouped) the per-list counts, then the per-head counts
        std::vector<int> cnt_list;
        if (grouped)
            for (int g = 0; g < n_lists; g++) cnt_list.push_back(cnt[size_t(g) * kv_mul]);
        const size_t db = desc.size() * sizeof(KvDesc);
        const size_t ib = (size_t(n_lists) * (grouped ? 2 : 1) + size_t(n_heads)) * sizeof(int);
        const size_t pb = size_t(n_heads) * nchunk * (2 + d) * sizeof(float);
        void *dv = nullptr, *hv = nullptr;
        int slot = 0;
        rc = scratch(S, db + ib + 256, s, &dv);
        if (!rc) rc = grow(S, &S->part, &S->part_bytes, pb);
        if (!rc) rc = staging(S, db + ib + 256, &hv, &slot);
        if (!rc) {
            char *hc = static_cast<char *>(hv), *dc = static_cast<char *>(dv);
            const size_t io = (db + 255) & ~size_t(255);
            if (db) memcpy(hc, desc.data(), db);
            int *hi = reinterpret_cast<int *>(hc + io);
            memcpy(hi, off.data(), size_t(n_lists) * sizeof(int));
            if (grouped) memcpy(hi + n_lists, cnt_list.data(), size_t(n_lists) * sizeof(int));
            memcpy(hi + n_lists * (grouped ? 2 : 1), cnt.data(), size_t(n_heads) * sizeof(int));
            if (hipMemcpyAsync(dc, hc, io + ib, hipMemcpyHostToDevice, s) != hipSuccess ||
                hipEventRecord(S->staged[slot], s) != hipSuccess)
                rc = -EIO;
            const KvDesc *dd = reinterpret_cast<const KvDesc *>(dc);
            const int *doff = reinterpret_cast<const int *>(dc + io);
            const int *dcnt_list = doff + n_lists, *dcnt = doff + n_lists * (grouped ? 2 : 1);
            const float scale = 1.0f / sqrtf(float(d));
            if (!rc && grouped) {
                const ListedBlocks lb{dd, doff, dcnt_list};
                if (d == 64) rc = launch_group<64>(kv_mul, lb, q, S->G, scale, nchunk, n_lists, n_heads, S->part, out, s);
                else if (d == 128) rc = launch_group<128>(kv_mul, lb, q, S->G, scale, nchunk, n_lists, n_heads, S->part, out, s);
                else rc = launch_group<256>(kv_mul, lb, q, S->G, scale, nchunk, n_lists, n_heads, S->part, out, s);
            } else if (!rc) {
                if (d == 64) launch_attend<1>(dd, doff, dcnt, q, S->G, scale, nchunk, n_heads, S->part, out, s);
                else if (d == 128) launch_attend<2>(dd, doff, dcnt, q, S->G, scale, nchunk, n_heads, S->part, out, s);
                else launch_attend<4>(dd, doff, dcnt, q, S->G, scale, nchunk, n_heads, S->part, out, s);
                rc = vh_check(hipGetLastError());
            }
        }
    }
    // src/kvstore_ooc.c:182: released once read (the kernels are enqueued
    // before any copy that could reuse these blocks' memory)
    for (KvBlock *b : leased)
        if (b->lease > 0) b->lease--;
    return rc;
}

VireoKV *create(VireoKVConfig cfg, int strategy, int budget) {
    if (cfg.n_layers <= 0 || (cfg.kv_dim != 64 && cfg.kv_dim != 128 && cfg.kv_dim != 256) ||
        cfg.block_tokens < 1 || cfg.block_tokens > 64 || cfg.sink_tokens < 0 || cfg.window_tokens < 0)
        return nullptr;
    if (strategy < VIREO_KV_SELECT_ALL || strategy > VIREO_KV_SELECT_TOPK) return nullptr;
    VireoKV *S = new (std::nothrow) VireoKV;
    if (!S) return nullptr;
    S->cfg = cfg;
    S->strategy = strategy;
    S->budget = strategy == VIREO_KV_SELECT_TOPK ? (budget > 0 ? budget : 8) : 0;
    S->d = cfg.kv_dim;
    S->G = cfg.block_tokens;
    S->sink_blocks = blocks_for(cfg.sink_tokens, cfg.block_tokens);
    S->window_blocks = blocks_for(cfg.window_tokens, cfg.block_tokens);
    S->block_bytes = 2ull * uint64_t(cfg.block_tokens) * uint64_t(cfg.kv_dim) * sizeof(float);
    S->layers.resize(size_t(cfg.n_layers));
    for (int i = 0; i < kStageRing; i++)
        if (hipEventCreateWithFlags(&S->staged[i], hipEventDisableTiming) != hipSuccess) {
            S->staged[i] = nullptr;
            vireo_kv_destroy(S);
            return nullptr;
        }
    return S;
}

}  // namespace

extern "C" VireoKV *vireo_kv_create_dense(VireoKVConfig cfg) {
    cfg.capacity_bytes = 0;
    cfg.sink_tokens = 0;
    cfg.window_tokens = 0;
    VireoKV *S = create(cfg, VIREO_KV_SELECT_ALL, 0);
    if (S) S->dense = true;
    return S;
}

extern "C" VireoKV *vireo_kv_create_paged(VireoKVConfig cfg, int strategy, int topk_budget) {
    return create(cfg, strategy, topk_budget);
}

extern "C" VireoKV *vireo_kv_create_contiguous(VireoKVConfig cfg, int max_tokens) {
    cfg.capacity_bytes = 0;
    cfg.sink_tokens = 0;
    cfg.window_tokens = 0;
    if (max_tokens < 1) return nullptr;
    VireoKV *S = create(cfg, VIREO_KV_SELECT_ALL, 0);
    if (!S) return nullptr;
    S->dense = true;
    S->contig = true;
    S->max_blocks = blocks_for(max_tokens, S->G);
    const size_t nblk = size_t(cfg.n_layers) * S->max_blocks;
    if (hipMalloc(reinterpret_cast<void **>(&S->cbase), nblk * S->block_bytes) != hipSuccess ||
        hipMalloc(reinterpret_cast<void **>(&S->cksum), nblk * S->d * sizeof(float)) != hipSuccess ||
        hipMemset(S->cksum, 0, nblk * S->d * sizeof(float)) != hipSuccess) {
        vireo_kv_destroy(S);
        return nullptr;
    }
    for (size_t l = 0; l < S->layers.size(); l++) {
        S->layers[l].ksum = S->cksum + l * S->max_blocks * S->d;
        S->layers[l].cap = S->max_blocks;
    }
    return S;
}

int vh_kv_contig_view(const VireoKV *S, KvContigView *v) {
    if (!S || !S->contig || !v) return -EINVAL;
    *v = KvContigView{S->cbase, S->cksum, S->cfg.n_layers, S->max_blocks, S->G, S->d};
    return 0;
}

extern "C" int vireo_kv_append_pos(VireoKV *S, int layer0, int n, const int32_t *pos, const float *k, const float *v,
                                   void *stream) {
    if (!S || !S->contig || !pos || n < 1 || layer0 < 0 || layer0 + n > S->cfg.n_layers || !k || !v) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(kv_append_pos_kernel, dim3(n), dim3(S->d < 256 ? S->d : 256), 0, s, S->cbase, S->cksum, layer0,
                       S->max_blocks, S->max_blocks * S->G, pos, k, v, S->d, S->G);
    return vh_finish(s, vh_check(hipGetLastError()));
}

extern "C" int vireo_kv_attend_gqa_pos(VireoKV *S, int layer0, int n_heads, int n_kv_heads, const int32_t *pos,
                                       const float *q, float *out, void *stream) {
    if (!S || !S->contig || !pos || !q || !out || n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads ||
        layer0 < 0 || layer0 + n_kv_heads > S->cfg.n_layers || (reinterpret_cast<uintptr_t>(q) & 15u))
        return -EINVAL;
    const int kv_mul = n_heads / n_kv_heads, d = S->d;
    if (kv_mul != 1 && kv_mul != 2 && kv_mul != 4 && kv_mul != 8) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int nchunk = (S->max_blocks + kGroupBlocks - 1) / kGroupBlocks;
    const size_t pb = size_t(n_heads) * nchunk * (2 + d) * sizeof(float);
    if (int rc = grow(S, &S->part, &S->part_bytes, pb)) return rc;  // the first call sizes the partials
    const ContiguousBlocks cb{S->cbase, pos, layer0, S->max_blocks, S->G, d};
    const float scale = 1.0f / sqrtf(float(d));
    int rc;
    if (d == 64) rc = launch_group<64>(kv_mul, cb, q, S->G, scale, nchunk, n_kv_heads, n_heads, S->part, out, s);
    else if (d == 128) rc = launch_group<128>(kv_mul, cb, q, S->G, scale, nchunk, n_kv_heads, n_heads, S->part, out, s);
    else rc = launch_group<256>(kv_mul, cb, q, S->G, scale, nchunk, n_kv_heads, n_heads, S->part, out, s);
    return vh_finish(s, rc);
}

extern "C" int vireo_kv_append_n(VireoKV *S, int layer0, int n, int pos, const float *k, const float *v,
                                 void *stream) {
    (void)pos;  // tokens are appended in order, as in the reference
    if (!S || n < 1 || n > kMaxAppend || layer0 < 0 || layer0 + n > S->cfg.n_layers || !k || !v) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return vh_finish(s, append_n(S, layer0, n, k, v, s));
}

extern "C" int vireo_kv_append(VireoKV *S, int layer, int pos, const float *k, const float *v, void *stream) {
    return vireo_kv_append_n(S, layer, 1, pos, k, v, stream);
}

extern "C" int vireo_kv_attend_gqa(VireoKV *S, int layer0, int n_heads, int n_kv_heads, const float *q, float *out,
                                   void *stream) {
    if (!S || !q || !out || n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads || layer0 < 0 ||
        layer0 + n_kv_heads > S->cfg.n_layers)
        return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return vh_finish(s, attend(S, layer0, n_heads, n_heads / n_kv_heads, q, out, s));
}

extern "C" int vireo_kv_attend(VireoKV *S, int layer, const float *q, float *out, void *stream) {
    return vireo_kv_attend_gqa(S, layer, 1, 1, q, out, stream);
}

extern "C" void vireo_kv_stats(const VireoKV *S, VireoKVStats *out) {
    if (!S || !out) return;
    if (S->dense) {  // src/kvstore_dense.c:56-63: no counters; the appended tokens' bytes
        memset(out, 0, sizeof *out);
        for (const auto &L : S->layers)
            for (const auto &b : L.blocks) out->resident_bytes += uint64_t(b.ntok) * uint64_t(S->d) * 2 * sizeof(float);
        return;
    }
    *out = S->st;
    out->resident_bytes = S->resident_bytes;
    out->capacity_bytes = S->cfg.capacity_bytes;
}

extern "C" void vireo_kv_destroy(VireoKV *S) {
    if (!S) return;
    (void)hipDeviceSynchronize();
    for (auto &L : S->layers) {
        for (auto &b : L.blocks)
            if (b.host) (void)hipHostFree(b.host);
        if (L.ksum && !S->contig) (void)hipFree(L.ksum);
    }
    if (S->cbase) (void)hipFree(S->cbase);
    if (S->cksum) (void)hipFree(S->cksum);
    for (void *p : S->slabs) (void)hipFree(p);
    if (S->dscratch) (void)hipFree(S->dscratch);
    if (S->part) (void)hipFree(S->part);
    for (void *p : S->retired) (void)hipFree(p);
    for (int i = 0; i < kStageRing; i++) {
        if (S->hstage[i]) (void)hipHostFree(S->hstage[i]);
        if (S->staged[i]) (void)hipEventDestroy(S->staged[i]);
    }
    delete S;
}
