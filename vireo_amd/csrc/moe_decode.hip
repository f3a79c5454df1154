// Decode-path expert kernels (one token per call, the latency-bound case).
//
// decode_gateup_kernel (512 threads, one workgroup per CU): every workgroup
// needs the top-k, so each one ranks the router parts itself: wave 0 runs the
// one-wave top-k while the other waves load the expert table into LDS, and
// every wave loads its slice of the input vector into registers - all of it
// issued before anything is used. Then each wave computes RPW rows of gate and
// up of the chosen expert blockIdx.y, a whole wave per row (lane l owns item
// l of every row, so its inputs and their run sums are loaded once), and
// writes h[j][o] = silu(gate_o . x) * (up_o . x) (src/gguf_run.c:205-207).
// A token whose top-k order is not certified by the fast wave is ranked again
// by the whole workgroup with exact logits (route_topk_block).
//
// down_combine_kernel (256 threads): a workgroup owns R output rows for all k
// chosen experts. Groups of L lanes each keep one expert's activations for
// their items in registers and take kDnRpg rows of that expert; the per-row
// results meet in LDS and x[o] += sum_j w_j * y_j is formed in selection order
// (src/gguf_run.c:208-213). Every output element has one writer: no atomics.
#include <hip/hip_runtime.h>
#include <algorithm>
#include "common.h"
#include "qdecode.h"
#include "route.h"
#include "route_kernels.h"

namespace {

int64_t row_bytes_of(uint32_t t, int n) {
    switch (t) {
    case VT_Q8_0: return int64_t(n / 32) * 34;
    case VT_Q4_K: return int64_t(n / 256) * 144;
    case VT_Q6_K: return int64_t(n / 256) * 210;
    case VT_Q5_0: return int64_t(n / 32) * 22;
    case VT_F16: return int64_t(n) * 2;
    default: return int64_t(n) * 4;
    }
}

// ------------------------------------------------------------------ fused top-k + gate/up
constexpr int kGuWaves = 8;

// grid (ceil(fe / (kGuWaves * RPW)), k), 512 threads, d = 2048 (lane l owns
// item l of a row), E <= 64 * Q. The arguments the prologue needs come first:
// they are the ones preloaded into SGPRs at launch.
// Warm-up of the down rows (pf_rows > 0): workgroup L runs on XCD L % 8,
// and so does the down kernel's workgroup b (rows [pf_rows b, pf_rows (b + 1))
// of every chosen expert) for b = L % 8 (mod 8). With gridDim.x and the down
// grid nbd both multiples of 8, the gridDim.x / 8 gate/up workgroups of expert
// slot j on XCD x share the nbd / 8 down workgroups b = x + 8 i of that XCD
// (i = q mod gridDim.x / 8 for the workgroup with blockIdx.x = x' + 8 q) and
// load one word of every 64-byte line of those rows of expert j's down
// matrix. Measured on MI355X: the down kernel's L2 miss bytes (FETCH_SIZE)
// are the same with or without it, so its reads are served from beyond the L2
// (the memory-side Infinity Cache), and this XCD-matched split is faster than
// a contiguous split of each matrix (18.3 against 18.65 us per Qwen3 layer).
constexpr int kPfPerThread = 3;  // warm-up lines per thread: at most 1536 per workgroup

template <int T, int Q, int RPW, bool ST>
__global__ void __launch_bounds__(512) decode_gateup_kernel(const RoutePart *__restrict__ parts,
                                                            const float *__restrict__ hb,
                                                            const void *const *__restrict__ table, int E, int k,
                                                            int fe, int d, int renorm, int64_t row_bytes,
                                                            const float *__restrict__ R,
                                                            const float *__restrict__ bias, float *__restrict__ h,
                                                            int32_t *__restrict__ idx_out, float *__restrict__ w_out,
                                                            uint32_t *__restrict__ flags_out,
                                                            DecodePlan *__restrict__ plan, int pf_rows, int pf_nbd,
                                                            int64_t pf_rb, NormRef nref,
                                                            uint64_t *__restrict__ stamps) {
    using F = Reg<T>;
    // stamps: 0 start, 1 router parts loaded, 2 top-k chosen, 3 first gate/up
    // row computed, 4 every row written, 7 1 when the order took the exact path
    PhaseStamps<ST> ps(stamps);
    ps.now(0);
    constexpr int NS = F::NS, TPL = 3 * Q;
    __shared__ TopKSmem sm;         // the exact fallback's workspace
    __shared__ __align__(16) float xref[2048];  // the fallback's inputs (with a library-normalised hb: the reference's xb)
    __shared__ float2 stage[64];    // the weights, in the workgroup that writes the plan
    __shared__ double2 cert[kGuWaves][64];  // per wave: the chosen experts' intervals
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int j = blockIdx.y;

    // 1. every load of the prologue, issued before any of them is used: the
    //    router parts, the layer's expert table (spread over the lanes) and
    //    this lane's item of the input
    // (unconditional: entries past E and 3 E repeat the last one; their keys
    // are masked in the selection and table_entry never reads them, so the
    // selection waits only for the parts)
    RoutePart p[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) p[q] = parts[min(lane + 64 * q, E - 1)];
    const void *tab[TPL];
#pragma unroll
    for (int s = 0; s < TPL; s++) tab[s] = table[min(TPL * lane + s, 3 * E - 1)];
    float xr[32], xs[NS];
    F::load_x(hb, lane, xr);
    F::sums(xr, xs);

    // 2. every wave selects on its own (no LDS, no barrier); a token whose
    //    order is not certified (the same verdict in every wave) is ranked
    //    again by the whole workgroup on exact logits
    int e_j, e_unused, rank[Q];
    ps.after(1, p[0].c);
    const bool ok = route_select_wave<Q>(p, E, k, j, e_j, j, e_unused, rank, cert[wv]);
    ps.mark(7, ok ? 0u : 1u);
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
    if (!ok) {
        const float *xe = hb;
        if (nref.x) {  // rank on the reference's own xb, not on the fp64-normalised hb
            reference_rmsnorm_block(xref, nref.x, nref.nw, nref.eps, d, &sm.red[0][0]);
            xe = xref;
        }
        // d = 2048: the contenders' chains are shared by the waves (no row buffers in LDS)
        route_topk_block(sm, parts, R, xe, bias, d, E, k, renorm, false, nullptr);
        e_j = sm.sel[j];
        if (writer && wv == 0 && lane < k) {
            const int e = sm.sel[lane];
            idx_out[lane] = e;
            w_out[lane] = sm.sel_w[lane];
            plan->w[lane] = sm.sel_w[lane];
            plan->down[lane] = table[3 * e + 2];
        }
        if (writer && tid == 0 && flags_out) flags_out[0] = sm.flag;
    } else if (writer && wv == 0) {
        int e;
        float w;
        route_weights_wave<Q>(p, rank, E, k, renorm, stage, e, w);
        // the down matrix from the table this wave already holds (a reload
        // from memory would hold the wave's own rows back by a round trip)
        const void *dn = table_gather<TPL>(tab, 3 * e + 2);
        if (lane < k) {
            idx_out[lane] = e;
            w_out[lane] = w;
            plan->w[lane] = w;
            plan->down[lane] = dn;
        }
        if (lane == 0 && flags_out) flags_out[0] = 0u;
    }

    // 3. RPW rows of gate and up of the chosen expert j, their loads first,
    //    then the down rows' warm-up. (Writing the plan after those loads
    //    instead of before measured slower: Qwen3 18.58 -> 18.97 us per layer,
    //    OLMoE Q8_0 24.08 -> 26.64.)
    ps.after(2, e_j);
    const uint8_t *G = table_entry<TPL>(tab, 3 * e_j);
    const uint8_t *U = table_entry<TPL>(tab, 3 * e_j + 1);
    const int o0 = (blockIdx.x * kGuWaves + wv) * RPW;
    if (!G || !U) {  // unregistered expert: contributes nothing (src/gguf_run.c:201)
#pragma unroll
        for (int r = 0; r < RPW; r++)
            if (lane == 63 && o0 + r < fe) h[size_t(j) * fe + o0 + r] = 0.0f;
        return;
    }
    typename F::Raw rg[RPW], ru[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int64_t o = min(o0 + r, fe - 1);
        rg[r] = F::fetch(gmem(G), o * row_bytes, lane);
        ru[r] = F::fetch(gmem(U), o * row_bytes, lane);
    }
    // the down rows' warm-up, issued after this workgroup's own loads.
    // Unconditional loads (threads past the last line repeat it) whose values
    // are used only by the asm statement at the end, so no wait for them, or
    // for the weights issued before them, comes earlier.
    uint32_t pf[kPfPerThread] = {};
    const uint8_t *D = table_entry<TPL>(tab, 3 * e_j + 2);
    if (pf_rows > 0 && D) {
        const int gq = gridDim.x >> 3, x8 = (blockIdx.y * gridDim.x + blockIdx.x) & 7, q = blockIdx.x >> 3;
        const int64_t span = int64_t(pf_rows) * pf_rb;           // bytes of one down workgroup's rows
        const int lines = int((span + 63) >> 6), per = (pf_nbd >> 3) / gq;  // down workgroups per gate/up one
#pragma unroll
        for (int u = 0; u < kPfPerThread; u++) {
            const int t = min(tid + 512 * u, per * lines - 1);
            const int i = q + gq * (t / lines), b = x8 + 8 * i;
            const int64_t off = (int64_t(b) * span + int64_t(t % lines) * 64) & ~int64_t(3);
            pf[u] = ld_u32(gmem(D) + off);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float g = F::compute(rg[r], lane, xr, xs);
        float u = F::compute(ru[r], lane, xr, xs);
        g = group_sum<64>(g);
        u = group_sum<64>(u);
        if (lane == 63 && o0 + r < fe) h[size_t(j) * fe + o0 + r] = swiglu(g, u);
        if (r == 0) ps.after(3, g);
    }
#pragma unroll
    for (int u = 0; u < kPfPerThread; u++) asm volatile("" ::"v"(pf[u]));  // keeps the warm-up loads
    ps.now(4);
    ps.store();
}

// ------------------------------------------------------------------ decode batch: top-k + gate/up
// decode_batch_gateup_kernel (512 threads, one or two workgroups per CU): the
// one-token kernel's work for nt tokens in one launch. Wave w < nt ranks
// token w with route_select_wave on the same parts and with the same
// certification as decode_gateup_kernel; a token whose order is not certified
// is ranked again by the whole workgroup on exact logits (route_topk_block).
// The tokens' chosen experts are merged into the ascending list of distinct
// experts, and the (distinct expert, gate/up row) items are cut into equal
// contiguous ranges, one per wave of the grid. A wave keeps D items' gate
// and up rows in flight (4, or 2 where two workgroups share a CU) and
// multiplies each row with every token that
// chose its expert, their inputs and run sums held in LDS in each lane's item
// order. h[t k + j][o] is formed with the operations of decode_gateup_kernel,
// so each token's activations - and, through down_combine_kernel, its output -
// are the bits of a one-token call. The outputs of a wave's items gather in
// LDS and are written after its last row (a store between the rows' loads
// would make the waits for them count a data-dependent number of stores),
// where the SwiGLU of each is formed by the wave's lanes side by side.
constexpr int kBgXPad = 36;  // a lane's 32 inputs, then their run sums (at most 4)
// the inputs' and outputs' LDS (dynamic; with the kernel's 23 KB of static LDS)
constexpr size_t kBgDynBytes = 128 * 1024;
__host__ __device__ inline size_t batch_xl_bytes(int nt) { return size_t(nt) * 64 * kBgXPad * sizeof(float); }

// D: items in flight per wave. D = 2 holds the kernel to 128 registers, so
// that two workgroups share a CU where their LDS fits.
template <int T, int Q, int D>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(D == 2 ? 4 : 1))) decode_batch_gateup_kernel(
    const RoutePart *__restrict__ parts, const float *__restrict__ hb, const void *const *__restrict__ table, int E,
    int k, int fe, int nt, int renorm, int64_t row_bytes, const float *__restrict__ R, const float *__restrict__ bias,
    float *__restrict__ h, int32_t *__restrict__ idx_out, float *__restrict__ w_out, uint32_t *__restrict__ flags_out,
    DecodePlan *__restrict__ plan, int cap) {
    using F = Reg<T>;
    constexpr int NS = F::NS, TPL = 3 * Q, NB = kDecodeBatchMax, d = 2048;
    static_assert(NS <= kBgXPad - 32, "the run sums fit in the lane's pad");
    __shared__ TopKSmem sm;                               // the exact ranking of an uncertified token
    __shared__ double2 cert[kGuWaves][64];
    __shared__ float2 stage[kGuWaves][64];
    __shared__ int sel[NB][64];           // token t's experts in selection order
    __shared__ float wsel[NB][64];        // and their weights (the plan writer's)
    __shared__ uint64_t chosen[NB][Q];    // token t: bit e % 64 of word e / 64 when it chose e
    __shared__ uint64_t uni[Q];           // their union
    __shared__ uint32_t okv[NB], flagv[NB];
    __shared__ int dlist[64];             // the distinct experts, ascending
    __shared__ uint64_t pmask[64];        // entry n: bit t k + j when token t's round j chose dlist[n]
    __shared__ int ndist;
    // dynamic LDS: token t, lane l: the inputs of item l, then their sums (at
    // xl + (64 t + l) kBgXPad); then per wave cap outputs
    extern __shared__ float4 dynl[];
    float *xl = reinterpret_cast<float *>(dynl);
    float4 *outbuf = dynl + batch_xl_bytes(nt) / sizeof(float4);
    // the wave index through readfirstlane: the compiler then keeps everything
    // derived from it (the item cursor, the pair masks) in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tw = min(wv, nt - 1);  // the token this wave ranks (waves past the last repeat it, writing nothing)
    const bool writer = blockIdx.x == 0;

    // 1. the prologue's loads, unconditional so that each wait counts exactly
    //    the loads issued after it: the router parts of token tw, the layer's
    //    expert table spread over the lanes (entries past 3 E repeat the last
    //    one and are never read) and this lane's item of token tw's input
    RoutePart p[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) p[q] = parts[size_t(tw) * E + min(lane + 64 * q, E - 1)];
    const void *tab[TPL];
#pragma unroll
    for (int s = 0; s < TPL; s++) tab[s] = table[min(TPL * lane + s, 3 * E - 1)];
    float xr[32];
    F::load_x(hb + size_t(tw) * d, lane, xr);

    // 2. token tw ranked and certified by this wave alone
    int e_unused0, e_unused1, rank[Q];
    const bool ok = route_select_wave<Q>(p, E, k, 0, e_unused0, 0, e_unused1, rank, cert[wv]);
    if (wv < nt) {
#pragma unroll
        for (int q = 0; q < Q; q++) {
            if (rank[q] >= 0) sel[wv][rank[q]] = lane + 64 * q;
            const uint64_t m = __ballot(rank[q] >= 0);
            if (lane == 0) chosen[wv][q] = m;
        }
        if (lane == 0) {
            okv[wv] = ok ? 1u : 0u;
            flagv[wv] = 0u;
        }
        if (ok && writer) {
            int e;
            float w;
            route_weights_wave<Q>(p, rank, E, k, renorm, stage[wv], e, w);
            if (lane < k) wsel[wv][lane] = w;
        }
        float xs[NS];
        F::sums(xr, xs);
        float4 *dst = reinterpret_cast<float4 *>(xl + (size_t(wv) * 64 + lane) * kBgXPad);
#pragma unroll
        for (int i = 0; i < 8; i++) dst[i] = make_float4(xr[4 * i], xr[4 * i + 1], xr[4 * i + 2], xr[4 * i + 3]);
        float sp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NS; i++) sp[i] = xs[i];
        dst[8] = make_float4(sp[0], sp[1], sp[2], sp[3]);
    }
    __syncthreads();

    // 3. the tokens whose order the bounds leave open, ranked again on exact
    //    logits by the whole workgroup (the same verdict in every workgroup)
    for (int t = 0; t < nt; t++) {
        if (okv[t]) continue;
        route_topk_block(sm, parts + size_t(t) * E, R, hb + size_t(t) * d, bias, d, E, k, renorm, false, nullptr);
        if (tid < k) {
            sel[t][tid] = sm.sel[tid];
            wsel[t][tid] = sm.sel_w[tid];
        }
        if (tid == 0) flagv[t] = sm.flag;
        if (tid < 64 * Q) {  // wave q: word q of token t's chosen set
            bool c = false;
            for (int j = 0; j < k; j++) c = c || sm.sel[j] == tid;
            const uint64_t m = __ballot(c);
            if (lane == 0) chosen[t][wv] = m;
        }
        __syncthreads();
    }

    // 4. the distinct experts in ascending order, the pairs that chose each,
    //    and (workgroup 0) the routing and the down kernel's plan
    if (tid < Q) {
        uint64_t u = 0;
        for (int t = 0; t < nt; t++) u |= chosen[t][tid];
        uni[tid] = u;
    }
    __syncthreads();
    if (tid < 64 * Q) {  // thread e: expert e
        const uint64_t u = uni[wv];
        int before = __popcll(u & ((uint64_t(1) << lane) - 1));
        for (int q = 0; q < wv; q++) before += __popcll(uni[q]);
        const bool in = (u >> lane) & 1u;
        if (in) {
            dlist[before] = tid;
            pmask[before] = 0;
        }
        if (tid == 64 * Q - 1) ndist = before + (in ? 1 : 0);
    }
    __syncthreads();
    const int P = nt * k;  // at most 64: the pairs are wave 0's lanes
    if (wv == 0) {
        const int pp = min(tid, P - 1);  // lanes past the last pair repeat it (the gather needs every lane)
        const int t = pp / k, j = pp - t * k, e = sel[t][j];
        const void *dn = table_gather<TPL>(tab, 3 * e + 2);  // the down matrix without a memory round trip
        if (tid < P) {
            int pos = __popcll(uni[e >> 6] & ((uint64_t(1) << (e & 63)) - 1));
            for (int q = 0; q < (e >> 6); q++) pos += __popcll(uni[q]);
            atomicOr(reinterpret_cast<unsigned long long *>(&pmask[pos]), 1ull << tid);
            if (writer) {
                idx_out[tid] = e;
                w_out[tid] = wsel[t][j];
                plan->w[tid] = wsel[t][j];
                plan->down[tid] = dn;
            }
        }
    }
    if (writer && tid < nt && flags_out) flags_out[tid] = flagv[tid];
    __syncthreads();

    // 5. this wave's items i in [i0, i1): distinct expert n = i / fe, row o = i % fe
    const int total = ndist * fe, W = int(gridDim.x) * kGuWaves;
    const int per = (total + W - 1) / W, gw = int(blockIdx.x) * kGuWaves + wv;
    const int i0 = min(gw * per, total), i1 = min(i0 + per, total);
    if (i0 >= i1) return;
    float4 *ob = outbuf + size_t(wv) * cap;  // (g, u, index in h) of each output, SwiGLU at the end
    int nout = 0;
    // an unregistered expert's items load from hb (any readable row bytes) and write zeros (src/gguf_run.c:201)
    const uint8_t *spare = reinterpret_cast<const uint8_t *>(hb);
    // the fetch cursor (uniform): item ic = (distinct expert nc, row oc), that expert's rows and pairs
    int ic = i0, nc = i0 / fe, oc = i0 - nc * fe;
    const uint8_t *Gc = nullptr, *Uc = nullptr;
    uint64_t pmc = 0;
    auto expert = [&]() {
        const int e = __builtin_amdgcn_readfirstlane(dlist[nc]);
        Gc = table_entry<TPL>(tab, 3 * e);
        Uc = table_entry<TPL>(tab, 3 * e + 1);
        const uint64_t v = pmask[nc];
        pmc = (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v >> 32))))) << 32) |
              uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v))));
    };
    expert();
    typename F::Raw rg[D], ru[D];
    uint64_t spm[D];
    int so[D];
    bool slive[D];
    // slot u: the cursor's item, then the cursor moves on (past the range it stays on the last item, fetched
    // again: every slot issues the same loads, so the waits stay exact)
    auto fetch = [&](int u) {
        const bool live = Gc && Uc;
        const int64_t off = int64_t(oc) * row_bytes;
        rg[u] = F::fetch(gmem(live ? Gc + off : spare), 0, lane);
        ru[u] = F::fetch(gmem(live ? Uc + off : spare), 0, lane);
        spm[u] = pmc;
        so[u] = oc;
        slive[u] = live;
        if (ic + 1 < i1) {
            ic++;
            if (++oc == fe) {
                oc = 0;
                nc++;
                expert();
            }
        }
    };
    int xt = -1;  // the token whose inputs xv / xs hold
    float xv[32], xs[NS];
    const int mk = (65536 + k - 1) / k;  // t = p / k as (p * mk) >> 16, exact for p < 64 and k <= 64
    auto compute = [&](int u) {
        uint64_t pm = spm[u];
        while (pm) {
            const int pr = __builtin_ctzll(pm);
            pm &= pm - 1;
            const int t = (pr * mk) >> 16;
            if (t != xt) {
                xt = t;
                const float4 *src = reinterpret_cast<const float4 *>(xl + (size_t(t) * 64 + lane) * kBgXPad);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float4 v = src[q];
                    xv[4 * q] = v.x;
                    xv[4 * q + 1] = v.y;
                    xv[4 * q + 2] = v.z;
                    xv[4 * q + 3] = v.w;
                }
                const float4 sv = src[8];
                const float sa[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                for (int q = 0; q < NS; q++) xs[q] = sa[q];
            }
            float g = F::compute(rg[u], lane, xv, xs);
            float v = F::compute(ru[u], lane, xv, xs);
            g = group_sum<64>(g);
            v = group_sum<64>(v);
            if (lane == 63)
                ob[nout] = slive[u] ? make_float4(g, v, __int_as_float(pr * fe + so[u]), 0.0f)
                                    : make_float4(0.0f, 0.0f, __int_as_float(pr * fe + so[u]), 0.0f);
            nout++;
        }
    };
#pragma unroll
    for (int u = 0; u < D; u++) fetch(u);
    for (int c = i0; c < i1; c += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (c + u < i1) compute(u);
            fetch(u);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // swiglu(0, 0) = +0: an unregistered expert's rows (src/gguf_run.c:201)
    for (int q = lane; q < nout; q += 64) {
        const float4 v = ob[q];
        h[__float_as_int(v.z)] = swiglu(v.x, v.y);
    }
}

// The down kernel's row blocks, for the warm-up (0 rows: none).
struct DownPrefetch {
    int rows, nbd;
    int64_t rb;
};

template <int T, int Q, int RPW>
int launch_decode_gateup(const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E,
                         int k, int fe, int renorm, const void *const *table, int64_t rb, float *h, int32_t *idx,
                         float *w, uint32_t *flags, DecodePlan *plan, DownPrefetch pf, NormRef nref, hipStream_t s) {
    constexpr int rows_per_block = kGuWaves * RPW;
    dim3 g((fe + rows_per_block - 1) / rows_per_block, k);
    bool warm = pf.rows > 0 && g.x % 8 == 0 && pf.nbd % 8 == 0 && (pf.nbd / 8) % (g.x / 8) == 0;
    if (warm) {  // every line of the workgroup's share within kPfPerThread loads per thread
        const int64_t lines = (int64_t(pf.rows) * pf.rb + 63) / 64, per = (pf.nbd / 8) / (g.x / 8);
        warm = per * lines <= 512 * kPfPerThread;
    }
    if (uint64_t *st = vh_stamps_for(1))
        VH_LAUNCH((decode_gateup_kernel<T, Q, RPW, true>), g, dim3(64 * kGuWaves), 0, s, parts, hb, table, E, k, fe,
                  d, renorm, rb, R, bias, h, idx, w, flags, plan, warm ? pf.rows : 0, pf.nbd, pf.rb, nref, st);
    else
        VH_LAUNCH((decode_gateup_kernel<T, Q, RPW, false>), g, dim3(64 * kGuWaves), 0, s, parts, hb, table, E, k, fe,
                  d, renorm, rb, R, bias, h, idx, w, flags, plan, warm ? pf.rows : 0, pf.nbd, pf.rb, nref, nullptr);
    return vh_check(hipGetLastError());
}

// rows per wave so that about 256 workgroups (one per CU) cover the k experts
int gateup_rpw(int fe, int k) {
    const int want = (fe * k + 256 * kGuWaves - 1) / (256 * kGuWaves);
    return want <= 2 ? 2 : want <= 3 ? 3 : 4;
}

template <int T, int Q>
int launch_gateup_rpw(int rpw, const RoutePart *parts, const float *R, const float *hb, const float *bias, int d,
                      int E, int k, int fe, int renorm, const void *const *table, int64_t rb, float *h, int32_t *idx,
                      float *w, uint32_t *flags, DecodePlan *plan, DownPrefetch pf, NormRef nref, hipStream_t s) {
    if (rpw == 2)
        return launch_decode_gateup<T, Q, 2>(parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags,
                                             plan, pf, nref, s);
    if (rpw == 3)
        return launch_decode_gateup<T, Q, 3>(parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags,
                                             plan, pf, nref, s);
    return launch_decode_gateup<T, Q, 4>(parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan,
                                         pf, nref, s);
}

template <int T>
int launch_gateup_t(int rpw, const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E,
                    int k, int fe, int renorm, const void *const *table, int64_t rb, float *h, int32_t *idx, float *w,
                    uint32_t *flags, DecodePlan *plan, DownPrefetch pf, NormRef nref, hipStream_t s) {
    if (E <= 64)
        return launch_gateup_rpw<T, 1>(rpw, parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags,
                                       plan, pf, nref, s);
    if (E <= 128)
        return launch_gateup_rpw<T, 2>(rpw, parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags,
                                       plan, pf, nref, s);
    return launch_gateup_rpw<T, 4>(rpw, parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan,
                                   pf, nref, s);
}

// A wave's outputs in decode_batch_gateup_kernel on a grid of g workgroups:
// its items (at most min(nt k, E) experts' fe rows over the grid's waves) times
// the tokens that chose an item's expert.
int batch_out_cap(int E, int k, int fe, int nt, int g) {
    const int64_t items = (int64_t(std::min(nt * k, E)) * fe + int64_t(g) * kGuWaves - 1) / (int64_t(g) * kGuWaves);
    return int(items * nt);
}

// The dynamic LDS of a grid of g workgroups: the inputs, then every wave's outputs.
size_t batch_lds(int E, int k, int fe, int nt, int g) {
    return batch_xl_bytes(nt) + size_t(kGuWaves) * batch_out_cap(E, k, fe, nt, g) * sizeof(float4);
}

// The kernel's static LDS, and its dynamic LDS limit raised to kBgDynBytes
// (once per process and instantiation); 0 on failure.
template <int T, int Q, int D>
size_t batch_static_lds() {
    static size_t bytes = 0;
    if (bytes == 0) {
        const void *f = reinterpret_cast<const void *>(&decode_batch_gateup_kernel<T, Q, D>);
        hipFuncAttributes a{};
        if (hipFuncGetAttributes(&a, f) != hipSuccess ||
            hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(kBgDynBytes)) != hipSuccess)
            return 0;
        bytes = a.sharedSizeBytes;
    }
    return bytes;
}

template <int T, int Q>
int launch_batch_gateup(const RoutePart *parts, const float *R, const float *hb, const float *bias, int E, int k,
                        int fe, int renorm, const void *const *table, int64_t rb, float *h, int32_t *idx, float *w,
                        uint32_t *flags, DecodePlan *plan, int nt, hipStream_t s) {
    constexpr size_t kCuLds = 160 * 1024;
    const int cus = vh_num_cus();
    // two workgroups per CU (two items in flight per wave, 128 registers)
    // where both workgroups' LDS fits in the CU's, else one (four in flight)
    const size_t lds2 = batch_lds(E, k, fe, nt, 2 * cus), st2 = batch_static_lds<T, Q, 2>();
    if (st2 && 2 * (st2 + lds2) <= kCuLds) {
        VH_LAUNCH((decode_batch_gateup_kernel<T, Q, 2>), dim3(2 * cus), dim3(64 * kGuWaves), lds2, s, parts, hb, table,
                  E, k, fe, nt, renorm, rb, R, bias, h, idx, w, flags, plan, batch_out_cap(E, k, fe, nt, 2 * cus));
        return vh_check(hipGetLastError());
    }
    const size_t lds = batch_lds(E, k, fe, nt, cus), st4 = batch_static_lds<T, Q, 4>();
    if (!st4 || lds > kBgDynBytes) return -EINVAL;
    VH_LAUNCH((decode_batch_gateup_kernel<T, Q, 4>), dim3(cus), dim3(64 * kGuWaves), lds, s, parts, hb, table, E, k,
              fe, nt, renorm, rb, R, bias, h, idx, w, flags, plan, batch_out_cap(E, k, fe, nt, cus));
    return vh_check(hipGetLastError());
}

template <int T>
int launch_batch_gateup_t(const RoutePart *parts, const float *R, const float *hb, const float *bias, int E, int k,
                          int fe, int renorm, const void *const *table, int64_t rb, float *h, int32_t *idx, float *w,
                          uint32_t *flags, DecodePlan *plan, int nt, hipStream_t s) {
    if (E <= 64)
        return launch_batch_gateup<T, 1>(parts, R, hb, bias, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, nt, s);
    if (E <= 128)
        return launch_batch_gateup<T, 2>(parts, R, hb, bias, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, nt, s);
    return launch_batch_gateup<T, 4>(parts, R, hb, bias, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, nt, s);
}

// ------------------------------------------------------------------ down + combine
constexpr int kDnRpg = 2;  // rows per lane group

// grid (d / R, tokens), 256 threads, R = kDnRpg * (256 / L) / k. Lane group
// g (L lanes) takes expert g % k and rows g / k + i * (256 / L / k), i <
// kDnRpg; lane li of the group owns items li, li + L, ... (at most IPL) of
// those rows. MT (a decode batch): workgroup row y takes token y - its
// selection's plan entries y k .. y k + k - 1, activations h[y k + j] and
// output row x[y] - with the same operations as a one-token call.
template <int T, int L, int IPL, bool ST, bool MT = false>
__global__ void __launch_bounds__(256) down_combine_kernel(const DecodePlan *__restrict__ plan,
                                                           const float *__restrict__ h, int d, int fe, int k, int R,
                                                           int64_t row_bytes, float *__restrict__ x,
                                                           uint64_t *__restrict__ stamps) {
    using F = Reg<T>;
    // stamps: 0 start, 1 plan loaded, 2 first row computed, 3 every row
    // computed (after the barrier), 4 outputs written
    PhaseStamps<ST> ps(stamps);
    ps.now(0);
    constexpr int NS = F::NS, NG = 256 / L;
    extern __shared__ float ys[];  // [k][R]
    const int tid = threadIdx.x, g = tid / L, li = tid % L;
    const int j = g % k, rstep = NG / k, rf = g / k;
    const int o0 = blockIdx.x * R;
    const int items = F::items(fe);
    const int lane = tid & 63;
    const void *const *pdown = plan->down;
    const float *pw = plan->w;
    int l2 = lane;
    if constexpr (MT) {
        const int y = blockIdx.y;
        pdown += y * k;
        pw += y * k;
        h += size_t(y) * k * fe;
        x += size_t(y) * d;
        l2 = lane < k ? lane : 0;  // within this token's k entries
    }
    const uint8_t *D = static_cast<const uint8_t *>(pdown[j]);
    // what the combine needs, loaded now: lane j2 < k of wave 0 holds expert
    // j2's weight and whether its lookup succeeded, thread tid < R its output
    // (unconditional loads: DecodePlan has 64 entries and lanes past k are not
    // read; the pointer is tested only in the combine, so nothing waits for it
    // earlier)
    const void *dj2 = pdown[l2];
    const float wj2 = pw[l2];
    const float xo = x[o0 + min(tid, R - 1)];
    // activations of expert j for this lane's items (independent of the plan;
    // items past the row repeat its last one, and their products are skipped)
    float xv[IPL][32], xs[IPL][NS];
#pragma unroll
    for (int m = 0; m < IPL; m++) F::load_x(h + size_t(j) * fe, min(li + L * m, items - 1), xv[m]);
    // every lane loads (items past the row repeat its last one and are not
    // used), through a global-address-space pointer, with no branch: all the
    // loads are in flight before the first is used. A failed lookup's lanes
    // load the first row bytes of h instead (readable; their values are not
    // used): inside a branch the compiler waits for nearly every load before
    // leaving it.
    typename F::Raw raw[kDnRpg][IPL];
    gbyte *Dg = D ? gmem(D) : gmem(h);
    const int64_t rsel = D ? row_bytes : 0;
#pragma unroll
    for (int rr = 0; rr < kDnRpg; rr++)
#pragma unroll
        for (int m = 0; m < IPL; m++)
            raw[rr][m] = F::fetch(Dg, int64_t(o0 + rf + rr * rstep) * rsel, min(li + L * m, items - 1));
#pragma unroll
    for (int m = 0; m < IPL; m++) F::sums(xv[m], xs[m]);
    ps.after(1, wj2);
#pragma unroll
    for (int rr = 0; rr < kDnRpg; rr++) {
        float acc = 0.0f;
        if (D) {
#pragma unroll
            for (int m = 0; m < IPL; m++) {
                const int it = li + L * m;
                if (it < items) acc += F::compute(raw[rr][m], it, xv[m], xs[m]);
            }
        }
        acc = group_sum<L>(acc);
        if (li == L - 1) ys[j * R + rf + rr * rstep] = acc;
        if (rr == 0) ps.after(2, acc);
    }
    __syncthreads();
    ps.now(3);
    if (tid < 64) {  // R <= 64: the combining threads are in wave 0
        const int pres = dj2 != nullptr;
        float a = 0.0f;
        for (int j2 = 0; j2 < k; j2++) {
            const int present = __builtin_amdgcn_readlane(pres, j2);
            const float wv2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wj2), j2));
            if (!present) continue;  // failed lookup: skipped (src/gguf_run.c:201)
            if (tid < R) a = add_rn(a, mul_rn(wv2, ys[j2 * R + tid]));
        }
        if (tid < R) x[o0 + tid] = add_rn(xo, a);
    }
    ps.now(4);
    ps.store();
}

// Lanes per row: the smallest of 8 / 16 / 32 with at most 3 items per lane and
// 256 / L lane groups divisible by k; 0 if none fits.
int down_lanes(int items, int k) {
    for (int L : {8, 16, 32})
        if ((items + L - 1) / L <= 3 && (256 / L) % k == 0) return L;
    return 0;
}

template <int T, int L, int IPL>
int launch_down(const DecodePlan *plan, const float *h, int d, int fe, int k, float *x, int nt, hipStream_t s) {
    const int R = kDnRpg * (256 / L) / k;
    const int64_t rb = row_bytes_of(T, fe);
    const dim3 g(d / R, nt);
    const uint32_t lds = uint32_t(size_t(k) * R * 4);
    if (nt > 1)
        VH_LAUNCH((down_combine_kernel<T, L, IPL, false, true>), g, dim3(256), lds, s, plan, h, d, fe, k, R, rb, x,
                  nullptr);
    else if (uint64_t *st = vh_stamps_for(2))
        VH_LAUNCH((down_combine_kernel<T, L, IPL, true>), g, dim3(256), lds, s, plan, h, d, fe, k, R, rb, x, st);
    else
        VH_LAUNCH((down_combine_kernel<T, L, IPL, false>), g, dim3(256), lds, s, plan, h, d, fe, k, R, rb, x, nullptr);
    return vh_check(hipGetLastError());
}

template <int T>
int launch_down_t(const DecodePlan *plan, const float *h, int d, int fe, int k, float *x, int nt, hipStream_t s) {
    const int items = Reg<T>::items(fe), L = down_lanes(items, k);
    if (!L) return -EINVAL;
    const int ipl = (items + L - 1) / L;
    if (L == 8)
        return ipl <= 2 ? launch_down<T, 8, 2>(plan, h, d, fe, k, x, nt, s)
                        : launch_down<T, 8, 3>(plan, h, d, fe, k, x, nt, s);
    if (L == 16)
        return ipl <= 2 ? launch_down<T, 16, 2>(plan, h, d, fe, k, x, nt, s)
                        : launch_down<T, 16, 3>(plan, h, d, fe, k, x, nt, s);
    return ipl <= 2 ? launch_down<T, 32, 2>(plan, h, d, fe, k, x, nt, s)
                    : launch_down<T, 32, 3>(plan, h, d, fe, k, x, nt, s);
}

}  // namespace

bool vh_decode_gateup_supported(uint32_t type, int d, int fe) {
    return d == 2048 && fe >= 1 && (type == VT_Q4_K || type == VT_Q8_0 || type == VT_Q6_K);
}

int vh_decode_gateup(uint32_t type, const RoutePart *parts, const float *R, const float *hb, const float *bias, int d,
                     int E, int k, int fe, int renorm, const void *const *table, float *h, int32_t *idx, float *w,
                     uint32_t *flags, DecodePlan *plan, uint32_t down_type, NormRef nref, hipStream_t s) {
    if (!vh_decode_gateup_supported(type, d, fe) || E > kMaxExperts || k > 64) return -EINVAL;
    const int64_t rb = row_bytes_of(type, d);
    const int rpw = gateup_rpw(fe, k);
    // The warm-up moves the down weights' HBM latency into the gate/up kernel;
    // measured on MI355X it shortens the layer for every shape built here
    // (by 0.9-1.9 us), including those whose selected gate/up and down bytes
    // exceed an XCD's 4 MB L2.
    DownPrefetch pf{0, 0, 0};
    if (down_type && vh_down_combine_supported(down_type, d, fe, k)) {
        const int L = down_lanes(Reg<VT_Q8_0>::items(fe), k);
        pf.rows = kDnRpg * (256 / L) / k;
        pf.nbd = d / pf.rows;
        pf.rb = row_bytes_of(down_type, fe);
    }
    switch (type) {
    case VT_Q4_K: return launch_gateup_t<VT_Q4_K>(rpw, parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, pf, nref, s);
    case VT_Q8_0: return launch_gateup_t<VT_Q8_0>(rpw, parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, pf, nref, s);
    case VT_Q6_K: return launch_gateup_t<VT_Q6_K>(rpw, parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, pf, nref, s);
    default: return -EINVAL;
    }
}

bool vh_decode_batch_supported(uint32_t type, int d, int fe, int E, int k, int nt) {
    return vh_decode_gateup_supported(type, d, fe) && E >= 1 && E <= kMaxExperts && k >= 1 && nt >= 2 &&
           nt <= kDecodeBatchMax && nt * k <= 64 && batch_lds(E, k, fe, nt, vh_num_cus()) <= kBgDynBytes;
}

int vh_decode_batch_gateup(uint32_t type, const RoutePart *parts, const float *R, const float *hb, const float *bias,
                           int d, int E, int k, int fe, int renorm, const void *const *table, float *h, int32_t *idx,
                           float *w, uint32_t *flags, DecodePlan *plan, int nt, hipStream_t s) {
    if (!vh_decode_batch_supported(type, d, fe, E, k, nt)) return -EINVAL;
    const int64_t rb = row_bytes_of(type, d);
    switch (type) {
    case VT_Q4_K: return launch_batch_gateup_t<VT_Q4_K>(parts, R, hb, bias, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, nt, s);
    case VT_Q8_0: return launch_batch_gateup_t<VT_Q8_0>(parts, R, hb, bias, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, nt, s);
    case VT_Q6_K: return launch_batch_gateup_t<VT_Q6_K>(parts, R, hb, bias, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, nt, s);
    default: return -EINVAL;
    }
}

bool vh_down_combine_supported(uint32_t type, int d, int fe, int k) {
    if (!(type == VT_Q4_K || type == VT_Q8_0 || type == VT_Q6_K)) return false;
    if (fe % (type == VT_Q8_0 ? 32 : 256) || k < 1 || k > 64) return false;
    const int L = down_lanes(fe / 32, k);
    if (!L) return false;
    const int R = kDnRpg * (256 / L) / k;
    return R >= 1 && d % R == 0;
}

int vh_down_combine(uint32_t type, const DecodePlan *plan, const float *h, int d, int fe, int k, float *x,
                    hipStream_t s, int nt) {
    if (!vh_down_combine_supported(type, d, fe, k) || nt < 1 || nt * k > 64) return -EINVAL;
    switch (type) {
    case VT_Q4_K: return launch_down_t<VT_Q4_K>(plan, h, d, fe, k, x, nt, s);
    case VT_Q8_0: return launch_down_t<VT_Q8_0>(plan, h, d, fe, k, x, nt, s);
    case VT_Q6_K: return launch_down_t<VT_Q6_K>(plan, h, d, fe, k, x, nt, s);
    default: return -EINVAL;
    }
}
