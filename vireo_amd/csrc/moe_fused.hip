// The one-token MoE experts as one kernel: top-k, gate/up SwiGLU, down,
// weighted combine and residual (src/gguf_run.c:186-214 after the router
// matvec), for the common decode shapes: k = 8, d = 2048, 256 workgroups of
// 512 threads (one per CU). An alternative to the decode plan's separate
// gate/up and down kernels (selected with vireo_hip_set_path(3)): it trades
// the kernel boundary between them for one grid-wide handoff and lets the
// down weights stream while gate/up computes; measured on MI355X it is about
// as fast as the two kernels, not faster.
//
// Workgroup b (blockIdx (bx, j)):
//   1. loads the router parts, the layer's expert table (over the lanes) and
//      its input item, and every wave selects the top-k on its own (as in
//      decode_gateup_kernel);
//   2. issues the loads of its RPW gate/up rows of expert j AND of its down
//      rows: output rows [8b, 8b + 8) of the expert chosen in round wv, for
//      wave wv - so the down weights stream while gate/up computes;
//   3. computes its gate/up rows and publishes h with write-through stores;
//   4. meets the other workgroups: each sets its flag, then waits until all
//      256 flags are set (the flags are zeroed by the router kernel before
//      every launch). The loads and stores on both sides bypass the
//      non-coherent L2 (sc1), so no cache-wide fence is needed;
//   5. reads the activations of its down expert, computes its down rows and
//      combines the k experts' rows in selection order into x.
// Every wait is bounded: a workgroup that waits too long records
// VIREO_DECODE_TIMEOUT in the token's flag word and in the device's sticky
// status word and goes on (the result is then not valid), so no launch can
// hang; synchronous calls report it as -ETIMEDOUT, stream calls through
// vireo_hip_status.
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route.h"
#include "route_kernels.h"

namespace {

constexpr int kFusedWaves = 8;      // = k: wave wv owns the down rows of round wv

// 16 bytes at byte offset off of p with the sc1 policy (bypass the L2 of this
// die, which other dies do not keep coherent); reads past `bytes` return zeros.
VH_DEV float4 load_sc1_x4(const float *p, uint32_t bytes, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), 0, int(bytes), 0x00020000);
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 16);
    return make_float4(v.x, v.y, v.z, v.w);
}

template <int TG, int TD, int Q, int RPW, int L, int IPL, int UPG>
__global__ void __launch_bounds__(512) decode_experts_kernel(
    const RoutePart *__restrict__ parts, const float *__restrict__ hb, const void *const *__restrict__ table, int E,
    int k, int fe, int d, int renorm, int64_t rb_gu, int64_t rb_dn, const float *__restrict__ R,
    const float *__restrict__ bias, float *__restrict__ h, uint32_t *__restrict__ bar, float *__restrict__ x,
    int32_t *__restrict__ idx_out, float *__restrict__ w_out, uint32_t *__restrict__ status, unsigned spin_limit,
    NormRef nref) {
    using FG = Reg<TG>;
    using FD = Reg<TD>;
    constexpr int NSG = FG::NS, NSD = FD::NS, TPL = 3 * Q, SUB = 64 / L;
    constexpr int RB = SUB * UPG;  // output rows per workgroup
    __shared__ TopKSmem sm;
    __shared__ __align__(16) float xref[2048];  // the fallback on a library-normalised hb: the reference's xb
    __shared__ float2 stage[64];
    __shared__ double2 cert[kFusedWaves][64];
    __shared__ float ys[kFusedWaves][RB];
    __shared__ int pres[kFusedWaves];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int j = blockIdx.y, G = int(gridDim.x * gridDim.y);
    const int b = blockIdx.y * gridDim.x + blockIdx.x;
    uint32_t *flag_out = bar + G;

    // 1. prologue loads and per-wave selection
    RoutePart p[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int e = lane + 64 * q;
        if (e < E) p[q] = parts[e];
        else p[q] = RoutePart{0.0, 0.0};
    }
    const void *tab[TPL];
#pragma unroll
    for (int s = 0; s < TPL; s++) {
        const int i = TPL * lane + s;
        tab[s] = i < 3 * E ? table[i] : nullptr;
    }
    float xr[32], xsg[NSG];
    FG::load_x(hb, lane, xr);
    FG::sums(xr, xsg);
    const int o_dn = b * RB;  // this workgroup's output rows
    float xo = 0.0f;
    if (tid < RB) xo = x[o_dn + tid];

    int e_j, e_dn, rank[Q];
    const bool ok = route_select_wave<Q>(p, E, k, j, e_j, wv, e_dn, rank, cert[wv]);
    float w_sel = 0.0f;  // wave 0, lane t < k: weight of round t
    int e_sel = 0;
    if (!ok) {  // the same verdict in every wave: the whole workgroup ranks on exact logits
        const float *xe = hb;
        if (nref.x) {  // on the reference's own xb, not on the fp64-normalised hb
            reference_rmsnorm_block(xref, nref.x, nref.nw, nref.eps, d, &sm.red[0][0]);
            xe = xref;
        }
        route_topk_block(sm, parts, R, xe, bias, d, E, k, renorm, false, nullptr);
        e_j = sm.sel[j];
        e_dn = sm.sel[wv];
        if (wv == 0 && lane < k) {
            e_sel = sm.sel[lane];
            w_sel = sm.sel_w[lane];
        }
        if (b == 0 && tid == 0) atomicOr(flag_out, sm.flag);
    } else if (wv == 0) {
        route_weights_wave<Q>(p, rank, E, k, renorm, stage, e_sel, w_sel);
    }
    if (b == 0 && wv == 0 && lane < k) {
        idx_out[lane] = e_sel;
        w_out[lane] = w_sel;
    }

    // 2. loads of the gate/up rows and of the down rows
    const uint8_t *Gp = table_entry<TPL>(tab, 3 * e_j);
    const uint8_t *Up = table_entry<TPL>(tab, 3 * e_j + 1);
    const uint8_t *Dp = table_entry<TPL>(tab, 3 * e_dn + 2);
    const int o0 = (blockIdx.x * kFusedWaves + wv) * RPW;
    const bool gu_ok = Gp && Up;
    typename FG::Raw rg[RPW], ru[RPW];
    if (gu_ok) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int64_t o = min(o0 + r, fe - 1);
            rg[r] = FG::fetch(Gp, o * rb_gu, lane);
            ru[r] = FG::fetch(Up, o * rb_gu, lane);
        }
    }
    const int grp = lane / L, li = lane % L, items_dn = FD::items(fe);
    typename FD::Raw rd[UPG][IPL];

    // 3. gate/up rows of expert j, published with write-through stores. The
    //    down loads are issued once the first row has arrived and been used,
    //    so that they stream while the remaining rows compute instead of
    //    delaying the gate/up bytes.
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float g = 0.0f, u = 0.0f;
        if (gu_ok) {
            g = FG::compute(rg[r], lane, xr, xsg);
            u = FG::compute(ru[r], lane, xr, xsg);
        }
        g = group_sum<64>(g);
        u = group_sum<64>(u);
        if (lane == 63 && o0 + r < fe)  // an unregistered expert contributes nothing (src/gguf_run.c:201)
            __hip_atomic_store(h + size_t(j) * fe + o0 + r, gu_ok ? swiglu(g, u) : 0.0f, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (r == 0) {
            asm volatile("" ::: "memory");
            if (Dp) {
#pragma unroll
                for (int u2 = 0; u2 < UPG; u2++)
#pragma unroll
                    for (int m = 0; m < IPL; m++) {
                        const int it = li + L * m;
                        if (it < items_dn) rd[u2][m] = FD::fetch(Dp, int64_t(o_dn + grp * UPG + u2) * rb_dn, it);
                    }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's h stores have completed
    __syncthreads();

    // 4. this workgroup's h rows are out: set its flag; then each wave waits
    //    for the gridDim.x workgroups that produce the h of its down expert
    //    (round wv), polling their flags with one load per lane
    if (tid == 0) __hip_atomic_store(bar + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    {
        const int nb = int(gridDim.x);
        const uint32_t *mine = bar + wv * nb;
        // at most spin_limit polls (0: give up at once, which lets a test
        // take the error path with every wave exiting normally)
        for (unsigned spins = 0;; spins++) {
            if (spins >= spin_limit) {
                if (lane == 0) {
                    atomicOr(flag_out, VIREO_DECODE_TIMEOUT);
                    atomicOr(status, VIREO_DECODE_TIMEOUT);
                }
                break;
            }
            const bool set = lane >= nb || __hip_atomic_load(const_cast<uint32_t *>(mine) + lane, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT) != 0u;
            if (__ballot(set) == __builtin_amdgcn_read_exec()) break;
        }
    }
    asm volatile("" ::: "memory");

    // 5. down rows of the expert of round wv, then the combine
    if (lane == 0) pres[wv] = Dp != nullptr;
    float xv[IPL][32], xsd[IPL][NSD];
    const float *hrow = h + size_t(wv) * fe;
    const uint32_t hbytes = uint32_t(fe) * 4u;
#pragma unroll
    for (int m = 0; m < IPL; m++) {
        const int it = li + L * m;
        // the item's inputs: runs of 8 (Q6_K), 16 (Q4_K) or 32 (Q8_0) columns
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int i0 = 4 * c;
            int cidx;
            if constexpr (TD == VT_Q6_K) cidx = Split<VT_Q6_K>::col0(it) + 32 * (i0 >> 3) + (i0 & 7);
            else if constexpr (TD == VT_Q4_K) cidx = Split<VT_Q4_K>::col0(it) + (i0 < 16 ? i0 : i0 + 16);
            else cidx = 32 * it + i0;
            const float4 v = it < items_dn ? load_sc1_x4(hrow, hbytes, uint32_t(cidx) * 4u) : make_float4(0, 0, 0, 0);
            xv[m][i0 + 0] = v.x;
            xv[m][i0 + 1] = v.y;
            xv[m][i0 + 2] = v.z;
            xv[m][i0 + 3] = v.w;
        }
    }
#pragma unroll
    for (int m = 0; m < IPL; m++) FD::sums(xv[m], xsd[m]);
#pragma unroll
    for (int u = 0; u < UPG; u++) {
        float acc = 0.0f;
        if (Dp) {
#pragma unroll
            for (int m = 0; m < IPL; m++) {
                const int it = li + L * m;
                if (it < items_dn) acc += FD::compute(rd[u][m], it, xv[m], xsd[m]);
            }
        }
        acc = group_sum<L>(acc);
        if (li == L - 1) ys[wv][grp * UPG + u] = acc;
    }
    __syncthreads();
    if (wv == 0) {
        float a = 0.0f;
        for (int t = 0; t < k; t++) {
            const float wt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w_sel), t));
            if (!pres[t]) continue;  // failed lookup: skipped (src/gguf_run.c:201)
            if (lane < RB) a = add_rn(a, mul_rn(wt, ys[t][lane]));
        }
        if (lane < RB) x[o_dn + lane] = add_rn(xo, a);
    }
}

template <int TG, int TD, int Q, int RPW, int L, int IPL, int UPG>
int launch_experts(const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E, int k,
                   int fe, int renorm, const void *const *table, float *h, uint32_t *bar, float *x, int32_t *idx,
                   float *w, NormRef nref, hipStream_t s) {
    constexpr int rows_per_block = kFusedWaves * RPW;
    const dim3 g(fe / rows_per_block, k);
    const int64_t rb_gu = TG == VT_Q8_0 ? int64_t(d / 32) * 34 : TG == VT_Q4_K ? int64_t(d / 256) * 144
                                                                               : int64_t(d / 256) * 210;
    const int64_t rb_dn = TD == VT_Q8_0 ? int64_t(fe / 32) * 34 : TD == VT_Q4_K ? int64_t(fe / 256) * 144
                                                                                : int64_t(fe / 256) * 210;
    uint32_t *status = nullptr;
    if (int rc = vh_status_word(&status)) return rc;
    VH_LAUNCH((decode_experts_kernel<TG, TD, Q, RPW, L, IPL, UPG>), g, dim3(64 * kFusedWaves), 0, s, parts, hb, table,
              E, k, fe, d, renorm, rb_gu, rb_dn, R, bias, h, bar, x, idx, w, status, vh_spin_limit(), nref);
    return vh_check(hipGetLastError());
}

// The shapes the fused kernel is built for: Qwen3-30B-A3B (E = 128, fe = 768)
// and OLMoE (E = 64, fe = 1024), d = 2048, k = 8, both with 256 workgroups.
int fused_variant(uint32_t tg, uint32_t td, int d, int E, int k, int fe) {
    if (d != 2048 || k != kFusedWaves) return 0;
    const bool types = (tg == VT_Q4_K && td == VT_Q6_K) || (tg == VT_Q8_0 && td == VT_Q8_0);
    if (!types) return 0;
    if (E > 64 && E <= 128 && fe == 768) return 1;
    if (E <= 64 && fe == 1024) return 2;
    return 0;
}

}  // namespace

// The workgroups meet once, so all of them must be resident together: one per
// CU (a second never fits beside the first), which needs kFusedBlocks CUs.
int vh_fused_blocks(uint32_t tg, uint32_t td, int d, int E, int k, int fe) {
    if (vh_num_cus() < kFusedBlocks) return 0;
    return fused_variant(tg, td, d, E, k, fe) ? kFusedBlocks : 0;
}

int vh_decode_experts(uint32_t tg, uint32_t td, const RoutePart *parts, const float *R, const float *hb,
                      const float *bias, int d, int E, int k, int fe, int renorm, const void *const *table, float *h,
                      uint32_t *bar, float *x, int32_t *idx, float *w, NormRef nref, hipStream_t s) {
    switch (fused_variant(tg, td, d, E, k, fe)) {
    case 1:  // 768 rows of gate/up per expert: 3 per wave; down rows 8 per workgroup, 8 lanes x 3 items each
        if (tg == VT_Q4_K)
            return launch_experts<VT_Q4_K, VT_Q6_K, 2, 3, 8, 3, 1>(parts, R, hb, bias, d, E, k, fe, renorm, table, h,
                                                                    bar, x, idx, w, nref, s);
        return launch_experts<VT_Q8_0, VT_Q8_0, 2, 3, 8, 3, 1>(parts, R, hb, bias, d, E, k, fe, renorm, table, h, bar,
                                                                x, idx, w, nref, s);
    case 2:  // 1024 rows: 4 per wave; down items 32 per row: 16 lanes x 2 items, 2 rows per lane group
        if (tg == VT_Q4_K)
            return launch_experts<VT_Q4_K, VT_Q6_K, 1, 4, 16, 2, 2>(parts, R, hb, bias, d, E, k, fe, renorm, table, h,
                                                                     bar, x, idx, w, nref, s);
        return launch_experts<VT_Q8_0, VT_Q8_0, 1, 4, 16, 2, 2>(parts, R, hb, bias, d, E, k, fe, renorm, table, h, bar,
                                                                 x, idx, w, nref, s);
    default: return -EINVAL;
    }
}
