// One MoE layer for one token in one launch (src/gguf_run.c:185-214, and with
// the RMSNorm in front for the stack and model paths, :161-165 + :238-239):
// router logits, top-k, gate/up SwiGLU, down, weighted combine and residual.
//
// 256 workgroups of 512 threads, one per CU, all resident together. They meet
// twice, through tagged data instead of flags or kernel boundaries:
//   1. workgroup e < E computes expert e's router part (the fp64 sum of the
//      rounded products and the bound on the reference's fp32 sum) and
//      publishes it as two 8-byte words that carry this launch's number; wave
//      0 of every workgroup polls the E records until all carry it;
//   2. every wave selects the top-k from those parts on its own (certified, as
//      the decode plan does, or ranked again on exact logits), then issues the
//      loads of its gate/up rows (expert slot blockIdx / 32) and of its down
//      rows (output rows [8b, 8b + 8) of the expert of round wave) at once;
//      gate/up rows are published as tagged 8-byte values; wave w polls the
//      fe tagged values of the expert of round w, copies them to LDS and
//      computes its down rows from weights that are already in registers;
//      the k rows of each output meet in LDS and are combined in selection
//      order into x.
// The launch number is per workgroup: workgroup b reads gen[b] at its start and
// writes gen[b] + 1 at its end, so every workgroup of one launch uses the same
// number without any atomic (each launch runs every workgroup exactly once),
// and a record written by an earlier launch never matches. The exchange area
// is zeroed once per device and shared by every launch there (stream order).
// Loads of other workgroups' records are agent-scope atomic loads (they bypass
// the L2 of this XCD, which does not see other XCDs' writes); stores are
// agent-scope atomic stores (write-through). Every wait is bounded: a wait that
// runs out sets VIREO_DECODE_TIMEOUT in the device's status word and lets the
// kernel finish with an invalid result.
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route.h"
#include "route_kernels.h"

namespace {

constexpr int kLB = kLayerBlocks;  // workgroups
constexpr int kWaves = 8;          // = k: wave w owns the down rows of round w
constexpr int kRB = 8;             // output rows per workgroup (2048 / 256)

VH_DEV uint64_t ld_agent64(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
VH_DEV void st_agent64(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A router part as two tagged words: c with its lowest 8 mantissa bits replaced
// by the tag (|change| <= 2^-44 |c|, added to the bound), and the bound rounded
// up to fp32 beside the full launch number.
VH_DEV void put_part(uint64_t *rec, double c, double beta, uint32_t epoch) {
    const double b = beta + fabs(c) * 5.684341886080802e-14;  // 2^-44
    const uint64_t cw = (uint64_t(__double_as_longlong(c)) & ~uint64_t(0xff)) | (epoch & 0xffu);
    st_agent64(rec, cw);
    st_agent64(rec + 1, (uint64_t(epoch) << 32) | __float_as_uint(__double2float_ru(b)));
}

template <int TG, int TD, int Q, int RPW, int L, int IPL, int UPG, bool NORM, bool ST>
__global__ void __launch_bounds__(512) moe_layer_kernel(
    const float *__restrict__ R, const float *xin, const void *const *__restrict__ table,
    LayerXchg *__restrict__ xg, int E, int k, int fe, int d, int renorm, int64_t rb_gu, int64_t rb_dn,
    const float *__restrict__ bias, float *x, int32_t *__restrict__ idx_out, float *__restrict__ w_out,
    uint32_t *__restrict__ flags_out, uint32_t *__restrict__ status, unsigned spin_limit, const float *__restrict__ nw,
    float eps, float *__restrict__ hb_out, uint64_t *__restrict__ stamps) {
    // stamps: 0 start, 1 router part computed, 2 every part received, 3 top-k
    // chosen, 4 first gate/up row computed, 5 activations published, 6 the
    // down expert's activations received, 7 end
    PhaseStamps<ST> ps(stamps);
    ps.now(0);
    using FG = Reg<TG>;
    using FD = Reg<TD>;
    constexpr int NSG = FG::NS, NSD = FD::NS, TPL = 3 * Q, SUB = 64 / L;
    static_assert(SUB * UPG == kRB, "a wave covers the workgroup's output rows");
    __shared__ TopKSmem sm;
    __shared__ __align__(16) float xref[NORM ? 2048 : 4];  // the fallback's reference xb (NORM)
    __shared__ float2 stage[64];
    __shared__ double2 cert[kWaves][64];
    __shared__ RoutePart sparts[64 * Q];
    __shared__ double red_d[3][kWaves];
    __shared__ __align__(16) float hs[kWaves][1024];
    __shared__ float ys[kWaves][kRB];
    __shared__ int pres[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int b = blockIdx.x;
    const uint32_t epoch = xg->gen[b] + 1u;

    // ---- 0. prologue loads: this lane's router columns and inputs, the layer's
    //         expert table over the lanes, the inputs of this lane's gate/up item,
    //         and the residual of this workgroup's output rows
    const float4 xin4 = reinterpret_cast<const float4 *>(xin)[tid];  // columns 4 tid .. 4 tid + 3
    float4 r4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (b < E) r4 = reinterpret_cast<const float4 *>(R + size_t(b) * d)[tid];
    const void *tab[TPL];
#pragma unroll
    for (int s = 0; s < TPL; s++) {
        const int i = TPL * lane + s;
        tab[s] = i < 3 * E ? table[i] : nullptr;
    }
    float xr[32], xsg[NSG];
    FG::load_x(xin, lane, xr);
    float xo = 0.0f;
    if (tid < kRB) xo = x[b * kRB + tid];
    float4 nw4 = make_float4(1.f, 1.f, 1.f, 1.f);
    float nwr[32];
    if constexpr (NORM) {
        if (nw) {
            nw4 = reinterpret_cast<const float4 *>(nw)[tid];
            FG::load_x(nw, lane, nwr);
        }
    }

    // ---- NORM: hb = rmsnorm(xin) as route_parts_norm_kernel forms it (fp64 sum
    //      of the squares, rounded once): the same operations in every workgroup
    float4 hv = xin4;
    if constexpr (NORM) {
        double ss = double(mul_rn(xin4.x, xin4.x)) + double(mul_rn(xin4.y, xin4.y)) +
                    double(mul_rn(xin4.z, xin4.z)) + double(mul_rn(xin4.w, xin4.w));
        ss = wave_sum_d(ss);
        if (lane == 0) red_d[2][wv] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) tot += red_d[2][w];
        const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(float(tot), float(d)), eps)));
        auto scale = [&](float v, float wgt) { return nw ? mul_rn(mul_rn(v, r), wgt) : mul_rn(v, r); };
        hv = make_float4(scale(xin4.x, nw4.x), scale(xin4.y, nw4.y), scale(xin4.z, nw4.z), scale(xin4.w, nw4.w));
#pragma unroll
        for (int i = 0; i < 32; i++) xr[i] = scale(xr[i], nw ? nwr[i] : 1.0f);
        if (b == 0 && hb_out) reinterpret_cast<float4 *>(hb_out)[tid] = hv;
    }
    FG::sums(xr, xsg);

    // ---- 1. the router part of expert b: fp64 sum of the rounded products in
    //         column order and 1.001 u sum_k |S_k| over its prefix sums
    if (b < E) {
        const float p0 = mul_rn(r4.x, hv.x), p1 = mul_rn(r4.y, hv.y), p2 = mul_rn(r4.z, hv.z),
                    p3 = mul_rn(r4.w, hv.w);
        const double t4 = ((double(p0) + double(p1)) + double(p2)) + double(p3);
        const double incl = wave_incl_scan_d(t4);
        if (lane == 63) red_d[0][wv] = incl;  // the wave's total
        __syncthreads();
        double off = 0.0, c = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const double v = red_d[0][w];
            if (w < wv) off += v;
            c += v;
        }
        double run = off + incl - t4, absum = 0.0;
        run += double(p0); absum += fabs(run);
        run += double(p1); absum += fabs(run);
        run += double(p2); absum += fabs(run);
        run += double(p3); absum += fabs(run);
        const double pabs = fabs(double(p0)) + fabs(double(p1)) + fabs(double(p2)) + fabs(double(p3));
        const double wa = wave_sum_d(absum), wp = wave_sum_d(pabs);
        __syncthreads();  // everyone has read red_d[0]
        if (lane == 0) {
            red_d[0][wv] = wa;
            red_d[1][wv] = wp;
        }
        __syncthreads();
        if (tid == 0) {
            double sa = 0.0, sp = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                sa += red_d[0][w];
                sp += red_d[1][w];
            }
            RoutePart p{c, 1.001 * 5.9604644775390625e-08 * sa + 1e-30};
            if constexpr (NORM) p = route_part_on_own_norm(p, sp, d, bias, b);
            else if (bias) p.c += double(bias[b]);
            put_part(xg->parts + 2 * b, p.c, p.beta, epoch);
        }
    }
    ps.now(1);

    // ---- 2. wave 0 polls the E parts until all carry this launch's number
    bool timed_out = false;
    if (wv == 0) {
        for (unsigned spins = 0;; spins++) {
            if (spins >= spin_limit) {
                timed_out = true;
                break;
            }
            // every load of the round first (each agent-scope load is awaited
            // where its value is used, so loads used one by one would travel
            // one round trip at a time), then the checks
            uint64_t a[Q], w2[Q];
#pragma unroll
            for (int q = 0; q < Q; q++) {
                const int e = min(lane + 64 * q, E - 1);
                a[q] = ld_agent64(xg->parts + 2 * e);
                w2[q] = ld_agent64(xg->parts + 2 * e + 1);
            }
            bool good = true;
#pragma unroll
            for (int q = 0; q < Q; q++) {
                const int e = lane + 64 * q;
                if (e < E) {
                    good &= (a[q] & 0xffu) == (epoch & 0xffu) && uint32_t(w2[q] >> 32) == epoch;
                    sparts[e] = RoutePart{__longlong_as_double(int64_t(a[q])), double(__uint_as_float(uint32_t(w2[q])))};
                }
            }
            if (__ballot(good) == __builtin_amdgcn_read_exec()) break;
        }
    }
    __syncthreads();
    ps.now(2);
    RoutePart p[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int e = lane + 64 * q;
        p[q] = e < E ? sparts[e] : RoutePart{0.0, 0.0};
    }

    // ---- 3. the ranking, by the whole workgroup in one counting pass, and
    //         its certification by every wave on its own (the same verdict in
    //         every wave and workgroup): gate/up expert of slot j, down expert
    //         of round wv. An order that cannot be certified is ranked again on
    //         exact logits by the whole workgroup (rare), before any weight is
    //         loaded.
    const int j = b / (kLB / kWaves);
    __shared__ __align__(16) uint32_t rkeys[64 * Q];
    __shared__ int rcnt[512];
    int rank[Q];
    route_rank_block<Q>(p, E, k, rkeys, rcnt, rank, nullptr);
    const bool certified = route_certify_wave<Q>(p, E, k, rank, cert[wv]);
    float w_sel = 0.0f;  // wave 0, lane t < k: the weight of round t
    int e_sel = 0;
    int e_j, e_dn;
    if (certified) {
        e_j = rank_owner<Q>(rank, j);
        e_dn = rank_owner<Q>(rank, wv);
        if (b == 0 && tid == 0 && flags_out) flags_out[0] = 0u;
    } else {
        const float *xe = xin;
        if constexpr (NORM) {  // on the reference's own xb, not on the fp64-normalised hb
            reference_rmsnorm_block(xref, xin, nw, eps, d, &sm.red[0][0]);
            xe = xref;
        }
        route_topk_block(sm, sparts, R, xe, bias, d, E, k, renorm, false, nullptr);
        e_j = sm.sel[j];
        e_dn = sm.sel[wv];
        if (wv == 0 && lane < k) {
            e_sel = sm.sel[lane];
            w_sel = sm.sel_w[lane];
        }
        if (b == 0 && tid == 0 && flags_out) flags_out[0] = sm.flag;
    }

    // ---- 4. every weight load of the workgroup: gate/up rows, then down rows
    ps.after(3, e_j);
    const uint8_t *Gp = table_entry<TPL>(tab, 3 * e_j);
    const uint8_t *Up = table_entry<TPL>(tab, 3 * e_j + 1);
    const uint8_t *Dp = table_entry<TPL>(tab, 3 * e_dn + 2);
    const bool gu_ok = Gp && Up;
    const int o0 = ((b % (kLB / kWaves)) * kWaves + wv) * RPW;
    typename FG::Raw rg[RPW], ru[RPW];
    if (gu_ok) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int64_t o = min(o0 + r, fe - 1);
            rg[r] = FG::fetch(gmem(Gp), o * rb_gu, lane);
            ru[r] = FG::fetch(gmem(Up), o * rb_gu, lane);
        }
    }
    const int grp = lane / L, li = lane % L, items_dn = FD::items(fe);
    const int o_dn = b * kRB;
    typename FD::Raw rd[UPG][IPL];
    if (Dp) {
#pragma unroll
        for (int u = 0; u < UPG; u++)
#pragma unroll
            for (int m = 0; m < IPL; m++)
                rd[u][m] = FD::fetch(gmem(Dp), int64_t(o_dn + grp * UPG + u) * rb_dn, min(li + L * m, items_dn - 1));
    }

    // the softmax weights of the certified order, by wave 0 while its loads
    // are in flight
    if (certified && wv == 0) route_weights_wave<Q>(p, rank, E, k, renorm, stage, e_sel, w_sel);
    if (b == 0 && wv == 0 && lane < k) {
        idx_out[lane] = e_sel;
        w_out[lane] = w_sel;
    }

    // ---- 5. gate/up rows of expert slot j, published as tagged values
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float g = 0.0f, u = 0.0f;
        if (gu_ok) {
            g = FG::compute(rg[r], lane, xr, xsg);
            u = FG::compute(ru[r], lane, xr, xsg);
        }
        g = group_sum<64>(g);
        u = group_sum<64>(u);
        if (r == 0) ps.after(4, g);
        if (lane == 63 && o0 + r < fe) {  // an unregistered expert contributes nothing (src/gguf_run.c:201)
            const float hval = gu_ok ? swiglu(g, u) : 0.0f;
            st_agent64(xg->h + size_t(j) * kMaxLayerFe + o0 + r, (uint64_t(epoch) << 32) | __float_as_uint(hval));
        }
    }
    // the workgroup's activations are stored (not necessarily visible yet):
    // one small record that consumers poll before reading the values, which
    // carry their own tags and are checked again, so the barrier orders
    // nothing in memory and need not wait for the down rows in flight
    lds_barrier();
    if (tid == 0) st_agent64(&xg->done[j][b % (kLB / kWaves)], epoch);
    ps.now(5);

    // ---- 6. wave wv polls the producers of the expert of round wv, then reads
    //         its activations (and reads them again until every tag is fresh)
    {
        const uint64_t *hw = xg->h + size_t(wv) * kMaxLayerFe;
        const uint64_t *dw = xg->done[wv];
        constexpr int per = RPW * 4;  // values per lane: fe = 256 RPW (768 or 1024)
        bool producers = false;
        for (unsigned spins = 0;; spins++) {
            if (spins >= spin_limit) {
                timed_out = true;
                break;
            }
            if (!producers) {
                const bool fresh = lane >= kLB / kWaves || uint32_t(ld_agent64(dw + lane)) == epoch;
                producers = __ballot(fresh) == __builtin_amdgcn_read_exec();
                if (!producers) continue;
            }
            uint64_t v[per];  // all of the round's loads first, then the checks
#pragma unroll
            for (int q = 0; q < per; q++) v[q] = ld_agent64(hw + lane + 64 * q);
            bool good = true;
#pragma unroll
            for (int q = 0; q < per; q++) {
                good &= uint32_t(v[q] >> 32) == epoch;
                hs[wv][lane + 64 * q] = __uint_as_float(uint32_t(v[q]));
            }
            if (__ballot(good) == __builtin_amdgcn_read_exec()) break;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    ps.now(6);

    // ---- 7. down rows of the expert of round wv from registers, then the combine
    if (lane == 0) pres[wv] = Dp != nullptr;
    float xv[IPL][32], xsd[IPL][NSD];
#pragma unroll
    for (int m = 0; m < IPL; m++) {
        FD::load_x(&hs[wv][0], min(li + L * m, items_dn - 1), xv[m]);  // the item's inputs, 16-byte LDS reads
        FD::sums(xv[m], xsd[m]);
    }
#pragma unroll
    for (int u = 0; u < UPG; u++) {
        float acc = 0.0f;
        if (Dp) {
#pragma unroll
            for (int m = 0; m < IPL; m++)
                if (li + L * m < items_dn) acc += FD::compute(rd[u][m], li + L * m, xv[m], xsd[m]);
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
            if (lane < kRB) a = add_rn(a, mul_rn(wt, ys[t][lane]));
        }
        if (lane < kRB) x[o_dn + lane] = add_rn(xo, a);
    }
    if (timed_out) atomicOr(status, VIREO_DECODE_TIMEOUT);
    if (tid == 0) xg->gen[b] = epoch;
    ps.now(7);
    ps.store();
}

template <int TG, int TD, int Q, int RPW, int L, int IPL, int UPG>
int launch_layer(const LayerArgs &a, hipStream_t s) {
    uint32_t *status = nullptr;
    if (int rc = vh_status_word(&status)) return rc;
    const int64_t rb_gu = vh_row_bytes(TG, a.d), rb_dn = vh_row_bytes(TD, a.fe);
    uint64_t *st = vh_stamps_for(0);
#define VH_LAYER(NORM, ST)                                                                                           \
    VH_LAUNCH((moe_layer_kernel<TG, TD, Q, RPW, L, IPL, UPG, NORM, ST>), dim3(kLB), dim3(64 * kWaves), 0, s, a.R,  \
              a.xin, a.table, a.xg, a.E, a.k, a.fe, a.d, a.renorm, rb_gu, rb_dn, a.bias, a.x, a.idx, a.w, a.flags,    \
              status, vh_spin_limit(), a.nw, a.eps, a.hb_out, st)
    if (a.norm && st) VH_LAYER(true, true);
    else if (a.norm) VH_LAYER(true, false);
    else if (st) VH_LAYER(false, true);
    else VH_LAYER(false, false);
#undef VH_LAYER
    return vh_check(hipGetLastError());
}

// The shapes the layer kernel is built for: d = 2048, k = 8, up to 128
// experts (one or two router parts per lane), expert width 768 (Qwen3-30B-A3B)
// or 1024 (OLMoE), gate/up Q4_K with down Q6_K or all Q8_0.
int layer_variant(uint32_t tg, uint32_t td, int d, int E, int k, int fe) {
    if (d != 2048 || k != kWaves || E < k || E > 128) return 0;
    const bool types = (tg == VT_Q4_K && td == VT_Q6_K) || (tg == VT_Q8_0 && td == VT_Q8_0);
    if (!types) return 0;
    if (fe == 768) return 1;
    if (fe == 1024) return 2;
    return 0;
}

template <int Q>
int launch_q(uint32_t tg, int variant, const LayerArgs &a, hipStream_t s) {
    if (variant == 1) {  // 768 gate/up rows per expert: 3 per wave; down: 8 lanes x 3 items per row, 8 rows
        if (tg == VT_Q4_K) return launch_layer<VT_Q4_K, VT_Q6_K, Q, 3, 8, 3, 1>(a, s);
        return launch_layer<VT_Q8_0, VT_Q8_0, Q, 3, 8, 3, 1>(a, s);
    }
    // 1024 rows: 4 per wave; down: 16 lanes x 2 items per row, 4 rows twice
    if (tg == VT_Q4_K) return launch_layer<VT_Q4_K, VT_Q6_K, Q, 4, 16, 2, 2>(a, s);
    return launch_layer<VT_Q8_0, VT_Q8_0, Q, 4, 16, 2, 2>(a, s);
}

}  // namespace

int vh_layer_supported(uint32_t tg, uint32_t td, int d, int E, int k, int fe) {
    if (vh_num_cus() < kLB) return 0;  // every workgroup must be resident at once
    return layer_variant(tg, td, d, E, k, fe) != 0;
}

int vh_moe_layer(uint32_t tg, uint32_t td, const LayerArgs &a, hipStream_t s) {
    // fe = 256 RPW of the variant (the activation polls take fe / 64 values per lane)
    if (!vh_layer_supported(tg, td, a.d, a.E, a.k, a.fe) || !a.xg || !a.idx || !a.w) return -EINVAL;
    const int v = layer_variant(tg, td, a.d, a.E, a.k, a.fe);
    return a.E <= 64 ? launch_q<1>(tg, v, a, s) : launch_q<2>(tg, v, a, s);
}
