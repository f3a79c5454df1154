// Decode-path expert kernels (one token per call, the latency-bound case).
//
// decode_gateup_kernel: every workgroup ranks the router parts itself (wave 0,
// route_topk; about 2 KB from L2), so there is no separate top-k launch and no
// cross-workgroup signalling. It then computes h[j][o] = silu(gate_o . x) *
// (up_o . x) (src/gguf_run.c:205-207) for a block of rows of the j-th chosen
// expert. x is lane-resident: a lane owns the same item (32 or 64 columns) of
// every row, so its slice of x (and, for Q4_K, the sums of that slice) is
// loaded once. A wave issues the loads of all its rows before computing.
//
// down_combine_kernel: a workgroup owns R output rows of one token for all k
// chosen experts. Each lane loads its items of one (row, expert) straight from
// HBM (all of them before computing), the k activations sit in LDS, and
// x[o] += sum_j w_j * y_j is formed in selection order (src/gguf_run.c:
// 208-213). No atomics: every output element has one writer.
#include <hip/hip_runtime.h>
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

template <int N>
struct XRegs {
    const float (&v)[N];
    VH_DEV float operator[](int i) const { return v[i]; }
};

// ------------------------------------------------------------------ fused top-k + gate/up
// grid (ceil(fe / (4 * RPW * 64/L)), k), 256 threads. L lanes per row; a row's
// items are the L lane ids (d = L * columns per item).
template <int T, int L, int RPW>
__global__ void __launch_bounds__(256) decode_gateup_kernel(const RoutePart *__restrict__ parts,
                                                            const float *__restrict__ R,
                                                            const float *__restrict__ hb,
                                                            const float *__restrict__ bias, int d, int E, int k,
                                                            int fe, int renorm, const void *const *__restrict__ table,
                                                            int64_t row_bytes, float *__restrict__ h,
                                                            int32_t *__restrict__ idx_out, float *__restrict__ w_out,
                                                            uint32_t *__restrict__ flags_out,
                                                            DecodePlan *__restrict__ plan) {
    using S = Split<T>;
    constexpr int NW = S::NW, SUB = 64 / L;
    __shared__ TopKSmem sm;
    __shared__ const void *s_tab[3 * kMaxExperts];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, sub = lane / L, li = lane % L;
    const int j = blockIdx.y;
    for (int i = tid; i < 3 * E; i += 256) s_tab[i] = table[i];
    // the lane's inputs, in the item's own order
    float xr[NW];
    {
        const auto xs = S::xrow(hb, li);
#pragma unroll
        for (int i = 0; i < NW; i++) xr[i] = xs[i];
    }
    float sl = 0.0f, sh = 0.0f;
    if constexpr (T == VT_Q4_K) {
#pragma unroll
        for (int i = 0; i < 16; i++) { sl += xr[i]; sh += xr[16 + i]; }
    }
    route_topk_block(sm, parts, R, hb, bias, d, E, k, renorm, false, nullptr);
    if (blockIdx.x == 0 && blockIdx.y == 0) {
        if (tid < k) {
            idx_out[tid] = sm.sel[tid];
            w_out[tid] = sm.sel_w[tid];
            plan->down[tid] = s_tab[3 * sm.sel[tid] + 2];
            plan->w[tid] = sm.sel_w[tid];
        }
        if (tid == 0 && flags_out) flags_out[0] = sm.flag;
    }
    const int e = sm.sel[j];
    const uint8_t *G = static_cast<const uint8_t *>(s_tab[3 * e]);
    const uint8_t *U = static_cast<const uint8_t *>(s_tab[3 * e + 1]);
    const int o0 = (blockIdx.x * 4 + wv) * RPW * SUB + sub;
    if (!G || !U) {  // unregistered expert: contributes nothing (src/gguf_run.c:201)
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int o = o0 + r * SUB;
            if (li == L - 1 && o < fe) h[size_t(j) * fe + o] = 0.0f;
        }
        return;
    }
    typename S::Raw rg[RPW], ru[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int64_t o = min(o0 + r * SUB, fe - 1);
        rg[r] = S::fetch(G, o * row_bytes, li);
        ru[r] = S::fetch(U, o * row_bytes, li);
    }
    const XRegs<NW> xv{xr};
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float g, u;
        if constexpr (T == VT_Q4_K) {
            g = S::compute(rg[r], li, xv, sl, sh);
            u = S::compute(ru[r], li, xv, sl, sh);
        } else {
            g = S::compute(rg[r], li, xv);
            u = S::compute(ru[r], li, xv);
        }
        g = group_sum<L>(g);
        u = group_sum<L>(u);
        const int o = o0 + r * SUB;
        if (li == L - 1 && o < fe) h[size_t(j) * fe + o] = swiglu(g, u);
    }
}

template <int T, int L, int RPW>
int launch_decode_gateup(const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E,
                         int k, int fe, int renorm, const void *const *table, int64_t rb, float *h, int32_t *idx,
                         float *w, uint32_t *flags, DecodePlan *plan, hipStream_t s) {
    constexpr int rows_per_block = 4 * RPW * (64 / L);
    dim3 g((fe + rows_per_block - 1) / rows_per_block, k);
    hipLaunchKernelGGL((decode_gateup_kernel<T, L, RPW>), g, dim3(256), 0, s, parts, R, hb, bias, d, E, k, fe,
                       renorm, table, rb, h, idx, w, flags, plan);
    return vh_check(hipGetLastError());
}

// ------------------------------------------------------------------ down + combine
// grid (d / R), 256 threads, R = 256 / (Q * k): unit (r, j) = output row o0 + r
// of expert j, handled by Q consecutive lanes; a lane takes items qi, qi + Q,
// ... (at most IPL of them). The k activations sit in LDS with one pad float
// per 32 and a stride that spreads a wave's simultaneous reads over the banks.
template <int T, int Q, int IPL>
__global__ void __launch_bounds__(256) down_combine_kernel(const DecodePlan *__restrict__ plan,
                                                           const float *__restrict__ h, int d, int fe, int k, int R,
                                                           int64_t row_bytes, int hstride, float *__restrict__ x) {
    using S = Split<T>;
    extern __shared__ float hs[];  // k padded rows of stride hstride, then ys [R][k]
    float *ys = hs + size_t(k) * hstride;
    const int o0 = blockIdx.x * R, tid = threadIdx.x;
    const int u = tid / Q, qi = tid % Q, r = u / k, jj = u % k;
    const int items = T == VT_Q8_0 ? fe / 64 : fe / 32;
    // this lane's rows' items, loaded before anything else
    const uint8_t *D = static_cast<const uint8_t *>(plan->down[jj]);
    typename S::Raw raw[IPL];
    const int64_t row = int64_t(o0 + r) * row_bytes;
    if (D) {
#pragma unroll
        for (int m = 0; m < IPL; m++) {
            const int it = qi + Q * m;
            if (it < items) raw[m] = S::fetch(D, row, it);
        }
    }
    // activations: float4 chunks never straddle a 32-float group
    const int fe4 = fe >> 2;
    for (int i = tid; i < k * fe4; i += 256) {
        const int j2 = i / fe4, c = 4 * (i - j2 * fe4);
        const float4 v = reinterpret_cast<const float4 *>(h)[i];
        float *dst = hs + j2 * hstride + c + (c >> 5);
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    }
    __syncthreads();
    float acc = 0.0f;
    if (D) {
        const float *hx = hs + size_t(jj) * hstride;
#pragma unroll
        for (int m = 0; m < IPL; m++) {
            const int it = qi + Q * m;
            if (it < items) acc += S::compute(raw[m], it, XPadded<T>{hx, it});
        }
    }
    acc = group_sum<Q>(acc);
    if (qi == Q - 1) ys[u] = acc;
    __syncthreads();
    if (tid < R) {
        float a = 0.0f;
        for (int j2 = 0; j2 < k; j2++) {
            if (!plan->down[j2]) continue;  // failed lookup: skipped (src/gguf_run.c:201)
            a = __fadd_rn(a, __fmul_rn(plan->w[j2], ys[tid * k + j2]));
        }
        x[o0 + tid] = __fadd_rn(x[o0 + tid], a);
    }
}

constexpr int kDownQ = 4;

// LDS stride between the k padded activation rows, chosen mod 64 banks so the
// items that the 64 lanes of a wave read together (4 lanes per (row, expert),
// 8 experts) fall in distinct banks: experts step the bank by 8 for Q8_0 (items
// are 66 padded floats apart, 2 banks), by 1 for Q6_K (items 8 apart) and by 5
// for Q4_K (items at 0/16/66/82).
int down_hstride(uint32_t type, int fe) {
    const int base = fe + (fe >> 5);
    const int target = type == VT_Q8_0 ? 8 : type == VT_Q6_K ? 1 : 5;
    return base + ((target - base % 64) + 64) % 64;
}

int items_of(uint32_t type, int fe) { return type == VT_Q8_0 ? fe / 64 : fe / 32; }

template <int T, int IPL>
int launch_down(const DecodePlan *plan, const float *h, int d, int fe, int k, float *x, hipStream_t s) {
    const int R = 256 / (kDownQ * k);
    const int64_t rb = row_bytes_of(T, fe);
    const int hstride = down_hstride(T, fe);
    const size_t lds = size_t(k) * hstride * 4 + size_t(R) * k * 4;
    hipLaunchKernelGGL((down_combine_kernel<T, kDownQ, IPL>), dim3(d / R), dim3(256), lds, s, plan, h, d, fe, k, R,
                       rb, hstride, x);
    return vh_check(hipGetLastError());
}

template <int T>
int launch_down_ipl(int ipl, const DecodePlan *plan, const float *h, int d, int fe, int k, float *x, hipStream_t s) {
    if (ipl <= 2) return launch_down<T, 2>(plan, h, d, fe, k, x, s);
    if (ipl <= 3) return launch_down<T, 3>(plan, h, d, fe, k, x, s);
    if (ipl <= 4) return launch_down<T, 4>(plan, h, d, fe, k, x, s);
    if (ipl <= 6) return launch_down<T, 6>(plan, h, d, fe, k, x, s);
    if (ipl <= 8) return launch_down<T, 8>(plan, h, d, fe, k, x, s);
    return -EINVAL;
}

}  // namespace

bool vh_decode_gateup_supported(uint32_t type, int d, int fe) {
    (void)fe;
    return d == 2048 && (type == VT_Q4_K || type == VT_Q8_0 || type == VT_Q6_K);
}

int vh_decode_gateup(uint32_t type, const RoutePart *parts, const float *R, const float *hb, const float *bias, int d,
                     int E, int k, int fe, int renorm, const void *const *table, float *h, int32_t *idx, float *w,
                     uint32_t *flags, DecodePlan *plan, hipStream_t s) {
    const int64_t rb = row_bytes_of(type, d);
    switch (type) {
    case VT_Q4_K: return launch_decode_gateup<VT_Q4_K, 64, 3>(parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, s);
    case VT_Q8_0: return launch_decode_gateup<VT_Q8_0, 32, 2>(parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, s);
    case VT_Q6_K: return launch_decode_gateup<VT_Q6_K, 64, 3>(parts, R, hb, bias, d, E, k, fe, renorm, table, rb, h, idx, w, flags, plan, s);
    default: return -EINVAL;
    }
}

bool vh_down_combine_supported(uint32_t type, int d, int fe, int k) {
    if (!(type == VT_Q4_K || type == VT_Q8_0 || type == VT_Q6_K)) return false;
    if (type == VT_Q8_0 && fe % 64) return false;
    if (k < 1 || k > 64 || 256 % (kDownQ * k)) return false;
    const int R = 256 / (kDownQ * k);
    if (d % R) return false;
    const int ipl = (items_of(type, fe) + kDownQ - 1) / kDownQ;
    if (ipl > 8) return false;
    return size_t(k) * down_hstride(type, fe) * 4 + size_t(R) * k * 4 <= 64 * 1024;
}

int vh_down_combine(uint32_t type, const DecodePlan *plan, const float *h, int d, int fe, int k, float *x,
                    hipStream_t s) {
    if (!vh_down_combine_supported(type, d, fe, k)) return -EINVAL;
    const int ipl = (items_of(type, fe) + kDownQ - 1) / kDownQ;
    switch (type) {
    case VT_Q4_K: return launch_down_ipl<VT_Q4_K>(ipl, plan, h, d, fe, k, x, s);
    case VT_Q8_0: return launch_down_ipl<VT_Q8_0>(ipl, plan, h, d, fe, k, x, s);
    case VT_Q6_K: return launch_down_ipl<VT_Q6_K>(ipl, plan, h, d, fe, k, x, s);
    default: return -EINVAL;
    }
}
