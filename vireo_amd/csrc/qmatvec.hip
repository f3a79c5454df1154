// qmatvec (gguf_matmul on the GPU) and qdequant_rows (gguf_dequant_row).
//
// qmatvec: each output row is split over L lanes of a wave (L chosen per shape
// so no lane idles), every lane decodes whole 32-weight items straight from
// the GGUF bytes with aligned loads, and the L partial sums are folded with a
// shuffle tree. Rows are streamed once; the kernel is HBM-bound. Matrices with
// many rows of 32..128 items (the LM head) take qmatvec_reg_kernel, which
// keeps each lane's inputs in registers across rows. With `accumulate` the
// kernels add their result to y (y_r + sum, one rounding, as a separate
// residual add of the stored result would give).
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route_kernels.h"
#include "vireo_hip.h"

namespace {

template <int T, bool PAIRED, int L>
__global__ void __launch_bounds__(256) qmatvec_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                      const uint8_t *__restrict__ w, int n, int d, int64_t row_bytes,
                                                      int accumulate) {
    using F = Fmt<T, PAIRED>;
    constexpr int RPW = 64 / L;
    const int lane = threadIdx.x & 63, sub = lane / L, li = lane % L;
    const int items = F::items(n);
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t nwaves = int64_t(gridDim.x) * 4;
    for (int64_t r0 = wave * RPW; r0 < d; r0 += nwaves * RPW) {
        const int64_t row = r0 + sub;
        float acc = 0.0f;
        if (row < d) {
            const int64_t ro = row * row_bytes;
            for (int it = li; it < items; it += L) acc += F::dot(w, ro, it, n, x);
        }
        acc = group_sum<L>(acc);
        if (li == L - 1 && row < d) y[row] = accumulate ? add_rn(y[row], acc) : acc;
    }
}

template <int T, bool PAIRED>
int launch_L(int L, float *y, const float *x, const uint8_t *w, int n, int d, int64_t rb, int acc, hipStream_t s) {
    const int rpw = 64 / L;
    int64_t waves = (int64_t(d) + rpw - 1) / rpw;
    int64_t blocks = (waves + 3) / 4;
    const int64_t cap = int64_t(vh_num_cus()) * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    dim3 g(static_cast<unsigned>(blocks)), b(256);
    switch (L) {
    case 64: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 64>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    case 32: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 32>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    case 16: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 16>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    case 8: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 8>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    case 4: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 4>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    case 2: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 2>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    default: hipLaunchKernelGGL((qmatvec_kernel<T, PAIRED, 1>), g, b, 0, s, y, x, w, n, d, rb, acc); break;
    }
    return vh_check(hipGetLastError());
}

// Up to three matrices over one input in one launch (a block's q, k and v
// projections): the rows of job 0, then of job 1, then of job 2 form one
// index space, and each row is computed as qmatvec_kernel computes it (L
// lanes, items li, li + L, ... summed in that order, then the lane tree),
// with the row's matrix type chosen at run time.
struct MvJob {
    float *y;
    const uint8_t *w;
    int64_t row_bytes;
    int d;
    uint32_t type;
};
template <int T, int L>
VH_DEV float row_partial(const uint8_t *w, int64_t ro, int li, int items, int n, const float *x) {
    float acc = 0.0f;
    for (int it = li; it < items; it += L) acc += Fmt<T, false>::dot(w, ro, it, n, x);
    return acc;
}
template <int L>
__global__ void __launch_bounds__(256) qmatvec3_kernel(MvJob j0, MvJob j1, MvJob j2, const float *__restrict__ x,
                                                       int n) {
    constexpr int RPW = 64 / L;
    const int lane = threadIdx.x & 63, sub = lane / L, li = lane % L;
    const int items = n / 32;
    const int64_t total = int64_t(j0.d) + j1.d + j2.d;
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t nwaves = int64_t(gridDim.x) * 4;
    for (int64_t r0 = wave * RPW; r0 < total; r0 += nwaves * RPW) {
        int64_t row = r0 + sub;
        MvJob j = j0;
        if (row >= j0.d) {
            row -= j0.d, j = j1;
            if (row >= j1.d) row -= j1.d, j = j2;
        }
        const bool live = row < j.d;
        float acc = 0.0f;
        if (live) {
            const int64_t ro = row * j.row_bytes;
            switch (j.type) {
            case VT_Q8_0: acc = row_partial<VT_Q8_0, L>(j.w, ro, li, items, n, x); break;
            case VT_Q4_K: acc = row_partial<VT_Q4_K, L>(j.w, ro, li, items, n, x); break;
            case VT_Q6_K: acc = row_partial<VT_Q6_K, L>(j.w, ro, li, items, n, x); break;
            case VT_Q5_0: acc = row_partial<VT_Q5_0, L>(j.w, ro, li, items, n, x); break;
            case VT_F16: acc = row_partial<VT_F16, L>(j.w, ro, li, items, n, x); break;
            default: acc = row_partial<VT_F32, L>(j.w, ro, li, items, n, x); break;
            }
        }
        acc = group_sum<L>(acc);
        if (li == L - 1 && live) j.y[row] = acc;
    }
}

// q, k and v on the register-resident decoders (Q4_K, Q6_K and Q8_0 rows of
// n = 64 IPL items or fewer, x 16-byte aligned): wave w takes kQ3Rows
// consecutive rows of one matrix - each matrix's row blocks numbered after
// the previous one's - and issues its inputs' loads and all its rows' raw
// words before using any (one memory round trip per wave), then reduces each
// row over the wave as qmatvec_reg_kernel does. NORM: the inputs are the
// RMSNorm of x with weights nw (null: unit weights), formed by every wave
// from the whole vector it holds, with rmsnorm_kernel's arithmetic (the
// squares summed in fp64 and rounded once, r = 1 / sqrtf(ss / n + eps),
// then (x r) w).
constexpr int kQ3Rows = 4;

template <int T, int IPL, bool NORM>
VH_DEV void q3_rows(const MvJob &j, int64_t r0, const float *__restrict__ x, const float *__restrict__ nw, float eps,
                    int n, int lane) {
    using F = Reg<T>;
    constexpr int NS = F::NS;
    const int items = F::items(n);
    float xr[IPL][32], xs[IPL][NS], wr[NORM ? IPL : 1][32];
    typename F::Raw raw[kQ3Rows][IPL];
#pragma unroll
    for (int m = 0; m < IPL; m++) F::load_x(x, min(lane + 64 * m, items - 1), xr[m]);
    if constexpr (NORM) {
#pragma unroll
        for (int m = 0; m < IPL; m++) F::load_x(nw ? nw : x, min(lane + 64 * m, items - 1), wr[m]);
    }
#pragma unroll
    for (int rr = 0; rr < kQ3Rows; rr++) {
        const int64_t row = min(r0 + rr, int64_t(j.d) - 1);  // unconditional: rows past the end repeat the last
#pragma unroll
        for (int m = 0; m < IPL; m++) raw[rr][m] = F::fetch(j.w, row * j.row_bytes, min(lane + 64 * m, items - 1));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the arithmetic
    if constexpr (NORM) {
        double ss = 0.0;
#pragma unroll
        for (int m = 0; m < IPL; m++)
            if (lane + 64 * m < items)  // each item once
#pragma unroll
                for (int i = 0; i < 32; i++) ss += double(mul_rn(xr[m][i], xr[m][i]));
        ss = wave_sum_d(ss);
        const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(float(ss), float(n)), eps)));
#pragma unroll
        for (int m = 0; m < IPL; m++)
#pragma unroll
            for (int i = 0; i < 32; i++) xr[m][i] = nw ? mul_rn(mul_rn(xr[m][i], r), wr[m][i]) : mul_rn(xr[m][i], r);
    }
#pragma unroll
    for (int m = 0; m < IPL; m++) F::sums(xr[m], xs[m]);
#pragma unroll
    for (int rr = 0; rr < kQ3Rows; rr++) {
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < IPL; m++) {
            const int it = lane + 64 * m;
            if (it < items) acc += F::compute(raw[rr][m], it, xr[m], xs[m]);
        }
        acc = group_sum<64>(acc);
        if (lane == 63 && r0 + rr < j.d) j.y[r0 + rr] = acc;
    }
}

template <int IPL, bool NORM>
__global__ void __launch_bounds__(256) qmatvec3_reg_kernel(MvJob j0, MvJob j1, MvJob j2, const float *__restrict__ x,
                                                           const float *__restrict__ nw, float eps, int n) {
    const int lane = threadIdx.x & 63;
    const int64_t w = int64_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t b0 = (j0.d + kQ3Rows - 1) / kQ3Rows, b1 = (j1.d + kQ3Rows - 1) / kQ3Rows,
                  b2 = (j2.d + kQ3Rows - 1) / kQ3Rows;
    MvJob j;
    int64_t r0;
    if (w < b0) {
        j = j0;
        r0 = w * kQ3Rows;
    } else if (w < b0 + b1) {
        j = j1;
        r0 = (w - b0) * kQ3Rows;
    } else if (w < b0 + b1 + b2) {
        j = j2;
        r0 = (w - b0 - b1) * kQ3Rows;
    } else {
        return;
    }
    switch (j.type) {
    case VT_Q4_K: q3_rows<VT_Q4_K, IPL, NORM>(j, r0, x, nw, eps, n, lane); break;
    case VT_Q6_K: q3_rows<VT_Q6_K, IPL, NORM>(j, r0, x, nw, eps, n, lane); break;
    default: q3_rows<VT_Q8_0, IPL, NORM>(j, r0, x, nw, eps, n, lane); break;
    }
}

// Lanes per row: the power of two (<= 64) that leaves the fewest idle item
// slots, preferring more lanes on a tie.
int pick_lanes(int items) {
    int best = 64, waste_best = 1 << 30;
    for (int L = 64; L >= 1; L >>= 1) {
        int waste = L * ((items + L - 1) / L) - items;
        if (waste < waste_best) { waste_best = waste; best = L; }
    }
    return best;
}

// Large matrices (the LM head): lane l of every wave owns items l, l + 64, ...
// (IPL of them, 32 weights each) of every row, so it loads its inputs (and
// their run sums) once and keeps them in registers for all the rows its wave
// computes; the wave fetches the raw words of RB rows at a time, then
// computes and reduces them (one full-wave DPP tree per row).
template <int T, int IPL, int RB>
__global__ void __launch_bounds__(256) qmatvec_reg_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                          const uint8_t *__restrict__ w, int n, int d,
                                                          int64_t row_bytes, int accumulate) {
    using F = Reg<T>;
    constexpr int NS = F::NS;
    const int lane = threadIdx.x & 63;
    const int items = F::items(n);
    float xr[IPL][32], xs[IPL][NS];
    // unconditional (lanes past the last item load it again, unused)
#pragma unroll
    for (int m = 0; m < IPL; m++) F::load_x(x, min(lane + 64 * m, items - 1), xr[m]);
#pragma unroll
    for (int m = 0; m < IPL; m++) F::sums(xr[m], xs[m]);
    const int64_t nw = int64_t(gridDim.x) * 4;
    for (int64_t r0 = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RB; r0 < d; r0 += nw * RB) {
        typename F::Raw raw[RB][IPL];
        // unconditional (items past the row repeat its last one and are not
        // used): under a condition the compiler waits for a row's loads before
        // the next row's are issued
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const int64_t row = r0 + rr < d ? r0 + rr : d - 1;
#pragma unroll
            for (int m = 0; m < IPL; m++) raw[rr][m] = F::fetch(w, row * row_bytes, min(lane + 64 * m, items - 1));
            // rows issued in order: the first row's arithmetic then waits for its own loads only
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            float acc = 0.0f;
#pragma unroll
            for (int m = 0; m < IPL; m++) {
                const int it = lane + 64 * m;
                if (it < items) acc += F::compute(raw[rr][m], it, xr[m], xs[m]);
            }
            acc = group_sum<64>(acc);
            if (lane == 63 && r0 + rr < d) y[r0 + rr] = accumulate ? add_rn(y[r0 + rr], acc) : acc;
        }
    }
}

template <int T, int RB>
int launch_reg_rb(float *y, const float *x, const uint8_t *w, int n, int d, int64_t rb, int acc, hipStream_t s) {
    const int items = n / 32;
    int64_t blocks = (int64_t(d) + 4 * RB - 1) / (4 * RB);
    const int64_t cap = int64_t(vh_num_cus()) * 8;
    if (blocks > cap) blocks = cap;
    dim3 g(static_cast<unsigned>(blocks)), b(256);
    if (items <= 64)
        hipLaunchKernelGGL((qmatvec_reg_kernel<T, 1, RB>), g, b, 0, s, y, x, w, n, d, rb, acc);
    else
        hipLaunchKernelGGL((qmatvec_reg_kernel<T, 2, RB>), g, b, 0, s, y, x, w, n, d, rb, acc);
    return vh_check(hipGetLastError());
}

// 8 rows per wave in flight, or 2 below 8192 rows, where 8 would leave too
// few workgroups to fill the chip (4096 Q4_K rows of 2048: 6.1 us at 8,
// 4.1 us at 2, 4.7 us at 1; 8192 Q8_0 rows: 5.9 us at 8, 7.2 us at 2)
template <int T>
int launch_reg(float *y, const float *x, const uint8_t *w, int n, int d, int64_t rb, int acc, hipStream_t s) {
    if (d >= 8192) return launch_reg_rb<T, 8>(y, x, w, n, d, rb, acc, s);
    return launch_reg_rb<T, 2>(y, x, w, n, d, rb, acc, s);
}

// the register-input kernel applies to Q8_0 / Q4_K / Q6_K rows of 32..128
// items with many rows and a 16-byte aligned input
bool reg_path(uint32_t type, const float *x, int n, int d) {
    if (type != VT_Q8_0 && type != VT_Q4_K && type != VT_Q6_K) return false;
    const int items = n / 32;
    return n % 32 == 0 && items >= 32 && items <= 128 && d >= 1024 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

// ---- dequant ----
template <int T>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t *__restrict__ src, float *__restrict__ dst, int n,
                                                      int rows, int64_t row_bytes, int items) {
#pragma clang fp contract(off)
    const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= int64_t(rows) * items) return;
    const int64_t row = gid / items;
    const int it = int(gid % items);
    const uint8_t *r = src + row * row_bytes;
    float *o = dst + row * int64_t(n);
    if constexpr (T == VT_Q8_0) {
        const uint8_t *b = r + 34 * it;
        const float d = h2f(ld_u16(b));
        for (int i = 0; i < 32; i++) o[32 * it + i] = mul_rn(float(int8_t(ld_u8(b + 2 + i))), d);
    } else if constexpr (T == VT_Q4_K) {
        // one 32-element sub-block j per thread (items = n/32): y = (d*sc)*q - dmin*m
        const int sbi = it >> 3, j = it & 7;
        const uint8_t *sb = r + 144 * sbi;
        const float d = h2f(ld_u16(sb)), dmin = h2f(ld_u16(sb + 2));
        const uint32_t s0 = ld_u32(sb + 4), s1 = ld_u32(sb + 8), s2 = ld_u32(sb + 12);
        int sc, m;
        q4k_scale_min(j, s0, s1, s2, sc, m);
        const float d1 = mul_rn(d, float(sc)), m1 = mul_rn(dmin, float(m));
        const uint8_t *q = sb + 16 + 32 * (j >> 1);
        const int sh = (j & 1) ? 4 : 0;
        for (int l = 0; l < 32; l++) o[256 * sbi + 32 * j + l] = sub_rn(mul_rn(d1, float((ld_u8(q + l) >> sh) & 15u)), m1);
    } else if constexpr (T == VT_Q6_K) {
        // 16 elements sharing one scale per thread (items = n/16)
        const int sbi = it >> 4, s = it & 15;
        const uint8_t *sb = r + 210 * sbi;
        const float d = h2f(ld_u16(sb + 208));
        const float ds = mul_rn(d, float(int8_t(ld_u8(sb + 192 + s))));
        const int hh = s >> 3, g = (s >> 1) & 3, half = s & 1;
        for (int i = 0; i < 16; i++) {
            const int l = 16 * half + i;
            const uint32_t qlb = ld_u8(sb + 64 * hh + l + 32 * (g & 1));
            const uint32_t lo4 = g >= 2 ? (qlb >> 4) : (qlb & 15u);
            const uint32_t hi2 = (ld_u8(sb + 128 + 32 * hh + l) >> (2 * g)) & 3u;
            o[256 * sbi + 128 * hh + 32 * g + l] = mul_rn(ds, float(int(lo4 | (hi2 << 4)) - 32));
        }
    } else if constexpr (T == VT_Q5_0) {
        const uint8_t *b = r + 22 * it;
        const float d = h2f(ld_u16(b));
        const uint32_t qh = ld_u16(b + 2) | (ld_u16(b + 4) << 16);
        for (int j = 0; j < 16; j++) {
            const uint32_t qs = ld_u8(b + 6 + j);
            o[32 * it + j] = mul_rn(float(int((qs & 15u) | (((qh >> j) & 1u) << 4)) - 16), d);
            o[32 * it + j + 16] = mul_rn(float(int((qs >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16), d);
        }
    } else if constexpr (T == VT_F16) {
        for (int i = 32 * it; i < n && i < 32 * it + 32; i++) o[i] = h2f(ld_u16(r + 2 * i));
    } else {
        const float *rf = reinterpret_cast<const float *>(r);
        for (int i = 32 * it; i < n && i < 32 * it + 32; i++) o[i] = rf[i];
    }
}

}  // namespace

// Host-side shape checks shared by the matvec entry points.
static int check_weights(uint32_t type, const void *data, int n, int d, int64_t *row_bytes) {
    int be, bb;
    if (vireo_type_block(type, &be, &bb) || type == VT_Q4_0) return -EINVAL;
    if (n <= 0 || d < 0 || n % be) return -EINVAL;
    if (!data && d) return -EINVAL;
    const uintptr_t a = reinterpret_cast<uintptr_t>(data);
    if (a & 3u) return -EINVAL;
    if (type == VT_Q4_K && (a & 15u)) return -EINVAL;
    *row_bytes = int64_t(n / be) * bb;
    return 0;
}

namespace {

int qmv(float *y, const float *x, const gguf_tensor *w, int n, int d, int acc, void *stream) {
    if (!w || (!y && d) || (!x && d)) return -EINVAL;
    int64_t rb;
    if (int rc = check_weights(w->ggml_type, w->data, n, d, &rb)) return rc;
    if (d == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *wd = static_cast<const uint8_t *>(w->data);
    if (reg_path(w->ggml_type, x, n, d)) {
        switch (w->ggml_type) {
        case VT_Q8_0: return launch_reg<VT_Q8_0>(y, x, wd, n, d, rb, acc, s);
        case VT_Q4_K: return launch_reg<VT_Q4_K>(y, x, wd, n, d, rb, acc, s);
        default: return launch_reg<VT_Q6_K>(y, x, wd, n, d, rb, acc, s);
        }
    }
    switch (w->ggml_type) {
    case VT_Q8_0:
        if (n % 64 == 0) return launch_L<VT_Q8_0, true>(pick_lanes(n / 64), y, x, wd, n, d, rb, acc, s);
        return launch_L<VT_Q8_0, false>(pick_lanes(n / 32), y, x, wd, n, d, rb, acc, s);
    case VT_Q4_K: return launch_L<VT_Q4_K, false>(pick_lanes(n / 32), y, x, wd, n, d, rb, acc, s);
    case VT_Q6_K: return launch_L<VT_Q6_K, false>(pick_lanes(n / 32), y, x, wd, n, d, rb, acc, s);
    case VT_Q5_0: return launch_L<VT_Q5_0, false>(pick_lanes(n / 32), y, x, wd, n, d, rb, acc, s);
    case VT_F16: return launch_L<VT_F16, false>(pick_lanes((n + 31) / 32), y, x, wd, n, d, rb, acc, s);
    case VT_F32: return launch_L<VT_F32, false>(pick_lanes((n + 31) / 32), y, x, wd, n, d, rb, acc, s);
    default: return -EINVAL;
    }
}

}  // namespace

extern "C" int qmatvec_async(float *y, const float *x, const gguf_tensor *w, int n, int d, void *stream) {
    return qmv(y, x, w, n, d, 0, stream);
}

int vh_qmatvec_acc(float *y, const float *x, const gguf_tensor *w, int n, int d, hipStream_t s) {
    return qmv(y, x, w, n, d, 1, s);
}

namespace {
// the three jobs of vh_qmatvec3 / vh_qmatvec3_normed, checked
int q3_jobs(int n, float *y0, const gguf_tensor *w0, int d0, float *y1, const gguf_tensor *w1, int d1, float *y2,
            const gguf_tensor *w2, int d2, MvJob (&j)[3]) {
    const gguf_tensor *w[3] = {w0, w1, w2};
    float *y[3] = {y0, y1, y2};
    const int d[3] = {d0, d1, d2};
    for (int i = 0; i < 3; i++) {
        if (!w[i] || !y[i] || d[i] <= 0) return -EINVAL;
        const uint32_t t = w[i]->ggml_type;
        if (t != VT_Q8_0 && t != VT_Q4_K && t != VT_Q6_K && t != VT_Q5_0 && t != VT_F16 && t != VT_F32) return -ENOTSUP;
        int64_t rb;
        if (int rc = check_weights(t, w[i]->data, n, d[i], &rb)) return rc;
        j[i] = MvJob{y[i], static_cast<const uint8_t *>(w[i]->data), rb, d[i], t};
    }
    return 0;
}

// the register-resident launch, where the types and sizes allow it
bool q3_reg_ok(const MvJob (&j)[3], const float *x, int n) {
    auto reg_type = [](uint32_t t) { return t == VT_Q4_K || t == VT_Q6_K || t == VT_Q8_0; };
    return reg_type(j[0].type) && reg_type(j[1].type) && reg_type(j[2].type) && n % 256 == 0 && n <= 64 * 32 * 2 &&
           (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

template <bool NORM>
int q3_reg_launch(const MvJob (&j)[3], const float *x, const float *nw, float eps, int n, hipStream_t s) {
    int64_t waves = 0;
    for (int i = 0; i < 3; i++) waves += (j[i].d + kQ3Rows - 1) / kQ3Rows;
    const dim3 g(static_cast<unsigned>((waves + 3) / 4)), b(256);
    if (n <= 64 * 32)
        hipLaunchKernelGGL((qmatvec3_reg_kernel<1, NORM>), g, b, 0, s, j[0], j[1], j[2], x, nw, eps, n);
    else
        hipLaunchKernelGGL((qmatvec3_reg_kernel<2, NORM>), g, b, 0, s, j[0], j[1], j[2], x, nw, eps, n);
    return vh_check(hipGetLastError());
}
}  // namespace

int vh_qmatvec3(const float *x, int n, float *y0, const gguf_tensor *w0, int d0, float *y1, const gguf_tensor *w1,
                int d1, float *y2, const gguf_tensor *w2, int d2, hipStream_t s) {
    if (!x || n <= 0 || n % 32) return -ENOTSUP;
    MvJob j[3];
    if (int rc = q3_jobs(n, y0, w0, d0, y1, w1, d1, y2, w2, d2, j)) return rc;
    if (q3_reg_ok(j, x, n)) return q3_reg_launch<false>(j, x, nullptr, 0.0f, n, s);
    const int L = pick_lanes(n / 32), rpw = 64 / L;
    const int64_t total = int64_t(d0) + d1 + d2;
    int64_t blocks = ((total + rpw - 1) / rpw + 3) / 4;
    const int64_t cap = int64_t(vh_num_cus()) * 16;
    if (blocks > cap) blocks = cap;
    dim3 g(static_cast<unsigned>(blocks)), b(256);
    switch (L) {
    case 64: hipLaunchKernelGGL(qmatvec3_kernel<64>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    case 32: hipLaunchKernelGGL(qmatvec3_kernel<32>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    case 16: hipLaunchKernelGGL(qmatvec3_kernel<16>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    case 8: hipLaunchKernelGGL(qmatvec3_kernel<8>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    case 4: hipLaunchKernelGGL(qmatvec3_kernel<4>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    case 2: hipLaunchKernelGGL(qmatvec3_kernel<2>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    default: hipLaunchKernelGGL(qmatvec3_kernel<1>, g, b, 0, s, j[0], j[1], j[2], x, n); break;
    }
    return vh_check(hipGetLastError());
}

int vh_qmatvec3_normed(const float *x, const float *nw, float eps, int n, float *y0, const gguf_tensor *w0, int d0,
                       float *y1, const gguf_tensor *w1, int d1, float *y2, const gguf_tensor *w2, int d2,
                       hipStream_t s) {
    if (!x || n <= 0 || n % 32 || (reinterpret_cast<uintptr_t>(nw) & 15u)) return -ENOTSUP;
    MvJob j[3];
    if (int rc = q3_jobs(n, y0, w0, d0, y1, w1, d1, y2, w2, d2, j)) return rc;
    if (!q3_reg_ok(j, x, n)) return -ENOTSUP;
    return q3_reg_launch<true>(j, x, nw, eps, n, s);
}

extern "C" int qmatvec(float *y, const float *x, const gguf_tensor *w, int n, int d) {
    return vh_finish(nullptr, qmatvec_async(y, x, w, n, d, nullptr));
}

extern "C" int qdequant_rows(uint32_t type, const void *src, float *dst, int n, int rows, void *stream) {
    int64_t rb;
    if (rows < 0 || (!dst && rows)) return -EINVAL;
    if (int rc = check_weights(type, src, n, rows, &rb)) return rc;
    if (rows == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *sp = static_cast<const uint8_t *>(src);
    int items;
    switch (type) {
    case VT_Q6_K: items = n / 16; break;
    case VT_F16: case VT_F32: items = (n + 31) / 32; break;
    default: items = n / 32; break;
    }
    const int64_t total = int64_t(rows) * items;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return -E2BIG;
    dim3 g(static_cast<unsigned>(blocks)), b(256);
    switch (type) {
    case VT_Q8_0: hipLaunchKernelGGL(dequant_kernel<VT_Q8_0>, g, b, 0, s, sp, dst, n, rows, rb, items); break;
    case VT_Q4_K: hipLaunchKernelGGL(dequant_kernel<VT_Q4_K>, g, b, 0, s, sp, dst, n, rows, rb, items); break;
    case VT_Q6_K: hipLaunchKernelGGL(dequant_kernel<VT_Q6_K>, g, b, 0, s, sp, dst, n, rows, rb, items); break;
    case VT_Q5_0: hipLaunchKernelGGL(dequant_kernel<VT_Q5_0>, g, b, 0, s, sp, dst, n, rows, rb, items); break;
    case VT_F16: hipLaunchKernelGGL(dequant_kernel<VT_F16>, g, b, 0, s, sp, dst, n, rows, rb, items); break;
    default: hipLaunchKernelGGL(dequant_kernel<VT_F32>, g, b, 0, s, sp, dst, n, rows, rb, items); break;
    }
    return vh_finish(s, vh_check(hipGetLastError()));
}
