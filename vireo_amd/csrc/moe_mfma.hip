// bf16 matrix-core (MFMA) grouped GEMMs for the grouped plan's large groups.
//
// moe_ffn (src/gguf_run.c:193-213) runs every (token, expert) pair as two
// matvecs; when a call carries many tokens, an expert's tokens form a group
// and its projections become GEMMs: H_e = silu(X_e G_e^T) * (X_e U_e^T) and
// Y_e = H_e D_e^T, with X_e the group's rows of hb gathered through the
// dispatch permutation. Groups of at least kMfmaMinTokens tokens run here on
// v_mfma_f32_16x16x32_bf16: the inputs are rounded to bf16, the weights are
// dequantized exactly (src/gguf_compute.c:52-120) and then rounded to bf16
// while they are staged, and products are accumulated in fp32. Smaller groups
// stay on the fp32 kernels of moe_grouped.hip.
//
// Tiles: a workgroup (256 threads, 4 waves in 2 x 2) owns kBM = 128 rows of
// one group (token tile) and 128 weight rows (gate/up: 64 rows of gate and the
// same 64 rows of up; down: 128 rows), and steps over K in kBK = 64 columns.
// Each step stages both operands in LDS, as 16-byte chunks of 8 consecutive
// K values laid out [K/8][row], so a 16-lane group's MFMA operand read is one
// contiguous 256-byte run. Global loads for step s + 1 are issued before the
// MFMAs of step s and written to the other LDS buffer after them; one barrier
// per step. The fp32 accumulators of a wave cover 64 rows x 64 columns.
//
// Outputs: gate/up writes h as bf16 rows in dispatch order (hs[offs[e] + i]),
// so the down GEMM reads its A operand contiguously; down writes the fp32 row
// y[pair] that the combine kernel reads, as on the fp32 plan.
#include <hip/hip_runtime.h>
#include "common.h"
#include "qdecode.h"
#include "route_kernels.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBK = 64, kBRows = 128, kThreads = 256;
constexpr int kChunks = kBK / 8;  // 16-byte chunks per row and K step

// 8 bytes at even byte offset c of a 4-aligned tensor, from aligned words
// that never leave [c - 2, c + 8): fetched into (w0, w1, w2) at load time,
// shifted into place (sh = c & 3 bytes) only when the values are needed, so
// the loads stay in flight across the MFMAs.
struct Even8 {
    uint32_t w0, w1, w2, sh;
    VH_DEV void load(gbyte *base, int64_t c) {
        sh = uint32_t(c) & 3u;
        gbyte *a = base + (c - int64_t(sh));
        w0 = ld_u32(a);
        w1 = ld_u32(a + 4);
        w2 = ld_u16(a + (sh ? 8 : 6));  // bytes c+6, c+7 (unused when sh == 0)
    }
    VH_DEV uint32_t lo() const { return align2(w1, w0, sh); }
    VH_DEV uint32_t hi() const { return align2(w2, w1, sh); }
};

// The raw bytes of 8 consecutive weights (columns c .. c+7, c a multiple of 8)
// of the row at byte offset ro of the 4-aligned tensor m, and their
// dequantization to fp32 with the reference's arithmetic (every value is that
// of gguf_dequant_row).
template <int T>
struct Chunk;

template <>
struct Chunk<VT_Q8_0> {  // src/gguf_compute.c:112-120: y = qs * d, exact
    Even8 q;
    uint32_t d;
    VH_DEV void load(gbyte *m, int64_t ro, int c) {
        const int64_t b = ro + 34 * int64_t(c >> 5);
        d = ld_u16(m + b);
        q.load(m, b + 2 + (c & 31));
    }
    VH_DEV void values(float (&v)[8]) const {
        const float s = h2f(d);
        const uint32_t w[2] = {q.lo(), q.hi()};
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = float(int(int8_t((w[i >> 2] >> (8 * (i & 3))) & 0xffu))) * s;
    }
};

template <>
struct Chunk<VT_Q4_K> {  // src/gguf_compute.c:52-66: y = (d*sc)*q - dmin*m
    uint4 hdr;
    uint2 q;
    int c;
    VH_DEV void load(gbyte *m, int64_t ro, int col) {
        gbyte *sb = m + ro + 144 * int64_t(col >> 8);
        const int cc = col & 255;
        c = cc;
        hdr = ld_u128(sb);
        q = ld_u64(sb + 16 + 32 * (cc >> 6) + (cc & 31));
    }
    VH_DEV void values(float (&v)[8]) const {
        const int j = 2 * (c >> 6) + ((c >> 5) & 1);  // sub-block; odd ones take the high nibbles
        int sc, mn;
        q4k_scale_min(j, hdr.y, hdr.z, hdr.w, sc, mn);
        const float d1 = h2f(hdr.x & 0xffffu) * float(sc), m1 = h2f(hdr.x >> 16) * float(mn);
        const uint32_t sh = (j & 1) ? 4u : 0u;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t qi = (((i < 4 ? q.x : q.y) >> (8 * (i & 3))) >> sh) & 15u;
            v[i] = d1 * float(qi) - m1;  // d1 * q is exact: one rounding, as in the reference
        }
    }
};

template <>
struct Chunk<VT_Q6_K> {  // src/gguf_compute.c:83-103: y = (d*sc)*(q - 32)
    Even8 ql, qh;
    uint32_t d, sc;
    int c;
    VH_DEV void load(gbyte *m, int64_t ro, int col) {
        const int64_t sbo = ro + 210 * int64_t(col >> 8);
        const int i = col & 255, h = i >> 7, g = (i >> 5) & 3, l = i & 31;
        c = i;
        ql.load(m, sbo + 64 * h + 32 * (g & 1) + l);
        qh.load(m, sbo + 128 + 32 * h + l);
        sc = ld_u8(m + sbo + 192 + 8 * h + (l >> 4) + 2 * g);
        d = ld_u16(m + sbo + 208);
    }
    VH_DEV void values(float (&v)[8]) const {
        const int g = (c >> 5) & 3;
        const float s = h2f(d) * float(int(int8_t(sc)));
        const uint32_t lsh = g >= 2 ? 4u : 0u, hsh = 2u * uint32_t(g);
        const uint32_t l2[2] = {ql.lo(), ql.hi()}, h2[2] = {qh.lo(), qh.hi()};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t lo = ((l2[i >> 2] >> (8 * (i & 3))) >> lsh) & 15u;
            const uint32_t hi = ((h2[i >> 2] >> (8 * (i & 3))) >> hsh) & 3u;
            v[i] = s * float(int(lo | (hi << 4)) - 32);
        }
    }
};

VH_DEV bf16x8 to_bf16(const float (&v)[8]) {
    f32x8 f;
#pragma unroll
    for (int i = 0; i < 8; i++) f[i] = v[i];
    return __builtin_convertvector(f, bf16x8);
}

// grid (rows_out / (GATEUP ? 64 : 128), max_tiles), 256 threads. Tile t of
// the plan is (expert e, first row m0 of its group). GATEUP: A = hb (fp32
// [T x K], row perm[i] / k), B = gate and up rows, out = hs (bf16 [P x rows],
// row i); else A = hs (bf16 [P x K], row i), B = down rows, out = y (fp32
// [P x rows], row perm[i]). i runs over offs[e] + m0 .. + kBM - 1 within the
// group.
template <int T, bool GATEUP>
__global__ void __launch_bounds__(kThreads) mfma_proj_kernel(const int32_t *__restrict__ tiles,
                                                             const int32_t *__restrict__ counts,
                                                             const int32_t *__restrict__ offs,
                                                             const int32_t *__restrict__ perm,
                                                             const void *const *__restrict__ table,
                                                             const void *__restrict__ src, int K, int rows, int k,
                                                             int64_t row_bytes, void *__restrict__ out) {
    __shared__ bf16x8 As[2][kChunks][kBM];
    __shared__ bf16x8 Bs[2][kChunks][kBRows];
    const int t = blockIdx.y;
    if (t >= tiles[0]) return;
    const int e = tiles[1 + 2 * t], m0 = tiles[2 + 2 * t];
    const int base = offs[e], mcnt = min(kBM, counts[e] - m0);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, wm = wv >> 1, wn = wv & 1;
    const int n0 = blockIdx.x * (GATEUP ? 64 : 128);

    gbyte *M0 = gmem(table[3 * e + (GATEUP ? 0 : 2)]);
    gbyte *M1 = GATEUP ? gmem(table[3 * e + 1]) : M0;
    if (!M0 || !M1) {
        // an unregistered expert contributes nothing (src/gguf_run.c:201): its
        // h rows are zero, and the combine skips its y rows
        if (GATEUP)
            for (int i = tid; i < mcnt * 64; i += kThreads)
                static_cast<__bf16 *>(out)[size_t(base + m0 + i / 64) * rows + n0 + i % 64] = __bf16(0.0f);
        return;
    }

    // this thread's staging slots: chunk tid + 256 q (q < 4) of each operand,
    // row (tid >> 3) + 32 q, K chunk tid & 7
    const int kc = tid & 7;
    // (rows past the group read its last row and stage zeros)
    const uint8_t *arow[4];
    bool aval[4];
    gbyte *bmat[4];
    int64_t boff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int r = (tid >> 3) + 32 * q;
        aval[q] = r < mcnt;
        const int i = base + m0 + min(r, mcnt - 1);
        arow[q] = GATEUP ? static_cast<const uint8_t *>(src) + size_t(perm[i] / k) * K * 4
                         : static_cast<const uint8_t *>(src) + size_t(i) * K * 2;
        bmat[q] = GATEUP ? (r < 64 ? M0 : M1) : M0;
        boff[q] = int64_t(GATEUP ? n0 + (r & 63) : n0 + r) * row_bytes;
    }

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // staged registers for one K step
    float4 ax[4][2];
    uint4 ah[4];
    Chunk<T> bw[4];
    auto load = [&](int k0) {
        const int c = k0 + 8 * kc;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (GATEUP) {
                ax[q][0] = *reinterpret_cast<const float4 *>(arow[q] + 4 * c);
                ax[q][1] = *reinterpret_cast<const float4 *>(arow[q] + 4 * c + 16);
            } else {
                ah[q] = *reinterpret_cast<const uint4 *>(arow[q] + 2 * c);
            }
            bw[q].load(bmat[q], boff[q], c);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int r = (tid >> 3) + 32 * q;
            if (GATEUP) {
                f32x8 f;
                f[0] = ax[q][0].x; f[1] = ax[q][0].y; f[2] = ax[q][0].z; f[3] = ax[q][0].w;
                f[4] = ax[q][1].x; f[5] = ax[q][1].y; f[6] = ax[q][1].z; f[7] = ax[q][1].w;
                As[buf][kc][r] = __builtin_convertvector(aval[q] ? f : f32x8{}, bf16x8);
            } else {
                As[buf][kc][r] = __builtin_bit_cast(bf16x8, aval[q] ? ah[q] : make_uint4(0u, 0u, 0u, 0u));
            }
            float w[8];
            bw[q].values(w);
            Bs[buf][kc][r] = to_bf16(w);
        }
    };

    // B rows of the wave's four 16-column fragments
    int bfr[4];
#pragma unroll
    for (int j = 0; j < 4; j++) bfr[j] = GATEUP ? (j < 2 ? 0 : 64) + 32 * wn + 16 * (j & 1) : 64 * wn + 16 * j;

    const int nk = K / kBK;
    load(0);
    store(0);
    __syncthreads();
    for (int s = 0; s < nk; s++) {
        const int buf = s & 1;
        if (s + 1 < nk) load((s + 1) * kBK);
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int kg = 4 * ks + (lane >> 4);
            bf16x8 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = As[buf][kg][64 * wm + 16 * i + (lane & 15)];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = Bs[buf][kg][bfr[j] + (lane & 15)];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds rows 4 (lane >> 4) + r, column lane & 15 of each
    // 16 x 16 fragment
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 64 * wm + 16 * i + 4 * (lane >> 4) + r;
            if (row >= mcnt) continue;
            const int pos = base + m0 + row;
            if (GATEUP) {
                __bf16 *hs = static_cast<__bf16 *>(out) + size_t(pos) * rows;
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    hs[n0 + 32 * wn + 16 * jj + (lane & 15)] = __bf16(swiglu(acc[i][jj][r], acc[i][2 + jj][r]));
                }
            } else {
                float *y = static_cast<float *>(out) + size_t(perm[pos]) * rows;
#pragma unroll
                for (int j = 0; j < 4; j++) y[n0 + 64 * wn + 16 * j + (lane & 15)] = acc[i][j][r];
            }
        }
}

// One workgroup: tiles = {n, (e, m0) x n} for the groups of at least
// min_tokens tokens (kBM rows per tile, experts ascending), and the list of
// the other non-empty groups in the dispatch kernel's `active` format
// (small[0 .. n), n at small[E]).
__global__ void __launch_bounds__(256) mfma_plan_kernel(const int32_t *__restrict__ counts, int E, int min_tokens,
                                                        int32_t *__restrict__ tiles, int32_t *__restrict__ small) {
    __shared__ int wsum[4][2];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int cnt = t < E ? counts[t] : 0;
    const bool big = cnt >= min_tokens;
    const int nt = big ? (cnt + kBM - 1) / kBM : 0, sm = (!big && cnt > 0) ? 1 : 0;
    int it = nt, is = sm;
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        const int ot = __shfl_up(it, sh, 64), os = __shfl_up(is, sh, 64);
        if (lane >= sh) { it += ot; is += os; }
    }
    if (lane == 63) { wsum[wv][0] = it; wsum[wv][1] = is; }
    __syncthreads();
    int bt = 0, bs = 0;
    for (int w = 0; w < wv; w++) { bt += wsum[w][0]; bs += wsum[w][1]; }
    const int ex_t = bt + it - nt, ex_s = bs + is - sm;
    for (int i = 0; i < nt; i++) {
        tiles[1 + 2 * (ex_t + i)] = t;
        tiles[2 + 2 * (ex_t + i)] = i * kBM;
    }
    if (sm) small[ex_s] = t;
    if (t == 255) {
        tiles[0] = ex_t + nt;
        small[E] = ex_s + sm;
    }
}

template <bool GATEUP>
int mfma_launch(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                const int32_t *perm, const void *const *table, const void *src, int K, int rows, int k,
                void *out, hipStream_t s) {
    const dim3 g(rows / (GATEUP ? 64 : 128), max_tiles);
    switch (type) {
    case VT_Q8_0:
        hipLaunchKernelGGL((mfma_proj_kernel<VT_Q8_0, GATEUP>), g, dim3(kThreads), 0, s, tiles, counts, offs, perm,
                           table, src, K, rows, k, vh_row_bytes(type, K), out);
        break;
    case VT_Q4_K:
        hipLaunchKernelGGL((mfma_proj_kernel<VT_Q4_K, GATEUP>), g, dim3(kThreads), 0, s, tiles, counts, offs, perm,
                           table, src, K, rows, k, vh_row_bytes(type, K), out);
        break;
    case VT_Q6_K:
        hipLaunchKernelGGL((mfma_proj_kernel<VT_Q6_K, GATEUP>), g, dim3(kThreads), 0, s, tiles, counts, offs, perm,
                           table, src, K, rows, k, vh_row_bytes(type, K), out);
        break;
    default: return -EINVAL;
    }
    return vh_check(hipGetLastError());
}

}  // namespace

bool vh_mfma_supported(uint32_t tg, uint32_t td, int d, int fe, int E) {
    auto ok = [](uint32_t t) { return t == VT_Q8_0 || t == VT_Q4_K || t == VT_Q6_K; };
    auto kq = [](uint32_t t, int n) { return t == VT_Q8_0 ? n % 32 == 0 : n % 256 == 0; };
    return ok(tg) && ok(td) && kq(tg, d) && kq(td, fe) && d % kBK == 0 && fe % kBK == 0 && fe % 64 == 0 &&
           d % 128 == 0 && E <= 256;
}

int vh_mfma_max_tiles(int P, int E) { return P / kBM + E; }

int vh_mfma_plan(const int32_t *counts, int E, int min_tokens, int32_t *tiles, int32_t *small, hipStream_t s) {
    if (E > 256) return -EINVAL;
    hipLaunchKernelGGL(mfma_plan_kernel, dim3(1), dim3(256), 0, s, counts, E, min_tokens, tiles, small);
    return vh_check(hipGetLastError());
}

int vh_mfma_gateup(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                   const int32_t *perm, const void *const *table, const float *hb, int d, int fe, int k, void *hs,
                   hipStream_t s) {
    return mfma_launch<true>(type, tiles, max_tiles, counts, offs, perm, table, hb, d, fe, k, hs, s);
}

int vh_mfma_down(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                 const int32_t *perm, const void *const *table, const void *hs, int d, int fe, float *ybuf,
                 hipStream_t s) {
    return mfma_launch<false>(type, tiles, max_tiles, counts, offs, perm, table, hs, fe, d, 1, ybuf, s);
}
