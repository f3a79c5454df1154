// bf16 matrix-core (MFMA) grouped GEMMs for the groups of large calls.
//
// moe_ffn (src/gguf_run.c:193-213) runs every (token, expert) pair as two
// matvecs; when a call carries many tokens, an expert's tokens form a group
// and its projections become GEMMs: H_e = silu(X_e G_e^T) * (X_e U_e^T) and
// Y_e = H_e D_e^T, with X_e the group's rows of hb gathered through the
// dispatch permutation. Every group of a call of at least kMfmaMinCall
// tokens runs here on v_mfma_f32_32x32x16_bf16 (a group smaller than a token
// tile leaves the tile's other rows unused; the tile's cost is staging its
// weights either way): the inputs are rounded to bf16, the weights are
// dequantized exactly (src/gguf_compute.c:52-120) and then rounded to bf16
// while they are staged, and products are accumulated in fp32.
//
// Tiles: a workgroup (512 threads) owns a token tile of 32, 64 or 128 rows of
// one group (whole 128-row tiles, the remainder in the smallest that holds
// it) and kBRows = 256 weight rows (gate/up: 128 rows of gate and the same
// 128 rows of up; down: 256 rows), and steps over K in kBK = 64 columns. The
// inputs pass through LDS as 16-byte chunks of 8 consecutive K values laid
// out [K/8][row] (row index XOR-swizzled by the chunk), so a 32-lane group's
// operand read is one contiguous 512-byte run. GGUF-row experts: four waves
// multiply and four stage the weights through LDS too (mfma_proj_kernel);
// pinned Q8_0 experts come from a copy in the operand order and every wave
// multiplies, reading its own weights (mfma_frag_kernel).
//
// Order: the workgroups are numbered so that each XCD (hardware dispatch sends
// workgroup b to XCD b mod 8) takes a contiguous run of (token tile, column
// tile) pairs, column tiles fastest: the workgroups sharing a token tile, and
// the consecutive token tiles of one expert that share its weight tiles, meet
// in the same L2. The runs are cut at equal shares of the staged bytes.
//
// Outputs: gate/up writes h as bf16 rows in dispatch order (hs[offs[e] + i]),
// so the down GEMM reads its A operand contiguously; down writes the fp32 row
// y[pair] that the combine kernel reads, as on the fp32 plan.
#include <hip/hip_runtime.h>
#include <vector>
#include <algorithm>
#include <type_traits>
#include "common.h"
#include "qdecode.h"
#include "route_kernels.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBK = 64, kBRows = 256, kThreads = 512, kXcds = 8;
constexpr int kChunks = kBK / 8;  // 16-byte chunks per row and K step
#ifndef VH_MFMA_SETS
#define VH_MFMA_SETS 2
#endif
// register sets of the staging waves: a step's global loads are issued
// sets<T>() - 1 K steps before its words are dequantized into LDS (a Q4_K
// set holds 64 registers, a Q6_K set 96: two fit)
template <int T>
constexpr int sets() { return (T & 0xff) == VT_Q8_0 ? VH_MFMA_SETS : 2; }

// The raw bytes of 8 consecutive weights of one row - K chunk kc (columns
// 64 s + 8 kc .. + 7) of K step s - and their dequantization to fp32 with the
// reference's arithmetic (every value is that of gguf_dequant_row). Pos holds
// what does not change with s (setup() takes the row's byte offset ro in the
// 4-aligned tensor, under 4 GiB); Raw holds one step's words (load()); the
// step enters the addresses only through uniform base pointers.
template <int T>
struct Chunk;

template <>
struct Chunk<VT_Q8_0> {  // src/gguf_compute.c:112-120: y = qs * d, exact
    // block (2 s + kc / 4) starts at ob + 68 s and the thread's 8 quant bytes
    // at oq + 68 s, an even offset: one 8-byte load (global memory accepts any
    // alignment), one 16-bit load of the scale
    struct Pos {
        uint32_t ob, oq;
    };
    struct Raw {
        uint32_t d;
        uint2 q;
    };
    static VH_DEV void setup(Pos &p, uint32_t ro, int kc) {
        p.ob = ro + 34u * uint32_t(kc >> 2);
        p.oq = p.ob + 2u + 8u * uint32_t(kc & 3);
    }
    static VH_DEV void load(const Pos &p, Raw &r, gbyte *m, int s) {
        gbyte *ms = m + 68 * s;
        r.d = ld_u16(ms + p.ob);
        r.q = ld_u64(ms + p.oq);
    }
    static VH_DEV void values(const Pos &, const Raw &r, int, float (&v)[8]) {
        // q + 128 as an unsigned byte, converted with v_cvt_f32_ubyte*; then
        // (q + 128) * s - 128 * s is q * s exactly (at most 19 significant bits)
        const float sc = h2f(r.d), off = -128.0f * sc;
        uint32_t u0 = r.q.x ^ 0x80808080u, u1 = r.q.y ^ 0x80808080u;
        asm volatile("" : "+v"(u0), "+v"(u1));
        const uint32_t w[2] = {u0, u1};
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = fmaf(float((w[i >> 2] >> (8 * (i & 3))) & 0xffu), sc, off);
    }
};

template <>
struct Chunk<VT_Q4_K> {  // src/gguf_compute.c:52-66: y = (d*sc)*q - dmin*m
    // step s lies in super-block s / 4 and its chunk pair s % 4 (both
    // uniform); the thread's 8 nibbles are bytes 8 (kc % 4) .. + 7 of the
    // pair's 32: low nibbles (sub-block 2 (s % 4)) for kc < 4, else high
    struct Pos {
        uint32_t ro, oq, hi;
    };
    struct Raw {
        uint4 hdr;
        uint2 q;
    };
    static VH_DEV void setup(Pos &p, uint32_t ro, int kc) {
        p.ro = ro;
        p.oq = ro + 16u + 8u * uint32_t(kc & 3);
        p.hi = uint32_t(kc >> 2);
    }
    static VH_DEV void load(const Pos &p, Raw &r, gbyte *m, int s) {
        gbyte *ms = m + 144 * (s >> 2);
        r.hdr = ld_u128(ms + p.ro);
        r.q = ld_u64(ms + 32 * (s & 3) + p.oq);
    }
    static VH_DEV void values(const Pos &p, const Raw &r, int s, float (&v)[8]) {
        int sc, mn;
        q4k_scale_min(2 * (s & 3) + int(p.hi), r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
        const float d1 = h2f(r.hdr.x & 0xffffu) * float(sc), m1 = h2f(r.hdr.x >> 16) * float(mn);
        const uint32_t sh = 4u * p.hi;
        uint32_t w0 = (r.q.x >> sh) & 0x0f0f0f0fu, w1 = (r.q.y >> sh) & 0x0f0f0f0fu;
        asm volatile("" : "+v"(w0), "+v"(w1));
        const uint32_t w[2] = {w0, w1};
#pragma unroll
        for (int i = 0; i < 8; i++)  // d1 * q is exact: one rounding, as in the reference
            v[i] = fmaf(d1, float((w[i >> 2] >> (8 * (i & 3))) & 0xffu), -m1);
    }
};

// 8 bytes at even byte offset c of a 4-aligned tensor, read as aligned words
// that stay in [c - 2, c + 8) and shifted into place (by sh = c & 3 bytes)
// when used. p points at c.
struct Even8 {
    uint32_t w0, w1, w2, sh;
    VH_DEV void load(gbyte *p, uint32_t shift) {
        sh = shift;
        gbyte *a = p - sh;
        w0 = ld_u32(a);
        w1 = ld_u32(a + 4);
        w2 = ld_u16(a + (sh ? 8 : 6));  // bytes c+6, c+7 (unused when sh == 0)
    }
    VH_DEV uint32_t lo() const { return align2(w1, w0, sh); }
    VH_DEV uint32_t hi() const { return align2(w2, w1, sh); }
};

template <>
struct Chunk<VT_Q6_K> {  // src/gguf_compute.c:83-103: y = (d*sc)*(q - 32)
    // step s: super-block b = s / 4 at byte U = 210 b of the row, half
    // h = (s % 4) / 2, both uniform. The thread's 8 elements are l = 8 (kc % 4)
    // .. + 7 of group g = 2 (s % 2) + kc / 4: the low (g < 2) or high nibbles
    // of ql[64 h + 32 (g % 2) + l], bits 2g of qh[32 h + l], scale
    // [8 h + l / 16 + 2 g]. U is even, so a field's alignment is that of its
    // offset within the row's first super-block plus 2 (b % 2).
    struct Pos {
        uint32_t oql, oqh, osc, od, gl;
    };
    struct Raw {
        Even8 ql, qh;
        uint32_t d, sc;
    };
    static VH_DEV void setup(Pos &p, uint32_t ro, int kc) {
        const uint32_t l = 8u * uint32_t(kc & 3);
        p.oql = ro + 32u * uint32_t(kc >> 2) + l;
        p.oqh = ro + 128u + l;
        p.osc = ro + 192u + (l >> 4) + 2u * uint32_t(kc >> 2);
        p.od = ro + 208u;
        p.gl = uint32_t(kc >> 2);
    }
    static VH_DEV void load(const Pos &p, Raw &r, gbyte *m, int s) {
        const int b = s >> 2, h = (s & 3) >> 1;
        gbyte *ms = m + 210 * b;
        const uint32_t odd = 2u * uint32_t(b & 1);
        r.ql.load(ms + 64 * h + p.oql, (p.oql + odd) & 3u);
        r.qh.load(ms + 32 * h + p.oqh, (p.oqh + odd) & 3u);
        r.sc = ld_u8(ms + 8 * h + 4 * (s & 1) + p.osc);
        r.d = ld_u16(ms + p.od);
    }
    static VH_DEV void values(const Pos &p, const Raw &r, int s, float (&v)[8]) {
        const uint32_t g = 2u * uint32_t(s & 1) + p.gl;
        const float sc = h2f(r.d) * float(int(int8_t(r.sc)));
        const uint32_t lsh = g >= 2 ? 4u : 0u, hsh = 2u * g;
        uint32_t w0 = ((r.ql.lo() >> lsh) & 0x0f0f0f0fu) | (((r.qh.lo() >> hsh) & 0x03030303u) << 4);
        uint32_t w1 = ((r.ql.hi() >> lsh) & 0x0f0f0f0fu) | (((r.qh.hi() >> hsh) & 0x03030303u) << 4);
        asm volatile("" : "+v"(w0), "+v"(w1));
        const uint32_t w[2] = {w0, w1};
        // sc * q - 32 sc is sc * (q - 32) exactly before its one rounding, as
        // in the reference's (d * sc) * (q - 32)
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = fmaf(sc, float((w[i >> 2] >> (8 * (i & 3))) & 0xffu), -32.0f * sc);
    }
};

VH_DEV bf16x8 to_bf16(const float (&v)[8]) {
    f32x8 f;
#pragma unroll
    for (int i = 0; i < 8; i++) f[i] = v[i];
    return __builtin_convertvector(f, bf16x8);
}

// One token tile of BM rows (32, 64 or 128) against kBRows weight rows, by
// the 512 threads of mfma_proj_kernel. A is bf16: GATEUP: xb [T x K], row
// perm[i] / k; else hs [P x K], row i. GATEUP: B = gate and up rows, out = hs
// (bf16 [P x rows], row i); else B = down rows, out = y (fp32 [P x rows], row
// perm[i]). i runs over base + m0 .. + mcnt - 1 (mcnt <= BM) within the
// group; rows of the tile past mcnt repeat the group's last row and are not
// stored.
//
// Waves 0-3 only multiply: WM x WN of them share the tile (BM = 128 and 64:
// 2 x 2, BM = 32: 1 x 4), wave c owning rows (BM / WM) (c / WN) .. + BM / WM - 1
// and kBRows / WN of the weight rows (gate/up: as many columns of gate as of
// up), FI x FJ 32 x 32 accumulator fragments. Waves 4-7 only stage: their
// global loads run sets<T>() K steps ahead in register sets, and each step
// they dequantize the set that arrived a step ago into the LDS buffer the
// multiplying waves will read next. Every SIMD holds one wave of each kind,
// so the matrix cores and the vector ALUs work at the same time; one barrier
// per K step. A tile of fewer rows stages fewer input bytes per step for the
// same weight bytes: small groups cost less than a full tile.
template <int T, bool GATEUP, int BM>
VH_DEV void mfma_tile(bf16x8 (&As)[2][kChunks][kBM], bf16x8 (&Bs)[2][kChunks][kBRows], int (&prow)[kBM], gbyte *M0,
                      gbyte *M1, const int32_t *__restrict__ perm, const __bf16 *__restrict__ src, int K, int rows,
                      int k, int64_t row_bytes, void *__restrict__ out, int base, int m0, int mcnt, int n0) {
    static_assert(BM == 32 || BM == 64 || BM == 128, "token tiles of 32, 64 or 128 rows");
    constexpr int NCOL = GATEUP ? kBRows / 2 : kBRows;  // output columns per workgroup
    constexpr int WM = BM >= 64 ? 2 : 1, WN = 4 / WM;    // multiplying waves along rows, columns
    constexpr int FI = BM / 32 / WM, FJ = kBRows / WN / 32;  // fragments per wave
    constexpr int AQ = BM / 32;                          // input rows staged per staging thread
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nk = K / kBK;
    // down: the y row of each tile row (the dispatch permutation) in LDS for
    // the epilogue, read once here (threads of the multiplying waves; the
    // first barrier below publishes it): loaded under the epilogue's row
    // condition, each store waited for its own load
    if (!GATEUP && tid < BM) prow[tid] = perm[base + m0 + min(tid, mcnt - 1)];

    if (wv >= 4) {
        // ---- staging waves: thread p stages K chunk kc = p & 7 of A rows
        // (p >> 3) + 32 q (q < AQ) and of B rows (p >> 3) + 32 q (q < 8).
        // In LDS, chunk kc of row r sits at [kc][r ^ kc]: the 8 lanes of a row
        // write 8 different bank groups, and a 32-lane operand read stays
        // conflict-free. The K step enters the global addresses only through
        // uniform base pointers.
        const int p = tid - 256, kc = p & 7, rx = (p >> 3) ^ kc;
        gbyte *abase = gmem(src);
        uint32_t aoff[AQ];
#pragma unroll
        for (int q = 0; q < AQ; q++) {
            const int i = base + m0 + min((p >> 3) + 32 * q, mcnt - 1);
            aoff[q] = uint32_t((GATEUP ? size_t(perm[i] / k) : size_t(i)) * K * 2) + 16u * uint32_t(kc);
        }
        // B rows (p >> 3) + 32 q lie 32 q rows (gate/up: 32 (q % 4) rows of
        // gate or up) past row p >> 3: one set of offsets, and per q a uniform
        // base pointer (32 rows are a multiple of 4 bytes, so alignments agree)
        using C = Chunk<T>;
        constexpr int kSets = sets<T>();
        typename C::Pos bp;
        C::setup(bp, uint32_t(n0 + (p >> 3)) * uint32_t(row_bytes), kc);
        gbyte *bm[8];
#pragma unroll
        for (int q = 0; q < 8; q++) bm[q] = (GATEUP && q >= 4 ? M1 : M0) + (GATEUP ? q & 3 : q) * 32 * row_bytes;

        struct Stage {
            uint4 ah[AQ];
            typename C::Raw bw[8];
        } st[kSets];
        auto load = [&](Stage &g, int step) {
            gbyte *as = abase + 128 * step;
#pragma unroll
            for (int q = 0; q < AQ; q++) g.ah[q] = ld_u128(as + aoff[q]);
#pragma unroll
            for (int q = 0; q < 8; q++) C::load(bp, g.bw[q], bm[q], step);
        };
        auto store = [&](const Stage &g, int buf, int step) {
#pragma unroll
            for (int q = 0; q < AQ; q++) As[buf][kc][rx + 32 * q] = __builtin_bit_cast(bf16x8, g.ah[q]);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                float w[8];
                C::values(bp, g.bw[q], step, w);
                Bs[buf][kc][rx + 32 * q] = to_bf16(w);
            }
        };
        // step t's words live in register set t % kSets: issued at step
        // t - kSets, dequantized into LDS at step t - 1
#pragma unroll
        for (int j = 0; j < kSets; j++) load(st[j], min(j, nk - 1));
        store(st[0], 0, 0);
        lds_barrier();
        for (int s0 = 0; s0 < nk; s0 += kSets) {
#pragma unroll
            for (int j = 0; j < kSets; j++) {
                // step s: the multiplying waves read buffer s & 1
                const int s = s0 + j;
                if (s >= nk) break;
                load(st[j], min(s + kSets, nk - 1));  // unconditional: the waits count only older loads
                if (s + 1 < nk) store(st[(j + 1) % kSets], (s + 1) & 1, s + 1);
                lds_barrier();  // LDS only: the loads in flight stay in flight
            }
        }
        return;
    }

    // ---- multiplying waves: v_mfma_f32_32x32x16_bf16 (lane l supplies row
    // l % 32, K values 8 (l / 32) .. + 7 of each operand; it holds column
    // l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 of the 32 x 32 result)
    const int wm = wv / WN, wn = wv % WN;
    // B rows of the wave's FJ 32-column fragments (gate/up: FJ / 2 of gate,
    // the same FJ / 2 of up)
    int bfr[FJ];
#pragma unroll
    for (int j = 0; j < FJ; j++)
        bfr[j] = GATEUP ? (j < FJ / 2 ? 0 : NCOL) + (NCOL / WN) * wn + 32 * (j % (FJ / 2)) : (kBRows / WN) * wn + 32 * j;
    f32x16 acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int j = 0; j < FJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    lds_barrier();  // buffer 0 staged
    for (int s = 0; s < nk; s++) {
        const int buf = s & 1;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int kg = 2 * ks + (lane >> 5), lx = (lane & 31) ^ kg;
            bf16x8 a[FI], b[FJ];
#pragma unroll
            for (int i = 0; i < FI; i++) a[i] = As[buf][kg][lx + (BM / WM) * wm + 32 * i];
#pragma unroll
            for (int j = 0; j < FJ; j++) b[j] = Bs[buf][kg][lx + bfr[j]];
#pragma unroll
            for (int i = 0; i < FI; i++)
#pragma unroll
                for (int j = 0; j < FJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        lds_barrier();
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = (BM / WM) * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row >= mcnt) continue;
            const int pos = base + m0 + row;
            if (GATEUP) {
                __bf16 *hs = static_cast<__bf16 *>(out) + size_t(pos) * rows;
#pragma unroll
                for (int jj = 0; jj < FJ / 2; jj++)
                    hs[n0 + (NCOL / WN) * wn + 32 * jj + (lane & 31)] = __bf16(swiglu(acc[i][jj][r], acc[i][FJ / 2 + jj][r]));
            } else {
                float *y = static_cast<float *>(out) + size_t(prow[row]) * rows;
#pragma unroll
                for (int j = 0; j < FJ; j++) y[n0 + (kBRows / WN) * wn + 32 * j + (lane & 31)] = acc[i][j][r];
            }
        }
}

// kXcds x slots workgroups of 512 threads (slots from tile_cost). The plan
// (mfma_plan_kernel) holds n tiles (expert, size, first row of its group)
// and, per launch, where each XCD's run of (tile, column tile) pairs starts:
// workgroup b runs on XCD b mod 8 (hardware dispatch) and takes pair
// start[b mod 8] + b / 8 of that XCD's contiguous run, column tiles fastest,
// so the workgroups sharing a token tile, and the consecutive token tiles of
// one expert that share its weight tiles, meet in the same L2. The runs are
// cut at equal shares of the staged bytes (tiles of fewer rows cost less).
template <int T, bool GATEUP>
__global__ void __launch_bounds__(kThreads) mfma_proj_kernel(const int32_t *__restrict__ tiles,
                                                             const int32_t *__restrict__ counts,
                                                             const int32_t *__restrict__ offs,
                                                             const int32_t *__restrict__ perm,
                                                             const void *const *__restrict__ table,
                                                             const __bf16 *__restrict__ src, int K, int rows, int k,
                                                             int64_t row_bytes, void *__restrict__ out) {
    constexpr int NCOL = GATEUP ? kBRows / 2 : kBRows;  // output columns per workgroup
    __shared__ bf16x8 As[2][kChunks][kBM];
    __shared__ bf16x8 Bs[2][kChunks][kBRows];
    __shared__ int prow[kBM];
    const int nct = rows / NCOL, xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
    const int32_t *run = tiles + (GATEUP ? kPlanRunsGU : kPlanRunsDN);
    const int L = run[xcd] + slot;
    if (L >= run[xcd + 1]) return;
    const int t = L / nct, n0 = (L % nct) * NCOL;
    const int code = tiles[kPlanHead + 2 * t], m0 = tiles[kPlanHead + 2 * t + 1];
    const int e = code & 0xffff, bmt = code >> 16;
    const int base = offs[e], mcnt = min(bmt, counts[e] - m0);
    const int tid = threadIdx.x;

    gbyte *M0 = gmem(table[3 * e + (GATEUP ? 0 : 2)]);
    gbyte *M1 = GATEUP ? gmem(table[3 * e + 1]) : M0;
    if (!M0 || !M1) {
        // an unregistered expert contributes nothing (src/gguf_run.c:201): its
        // h rows are zero, and the combine skips its y rows
        if (GATEUP)
            for (int i = tid; i < mcnt * NCOL; i += kThreads)
                static_cast<__bf16 *>(out)[size_t(base + m0 + i / NCOL) * rows + n0 + i % NCOL] = __bf16(0.0f);
        return;
    }
    if (bmt == 32)
        mfma_tile<T, GATEUP, 32>(As, Bs, prow, M0, M1, perm, src, K, rows, k, row_bytes, out, base, m0, mcnt, n0);
    else if (bmt == 64)
        mfma_tile<T, GATEUP, 64>(As, Bs, prow, M0, M1, perm, src, K, rows, k, row_bytes, out, base, m0, mcnt, n0);
    else
        mfma_tile<T, GATEUP, 128>(As, Bs, prow, M0, M1, perm, src, K, rows, k, row_bytes, out, base, m0, mcnt, n0);
}

// ---- Q8_0 experts packed in the matrix cores' operand order (kQ8Frag) ----
//
// A pinned Q8_0 layer's experts are copied once (vh_mfma_pack_q8) into
// fragments: fragment (g, s) of a matrix is the 32 weight rows one
// v_mfma_f32_32x32x16_bf16 B operand takes (gate/up: rows 16 g .. 16 g + 15 of
// gate, then the same rows of up; down: rows 32 g .. 32 g + 31) over K step s
// (64 columns), kFragBytes bytes: first, lane l's 32 quant bytes - row l % 32,
// columns 64 s + 16 ks + 8 (l / 32) .. + 7 for ks = 0..3, the 8 bytes it
// supplies to sub-step ks - then the rows' two block scales (2 x fp16 per row,
// blocks 2 s and 2 s + 1). A wave reads its B operand for a K step with two
// 1 KB and one 128 B load instructions of consecutive bytes and dequantizes
// it in its own registers; only the activations pass through LDS.
constexpr int kFragBytes = 2176;

// One token tile of BM rows against 8 fragments (gate/up: 128 output columns;
// down: 256), 512 threads: wave w multiplies all BM rows by fragment w, FI =
// BM / 32 accumulators. Per K step every thread dequantizes its wave's B
// operand loaded two steps earlier (the values of Chunk<VT_Q8_0>, rounded to
// bf16 the same way, in the same K order: the results equal mfma_tile's bit for
// bit), issues the loads of two steps ahead, multiplies, and stores the
// inputs of the next step into the other LDS buffer. The barrier is LDS-only:
// global loads stay in flight across it.
template <bool GATEUP, int BM>
VH_DEV void frag_tile(bf16x8 (&As)[2][kChunks][kBM], int (&prow)[kBM], gbyte *F, const int32_t *__restrict__ perm,
                      const __bf16 *__restrict__ src, int K, int rows, int k, void *__restrict__ out, int base, int m0,
                      int mcnt, int n0) {
    constexpr int FI = BM / 32, AQ = (BM * kChunks + kThreads - 1) / kThreads;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nk = K / kBK;
    // down: the y row of each tile row in LDS for the epilogue (as mfma_tile;
    // the first barrier below publishes it)
    if (!GATEUP && tid < BM) prow[tid] = perm[base + m0 + min(tid, mcnt - 1)];
    // this wave's fragments: g = n0 / 16 + wv (gate/up) or n0 / 32 + wv (down)
    gbyte *fb = F + size_t((GATEUP ? n0 / 16 : n0 / 32) + wv) * nk * kFragBytes;
    gbyte *fq = fb + 32 * lane, *fs = fb + 2048 + 4 * (lane & 31);
    // input staging: chunk slot c = tid + 512 q holds K chunk c & 7 of tile row
    // c >> 3 (rows past the group repeat its last row; slots past the tile
    // fill LDS rows that are not read). Every load is unconditional (steps
    // past the end repeat the last one), so the waits before each use count
    // exactly the loads issued after it.
    gbyte *abase = gmem(src);
    uint32_t aoff[AQ];
    int arow[AQ];
#pragma unroll
    for (int q = 0; q < AQ; q++) {
        const int c = tid + kThreads * q, r = c >> 3, kc = c & 7;
        const int i = base + m0 + min(r, mcnt - 1);
        aoff[q] = uint32_t((GATEUP ? size_t(perm[i] / k) : size_t(i)) * K * 2) + 16u * uint32_t(kc);
        arow[q] = r ^ kc;
    }
    uint4 av[2][AQ], bq[2][2];
    uint32_t bs[2];
    auto loadA = [&](int set, int step) {
#pragma unroll
        for (int q = 0; q < AQ; q++) av[set][q] = ld_u128(abase + 128 * step + aoff[q]);
    };
    auto storeA = [&](int set, int buf) {
#pragma unroll
        for (int q = 0; q < AQ; q++)
            As[buf][(tid + kThreads * q) & 7][arow[q]] = __builtin_bit_cast(bf16x8, av[set][q]);
    };
    auto loadB = [&](int set, int step) {
        bq[set][0] = ld_u128(fq + size_t(step) * kFragBytes);
        bq[set][1] = ld_u128(fq + size_t(step) * kFragBytes + 16);
        bs[set] = ld_u32(fs + size_t(step) * kFragBytes);
    };
    f32x16 acc[FI];
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;

    // K step s: B(s) in register set s % 2, A(s + 1) in set (s + 1) % 2, LDS
    // buffer s % 2 holds A(s)
    auto step = [&](int s, auto SET) {
        constexpr int set = decltype(SET)::value, nset = 1 - set;
        // B(s): (q + 128) * d - 128 * d = q * d exactly, then bf16
        bf16x8 b[4];
        const uint32_t w[8] = {bq[set][0].x, bq[set][0].y, bq[set][0].z, bq[set][0].w,
                               bq[set][1].x, bq[set][1].y, bq[set][1].z, bq[set][1].w};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const float sc = h2f(ks < 2 ? bs[set] & 0xffffu : bs[set] >> 16), off = -128.0f * sc;
            uint32_t u0 = w[2 * ks] ^ 0x80808080u, u1 = w[2 * ks + 1] ^ 0x80808080u;
            asm volatile("" : "+v"(u0), "+v"(u1));
            const uint32_t uu[2] = {u0, u1};
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = fmaf(float((uu[i >> 2] >> (8 * (i & 3))) & 0xffu), sc, off);
            b[ks] = to_bf16(v);
        }
        loadB(set, min(s + 2, nk - 1));
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int kg = 2 * ks + (lane >> 5), lx = (lane & 31) ^ kg;
#pragma unroll
            for (int i = 0; i < FI; i++)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(As[set][kg][lx + 32 * i], b[ks], acc[i], 0, 0, 0);
        }
        storeA(nset, nset);
        loadA(nset, min(s + 3, nk - 1));
        lds_barrier();
    };
    loadA(0, 0);
    loadB(0, 0);
    loadA(1, min(1, nk - 1));
    loadB(1, min(1, nk - 1));
    storeA(0, 0);
    loadA(0, min(2, nk - 1));
    lds_barrier();
    int s = 0;
    for (; s + 1 < nk; s += 2) {
        step(s, std::integral_constant<int, 0>());
        step(s + 1, std::integral_constant<int, 1>());
    }
    if (s < nk) step(s, std::integral_constant<int, 0>());

    // epilogue: lane l holds column l % 32 of the fragment (gate/up: gate
    // column l % 16 in lanes l % 32 < 16, up in the others)
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (GATEUP) {
                const float g = acc[i][r], u = __shfl_xor(g, 16, 64);
                if (row < mcnt && !(lane & 16))
                    static_cast<__bf16 *>(out)[size_t(base + m0 + row) * rows + n0 + 16 * wv + (lane & 15)] =
                        __bf16(swiglu(g, u));
            } else if (row < mcnt) {
                static_cast<float *>(out)[size_t(prow[row]) * rows + n0 + 32 * wv + (lane & 31)] = acc[i][r];
            }
        }
}

// mfma_proj_kernel's grid, plan and outputs on kQ8Frag experts: table[3 e] =
// the expert's gate/up fragments, table[3 e + 2] its down fragments. Held to
// 128 registers (four waves per SIMD): two workgroups share a CU, one
// multiplying while the other waits at its barrier.
template <bool GATEUP>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) mfma_frag_kernel(const int32_t *__restrict__ tiles,
                                                             const int32_t *__restrict__ counts,
                                                             const int32_t *__restrict__ offs,
                                                             const int32_t *__restrict__ perm,
                                                             const void *const *__restrict__ table,
                                                             const __bf16 *__restrict__ src, int K, int rows, int k,
                                                             void *__restrict__ out) {
    constexpr int NCOL = GATEUP ? kBRows / 2 : kBRows;
    __shared__ bf16x8 As[2][kChunks][kBM];
    __shared__ int prow[kBM];
    const int nct = rows / NCOL, xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
    const int32_t *run = tiles + (GATEUP ? kPlanRunsGU : kPlanRunsDN);
    const int L = run[xcd] + slot;
    if (L >= run[xcd + 1]) return;
    const int t = L / nct, n0 = (L % nct) * NCOL;
    const int code = tiles[kPlanHead + 2 * t], m0 = tiles[kPlanHead + 2 * t + 1];
    const int e = code & 0xffff, bmt = code >> 16;
    const int base = offs[e], mcnt = min(bmt, counts[e] - m0);
    gbyte *F = gmem(table[3 * e + (GATEUP ? 0 : 2)]);
    if (!F) {
        // an unregistered expert contributes nothing (src/gguf_run.c:201)
        if (GATEUP)
            for (int i = threadIdx.x; i < mcnt * NCOL; i += kThreads)
                static_cast<__bf16 *>(out)[size_t(base + m0 + i / NCOL) * rows + n0 + i % NCOL] = __bf16(0.0f);
        return;
    }
    if (bmt == 32)
        frag_tile<GATEUP, 32>(As, prow, F, perm, src, K, rows, k, out, base, m0, mcnt, n0);
    else if (bmt == 64)
        frag_tile<GATEUP, 64>(As, prow, F, perm, src, K, rows, k, out, base, m0, mcnt, n0);
    else
        frag_tile<GATEUP, 128>(As, prow, F, perm, src, K, rows, k, out, base, m0, mcnt, n0);
}

// bf16 copy of n4 x 4 fp32 values (both 16-byte aligned) by workgroup blk of nblk
VH_DEV void bf16_copy(const float4 *__restrict__ x, uint2 *__restrict__ y, int64_t n4, int blk, int nblk) {
    for (int64_t i = blk * int64_t(256) + threadIdx.x; i < n4; i += int64_t(nblk) * 256) {
        const float4 v = x[i];
        typedef float f32x4_ __attribute__((ext_vector_type(4)));
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        const bf16x4 b = __builtin_convertvector(f32x4_{v.x, v.y, v.z, v.w}, bf16x4);
        y[i] = __builtin_bit_cast(uint2, b);
    }
}

__global__ void __launch_bounds__(256) to_bf16_kernel(const float4 *__restrict__ x, uint2 *__restrict__ y, int64_t n4) {
    bf16_copy(x, y, n4, blockIdx.x, gridDim.x);
}

// The bytes a token tile of bm rows stages per K step (the weights' wb and
// the inputs), in 64-byte units: the cost by which the XCDs' runs are cut.
__host__ __device__ constexpr int tile_step_cost(int wb, int bm) { return (wb + bm * kBK * 2) / 64; }

// A group's token tiles: n128 of 128 rows, then one of rbm (32 or 64) rows if
// rbm != 0 - the remainder in the smallest tile that holds it (above 64 rows,
// a whole tile).
struct GroupTiles {
    int n128, rbm;
    __host__ __device__ explicit GroupTiles(int cnt) {
        n128 = cnt / 128;
        int r = cnt - 128 * n128;
        if (r > 64) {
            n128++;
            r = 0;
        }
        rbm = r == 0 ? 0 : r <= 32 ? 32 : 64;
    }
    __host__ __device__ int count() const { return n128 + (rbm ? 1 : 0); }
    __host__ __device__ int rows(int i) const { return i < n128 ? 128 : rbm; }
};

// One workgroup of 256 threads (thread e = expert e, E <= 256). The plan:
//   tiles[0]               n, the number of token tiles
//   tiles[kPlanRunsGU + x]  x = 0..8: where XCD x's run of gate/up (tile,
//                           column tile) pairs starts (x = 8: the end)
//   tiles[kPlanRunsDN + x]  the same for the down launch
//   tiles[kPlanHead + 2 t]  tile t: expert | rows << 16 (32, 64 or 128), then
//                           the tile's first row within its group
// for the groups of at least min_tokens tokens (experts ascending, tiles as
// GroupTiles), and the list of the other non-empty groups in the dispatch
// kernel's `active` format (small[0 .. n), n at small[E]). The runs are cut
// at equal shares of the launch's staged bytes (tile_step_cost per pair); a
// cut that would give an XCD more pairs than the launch has slots per XCD
// falls back to equal shares of pairs.
__global__ void __launch_bounds__(256) mfma_plan_kernel(const int32_t *__restrict__ counts, int E, int min_tokens,
                                                        int nct_gu, int wb_gu, int slots_gu, int nct_dn,
                                                        int wb_dn, int slots_dn, int32_t *__restrict__ tiles,
                                                        int32_t *__restrict__ small, const float4 *__restrict__ x,
                                                        uint2 *__restrict__ y, int64_t n4) {
    if (blockIdx.x > 0) {  // the other workgroups: the bf16 copy of the inputs (to_bf16_kernel)
        bf16_copy(x, y, n4, blockIdx.x - 1, gridDim.x - 1);
        return;
    }
    __shared__ int wsum[4][2];
    __shared__ int wcost[4][2];
    __shared__ int runs[2][kXcds + 1];
    __shared__ int total[2];
    __shared__ int ntiles;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int cnt = t < E ? counts[t] : 0;
    const bool on = cnt > 0 && cnt >= min_tokens;
    const GroupTiles gt(on ? cnt : 0);
    const int nt = gt.count(), sm = (!on && cnt > 0) ? 1 : 0;
    const int ncts[2] = {nct_gu, nct_dn};
    const int wbs[2] = {wb_gu, wb_dn};
    int c[2];
#pragma unroll
    for (int l = 0; l < 2; l++)
        c[l] = ncts[l] * (gt.n128 * tile_step_cost(wbs[l], kBM) + (gt.rbm ? tile_step_cost(wbs[l], gt.rbm) : 0));
    int it = nt, is = sm;
    int ic[2] = {c[0], c[1]};
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        const int ot = __shfl_up(it, sh, 64), os = __shfl_up(is, sh, 64);
        const int o0 = __shfl_up(ic[0], sh, 64), o1 = __shfl_up(ic[1], sh, 64);
        if (lane >= sh) {
            it += ot;
            is += os;
            ic[0] += o0;
            ic[1] += o1;
        }
    }
    if (lane == 63) {
        wsum[wv][0] = it;
        wsum[wv][1] = is;
        wcost[wv][0] = ic[0];
        wcost[wv][1] = ic[1];
    }
    __syncthreads();
    int bt = 0, bs = 0;
    int bc[2] = {0, 0};
    for (int w = 0; w < wv; w++) {
        bt += wsum[w][0];
        bs += wsum[w][1];
        bc[0] += wcost[w][0];
        bc[1] += wcost[w][1];
    }
    const int ex_t = bt + it - nt, ex_s = bs + is - sm;
    for (int i = 0; i < nt; i++) {
        tiles[kPlanHead + 2 * (ex_t + i)] = t | (gt.rows(i) << 16);
        tiles[kPlanHead + 2 * (ex_t + i) + 1] = kBM * i;
    }
    if (sm) small[ex_s] = t;
    if (t == 255) {
        ntiles = ex_t + nt;
        total[0] = bc[0] + ic[0];
        total[1] = bc[1] + ic[1];
        tiles[0] = ex_t + nt;
        small[E] = ex_s + sm;
    }
    __syncthreads();
    // the cuts: XCD x's run starts at the pair holding staged byte x * total / 8
#pragma unroll
    for (int l = 0; l < 2; l++) {
        const int ex_c = bc[l] + ic[l] - c[l];
        for (int x = 1; x < kXcds; x++) {
            const int target = int(int64_t(x) * total[l] / kXcds);
            if (c[l] > 0 && ex_c <= target && target < ex_c + c[l]) {
                // the tile holding the target (a whole 128-row tile or the last), then its column
                const int off = target - ex_c, c128 = tile_step_cost(wbs[l], kBM), full = gt.n128 * ncts[l] * c128;
                const int i = off < full ? off / (ncts[l] * c128) : gt.n128;
                const int rest = off - i * ncts[l] * c128;
                runs[l][x] = (ex_t + i) * ncts[l] + min(rest / tile_step_cost(wbs[l], gt.rows(i)), ncts[l] - 1);
            }
        }
    }
    if (t == 0) {
        runs[0][0] = runs[1][0] = 0;
        runs[0][kXcds] = ntiles * nct_gu;
        runs[1][kXcds] = ntiles * nct_dn;
        if (total[0] == 0)
            for (int x = 1; x < kXcds; x++) runs[0][x] = 0;
        if (total[1] == 0)
            for (int x = 1; x < kXcds; x++) runs[1][x] = 0;
    }
    __syncthreads();
    if (t < 2) {
        const int slots = t ? slots_dn : slots_gu, live = runs[t][kXcds];
        bool ok = true;
        for (int x = 0; x < kXcds; x++) ok = ok && runs[t][x] <= runs[t][x + 1] && runs[t][x + 1] - runs[t][x] <= slots;
        const int per = (live + kXcds - 1) / kXcds;
        for (int x = 0; x <= kXcds; x++) tiles[(t ? kPlanRunsDN : kPlanRunsGU) + x] = ok ? runs[t][x] : min(x * per, live);
    }
}

// The column tiles, weight bytes per K step and workgroup slots per XCD of a
// launch: enough slots for any cut mfma_plan_kernel makes (an XCD's share of
// the staged bytes plus one pair, at the cheapest pair's cost).
struct TileCost {
    int nct, wb, slots;
};
TileCost tile_cost(uint32_t type, int K, int rows, bool gateup, int max_tiles) {
    TileCost c;
    c.nct = rows / (gateup ? kBRows / 2 : kBRows);
    c.wb = int(int64_t(kBRows) * vh_row_bytes(type, K) * kBK / K);  // a multiple of 64 for these types
    const int64_t cmax = tile_step_cost(c.wb, kBM), cmin = tile_step_cost(c.wb, 32);
    c.slots = int((int64_t(max_tiles) * c.nct * cmax / kXcds + cmax) / cmin + 1);
    return c;
}

template <bool GATEUP>
int mfma_launch(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                const int32_t *perm, const void *const *table, bool packed, const __bf16 *src, int K, int rows, int k,
                void *out, hipStream_t s) {
    if (packed && type != VT_Q8_0) return -EINVAL;
    const TileCost tc = tile_cost(type, K, rows, GATEUP, max_tiles);
    const dim3 g(unsigned(tc.slots) * kXcds);
    switch (type) {
    case VT_Q8_0:
        if (packed)
            hipLaunchKernelGGL((mfma_frag_kernel<GATEUP>), g, dim3(kThreads), 0, s, tiles, counts, offs, perm, table,
                               src, K, rows, k, out);
        else
            hipLaunchKernelGGL((mfma_proj_kernel<VT_Q8_0, GATEUP>), g, dim3(kThreads), 0, s, tiles, counts, offs,
                               perm, table, src, K, rows, k, vh_row_bytes(type, K), out);
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
    return ok(tg) && ok(td) && kq(tg, d) && kq(td, fe) && d % kBRows == 0 && fe % (kBRows / 2) == 0 &&
           d % kBK == 0 && fe % kBK == 0 && E <= 256;
}

int vh_mfma_max_tiles(int P, int E) { return P / kBM + E; }

int vh_mfma_plan_words(int P, int E) { return kPlanHead + 2 * vh_mfma_max_tiles(P, E); }

int vh_mfma_plan(const int32_t *counts, int E, int P, int min_tokens, uint32_t tg, uint32_t td, int d, int fe,
                 int32_t *tiles, int32_t *small, const float *hb, void *xb, int64_t n, hipStream_t s) {
    if (E > 256 || (hb && (n % 4 || ((reinterpret_cast<uintptr_t>(hb) | reinterpret_cast<uintptr_t>(xb)) & 15u))))
        return -EINVAL;
    const int64_t n4 = hb ? n / 4 : 0;
    const unsigned copy_blocks = unsigned(std::min<int64_t>((n4 + 255) / 256, 4096));
    const int mt = vh_mfma_max_tiles(P, E);
    const TileCost gu = tile_cost(tg, d, fe, true, mt), dn = tile_cost(td, fe, d, false, mt);
    // the plan's costs are 32-bit sums over every (tile, column tile) pair
    if (int64_t(mt) * std::max(gu.nct, dn.nct) * tile_step_cost(std::max(gu.wb, dn.wb), kBM) > INT32_MAX)
        return -E2BIG;
    hipLaunchKernelGGL(mfma_plan_kernel, dim3(1 + copy_blocks), dim3(256), 0, s, counts, E, min_tokens, gu.nct,
                       gu.wb, gu.slots, dn.nct, dn.wb, dn.slots, tiles, small,
                       reinterpret_cast<const float4 *>(hb), static_cast<uint2 *>(xb), n4);
    return vh_check(hipGetLastError());
}

int vh_to_bf16(const float *x, void *y, int64_t n, hipStream_t s) {
    if (n % 4 || (reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(y) & 15u)) return -EINVAL;
    const int64_t n4 = n / 4;
    const unsigned blocks = unsigned(std::min<int64_t>((n4 + 255) / 256, 4096));
    hipLaunchKernelGGL(to_bf16_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const float4 *>(x),
                       static_cast<uint2 *>(y), n4);
    return vh_check(hipGetLastError());
}

int vh_mfma_gateup(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                   const int32_t *perm, const void *const *table, bool packed, const void *xb, int d, int fe, int k,
                   void *hs, hipStream_t s) {
    return mfma_launch<true>(type, tiles, max_tiles, counts, offs, perm, table, packed,
                             static_cast<const __bf16 *>(xb), d, fe, k, hs, s);
}

int vh_mfma_down(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                 const int32_t *perm, const void *const *table, bool packed, const void *hs, int d, int fe,
                 float *ybuf, hipStream_t s) {
    return mfma_launch<false>(type, tiles, max_tiles, counts, offs, perm, table, packed,
                              static_cast<const __bf16 *>(hs), fe, d, 1, ybuf, s);
}

namespace {
// One workgroup per (fragment, expert), 544 threads: thread w writes word w
// of the fragment's kFragBytes (kQ8Frag layout, above) from the expert's
// GGUF rows. gateup: fragments of gate and up (rows 16 g + r % 16 of gate for
// r < 16, of up above), else of down (rows 32 g + r); nk K steps per row.
__global__ void __launch_bounds__(576) q8_frag_pack_kernel(const void *const *__restrict__ src_tab,
                                                           void *const *__restrict__ dst_tab, int gateup, int nk,
                                                           int64_t row_bytes) {
    const int e = blockIdx.y, f = blockIdx.x, g = f / nk, st = f - g * nk, w = threadIdx.x;
    uint8_t *dst = static_cast<uint8_t *>(dst_tab[3 * e + (gateup ? 0 : 2)]);
    if (!dst || w >= kFragBytes / 4) return;
    const int r = w < 512 ? (w >> 3) & 31 : w - 512;  // the fragment row this word belongs to
    const uint8_t *row = gateup ? static_cast<const uint8_t *>(src_tab[3 * e + (r < 16 ? 0 : 1)]) +
                                      int64_t(16 * g + (r & 15)) * row_bytes
                                : static_cast<const uint8_t *>(src_tab[3 * e + 2]) + int64_t(32 * g + r) * row_bytes;
    uint32_t v;
    if (w < 512) {
        // lane w / 8, bytes 4 (w % 8) .. + 3 of its 32: sub-step (w % 8) / 2, half w % 2
        const int lane = w >> 3, ks = (w & 7) >> 1, K0 = 64 * st + 16 * ks + 8 * (lane >> 5) + 4 * (w & 1);
        const uint8_t *q = row + 34 * (K0 >> 5) + 2 + (K0 & 31);  // even: two 16-bit loads
        v = uint32_t(*reinterpret_cast<const uint16_t *>(q)) | uint32_t(*reinterpret_cast<const uint16_t *>(q + 2)) << 16;
    } else {
        v = uint32_t(*reinterpret_cast<const uint16_t *>(row + 68 * st)) |
            uint32_t(*reinterpret_cast<const uint16_t *>(row + 68 * st + 34)) << 16;
    }
    *reinterpret_cast<uint32_t *>(dst + int64_t(f) * kFragBytes + 4 * w) = v;
}
}  // namespace

uint64_t vh_mfma_pack_bytes(int E, int d, int fe) {
    if (E < 1 || d < kBRows || fe < kBK || d % kBRows || fe % (kBRows / 2) || d % kBK || fe % kBK) return 0;
    const uint64_t gb = uint64_t(fe) * vh_row_bytes(VT_Q8_0, d), db = uint64_t(d) * vh_row_bytes(VT_Q8_0, fe);
    return (2 * gb + db) * E;
}

int vh_mfma_pack_q8(const void *const *table, int E, int d, int fe, void *buf, void **tab_out, hipStream_t s) {
    *tab_out = nullptr;
    if (!buf || !vh_mfma_pack_bytes(E, d, fe)) return -EINVAL;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (int rc = vh_check(hipStreamIsCapturing(s, &cap))) return rc;
    if (cap != hipStreamCaptureStatusNone) return -EBUSY;  // no allocation under capture
    const int64_t rg = vh_row_bytes(VT_Q8_0, d), rd = vh_row_bytes(VT_Q8_0, fe);
    const size_t gb = size_t(fe) * rg, db = size_t(d) * rd, per = 2 * gb + db;
    std::vector<const void *> src(size_t(3) * E), dst(size_t(3) * E, nullptr);
    if (int rc = vh_check(hipMemcpyAsync(src.data(), table, src.size() * sizeof(void *), hipMemcpyDeviceToHost, s)))
        return rc;
    if (int rc = vh_check(hipStreamSynchronize(s))) return rc;
    void *tab = nullptr;
    if (hipMalloc(&tab, src.size() * sizeof(void *)) != hipSuccess) return -ENOMEM;
    char *b = static_cast<char *>(buf);
    for (int e = 0; e < E; e++) {
        if (!src[3 * e] || !src[3 * e + 1] || !src[3 * e + 2]) continue;  // unregistered: stays NULL
        dst[3 * e] = dst[3 * e + 1] = b + per * e;  // gate/up fragments
        dst[3 * e + 2] = b + per * e + 2 * gb;       // down fragments
    }
    int rc = vh_check(hipMemcpy(tab, dst.data(), dst.size() * sizeof(void *), hipMemcpyHostToDevice));
    if (!rc) {
        void *const *dt = static_cast<void *const *>(tab);
        const dim3 gg(fe / 16 * (d / kBK), E), gd(d / 32 * (fe / kBK), E);
        hipLaunchKernelGGL(q8_frag_pack_kernel, gg, dim3(576), 0, s, table, dt, 1, d / kBK, rg);
        hipLaunchKernelGGL(q8_frag_pack_kernel, gd, dim3(576), 0, s, table, dt, 0, fe / kBK, rd);
        rc = vh_check(hipGetLastError());
    }
    if (rc) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(tab);
        return rc;
    }
    *tab_out = tab;
    return 0;
}
