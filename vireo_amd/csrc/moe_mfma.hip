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
// Tiles: a workgroup (512 threads) owns kBM = 128 rows of one group (a token
// tile) and kBRows = 256 weight rows (gate/up: 128 rows of gate and the same
// 128 rows of up; down: 256 rows), and steps over K in kBK = 64 columns. Each
// step stages both operands in LDS as 16-byte chunks of 8 consecutive K
// values laid out [K/8][row] (row index XOR-swizzled by the chunk), so a
// 32-lane group's operand read is one contiguous 512-byte run. Four waves
// multiply and four stage (see mfma_proj_kernel).
//
// Order: the workgroups are numbered so that each XCD (hardware dispatch sends
// workgroup b to XCD b mod 8) takes a contiguous run of (token tile, column
// tile) pairs, column tiles fastest: the workgroups sharing a token tile, and
// the consecutive token tiles of one expert that share its weight tiles, meet
// in the same L2.
//
// Outputs: gate/up writes h as bf16 rows in dispatch order (hs[offs[e] + i]),
// so the down GEMM reads its A operand contiguously; down writes the fp32 row
// y[pair] that the combine kernel reads, as on the fp32 plan.
#include <hip/hip_runtime.h>
#include <vector>
#include <algorithm>
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

// Q8_0 rows copied once into row octets for these GEMMs (kQ8Oct): tile (row
// octet o, K step s) at (o * ns + s) * 544 holds rows 8 o .. 8 o + 7's bytes
// 68 s .. 68 s + 67 (the step's two blocks) one after the other, so each
// staging load instruction - eight consecutive rows' chunks of one step -
// reads 544 consecutive bytes instead of eight 68-byte pieces 2176 bytes
// apart. A tile column of 8 rows takes ns * 544 = 8 * row_bytes bytes, as
// the rows do: the per-q base pointers are the same. Values as Chunk<VT_Q8_0>.
constexpr int kQ8Oct = 0x100 | VT_Q8_0;
template <>
struct Chunk<kQ8Oct> {
    using Pos = Chunk<VT_Q8_0>::Pos;
    using Raw = Chunk<VT_Q8_0>::Raw;
    static VH_DEV void setup_row(Pos &p, uint32_t row, uint32_t row_bytes, int kc) {
        p.ob = (row >> 3) * 8u * row_bytes + (row & 7u) * 68u + 34u * uint32_t(kc >> 2);
        p.oq = p.ob + 2u + 8u * uint32_t(kc & 3);
    }
    static VH_DEV void load(const Pos &p, Raw &r, gbyte *m, int s) {
        gbyte *ms = m + 544 * s;
        r.d = ld_u16(ms + p.ob);
        r.q = ld_u64(ms + p.oq);
    }
    static VH_DEV void values(const Pos &p, const Raw &r, int s, float (&v)[8]) {
        Chunk<VT_Q8_0>::values(p, r, s, v);
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

// 1-D grid of at least (column tiles) x (tile-plan capacity) workgroups, a
// multiple of kXcds; 512 threads. Tile t of the plan is (expert e, first row
// m0 of its group). A is bf16: GATEUP: xb [T x K], row perm[i] / k; else hs
// [P x K], row i. GATEUP: B = gate and up rows, out = hs (bf16 [P x rows],
// row i); else B = down rows, out = y (fp32 [P x rows], row perm[i]). i runs
// over offs[e] + m0 .. + kBM - 1 within the group.
//
// Waves 0-3 only multiply: wave c owns rows 64 (c / 2) .. + 63 of the tile
// and 128 of its weight rows (gate/up: 64 columns of gate and the same 64 of
// up), eight 32 x 32 accumulator fragments. Waves 4-7 only stage: their global loads run
// two K steps ahead in two register sets, and each step they dequantize the
// set that arrived a step ago into the LDS buffer the multiplying waves will
// read next. Every SIMD holds one wave of each kind, so the matrix cores and
// the vector ALUs work at the same time; one barrier per K step.
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
    // XCD-contiguous numbering of the live (token tile, column tile) pairs
    const int nct = rows / NCOL, live = tiles[0] * nct, per = (live + kXcds - 1) / kXcds;
    const int slot = blockIdx.x / kXcds, L = (blockIdx.x % kXcds) * per + slot;
    if (slot >= per || L >= live) return;
    const int t = L / nct, n0 = (L % nct) * NCOL;
    const int e = tiles[1 + 2 * t], m0 = tiles[2 + 2 * t];
    const int base = offs[e], mcnt = min(kBM, counts[e] - m0);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool mult = wv < 4;

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
    const int nk = K / kBK;

    if (!mult) {
        // ---- staging waves: thread p stages K chunk kc = p & 7 of A rows
        // (p >> 3) + 32 q (q < 4; rows past the group repeat its last row,
        // whose results are not stored) and of B rows (p >> 3) + 32 q (q < 8).
        // In LDS, chunk kc of row r sits at [kc][r ^ kc]: the 8 lanes of a row
        // write 8 different bank groups, and a 32-lane operand read stays
        // conflict-free. The K step enters the global addresses only through
        // uniform base pointers.
        const int p = tid - 256, kc = p & 7, rx = (p >> 3) ^ kc;
        gbyte *abase = gmem(src);
        uint32_t aoff[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int i = base + m0 + min((p >> 3) + 32 * q, mcnt - 1);
            aoff[q] = uint32_t((GATEUP ? size_t(perm[i] / k) : size_t(i)) * K * 2) + 16u * uint32_t(kc);
        }
        // B rows (p >> 3) + 32 q lie 32 q rows (gate/up: 32 (q % 4) rows of
        // gate or up) past row p >> 3: one set of offsets, and per q a uniform
        // base pointer (32 rows are a multiple of 4 bytes, so alignments agree)
        using C = Chunk<T>;
        constexpr int kSets = sets<T>();
        typename C::Pos bp;
        if constexpr (T == kQ8Oct)
            C::setup_row(bp, uint32_t(n0 + (p >> 3)), uint32_t(row_bytes), kc);
        else
            C::setup(bp, uint32_t(n0 + (p >> 3)) * uint32_t(row_bytes), kc);
        gbyte *bm[8];
#pragma unroll
        for (int q = 0; q < 8; q++) bm[q] = (GATEUP && q >= 4 ? M1 : M0) + (GATEUP ? q & 3 : q) * 32 * row_bytes;

        struct Stage {
            uint4 ah[4];
            typename C::Raw bw[8];
        } st[kSets];
        auto load = [&](Stage &g, int step) {
            gbyte *as = abase + 128 * step;
#pragma unroll
            for (int q = 0; q < 4; q++) g.ah[q] = ld_u128(as + aoff[q]);
#pragma unroll
            for (int q = 0; q < 8; q++) C::load(bp, g.bw[q], bm[q], step);
        };
        auto store = [&](const Stage &g, int buf, int step) {
#pragma unroll
            for (int q = 0; q < 4; q++) As[buf][kc][rx + 32 * q] = __builtin_bit_cast(bf16x8, g.ah[q]);
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
        for (int j = 0; j < kSets; j++)
            if (j < nk) load(st[j], j);
        store(st[0], 0, 0);
        __syncthreads();
        for (int s0 = 0; s0 < nk; s0 += kSets) {
#pragma unroll
            for (int j = 0; j < kSets; j++) {
                // step s: the multiplying waves read buffer s & 1
                const int s = s0 + j;
                if (s >= nk) break;
                if (s + kSets < nk) load(st[j], s + kSets);
                if (s + 1 < nk) store(st[(j + 1) % kSets], (s + 1) & 1, s + 1);
                __syncthreads();
            }
        }
        return;
    }

    // ---- multiplying waves: v_mfma_f32_32x32x16_bf16 (lane l supplies row
    // l % 32, K values 8 (l / 32) .. + 7 of each operand; it holds column
    // l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 of the 32 x 32 result)
    const int wm = wv >> 1, wn = wv & 1;
    // B rows of the wave's four 32-column fragments (gate/up: two of gate,
    // the same two of up)
    int bfr[4];
#pragma unroll
    for (int j = 0; j < 4; j++) bfr[j] = GATEUP ? (j < 2 ? 0 : NCOL) + 64 * wn + 32 * (j & 1) : 128 * wn + 32 * j;
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    __syncthreads();  // buffer 0 staged
    for (int s = 0; s < nk; s++) {
        const int buf = s & 1;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int kg = 2 * ks + (lane >> 5), lx = (lane & 31) ^ kg;
            bf16x8 a[2], b[4];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = As[buf][kg][lx + 64 * wm + 32 * i];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = Bs[buf][kg][lx + bfr[j]];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row >= mcnt) continue;
            const int pos = base + m0 + row;
            if (GATEUP) {
                __bf16 *hs = static_cast<__bf16 *>(out) + size_t(pos) * rows;
#pragma unroll
                for (int jj = 0; jj < 2; jj++)
                    hs[n0 + 64 * wn + 32 * jj + (lane & 31)] = __bf16(swiglu(acc[i][jj][r], acc[i][2 + jj][r]));
            } else {
                float *y = static_cast<float *>(out) + size_t(perm[pos]) * rows;
#pragma unroll
                for (int j = 0; j < 4; j++) y[n0 + 128 * wn + 32 * j + (lane & 31)] = acc[i][j][r];
            }
        }
}

// bf16 copy of n fp32 values (n a multiple of 4, both 16-byte aligned)
__global__ void __launch_bounds__(256) to_bf16_kernel(const float4 *__restrict__ x, uint2 *__restrict__ y, int64_t n4) {
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n4; i += int64_t(gridDim.x) * 256) {
        const float4 v = x[i];
        typedef float f32x4_ __attribute__((ext_vector_type(4)));
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        const bf16x4 b = __builtin_convertvector(f32x4_{v.x, v.y, v.z, v.w}, bf16x4);
        y[i] = __builtin_bit_cast(uint2, b);
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
                const int32_t *perm, const void *const *table, bool packed, const __bf16 *src, int K, int rows, int k,
                void *out, hipStream_t s) {
    if (packed && type != VT_Q8_0) return -EINVAL;
    const int64_t nwg = int64_t(rows / (GATEUP ? kBRows / 2 : kBRows)) * max_tiles;
    const dim3 g(unsigned((nwg + kXcds - 1) / kXcds * kXcds));
    switch (type) {
    case VT_Q8_0:
        if (packed)
            hipLaunchKernelGGL((mfma_proj_kernel<kQ8Oct, GATEUP>), g, dim3(kThreads), 0, s, tiles, counts, offs,
                               perm, table, src, K, rows, k, vh_row_bytes(type, K), out);
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

int vh_mfma_plan(const int32_t *counts, int E, int min_tokens, int32_t *tiles, int32_t *small, hipStream_t s) {
    if (E > 256) return -EINVAL;
    hipLaunchKernelGGL(mfma_plan_kernel, dim3(1), dim3(256), 0, s, counts, E, min_tokens, tiles, small);
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
// One workgroup per (tile, expert) of matrix `which`: 272 threads copy two
// bytes each of the tile's 544 (row rr = t / 34 of the octet).
__global__ void __launch_bounds__(320) q8_octet_pack_kernel(const void *const *__restrict__ src_tab,
                                                            void *const *__restrict__ dst_tab, int which, int ns,
                                                            int64_t row_bytes) {
    const int e = blockIdx.y, tile = blockIdx.x, o = tile / ns, st = tile - o * ns, t = threadIdx.x;
    const uint8_t *src = static_cast<const uint8_t *>(src_tab[3 * e + which]);
    uint8_t *dst = static_cast<uint8_t *>(dst_tab[3 * e + which]);
    if (!src || !dst || t >= 272) return;
    const int rr = t / 34, b = 2 * (t - 34 * rr);
    *reinterpret_cast<uint16_t *>(dst + int64_t(tile) * 544 + 68 * rr + b) =
        *reinterpret_cast<const uint16_t *>(src + int64_t(8 * o + rr) * row_bytes + 68 * st + b);
}
}  // namespace

int vh_mfma_pack_q8(const void *const *table, int E, int d, int fe, void **buf_out, void **tab_out, hipStream_t s) {
    *buf_out = *tab_out = nullptr;
    if (E < 1 || d % kBK || fe % kBK || d % 8 || fe % 8) return -EINVAL;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (int rc = vh_check(hipStreamIsCapturing(s, &cap))) return rc;
    if (cap != hipStreamCaptureStatusNone) return -EBUSY;  // no allocation under capture
    const int64_t rg = vh_row_bytes(VT_Q8_0, d), rd = vh_row_bytes(VT_Q8_0, fe);
    const size_t gb = size_t(fe) * rg, db = size_t(d) * rd, per = 2 * gb + db;
    std::vector<const void *> src(size_t(3) * E), dst(size_t(3) * E, nullptr);
    if (int rc = vh_check(hipMemcpyAsync(src.data(), table, src.size() * sizeof(void *), hipMemcpyDeviceToHost, s)))
        return rc;
    if (int rc = vh_check(hipStreamSynchronize(s))) return rc;
    void *buf = nullptr, *tab = nullptr;
    if (hipMalloc(&buf, per * E) != hipSuccess) return -ENOMEM;
    if (hipMalloc(&tab, src.size() * sizeof(void *)) != hipSuccess) {
        (void)hipFree(buf);
        return -ENOMEM;
    }
    char *b = static_cast<char *>(buf);
    for (int e = 0; e < E; e++) {
        if (!src[3 * e] || !src[3 * e + 1] || !src[3 * e + 2]) continue;  // unregistered: stays NULL
        dst[3 * e] = b + per * e;
        dst[3 * e + 1] = b + per * e + gb;
        dst[3 * e + 2] = b + per * e + 2 * gb;
    }
    int rc = vh_check(hipMemcpy(tab, dst.data(), dst.size() * sizeof(void *), hipMemcpyHostToDevice));
    if (!rc) {
        void *const *dt = static_cast<void *const *>(tab);
        const dim3 gg(fe / 8 * (d / kBK), E), gd(d / 8 * (fe / kBK), E);
        hipLaunchKernelGGL(q8_octet_pack_kernel, gg, dim3(320), 0, s, table, dt, 0, d / kBK, rg);
        hipLaunchKernelGGL(q8_octet_pack_kernel, gg, dim3(320), 0, s, table, dt, 1, d / kBK, rg);
        hipLaunchKernelGGL(q8_octet_pack_kernel, gd, dim3(320), 0, s, table, dt, 2, fe / kBK, rd);
        rc = vh_check(hipGetLastError());
    }
    if (rc) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(tab);
        (void)hipFree(buf);
        return rc;
    }
    *buf_out = buf;
    *tab_out = tab;
    return 0;
}
