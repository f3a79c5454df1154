// Decode-batch grouped projections on the matrix cores, for calls of fewer
// than kMfmaMinCall tokens whose experts are Q4_K (gate, up) and Q6_K (down),
// the Q4_K_M layout. Such a call sends a few tokens to each expert (32 tokens,
// top-8 of 128 experts: about two), and the fp32 decode-batch kernels
// (moe_gdec.hip) convert every weight to fp32 again for each of them: they are
// bound by the vector ALUs, not by HBM. Here a weight is converted once into a
// 16-bit matrix operand and up to 16 tokens of its expert are multiplied
// against it in one instruction.
//
// The operands hold the reference's values exactly - split where one 16-bit
// value cannot hold them - and products are summed in fp32 (the weights of
// src/gguf_compute.c:52-66 and :83-103, the sums of the matvec of :202-207):
//  - gate/up, v_mfma_f32_16x16x32_f16. A Q4_K weight of sub-block s is
//    d*sc_s*q - dmin*m_s. The weight operand holds sc_s*q (an integer below
//    1024, exact in fp16, formed by a packed fp16 fma that rounds once); per
//    super-block the matrix cores form C = sum sc*q*x, and M = sum_s m_s X_s
//    from the sub-blocks' input sums X_s (one instruction per super-block);
//    the row adds d*C - dmin*M in fp32. The inputs, scaled by a power of two
//    per token that keeps them below 2^14 in magnitude (no fp16 overflow),
//    are split into fp16 parts hi + lo (22 significant bits) by
//    mdec_prep_kernel, in the order the weight operand's slots take; it also
//    writes X_s / 32 (below 2^14) as fp16 hi + lo.
//  - down, v_mfma_f32_16x16x32_bf16. A Q6_K weight of sub-block s (16
//    weights) is d*sc_s*(q - 32). The operand holds q + 128 (exact in bf16)
//    and a second product with the constant -160 completes q - 32; each
//    sub-block's sum is scaled by d*sc_s in fp32. The activations h are split
//    into bf16 parts hi + lo (16 significant bits, fp32's range, no scale) by
//    the gate/up kernel as it writes them, in the order the down operand's
//    slots take; one instruction's 32 k slots take a sub-block's 16 hi parts
//    and its 16 lo parts against the weights repeated.
// Products of 16-bit parts are exact in fp32, so the results differ from the
// fp32 kernels' only by the order of the fp32 sums and the dropped low bits of
// the split inputs (relative 2^-22 and 2^-17 of the largest input).
//
// Matrix operands (both instructions): A is tokens x K - lane l supplies
// token l % 16 -, B is K x weight rows - lane l supplies row l % 16 -, and the
// lanes l / 16 = g supply the same K positions of A and B (8 per lane); lane
// l receives rows 4 g .. 4 g + 3 (tokens) of
// column l % 16 (weight row) of the result. Which K position a slot holds is
// free as long as A and B agree: it is fixed by how a weight word is unpacked,
// and the inputs are laid out to match.
//
// Grids: (row chunk, active expert slot, 16-token tile); gate/up: 256
// threads, waves of 16 rows of gate and the same 16 of up; down: 4 or 8
// waves of 16 rows. A call of moe_ffn_forward (MdecSelf) launches no
// dispatch and no combine kernel: the grids' second dimension is the expert
// id, each workgroup lists its expert's pairs from the routing itself
// (expert_group: one load of idx and two barriers, where a dispatch kernel
// cost about 7 us), and the down kernel's workgroups combine: the last of a
// token's k experts to write a workgroup's chunk of y adds the chunk's k rows
// into x (agent-scope stores, counters and loads). Qwen3 Q4_K_M, 32 tokens:
// 113.3 -> 110.3 us per layer; OLMoE Q4_K_M 16 tokens: 85.5 -> 79.0. Q6_K rows (210 bytes per super-block) start at
// any even address; their 16-byte loads rely on global memory accepting any
// alignment.
#include <hip/hip_runtime.h>
#include <vector>
#include "common.h"
#include "qdecode.h"
#include "route.h"
#include "route_kernels.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTok = 16;  // tokens per tile (the A operand's rows)
constexpr int kDnTok = 8;  // tokens per down tile: its LDS holds their activations, and few experts of a
                           // decode call serve more (the MFMA rows past them are idle either way)
constexpr int kGroupMax = 64;     // a call's tokens per expert (at most one pair per token; calls < 64 tokens)

// The pairs p < P routed to expert e (idx[p] == e) in ascending order into
// list (at most kGroupMax kept); returns their number. Called by every thread
// of a workgroup of NT threads; the first two rounds' loads are issued
// together, and the function ends with a barrier.
template <int NT>
VH_DEV int expert_group(const int32_t *__restrict__ idx, int P, int e, int *list, int *wc) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int v0 = tid < P ? idx[tid] : -1, v1 = tid + NT < P ? idx[tid + NT] : -1;
    int base = 0;
    for (int p0 = 0; p0 < P; p0 += NT) {
        const int p = p0 + tid;
        const int v = p0 == 0 ? v0 : p0 == NT ? v1 : (p < P ? idx[p] : -1);
        const bool hit = v == e;
        const uint64_t m = __ballot(hit);
        if (lane == 0) wc[wv] = __popcll(m);
        __syncthreads();
        int before = base, tot = base;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const int c = wc[w];
            before += w < wv ? c : 0;
            tot += c;
        }
        const int at = before + __popcll(m & ((1ull << lane) - 1ull));
        if (hit && at < kGroupMax) list[at] = p;
        base = tot;
        __syncthreads();  // wc is written again by the next round
    }
    return min(base, kGroupMax);
}

VH_DEV f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
VH_DEV uint32_t u4_at(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// ---- gate/up operand layout ---------------------------------------------------
// Super-block b (256 weights), step u (0..7), lane group g: the qs word 8 g + u
// (bytes 32 g + 4 u .. + 3 of the 128 qs bytes: weights 4 u .. 4 u + 3 of
// sub-blocks 2 g (low nibbles) and 2 g + 1 (high nibbles)). Slot j of the
// operand holds weight 32 (2 g + j / 4) + 4 u + {0, 2, 1, 3}[j % 4] of the
// super-block. The inputs of one token: 16 fp16 values per (b, u, g) - the 8
// hi parts, then the 8 lo parts - at ((b * 8 + u) * 4 + g) * 16.
VH_DEV int q4k_slot_of(int r, int &chunk) {  // r = position in the super-block
    const int g = r >> 6, hsub = (r >> 5) & 1, e = r & 31, u = e >> 2, p = e & 3;
    chunk = u * 4 + g;
    return 4 * hsub + (p == 1 ? 2 : p == 2 ? 1 : p);
}

// (a & m) | e with all three in vector registers: the compiler's own form
// takes at most one constant from outside them and splits the operation in two
VH_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t e) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(e));
    return r;
}

// sc*q for the 8 nibbles of qs word w: each nibble becomes the mantissa bits
// of an fp16 with exponent 2^10 in place - bits 0-3 give 1024 + q, bits 4-7
// give 1024 + 16 q - and one packed fp16 fma per pair, (1024 + q) sc - 1024 sc
// or (1024 + 16 q) (sc / 16) - 64 sc, forms the product exactly (an integer
// below 1024; sc / 16 and 64 sc have at most 6 significant bits). kLo =
// 0x000f000f, kHi = 0x00f000f0 and kE = 0x64006400 come in registers.
VH_DEV f16x8 q4k_operand(uint32_t w, f16x2 s0, f16x2 n0, f16x2 s1, f16x2 n1, uint32_t kLo, uint32_t kHi,
                         uint32_t kE) {
    const uint32_t w8 = w >> 8;
    const f16x2 a = __builtin_elementwise_fma(as_h2(and_or(w, kLo, kE)), s0, n0);
    const f16x2 b = __builtin_elementwise_fma(as_h2(and_or(w8, kLo, kE)), s0, n0);
    const f16x2 c = __builtin_elementwise_fma(as_h2(and_or(w, kHi, kE)), s1, n1);
    const f16x2 e = __builtin_elementwise_fma(as_h2(and_or(w8, kHi, kE)), s1, n1);
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], e[0], e[1]};
}

// The 6-bit scale and min of sub-block j (0..7, a per-lane value) from the 12
// packed bytes s0..s2 (src/gguf_compute.c:45-51), without branches.
VH_DEV void q4k_scale_min_v(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
    const uint32_t bj = uint32_t(((uint64_t(s1) << 32) | s0) >> (8 * j)) & 0xffu;             // byte j
    const uint32_t bj4 = (j < 4 ? s1 >> (8 * j) : s2 >> (8 * (j - 4))) & 0xffu;            // byte j + 4
    const uint32_t bjm4 = (s0 >> (8 * (j & 3))) & 0xffu;                                   // byte j - 4 (j >= 4)
    const int lo_sc = int(bj & 63u), lo_mn = int(bj4 & 63u);
    const int hi_sc = int((bj4 & 15u) | ((bjm4 >> 6) << 4)), hi_mn = int((bj4 >> 4) | ((bj >> 6) << 4));
    sc = j < 4 ? lo_sc : hi_sc;
    mn = j < 4 ? lo_mn : hi_mn;
}

// ---- down operand layout -------------------------------------------------------
// Q6_K sub-block s = 8 h + 2 j + lh of super-block b holds weights
// 128 h + 32 j + 16 lh + (0..15) (src/gguf_compute.c:83-103); lane group g
// takes weights 16 s + 4 g + {0, 2, 1, 3} (slot order). Activation k of a pair
// is slot {0, 2, 1, 3}^-1 (k % 4) of chunk k / 4: 8 bf16 values per chunk,
// the 4 hi parts then the 4 lo parts.
VH_DEV int q6k_slot_of(int k) {
    const int p = k & 3;
    return p == 1 ? 2 : p == 2 ? 1 : p;
}

// One workgroup of 256 threads per token: the largest |x|, the power of two,
// the fp16 split of every input into the gate/up operand order, and the sums
// X_s of the scaled inputs over each 32-input sub-block, X_s / 32 split into
// fp16 hi + lo at xsum + ((t * nb + b) * 4 + g) * 4: hi, lo of sub-block 2 g,
// then of 2 g + 1 (the slots lane group g supplies to the min term).
__global__ void __launch_bounds__(256) mdec_prep_kernel(const float *__restrict__ hb, int d,
                                                        _Float16 *__restrict__ xp, float *__restrict__ xsc,
                                                        _Float16 *__restrict__ xsum) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x, nb = d / 256;
    const float *x = hb + size_t(t) * d;
    float m = 0.0f;
    for (int i = tid; i < d; i += 256) m = fmaxf(m, fabsf(x[i]));
    m = wave_max_f(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (m > 0.0f && m <= 3.4028234663852886e38f) frexpf(m, &ex);  // m < 2^ex
    const int sh = max(-120, min(120, 14 - ex));                  // |x 2^sh| < 2^14
    const float up = ldexpf(1.0f, sh);
    if (tid == 0) xsc[t] = ldexpf(1.0f, -sh);
    _Float16 *o = xp + size_t(t) * d * 2;
    int chunk;
    const int j = q4k_slot_of(tid, chunk);
    for (int b = 0; b < nb; b++) {  // d % 256 == 0: every thread takes every step
        const float v = x[256 * b + tid] * up;
        const _Float16 hi = _Float16(v);
        const _Float16 lo = _Float16(v - float(hi));  // v - hi is exact in fp32
        const size_t c = (size_t(b) * 32 + chunk) * 16;
        o[c + j] = hi;
        o[c + 8 + j] = lo;
        float sv = v;  // sub-block tid / 32: lanes 32 s .. 32 s + 31 of the workgroup
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) sv += __shfl_xor(sv, off, 32);
        if ((tid & 31) == 0) {
            const int sb = tid >> 5;
            const float q = sv * 0.03125f;  // |X_s| < 2^19
            const _Float16 qh = _Float16(q);
            _Float16 *xs = xsum + ((size_t(t) * nb + b) * 4 + (sb >> 1)) * 4 + 2 * (sb & 1);
            xs[0] = qh;
            xs[1] = _Float16(q - float(qh));
        }
    }
}

// Router parts of T >= 2 tokens, d = 2048, by tiles of 4 experts x 4 tokens:
// the arithmetic of route_row_part<32> per (expert, token) - lane l's 32
// products, their fp64 sum and the bound on the reference's rounding - so
// the same parts as one wave per pair, with the tokens' inputs read once per
// tile (through LDS) instead of once per expert, and each wave's router row
// read once for its 4 tokens. Wave w copies token t0 + w and takes expert
// e0 + w. With xp given, the workgroups of experts 0..3 also write
// mdec_prep_kernel's outputs for their tokens (lane l's 32 inputs are
// sub-block l % 8 of super-block l / 8; its sum is taken in order in the lane).
constexpr int kRpTile = 4, kRpLaneF = 36;  // 32 inputs per lane in LDS, plus 4 floats (no bank conflicts)

__global__ void __launch_bounds__(256) mdec_route_prep_kernel(const float *__restrict__ R, const float *__restrict__ hb,
                                                              const float *__restrict__ bias, int E, int T,
                                                              RoutePart *__restrict__ parts, _Float16 *__restrict__ xp,
                                                              float *__restrict__ xsc, _Float16 *__restrict__ xsum) {
    constexpr int d = 2048, C = 32, nb = d / 256;
    __shared__ __align__(16) float xs[kRpTile][64 * kRpLaneF];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int e = blockIdx.x * kRpTile + w, t0 = blockIdx.y * kRpTile;
    float rv[C], xv[C];
    const float4 *x4 = reinterpret_cast<const float4 *>(hb + size_t(min(t0 + w, T - 1)) * d + lane * C);
#pragma unroll
    for (int i = 0; i < C / 4; i++) {
        const float4 v = x4[i];
        xv[4 * i] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
    }
    const float4 *r4 = reinterpret_cast<const float4 *>(R + size_t(min(e, E - 1)) * d + lane * C);
#pragma unroll
    for (int i = 0; i < C / 4; i++) {
        const float4 v = r4[i];
        rv[4 * i] = v.x;
        rv[4 * i + 1] = v.y;
        rv[4 * i + 2] = v.z;
        rv[4 * i + 3] = v.w;
    }
    float4 *dst = reinterpret_cast<float4 *>(&xs[w][lane * kRpLaneF]);
#pragma unroll
    for (int i = 0; i < C / 4; i++) dst[i] = make_float4(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2], xv[4 * i + 3]);
    const int t = t0 + w;
    if (xp && blockIdx.x == 0 && t < T) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < C; i++) m = fmaxf(m, fabsf(xv[i]));
        m = wave_max_f(m);
        int ex = 0;
        if (m > 0.0f && m <= 3.4028234663852886e38f) frexpf(m, &ex);  // m < 2^ex
        const int sh = max(-120, min(120, 14 - ex));                  // |x 2^sh| < 2^14
        const float up = ldexpf(1.0f, sh);
        if (lane == 0) xsc[t] = ldexpf(1.0f, -sh);
        const int b = lane >> 3, g = (lane & 7) >> 1, hs = lane & 1;
        _Float16 *o = xp + size_t(t) * d * 2;
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float v = xv[4 * u + q] * up;
                hi[q] = _Float16(v);
                lo[q] = _Float16(v - float(hi[q]));  // exact in fp32
                sum += v;
            }
            // slots 4 hs .. 4 hs + 3 of chunk (b, u, g) hold positions 0, 2, 1, 3
            typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
            f16x4 *c = reinterpret_cast<f16x4 *>(o + (size_t(b) * 32 + u * 4 + g) * 16 + 4 * hs);
            c[0] = f16x4{hi[0], hi[2], hi[1], hi[3]};
            c[2] = f16x4{lo[0], lo[2], lo[1], lo[3]};
        }
        const float q = sum * 0.03125f;  // |X_s| < 2^19
        const _Float16 qh = _Float16(q);
        _Float16 *xsp = xsum + ((size_t(t) * nb + b) * 4 + g) * 4 + 2 * hs;
        xsp[0] = qh;
        xsp[1] = _Float16(q - float(qh));
    }
    __syncthreads();
    if (e >= E) return;
    for (int j = 0; j < kRpTile && t0 + j < T; j++) {
        const float4 *src = reinterpret_cast<const float4 *>(&xs[j][lane * kRpLaneF]);
        float p[C];
#pragma unroll
        for (int i = 0; i < C / 4; i++) {
            const float4 v = src[i];
            p[4 * i] = mul_rn(rv[4 * i], v.x);
            p[4 * i + 1] = mul_rn(rv[4 * i + 1], v.y);
            p[4 * i + 2] = mul_rn(rv[4 * i + 2], v.z);
            p[4 * i + 3] = mul_rn(rv[4 * i + 3], v.w);
        }
        double tot = 0.0, absum = 0.0;
#pragma unroll
        for (int i = 0; i < C; i++) tot += double(p[i]);
        double run = wave_incl_scan_d(tot) - tot;
#pragma unroll
        for (int i = 0; i < C; i++) {
            run += double(p[i]);
            absum += fabs(run);
        }
        RoutePart out;
        out.c = wave_sum_d(tot);
        out.beta = 1.001 * 5.9604644775390625e-08 * wave_sum_d(absum) + 1e-30;
        if (bias) out.c += double(bias[e]);
        if (lane == 0) parts[size_t(t0 + j) * E + e] = out;
    }
}

// The experts of a pinned layer can be copied once into 16-row tiles, so that
// every load instruction of the gate/up and down kernels reads 1 KB of
// consecutive bytes (the GGUF rows give each instruction 16 rows' short
// pieces: half the rate from HBM). Tile (G, b) of a matrix - rows 16 G ..
// 16 G + 15, super-block b - sits at (G * nb + b) * tile bytes; its bytes are
// the rows' own, reordered so that lane l = r + 16 g of a wave loads 16
// consecutive bytes from each part:
//   Q4_K (2368 bytes): the 16 rows' d and dmin (4 bytes, row r at 4 r), then
//     lane l's four 6-bit scales and mins, decoded once - sc and m of
//     sub-blocks 2 g and 2 g + 1 of row r, one byte each - at 64 + 4 l, then
//     qs bytes 32 g .. 32 g + 15 of row r at 320 + 16 l, then qs bytes 32 g +
//     16 .. 32 g + 31 at 1344 + 16 l (64 bytes more than the rows: the
//     kernel's scale decoding is gone);
//   Q6_K (3360 bytes): the words lane l's sub-block steps read - word g of
//     each of row r's 16-byte ql chunks 0-3 at 16 l, of chunks 4-7 at 1024 +
//     16 l, of its qh chunks 0-3 at 2048 + 16 l (so no exchange through LDS)
//     - then the rows' scales (16 bytes each) at 3072 + 16 r, their d at
//     3328 + 2 r.
constexpr int kQ4Tile = 2368, kQ6Tile = 16 * 210;

// the byte of row `row`'s super-block that Q6_K tile byte o (even) holds
VH_DEV int pk_src_q6k(int o, int &row) {
    if (o < 3072) {  // word w of lane L's piece: word g of ql chunk w (w + 4), or of qh chunk w
        const int part = o >> 10, q = o & 1023, L = q >> 4, g = L >> 4, w = (q & 15) >> 2;
        row = L & 15;
        const int c = part == 1 ? w + 4 : w;
        return (part == 2 ? 128 : 0) + 16 * c + 4 * g + (q & 3);
    }
    if (o < 3328) {
        row = (o - 3072) >> 4;
        return 192 + ((o - 3072) & 15);
    }
    row = (o - 3328) >> 1;
    return 208 + ((o - 3328) & 1);
}

// One workgroup per (tile, expert) of matrix `which` (0 gate, 1 up, 2 down).
// Q6_K: two bytes per thread and step (every field is at an even offset).
__global__ void __launch_bounds__(256) mdec_pack_q6k_kernel(const void *const *__restrict__ src_tab,
                                                            void *const *__restrict__ dst_tab, int which, int nb,
                                                            int64_t row_bytes) {
    const int e = blockIdx.y, tile = blockIdx.x, G = tile / nb, b = tile - G * nb;
    const uint8_t *src = static_cast<const uint8_t *>(src_tab[3 * e + which]);
    uint8_t *dst = static_cast<uint8_t *>(dst_tab[3 * e + which]);
    if (!src || !dst) return;
    for (int o = 2 * int(threadIdx.x); o < kQ6Tile; o += 512) {
        int row;
        const int off = pk_src_q6k(o, row);
        const uint16_t v = *reinterpret_cast<const uint16_t *>(src + int64_t(16 * G + row) * row_bytes + 210 * b + off);
        *reinterpret_cast<uint16_t *>(dst + int64_t(tile) * kQ6Tile + o) = v;
    }
}
// Q4_K: threads 0-15 copy row t's d and dmin, 16-79 decode lane t - 16's
// scales and mins (q4k_scale_min_v, as the kernels did), 80-207 copy the qs
// pieces (16-byte aligned: Q4_K rows are 144 bytes per super-block).
__global__ void __launch_bounds__(256) mdec_pack_q4k_kernel(const void *const *__restrict__ src_tab,
                                                            void *const *__restrict__ dst_tab, int which, int nb,
                                                            int64_t row_bytes) {
    const int e = blockIdx.y, tile = blockIdx.x, G = tile / nb, b = tile - G * nb, t = threadIdx.x;
    const uint8_t *src = static_cast<const uint8_t *>(src_tab[3 * e + which]);
    uint8_t *dst = static_cast<uint8_t *>(dst_tab[3 * e + which]) + int64_t(tile) * kQ4Tile;
    if (!src || !dst) return;
    auto blk = [&](int row) { return src + int64_t(16 * G + row) * row_bytes + 144 * b; };
    if (t < 16) {
        *reinterpret_cast<uint32_t *>(dst + 4 * t) = *reinterpret_cast<const uint32_t *>(blk(t));
    } else if (t < 80) {
        const int l = t - 16, r = l & 15, g = l >> 4;
        const uint32_t *h = reinterpret_cast<const uint32_t *>(blk(r));
        int sc0, mn0, sc1, mn1;
        q4k_scale_min_v(2 * g, h[1], h[2], h[3], sc0, mn0);
        q4k_scale_min_v(2 * g + 1, h[1], h[2], h[3], sc1, mn1);
        *reinterpret_cast<uint32_t *>(dst + 64 + 4 * l) =
            uint32_t(sc0) | (uint32_t(sc1) << 8) | (uint32_t(mn0) << 16) | (uint32_t(mn1) << 24);
    } else if (t < 208) {
        const int P = t - 80, l = P & 63, r = l & 15, g = l >> 4, second = P >> 6;
        *reinterpret_cast<uint4 *>(dst + (second ? 1344 : 320) + 16 * l) =
            *reinterpret_cast<const uint4 *>(blk(r) + (second ? 32 : 16) + 32 * g);
    }
}

// gate/up: wave w of workgroup (c, s, z) owns rows 64 c + 16 w .. + 15 of gate
// and up of expert active[s] for tokens 16 z .. of its group, and writes
// h = silu(gate . x) * (up . x) (src/gguf_run.c:205-207) as bf16 hi + lo parts
// in the down operand's order into hp (4 bytes per activation, rows of fe).
// The tile's split inputs pass through LDS one super-block at a time, double
// buffered (every wave reads them; they are loaded once per workgroup). Each
// wave's GGUF rows are requested two super-blocks ahead of the one it
// multiplies (three register sets in turn: the loop over the NB = d / 256
// super-blocks is unrolled), so two blocks of its rows are in flight from
// HBM while it computes; from tiles (PK), whose loads stream at full rate,
// one ahead, which keeps the kernel within 128 registers (four waves per
// SIMD instead of three).
constexpr int kGuTokStride = 260;  // dwords per token and super-block in LDS: 256 + 4 (no bank conflicts)
constexpr int kGuMaxBlocks = 8;    // d <= 2048

template <int NB, bool PK, bool SELF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PK ? 4 : 3))) mdec_gateup_kernel(const int32_t *__restrict__ counts,
                                                          const int32_t *__restrict__ offs,
                                                          const int32_t *__restrict__ perm,
                                                          const int32_t *__restrict__ active,
                                                          const void *const *__restrict__ table,
                                                          const uint4 *__restrict__ xp, const float *__restrict__ xsc,
                                                          const uint2 *__restrict__ xsum, int fe, int k, int E,
                                                          int64_t row_bytes, uint16_t *__restrict__ hp, MdecSelf sf) {
    constexpr int d = 256 * NB;
    __shared__ __align__(16) uint32_t xs[2][kTok * kGuTokStride];
    __shared__ int glist[SELF ? kGroupMax : 1], gwc[SELF ? 4 : 1];
    const int t0 = blockIdx.z * kTok;
    int e, cnt, base = 0;
    if constexpr (SELF) {  // this expert's pairs from the routing itself; the down kernel's counters start at 0
        if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
            for (int i = threadIdx.x; i < sf.nctr; i += blockDim.x) sf.ctr[i] = 0u;
        e = blockIdx.y;
        cnt = expert_group<256>(sf.idx, sf.T * k, e, glist, gwc);
    } else {
        const int s = blockIdx.y;
        if (s >= active[E]) return;
        e = active[s];
        cnt = counts[e];
        base = offs[e];
    }
    if (t0 >= cnt) return;
    // pair i of the expert's group (token pair / k, selection slot pair % k)
    auto pair_of = [&](int i) { return SELF ? glist[i] : perm[base + i]; };
    const int tn = min(kTok, cnt - t0);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r = lane & 15, g = lane >> 4;
    const int o = min((blockIdx.x * 4 + wv) * 16, fe - 16) + r;  // fe % 16 == 0: a wave past fe repeats rows
    const bool live = (blockIdx.x * 4 + wv) * 16 < fe;
    auto put = [&](int tt, float v) {  // activation of token tt of the tile at row o
        const int pair = pair_of(t0 + tt);
        const __bf16 hi = __bf16(v);
        const __bf16 lo = __bf16(v - float(hi));
        uint16_t *row = hp + size_t(pair) * fe * 2 + (o >> 2) * 8;
        const int j = q6k_slot_of(o);
        row[j] = __builtin_bit_cast(uint16_t, hi);
        row[4 + j] = __builtin_bit_cast(uint16_t, lo);
    };
    gbyte *G = gmem(table[3 * e]);
    gbyte *U = gmem(table[3 * e + 1]);
    if (!G || !U) {  // an unregistered expert contributes nothing (src/gguf_run.c:201)
        if (live)
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (4 * g + i < tn) put(4 * g + i, 0.0f);
        return;
    }
    // the split inputs of the tile's tokens: thread tid copies 16-byte piece
    // tid % 64 of token tid / 64 + 4 i's super-block
    const int pc = tid & 63, pt = tid >> 6;
    uint32_t srow[4];  // the tokens' rows of xp, in 16-byte pieces
#pragma unroll
    for (int i = 0; i < 4; i++) srow[i] = uint32_t(pair_of(t0 + min(pt + 4 * i, tn - 1)) / k) * uint32_t(d / 4) + pc;
    uint32_t *xdst = &xs[0][pt * kGuTokStride + 4 * pc];
    // this lane's token (row r of the input operand) in the sub-block sums
    const uint2 *xsr = xsum + size_t(pair_of(t0 + min(r, tn - 1)) / k) * NB * 4 + g;
    // PK: the wave's 16-row group's tiles (see mdec_pack_kernel); else its rows
    gbyte *gr = PK ? G + int64_t(o - r) / 16 * NB * kQ4Tile : G + int64_t(o) * row_bytes;
    gbyte *ur = PK ? U + int64_t(o - r) / 16 * NB * kQ4Tile : U + int64_t(o) * row_bytes;
    struct Wt {
        uint4 hd, q0, q1;
    };
    struct Blk {
        Wt gw, uw;
        uint2 xsm;
    };
    auto load = [&](int b, Blk &w) {
        if constexpr (PK) {  // per matrix: d and dmin, the decoded scales, two 1 KB-wide qs loads
            gbyte *p = gr + kQ4Tile * b;
            w.gw.hd = make_uint4(ld_u32(p + 4 * r), ld_u32(p + 64 + 4 * lane), 0u, 0u);
            w.gw.q0 = ld_u128(p + 320 + 16 * lane);
            w.gw.q1 = ld_u128(p + 1344 + 16 * lane);
            p = ur + kQ4Tile * b;
            w.uw.hd = make_uint4(ld_u32(p + 4 * r), ld_u32(p + 64 + 4 * lane), 0u, 0u);
            w.uw.q0 = ld_u128(p + 320 + 16 * lane);
            w.uw.q1 = ld_u128(p + 1344 + 16 * lane);
        } else {
            gbyte *p = gr + 144 * b;
            w.gw.hd = ld_u128(p);
            w.gw.q0 = ld_u128(p + 16 + 32 * g);
            w.gw.q1 = ld_u128(p + 32 + 32 * g);
            p = ur + 144 * b;
            w.uw.hd = ld_u128(p);
            w.uw.q0 = ld_u128(p + 16 + 32 * g);
            w.uw.q1 = ld_u128(p + 32 + 32 * g);
        }
        w.xsm = xsr[4 * b];
    };
    // weights this many super-blocks ahead: two for GGUF rows, one for tiles
    // (their loads stream at full rate; the registers saved keep four waves per SIMD)
    constexpr int AH = PK ? 1 : 2;
    Blk blk[AH + 1];
    // rows 4 .. 15 only when the tile has more than 4 tokens (a branch the
    // whole workgroup takes alike); lanes of padding rows read the last
    // token's row
    const bool wide = tn > 4;
    uint4 xv0, xv1, xv2, xv3;
    xv0 = xp[srow[0]];
    if (wide) {
        xv1 = xp[srow[1]];
        xv2 = xp[srow[2]];
        xv3 = xp[srow[3]];
    }
    load(0, blk[0]);
    if (AH > 1 && NB > 1) load(1, blk[1]);
    *reinterpret_cast<uint4 *>(xdst) = xv0;
    if (wide) {
        *reinterpret_cast<uint4 *>(xdst + 4 * kGuTokStride) = xv1;
        *reinterpret_cast<uint4 *>(xdst + 8 * kGuTokStride) = xv2;
        *reinterpret_cast<uint4 *>(xdst + 12 * kGuTokStride) = xv3;
    }
    __syncthreads();
    // the nibble masks and the fp16 exponent, held in registers (see and_or)
    uint32_t kLo = 0x000f000fu, kHi = 0x00f000f0u, kE = 0x64006400u;
    asm volatile("" : "+v"(kLo), "+v"(kHi), "+v"(kE));
    const uint32_t *xr = &xs[0][min(r, tn - 1) * kGuTokStride + 8 * g];  // this lane's token, lane group g
    f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = accg;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b + 1 < NB) {
            xv0 = xp[srow[0] + 64 * (b + 1)];
            if (wide) {
                xv1 = xp[srow[1] + 64 * (b + 1)];
                xv2 = xp[srow[2] + 64 * (b + 1)];
                xv3 = xp[srow[3] + 64 * (b + 1)];
            }
        }
        if (b + AH < NB) load(b + AH, blk[(b + AH) % (AH + 1)]);
        const Blk &cb = blk[b % (AH + 1)];
        const Wt &cg = cb.gw, &cu = cb.uw;
        const uint32_t *xb = xr + (b & 1) * (kTok * kGuTokStride);
        f16x2 s0g, n0g, s1g, n1g, s0u, n0u, s1u, n1u;
        f16x8 mopg, mopu;
        // the fp16 factors of sub-blocks 2 g and 2 g + 1 (see q4k_operand), and
        // the min operand m_2g, m_2g, m_2g+1, m_2g+1 against the sums' slots
        auto scales = [&](const uint4 &hd, f16x2 &s0, f16x2 &n0, f16x2 &s1, f16x2 &n1, f16x8 &mop) {
            int sc0, mn0, sc1, mn1;
            if constexpr (PK) {  // decoded when the tiles were made
                sc0 = int(hd.y & 0xffu);
                sc1 = int((hd.y >> 8) & 0xffu);
                mn0 = int((hd.y >> 16) & 0xffu);
                mn1 = int(hd.y >> 24);
            } else {
                q4k_scale_min_v(2 * g, hd.y, hd.z, hd.w, sc0, mn0);
                q4k_scale_min_v(2 * g + 1, hd.y, hd.z, hd.w, sc1, mn1);
            }
            const _Float16 a0 = _Float16(sc0), a1 = _Float16(float(sc1) * 0.0625f);
            const _Float16 m0 = _Float16(mn0), m1 = _Float16(mn1), z = _Float16(0.0f);
            s0 = f16x2{a0, a0};
            s1 = f16x2{a1, a1};
            n0 = f16x2{_Float16(-1024 * sc0), _Float16(-1024 * sc0)};
            n1 = f16x2{_Float16(-64 * sc1), _Float16(-64 * sc1)};
            mop = f16x8{m0, m0, m1, m1, z, z, z, z};
        };
        scales(cg.hd, s0g, n0g, s1g, n1g, mopg);
        scales(cu.hd, s0u, n0u, s1u, n1u, mopu);
        const uint32_t wgs[8] = {cg.q0.x, cg.q0.y, cg.q0.z, cg.q0.w, cg.q1.x, cg.q1.y, cg.q1.z, cg.q1.w};
        const uint32_t wus[8] = {cu.q0.x, cu.q0.y, cu.q0.z, cu.q0.w, cu.q1.x, cu.q1.y, cu.q1.z, cu.q1.w};
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const f16x8 xsop = __builtin_bit_cast(f16x8, make_uint4(cb.xsm.x, cb.xsm.y, 0u, 0u));
        const f32x4 m_g = __builtin_amdgcn_mfma_f32_16x16x32_f16(xsop, mopg, zero, 0, 0, 0);
        const f32x4 m_u = __builtin_amdgcn_mfma_f32_16x16x32_f16(xsop, mopu, zero, 0, 0, 0);
        f32x4 c_g = zero, c_u = zero;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const f16x8 xh = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4 *>(xb + 32 * u));
            const f16x8 xl = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4 *>(xb + 32 * u + 4));
            const f16x8 bg = q4k_operand(wgs[u], s0g, n0g, s1g, n1g, kLo, kHi, kE);
            const f16x8 bu = q4k_operand(wus[u], s0u, n0u, s1u, n1u, kLo, kHi, kE);
            c_g = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bg, c_g, 0, 0, 0);
            c_g = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bg, c_g, 0, 0, 0);
            c_u = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bu, c_u, 0, 0, 0);
            c_u = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bu, c_u, 0, 0, 0);
        }
        // M holds sum m_s X_s / 32
        const float dg = h2f(cg.hd.x & 0xffffu), mg = 32.0f * h2f(cg.hd.x >> 16);
        const float du = h2f(cu.hd.x & 0xffffu), mu = 32.0f * h2f(cu.hd.x >> 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            accg[i] = fmaf(dg, c_g[i], fmaf(-mg, m_g[i], accg[i]));
            accu[i] = fmaf(du, c_u[i], fmaf(-mu, m_u[i], accu[i]));
        }
        // the block's sums are added here, not deferred past the later blocks
        // (which would hold every block's results in registers)
        asm volatile("" : "+v"(accg), "+v"(accu));
        if (b + 1 < NB) {  // into the buffer read two super-blocks ago
            uint32_t *dst = xdst + ((b + 1) & 1) * (kTok * kGuTokStride);
            *reinterpret_cast<uint4 *>(dst) = xv0;
            if (wide) {
                *reinterpret_cast<uint4 *>(dst + 4 * kGuTokStride) = xv1;
                *reinterpret_cast<uint4 *>(dst + 8 * kGuTokStride) = xv2;
                *reinterpret_cast<uint4 *>(dst + 12 * kGuTokStride) = xv3;
            }
            __syncthreads();
        }
    }
    if (!live) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int tt = 4 * g + i;
        if (tt >= tn) continue;
        const float sc = xsc[pair_of(t0 + tt) / k];
        put(tt, swiglu(accg[i] * sc, accu[i] * sc));
    }
}

// down: wave w of workgroup (c, s, z) of NW waves owns rows 16 NW c + 16 w ..
// + 15 of down of expert active[s] (one 16-row tile) for its group's tokens
// in tiles of kDnTok, and writes y[pair][row] = down_row . h[pair]
// (src/gguf_run.c:208), combined in selection order by the combine kernel or
// (SELF) by the kernel itself. Every super-block of the lane's row is
// requested first; then each tile's activations (all of fe) are copied to LDS
// for the workgroup's waves; each wave passes its
// rows' ql and qh bytes through its own LDS (coalesced 16-byte loads in, the
// words its lanes need out).
constexpr int kDnRowStride = 52;  // dwords per weight row in LDS: 32 ql + 16 qh + 4 (no bank conflicts)
constexpr int kDnMaxBlocks = 4;   // fe <= 1024
template <bool PK, bool SELF, int NW>
__global__ void __launch_bounds__(64 * NW) mdec_down_kernel(const int32_t *__restrict__ counts,
                                                                  const int32_t *__restrict__ offs,
                                                                  const int32_t *__restrict__ perm,
                                                                  const int32_t *__restrict__ active,
                                                                  const void *const *__restrict__ table,
                                                                  const uint4 *__restrict__ hp, int fe, int d, int E,
                                                                  int64_t row_bytes, float *__restrict__ y, MdecSelf sf) {
    extern __shared__ __align__(16) uint32_t hs[];  // [kDnTok][fe + 4]
    constexpr int CR = 16 * NW;  // output rows of one workgroup (the combine's unit)
    __shared__ __align__(16) uint32_t wq[PK ? 1 : NW][PK ? 4 : 16 * kDnRowStride];  // GGUF rows only
    __shared__ int glist[SELF ? kGroupMax : 1], gwc[SELF ? NW : 1], last[SELF ? kGroupMax + 1 : 1];
    int e, cnt, base = 0;
    if constexpr (SELF) {
        e = blockIdx.y;
        cnt = expert_group<64 * NW>(sf.idx, sf.T * sf.k, e, glist, gwc);
    } else {
        const int s = blockIdx.y;
        if (s >= active[E]) return;
        e = active[s];
        cnt = counts[e];
        base = offs[e];
    }
    if (int(blockIdx.z) * kDnTok >= cnt) return;
    auto pair_of = [&](int i) { return SELF ? glist[i] : perm[base + i]; };
    gbyte *D = gmem(table[3 * e + 2]);
    // an unregistered expert: skipped by the combine kernel, or (SELF) its rows
    // of y are zeros, which the combine below adds without changing a bit
    // (src/gguf_run.c:201)
    if (!SELF && !D) return;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r = lane & 15, g = lane >> 4;
    const int o0 = min((blockIdx.x * NW + wv) * 16, d - 16);  // d % 16 == 0: a wave past d repeats rows
    const bool live = (blockIdx.x * NW + wv) * 16 < d;
    gbyte *row = D + int64_t(o0 + r) * row_bytes;
    const int nb = fe / 256;
    uint4 a0[kDnMaxBlocks], a1[kDnMaxBlocks], qq[kDnMaxBlocks], scb[kDnMaxBlocks];
    uint32_t ddb[kDnMaxBlocks];
    if (D) {  // the rows' weights, held in registers for every token tile of the expert
#pragma unroll
        for (int b = 0; b < kDnMaxBlocks; b++) {
            if (b >= nb) break;
            if constexpr (PK) {  // the wave's tile of super-block b: 1 KB-wide loads of ql, ql, qh, then scales and d
                gbyte *p = D + (int64_t(o0 / 16) * nb + b) * kQ6Tile;
                a0[b] = ld_u128(p + 16 * lane);
                a1[b] = ld_u128(p + 1024 + 16 * lane);
                qq[b] = ld_u128(p + 2048 + 16 * lane);
                scb[b] = ld_u128(p + 3072 + 16 * r);
                ddb[b] = ld_u16(p + 3328 + 2 * r);
            } else {
                gbyte *p = row + 210 * b;
                a0[b] = ld_u128(p + 16 * g);
                a1[b] = ld_u128(p + 64 + 16 * g);
                qq[b] = ld_u128(p + 128 + 16 * g);
                scb[b] = ld_u128(p + 192);
                ddb[b] = ld_u16(p + 208);
            }
        }
    }
    // the expert's tokens in tiles of kDnTok (with one workgroup on the z
    // axis: every tile; the weights are read once)
    for (int t0 = blockIdx.z * kDnTok; t0 < cnt; t0 += gridDim.z * kDnTok) {
    const int tn = min(kDnTok, cnt - t0);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (D) {
        // the tile's activations: token i's fe / 4 pieces of 16 bytes
        const int hstride = fe + 4, npc = fe / 4;
        if (t0 != int(blockIdx.z) * kDnTok) __syncthreads();  // every wave is done with the previous tile
        for (int i = tid; i < tn * npc; i += 64 * NW) {
            const int tt = i / npc, c = i - tt * npc;
            *reinterpret_cast<uint4 *>(&hs[tt * hstride + 4 * c]) = hp[size_t(pair_of(t0 + tt)) * npc + c];
        }
        __syncthreads();  // the activations are in LDS (and the weights have arrived)
        const uint4 *xr = reinterpret_cast<const uint4 *>(&hs[min(r, tn - 1) * hstride]) + g;
        // bf16 q + 128 is the byte q under the byte 0x43: v_perm_b32 takes
        // bytes 0 and 2 (w0) or 1 and 3 (w1) of q (selectors 4-7: its bytes)
        // with a 0x43 byte of the constant (selector 0) above each
        constexpr uint32_t kB = 0x43434343u, kSel0 = 0x00060004u, kSel1 = 0x00070005u;
        const bf16x8 k160 = __builtin_bit_cast(bf16x8, make_uint4(0xC320C320u, 0xC320C320u, 0xC320C320u, 0xC320C320u));  // bf16 -160
        uint32_t *wl = PK ? &wq[0][0] : &wq[wv][r * kDnRowStride];
#pragma unroll
        for (int b = 0; b < kDnMaxBlocks; b++) {
            if (b >= nb) break;
            {  // the super-block's words pass an empty asm statement in every tile: nothing
               // derived from them is hoisted out of the token loop (into registers for all tiles)
                u32x4 v0 = __builtin_bit_cast(u32x4, a0[b]), v1 = __builtin_bit_cast(u32x4, a1[b]);
                u32x4 v2 = __builtin_bit_cast(u32x4, qq[b]), v3 = __builtin_bit_cast(u32x4, scb[b]);
                asm volatile("" : "+v"(v0), "+v"(v1), "+v"(v2), "+v"(v3), "+v"(ddb[b]));
                a0[b] = __builtin_bit_cast(uint4, v0);
                a1[b] = __builtin_bit_cast(uint4, v1);
                qq[b] = __builtin_bit_cast(uint4, v2);
                scb[b] = __builtin_bit_cast(uint4, v3);
            }
            // ql chunks g and g + 4, qh chunk g of the row into the wave's LDS;
            // lane group g then reads word g of the chunk each step needs
            if constexpr (!PK) {
                *reinterpret_cast<uint4 *>(wl + 4 * g) = a0[b];
                *reinterpret_cast<uint4 *>(wl + 16 + 4 * g) = a1[b];
                *reinterpret_cast<uint4 *>(wl + 32 + 4 * g) = qq[b];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            const float dd = h2f(ddb[b]);
            const uint32_t scw[4] = {scb[b].x, scb[b].y, scb[b].z, scb[b].w};
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int lh = 0; lh < 2; lh++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int sb = 8 * h + 2 * j + lh, ql_c = 4 * h + 2 * (j & 1) + lh, qh_c = 2 * h + lh;
                        // slots 0-3: the hi parts of the lane's 4 activations, 4-7 their lo parts;
                        // the weight operand repeats q + 128 for both
                        const bf16x8 xa = __builtin_bit_cast(bf16x8, xr[64 * b + 4 * sb]);
                        // word g of ql chunk ql_c and of qh chunk qh_c: from LDS, or (tiles) the
                        // lane's own loads, which hold exactly those words
                        const uint4 la = PK ? (ql_c < 4 ? a0[b] : a1[b]) : make_uint4(0u, 0u, 0u, 0u);
                        const uint32_t lw = PK ? u4_at(la, ql_c & 3) : wl[4 * ql_c + g];
                        const uint32_t hw = PK ? u4_at(qq[b], qh_c) : wl[32 + 4 * qh_c + g];
                        const uint32_t q = ((lw >> (j >= 2 ? 4 : 0)) & 0x0f0f0f0fu) | (((hw >> (2 * j)) & 0x03030303u) << 4);
                        const uint32_t w0 = __builtin_amdgcn_perm(q, kB, kSel0), w1 = __builtin_amdgcn_perm(q, kB, kSel1);
                        const bf16x8 wb = __builtin_bit_cast(bf16x8, make_uint4(w0, w1, w0, w1));
                        f32x4 c = {0.f, 0.f, 0.f, 0.f};
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, wb, c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, k160, c, 0, 0, 0);
                        const float ds = dd * float(int(int8_t(scw[sb >> 2] >> (8 * (sb & 3)))));
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[i] = fmaf(ds, c[i], acc[i]);
                    }
            if constexpr (!PK) {  // every lane is done with this super-block's words before the next overwrite them
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
    }  // D
    // y (SELF: agent-scope stores, for the combine below)
    if (live) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tt = 4 * g + i;
            if (tt >= tn) continue;
            float *dst = &y[size_t(pair_of(t0 + tt)) * d + o0 + r];
            if constexpr (SELF) __hip_atomic_store(dst, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else *dst = acc[i];
        }
    }
    }  // token tiles
    if constexpr (SELF) {
        // The combine (src/gguf_run.c:208-212) of output rows [CR c,
        // + CR) of a token is done by the last of its k experts'
        // workgroups to write them: y goes out as agent-scope stores, each
        // workgroup waits until its stores are done, then counts one arrival
        // per token at ctr[c][t] (agent-scope atomics); the workgroup that
        // brings a count to k reads the k rows with agent-scope loads (they
        // bypass this XCD's L2, which need not hold the other XCDs' writes).
        if (tid == 0) last[kGroupMax] = 0;
        VH_WAIT_VMCNT(0);
        __syncthreads();
        const int c = blockIdx.x, k = sf.k;
        // the tokens of this workgroup's tiles (cnt <= kGroupMax < 64 NW)
        if (tid < cnt && (tid / kDnTok) % int(gridDim.z) == int(blockIdx.z)) {
            const int t = pair_of(tid) / k;
            const uint32_t n = __hip_atomic_fetch_add(&sf.ctr[c * kGroupMax + t], 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            if (n == uint32_t(k - 1)) last[atomicAdd(&last[kGroupMax], 1)] = t;  // this workgroup combines token t
        }
        __syncthreads();
        // the (token, row) items of the combines, kItems per thread with every
        // load of a thread issued before the first sum (the combine kernel's
        // arithmetic, in selection order)
        constexpr int kItems = kDnTok * CR / (64 * NW);
        const int nl = last[kGroupMax];
        if (nl == 0 || nl > kDnTok || k > 8) {
            for (int it = tid; it < nl * CR; it += 64 * NW) {  // k > 8 or tokens of several tiles: one item at a time
                const int t = last[it / CR], o = c * CR + it % CR;
                if (o >= d) continue;
                float a = 0.0f;
                for (int j = 0; j < k; j++)
                    a = add_rn(a, mul_rn(sf.w[size_t(t) * k + j],
                                         __hip_atomic_load(&y[(size_t(t) * k + j) * d + o], __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)));
                sf.x[size_t(t) * d + o] = add_rn(sf.x[size_t(t) * d + o], a);
            }
            return;
        }
        float yv[kItems][8], wt[kItems][8], xo[kItems];
#pragma unroll
        for (int q = 0; q < kItems; q++) {
            const int it = min(tid + 64 * NW * q, nl * CR - 1);
            const int t = last[it / CR], o = min(c * CR + it % CR, d - 1);
            xo[q] = sf.x[size_t(t) * d + o];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int jj = min(j, k - 1);
                yv[q][j] = __hip_atomic_load(&y[(size_t(t) * k + jj) * d + o], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
                wt[q][j] = sf.w[size_t(t) * k + jj];
            }
        }
#pragma unroll
        for (int q = 0; q < kItems; q++) {
            const int it = tid + 64 * NW * q;
            const int o = c * CR + it % CR;
            if (it >= nl * CR || o >= d) continue;
            const int t = last[it / CR];
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (j < k) a = add_rn(a, mul_rn(wt[q][j], yv[q][j]));
            sf.x[size_t(t) * d + o] = add_rn(xo[q], a);
        }
    }
}

}  // namespace

bool vh_mdec_supported(uint32_t tg, uint32_t td, int d, int fe) {
    // d: whole super-blocks (at most kGuMaxBlocks, the gate/up kernel's
    // unrolled loop) and 32-row waves; fe: whole super-blocks, 16-row waves and
    // the activations of a 16-token tile in LDS
    return tg == VT_Q4_K && td == VT_Q6_K && d % 256 == 0 && d <= 256 * kGuMaxBlocks && fe % 256 == 0 &&
           fe <= 256 * kDnMaxBlocks;
}

int vh_route_parts_tiled(const float *R, const float *hb, const float *bias, int d, int E, int T, RoutePart *parts,
                         void *xp, float *xsc, hipStream_t s) {
    if (d != 2048 || T < 2 || E < 1 || ((reinterpret_cast<uintptr_t>(R) | reinterpret_cast<uintptr_t>(hb)) & 15u))
        return -EINVAL;
    const dim3 g((E + kRpTile - 1) / kRpTile, (T + kRpTile - 1) / kRpTile);
    hipLaunchKernelGGL(mdec_route_prep_kernel, g, dim3(256), 0, s, R, hb, bias, E, T, parts,
                       static_cast<_Float16 *>(xp), xsc,
                       xp ? static_cast<_Float16 *>(vh_mdec_xsum(xp, T, d)) : nullptr);
    return vh_check(hipGetLastError());
}

int vh_mdec_prep(const float *hb, int T, int d, void *xp, float *xsc, hipStream_t s) {
    if (T < 1 || d % 256) return -EINVAL;
    hipLaunchKernelGGL(mdec_prep_kernel, dim3(T), dim3(256), 0, s, hb, d, static_cast<_Float16 *>(xp), xsc,
                       static_cast<_Float16 *>(vh_mdec_xsum(xp, T, d)));
    return vh_check(hipGetLastError());
}

int vh_mdec_gateup(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                   const void *const *table, bool packed, const void *xp, const float *xsc, int T, int d, int fe,
                   int k, int E, int max_slots, int max_count, void *hp, hipStream_t s, const MdecSelf *self) {
    if (max_count < 1 || T < 1 || d % 256 || d > 256 * kGuMaxBlocks || fe % 16) return -EINVAL;
    if (self && (self->T != T || T > kGroupMax || self->k != k || self->nctr < vh_mdec_ctr_words(d))) return -EINVAL;
    const MdecSelf sf = self ? *self : MdecSelf{};
    const dim3 g((fe + 63) / 64, self ? E : max_slots, (max_count + kTok - 1) / kTok);
    const uint4 *x4 = static_cast<const uint4 *>(xp);
    const uint2 *xs = static_cast<const uint2 *>(vh_mdec_xsum(const_cast<void *>(xp), T, d));
    const int64_t rb = vh_row_bytes(VT_Q4_K, d);
    uint16_t *h = static_cast<uint16_t *>(hp);
#define VH_GU_PK(NB, PK)                                                                                           \
    if (self)                                                                                                      \
        hipLaunchKernelGGL((mdec_gateup_kernel<NB, PK, true>), g, dim3(256), 0, s, counts, offs, perm, active,    \
                           table, x4, xsc, xs, fe, k, E, rb, h, sf);                                               \
    else                                                                                                           \
        hipLaunchKernelGGL((mdec_gateup_kernel<NB, PK, false>), g, dim3(256), 0, s, counts, offs, perm, active,   \
                           table, x4, xsc, xs, fe, k, E, rb, h, sf);
#define VH_GU(NB)                                                                                                  \
    case NB:                                                                                                       \
        if (packed) {                                                                                              \
            VH_GU_PK(NB, true)                                                                                     \
        } else {                                                                                                   \
            VH_GU_PK(NB, false)                                                                                    \
        }                                                                                                          \
        break;
    switch (d / 256) {
        VH_GU(1) VH_GU(2) VH_GU(3) VH_GU(4) VH_GU(5) VH_GU(6) VH_GU(7) VH_GU(8)
    }
#undef VH_GU
#undef VH_GU_PK
    return vh_check(hipGetLastError());
}

namespace {
// The down kernel's launch with NW waves (16 NW rows of d) per workgroup.
template <int NW>
int mdec_down_launch(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                     const void *const *table, bool packed, const uint4 *h4, int d, int fe, int E, int max_slots,
                     int max_count, float *ybuf, hipStream_t s, const MdecSelf *self) {
    const MdecSelf sf = self ? *self : MdecSelf{};
    // one workgroup per (row chunk, expert) takes all of the expert's tokens
    // where it finds them itself; else the token tiles spread over z
    const dim3 g((d + 16 * NW - 1) / (16 * NW), self ? E : max_slots, self ? 1 : (max_count + kDnTok - 1) / kDnTok);
    const size_t lds = size_t(kDnTok) * (fe + 4) * 4;
    static bool attr = false;  // dynamic LDS above the default limit: raised once per process
    if (!attr) {
        for (const void *f : {reinterpret_cast<const void *>(&mdec_down_kernel<true, false, NW>),
                              reinterpret_cast<const void *>(&mdec_down_kernel<false, false, NW>),
                              reinterpret_cast<const void *>(&mdec_down_kernel<true, true, NW>),
                              reinterpret_cast<const void *>(&mdec_down_kernel<false, true, NW>)})
            if (int rc = vh_check(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024)))
                return rc;
        attr = true;
    }
    const int64_t rb = vh_row_bytes(VT_Q6_K, fe);
    const dim3 b(64 * NW);
    if (packed && self)
        hipLaunchKernelGGL((mdec_down_kernel<true, true, NW>), g, b, lds, s, counts, offs, perm, active, table, h4, fe,
                           d, E, rb, ybuf, sf);
    else if (packed)
        hipLaunchKernelGGL((mdec_down_kernel<true, false, NW>), g, b, lds, s, counts, offs, perm, active, table, h4,
                           fe, d, E, rb, ybuf, sf);
    else if (self)
        hipLaunchKernelGGL((mdec_down_kernel<false, true, NW>), g, b, lds, s, counts, offs, perm, active, table, h4,
                           fe, d, E, rb, ybuf, sf);
    else
        hipLaunchKernelGGL((mdec_down_kernel<false, false, NW>), g, b, lds, s, counts, offs, perm, active, table, h4,
                           fe, d, E, rb, ybuf, sf);
    return vh_check(hipGetLastError());
}
}  // namespace

int vh_mdec_down(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                 const void *const *table, bool packed, const void *hp, int d, int fe, int E, int max_slots,
                 int max_count, float *ybuf, hipStream_t s, const MdecSelf *self) {
    if (max_count < 1 || d % 16 || fe % 256 || fe > 256 * kDnMaxBlocks) return -EINVAL;
    if (self && (self->T > kGroupMax || self->T < max_count || !self->x || !self->w || self->k < 1 ||
                 self->nctr < vh_mdec_ctr_words(d)))
        return -EINVAL;
    if (size_t(kDnTok) * (fe + 4) * 4 > 96 * 1024) return -EINVAL;
    const uint4 *h4 = static_cast<const uint4 *>(hp);
    // four-wave workgroups for rows of up to three super-blocks (a 768-wide
    // down: 108.3 -> 106.9 us per 32-token layer call), eight for four (a
    // 1024-wide down: 79.2 us per 16-token call with four, 77.8 with eight)
    if (fe <= 768)
        return mdec_down_launch<4>(counts, offs, perm, active, table, packed, h4, d, fe, E, max_slots, max_count, ybuf,
                                   s, self);
    return mdec_down_launch<8>(counts, offs, perm, active, table, packed, h4, d, fe, E, max_slots, max_count, ybuf, s,
                               self);
}

namespace {
// Bytes of one expert's tiles: gate and up, then down.
size_t mdec_pack_per(int d, int fe, size_t *gb_out) {
    const size_t gb = size_t(fe / 16) * (d / 256) * kQ4Tile, db = size_t(d) * vh_row_bytes(VT_Q6_K, fe);
    if (gb_out) *gb_out = gb;
    return 2 * gb + db;
}
}  // namespace

uint64_t vh_mdec_pack_bytes(int E, int d, int fe) {
    if (E < 1 || d < 256 || fe < 256 || d % 256 || fe % 256) return 0;
    return uint64_t(mdec_pack_per(d, fe, nullptr)) * E;
}

int vh_mdec_pack_layer(const void *const *table, int E, int d, int fe, void *buf, void **tab_out, hipStream_t s) {
    *tab_out = nullptr;
    if (!buf || !vh_mdec_pack_bytes(E, d, fe)) return -EINVAL;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (int rc = vh_check(hipStreamIsCapturing(s, &cap))) return rc;
    if (cap != hipStreamCaptureStatusNone) return -EBUSY;  // no allocation under capture
    const int64_t rg = vh_row_bytes(VT_Q4_K, d), rd = vh_row_bytes(VT_Q6_K, fe);
    size_t gb = 0;
    const size_t per = mdec_pack_per(d, fe, &gb);
    std::vector<const void *> src(size_t(3) * E), dst(size_t(3) * E, nullptr);
    if (int rc = vh_check(hipMemcpyAsync(src.data(), table, src.size() * sizeof(void *), hipMemcpyDeviceToHost, s)))
        return rc;
    if (int rc = vh_check(hipStreamSynchronize(s))) return rc;
    void *tab = nullptr;
    if (hipMalloc(&tab, src.size() * sizeof(void *)) != hipSuccess) return -ENOMEM;
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
        const dim3 gg(fe / 16 * (d / 256), E), gd(d / 16 * (fe / 256), E);
        hipLaunchKernelGGL(mdec_pack_q4k_kernel, gg, dim3(256), 0, s, table, dt, 0, d / 256, rg);
        hipLaunchKernelGGL(mdec_pack_q4k_kernel, gg, dim3(256), 0, s, table, dt, 1, d / 256, rg);
        hipLaunchKernelGGL(mdec_pack_q6k_kernel, gd, dim3(256), 0, s, table, dt, 2, fe / 256, rd);
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
