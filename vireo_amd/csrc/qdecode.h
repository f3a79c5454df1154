// Per-format decoding of GGUF weight rows into partial dot products.
//
// A row is split into "items" of 32 weights (64 for paired Q8_0 blocks); a lane
// takes whole items, so a wave covers a row with L lanes and the partial sums
// are added with a DPP tree. Layouts follow the reference dequant
// (src/gguf_compute.c:38-124); the dot products use fp32 FMA on the integer
// quants and apply the block scales once per sub-block, which is the same sum
// as dequantize-then-dot up to fp32 reassociation.
//
// Addressing: every function takes a 4-byte-aligned base (a tensor in HBM or a
// staged copy in LDS) and a byte offset. Q8_0, Q6_K and Q5_0 blocks start at
// even offsets only (34-, 210- and 22-byte blocks), so their fields are read
// with aligned loads of a window that stays inside the block, and the
// misalignment (0 or 2 bytes) is taken from the offset, never from the pointer.
#pragma once
#include "common.h"

// ---------------------------------------------------------------- Q8_0 (34 B / 32)
// Block {f16 d; int8 qs[32]} at even offset b. For b = 2 mod 4 the window
// starts two bytes before the block; those bytes belong to the tensor because
// the tensor starts 4-aligned.
VH_DEV float q8_0_block_dot(const uint8_t *base, int64_t b, const float *x) {
    const uint32_t s = uint32_t(b) & 3u;
    const uint8_t *a = base + (b - int64_t(s));
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = ld_u32(a + 4 * i);
    uint32_t t0 = ld_u16(a + 32), t1 = 0;
    if (s) t1 = ld_u16(a + 34);
    w[8] = t0 | (t1 << 16);
    const float d = h2f((w[0] >> (8 * s)) & 0xffffu);
    const uint32_t sh = 16 + 8 * s;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t q = uint32_t(((uint64_t(w[i + 1]) << 32) | w[i]) >> sh);
#pragma unroll
        for (int k = 0; k < 4; k++) acc = fmaf(float(int(int8_t(q >> (8 * k)))), x[4 * i + k], acc);
    }
    return acc * d;
}

// Two consecutive blocks (68 B) at a 4-aligned offset: 17 aligned dwords.
VH_DEV float q8_0_pair_dot(const uint8_t *base, int64_t off, const float *x) {
    const uint8_t *p = base + off;
    uint32_t w[17];
#pragma unroll
    for (int i = 0; i < 17; i++) w[i] = ld_u32(p + 4 * i);
    const float d0 = h2f(w[0] & 0xffffu), d1 = h2f(w[8] >> 16);
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t q0 = align2(w[i + 1], w[i], 2), q1 = w[9 + i];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            a0 = fmaf(float(int(int8_t(q0 >> (8 * k)))), x[4 * i + k], a0);
            a1 = fmaf(float(int(int8_t(q1 >> (8 * k)))), x[32 + 4 * i + k], a1);
        }
    }
    return a0 * d0 + a1 * d1;
}

// ---------------------------------------------------------------- Q4_K (144 B / 256)
// 6-bit scale and min of sub-block j from the 12 packed bytes
// (src/gguf_compute.c:45-51), given those bytes as three little-endian words.
VH_DEV void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
    auto byte = [&](int i) -> int {
        const uint32_t w = i < 4 ? s0 : i < 8 ? s1 : s2;
        return int((w >> (8 * (i & 3))) & 0xffu);
    };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 15) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Item (c, h) of the super-block at 16-aligned offset sbo: its 16 qs bytes
// hold 16 low nibbles (sub-block 2c, elements 64c+16h..+15) and 16 high nibbles
// (sub-block 2c+1, elements 64c+32+16h..+15). x points at the super-block's
// first element.
VH_DEV float q4k_item_dot(const uint8_t *base, int64_t sbo, int c, int h, const float *x) {
    const uint4 hdr = *reinterpret_cast<const uint4 *>(base + sbo);
    const uint4 q = *reinterpret_cast<const uint4 *>(base + sbo + 16 + 32 * c + 16 * h);
    const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_scale_min(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
    q4k_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
    const float *xl = x + 64 * c + 16 * h, *xh = xl + 32;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    float dl = 0.0f, dh = 0.0f, sl = 0.0f, shs = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = qw[i] & 0x0f0f0f0fu, hi = (qw[i] >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float a = xl[4 * i + k], bb = xh[4 * i + k];
            dl = fmaf(float((lo >> (8 * k)) & 0xffu), a, dl);
            dh = fmaf(float((hi >> (8 * k)) & 0xffu), bb, dh);
            sl += a;
            shs += bb;
        }
    }
    return (d * float(sc0)) * dl - (dmin * float(m0)) * sl + (d * float(sc1)) * dh - (dmin * float(m1)) * shs;
}

// ---------------------------------------------------------------- Q6_K (210 B / 256)
// Item (hh, q) of the super-block at even offset sbo covers elements
// 128hh + 32g + 8q + i (g < 4, i < 8): the low (g < 2) or high nibble of
// ql[64hh + 32(g&1) + 8q + i], bits 2g of qh[32hh + 8q + i], minus 32, scaled by
// d * scales[8hh + q/2 + 2g] (src/gguf_compute.c:83-103).
struct Q6Raw {
    uint32_t a0, a1, b0, b1, h0, h1;  // ql[.. +8q], ql[.. +32 +8q], qh[.. +8q]: 8 bytes each
    uint32_t sc;                      // the four int8 scales, g in byte g
    uint32_t d;                       // f16 bits
};
// 8 bytes at even offset `off` of 4-aligned `base`, from the 12-byte aligned
// window that ends at the first multiple of 4 at or after off + 8 (so the window
// never reaches past off + 10).
template <class P>
VH_DEV void ld8_end(P base, int off, uint32_t &w0, uint32_t &w1) {
    const int end = (off + 8 + 3) & ~3;
    const u32x3 v = ld_u96(base + end - 12);
    const bool four = ((off & 3) == 0);  // bytes [off, off+8) start 4 into the window, else 2
    w0 = four ? v.y : align2(v.y, v.x, 2);
    w1 = four ? v.z : align2(v.z, v.y, 2);
}
template <class P>
VH_DEV Q6Raw q6k_fetch(P base, int64_t sbo, int hh, int q) {
    Q6Raw r;
    const int o = int(sbo & 3);
    P sb = base + (sbo - o);  // 4-aligned; offsets below are relative to it
    // windows [start, start+12) with start >= field - 2 >= -2 and end <= 196
    ld12_even(sb, o + 64 * hh + 8 * q, r.a0, r.a1);
    ld12_even(sb, o + 64 * hh + 32 + 8 * q, r.b0, r.b1);
    ld12_even(sb, o + 128 + 32 * hh + 8 * q, r.h0, r.h1);
    // scales[8hh .. 8hh+7] (bytes 192+8hh ..), window ending at most at byte 210
    uint32_t s0, s1;
    ld8_end(sb, o + 192 + 8 * hh, s0, s1);
    const uint32_t sh = 8u * uint32_t(q >> 1);  // scales 8hh + q/2 + 2g -> bytes q/2, q/2+2 of each word
    const uint32_t t0 = (s0 >> sh) & 0x00ff00ffu, t1 = (s1 >> sh) & 0x00ff00ffu;
    r.sc = (t0 & 0xffu) | ((t0 >> 8) & 0xff00u) | ((t1 & 0xffu) << 16) | ((t1 << 8) & 0xff000000u);
    r.d = ld_u16(sb + o + 208);
    return r;
}
// The same item as the aligned windows the loads return, before any
// arithmetic on them: a kernel that issues many items' loads before using any
// keeps them all in flight (arithmetic on a loaded word waits for the load).
struct Q6Win {
    u32x3 a, b, h, s;  // 12-byte windows holding ql[.. +8q], ql[.. +32 +8q], qh[.. +8q], scales[8hh ..]
    uint32_t d;        // f16 bits
    uint32_t o;        // sbo & 3 (0 or 2): where each field starts in its window
};
template <class P>
VH_DEV Q6Win q6k_fetch_raw(P base, int64_t sbo, int hh, int q) {
    Q6Win r;
    r.o = uint32_t(sbo & 3);
    P sb = base + (sbo - int64_t(r.o));
    // the windows of ld12_even (fields at offsets o + 8m, o even) and ld8_end
    r.a = ld_u96(sb + 64 * hh + 8 * q);
    r.b = ld_u96(sb + 64 * hh + 32 + 8 * q);
    r.h = ld_u96(sb + 128 + 32 * hh + 8 * q);
    r.s = ld_u96(sb + ((int(r.o) + 192 + 8 * hh + 8 + 3) & ~3) - 12);
    r.d = ld_u16(sb + r.o + 208);
    return r;
}
// q6k_fetch's words from the windows (q = item index mod 4)
VH_DEV Q6Raw q6k_resolve(const Q6Win &w, int q) {
    Q6Raw r;
    r.a0 = align2(w.a.y, w.a.x, w.o);
    r.a1 = align2(w.a.z, w.a.y, w.o);
    r.b0 = align2(w.b.y, w.b.x, w.o);
    r.b1 = align2(w.b.z, w.b.y, w.o);
    r.h0 = align2(w.h.y, w.h.x, w.o);
    r.h1 = align2(w.h.z, w.h.y, w.o);
    const bool four = w.o == 0u;  // as ld8_end
    const uint32_t s0 = four ? w.s.y : align2(w.s.y, w.s.x, 2), s1 = four ? w.s.z : align2(w.s.z, w.s.y, 2);
    const uint32_t sh = 8u * uint32_t(q >> 1);
    const uint32_t t0 = (s0 >> sh) & 0x00ff00ffu, t1 = (s1 >> sh) & 0x00ff00ffu;
    r.sc = (t0 & 0xffu) | ((t0 >> 8) & 0xff00u) | ((t1 & 0xffu) << 16) | ((t1 << 8) & 0xff000000u);
    r.d = w.d;
    return r;
}
// xv: the item's 32 inputs, g-major (xv[8g + i] = x[128hh + 32g + 8q + i])
template <class XV>
VH_DEV float q6k_compute(const Q6Raw &r, const XV &xv) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t qa = ((i < 4 ? r.a0 : r.a1) >> (8 * (i & 3))) & 0xffu;
        const uint32_t qb = ((i < 4 ? r.b0 : r.b1) >> (8 * (i & 3))) & 0xffu;
        const uint32_t qh = ((i < 4 ? r.h0 : r.h1) >> (8 * (i & 3))) & 0xffu;
        acc[0] = fmaf(float(int((qa & 15u) | ((qh & 3u) << 4)) - 32), xv[i], acc[0]);
        acc[1] = fmaf(float(int((qb & 15u) | (((qh >> 2) & 3u) << 4)) - 32), xv[8 + i], acc[1]);
        acc[2] = fmaf(float(int((qa >> 4) | (((qh >> 4) & 3u) << 4)) - 32), xv[16 + i], acc[2]);
        acc[3] = fmaf(float(int((qb >> 4) | (((qh >> 6) & 3u) << 4)) - 32), xv[24 + i], acc[3]);
    }
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) s = fmaf(float(int(int8_t(r.sc >> (8 * g)))), acc[g], s);
    return h2f(r.d) * s;
}
// inputs read from a row vector x (global or LDS) at the super-block's element 0
struct Q6XFromRow {
    const float *p;  // x + 128hh + 8q
    VH_DEV float operator[](int i) const { return p[32 * (i >> 3) + (i & 7)]; }
};
VH_DEV float q6k_item_dot(const uint8_t *base, int64_t sbo, int hh, int q, const float *x) {
    const Q6Raw r = q6k_fetch(base, sbo, hh, q);
    return q6k_compute(r, Q6XFromRow{x + 128 * hh + 8 * q});
}

// ---------------------------------------------------------------- Q5_0 (22 B / 32)
VH_DEV float q5_0_block_dot(const uint8_t *base, int64_t b, const float *x) {
    const uint8_t *p = base + b;  // even
    const float d = h2f(ld_u16(p));
    const uint32_t qh = ld_u16(p + 2) | (ld_u16(p + 4) << 16);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t two = ld_u16(p + 6 + 2 * j);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int e = 2 * j + k;
            const uint32_t qs = (two >> (8 * k)) & 0xffu;
            const int x0 = int((qs & 15u) | (((qh >> e) & 1u) << 4)) - 16;
            const int x1 = int((qs >> 4) | (((qh >> (e + 16)) & 1u) << 4)) - 16;
            acc = fmaf(float(x0), x[e], acc);
            acc = fmaf(float(x1), x[e + 16], acc);
        }
    }
    return acc * d;
}

// ---------------------------------------------------------------- dense rows
// Elements [32*it, min(32*it+32, n)) of an F32 / F16 row at offset off.
VH_DEV float f32_item_dot(const uint8_t *base, int64_t off, int it, int n, const float *x) {
    const float *r = reinterpret_cast<const float *>(base + off);
    float acc = 0.0f;
    const int i0 = 32 * it;
    if (i0 + 32 <= n) {
#pragma unroll
        for (int i = 0; i < 32; i++) acc = fmaf(r[i0 + i], x[i0 + i], acc);
    } else {
        for (int i = i0; i < n; i++) acc = fmaf(r[i], x[i], acc);
    }
    return acc;
}
VH_DEV float f16_item_dot(const uint8_t *base, int64_t off, int it, int n, const float *x) {
    float acc = 0.0f;
    const int i0 = 32 * it;
    const int i1 = i0 + 32 < n ? i0 + 32 : n;
    for (int i = i0; i < i1; i++) acc = fmaf(h2f(ld_u16(base + off + 2 * i)), x[i], acc);
    return acc;
}

// ---------------------------------------------------------------- dispatch by type
// Items per row of n elements (the same 32-weight granularity for every type,
// pairs of blocks for PAIRED Q8_0); dot(base, row_off, it, n, x) is the partial
// dot of item it of the row that starts at byte row_off.
template <int T, bool PAIRED = false>
struct Fmt {
    static __host__ __device__ int items(int n) { return T == VT_Q8_0 && PAIRED ? n / 64 : (n + 31) / 32; }
    static VH_DEV float dot(const uint8_t *base, int64_t row, int it, int n, const float *x) {
        if constexpr (T == VT_Q8_0) {
            if constexpr (PAIRED) return q8_0_pair_dot(base, row + 68 * it, x + 64 * it);
            else return q8_0_block_dot(base, row + 34 * it, x + 32 * it);
        } else if constexpr (T == VT_Q4_K) {
            const int sbi = it >> 3, r = it & 7;
            return q4k_item_dot(base, row + 144 * sbi, r >> 1, r & 1, x + 256 * sbi);
        } else if constexpr (T == VT_Q6_K) {
            const int sbi = it >> 3, r = it & 7;
            return q6k_item_dot(base, row + 210 * sbi, r >> 2, r & 3, x + 256 * sbi);
        } else if constexpr (T == VT_Q5_0) {
            return q5_0_block_dot(base, row + 22 * it, x + 32 * it);
        } else if constexpr (T == VT_F16) {
            return f16_item_dot(base, row, it, n, x);
        } else {
            return f32_item_dot(base, row, it, n, x);
        }
    }
};

// ---------------------------------------------------------------- split fetch / compute
// Item decoders with the loads separated from the arithmetic, so a lane can
// issue the loads of several items before it needs any of them. An input
// accessor X gives the item's inputs in the item's own order:
//   Q8_0 (pair): 64 consecutive columns; Q4_K: 16 low-nibble columns then the
//   16 high-nibble columns 32 further on; Q6_K: four runs of 8 columns 32 apart.
template <int T>
struct Split;

template <>
struct Split<VT_Q8_0> {  // paired blocks, 4-aligned
    static constexpr int NW = 64;
    struct Raw { uint32_t w[17]; };
    static VH_DEV int col0(int it) { return 64 * it; }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        Raw r;
        P p = base + row + 68 * it;
#pragma unroll
        for (int i = 0; i < 17; i++) r.w[i] = ld_u32(p + 4 * i);
        return r;
    }
    template <class X>
    static VH_DEV float compute(const Raw &r, int, const X &x) {
        const float d0 = h2f(r.w[0] & 0xffffu), d1 = h2f(r.w[8] >> 16);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q0 = align2(r.w[i + 1], r.w[i], 2), q1 = r.w[9 + i];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                a0 = fmaf(float(int(int8_t(q0 >> (8 * k)))), x[4 * i + k], a0);
                a1 = fmaf(float(int(int8_t(q1 >> (8 * k)))), x[32 + 4 * i + k], a1);
            }
        }
        return a0 * d0 + a1 * d1;
    }
    struct XRow {  // inputs from a row vector
        const float *p;
        VH_DEV float operator[](int i) const { return p[i]; }
    };
    static VH_DEV XRow xrow(const float *x, int it) { return XRow{x + 64 * it}; }
    static VH_DEV int col(int it, int i) { return 64 * it + i; }
};

template <>
struct Split<VT_Q4_K> {  // 16-aligned super-blocks
    static constexpr int NW = 32;
    struct Raw { uint4 hdr, q; };
    static VH_DEV int col0(int it) { const int sb = it >> 3, r = it & 7; return 256 * sb + 64 * (r >> 1) + 16 * (r & 1); }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        const int sb = it >> 3, r = it & 7;
        P p = base + row + 144 * sb;
        Raw w;
        w.hdr = ld_u128(p);
        w.q = ld_u128(p + 16 + 32 * (r >> 1) + 16 * (r & 1));
        return w;
    }
    // sl, sh: sums of the low-run and high-run inputs
    template <class X>
    static VH_DEV float compute(const Raw &r, int it, const X &x, float sl, float sh) {
        const int c = (it & 7) >> 1;
        const float d = h2f(r.hdr.x & 0xffffu), dmin = h2f(r.hdr.x >> 16);
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, r.hdr.y, r.hdr.z, r.hdr.w, sc0, m0);
        q4k_scale_min(2 * c + 1, r.hdr.y, r.hdr.z, r.hdr.w, sc1, m1);
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float dl = 0.0f, dh = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t lo = qw[i] & 0x0f0f0f0fu, hi = (qw[i] >> 4) & 0x0f0f0f0fu;
            // keep the masked words as they are, so each byte below converts with
            // one v_cvt_f32_ubyte{0..3} (otherwise the masks fold into bitfield
            // extracts and every quant costs an extra instruction)
            asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
            for (int k = 0; k < 4; k++) {
                dl = fmaf(float((lo >> (8 * k)) & 0xffu), x[4 * i + k], dl);
                dh = fmaf(float((hi >> (8 * k)) & 0xffu), x[16 + 4 * i + k], dh);
            }
        }
        return (d * float(sc0)) * dl - (dmin * float(m0)) * sl + (d * float(sc1)) * dh - (dmin * float(m1)) * sh;
    }
    template <class X>
    static VH_DEV float compute(const Raw &r, int it, const X &x) {
        float sl = 0.0f, sh = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) { sl += x[i]; sh += x[16 + i]; }
        return compute(r, it, x, sl, sh);
    }
    struct XRow {
        const float *p;
        VH_DEV float operator[](int i) const { return p[i < 16 ? i : i + 16]; }
    };
    static VH_DEV XRow xrow(const float *x, int it) { return XRow{x + col0(it)}; }
    static VH_DEV int col(int it, int i) { return col0(it) + (i < 16 ? i : i + 16); }
};

template <>
struct Split<VT_Q6_K> {  // even-offset super-blocks
    static constexpr int NW = 32;
    using Raw = Q6Raw;
    static VH_DEV int col0(int it) { const int sb = it >> 3, r = it & 7; return 256 * sb + 128 * (r >> 2) + 8 * (r & 3); }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        const int sb = it >> 3, r = it & 7;
        return q6k_fetch(base, row + 210 * sb, r >> 2, r & 3);
    }
    template <class X>
    static VH_DEV float compute(const Raw &r, int, const X &x) { return q6k_compute(r, x); }
    struct XRow {
        const float *p;
        VH_DEV float operator[](int i) const { return p[32 * (i >> 3) + (i & 7)]; }
    };
    static VH_DEV XRow xrow(const float *x, int it) { return XRow{x + col0(it)}; }
    static VH_DEV int col(int it, int i) { return col0(it) + 32 * (i >> 3) + (i & 7); }
};

// Inputs from a row held in LDS with one pad float after every 32 (element c
// at c + c/32), which spreads the items that a wave reads at once over
// different banks.
template <int T>
struct XPadded {
    const float *p;
    int it;
    VH_DEV float operator[](int i) const {
        const int c = Split<T>::col(it, i);
        return p[c + (c >> 5)];
    }
};
VH_DEV int padded_len(int n) { return n + (n >> 5); }

// ---------------------------------------------------------------- register-resident inputs
// Decoders for kernels that keep an item's 32 inputs in registers (x[32], in the
// item's own order as above) together with sums of runs of those inputs, so
// per-run constants (Q4_K mins, the Q6_K offset of 32) are applied once per run
// instead of once per weight:
//   Q4_K  sums[0] = x[0..15], sums[1] = x[16..31] (the low- and high-nibble runs)
//   Q6_K  sums[g] = x[8g .. 8g+7]
//   Q8_0  no sums (an unpaired 34-byte block at an even offset)
template <int T>
struct Reg;

// float4 loads of an item's inputs from a row vector; runs of R columns, RS apart.
template <int RUNS, int R, int RS>
VH_DEV void load_runs(const float *__restrict__ p, float (&x)[32]) {
#pragma unroll
    for (int g = 0; g < RUNS; g++)
#pragma unroll
        for (int i = 0; i < R / 4; i++) {
            const float4 v = *reinterpret_cast<const float4 *>(p + g * RS + 4 * i);
            x[g * R + 4 * i + 0] = v.x;
            x[g * R + 4 * i + 1] = v.y;
            x[g * R + 4 * i + 2] = v.z;
            x[g * R + 4 * i + 3] = v.w;
        }
}

template <>
struct Reg<VT_Q4_K> {
    static constexpr int NS = 2;
    using Raw = Split<VT_Q4_K>::Raw;  // two 16-byte loads: nothing to resolve
    using Words = Raw;
    static VH_DEV const Words &resolve(const Raw &r, int) { return r; }
    static __host__ __device__ int items(int n) { return n / 32; }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) { return Split<VT_Q4_K>::fetch(base, row, it); }
    static VH_DEV void load_x(const float *row, int it, float (&x)[32]) {
        load_runs<2, 16, 32>(row + Split<VT_Q4_K>::col0(it), x);
    }
    static VH_DEV void sums(const float (&x)[32], float (&s)[NS]) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) { a += x[i]; b += x[16 + i]; }
        s[0] = a;
        s[1] = b;
    }
    static VH_DEV float compute(const Raw &r, int it, const float (&x)[32], const float (&s)[NS]) {
        return Split<VT_Q4_K>::compute(r, it, x, s[0], s[1]);
    }
};

// Q6_K: the four runs' 6-bit quants are assembled four to a word (one per byte)
// and converted with v_cvt_f32_ubyte*; sum_i (q_i - 32) x_i is formed as
// sum_i q_i x_i - 32 sum_i x_i.
VH_DEV float q6k_compute_s(const Q6Raw &r, const float (&x)[32], const float (&sx)[4]) {
    uint32_t t[4][2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t A = h ? r.a1 : r.a0, B = h ? r.b1 : r.b0, H = h ? r.h1 : r.h0;
        t[0][h] = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
        t[1][h] = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
        t[2][h] = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
        t[3][h] = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
    }
    asm volatile("" : "+v"(t[0][0]), "+v"(t[0][1]), "+v"(t[1][0]), "+v"(t[1][1]), "+v"(t[2][0]), "+v"(t[2][1]),
                 "+v"(t[3][0]), "+v"(t[3][1]));
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) acc = fmaf(float((t[g][i >> 2] >> (8 * (i & 3))) & 0xffu), x[8 * g + i], acc);
        s = fmaf(float(int(int8_t(r.sc >> (8 * g)))), fmaf(-32.0f, sx[g], acc), s);
    }
    return h2f(r.d) * s;
}

template <>
struct Reg<VT_Q6_K> {
    static constexpr int NS = 4;
    using Raw = Q6Win;
    using Words = Q6Raw;
    static __host__ __device__ int items(int n) { return n / 32; }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        const int sb = it >> 3, r = it & 7;
        return q6k_fetch_raw(base, row + 210 * sb, r >> 2, r & 3);
    }
    static VH_DEV Words resolve(const Raw &r, int it) { return q6k_resolve(r, it & 3); }
    static VH_DEV void load_x(const float *row, int it, float (&x)[32]) {
        load_runs<4, 8, 32>(row + Split<VT_Q6_K>::col0(it), x);
    }
    static VH_DEV void sums(const float (&x)[32], float (&s)[NS]) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) a += x[8 * g + i];
            s[g] = a;
        }
    }
    static VH_DEV float compute(const Raw &r, int it, const float (&x)[32], const float (&s)[NS]) {
        return q6k_compute_s(resolve(r, it), x, s);
    }
};

template <>
struct Reg<VT_Q8_0> {
    static constexpr int NS = 1;
    struct Raw { uint32_t w[8], lo, hi, s; };
    struct Words { uint32_t w[9], s; };
    static __host__ __device__ int items(int n) { return n / 32; }
    // block it of the row at byte offset row (even): the aligned window from
    // the dword holding its first byte, its first 32 bytes as two 16-byte
    // loads (4-aligned: the Q6_K windows' 12-byte loads take the same). Its
    // last word is two 16-bit loads, at a + 32 and at a + 32 + s (the same
    // halfword when the block starts 4-aligned), so nothing past the block is
    // read and no load depends on another: four load instructions per block.
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        const int64_t b = row + 34 * int64_t(it);
        Raw r;
        r.s = uint32_t(b) & 3u;
        P a = base + (b - int64_t(r.s));
        const uint4 v0 = ld_u128(a), v1 = ld_u128(a + 16);
        r.w[0] = v0.x;
        r.w[1] = v0.y;
        r.w[2] = v0.z;
        r.w[3] = v0.w;
        r.w[4] = v1.x;
        r.w[5] = v1.y;
        r.w[6] = v1.z;
        r.w[7] = v1.w;
        r.lo = ld_u16(a + 32);
        r.hi = ld_u16(a + 32 + r.s);
        return r;
    }
    static VH_DEV Words resolve(const Raw &r, int) {
        Words v;
#pragma unroll
        for (int i = 0; i < 8; i++) v.w[i] = r.w[i];
        v.w[8] = r.lo | (r.hi << 16);  // the high half is not read when s == 0
        v.s = r.s;
        return v;
    }
    static VH_DEV void load_x(const float *row, int it, float (&x)[32]) { load_runs<1, 32, 32>(row + 32 * it, x); }
    static VH_DEV void sums(const float (&)[32], float (&s)[NS]) { s[0] = 0.0f; }
    static VH_DEV float compute(const Raw &raw, int it, const float (&x)[32], const float (&)[NS]) {
        const Words r = resolve(raw, it);
        const float d = h2f((r.w[0] >> (8 * r.s)) & 0xffffu);
        const uint32_t sh = 16 + 8 * r.s;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = uint32_t(((uint64_t(r.w[i + 1]) << 32) | r.w[i]) >> sh);
#pragma unroll
            for (int k = 0; k < 4; k++) acc = fmaf(float(int(int8_t(q >> (8 * k)))), x[4 * i + k], acc);
        }
        return acc * d;
    }
};

// Expert rows of the other types the reference computes with gguf_matmul
// (src/gguf_compute.c:68-82 Q5_0 by dequant-then-dot, :202-213 F16 / F32), for
// the grouped projections: a 32-weight item's words (fetch), resolved into
// the block's own bytes (resolve); the grouped kernels dequantize them with
// deq_raw. Items are 32 consecutive columns.
//   Q5_0 {f16 d; u8 qh[4]; u8 qs[16]} = 22 bytes: the block at an even offset
//        b is read as the aligned 24-byte window from b - (b & 3) - five dwords
//        and a last word of two 16-bit loads, as Reg<VT_Q8_0> does, so nothing
//        past the block is read;
//   F16  64 bytes, F32 128 bytes per item (rows of n % 32 == 0 elements).
template <>
struct Reg<VT_Q5_0> {
    struct Raw { uint32_t w[5], lo, hi, s; };
    struct Words { uint32_t b[6]; };  // block bytes [0, 24): bytes 22 and 23 unused
    static __host__ __device__ int items(int n) { return n / 32; }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        const int64_t b = row + 22 * int64_t(it);
        Raw r;
        r.s = uint32_t(b) & 3u;
        P a = base + (b - int64_t(r.s));
#pragma unroll
        for (int i = 0; i < 5; i++) r.w[i] = ld_u32(a + 4 * i);
        r.lo = ld_u16(a + 20);
        r.hi = ld_u16(a + 20 + r.s);
        return r;
    }
    static VH_DEV Words resolve(const Raw &r, int) {
        const uint32_t win[6] = {r.w[0], r.w[1], r.w[2], r.w[3], r.w[4], r.lo | (r.hi << 16)};
        Words v;
#pragma unroll
        for (int i = 0; i < 5; i++) v.b[i] = align2(win[i + 1], win[i], r.s);
        v.b[5] = r.s ? (win[5] >> 16) : win[5];
        return v;
    }
};
template <>
struct Reg<VT_F16> {
    struct Raw { uint4 q[4]; };
    using Words = Raw;
    static __host__ __device__ int items(int n) { return n / 32; }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        Raw r;
#pragma unroll
        for (int i = 0; i < 4; i++) r.q[i] = ld_u128(base + row + 64 * int64_t(it) + 16 * i);
        return r;
    }
    static VH_DEV const Words &resolve(const Raw &r, int) { return r; }
};
template <>
struct Reg<VT_F32> {
    struct Raw { uint4 q[8]; };
    using Words = Raw;
    static __host__ __device__ int items(int n) { return n / 32; }
    template <class P>
    static VH_DEV Raw fetch(P base, int64_t row, int it) {
        Raw r;
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = ld_u128(base + row + 128 * int64_t(it) + 16 * i);
        return r;
    }
    static VH_DEV const Words &resolve(const Raw &r, int) { return r; }
};
