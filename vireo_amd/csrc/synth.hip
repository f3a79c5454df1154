// Synthetic weights and hidden states for the MoE-FFN workloads (declared in
// include/vireo_synth.h). Host and device share every function below, compiled
// with contraction off, and use only correctly rounded fp64 operations (+, -,
// *, /, conversions), so both produce identical bytes.
#include <hip/hip_runtime.h>
#include <errno.h>
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <thread>
#include <vector>
#include "vireo_synth.h"

#pragma clang fp contract(off)

#define VS __host__ __device__ static inline

namespace {

enum { T_F32 = 0, T_F16 = 1, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

// ---- counter-based random bits (SplitMix64 finaliser) ----
VS uint64_t mix64(uint64_t z) {
    z ^= z >> 30; z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27; z *= 0x94d049bb133111ebULL;
    z ^= z >> 31;
    return z;
}
VS uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(seed ^ mix64(stream + 0x632be59bd9b4e019ULL)); }
VS uint64_t draw_bits(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9e3779b97f4a7c15ULL); }

VS double pow2(int k) {  // exact 2^k for -1022 <= k <= 1023
    uint64_t b = (uint64_t)(k + 1023) << 52;
    double r;
    memcpy(&r, &b, 8);
    return r;
}

// ln(v) for an integer 1 <= v < 2^53: v = m * 2^e with m in [sqrt(1/2), sqrt(2)),
// ln m = 2 atanh(s), s = (m-1)/(m+1), |s| < 0.172, ten series terms.
VS double ln_int(uint64_t v) {
    int e = 63 - __builtin_clzll(v);
    double m = (double)v * pow2(-e);
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    double s = (m - 1.0) / (m + 1.0), s2 = s * s, t = s, acc = s;
    for (int k = 3; k <= 21; k += 2) { t = t * s2; acc = acc + t / (double)k; }
    return (double)e * 0.6931471805599453 + 2.0 * acc;
}

// sqrt(a), a > 0: a = m * 4^k with m in [1,4), six Newton steps from (1+m)/2.
VS double sqrt_pos(double a) {
    uint64_t b;
    memcpy(&b, &a, 8);
    int ex = (int)((b >> 52) & 0x7ff) - 1023;
    int k = (ex - (ex & 1)) / 2;
    double m = a * pow2(-2 * k), y = (1.0 + m) * 0.5;
    for (int i = 0; i < 6; i++) y = 0.5 * (y + m / y);
    return y * pow2(k);
}

// cos(2*pi*u) for u = bits / 2^32: quadrant from the top two bits, Taylor
// series of sin/cos on [0, pi/2) through degree 21/20.
VS double cos_turn(uint32_t bits) {
    uint32_t q = bits >> 30;
    double th = (double)(bits & 0x3fffffffu) * pow2(-30) * 1.5707963267948966;
    double t2 = th * th;
    double c = 1.0, s = 1.0, tc = 1.0, ts = 1.0;
    for (int j = 1; j <= 10; j++) {
        tc = -tc * t2 / (double)((2 * j - 1) * (2 * j));
        ts = -ts * t2 / (double)((2 * j) * (2 * j + 1));
        c = c + tc;
        s = s + ts;
    }
    s = s * th;
    return q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
}

// Box-Muller: z = sqrt(-2 ln u1) cos(2 pi u2), u1 = (2h+1)/2^33 in (0,1).
VS float normal_at(uint64_t key, uint64_t i, float sigma) {
    uint64_t r = draw_bits(key, i);
    uint64_t v = 2 * (r >> 32) + 1;
    double a = -2.0 * (ln_int(v) - 33.0 * 0.6931471805599453);
    double rad = a > 0.0 ? sqrt_pos(a) : 0.0;
    return (float)((double)sigma * (rad * cos_turn((uint32_t)r)));
}

// ---- binary16 ----
VS float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 31u, man = h & 1023u, bits;
    float f;
    if (ex == 31u) bits = sign | 0x7f800000u | (man << 13);
    else if (ex) bits = sign | ((ex + 112u) << 23) | (man << 13);
    else { f = (float)man * 5.9604644775390625e-08f; memcpy(&bits, &f, 4); bits |= sign; }
    memcpy(&f, &bits, 4);
    return f;
}
// round-to-nearest-even float -> binary16
VS uint16_t f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t r = ax - (112u << 23);
        r = r + 0xfffu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    uint32_t e = ax >> 23;
    if (e == 0u) return (uint16_t)sign;
    int shift = 126 - (int)e;
    if (shift > 24) return (uint16_t)sign;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u, q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

VS int round_half_away(double v) { return v >= 0.0 ? (int)(v + 0.5) : -(int)(-v + 0.5); }
VS int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
VS double absd(double v) { return v < 0.0 ? -v : v; }
VS void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)(v & 0xff); p[1] = (uint8_t)(v >> 8); }

// ---- block quantizers: x holds one block's floats, out its bytes ----
VS void quant_q8_0(const float *x, uint8_t *out) {
    double amax = 0.0;
    for (int i = 0; i < 32; i++) { double a = absd(x[i]); if (a > amax) amax = a; }
    uint16_t dh = f2h((float)(amax / 127.0));
    double dq = h2f(dh), id = dq > 0.0 ? 1.0 / dq : 0.0;
    put16(out, dh);
    for (int i = 0; i < 32; i++) out[2 + i] = (uint8_t)(int8_t)clampi(round_half_away((double)x[i] * id), -127, 127);
}

// Q4_K: per 32-element sub-block an affine map y = (d*sc)*q - dmin*m with
// q in [0,15] and 6-bit sc, m; packing is the inverse of the reference's
// scale/min unpack (src/gguf_compute.c:45-51).
VS void quant_q4_k(const float *x, uint8_t *out) {
    double scale[8], negmin[8], smax = 0.0, mmax = 0.0;
    for (int j = 0; j < 8; j++) {
        double lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; l++) { double v = x[32 * j + l]; if (v < lo) lo = v; if (v > hi) hi = v; }
        if (lo > 0.0) lo = 0.0;
        scale[j] = (hi - lo) / 15.0;
        negmin[j] = -lo;
        if (scale[j] > smax) smax = scale[j];
        if (negmin[j] > mmax) mmax = negmin[j];
    }
    uint16_t dh = f2h((float)(smax / 63.0)), mh = f2h((float)(mmax / 63.0));
    double dq = h2f(dh), mq = h2f(mh);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = dq > 0.0 ? clampi(round_half_away(scale[j] / dq), 0, 63) : 0;
        mn[j] = mq > 0.0 ? clampi(round_half_away(negmin[j] / mq), 0, 63) : 0;
    }
    put16(out, dh);
    put16(out + 2, mh);
    uint8_t *s = out + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        double d1 = dq * (double)sc[j], m1 = mq * (double)mn[j];
        for (int l = 0; l < 32; l++)
            q[32 * j + l] = (uint8_t)(d1 > 0.0 ? clampi(round_half_away(((double)x[32 * j + l] + m1) / d1), 0, 15) : 0);
    }
    uint8_t *qs = out + 16;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

// Q6_K: 16 groups of 16 consecutive elements, each with an int8 scale under
// one f16 d; q in [-32,31] stored as q+32 split into a nibble (ql) and two bits
// (qh) at the positions the reference dequant reads (src/gguf_compute.c:83-103).
VS void quant_q6_k(const float *x, uint8_t *out) {
    double gs[16], smax = 0.0;
    for (int g = 0; g < 16; g++) {
        double amax = 0.0;
        for (int l = 0; l < 16; l++) { double a = absd(x[16 * g + l]); if (a > amax) amax = a; }
        gs[g] = amax / 31.0;
        if (gs[g] > smax) smax = gs[g];
    }
    uint16_t dh = f2h((float)(smax / 127.0));
    double dq = h2f(dh);
    int8_t sc[16];
    for (int g = 0; g < 16; g++) sc[g] = (int8_t)(dq > 0.0 ? clampi(round_half_away(gs[g] / dq), -128, 127) : 0);
    memset(out, 0, 210);
    for (int i = 0; i < 256; i++) {
        int g = i / 16;
        double step = dq * (double)sc[g];
        int q = step != 0.0 ? clampi(round_half_away((double)x[i] / step), -32, 31) : 0;
        int u = q + 32;
        int h = i >> 7, gg = (i >> 5) & 3, l = i & 31;
        int qli = 64 * h + l + 32 * (gg & 1);
        out[qli] = (uint8_t)(out[qli] | ((gg >= 2 ? (u & 15) << 4 : (u & 15))));
        out[128 + 32 * h + l] = (uint8_t)(out[128 + 32 * h + l] | ((u >> 4) << (2 * gg)));
    }
    for (int g = 0; g < 16; g++) out[192 + g] = (uint8_t)sc[g];
    put16(out + 208, dh);
}

// Q5_0: symmetric 5-bit, q in [-16,15] stored as q+16; element j<16 in the
// low nibble of qs[j], element j+16 in its high nibble, bit 4 of element j in
// bit j of qh (src/gguf_compute.c:67-82).
VS void quant_q5_0(const float *x, uint8_t *out) {
    double amax = 0.0;
    for (int i = 0; i < 32; i++) { double a = absd(x[i]); if (a > amax) amax = a; }
    uint16_t dh = f2h((float)(amax / 15.0));
    double dq = h2f(dh);
    uint32_t qh = 0;
    uint8_t *qs = out + 6;
    for (int j = 0; j < 16; j++) qs[j] = 0;
    for (int i = 0; i < 32; i++) {
        int q = dq > 0.0 ? clampi(round_half_away((double)x[i] / dq), -16, 15) : 0;
        int u = q + 16;
        if (i < 16) qs[i] = (uint8_t)(qs[i] | (u & 15));
        else qs[i - 16] = (uint8_t)(qs[i - 16] | ((u & 15) << 4));
        qh |= (uint32_t)(u >> 4) << i;
    }
    put16(out, dh);
    out[2] = (uint8_t)qh; out[3] = (uint8_t)(qh >> 8); out[4] = (uint8_t)(qh >> 16); out[5] = (uint8_t)(qh >> 24);
}

VS int block_geom(uint32_t type, int *be, int *bb) {
    switch (type) {
    case T_F32:  *be = 1;   *bb = 4;   return 0;
    case T_F16:  *be = 1;   *bb = 2;   return 0;
    case T_Q8_0: *be = 32;  *bb = 34;  return 0;
    case T_Q5_0: *be = 32;  *bb = 22;  return 0;
    case T_Q4_K: *be = 256; *bb = 144; return 0;
    case T_Q6_K: *be = 256; *bb = 210; return 0;
    default: return -1;
    }
}

VS void quant_block(uint32_t type, const float *x, uint8_t *out) {
    switch (type) {
    case T_Q8_0: quant_q8_0(x, out); break;
    case T_Q4_K: quant_q4_k(x, out); break;
    case T_Q6_K: quant_q6_k(x, out); break;
    case T_Q5_0: quant_q5_0(x, out); break;
    case T_F16: put16(out, f2h(x[0])); break;
    default: memcpy(out, x, 4); break;
    }
}

// block b of rows [first_row, first_row + rows) of a matrix with n columns:
// generate its elements and quantize them
VS void synth_block(uint32_t type, uint8_t *dst, int n, int be, int bb, int64_t first_row, int64_t b, uint64_t key,
                    float sigma) {
    float x[256];
    int64_t per_row = n / be, row = first_row + b / per_row, col0 = (b % per_row) * be;
    uint64_t first = (uint64_t)row * (uint64_t)n + (uint64_t)col0;
    for (int i = 0; i < be; i++) x[i] = normal_at(key, first + (uint64_t)i, sigma);
    quant_block(type, x, dst + b * bb);
}

__global__ void synth_matrix_kernel(uint32_t type, uint8_t *dst, int n, int be, int bb, int64_t first_row,
                                    int64_t nblocks, uint64_t key, float sigma) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b < nblocks) synth_block(type, dst, n, be, bb, first_row, b, key, sigma);
}

template <class F>
void parallel_for(int64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (n < 4096 || nt == 1) { for (int64_t i = 0; i < n; i++) f(i); return; }
    std::vector<std::thread> th;
    int64_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        int64_t lo = (int64_t)t * chunk, hi = lo + chunk < n ? lo + chunk : n;
        if (lo >= hi) break;
        th.emplace_back([=] { for (int64_t i = lo; i < hi; i++) f(i); });
    }
    for (auto &t : th) t.join();
}

}  // namespace

extern "C" int64_t vireo_row_bytes(uint32_t type, int n) {
    int be, bb;
    if (block_geom(type, &be, &bb) || n <= 0 || n % be) return -EINVAL;
    return (int64_t)(n / be) * bb;
}

extern "C" int vireo_synth_normal(float *dst, uint64_t n, uint64_t seed, uint64_t stream, uint64_t first, float sigma) {
    if (!dst && n) return -EINVAL;
    uint64_t key = stream_key(seed, stream);
    parallel_for((int64_t)n, [&](int64_t i) { dst[i] = normal_at(key, first + (uint64_t)i, sigma); });
    return 0;
}

extern "C" int vireo_quantize(uint32_t type, const float *src, void *dst, int n, int64_t rows) {
    int be, bb;
    if (block_geom(type, &be, &bb) || n <= 0 || n % be || rows < 0 || (!src && rows) || (!dst && rows)) return -EINVAL;
    int64_t nblocks = rows * (n / be);
    uint8_t *out = (uint8_t *)dst;
    parallel_for(nblocks, [&](int64_t b) { quant_block(type, src + b * be, out + b * bb); });
    return 0;
}

extern "C" int vireo_synth_matrix(uint32_t type, void *dst, int n, int64_t first_row, int64_t rows, uint64_t seed,
                                  uint64_t stream, float sigma) {
    int be, bb;
    if (block_geom(type, &be, &bb) || n <= 0 || n % be || rows < 0 || first_row < 0 || (!dst && rows)) return -EINVAL;
    uint64_t key = stream_key(seed, stream);
    int64_t nblocks = rows * (n / be);
    uint8_t *out = (uint8_t *)dst;
    parallel_for(nblocks, [&](int64_t b) { synth_block(type, out, n, be, bb, first_row, b, key, sigma); });
    return 0;
}

// x[t] = draws [t*n, t*n + n) of (seed, stream), N(0,1); hb[t] = rmsnorm(x[t])
// with unit weight, evaluated as the reference does (src/gguf_run.c:161-165):
// sequential fp32 sum of squares, r = 1/sqrtf(ss/n + eps), hb = (x*r)*1.
extern "C" int vireo_synth_hidden(float *x, float *hb, int n, int64_t tokens, uint64_t seed, uint64_t stream,
                                  float eps) {
    if (n <= 0 || tokens < 0 || (tokens && (!x || !hb))) return -EINVAL;
    uint64_t key = stream_key(seed, stream);
    parallel_for(tokens, [&](int64_t t) {
        float *xr = x + t * n, *hr = hb + t * n;
        for (int i = 0; i < n; i++) xr[i] = normal_at(key, (uint64_t)t * (uint64_t)n + (uint64_t)i, 1.0f);
        float ss = 0.0f;
        for (int i = 0; i < n; i++) ss = ss + xr[i] * xr[i];
        float r = 1.0f / sqrtf(ss / (float)n + eps);
        for (int i = 0; i < n; i++) hr[i] = (xr[i] * r) * 1.0f;
    });
    return 0;
}

extern "C" int vireo_synth_matrix_dev(uint32_t type, void *dst_dev, int n, int64_t first_row, int64_t rows,
                                      uint64_t seed, uint64_t stream, float sigma, void *hip_stream) {
    int be, bb;
    if (block_geom(type, &be, &bb) || n <= 0 || n % be || rows < 0 || first_row < 0 || (!dst_dev && rows))
        return -EINVAL;
    int64_t nblocks = rows * (n / be);
    if (!nblocks) return 0;
    const int threads = 64;
    int64_t grid = (nblocks + threads - 1) / threads;
    if (grid > 0x7fffffff) return -E2BIG;
    hipLaunchKernelGGL(synth_matrix_kernel, dim3(static_cast<unsigned>(grid)), dim3(threads), 0,
                       (hipStream_t)hip_stream, type, (uint8_t *)dst_dev, n, be, bb, first_row, nblocks,
                       stream_key(seed, stream), sigma);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -EIO;
}
