// Shared device helpers for the vireo-hip kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <errno.h>
#include <stdint.h>

#define VH_DEV __device__ __forceinline__

// Events on which the next launch records its own begin and end (taken from
// the dispatch itself by hipExtLaunchKernelGGL). Both are null except while
// moe_decode_stage_timed times a launch.
struct VhLaunchTiming {
    hipEvent_t start, stop;
};
extern VhLaunchTiming g_vh_timing;
#define VH_LAUNCH(K, G, B, SH, ST, ...) \
    hipExtLaunchKernelGGL(K, G, B, SH, ST, g_vh_timing.start, g_vh_timing.stop, 0, __VA_ARGS__)

enum { VT_F32 = 0, VT_F16 = 1, VT_Q4_0 = 2, VT_Q5_0 = 6, VT_Q8_0 = 8, VT_Q4_K = 12, VT_Q6_K = 14 };

// ---- phase timestamps ----------------------------------------------------------
// The one-token decode kernels can record when each workgroup reaches each of
// its phases: wave 0 reads s_memrealtime (the device's 100 MHz clock, the
// same on every CU) and thread 0 stores up to kStampSlots stamps per
// workgroup at stamps[workgroup * kStampSlots + slot], for the first
// kStampBlocks workgroups. The stamped kernels are separate instantiations
// (PhaseStamps<true>), launched only while stamps are being recorded: a
// runtime branch per stamp in the production kernels cost 0.5 us per layer. g_vh_stamps is where the launches being issued record:
// kernel i of a layer call at g_vh_stamps + i * kStampBlocks * kStampSlots;
// null except inside moe_decode_phases.
constexpr int kStampSlots = 8, kStampBlocks = 256, kStampKernels = 3;
extern uint64_t *g_vh_stamps;
inline uint64_t *vh_stamps_for(int kernel) {
    return g_vh_stamps ? g_vh_stamps + size_t(kernel) * kStampBlocks * kStampSlots : nullptr;
}
template <bool ON>
struct PhaseStamps {  // ON: the launch's stamps buffer (vh_stamps_for) is set; off, every call compiles to nothing
    uint64_t *out;
    uint64_t t[ON ? kStampSlots : 1];
    __device__ explicit PhaseStamps(uint64_t *o) : out(o) {
        if constexpr (ON)
            for (int i = 0; i < kStampSlots; i++) t[i] = 0;
    }
    __device__ __forceinline__ void now(int i) {
        if constexpr (ON) t[i] = __builtin_amdgcn_s_memrealtime();
    }
    // the stamp after v is available (the wait for a load that produces v comes first)
    template <class V>
    __device__ __forceinline__ void after(int i, V v) {
        if constexpr (ON) {
            asm volatile("" ::"v"(v));
            t[i] = __builtin_amdgcn_s_memrealtime();
        }
    }
    __device__ __forceinline__ void mark(int i, uint64_t v) {
        if constexpr (ON) t[i] = v;
    }
    __device__ __forceinline__ void store() {
        if constexpr (ON) {
            const int b = int(blockIdx.y * gridDim.x + blockIdx.x);
            if (threadIdx.x == 0 && b < kStampBlocks)
                for (int i = 0; i < kStampSlots; i++) out[size_t(b) * kStampSlots + i] = t[i];
        }
    }
};

// ---- host-side helpers ------------------------------------------------------
int vh_check(hipError_t e);            // hipSuccess -> 0, else records the error and returns -EIO
int vh_finish(hipStream_t s, int rc);  // synchronise when the caller passed no stream
int vh_device_workspace(size_t bytes, void **out);  // per-device scratch, grown on demand
int vh_counters(int n, unsigned **out);              // per-device zeroed counters (self-resetting use)
int vh_reduce_scratch(size_t bytes, void **out);     // per-device scratch for reduction partials
int vh_num_cus();
// The per-device stream that expert page-in copies run on (created on first use).
int vh_copy_stream(hipStream_t *out);
// Pinned host memory for small per-call transfers (grow-only, per device; two
// buffers taken in turn, so a call does not wait for the one just before it).
// A call that takes a buffer first waits until the copies of the last call
// that used that buffer have run (the event vh_host_staging_done recorded on
// that call's stream).
int vh_host_staging(size_t bytes, void **out);
int vh_host_staging_done(hipStream_t s);
// Sticky per-device status bits that kernels with grid-wide waits set when a
// wait gives up (VIREO_DECODE_TIMEOUT), the poll limit of such waits
// (vireo_hip_set_spin_limit), and a read-and-clear after the stream's work.
int vh_status_word(uint32_t **out);
unsigned vh_spin_limit();
int vh_take_status(hipStream_t s);
// This device's address of moe_ffn_forward_noalloc's static scratch (moe.hip),
// looked up once per device; out may be NULL.
int vh_noalloc_setup(void **out);
// bytes of a row of n weights of ggml type t (src/gguf.c:27-38; F32 otherwise)
inline int64_t vh_row_bytes(uint32_t t, int n) {
    switch (t) {
    case VT_Q8_0: return int64_t(n / 32) * 34;
    case VT_Q4_K: return int64_t(n / 256) * 144;
    case VT_Q6_K: return int64_t(n / 256) * 210;
    case VT_Q5_0: return int64_t(n / 32) * 22;
    case VT_F16: return int64_t(n) * 2;
    default: return int64_t(n) * 4;
    }
}

// ---- loads ------------------------------------------------------------------
// All quantized rows used here are made of 2-byte units and start 4-byte
// aligned, so any field starts at an address that is 0 or 2 mod 4. Fields are
// read with naturally aligned dword loads of a window that never leaves the
// field's own block, then shifted into place with v_alignbyte_b32.
VH_DEV uint32_t ld_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
VH_DEV uint32_t ld_u16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }
VH_DEV uint32_t ld_u8(const uint8_t *p) { return *p; }

// Global-memory views of pointers the compiler cannot trace to a kernel
// argument (expert tables hold generic pointers): loads through them are
// global_load, not flat_load, which would also count against the LDS wait
// counter and make every LDS wait drain the weight prefetches.
typedef const __attribute__((address_space(1))) uint8_t gbyte;
VH_DEV gbyte *gmem(const void *p) { return (gbyte *)p; }
template <class V>
VH_DEV V ldg(gbyte *p) { return *(const __attribute__((address_space(1))) V *)p; }  // scalar or ext_vector V
VH_DEV uint32_t ld_u32(gbyte *p) { return ldg<uint32_t>(p); }
VH_DEV uint32_t ld_u16(gbyte *p) { return ldg<uint16_t>(p); }
VH_DEV uint32_t ld_u8(gbyte *p) { return *p; }
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
VH_DEV u32x3 ld_u96(gbyte *p) { return ldg<u32x3>(p); }
// the same loads through generic pointers (tensors in LDS or traced to an argument)
VH_DEV uint4 ld_u128(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
VH_DEV u32x3 ld_u96(const uint8_t *p) { return *reinterpret_cast<const u32x3 *>(p); }
VH_DEV uint2 ld_u64(gbyte *p) {
    const u32x2 v = ldg<u32x2>(p);
    return make_uint2(v.x, v.y);
}
VH_DEV uint4 ld_u128(gbyte *p) {
    const u32x4 v = ldg<u32x4>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// Global loads with the non-temporal hint, for weights a call streams once:
// measured on MI355X, streaming 24 MB of weights this way between reads of a
// 1 MB router keeps the router in the memory-side Infinity Cache (its read
// 4.4 -> 2.9 us), where ordinary loads let the weights evict it. The same
// fetch code takes an NtPtr where it takes a gbyte pointer.
struct NtPtr {
    gbyte *p;
    VH_DEV NtPtr operator+(int64_t o) const { return NtPtr{p + o}; }
    VH_DEV NtPtr operator-(int64_t o) const { return NtPtr{p - o}; }
};
VH_DEV NtPtr ntmem(const void *p) { return NtPtr{gmem(p)}; }
template <class V>
VH_DEV V ldnt(NtPtr a) { return __builtin_nontemporal_load((const __attribute__((address_space(1))) V *)a.p); }
VH_DEV uint32_t ld_u32(NtPtr a) { return ldnt<uint32_t>(a); }
VH_DEV uint32_t ld_u16(NtPtr a) { return ldnt<uint16_t>(a); }
VH_DEV u32x3 ld_u96(NtPtr a) { return ldnt<u32x3>(a); }
VH_DEV uint2 ld_u64(NtPtr a) {
    const u32x2 v = ldnt<u32x2>(a);
    return make_uint2(v.x, v.y);
}
VH_DEV uint4 ld_u128(NtPtr a) {
    const u32x4 v = ldnt<u32x4>(a);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// bytes [b, b + 4) of the 8-byte value hi:lo, b in 0..3 (v_alignbyte takes b mod 4)
VH_DEV uint32_t align2(uint32_t hi, uint32_t lo, uint32_t bytes) { return __builtin_amdgcn_alignbyte(hi, lo, bytes); }

// ---- binary16 -> binary32 (exact; v_cvt_f32_f16) --------------------------------
VH_DEV float h2f(uint32_t h) {
    _Float16 v;
    uint16_t b = uint16_t(h);
    __builtin_memcpy(&v, &b, 2);
    return float(v);
}

// 12 bytes at byte offset off (even) of a 4-aligned base, as three dwords:
// one aligned dwordx3 load of [off&~3, (off&~3)+12), shifted into place. The
// first two words hold bytes [off, off+8); callers keep the window in bounds.
template <class P>
VH_DEV void ld12_even(P base, int off, uint32_t &w0, uint32_t &w1) {
    const uint32_t s = uint32_t(off) & 3u;
    const u32x3 v = ld_u96(base + (off - int(s)));
    w0 = align2(v.y, v.x, s);
    w1 = align2(v.z, v.y, s);
}

// ---- wave reductions (DPP, fixed order) --------------------------------------------
// dpp_ctrl values (GFX9 DPP): quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] =
// 0x4E, row_half_mirror = 0x141, row_mirror = 0x140, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf>
VH_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
VH_DEV uint32_t dpp_u(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, ROW_MASK, 0xf, false));
}
// A workgroup barrier that orders LDS only: it waits for this wave's LDS
// operations, not for its global loads in flight (__syncthreads waits for
// those too), so loads issued before it keep streaming across it.
// s_waitcnt for vmcnt <= n, the other counters left as they are (gfx9 encoding)
#define VH_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
// A workgroup barrier that waits for nothing itself. The fence of
// __syncthreads (and of a local-only fence) makes the compiler drain every
// direct-to-LDS load first, prefetches included; callers of this one have
// waited for the loads the next step reads (VH_WAIT_VMCNT) and consumed the
// LDS values read before it. The memory clobber keeps the compiler from
// moving LDS accesses across it.
VH_DEV void dma_barrier() { asm volatile("s_barrier" ::: "memory"); }
typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gvoid;
VH_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Sum over aligned groups of L lanes (L a power of two <= 64). The total is in
// the last lane of each group (lane % L == L-1); for L <= 16 every lane of the
// group holds it. Must be called with all 64 lanes active.
template <int L>
VH_DEV float group_sum(float v) {
    if constexpr (L >= 2) v += dpp_f<0xB1>(v);
    if constexpr (L >= 4) v += dpp_f<0x4E>(v);
    if constexpr (L >= 8) v += dpp_f<0x141>(v);
    if constexpr (L >= 16) v += dpp_f<0x140>(v);
    if constexpr (L >= 32) v += dpp_f<0x142, 0xA>(v);
    if constexpr (L >= 64) v += dpp_f<0x143, 0xC>(v);
    return v;
}
template <int CTRL, int ROW_MASK = 0xf>
VH_DEV float dpp_keep(float v) {  // rows outside ROW_MASK read their own value
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
// Wave-wide max of floats, returned on every lane.
VH_DEV float wave_max_f(float v) {
    v = fmaxf(v, dpp_keep<0xB1>(v));
    v = fmaxf(v, dpp_keep<0x4E>(v));
    v = fmaxf(v, dpp_keep<0x141>(v));
    v = fmaxf(v, dpp_keep<0x140>(v));
    v = fmaxf(v, dpp_keep<0x142, 0xA>(v));
    v = fmaxf(v, dpp_keep<0x143, 0xC>(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Wave-wide sum / unsigned max, returned on every lane (readlane of lane 63).
VH_DEV float wave_sum_f(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_sum<64>(v)), 63)); }
VH_DEV uint32_t wave_max_u(uint32_t v) {
    v = max(v, dpp_u<0xB1>(v));
    v = max(v, dpp_u<0x4E>(v));
    v = max(v, dpp_u<0x141>(v));
    v = max(v, dpp_u<0x140>(v));
    v = max(v, dpp_u<0x142, 0xA>(v));
    v = max(v, dpp_u<0x143, 0xC>(v));
    return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}
VH_DEV double readlane_d(double v, int lane) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), lane));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), lane));
    return __longlong_as_double(int64_t((uint64_t(hi) << 32) | lo));
}
// DPP move of a double (two 32-bit halves); lanes without a source read 0.
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = false>
VH_DEV double dpp_d(double v) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(b)), CTRL, ROW_MASK, 0xf, BOUND_ZERO));
    const uint32_t hi = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(b >> 32)), CTRL, ROW_MASK, 0xf, BOUND_ZERO));
    return __longlong_as_double(int64_t((uint64_t(hi) << 32) | lo));
}
// Wave-wide fp64 sum (fixed tree), returned on every lane.
VH_DEV double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    v += dpp_d<0x142, 0xA>(v);
    v += dpp_d<0x143, 0xC>(v);
    return readlane_d(v, 63);
}
// Inclusive fp64 prefix sum over the 64 lanes (Hillis-Steele inside each
// 16-lane row with row_shr 1/2/4/8, then the row totals carried forward with
// row_bcast 15/31).
VH_DEV double wave_incl_scan_d(double v) {
    v += dpp_d<0x111, 0xf, true>(v);
    v += dpp_d<0x112, 0xf, true>(v);
    v += dpp_d<0x114, 0xf, true>(v);
    v += dpp_d<0x118, 0xf, true>(v);
    v += dpp_d<0x142, 0xA>(v);
    v += dpp_d<0x143, 0xC>(v);
    return v;
}

// ---- fp32 operations rounded one at a time ---------------------------------------
// The reference's C arithmetic rounds every product and every sum. HIP's
// __fmul_rn / __fadd_rn are plain * and +, which the compiler fuses into one
// fma (one rounding) under its default contraction; these never fuse.
VH_DEV float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
VH_DEV float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
VH_DEV float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// ---- SwiGLU gate: silu(g) * u, as src/gguf_run.c:207 -----------------------------
VH_DEV float swiglu(float g, float u) { return (g / (1.0f + expf(-g))) * u; }
