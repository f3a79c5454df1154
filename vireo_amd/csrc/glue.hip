// Model glue around the MoE layers: rmsnorm (src/gguf_run.c:161-165) and
// argmax (src/gguf_run.c:254).
#include <hip/hip_runtime.h>
#include "common.h"
#include "vireo_hip.h"

namespace {

// One workgroup per row. The sum of squares is reduced in fp64 and rounded
// once, so it is the correctly rounded value of the exact sum; the reference
// adds in fp32 sequentially, which is within n*2^-24 relative of it.
__global__ void __launch_bounds__(256) rmsnorm_kernel(float *o, const float *x,
                                                      const float *__restrict__ w, int n, float eps) {
    __shared__ double part[4];
    const size_t row = blockIdx.x;
    const float *xr = x + row * n;
    float *orow = o + row * n;
    double acc = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        acc += double(__fmul_rn(v, v));
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float ss = float((part[0] + part[1]) + (part[2] + part[3]));
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, float(n)), eps)));
    for (int i = threadIdx.x; i < n; i += 256) orow[i] = __fmul_rn(__fmul_rn(xr[i], r), w[i]);
}

__global__ void __launch_bounds__(1024) argmax_kernel(const float *__restrict__ v, int n, int32_t *__restrict__ out) {
    __shared__ float bvs[16];
    __shared__ int bis[16];
    float bv = v[0];
    int bi = 0;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float c = v[i];
        if (c > bv || (c == bv && i < bi)) { bv = c; bi = i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bvs[threadIdx.x >> 6] = bv; bis[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int wv = 1; wv < 16; wv++)
            if (bvs[wv] > bv || (bvs[wv] == bv && bis[wv] < bi)) { bv = bvs[wv]; bi = bis[wv]; }
        // the reference scans upward with a strict '>' from v[0]: the first maximum
        *out = bi;
    }
}

}  // namespace

extern "C" int vireo_rmsnorm(float *o, const float *x, const float *w, int n, int rows, float eps, void *stream) {
    if (n <= 0 || rows < 0 || (rows && (!o || !x || !w))) return -EINVAL;
    if (rows == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, o, x, w, n, eps);
    return vh_finish(s, vh_check(hipGetLastError()));
}

extern "C" int vireo_argmax(const float *v, int n, int32_t *out, void *stream) {
    if (n <= 0 || !v || !out) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, v, n, out);
    return vh_finish(s, vh_check(hipGetLastError()));
}
