/* Synthetic inputs for the quantized MoE-FFN benchmarks and tests.
 *
 * No counterpart in the reference: it only dequantizes GGUF weights that come
 * from real models (src/gguf_compute.c) and ships no quantizer. The workloads
 * it is measured on are synthetic (N(0,0.02) weights quantized to Q8_0 / Q4_K /
 * Q6_K, N(0,1) hidden states), so this library defines how those bytes are
 * made. Host and device generators produce identical bytes: every value comes
 * from a counter-based hash of (seed, stream, index) followed by a Box-Muller
 * transform evaluated with correctly rounded fp64 operations only, and the
 * quantizers use the same operation sequence on both sides.
 *
 * All functions return 0 or a negative errno value. */
#ifndef VIREO_SYNTH_H
#define VIREO_SYNTH_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dst[i] = (float)(sigma * z) with z ~ N(0,1) the draw with index first+i of
 * stream (seed, stream). */
int vireo_synth_normal(float *dst, uint64_t n, uint64_t seed, uint64_t stream, uint64_t first, float sigma);

/* Quantize rows x n floats (row-major) to ggml `type` (Q8_0, Q4_K, Q6_K, Q5_0,
 * F16 or F32), writing rows * row_bytes(type, n) bytes. */
int vireo_quantize(uint32_t type, const float *src, void *dst, int n, int64_t rows);

/* Rows [first_row, first_row + rows) of a matrix with n columns whose element
 * (r, c) is draw r*n + c of (seed, stream) scaled by sigma, quantized to
 * `type`, on the host. A stacked expert tensor [E x rows_e x n] is one such
 * matrix, so expert e alone is first_row = e*rows_e, rows = rows_e. */
int vireo_synth_matrix(uint32_t type, void *dst, int n, int64_t first_row, int64_t rows, uint64_t seed,
                       uint64_t stream, float sigma);

/* The same bytes as vireo_synth_matrix, produced on the GPU directly into the
 * device buffer dst_dev (no fp32 copy is materialised). hip_stream may be NULL
 * (the call then only enqueues on the default stream). */
int vireo_synth_matrix_dev(uint32_t type, void *dst_dev, int n, int64_t first_row, int64_t rows, uint64_t seed,
                           uint64_t stream, float sigma, void *hip_stream);

/* Hidden states for `tokens` tokens: x[t] = N(0,1) draws [t*n, t*n+n) of
 * (seed, stream), and hb[t] = x[t] RMSNorm'd with unit weight, computed with
 * the reference's formula and fp32 operation order (src/gguf_run.c:161-165). */
int vireo_synth_hidden(float *x, float *hb, int n, int64_t tokens, uint64_t seed, uint64_t stream, float eps);

/* Bytes per row of n elements for ggml `type` (src/gguf.c:27-38 block sizes),
 * or -EINVAL. */
int64_t vireo_row_bytes(uint32_t type, int n);

#ifdef __cplusplus
}
#endif
#endif
