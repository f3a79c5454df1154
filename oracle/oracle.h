/* CPU oracle for vireo's quantized MoE-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; it is never linked into, loaded by or called from the
 * product library. Only tests/, the smoke check and the CPU-baseline leg of
 * the benchmark may use it.
 *
 * It restates, in plain C with the same floating-point operation order, the
 * reference's CPU path:
 *   src/gguf_compute.c      f16 -> f32, row dequant, gguf_matmul
 *   src/gguf.c:27-38        block sizes
 *   src/gguf_run.c:161-165  rmsnorm
 *   src/gguf_run.c:181-214  softmax_n and moe_ffn (router, top-k, renorm,
 *                           SwiGLU experts, weighted combine, residual)
 *   src/gguf_run.c:254      argmax
 *   src/expert_store.c      lease-LRU expert pager
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   or_f16_to_f32    all 65536 inputs against IEEE binary16 (numpy)
 *   or_dequant_row   golden vectors from the reference compiled from source,
 *                    plus closed forms (Q8_0 q*d exact; Q4_K/Q6_K scale unpack)
 *   or_matmul        golden vectors (bit-exact) + fp64 brute-force error bound
 *   or_rmsnorm, or_softmax, or_topk, or_argmax
 *                    golden vectors + closed forms (sum to 1, ordering rules)
 *   or_moe_ffn       golden vectors (bit-exact outputs and expert order)
 *   or_store_*       the reference unit test's scenario and its printed stats
 *
 * Extensions with no reference counterpart (defined here, pinned by closed
 * form): an optional per-expert router logit bias, added to the F32 router
 * logits before the softmax (with a zero bias the path is the reference's).
 */
#ifndef VIREO_ORACLE_H
#define VIREO_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_F16 = 1, OR_Q5_0 = 6, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14 };

float or_f16_to_f32(uint16_t h);
int   or_type_block(uint32_t type, int *block_elems, int *block_bytes);
void  or_dequant_row(uint32_t type, const void *src, float *dst, int n);
/* y[o] = sum_i W[o][i] * x[i] for o < d; W rows hold n elements. */
void  or_matmul(float *y, const float *x, uint32_t type, const void *w, int n, int d);
void  or_rmsnorm(float *o, const float *x, const float *w, int n, float eps);
void  or_softmax(float *v, int n);
void  or_topk(const float *p, int ne, int k, int renorm, int *idx, float *w);
int   or_argmax(const float *v, int n);

typedef struct {
    int d, ne, k, fe, renorm;
    uint32_t gate_type, up_type, down_type;
} or_moe_cfg;

/* moe_ffn over n_tokens tokens, one at a time: x[t] += moe(hb[t]).
 * gate/up/down: per-expert slice pointers (NULL = unregistered, skipped as the
 * reference skips a failed lookup). logit_bias: optional [ne]. Outputs are
 * optional: idx_out/w_out [n_tokens x k], prob_out [n_tokens x ne]. */
void or_moe_ffn(const or_moe_cfg *c, const float *router, const float *logit_bias,
                const void *const *gate, const void *const *up, const void *const *down,
                float *x, const float *hb, int n_tokens,
                int *idx_out, float *w_out, float *prob_out);

/* Lease-LRU pager (src/expert_store.c). */
typedef struct or_store or_store;
typedef struct { const void *gate, *up, *down; void *slot; } or_view;
or_store *or_store_create(int fd, uint64_t capacity_bytes, int n_layers, int n_experts);
void or_store_register(or_store *s, int layer, int expert, uint64_t gate_off, uint64_t up_off,
                       uint64_t down_off, uint32_t gate_bytes, uint32_t up_bytes, uint32_t down_bytes);
int  or_store_lookup(or_store *s, int layer, int expert, or_view *v);
void or_store_release(or_store *s, or_view *v);
/* out: requests, hits, misses, bytes_read, resident_bytes, capacity_bytes, experts_resident */
void or_store_stats(const or_store *s, uint64_t out[7]);
void or_store_destroy(or_store *s);

#ifdef __cplusplus
}
#endif
#endif
