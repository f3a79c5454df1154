/* vireo-hip: MI355X (gfx950) kernels for vireo's quantized MoE-FFN path.
 *
 * A drop-in for the compute interface that the reference's GGUF runner uses:
 *   gguf_matmul      (src/gguf_compute.h:10)  -> qmatvec / qmatvec_async
 *   gguf_dequant_row (src/gguf_compute.h:9)   -> qdequant_rows
 *   moe_ffn          (src/gguf_run.c:185-214, static in the reference)
 *                                              -> moe_ffn_forward
 *   expert_store_*   (src/expert_store.h)     -> vireo_expert_store.h (HBM pool)
 *   rmsnorm / argmax (src/gguf_run.c:161-165, :254) -> vireo_rmsnorm / vireo_argmax
 *
 * Conventions
 *   - Every pointer to tensor data, activations or outputs is a device pointer;
 *     structs (gguf_tensor, vireo_moe_model, ...) live in host memory.
 *   - Every entry point returns 0 or a negative errno value (-EINVAL for bad
 *     arguments or an unsupported ggml type, -ENOMEM, -EIO for a HIP runtime
 *     failure). The reference returns void and silently skips unknown types;
 *     for valid inputs the outputs have the reference's meaning.
 *   - `stream` is a hipStream_t passed as void*. With stream == NULL the call
 *     runs on the default stream and returns after the work has finished (the
 *     reference is synchronous); with a stream the call only enqueues.
 *   - Tensor data must be 4-byte aligned at its start (hipMalloc gives 256);
 *     every row in these formats is a whole number of 2-byte units.
 *   - Calls on one device must not overlap: the library keeps one workspace
 *     per device, like the reference's single Model buffers
 *     (src/gguf_run.c:346-350), so calls from other threads, or on other
 *     streams whose work may run at the same time, race. Calls enqueued on
 *     one stream are ordered and safe.
 */
#ifndef VIREO_HIP_H
#define VIREO_HIP_H

#include <stdint.h>
#include "vireo_gguf.h"
#include "vireo_expert_store.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- library ---------------------------------------------------------------- */

/* Select the device the library works on (default: the current HIP device). */
int vireo_hip_init(int device);
/* Text for an error code returned by this library. */
const char *vireo_hip_strerror(int err);
/* Block geometry of a ggml type: src/gguf.c:27-38 (F32, F16, Q8_0, Q5_0, Q4_K,
 * Q6_K are supported by the kernels; Q4_0 is sized but, as in the reference,
 * not computable). Returns 0 or -EINVAL. */
int vireo_type_block(uint32_t ggml_type, int *block_elems, int *block_bytes);

/* ---- quantized compute (src/gguf_compute.h) ---------------------------------- */

/* gguf_matmul (src/gguf_compute.c:159-214): y[o] = sum_i W[o][i] * x[i] for
 * o < d, with W = w->data holding d rows of n elements of type w->ggml_type.
 * y, x, w->data are device pointers; y must not alias x. Synchronous. */
int qmatvec(float *y, const float *x, const gguf_tensor *w, int n, int d);
/* The same, enqueued on `stream`. */
int qmatvec_async(float *y, const float *x, const gguf_tensor *w, int n, int d, void *stream);

/* gguf_dequant_row (src/gguf_compute.c:105-124) applied to `rows` consecutive
 * rows of n elements: dst[r*n + i] = dequant(src row r)[i]. Bit-identical to
 * the reference (every dequantized value has at most one rounding). */
int qdequant_rows(uint32_t ggml_type, const void *src, float *dst, int n, int rows, void *stream);

/* ---- model glue used by the MoE stack --------------------------------------- */

/* rmsnorm (src/gguf_run.c:161-165) on `rows` rows of n floats:
 * o = x * (1/sqrt(mean(x^2) + eps)) * w. w: device [n] F32 weight, or NULL
 * for a unit weight. o may equal x. */
int vireo_rmsnorm(float *o, const float *x, const float *w, int n, int rows, float eps, void *stream);
/* The same for one row, bit for bit the reference's: its in-order fp32 sum of
 * squares (src/gguf_run.c:162), then the scale and the products in its order
 * (vireo_rmsnorm sums the squares in fp64 and rounds once: within 2e-5 of
 * this, and parallel). One workgroup adds the n squares in order, about 7 us
 * for n = 2048. o must not alias x. */
int vireo_rmsnorm_exact(float *o, const float *x, const float *w, int n, float eps, void *stream);
/* The router logits exactly as the reference forms them (the F32 gguf_matmul,
 * src/gguf_compute.c:202-207: per expert an in-order fp32 sum of fp32
 * products, no contraction): out[t*E + e] = row e of R . hb[t], for T
 * tokens. R: device [E x d] F32; hb: [T x d]; out: [T x E]. The routing
 * kernels compute these chains for the tokens whose fp64 bounds do not
 * certify their top k; for d = 2048 (16-byte aligned rows) a whole wave
 * shares one chain. */
int vireo_router_logits(const float *R, const float *hb, int d, int E, int T, float *out, void *stream);
/* argmax (src/gguf_run.c:254): first index of the maximum of v[0..n). */
int vireo_argmax(const float *v, int n, int32_t *out, void *stream);
/* Embedding lookup (src/gguf_run.c:218, gguf_dequant_row of a tok_embd row):
 * dst[i*n + j] = dequant(row tokens[i] of table)[j] for i < count. table:
 * device [n_rows x n] of type Q8_0, F16 or F32; tokens: device int32 (an
 * argmax output, so a decode loop needs no host round trip); a token outside
 * [0, n_rows) gives a zero row. */
int vireo_embed(uint32_t type, const void *table, int n, int n_rows, const int32_t *tokens, int count, float *dst,
                void *stream);

/* ---- MoE FFN (src/gguf_run.c:185-214) ---------------------------------------- */

/* The MoE layer tensors moe_ffn reads from Layer (src/gguf_run.c:144). */
typedef struct {
    const gguf_tensor *router;     /* F32 [n_experts x dim]; data: device */
    const gguf_tensor *gate_exps;  /* only ggml_type is read: expert bytes  */
    const gguf_tensor *up_exps;    /*   come from the ExpertStore, as in    */
    const gguf_tensor *down_exps;  /*   src/gguf_run.c:201-204              */
    /* Optional device [n_experts] F32 bias added to the router logits before
     * the softmax; NULL = none. No counterpart in the reference (its router has
     * no bias); used to skew routing for prefill workloads. */
    const float *logit_bias;
} vireo_moe_layer;

/* The fields moe_ffn reads from Model (src/gguf_run.c:146-157). */
typedef struct {
    int dim;          /* d */
    int n_experts;    /* E */
    int n_used;       /* k (top-k), 1 <= k <= min(E, 64); -EINVAL beyond, where the
                         reference truncates to 64 (src/gguf_run.c:190) */
    int ffn_exp;      /* expert intermediate size fe */
    int topk_renorm;  /* renormalise the k weights (src/gguf_run.c:292-293) */
    int n_layers;
    const vireo_moe_layer *layers;   /* host array [n_layers] */
    ExpertStore *es;
} vireo_moe_model;

/* Routing flags, one word per token (moe_route `flags`). */
#define VIREO_ROUTE_EXACT_FALLBACK 1u  /* the fast fp64 router could not certify
                                          the order; exact fp32 sums were used */
#define VIREO_ROUTE_NEAR_TIE       2u  /* a selection boundary had an exact logit
                                          gap below 1e-6 (reported exception)  */
#define VIREO_DECODE_TIMEOUT       4u  /* a kernel with a grid-wide wait gave up
                                          waiting (not every workgroup was
                                          resident): that call's result is invalid */

/* Kernels that meet across the whole grid (the fused decode plan) bound every
 * wait by a number of polls; a wait that runs out sets VIREO_DECODE_TIMEOUT in
 * a sticky per-device status word and lets the kernel finish (no hang).
 * vireo_hip_status waits for `stream` (NULL: the null stream), then reads and
 * clears that word: -ETIMEDOUT if a wait gave up since the last read, else 0.
 * Synchronous calls (stream NULL) check it themselves and return -ETIMEDOUT.
 * vireo_hip_set_spin_limit sets the poll bound (default 262144; 0 makes every
 * such wait give up at once, which tests the error path without a hang). No
 * counterpart in the reference. */
int vireo_hip_status(void *stream);
int vireo_hip_set_spin_limit(unsigned polls);

/* Stage 1 of moe_ffn_forward: router logits (F32 matvec), softmax, top-k with
 * lowest-index tie-break, optional renorm (src/gguf_run.c:187-192), for
 * n_tokens tokens. hb: device [n_tokens x dim]. idx [n_tokens x k] (int32) and
 * w [n_tokens x k] receive the chosen experts in selection order and their
 * weights; flags [n_tokens] (optional) receives VIREO_ROUTE_* bits; probs
 * [n_tokens x E] (optional) receives the softmax probabilities. The expert
 * ids equal the reference's bit for bit except where flags report a near tie. */
int moe_route(const vireo_moe_model *m, int layer, const float *hb, int n_tokens,
              int32_t *idx, float *w, uint32_t *flags, float *probs, void *stream);

/* Stage 2: bucket the n_tokens*k (token, slot) pairs by expert. counts [E],
 * offs [E+1] (exclusive prefix sum, offs[E] = n_tokens*k) and perm
 * [n_tokens*k], where perm lists pair ids t*k + j sorted by (expert, t). No
 * counterpart in the reference (it runs tokens one at a time). */
int moe_dispatch(const int32_t *idx, int n_tokens, int k, int n_experts,
                 int32_t *counts, int32_t *offs, int32_t *perm, void *stream);

/* moe_ffn for n_tokens independent tokens: x[t] += sum_j w_tj * down_e(
 * silu(gate_e hb[t]) * up_e hb[t]) over the k routed experts e = idx[t][j],
 * combined in selection order without atomics. x, hb: device
 * [n_tokens x dim]; idx_out / w_out (optional) receive the routing.
 * Expert slices come from m->es, which must be a store made by this library
 * (a store from the reference's CPU src/expert_store.c is refused: -EINVAL).
 * When the store's capacity holds every registered expert of every layer (0 =
 * unbounded), the first call for a layer looks each of its experts up once and
 * holds the leases (expert_store_pin_layer), as there is no host round trip
 * per token; a layer the caller pinned explicitly is used the same way.
 * Otherwise every call copies the per-expert token counts and the routing to
 * the host and looks the routed experts up in batches that fit the room beside
 * the leased experts (misses read from the store's file while earlier batches
 * compute and copied to HBM on a copy stream; least recently used unleased
 * experts evicted, their blocks reused only after the kernels reading them);
 * such a call synchronizes the stream once and cannot be captured in a graph.
 * A paged call of at most 8 tokens on a file-backed store also guesses the
 * next layer's experts - that layer's router applied to this call's hb - and
 * the next call on that layer reads the guessed experts not yet resident
 * while it waits for its own routing (expert_store_set_prefetch turns this
 * off); a guess changes what the pool holds, never a result.
 * expert_store_stats then counts what the reference would: one lookup per
 * (token, routed expert) in token and selection order (see
 * expert_store_hbm_stats for what the HBM pool itself did). An expert that is
 * not registered contributes nothing, as in the reference.
 * Graph capture: capture after one uncaptured call of each shape. Buffers the
 * library grows later are new allocations; the ones captured graphs use stay
 * allocated, so such graphs remain valid. Calls captured in a graph are not
 * counted in expert_store_stats (the host does not see replays). */
int moe_ffn_forward(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens,
                    int32_t *idx_out, float *w_out, void *stream);

/* moe_ffn_forward for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc): no counterpart in
 * the reference. The same results as moe_ffn_forward, but every intermediate
 * lives in a fixed 32 MiB region of device memory that the library holds per
 * device from its first use (vireo_hip_init, or the first call on a device)
 * until the process ends, and the call makes no allocation of any kind.
 * Limits: the layer must already be resident and pinned
 * (expert_store_pin_layer, or one earlier moe_ffn_forward on it; else
 * -EINVAL); calls whose intermediates exceed the region return -E2BIG (about
 * 400 tokens for the Qwen3-30B-A3B layer); the fused plan (vireo_hip_set_path
 * 3) is not used; calls are not counted in expert_store_stats. Every call on a
 * device shares the region, which keeps the last call's contents: calls that
 * may overlap on one device (other streams, other threads) race. */
int moe_ffn_forward_noalloc(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens,
                            int32_t *idx_out, float *w_out, void *stream);

/* Execution plan for moe_ffn_forward (a tuning and testing knob; no
 * counterpart in the reference): 0 = automatic (default), 1 = the one-token
 * decode plan whenever it applies (also to calls of 2 to 8 tokens, at most 64
 * (token, routed expert) pairs: every token then gets the bits of a one-token
 * call; plan 0 does this up to 4 tokens on Q4_K gate/up + Q6_K down layers,
 * whose larger calls take the matrix cores, and up to 8 on the other types
 * the one-token kernels take), 2 = always the grouped plan, 3 = the
 * one-token decode plan with its experts fused into one kernel where that
 * kernel is built for the shapes (see moe_decode_stage), 4 = always the
 * grouped plan, with every group on the fp32 kernels, 5 = one token through
 * the whole layer (router, top-k, experts, combine; with the RMSNorm in front
 * in moe_stack_step and vireo_model_step) in one launch whose workgroups meet
 * through tagged records, where it is built for the shapes (d = 2048, k = 8,
 * up to 128 experts, expert width 768 or 1024, Q4_K/Q6_K or Q8_0 experts,
 * 256 CUs); its waits are bounded like plan 3's (vireo_hip_status).
 * Under plans 0 and 2, calls of at least 64 tokens run every group as bf16
 * matrix-core GEMMs (inputs and dequantized weights rounded
 * to bf16, fp32 accumulation; the layer's contribution then agrees with the
 * reference to about 1e-2 of its largest magnitude instead of 2e-3); the
 * routing is unaffected. */
int vireo_hip_set_path(int path);

/* Decode-batch calls (5 to 63 tokens, or 3 and 4 under plan 2) on a pinned layer with Q4_K gate/up and
 * Q6_K down run on the matrix cores, whose loads read 16 rows of a matrix at
 * a time. With packing on (the default), the first such call on a layer that
 * may allocate (not moe_ffn_forward_noalloc, not under graph capture) copies
 * the layer's experts once into tiles of 16 rows x one super-block, the same
 * bytes reordered so that every load instruction reads 1 KB of consecutive
 * memory; later calls read the copy. The copy (as much again as the layer's
 * expert bytes) counts against the store's capacity like resident experts:
 * it is made only while the resident experts and the copies fit the capacity
 * with it (cut from the pool's own device block when that has room), else
 * the calls read the GGUF rows; an unbounded store (capacity 0) always makes
 * it. expert_store_packed_bytes reports the copies' bytes. A copy is made
 * from the pinned views and freed with the pin (expert_store_unpin_layer) or
 * the store; a caller that rewrites a pinned layer's expert bytes in place
 * must unpin and pin it again. Calls of 64 or more tokens on a pinned Q8_0 layer make
 * and read, the same way, a copy in matrix-operand fragments (each lane's
 * bytes of a 32-row, 64-column step together) for the prefill GEMMs. Results
 * are the same bit for bit either way. 0 turns both off for later calls
 * (existing copies stay until unpinned). No counterpart in the reference. */
int vireo_hip_set_packed(int on);

/* The one-token decode plan of moe_ffn_forward as separate launches over a
 * caller-owned device `state` buffer of moe_decode_state_bytes(m) bytes (no
 * counterpart in the reference, whose moe_ffn is one function):
 *   stage 0  router logits of hb into state
 *   stage 1  top-k and the gate/up SwiGLU into state; idx_out / w_out
 *            (optional, k entries) receive the routing. Under plan 3
 *            (vireo_hip_set_path) and for the shapes the fused kernel is
 *            built for (d = 2048, k = 8, 256 CUs; Qwen3-30B-A3B and OLMoE
 *            layers with Q4_K/Q6_K or Q8_0 experts) one launch computes
 *            gate/up, down and the combine and updates x
 *   stage 2  down projections and the combine, x += ... (nothing to do when
 *            stage 1 was the fused kernel)
 * Running 0, 1, 2 in order gives moe_ffn_forward's result for one token bit
 * for bit. Each stage reads only what the previous one left in state (stage
 * 1 needs stage 0 of the same state right before it: stage 0 also clears the
 * fused kernel's flags), so one state per (layer, token) lets a caller (a
 * profiler, a scheduler that interleaves other work) launch and time each
 * stage on its own. The token's flag word (VIREO_ROUTE_* bits, and 4 if a
 * fused launch waited too long for its workgroups, which makes its result
 * invalid) is the last word written by stage 1.
 * moe_decode_state_bytes returns -EINVAL when the model's shapes or types
 * have no decode plan (moe_ffn_forward then always uses the grouped plan). */
int64_t moe_decode_state_bytes(const vireo_moe_model *m);
int moe_decode_stage(const vireo_moe_model *m, int layer, int stage, float *x, const float *hb, void *state,
                     int32_t *idx_out, float *w_out, void *stream);
/* Profiling form of moe_decode_stage: launches `stage` n times back to back,
 * launch i on layer layers[i] (host array) with token row i of x / hb
 * (device [n x dim]), state i at states + i * state_stride (256-aligned,
 * at least moe_decode_state_bytes) and routing row i of idx / w
 * (device [n x n_used]). Each launch records its own begin and end on HIP
 * events (hipExtLaunchKernelGGL, the dispatch's timestamps); the call waits
 * for the last one and writes the n kernel durations in microseconds to
 * us_out (host). Results are those of n moe_decode_stage calls. */
int moe_decode_stage_timed(const vireo_moe_model *m, int stage, int n, const int *layers, float *x, const float *hb,
                           void *states, int64_t state_stride, int32_t *idx, float *w, float *us_out, void *stream);
/* Per-phase timestamps of one-token layer calls (a measurement aid with no
 * counterpart in the reference). Enqueues n moe_ffn_forward calls on stream,
 * call i on layer layers[i] (host array) with token row i of x / hb (device
 * [n x dim]); the one-token decode kernels of call i record, per workgroup
 * (the first 256) and phase, the device clock (s_memrealtime, 100 MHz, one
 * clock for all CUs) into stamps + i * VIREO_PHASE_WORDS (device uint64_t,
 * zeroed by the caller): word (kernel * 256 + workgroup) * 8 + phase.
 * Kernels and phases of the three-kernel decode plan:
 *   0 router:    0 start, 1 the expert's router part computed
 *   1 gate/up:   0 start, 1 router parts loaded, 2 top-k chosen, 3 first
 *                row computed, 4 every row written; word 7 is 1 when the
 *                order took the exact-logit path
 *   2 down:      0 start, 1 plan loaded, 2 first row computed, 3 every row
 *                computed, 4 outputs written
 * and of the one-launch layer kernel (kernel 0): 0 start, 1 router part,
 * 2 every part received, 3 top-k chosen, 4 first gate/up row, 5 activations
 * published, 6 activations received, 7 end. Results are moe_ffn_forward's.
 * The calls may be captured in a HIP graph. */
#define VIREO_PHASE_WORDS (3 * 256 * 8)
int moe_decode_phases(const vireo_moe_model *m, int n, const int *layers, float *x, const float *hb,
                      uint64_t *stamps, void *stream);

/* ---- MoE stack decode step (src/gguf_run.c:216-254) --------------------------- */

/* An attention-free stack of MoE layers with an LM head. */
typedef struct {
    const vireo_moe_model *moe;    /* the n_layers MoE layers */
    const float *const *ffn_norm;  /* host array [n_layers] of device [dim] F32 RMSNorm weights (an
                                      entry or the array NULL: unit weight) */
    const float *out_norm;         /* device [dim] F32, or NULL (unit weight) */
    const gguf_tensor *lm_head;    /* [vocab x dim], data on the device */
    int vocab;
    float eps;
    const gguf_tensor *tok_embd;   /* [vocab x dim] token embedding (Q8_0, F16 or F32), data on the
                                      device; NULL: lm_head (a tied model, src/gguf_run.c:297) */
} vireo_moe_stack;

/* One greedy decode step, forward() (src/gguf_run.c:216-251) with attention
 * omitted, then argmax (:254): x = embed(token[0]); for each layer l,
 * xb = rmsnorm(x, ffn_norm[l]) and moe_ffn_forward(l) adds to x; then
 * logits = lm_head * rmsnorm(x, out_norm) and token[0] = argmax(logits).
 * token (int32 [1]), x, xb ([dim]) and logits ([vocab]) are caller-owned
 * device buffers; with a stream every launch is only enqueued there, so a
 * caller can capture a loop of steps in a graph (after one uncaptured step:
 * the first call on a layer pins its expert leases). */
int moe_stack_step(const vireo_moe_stack *st, int32_t *token, float *x, float *xb, float *logits, void *stream);
/* moe_stack_step that also records every layer's routing: idx (device int32
 * [n_layers x n_used]) receives layer l's experts in selection order and
 * flags (device uint32 [n_layers]) its VIREO_ROUTE_* bits. The same launches
 * as moe_stack_step plus one 4-byte copy per layer; for parity checks of a
 * whole stack. No counterpart in the reference. */
int moe_stack_step_trace(const vireo_moe_stack *st, int32_t *token, float *x, float *xb, float *logits,
                         int32_t *idx, uint32_t *flags, void *stream);

/* ---- MoE models from GGUF files (src/gguf_run.c:266-333) ---------------------- */

/* A MoE model read from a GGUF file: the metadata and MoE tensors bound as the
 * reference's loader binds them, the routers, FFN norms, output norm and LM head
 * copied to the device, and every expert's gate/up/down slice registered with
 * an ExpertStore that pages them from the open file into HBM. */
typedef struct {
    gguf_ctx *gguf;          /* the parsed file (host mapping), from vireo_gguf_open */
    char arch[64];           /* general.architecture ("qwen2" if absent, as the reference) */
    vireo_moe_model model;   /* ready for moe_ffn_forward */
    vireo_moe_stack stack;   /* ready for moe_stack_step when lm_head != NULL */
    int vocab;               /* token_embd.weight dims[1]; 0 without that tensor */
    float eps;               /* <arch>.attention.layer_norm_rms_epsilon (0 if absent, as the reference) */
    void *priv;              /* the library's allocations */
} vireo_gguf_moe;

/* Read an MoE GGUF file (general.architecture, <arch>.block_count,
 * embedding_length, feed_forward_length, expert_count, expert_used_count
 * (default 8), expert_feed_forward_length (default feed_forward_length),
 * expert_weights_norm (default: renormalise unless the architecture is
 * "olmoe"), as src/gguf_run.c:276-292), bind blk.<l>.ffn_gate_inp / ffn_gate_exps
 * / ffn_up_exps / ffn_down_exps / ffn_norm (:315-318), and register expert e of
 * layer l at tensor offset + e * (nbytes / n_experts) (:320-333) with an
 * ExpertStore of expert_capacity_bytes (0 = unbounded) over the file. With
 * load_head, output_norm.weight and the LM head (output.weight, else
 * token_embd.weight, :297-299) and token_embd.weight go to the device too.
 * Returns 0, -EINVAL for a file that is not such a model (the message names
 * what is missing or inconsistent: vireo_gguf_moe_error), or -errno. */
int vireo_gguf_moe_load(const char *path, uint64_t expert_capacity_bytes, int load_head, vireo_gguf_moe **out);
/* Why the last vireo_gguf_moe_load on this thread failed ("" after a success). */
const char *vireo_gguf_moe_error(void);
/* Destroy the store, free the device copies and close the file. */
void vireo_gguf_moe_free(vireo_gguf_moe *m);

/* ---- Whole-model decode (src/gguf_run.c:216-251) ---------------------------- */

struct VireoKV; /* the GPU KV store, include/vireo_kv.h */

/* One transformer block's tensors (the reference's Layer, src/gguf_run.c:141-145),
 * data on the device. Matrices may be of any type qmatvec takes; norms and
 * biases are F32 vectors. */
typedef struct {
    const float *attn_norm;              /* [dim], NULL: unit weight */
    const gguf_tensor *wq, *wk, *wv;     /* [n_heads*hs x dim], [n_kv_heads*hs x dim] x 2 */
    const float *bq, *bk, *bv;           /* biases (add_bias, :166), NULL: none */
    const float *q_norm, *k_norm;        /* QK-norm weights, NULL: none (:226-229) */
    int q_norm_len, k_norm_len;          /* == head_size: per head (rmsnorm_heads, :177-179);
                                            otherwise one norm over the whole vector */
    const gguf_tensor *wo;               /* [dim x n_heads*hs] */
    const float *ffn_norm;               /* [dim], NULL: unit weight */
    const gguf_tensor *wg, *wu, *wd;     /* dense SwiGLU FFN [ffn x dim] x 2, [dim x ffn]; unused when
                                            the model's FFNs are MoE layers */
} vireo_block;

/* The reference's Model (src/gguf_run.c:146-157) as the decode step reads it. */
typedef struct {
    int n_layers, dim, n_heads, n_kv_heads, head_size, ffn, vocab;
    float eps, rope_base;
    const vireo_block *blocks;           /* host array [n_layers] */
    const vireo_moe_model *moe;          /* the MoE FFNs (same n_layers and dim), NULL: dense FFNs */
    const gguf_tensor *tok_embd;         /* [vocab x dim] Q8_0, F16 or F32 */
    const float *out_norm;               /* [dim], NULL: unit weight */
    const gguf_tensor *lm_head;          /* [vocab x dim] */
    const float *rope;                   /* device [max_pos x head_size] from vireo_rope_table */
    int max_pos;
} vireo_model;

/* NEOX RoPE angles (rope_neox, src/gguf_run.c:169-174) for positions 0 ..
 * max_pos - 1: row p of dev_out [max_pos x head_size] holds cosf(a_j) for
 * j < head_size / 2, then sinf(a_j), with a_j = p * powf(base, -2j / hs) in the
 * reference's float expression order, computed on the host with the C library
 * (the same values the reference computes per call). */
int vireo_rope_table(float base, int head_size, int max_pos, float *dev_out);
/* Bytes of the caller-owned device state a vireo_model_step needs (activation
 * buffers: xb, q, k, v, attention output, FFN intermediates). */
int64_t vireo_model_state_bytes(const vireo_model *m);
/* One token through the whole model: forward() (src/gguf_run.c:216-251).
 * x = embed(token[0]); per block: xb = rmsnorm(x, attn_norm); q, k, v = wq, wk,
 * wv . xb (+ biases); QK-norms; RoPE at `pos`; k, v appended to kv as token pos
 * of layers l * n_kv_heads + h; each query head attends (grouped: head hh reads
 * kv head hh / (n_heads / n_kv_heads)); x += wo . attention; then
 * xb = rmsnorm(x, ffn_norm) and x += moe_ffn(xb) or the dense SwiGLU FFN. With
 * want_logits: logits = lm_head . rmsnorm(x, out_norm) and token[0] =
 * argmax(logits) (:254). kv: n_layers * n_kv_heads layers of head_size.
 * token (int32 [1]), x ([dim]), logits ([vocab], may be NULL without
 * want_logits) and state (vireo_model_state_bytes, 256-aligned) are device
 * buffers; 0 <= pos < max_pos. Every launch goes to `stream`. */
int vireo_model_step(const vireo_model *m, struct VireoKV *kv, int32_t *token, int pos, int want_logits, float *x,
                     float *logits, void *state, void *stream);
/* vireo_model_step at the position *pos (device int32), which the call then
 * advances by one; kv must be a contiguous store (vireo_kv_create_contiguous)
 * driven by device positions. Every launch reads the position from device
 * memory, so a loop of steps can be captured in one HIP graph (after one
 * uncaptured step: first calls size buffers and pin expert leases). A
 * position outside [0, max_pos) or past the store's tokens makes the step's
 * RoPE and KV writes no-ops. No counterpart in the reference. */
int vireo_model_step_pos(const vireo_model *m, struct VireoKV *kv, int32_t *token, int32_t *pos, int want_logits,
                         float *x, float *logits, void *state, void *stream);

/* A whole model read from a GGUF file: every tensor forward() reads bound as
 * the reference's loader binds it (src/gguf_run.c:276-318) and moved to the
 * device, MoE experts registered with an ExpertStore over the file. */
typedef struct {
    gguf_ctx *gguf;
    char arch[64];
    vireo_model model;                   /* ready for vireo_model_step */
    vireo_moe_model moe;                 /* model.moe points here for MoE files */
    void *priv;
} vireo_gguf_model;

/* Read a GGUF model (metadata src/gguf_run.c:276-293: block_count,
 * embedding_length, feed_forward_length, attention.head_count,
 * head_count_kv, layer_norm_rms_epsilon, rope.freq_base (default 10000),
 * attention.key_length (default dim / heads), and the MoE keys of
 * vireo_gguf_moe_load when expert_count is present); bind blk.<l>.attn_norm,
 * attn_q/k/v (+ .bias), attn_q_norm / attn_k_norm, attn_output, ffn_norm and
 * either the MoE tensors or ffn_gate / ffn_up / ffn_down (:300-318), and
 * token_embd, output_norm, output (else token_embd). Norms and biases of any
 * dequantizable type become F32 on the device. max_pos sizes the RoPE table.
 * Returns 0, -EINVAL (vireo_gguf_moe_error says why) or -errno. */
int vireo_gguf_model_load(const char *path, uint64_t expert_capacity_bytes, int max_pos, vireo_gguf_model **out);
void vireo_gguf_model_free(vireo_gguf_model *m);

/* ---- ExpertStore extensions (HBM pool) -------------------------------------- */

/* A store whose backing "file" is already in device memory (dev_base, size
 * bytes), for weights generated or uploaded on the GPU: slices registered
 * with offsets into dev_base become resident without a copy. */
ExpertStore *expert_store_create_device(const void *dev_base, uint64_t size, uint64_t capacity_bytes,
                                        int n_layers, int n_experts);
/* Look up every registered expert of `layer` once and hold the leases, and
 * return a device table [n_experts x 3] of {gate, up, down} pointers (NULL for
 * unregistered experts). Later calls return the same table. -ENOSPC (nothing
 * evicted) when the layer's experts exceed the capacity, or when the leased
 * experts of other layers leave no room for them. */
int expert_store_pin_layer(ExpertStore *s, int layer, const void *const **dev_table);
/* Release the leases taken by expert_store_pin_layer for `layer`. */
int expert_store_unpin_layer(ExpertStore *s, int layer);
/* What the HBM pool did, in ExpertStats form: every lookup the library made
 * (whole layers pinned, routed experts paged per call) and the caller's own
 * lookups, the bytes copied into HBM (or aliased, for a device-backed store),
 * and the bytes and experts resident in HBM now (resident_bytes includes the
 * kernels' packed copies of pinned layers, expert_store_packed_bytes).
 * expert_store_stats reports the reference's accounting of the same work
 * instead. */
void expert_store_hbm_stats(const ExpertStore *s, ExpertStats *out);
/* Device bytes of the packed copies of pinned layers (vireo_hip_set_packed)
 * the store holds now, 0 for NULL or a foreign store. No counterpart in the
 * reference. */
uint64_t expert_store_packed_bytes(const ExpertStore *s);
/* Prefetch by paged calls (no counterpart in the reference, whose
 * ROADMAP.md:46-47 lists it as open): on by default for a store that reads a
 * file; 0 turns it off. -EINVAL for a store this library did not make. */
int expert_store_set_prefetch(ExpertStore *s, int on);
/* out[0] experts read ahead, out[1] of those looked up before being evicted,
 * out[2] bytes read ahead (also counted in expert_store_hbm_stats's
 * bytes_read). */
void expert_store_prefetch_stats(const ExpertStore *s, uint64_t out[3]);

#ifdef __cplusplus
}
#endif
#endif
