// Host-side launchers shared between the routing, decode and grouped kernels.
#pragma once
#include <hip/hip_runtime.h>
#include "route.h"
#include "vireo_hip.h"

// Router logits of T tokens into parts[T x E] (fast bounded, or exact); the
// launch also sets zero[0 .. nzero) to 0 (the fused decode kernel's flags).
int vh_route_parts(const float *R, const float *hb, const float *bias, int d, int E, int T, bool exact,
                   RoutePart *parts, hipStream_t s, uint32_t *zero = nullptr, int nzero = 0);
// The same parts of the RMSNorm of x (weight nw, NULL = unit): the launch also
// writes hb_out = rmsnorm(x) for the later stages. d == 2048, x and hb_out
// 16-byte aligned, else -EINVAL.
int vh_route_parts_norm(const float *R, const float *x, const float *nw, float eps, float *hb_out, const float *bias,
                        int d, int E, int T, RoutePart *parts, hipStream_t s, uint32_t *zero = nullptr, int nzero = 0);
// One MoE layer of a stack for one token: xb = rmsnorm(x, nw); x += moe(xb).
// The one-token decode plan folds the RMSNorm into its router launch; other
// shapes run vireo_rmsnorm and moe_ffn_forward.
// ExpertStore internals for the MoE plans (expert_store.c): an expert's bytes
// in the pool (0 if unregistered), the capacity (0 = unbounded), whether a
// store is one of this library's, a pinned layer's table (NULL if none; never
// allocates) and its reordered copies for the decode batch's and the
// prefill's kernels (held and freed by the store with the pin), whether every
// layer fits at once, the bytes
// that hold leases,
// lookups / lease drops for paged calls (page-ins on a copy stream, blocks
// protected by events until the kernels that read them are done), and the
// routing copies that feed the reference's statistics.
extern "C" {
uint64_t vh_store_expert_bytes(const ExpertStore *s, int layer, int expert);
uint64_t vh_store_capacity(const ExpertStore *s);
int vh_store_valid(const ExpertStore *s);
const void *const *vh_store_layer_table(const ExpertStore *s, int layer);
const void *const *vh_store_packed_table(const ExpertStore *s, int layer, int kind);
void *vh_store_packed_begin(ExpertStore *s, int layer, int kind, uint64_t bytes);
int vh_store_set_packed(ExpertStore *s, int layer, int kind, void *tab);
void vh_store_packed_abort(ExpertStore *s, int layer, int kind);
int vh_store_fits_all(const ExpertStore *s);
uint64_t vh_store_leased_bytes(const ExpertStore *s);
int vh_store_acquire(ExpertStore *s, int layer, int expert, ExpertView *view, hipStream_t cs);
int vh_store_drop(ExpertStore *s, ExpertView *view, hipStream_t stream);
int vh_store_copy_fence(ExpertStore *s, hipStream_t cs, hipStream_t stream);
void vh_store_hint(ExpertStore *s, int layer, const int32_t *ids, int n);
int vh_store_prefetch_next(ExpertStore *s, int layer, hipStream_t cs);
int vh_store_prefetching(const ExpertStore *s);
int vh_store_note_routing(ExpertStore *s, int layer, const int32_t *idx_dev, int T, int k, hipStream_t stream);
void vh_store_note_routing_host(ExpertStore *s, int layer, const int32_t *idx, int T, int k);
}

// idx_out (k entries) / flags_out (one word), device, optional: the layer's
// routing and VIREO_ROUTE_* flags.
int vh_moe_layer_normed(const vireo_moe_model *m, int layer, float *x, const float *nw, float eps, float *xb,
                        hipStream_t s, int32_t *idx_out = nullptr, uint32_t *flags_out = nullptr);
// True under the plans whose kernels' workgroups wait for each other with a
// bounded poll (3, 5): a synchronous caller reads the status word after them.
bool vh_plan_waits();
// y += W x (qmatvec_async with each result added to y[r], one rounding)
int vh_qmatvec_acc(float *y, const float *x, const gguf_tensor *w, int n, int d, hipStream_t s);
// y_i = W_i x for three matrices of n columns in one launch; -ENOTSUP when a
// type or n has no such launch (then one qmatvec_async per matrix)
int vh_qmatvec3(const float *x, int n, float *y0, const gguf_tensor *w0, int d0, float *y1, const gguf_tensor *w1,
                int d1, float *y2, const gguf_tensor *w2, int d2, hipStream_t s);
// The same on the RMSNorm of x with weights nw (null: unit weights), formed
// in the launch as vireo_rmsnorm forms it; -ENOTSUP when a type or n has no
// such launch (then vireo_rmsnorm and vh_qmatvec3)
int vh_qmatvec3_normed(const float *x, const float *nw, float eps, int n, float *y0, const gguf_tensor *w0, int d0,
                       float *y1, const gguf_tensor *w1, int d1, float *y2, const gguf_tensor *w2, int d2,
                       hipStream_t s);
// Per-token top-k from parts: idx/w [T x k], flags [T], probs [T x E] optional.
int vh_route_finish(const RoutePart *parts, const float *R, const float *hb, const float *bias, int d, int E, int k,
                    int renorm, bool exact, int T, int32_t *idx, float *w, uint32_t *flags, float *probs,
                    hipStream_t s);

// Where hb came from when the library normalised it itself (the stack and
// model paths): the residual x, the norm weight (NULL: unit) and eps, so that
// an uncertified routing can be decided on the reference's own xb (its
// in-order RMSNorm, recomputed exactly). x == NULL: hb is the caller's input.
struct NormRef {
    const float *x = nullptr;
    const float *nw = nullptr;
    float eps = 0.0f;
};
// hb_out = the reference's RMSNorm of x (src/gguf_run.c:161-165) bit for bit
// (its in-order fp32 sum of squares), for one row of n.
int vh_rmsnorm_ref(float *hb_out, const float *x, const float *nw, int n, float eps, hipStream_t s);

// What the decode gate/up kernel hands to the down kernel: the chosen experts'
// down matrices (NULL for an unregistered expert) and weights, in selection order.
struct DecodePlan {
    const void *down[64];
    float w[64];
};

// Decode path (one token): gate/up with the top-k fused in, then down + combine.
int vh_decode_gateup(uint32_t type, const RoutePart *parts, const float *R, const float *hb, const float *bias, int d,
                     int E, int k, int fe, int renorm, const void *const *table, float *h, int32_t *idx, float *w,
                     uint32_t *flags, DecodePlan *plan, uint32_t down_type, NormRef nref, hipStream_t s);
bool vh_decode_gateup_supported(uint32_t type, int d, int fe);
// The same for a decode batch of 2 <= nt <= kDecodeBatchMax tokens (nt k <=
// 64): parts [nt x E], hb [nt x d]; h [nt k x fe], idx / w [nt k], flags [nt]
// and plan entries t k + j as the one-token kernel writes them for each token.
constexpr int kDecodeBatchMax = 8;
// Whether vh_decode_batch_gateup takes the shape (its outputs' LDS included).
bool vh_decode_batch_supported(uint32_t type, int d, int fe, int E, int k, int nt);
int vh_decode_batch_gateup(uint32_t type, const RoutePart *parts, const float *R, const float *hb, const float *bias,
                           int d, int E, int k, int fe, int renorm, const void *const *table, float *h, int32_t *idx,
                           float *w, uint32_t *flags, DecodePlan *plan, int nt, hipStream_t s);
// Down projection + weighted combine + residual, for nt tokens (nt k <= 64):
// x[t] += sum_j plan.w[t k + j] * down_j h[t k + j], in selection order.
int vh_down_combine(uint32_t type, const DecodePlan *plan, const float *h, int d, int fe, int k, float *x,
                    hipStream_t s, int nt = 1);
bool vh_down_combine_supported(uint32_t type, int d, int fe, int k);

// Grouped path (any number of tokens): dispatch, grouped gate/up, grouped
// down, combine.
int vh_dispatch(const int32_t *idx, int P, int E, int32_t *counts, int32_t *offs, int32_t *perm, int32_t *active,
                hipStream_t s);
int vh_grouped_gateup(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                      const int32_t *active, const void *const *table, const float *hb, int d, int fe, int k, int E,
                      int max_slots, float *h, hipStream_t s);
int vh_grouped_down(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                    const int32_t *active, const void *const *table, const float *h, int d, int fe, int E,
                    int max_slots, float *ybuf, hipStream_t s);
int vh_combine(const int32_t *idx, const float *w, const void *const *table, const float *ybuf, int d, int k, int T,
               float *x, hipStream_t s);

// Decode-style grouped projections (moe_gdec.hip): the same inputs and outputs
// as vh_grouped_gateup / vh_grouped_down; Q8_0 / Q4_K / Q6_K rows of at most
// 2048 weights and a 16-byte aligned hb.
bool vh_gdec_supported(uint32_t tg, uint32_t td, int d, int fe, const float *hb);
int vh_gdec_gateup(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                   const int32_t *active, const void *const *table, const float *hb, int d, int fe, int k, int E,
                   int max_slots, int max_count, float *h, hipStream_t s);
int vh_gdec_down(uint32_t type, const int32_t *counts, const int32_t *offs, const int32_t *perm,
                 const int32_t *active, const void *const *table, const float *h, int d, int fe, int E, int max_slots,
                 int max_count, float *ybuf, hipStream_t s);

// Decode-batch projections on the matrix cores (moe_mdec.hip), for calls of
// fewer than kMfmaMinCall tokens with Q4_K gate/up and Q6_K down: the same
// groups and outputs as vh_gdec_*. vh_mdec_prep splits hb [T x d] into xp
// (vh_mdec_xp_bytes: the split inputs, T x d x 4 bytes, then their sub-block
// sums, T x d / 8 bytes, at vh_mdec_xsum) and xsc [T]; gate/up writes the
// activations as hp (P x fe x 4 bytes, not fp32 h) for vh_mdec_down.
inline size_t vh_mdec_xp_bytes(int T, int d) { return size_t(T) * d * 4 + size_t(T) * (d / 8); }
inline void *vh_mdec_xsum(void *xp, int T, int d) { return static_cast<char *>(xp) + size_t(T) * d * 4; }
bool vh_mdec_supported(uint32_t tg, uint32_t td, int d, int fe);
// The router parts of T >= 2 tokens (the same values as vh_route_parts'
// bounded parts) by 4 x 4 tiles of (expert, token), d == 2048 and 16-byte
// aligned R and hb, else -EINVAL; with xp given, also vh_mdec_prep's outputs.
int vh_route_parts_tiled(const float *R, const float *hb, const float *bias, int d, int E, int T, RoutePart *parts,
                         void *xp, float *xsc, hipStream_t s);
int vh_mdec_prep(const float *hb, int T, int d, void *xp, float *xsc, hipStream_t s);
// A decode-batch call whose matrix-core kernels find each expert's pairs in
// the routing themselves (no dispatch: workgroup column e takes expert e)
// and whose down kernel also combines into x in selection order (no combine
// kernel): idx and w [T x k], x [T x d], ctr [nctr] arrival counters
// (vh_mdec_ctr_words), which the gate/up kernel zeroes. T < 64.
struct MdecSelf {
    const int32_t *idx;
    const float *w;
    float *x;
    uint32_t *ctr;
    int nctr, T, k;
};
// the down kernel's arrival counters: 64 tokens per chunk of 64 or 128 rows of d
inline int vh_mdec_ctr_words(int d) { return (d + 63) / 64 * 64; }
// `packed`: table points at vh_mdec_pack_layer's tiles instead of GGUF rows;
// `self` (optional): the call's routing (counts, offs, perm and active unused).
int vh_mdec_gateup(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                   const void *const *table, bool packed, const void *xp, const float *xsc, int T, int d, int fe,
                   int k, int E, int max_slots, int max_count, void *hp, hipStream_t s,
                   const MdecSelf *self = nullptr);
int vh_mdec_down(const int32_t *counts, const int32_t *offs, const int32_t *perm, const int32_t *active,
                 const void *const *table, bool packed, const void *hp, int d, int fe, int E, int max_slots,
                 int max_count, float *ybuf, hipStream_t s, const MdecSelf *self = nullptr);
// A copy of the experts behind `table` (device [E x 3]: Q4_K gate, up; Q6_K
// down) in the decode batch's 16-row tiles, written into buf (device,
// vh_mdec_pack_bytes(E, d, fe) bytes, 0 for a shape it does not take), with
// tab_out its new device table (NULL where table is). Enqueued on s after a
// synchronizing read of the table; -EBUSY while s is being captured.
uint64_t vh_mdec_pack_bytes(int E, int d, int fe);
int vh_mdec_pack_layer(const void *const *table, int E, int d, int fe, void *buf, void **tab_out, hipStream_t s);

// Matrix-core grouped GEMMs (moe_mfma.hip) for the groups of calls of at
// least kMfmaMinCall tokens. vh_mfma_plan lists the token tiles of groups of
// at least min_tokens tokens (32, 64 or 128 rows each) and the two launches'
// per-XCD runs in tiles[0 .. vh_mfma_plan_words) (layout: mfma_plan_kernel),
// for the expert types and sizes the launches will get, and the other
// non-empty groups in small[E + 1] (the `active` format); gate/up writes
// bf16 h rows in dispatch order into hs [P x fe]; down writes ybuf rows like
// vh_grouped_down. The forward pass sends every group of such a call to the
// matrix cores (min_tokens 1): a tile's cost is its weight staging, so even a
// one-token group is cheaper there than on the fp32 kernels (a 2048-token
// Qwen3 Q8_0 prefill: 646 us per layer with every group on the matrix cores,
// 666 / 678 / 727 us with groups below 4 / 8 / 16 tokens on the fp32 kernels).
constexpr int kMfmaMinCall = 64;
bool vh_mfma_supported(uint32_t tg, uint32_t td, int d, int fe, int E);
constexpr int kPlanRunsGU = 1, kPlanRunsDN = 10, kPlanHead = 19;  // offsets in the tile plan
int vh_mfma_max_tiles(int P, int E);
int vh_mfma_plan_words(int P, int E);
// hb (optional): the same launch also writes xb, the bf16 copy of hb's n
// values (as vh_to_bf16).
int vh_mfma_plan(const int32_t *counts, int E, int P, int min_tokens, uint32_t tg, uint32_t td, int d, int fe,
                 int32_t *tiles, int32_t *small, const float *hb, void *xb, int64_t n, hipStream_t s);
// xb: the bf16 copy of hb (vh_to_bf16)
int vh_to_bf16(const float *x, void *y, int64_t n, hipStream_t s);
// `packed`: table points at vh_mfma_pack_q8's fragments (Q8_0 only).
int vh_mfma_gateup(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                   const int32_t *perm, const void *const *table, bool packed, const void *xb, int d, int fe, int k,
                   void *hs, hipStream_t s);
int vh_mfma_down(uint32_t type, const int32_t *tiles, int max_tiles, const int32_t *counts, const int32_t *offs,
                 const int32_t *perm, const void *const *table, bool packed, const void *hs, int d, int fe,
                 float *ybuf, hipStream_t s);
// A copy of the Q8_0 experts behind `table` (gate, up: fe rows of d; down: d
// rows of fe) in the matrix cores' operand order (32-row fragments per K step
// of 64, each lane's bytes together; the same bytes, -EBUSY under capture),
// for the GEMMs of pinned layers, written into buf (vh_mfma_pack_bytes(E, d,
// fe) bytes) with tab_out its new device table.
uint64_t vh_mfma_pack_bytes(int E, int d, int fe);
int vh_mfma_pack_q8(const void *const *table, int E, int d, int fe, void *buf, void **tab_out, hipStream_t s);

// Fused one-token experts kernel (moe_fused.hip): top-k, gate/up, down and
// combine in one launch of kFusedBlocks workgroups that meet once through
// bar[0 .. kFusedBlocks) (zeroed by vh_route_parts); bar[kFusedBlocks] is the
// token's flag word (VIREO_ROUTE_* bits, VIREO_DECODE_TIMEOUT).
constexpr int kFusedBlocks = 256;
int vh_fused_blocks(uint32_t tg, uint32_t td, int d, int E, int k, int fe);  // kFusedBlocks, or 0 if not built for it
int vh_decode_experts(uint32_t tg, uint32_t td, const RoutePart *parts, const float *R, const float *hb,
                      const float *bias, int d, int E, int k, int fe, int renorm, const void *const *table, float *h,
                      uint32_t *bar, float *x, int32_t *idx, float *w, NormRef nref, hipStream_t s);

// One MoE layer for one token in one launch (moe_layer.hip): router, top-k,
// gate/up, down, combine, residual, with the RMSNorm in front when norm is
// set (xin is then the residual x itself). kLayerBlocks workgroups, all
// resident at once, meet through tagged records in a LayerXchg that is zeroed
// once per device (vh_layer_xchg) and shared by every launch there.
constexpr int kLayerBlocks = 256;
constexpr int kMaxLayerFe = 1024;
struct LayerXchg {
    uint32_t gen[kLayerBlocks];        // per workgroup: the number of its last launch
    uint64_t parts[2 * 128];           // router parts, two tagged words per expert
    uint64_t h[8 * kMaxLayerFe];       // SwiGLU activations per round, tagged
    uint64_t done[8][kLayerBlocks / 8];  // per round and producer workgroup: its activations are stored
};
struct LayerArgs {
    const float *R;                    // router [E x d]
    const float *xin;                  // hb, or (norm) the residual x
    const void *const *table;          // the layer's expert table [E x 3]
    LayerXchg *xg;
    int E, k, fe, d, renorm;
    const float *bias;                 // logit bias or NULL
    float *x;                          // residual, updated in place
    int32_t *idx;                      // [k] routing out
    float *w;                          // [k] weights out
    uint32_t *flags;                   // [1] VIREO_ROUTE_* bits out, or NULL
    bool norm;
    const float *nw;                   // norm weight or NULL (unit)
    float eps;
    float *hb_out;                     // (norm) hb written here when not NULL
};
int vh_layer_supported(uint32_t tg, uint32_t td, int d, int E, int k, int fe);
int vh_moe_layer(uint32_t tg, uint32_t td, const LayerArgs &a, hipStream_t s);
int vh_layer_xchg(LayerXchg **out);
