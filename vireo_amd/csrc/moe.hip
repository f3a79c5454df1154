// moe_route / moe_dispatch / moe_ffn_forward: host orchestration of the MoE
// kernels (route.hip, moe_decode.hip, moe_grouped.hip, moe_mfma.hip).
//
// Reference: moe_ffn, src/gguf_run.c:185-214. Two execution plans produce its
// result for a batch of independent tokens:
//   decode (one token, or a decode batch of up to kDecodeBatchMax tokens):
//                        router parts -> fused top-k + gate/up SwiGLU ->
//                        down + combine + residual               (3 kernels)
//   grouped (any count): router -> top-k -> dispatch -> grouped gate/up ->
//                        grouped down -> combine + residual      (6 kernels)
// The grouped plan reads each routed expert's weights once per call however
// many tokens chose it. In calls of at least kMfmaMinCall tokens every group
// runs as bf16 matrix-core GEMMs (moe_mfma.hip; 4 more kernels); calls of
// kMdecMinTokens to kMfmaMinCall - 1 tokens with Q4_K_M experts run their
// groups on the matrix cores with exact 16-bit operands (moe_mdec.hip), and
// smaller calls (or other types) on moe_gdec.hip's kernels, which keep a
// group's inputs in registers and stream each weight row once; plan 4 runs
// every call on the fp32 grouped kernels (moe_grouped.hip).
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>
#include "common.h"
#include "route_kernels.h"
#include "vireo_hip.h"

namespace {

// 0 auto, 1 decode plan when possible, 2 grouped plan, 3 decode plan with the
// fused experts kernel, 4 grouped plan without the matrix-core GEMMs
int g_path = 0;
// 1: a pinned layer's first matrix-core decode-batch call copies its experts
// into 16-row tiles (vh_mdec_pack_layer) that later calls read; 0: GGUF rows
int g_packed = 1;
// From this many tokens on, every logit is the reference's exact sequential
// fp32 sum (route_exact_kernel): its latency, one chain of 2 d dependent
// operations, is then hidden by the chains of many tokens. Fewer tokens take
// the certified fp64 parts, whose exact recomputation (route_topk_block) is
// needed for the few tokens whose order the bounds leave open; a token's
// result does not depend on the other tokens of its call either way.
constexpr int kExactRouteTokens = 64;
// From this many tokens on, a decode-batch call's groups run on the matrix
// cores (moe_mdec.hip): a tile takes 16 tokens of an expert, and with two
// tokens per call converting each weight for the fp32 kernels costs less
// than the tile's unused rows. Measured per layer on the packed tiles
// (matrix cores / fp32): OLMoE Q4_K_M B=2 43.2 / 42.7 us, B=3 51.2 / 52.2,
// B=4 54.0 / 67.4, B=6 65.1 / 91.5; Qwen3 Q4_K_M B=2 43.0 / 40.6, B=3
// 48.8 / 49.5, B=4 52.8 / 59.7, B=6 59.6 / 78.9.
constexpr int kMdecMinTokens = 3;
// Calls of 2 to kDecodeBatchMax tokens whose shapes the one-token kernels
// take run the decode plan for every token at once: router parts -> top-k
// and gate/up of the distinct chosen experts -> down + combine per token,
// each token's bits those of a one-token call. Its fp32 arithmetic grows with
// the tokens (a weight is converted again for every token that reads it), so
// on layers whose groups the matrix cores take (moe_mdec.hip) plan 0 uses it
// only up to kDecodeBatchAuto tokens. Measured per layer (decode batch /
// matrix cores, or / fp32 grouped kernels for Q8_0): OLMoE Q4_K_M B=2 32.2 /
// 42.5 us, B=3 42.8 / 48.2, B=4 51.2 / 53.2, B=5 61.3 / 57.8, B=8 96.1 /
// 68.6; Qwen3 Q4_K_M B=2 30.4 / 40.3, B=4 46.3 / 57.2, B=5 55.0 / 59.6, B=6
// 64.2 / 63.3, B=8 84.7 / 69.6; OLMoE Q8_0 B=2 39.9 / 49.2, B=4 62.8 / 74.2,
// B=8 108.4 / 131.1.
constexpr int kDecodeBatchAuto = 4;

bool type_ok(uint32_t t, int n) {
    // the expert formats of the MoE models (Q8_0, Q4_K gate/up, Q6_K down), and
    // the other types the reference's gguf_matmul computes (src/gguf_run.c:
    // 202-208, src/gguf_compute.c:68-82, 183-213), which the grouped fp32
    // kernels take in items of 32 columns
    switch (t) {
    case VT_Q8_0: case VT_Q5_0: case VT_F16: case VT_F32: return n % 32 == 0;
    case VT_Q4_K: case VT_Q6_K: return n % 256 == 0;
    default: return false;
    }
}

int check_model(const vireo_moe_model *m, int layer) {
    if (!m || layer < 0 || layer >= m->n_layers || !m->layers) return -EINVAL;
    const vireo_moe_layer &L = m->layers[layer];
    if (m->dim <= 0 || m->ffn_exp <= 0 || m->n_experts <= 0 || m->n_experts > kMaxExperts) return -EINVAL;
    if (m->n_used < 1 || m->n_used > 64 || m->n_used > m->n_experts) return -EINVAL;
    if (!L.router || L.router->ggml_type != VT_F32 || !L.router->data) return -EINVAL;
    if (reinterpret_cast<uintptr_t>(L.router->data) & 3u) return -EINVAL;
    return 0;
}

size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

struct Ws {
    RoutePart *parts;
    int32_t *idx, *counts, *offs, *perm, *active;
    float *w, *h, *ybuf;
    uint32_t *flags;
    uint32_t *bar;  // decode plan: kFusedBlocks barrier flags, then the token's flag word
    DecodePlan *plan;
    int32_t *tiles, *small;  // matrix-core plan: token tiles, the other groups
    void *hs;                // matrix-core plan: bf16 h rows in dispatch order
    void *xb;                // matrix-core plan: bf16 copy of hb
    void *xp;                // decode-batch matrix-core plan: split inputs [T x d x 4 bytes]
    float *xsc;              // and their per-token scales [T]
    uint32_t *ctr;           // and the down kernel's arrival counters (vh_mdec_ctr_words)
    const void **tab;        // paged plan: [E + 1] expert tables [3 E] (one per batch, then the combine's)
    int32_t *act;            // paged plan: [E] active lists [E + 1] (one per batch)
    int32_t *pidx;           // paged plan: the next layer's guessed routing [T x k]
    float *pw;               // and its weights (unused)
    uint32_t *pflags;        // and flags (unused)
};

// Where a call's workspace comes from: the library's grow-only per-device
// buffer (base == nullptr), or a fixed region of cap bytes that is never
// grown (the scratch of moe_ffn_forward_noalloc).
struct WsSource {
    char *base;
    size_t cap;
};

int get_ws(int T, int E, int k, int d, int fe, bool experts, bool grouped, Ws *ws, bool mfma = false,
           bool paged = false, const WsSource *src = nullptr) {
    const size_t P = size_t(T) * k;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += al256(bytes); return o; };
    const size_t o_parts = take(size_t(T) * E * sizeof(RoutePart));
    const size_t o_idx = take(P * 4), o_w = take(P * 4), o_flags = take(size_t(T) * 4);
    const size_t o_plan = take(sizeof(DecodePlan));
    const size_t o_bar = take((kFusedBlocks + 1) * 4);
    const size_t o_counts = take(size_t(E) * 4), o_offs = take(size_t(E + 1) * 4), o_perm = take(P * 4),
                 o_active = take(size_t(E + 1) * 4);
    const size_t o_h = (experts && !mfma) ? take(P * fe * 4) : 0;  // the matrix cores keep h in hs
    const size_t o_y = (experts && grouped) ? take(P * d * 4) : 0;
    const size_t o_tiles = mfma ? take(size_t(vh_mfma_plan_words(int(P), E)) * 4) : 0;
    const size_t o_small = mfma ? take(size_t(E + 1) * 4) : 0;
    const size_t o_hs = mfma ? take(P * fe * 2) : 0;
    const size_t o_xb = mfma ? take(size_t(T) * d * 2) : 0;
    const bool small = experts && grouped && T < kMfmaMinCall;
    const size_t o_xp = small ? take(vh_mdec_xp_bytes(T, d)) : 0, o_xsc = small ? take(size_t(T) * 4) : 0;
    const size_t o_ctr = small ? take(size_t(vh_mdec_ctr_words(d)) * 4) : 0;
    const size_t ntab = paged ? size_t(E + 1) : 1, nact = paged ? size_t(E) : 1;
    const size_t o_tab = take(ntab * 3 * E * sizeof(void *)), o_act = take(nact * (E + 1) * 4);
    const size_t o_pidx = paged ? take(P * 4) : 0, o_pw = paged ? take(P * 4) : 0,
                 o_pflags = paged ? take(size_t(T) * 4) : 0;
    void *base;
    if (src && src->base) {
        if (off > src->cap) return -E2BIG;
        base = src->base;
    } else if (int rc = vh_device_workspace(off, &base)) {
        return rc;
    }
    char *b = static_cast<char *>(base);
    ws->parts = reinterpret_cast<RoutePart *>(b + o_parts);
    ws->idx = reinterpret_cast<int32_t *>(b + o_idx);
    ws->w = reinterpret_cast<float *>(b + o_w);
    ws->flags = reinterpret_cast<uint32_t *>(b + o_flags);
    ws->plan = reinterpret_cast<DecodePlan *>(b + o_plan);
    ws->bar = reinterpret_cast<uint32_t *>(b + o_bar);
    ws->counts = reinterpret_cast<int32_t *>(b + o_counts);
    ws->offs = reinterpret_cast<int32_t *>(b + o_offs);
    ws->perm = reinterpret_cast<int32_t *>(b + o_perm);
    ws->active = reinterpret_cast<int32_t *>(b + o_active);
    ws->h = (experts && !mfma) ? reinterpret_cast<float *>(b + o_h) : nullptr;
    ws->ybuf = (experts && grouped) ? reinterpret_cast<float *>(b + o_y) : nullptr;
    ws->tiles = mfma ? reinterpret_cast<int32_t *>(b + o_tiles) : nullptr;
    ws->small = mfma ? reinterpret_cast<int32_t *>(b + o_small) : nullptr;
    ws->hs = mfma ? b + o_hs : nullptr;
    ws->xb = mfma ? b + o_xb : nullptr;
    ws->xp = small ? b + o_xp : nullptr;
    ws->xsc = small ? reinterpret_cast<float *>(b + o_xsc) : nullptr;
    ws->ctr = small ? reinterpret_cast<uint32_t *>(b + o_ctr) : nullptr;
    ws->tab = reinterpret_cast<const void **>(b + o_tab);
    ws->act = reinterpret_cast<int32_t *>(b + o_act);
    ws->pidx = paged ? reinterpret_cast<int32_t *>(b + o_pidx) : nullptr;
    ws->pw = paged ? reinterpret_cast<float *>(b + o_pw) : nullptr;
    ws->pflags = paged ? reinterpret_cast<uint32_t *>(b + o_pflags) : nullptr;
    return 0;
}

bool decode_supported(const vireo_moe_model *m, int layer) {
    const vireo_moe_layer &L = m->layers[layer];
    if (!L.gate_exps || !L.up_exps || !L.down_exps) return false;
    const uint32_t tg = L.gate_exps->ggml_type, tu = L.up_exps->ggml_type, td = L.down_exps->ggml_type;
    return tg == tu && vh_decode_gateup_supported(tg, m->dim, m->ffn_exp) &&
           vh_down_combine_supported(td, m->dim, m->ffn_exp, m->n_used);
}

// The layer's expert table: 0 with *table set when its experts are pinned
// (pinning them now when the store holds every layer at once), 1 when the call
// must page its routed experts instead, or -errno. Pinning only a part of the
// model would leave the rest too little room and keep it over budget, so a
// store smaller than the model pages every layer the caller has not pinned.
int layer_table(const vireo_moe_model *m, int layer, const void *const **table) {
    if (!vh_store_valid(m->es)) return -EINVAL;  // NULL, or a store this library did not make
    *table = vh_store_layer_table(m->es, layer);
    if (*table) return 0;
    if (!vh_store_fits_all(m->es)) return 1;
    const int rc = expert_store_pin_layer(m->es, layer, table);
    return rc == -ENOSPC ? 1 : rc;
}

// Where the decode stages keep what they hand to each other.
struct DecodeState {
    RoutePart *parts;  // [E]
    DecodePlan *plan;
    float *h;          // [k x fe]
    uint32_t *bar;     // [kFusedBlocks] barrier flags of the fused kernel, then the token's flag word
    uint32_t *flags() const { return bar + kFusedBlocks; }
};

size_t decode_state_layout(const vireo_moe_model *m, size_t off[4]) {
    size_t o = 0;
    off[0] = o; o += al256(size_t(m->n_experts) * sizeof(RoutePart));
    off[1] = o; o += al256(sizeof(DecodePlan));
    off[2] = o; o += al256(size_t(m->n_used) * m->ffn_exp * sizeof(float));
    off[3] = o; o += al256((kFusedBlocks + 1) * sizeof(uint32_t));
    return o;
}

// Plan 5 (and plan 0 once it is measured faster): the whole layer in one launch.
bool layer_kernel(const vireo_moe_model *m, int layer, const float *xin, const float *x, hipStream_t s) {
    (void)s;
    if (g_path != 5) return false;
    const vireo_moe_layer &L = m->layers[layer];
    if ((reinterpret_cast<uintptr_t>(xin) | reinterpret_cast<uintptr_t>(x) |
         reinterpret_cast<uintptr_t>(L.router->data)) & 15u)
        return false;
    const uint32_t tg = L.gate_exps->ggml_type, td = L.down_exps->ggml_type;
    return vh_layer_supported(tg, td, m->dim, m->n_experts, m->n_used, m->ffn_exp) != 0;
}

// One token through layer `layer` with the layer kernel: xin = hb (norm false)
// or the residual x (norm true, RMSNorm by nw / eps in front; hb_out receives hb).
int run_layer_kernel(const vireo_moe_model *m, int layer, const void *const *table, const float *xin, float *x,
                     bool norm, const float *nw, float eps, float *hb_out, int32_t *idx, float *w, uint32_t *flags,
                     hipStream_t s) {
    const vireo_moe_layer &L = m->layers[layer];
    LayerXchg *xg = nullptr;
    if (int rc = vh_layer_xchg(&xg)) return rc;
    LayerArgs a;
    a.R = static_cast<const float *>(L.router->data);
    a.xin = xin;
    a.table = table;
    a.xg = xg;
    a.E = m->n_experts;
    a.k = m->n_used;
    a.fe = m->ffn_exp;
    a.d = m->dim;
    a.renorm = m->topk_renorm;
    a.bias = L.logit_bias;
    a.x = x;
    a.idx = idx;
    a.w = w;
    a.flags = flags;
    a.norm = norm;
    a.nw = nw;
    a.eps = eps;
    a.hb_out = hb_out;
    return vh_moe_layer(L.gate_exps->ggml_type, L.down_exps->ggml_type, a, s);
}

}  // namespace

// Plans 3 and 5 launch kernels whose workgroups wait for each other with a
// bounded poll: a synchronous call then reads the status word.
bool vh_plan_waits() { return g_path == 3 || g_path == 5; }

namespace {

bool fused(const vireo_moe_model *m, int layer) {
    if (g_path != 3) return false;
    const vireo_moe_layer &L = m->layers[layer];
    return vh_fused_blocks(L.gate_exps->ggml_type, L.down_exps->ggml_type, m->dim, m->n_experts, m->n_used,
                           m->ffn_exp) > 0;
}

// Stage 0: router logits (and the barrier flags cleared). Stage 1: the fused
// experts kernel where it is built for the shapes (x is updated there and
// stage 2 has nothing left to do), else top-k + gate/up. Stage 2: down +
// combine.
int decode_stage(const vireo_moe_model *m, int layer, int stage, const void *const *table, float *x,
                 const float *hb, const DecodeState &st, int32_t *idx, float *w, hipStream_t s,
                 bool allow_fused = true, NormRef nref = NormRef{}) {
    const vireo_moe_layer &L = m->layers[layer];
    const float *R = static_cast<const float *>(L.router->data);
    const int d = m->dim, fe = m->ffn_exp, k = m->n_used, E = m->n_experts;
    const uint32_t tg = L.gate_exps->ggml_type, td = L.down_exps->ggml_type;
    switch (stage) {
    case 0: return vh_route_parts(R, hb, L.logit_bias, d, E, 1, false, st.parts, s, st.bar, kFusedBlocks + 1);
    case 1:
        if (allow_fused && fused(m, layer))
            return vh_decode_experts(tg, td, st.parts, R, hb, L.logit_bias, d, E, k, fe, m->topk_renorm, table, st.h,
                                     st.bar, x, idx, w, nref, s);
        return vh_decode_gateup(tg, st.parts, R, hb, L.logit_bias, d, E, k, fe, m->topk_renorm, table, st.h, idx, w,
                                st.flags(), st.plan, td, nref, s);
    case 2:
        if (allow_fused && fused(m, layer)) return 0;
        return vh_down_combine(td, st.plan, st.h, d, fe, k, x, s);
    default: return -EINVAL;
    }
}

}  // namespace

namespace {
int ffn_forward(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens, int32_t *idx_out,
                float *w_out, hipStream_t s, const WsSource *src, uint32_t *flags_out);
}  // namespace

int vh_moe_layer_normed(const vireo_moe_model *m, int layer, float *x, const float *nw, float eps, float *xb,
                        hipStream_t s, int32_t *idx_out, uint32_t *flags_out) {
    if (int rc = check_model(m, layer)) return rc;
    if (!x || !xb || !m->es) return -EINVAL;
    const bool decode = g_path != 2 && g_path != 4 && decode_supported(m, layer) && m->dim == 2048 &&
                        !((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(xb)) & 15u) &&
                        !(reinterpret_cast<uintptr_t>(m->layers[layer].router->data) & 15u);
    if (!decode) {  // the reference's own RMSNorm, bit for bit, so the routing is certified on its xb
        if (int rc = vh_rmsnorm_ref(xb, x, nw, m->dim, eps, s)) return rc;
        return ffn_forward(m, layer, x, xb, 1, idx_out, nullptr, s, nullptr, flags_out);
    }
    const vireo_moe_layer &L = m->layers[layer];
    const void *const *table = nullptr;
    if (int rc = layer_table(m, layer, &table)) {
        if (rc < 0) return rc;
        if ((rc = vh_rmsnorm_ref(xb, x, nw, m->dim, eps, s))) return rc;
        return ffn_forward(m, layer, x, xb, 1, idx_out, nullptr, s, nullptr, flags_out);  // pages the routed experts
    }
    Ws ws;
    if (int rc = get_ws(1, m->n_experts, m->n_used, m->dim, m->ffn_exp, true, false, &ws)) return rc;
    if (layer_kernel(m, layer, x, x, s)) {  // RMSNorm, router, experts and combine in one launch
        int32_t *idx = idx_out ? idx_out : ws.idx;
        int rc = run_layer_kernel(m, layer, table, x, x, true, nw, eps, xb, idx, ws.w, flags_out, s);
        if (!rc) rc = vh_store_note_routing(m->es, layer, idx, 1, m->n_used, s);
        return rc;
    }
    const DecodeState st{ws.parts, ws.plan, ws.h, ws.bar};
    int rc = vh_route_parts_norm(static_cast<const float *>(L.router->data), x, nw, eps, xb, L.logit_bias, m->dim,
                                 m->n_experts, 1, st.parts, s, st.bar, kFusedBlocks + 1);
    int32_t *idx = idx_out ? idx_out : ws.idx;
    // hb is the fp64-normalised x: the router parts carry the widened bounds
    // (route_part_on_own_norm) and an uncertified token is ranked on the
    // reference's own xb, recomputed from x
    NormRef nref;
    nref.x = x;
    nref.nw = nw;
    nref.eps = eps;
    for (int stage = 1; stage < 3 && !rc; stage++)
        rc = decode_stage(m, layer, stage, table, x, xb, st, idx, ws.w, s, true, nref);
    if (!rc && flags_out) rc = vh_check(hipMemcpyAsync(flags_out, st.flags(), 4, hipMemcpyDeviceToDevice, s));
    if (!rc) rc = vh_store_note_routing(m->es, layer, idx, 1, m->n_used, s);
    return rc;
}

extern "C" int64_t moe_decode_state_bytes(const vireo_moe_model *m) {
    if (check_model(m, 0) || !decode_supported(m, 0)) return -EINVAL;
    size_t off[4];
    return int64_t(decode_state_layout(m, off));
}

extern "C" int moe_decode_stage(const vireo_moe_model *m, int layer, int stage, float *x, const float *hb, void *state,
                                int32_t *idx_out, float *w_out, void *stream) {
    if (int rc = check_model(m, layer)) return rc;
    if (!decode_supported(m, layer) || !state || !hb || stage < 0 || stage > 2) return -EINVAL;
    if (reinterpret_cast<uintptr_t>(hb) & 15u) return -EINVAL;  // the decode kernels read hb in 16-byte units
    if (stage == 2 && !x) return -EINVAL;
    if (reinterpret_cast<uintptr_t>(state) & 255u) return -EINVAL;
    if (!vh_store_valid(m->es)) return -EINVAL;
    const void *const *table = nullptr;
    if (int rc = expert_store_pin_layer(m->es, layer, &table)) return rc;
    size_t off[4];
    decode_state_layout(m, off);
    char *b = static_cast<char *>(state);
    const DecodeState st{reinterpret_cast<RoutePart *>(b + off[0]), reinterpret_cast<DecodePlan *>(b + off[1]),
                         reinterpret_cast<float *>(b + off[2]), reinterpret_cast<uint32_t *>(b + off[3])};
    if (stage == 1 && !x && fused(m, layer)) return -EINVAL;  // the fused stage 1 updates x
    int32_t *idx = idx_out;
    float *w = w_out;
    Ws ws;
    if (stage == 1 && (!idx || !w)) {  // the kernel always writes the routing somewhere
        if (int rc = get_ws(1, m->n_experts, m->n_used, m->dim, m->ffn_exp, false, false, &ws)) return rc;
        if (!idx) idx = ws.idx;
        if (!w) w = ws.w;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = vh_finish(s, decode_stage(m, layer, stage, table, x, hb, st, idx, w, s));
    if (!rc && !s && stage == 1 && fused(m, layer)) rc = vh_take_status(s);  // a grid-wide wait that gave up
    return rc;
}

extern "C" int moe_decode_stage_timed(const vireo_moe_model *m, int stage, int n, const int *layers, float *x,
                                      const float *hb, void *states, int64_t state_stride, int32_t *idx, float *w,
                                      float *us_out, void *stream) {
    if (int rc = check_model(m, 0)) return rc;
    if (n <= 0 || !layers || !hb || !states || !idx || !w || !us_out || stage < 0 || stage > 2) return -EINVAL;
    if (stage > 0 && !x) return -EINVAL;
    if (reinterpret_cast<uintptr_t>(hb) & 15u || (m->dim * 4) & 15) return -EINVAL;
    size_t off[4];
    if (!decode_supported(m, 0) || state_stride < int64_t(decode_state_layout(m, off)) || (state_stride & 255) ||
        (reinterpret_cast<uintptr_t>(states) & 255u))
        return -EINVAL;
    static hipEvent_t *ev = nullptr;
    static int nev = 0;
    if (2 * n > nev) {
        hipEvent_t *ne = static_cast<hipEvent_t *>(realloc(ev, sizeof(hipEvent_t) * 2 * n));
        if (!ne) return -ENOMEM;
        ev = ne;
        for (; nev < 2 * n; nev++)
            if (int rc = vh_check(hipEventCreate(&ev[nev]))) return rc;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int d = m->dim, k = m->n_used;
    int rc = 0;
    for (int i = 0; i < n && !rc; i++) {
        const int layer = layers[i];
        if (layer < 0 || layer >= m->n_layers || !decode_supported(m, layer)) { rc = -EINVAL; break; }
        const void *const *table = nullptr;
        if ((rc = expert_store_pin_layer(m->es, layer, &table))) break;
        char *b = static_cast<char *>(states) + i * state_stride;
        const DecodeState st{reinterpret_cast<RoutePart *>(b + off[0]), reinterpret_cast<DecodePlan *>(b + off[1]),
                             reinterpret_cast<float *>(b + off[2]), reinterpret_cast<uint32_t *>(b + off[3])};
        us_out[i] = (stage == 2 && fused(m, layer)) ? -1.0f : 0.0f;  // -1: no kernel to time (done in stage 1)
        g_vh_timing = {ev[2 * i], ev[2 * i + 1]};
        rc = decode_stage(m, layer, stage, table, x ? x + size_t(i) * d : nullptr, hb + size_t(i) * d, st,
                          idx + size_t(i) * k, w + size_t(i) * k, s);
        g_vh_timing = {nullptr, nullptr};
    }
    if (!rc) rc = vh_check(hipStreamSynchronize(s));
    for (int i = 0; i < n && !rc; i++) {
        if (us_out[i] < 0.0f) {
            us_out[i] = 0.0f;
            continue;
        }
        float ms = 0.0f;
        rc = vh_check(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
        us_out[i] = ms * 1000.0f;
    }
    return rc;
}

extern "C" int moe_decode_phases(const vireo_moe_model *m, int n, const int *layers, float *x, const float *hb,
                                 uint64_t *stamps, void *stream) {
    if (int rc = check_model(m, 0)) return rc;
    if (n <= 0 || !layers || !x || !hb || !stamps || (reinterpret_cast<uintptr_t>(stamps) & 7u)) return -EINVAL;
    for (int i = 0; i < n; i++)
        if (layers[i] < 0 || layers[i] >= m->n_layers) return -EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int d = m->dim;
    int rc = 0;
    for (int i = 0; i < n && !rc; i++) {
        g_vh_stamps = stamps + size_t(i) * kStampKernels * kStampBlocks * kStampSlots;
        rc = ffn_forward(m, layers[i], x + size_t(i) * d, hb + size_t(i) * d, 1, nullptr, nullptr, s, nullptr,
                         nullptr);
        g_vh_stamps = nullptr;
    }
    return vh_finish(s, rc);
}

// The tiled copy of a pinned layer's experts for the matrix-core decode batch,
// made on the first call that may allocate (never under graph capture) and
// held by the store with the pin; NULL: read the GGUF rows.
// kind 0: the decode batch's tiles (vh_mdec_pack_layer), 1: the prefill
// GEMMs' Q8_0 row octets (vh_mfma_pack_q8).
const void *const *packed_table(const vireo_moe_model *m, int layer, const void *const *table, bool may_alloc,
                                hipStream_t s, int kind = 0) {
    if (!g_packed) return nullptr;
    const void *const *pt = vh_store_packed_table(m->es, layer, kind);
    if (pt || !may_alloc) return pt;
    const int E = m->n_experts, d = m->dim, fe = m->ffn_exp;
    const uint64_t bytes = kind ? vh_mfma_pack_bytes(E, d, fe) : vh_mdec_pack_bytes(E, d, fe);
    void *buf = vh_store_packed_begin(m->es, layer, kind, bytes);
    if (!buf) return nullptr;  // over the store's capacity: read the GGUF rows
    void *tab = nullptr;
    int rc = kind ? vh_mfma_pack_q8(table, E, d, fe, buf, &tab, s) : vh_mdec_pack_layer(table, E, d, fe, buf, &tab, s);
    if (!rc) rc = vh_store_set_packed(m->es, layer, kind, tab);
    if (rc) {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(s);
        if (tab) (void)hipFree(tab);
        vh_store_packed_abort(m->es, layer, kind);
        return nullptr;
    }
    return static_cast<const void *const *>(tab);
}

extern "C" int vireo_hip_set_packed(int on) {
    if (on != 0 && on != 1) return -EINVAL;
    g_packed = on;
    return 0;
}

extern "C" int vireo_hip_set_path(int path) {
    if (path < 0 || path > 5) return -EINVAL;
    g_path = path;
    return 0;
}

extern "C" int moe_route(const vireo_moe_model *m, int layer, const float *hb, int n_tokens, int32_t *idx, float *w,
                         uint32_t *flags, float *probs, void *stream) {
    if (int rc = check_model(m, layer)) return rc;
    if (n_tokens < 0 || (n_tokens && (!hb || !idx || !w))) return -EINVAL;
    if (n_tokens == 0) return 0;
    if (n_tokens > 65535) return -E2BIG;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vireo_moe_layer &L = m->layers[layer];
    const float *R = static_cast<const float *>(L.router->data);
    Ws ws;
    if (int rc = get_ws(n_tokens, m->n_experts, m->n_used, m->dim, m->ffn_exp, false, false, &ws)) return rc;
    const bool exact = n_tokens >= kExactRouteTokens;
    int rc = vh_route_parts(R, hb, L.logit_bias, m->dim, m->n_experts, n_tokens, exact, ws.parts, s);
    if (!rc) rc = vh_route_finish(ws.parts, R, hb, L.logit_bias, m->dim, m->n_experts, m->n_used, m->topk_renorm,
                                  exact, n_tokens, idx, w, flags, probs, s);
    return vh_finish(s, rc);
}

extern "C" int moe_dispatch(const int32_t *idx, int n_tokens, int k, int n_experts, int32_t *counts, int32_t *offs,
                            int32_t *perm, void *stream) {
    if (n_tokens < 0 || k < 1 || n_experts < 1 || n_experts > kMaxExperts) return -EINVAL;
    if (!counts || !offs || (n_tokens && (!idx || !perm))) return -EINVAL;
    const int64_t P = int64_t(n_tokens) * k;
    if (P > (int64_t(1) << 30)) return -E2BIG;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return vh_finish(s, vh_dispatch(idx, int(P), n_experts, counts, offs, perm, nullptr, s));
}

// moe_ffn_forward when the ExpertStore does not hold every layer at once. The
// reference looks each routed expert up in turn and releases it after use
// (src/gguf_run.c:193-213), so a store of any size serves it. Here the routing
// and the dispatch run on the device; the per-expert counts and the routing
// come back to the host (the routing also feeds the store's statistics), and
// the routed experts are taken in batches that fit the room the store has
// beside the experts that hold leases: look the batch up (misses are read from
// the store's file into pinned staging while earlier batches compute, and
// copied to HBM on the copy stream), make the compute stream wait for those
// copies, run the grouped projections on the batch, and drop its leases at
// once - every block the batch read carries an event recorded after its
// kernels, and a later page-in into that block waits for it. The combine runs
// once all batches have written their rows. The stream is synchronized once
// (the host needs the routing), so such a call cannot be captured in a graph.
//
// Prefetch (the reference lists it as open, ROADMAP.md:46-47): a call of at
// most 8 tokens also applies the next layer's router to this call's hb - the
// residual stream changes little from one layer to the next - and hands the
// guessed experts, most likely first, to the store. The next call on that
// layer reads the guessed experts that are not resident while the device
// runs the kernels before its routing (the previous layer's experts, this
// layer's router), and stops as soon as its routing has landed: the host is
// otherwise idle then. A wrong guess costs pool room and copy bandwidth, never
// a result; the reference's statistics do not see guesses.
int paged_events(hipEvent_t **out) {
    static hipEvent_t ev[64][2];
    int dev = 0;
    if (int rc = vh_check(hipGetDevice(&dev))) return rc;
    if (dev < 0 || dev >= 64) return -ENODEV;
    for (int i = 0; i < 2; i++)
        if (!ev[dev][i] && vh_check(hipEventCreateWithFlags(&ev[dev][i], hipEventDisableTiming))) {
            ev[dev][i] = nullptr;
            return -EIO;
        }
    *out = ev[dev];
    return 0;
}

constexpr int kPrefetchIds = 64;  // guessed (token, rank) pairs per call at most

int paged_forward(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens, int32_t *idx_out,
                  float *w_out, hipStream_t s, uint32_t *flags_out) {
    const vireo_moe_layer &L = m->layers[layer];
    const uint32_t tg = L.gate_exps->ggml_type, td = L.down_exps->ggml_type;
    const int d = m->dim, fe = m->ffn_exp, k = m->n_used, E = m->n_experts;
    const int P = n_tokens * k, slots = P < E ? P : E;
    Ws ws;
    if (int rc = get_ws(n_tokens, E, k, d, fe, true, true, &ws, false, true)) return rc;
    int32_t *idx = idx_out ? idx_out : ws.idx;
    float *w = w_out ? w_out : ws.w;
    const float *R = static_cast<const float *>(L.router->data);
    const bool exact = n_tokens >= kExactRouteTokens;
    const bool mdec = n_tokens >= kMdecMinTokens && n_tokens < kMfmaMinCall && g_path != 4 &&
                      vh_mdec_supported(tg, td, d, fe);
    int rc = mdec ? vh_route_parts_tiled(R, hb, L.logit_bias, d, E, n_tokens, ws.parts, ws.xp, ws.xsc, s) : -EINVAL;
    const bool prepped = rc == 0;
    if (rc == -EINVAL) rc = vh_route_parts(R, hb, L.logit_bias, d, E, n_tokens, exact, ws.parts, s);
    if (!rc) rc = vh_route_finish(ws.parts, R, hb, L.logit_bias, d, E, k, m->topk_renorm, exact, n_tokens, idx, w,
                                  ws.flags, nullptr, s);
    if (!rc) rc = vh_dispatch(idx, P, E, ws.counts, ws.offs, ws.perm, ws.active, s);
    if (!rc && flags_out)
        rc = vh_check(hipMemcpyAsync(flags_out, ws.flags, size_t(n_tokens) * 4, hipMemcpyDeviceToDevice, s));
    // pinned host memory: counts [E], routing [P], then per batch a table [3 E]
    // and an active list [E + 1], then the combine's table [3 E]
    const size_t tab_n = size_t(3) * E, act_n = size_t(E) + 1;
    const size_t o_idx = al256(size_t(E) * 4), o_tabs = o_idx + al256(size_t(P) * 4),
                 o_acts = o_tabs + al256(size_t(E + 1) * tab_n * sizeof(void *)),
                 o_pred = o_acts + al256(size_t(E) * act_n * 4), host_bytes = o_pred + size_t(P) * 4;
    const int nl = layer + 1;
    const bool predict = P <= kPrefetchIds && nl < m->n_layers && vh_store_prefetching(m->es) &&
                         m->layers[nl].router && m->layers[nl].router->data;
    void *hst = nullptr;
    if (!rc) rc = vh_host_staging(host_bytes, &hst);
    if (rc) return rc;
    char *hb8 = static_cast<char *>(hst);
    int32_t *counts = reinterpret_cast<int32_t *>(hb8);
    int32_t *idx_h = reinterpret_cast<int32_t *>(hb8 + o_idx);
    const void **tabs_h = reinterpret_cast<const void **>(hb8 + o_tabs);
    int32_t *acts_h = reinterpret_cast<int32_t *>(hb8 + o_acts);
    int32_t *pred_h = reinterpret_cast<int32_t *>(hb8 + o_pred);
    hipEvent_t *ev = nullptr;
    rc = paged_events(&ev);
    if (!rc) rc = vh_check(hipMemcpyAsync(counts, ws.counts, size_t(E) * 4, hipMemcpyDeviceToHost, s));
    if (!rc) rc = vh_check(hipMemcpyAsync(idx_h, idx, size_t(P) * 4, hipMemcpyDeviceToHost, s));
    if (!rc) rc = vh_check(hipEventRecord(ev[0], s));
    if (!rc && predict) {  // the next layer's router on this hb: a guess of its routing
        const vireo_moe_layer &N = m->layers[nl];
        const float *RN = static_cast<const float *>(N.router->data);
        rc = vh_route_parts(RN, hb, N.logit_bias, d, E, n_tokens, false, ws.parts, s);
        if (!rc) rc = vh_route_finish(ws.parts, RN, hb, N.logit_bias, d, E, k, m->topk_renorm, false, n_tokens,
                                      ws.pidx, ws.pw, ws.pflags, nullptr, s);
        if (!rc) rc = vh_check(hipMemcpyAsync(pred_h, ws.pidx, size_t(P) * 4, hipMemcpyDeviceToHost, s));
        if (!rc) rc = vh_check(hipEventRecord(ev[1], s));
    }
    hipStream_t cs = nullptr;
    if (!rc) rc = vh_copy_stream(&cs);
    // while the routing is on its way: read the experts an earlier call guessed for this layer
    while (!rc && hipEventQuery(ev[0]) == hipErrorNotReady) {
        const int r = vh_store_prefetch_next(m->es, layer, cs);
        if (r < 0) rc = r;
        if (r <= 0) break;
    }
    (void)hipGetLastError();  // a query that found the copy not done yet is no error
    if (!rc) rc = vh_check(hipEventSynchronize(ev[0]));
    if (rc) {
        (void)hipStreamSynchronize(s);  // no copy may still target the host staging
        (void)vh_host_staging_done(s);
        return rc;
    }
    vh_store_note_routing_host(m->es, layer, idx_h, n_tokens, k);
    const uint64_t cap = vh_store_capacity(m->es), leased = vh_store_leased_bytes(m->es);
    const uint64_t room = cap > leased ? cap - leased : 1;  // cap 0: unbounded (room unused)
    const bool gdec = !mdec && n_tokens < kMfmaMinCall && vh_gdec_supported(tg, td, d, fe, hb);
    if (mdec && !prepped) rc = vh_mdec_prep(hb, n_tokens, d, ws.xp, ws.xsc, s);
    const void **present = tabs_h + size_t(E) * tab_n;  // the combine's table (the last one)
    memset(present, 0, tab_n * sizeof(void *));
    ExpertView views[kMaxExperts];
    int e0 = 0, nb = 0;
    while (!rc) {
        while (e0 < E && counts[e0] == 0) e0++;
        if (e0 == E) break;
        // the next batch: routed experts in id order while their bytes fit (at least one)
        const void **tab = tabs_h + size_t(nb) * tab_n;
        int32_t *act = acts_h + size_t(nb) * act_n;
        int n = 0, e1 = e0;
        uint64_t bytes = 0;
        for (; e1 < E; e1++) {
            if (counts[e1] == 0) continue;
            const uint64_t b = vh_store_expert_bytes(m->es, layer, e1);
            if (n && cap && bytes + b > room) break;
            bytes += b;
            act[n++] = e1;
        }
        memset(tab, 0, tab_n * sizeof(void *));
        int got = 0;
        for (int i = 0; i < n && !rc; i++) {
            const int e = act[i];
            const int lr = vh_store_acquire(m->es, layer, e, &views[e], cs);
            if (lr == -1) continue;  // unregistered: skipped (src/gguf_run.c:201)
            if (lr) { rc = lr; break; }
            tab[3 * e] = views[e].gate;
            tab[3 * e + 1] = views[e].up;
            tab[3 * e + 2] = views[e].down;
            present[3 * e + 2] = views[e].down;
            act[got++] = e;
        }
        act[E] = got;
        if (!rc && got) {
            const void **dt = ws.tab + size_t(nb) * tab_n;
            int32_t *da = ws.act + size_t(nb) * act_n;
            rc = vh_store_copy_fence(m->es, cs, s);  // the batch's page-ins land before its kernels
            if (!rc) rc = vh_check(hipMemcpyAsync(dt, tab, tab_n * sizeof(void *), hipMemcpyHostToDevice, s));
            if (!rc) rc = vh_check(hipMemcpyAsync(da, act, act_n * 4, hipMemcpyHostToDevice, s));
            if (mdec) {
                if (!rc) rc = vh_mdec_gateup(ws.counts, ws.offs, ws.perm, da, dt, false, ws.xp, ws.xsc, n_tokens, d,
                                             fe, k, E, slots, n_tokens, ws.h, s);
                if (!rc) rc = vh_mdec_down(ws.counts, ws.offs, ws.perm, da, dt, false, ws.h, d, fe, E, slots,
                                           n_tokens, ws.ybuf, s);
            } else if (gdec) {
                if (!rc) rc = vh_gdec_gateup(tg, ws.counts, ws.offs, ws.perm, da, dt, hb, d, fe, k, E, slots, n_tokens, ws.h, s);
                if (!rc) rc = vh_gdec_down(td, ws.counts, ws.offs, ws.perm, da, dt, ws.h, d, fe, E, slots, n_tokens, ws.ybuf, s);
            } else {
                if (!rc) rc = vh_grouped_gateup(tg, ws.counts, ws.offs, ws.perm, da, dt, hb, d, fe, k, E, slots, ws.h, s);
                if (!rc) rc = vh_grouped_down(td, ws.counts, ws.offs, ws.perm, da, dt, ws.h, d, fe, E, slots, ws.ybuf, s);
            }
        }
        if (rc) (void)hipStreamSynchronize(s);  // nothing enqueued may outlive the leases dropped below
        for (int i = 0; i < got; i++) {
            const int dr = vh_store_drop(m->es, &views[act[i]], s);
            if (!rc) rc = dr;
        }
        nb++;
        e0 = e1;
    }
    // the combine reads only whether each expert was found
    const void **dt = ws.tab + size_t(nb) * tab_n;
    if (!rc) rc = vh_check(hipMemcpyAsync(dt, present, tab_n * sizeof(void *), hipMemcpyHostToDevice, s));
    if (!rc) rc = vh_combine(idx, w, dt, ws.ybuf, d, k, n_tokens, x, s);
    if (!rc && predict) {  // hand the guess to the store, every token's first choice first
        rc = vh_check(hipEventSynchronize(ev[1]));
        int32_t hint[kPrefetchIds];
        for (int j = 0; j < k; j++)
            for (int t = 0; t < n_tokens; t++) hint[j * n_tokens + t] = pred_h[t * k + j];
        if (!rc) vh_store_hint(m->es, nl, hint, P);
    }
    const int hr = vh_host_staging_done(s);
    return rc ? rc : hr;
}

namespace {

// moe_ffn_forward; with src, on a fixed workspace and allocating nothing: the
// layer must already be pinned (the paged plan and the first pin allocate),
// the fused plan is not used (its status word is allocated on first use) and
// the routing is not copied for the store's statistics (its host ring is).
int ffn_forward(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens, int32_t *idx_out,
                float *w_out, hipStream_t s, const WsSource *src, uint32_t *flags_out) {
    if (int rc = check_model(m, layer)) return rc;
    if (n_tokens < 0 || (n_tokens && (!x || !hb))) return -EINVAL;
    if (n_tokens == 0) return 0;
    const vireo_moe_layer &L = m->layers[layer];
    if (!L.gate_exps || !L.up_exps || !L.down_exps) return -EINVAL;
    const uint32_t tg = L.gate_exps->ggml_type, tu = L.up_exps->ggml_type, td = L.down_exps->ggml_type;
    const int d = m->dim, fe = m->ffn_exp, k = m->n_used, E = m->n_experts;
    if (tg != tu || !type_ok(tg, d) || !type_ok(td, fe) || fe % 4) return -EINVAL;
    if (int64_t(n_tokens) * k > 65535 || n_tokens > 65535) return -E2BIG;
    const void *const *table = nullptr;
    if (src) {
        if (!vh_store_valid(m->es) || !(table = vh_store_layer_table(m->es, layer))) return -EINVAL;
    } else if (int lt = layer_table(m, layer, &table)) {
        if (lt < 0) return lt;
        // the store does not hold every layer: page the routed experts per call
        return vh_finish(s, paged_forward(m, layer, x, hb, n_tokens, idx_out, w_out, s, flags_out));
    }
    const float *R = static_cast<const float *>(L.router->data);

    const bool decode = n_tokens == 1 && g_path != 2 && g_path != 4 && decode_supported(m, layer) &&
                        (reinterpret_cast<uintptr_t>(hb) & 15u) == 0;
    const int batch_max = g_path == 1   ? kDecodeBatchMax
                          : g_path == 0 ? (vh_mdec_supported(tg, td, d, fe) ? kDecodeBatchAuto : kDecodeBatchMax)
                                        : 0;
    const bool dbatch = n_tokens >= 2 && n_tokens <= batch_max && decode_supported(m, layer) &&
                        vh_decode_batch_supported(tg, d, fe, E, k, n_tokens) &&
                        (reinterpret_cast<uintptr_t>(hb) & 15u) == 0;
    const bool mfma = !decode && !dbatch && g_path != 4 && n_tokens >= kMfmaMinCall &&
                      vh_mfma_supported(tg, td, d, fe, E) && (reinterpret_cast<uintptr_t>(hb) & 15u) == 0;
    Ws ws;
    if (int rc = get_ws(n_tokens, E, k, d, fe, true, !decode && !dbatch, &ws, mfma, false, src)) return rc;
    int32_t *idx = idx_out ? idx_out : ws.idx;
    float *w = w_out ? w_out : ws.w;
    int rc;
    if (decode && !src && layer_kernel(m, layer, hb, x, s)) {  // the whole layer in one launch
        rc = run_layer_kernel(m, layer, table, hb, x, false, nullptr, 0.0f, nullptr, idx, w, flags_out, s);
        if (!rc) rc = vh_store_note_routing(m->es, layer, idx, 1, k, s);
        rc = vh_finish(s, rc);
        if (!rc && !s) rc = vh_take_status(s);  // a grid-wide wait that gave up
        return rc;
    }
    if (decode) {
        const DecodeState st{ws.parts, ws.plan, ws.h, ws.bar};
        rc = 0;
        for (int stage = 0; stage < 3 && !rc; stage++)
            rc = decode_stage(m, layer, stage, table, x, hb, st, idx, w, s, !src);
        if (!rc && flags_out) rc = vh_check(hipMemcpyAsync(flags_out, st.flags(), 4, hipMemcpyDeviceToDevice, s));
        if (!rc && !src) rc = vh_store_note_routing(m->es, layer, idx, 1, k, s);
        rc = vh_finish(s, rc);
        if (!rc && !s && !src && fused(m, layer)) rc = vh_take_status(s);  // a grid-wide wait that gave up
        return rc;
    }
    if (dbatch) {  // the decode plan for every token at once
        rc = vh_route_parts(R, hb, L.logit_bias, d, E, n_tokens, false, ws.parts, s);
        if (!rc)
            rc = vh_decode_batch_gateup(tg, ws.parts, R, hb, L.logit_bias, d, E, k, fe, m->topk_renorm, table, ws.h,
                                        idx, w, flags_out ? flags_out : ws.flags, ws.plan, n_tokens, s);
        if (!rc) rc = vh_down_combine(td, ws.plan, ws.h, d, fe, k, x, s, n_tokens);
        if (!rc && !src) rc = vh_store_note_routing(m->es, layer, idx, n_tokens, k, s);
        return vh_finish(s, rc);
    }
    const bool exact = n_tokens >= kExactRouteTokens;
    const int P = n_tokens * k, slots = P < E ? P : E;
    const bool mdec = !mfma && n_tokens >= kMdecMinTokens && n_tokens < kMfmaMinCall && g_path != 4 &&
                      vh_mdec_supported(tg, td, d, fe);
    // the matrix-core decode batch's split inputs come with the router parts where the tiled kernel runs
    rc = mdec ? vh_route_parts_tiled(R, hb, L.logit_bias, d, E, n_tokens, ws.parts, ws.xp, ws.xsc, s) : -EINVAL;
    const bool prepped = rc == 0;
    if (rc == -EINVAL) rc = vh_route_parts(R, hb, L.logit_bias, d, E, n_tokens, exact, ws.parts, s);
    if (!rc) rc = vh_route_finish(ws.parts, R, hb, L.logit_bias, d, E, k, m->topk_renorm, exact, n_tokens, idx, w,
                                  ws.flags, nullptr, s);
    // the matrix-core decode batch finds each expert's tokens itself
    // (the matrix-core plan lists its groups itself: no active list)
    if (!rc && !mdec) rc = vh_dispatch(idx, P, E, ws.counts, ws.offs, ws.perm, mfma ? nullptr : ws.active, s);
    if (!rc && flags_out)
        rc = vh_check(hipMemcpyAsync(flags_out, ws.flags, size_t(n_tokens) * 4, hipMemcpyDeviceToDevice, s));
    if (mfma) {  // every group on the matrix cores (its small list stays empty)
        const int mt = vh_mfma_max_tiles(P, E);
        // Q8_0 experts of a pinned layer: the fragment copy (made on the first such call that may allocate)
        const void *const *pt =
            (!rc && tg == VT_Q8_0 && td == VT_Q8_0) ? packed_table(m, layer, table, !src, s, 1) : nullptr;
        // the tile plan and the GEMMs' bf16 inputs in one launch
        if (!rc) rc = vh_mfma_plan(ws.counts, E, P, 1, tg, td, d, fe, ws.tiles, ws.small, hb, ws.xb,
                                   int64_t(n_tokens) * d, s);
        const void *const *tb = pt ? pt : table;
        if (!rc) rc = vh_mfma_gateup(tg, ws.tiles, mt, ws.counts, ws.offs, ws.perm, tb, pt != nullptr, ws.xb, d, fe, k,
                                     ws.hs, s);
        if (!rc) rc = vh_mfma_down(td, ws.tiles, mt, ws.counts, ws.offs, ws.perm, tb, pt != nullptr, ws.hs, d, fe,
                                   ws.ybuf, s);
    } else if (mdec) {
        // calls of a decode batch's size, Q4_K_M experts: the matrix cores
        if (!rc && !prepped) rc = vh_mdec_prep(hb, n_tokens, d, ws.xp, ws.xsc, s);
        const void *const *pt = rc ? nullptr : packed_table(m, layer, table, !src, s);
        const void *const *tb = pt ? pt : table;
        // no dispatch and no combine kernel: the gate/up and down kernels take
        // their experts' tokens from idx, and the down kernel combines into x
        const MdecSelf sf{idx, w, x, ws.ctr, vh_mdec_ctr_words(d), n_tokens, k};
        if (!rc) rc = vh_mdec_gateup(ws.counts, ws.offs, ws.perm, ws.active, tb, pt != nullptr, ws.xp, ws.xsc,
                                     n_tokens, d, fe, k, E, slots, n_tokens, ws.h, s, &sf);
        if (!rc) rc = vh_mdec_down(ws.counts, ws.offs, ws.perm, ws.active, tb, pt != nullptr, ws.h, d, fe, E, slots,
                                   n_tokens, ws.ybuf, s, &sf);
    } else if (n_tokens < kMfmaMinCall && vh_gdec_supported(tg, td, d, fe, hb)) {
        // calls of a decode batch's size (a few tokens per group): inputs in registers
        if (!rc) rc = vh_gdec_gateup(tg, ws.counts, ws.offs, ws.perm, ws.active, table, hb, d, fe, k, E, slots, n_tokens, ws.h, s);
        if (!rc) rc = vh_gdec_down(td, ws.counts, ws.offs, ws.perm, ws.active, table, ws.h, d, fe, E, slots, n_tokens, ws.ybuf, s);
    } else {
        if (!rc) rc = vh_grouped_gateup(tg, ws.counts, ws.offs, ws.perm, ws.active, table, hb, d, fe, k, E, slots, ws.h, s);
        if (!rc) rc = vh_grouped_down(td, ws.counts, ws.offs, ws.perm, ws.active, table, ws.h, d, fe, E, slots, ws.ybuf, s);
    }
    if (!rc && !mdec) rc = vh_combine(idx, w, table, ws.ybuf, d, k, n_tokens, x, s);
    if (!rc && !src) rc = vh_store_note_routing(m->es, layer, idx, n_tokens, k, s);
    return vh_finish(s, rc);
}

// The workspace of moe_ffn_forward_noalloc: a fixed region of device memory
// in the library's code object (each device holds its own copy until the
// process ends), shared by every such call on a device.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
void *g_scratch_dev[64];  // per device: scratch's device address (host code never uses the symbol itself)

}  // namespace

// Look up this device's address of `scratch` once (from vireo_hip_init, or the
// first moe_ffn_forward_noalloc on a device).
int vh_noalloc_setup(void **out) {
    int dev = 0;
    if (int rc = vh_check(hipGetDevice(&dev))) return rc;
    if (dev < 0 || dev >= 64) return -ENODEV;
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        if (int rc = vh_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))) return rc;
        if (!p) return -EIO;
        g_scratch_dev[dev] = p;
    }
    if (out) *out = g_scratch_dev[dev];
    return 0;
}

extern "C" int moe_ffn_forward(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens,
                               int32_t *idx_out, float *w_out, void *stream) {
    return ffn_forward(m, layer, x, hb, n_tokens, idx_out, w_out, static_cast<hipStream_t>(stream), nullptr,
                       nullptr);
}

extern "C" int moe_ffn_forward_noalloc(const vireo_moe_model *m, int layer, float *x, const float *hb, int n_tokens,
                                       int32_t *idx_out, float *w_out, void *stream) {
    void *base = nullptr;
    if (int rc = vh_noalloc_setup(&base)) return rc;
    const WsSource src{static_cast<char *>(base), kNoAllocScratchBytes};
    return ffn_forward(m, layer, x, hb, n_tokens, idx_out, w_out, static_cast<hipStream_t>(stream), &src,
                       nullptr);
}
