/* KV cache on the GPU: the reference's KVStore (src/kvstore.h) with its
 * vectors in device memory.
 *
 * Its configuration and statistics structs have the layout of the reference's
 * KVConfig / KVStats (src/kvstore.h:26-45) under names of their own
 * (VireoKVConfig, VireoKVStats), so this header and src/kvstore.h can be
 * included in either order; a caller holding a KVConfig copies it field by
 * field (or passes it through a cast: the members, types and order are the same).
 *
 * A store keeps, per "layer" (the reference indexes layer * n_kv_heads +
 * kv_head), the keys and values appended so far in blocks of
 * cfg.block_tokens tokens in HBM. kvstore_ooc semantics (src/kvstore_ooc.c):
 *   - a paged store holds at most cfg.capacity_bytes of blocks in HBM (0 =
 *     unbounded); the sinks (the first ceil(sink_tokens / G) blocks), the
 *     recent window (the last ceil(window_tokens / G)) and the block being
 *     written stay resident; to make room the least recently used other
 *     block without a lease is spilled to host memory, and paged back when a
 *     query selects it;
 *   - a query attends to the blocks its strategy selects plus the sinks and
 *     the window, in ascending block order (VIREO_KV_SELECT_ALL: every block,
 *     the dense store's result; _RECENT: sinks and window only; _TOPK: the
 *     `budget` other blocks whose running mean key scores highest against
 *     the query, src/select/select_topk.c);
 *   - the statistics count as the reference's do.
 * A dense store (vireo_kv_create_dense) is a paged store with unbounded
 * capacity and every block selected (src/kvstore_dense.c).
 *
 * Attention is the reference's softmax(q . k / sqrt(kv_dim)) . v over the
 * selected tokens (src/kvstore.h:68-99), computed in fp32 in parallel: the
 * result agrees with the reference's sequential online softmax to rounding,
 * and is the same bits whether a block was resident, spilled or paged back.
 *
 * Vectors (k, v, q, out) are device pointers. Calls enqueue on the given
 * stream (NULL: the null stream, synchronously); every call on a store must use
 * the same stream. A TOPK query copies its block scores to the host and so
 * synchronizes that stream. Not thread-safe, like the reference. */
#ifndef VIREO_KV_H
#define VIREO_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KVConfig (src/kvstore.h:26-33): same members, types and order */
typedef struct {
    int n_layers;
    int kv_dim;              /* length of each key and value vector        */
    int block_tokens;        /* tokens grouped per block (G)               */
    int sink_tokens;         /* always-resident attention sinks (prefix)   */
    int window_tokens;       /* always-resident recent window              */
    uint64_t capacity_bytes; /* budget for resident blocks (0 = unbounded) */
} VireoKVConfig;

/* KVStats (src/kvstore.h:35-44): same members, types and order */
typedef struct {
    uint64_t requests;
    uint64_t hits;
    uint64_t misses;
    uint64_t prefetched;
    uint64_t bytes_read;
    uint64_t bytes_spilled;
    uint64_t resident_bytes;
    uint64_t capacity_bytes;
} VireoKVStats;

typedef struct VireoKV VireoKV;

enum { VIREO_KV_SELECT_ALL = 0, VIREO_KV_SELECT_RECENT = 1, VIREO_KV_SELECT_TOPK = 2 };

/* src/kvstore_dense.c:kvstore_dense_create. kv_dim: 64, 128 or 256;
 * block_tokens: 1..64. NULL on failure. */
VireoKV *vireo_kv_create_dense(VireoKVConfig cfg);
/* src/kvstore_ooc.c:kvstore_ooc_create with the strategy VIREO_KV_SELECT_*
 * (topk_budget: the TOPK budget, as vireo_select_topk(budget); <= 0: 8).
 * Spilled blocks go to host memory. NULL on failure. */
VireoKV *vireo_kv_create_paged(VireoKVConfig cfg, int strategy, int topk_budget);
/* kv_append (src/kvstore.h:58-61): k and v ([kv_dim] each) become token pos
 * of `layer`. Returns 0 or -errno. */
int vireo_kv_append(VireoKV *s, int layer, int pos, const float *k, const float *v, void *stream);
/* The same for n consecutive layers layer0 .. layer0 + n - 1 (n <= 16; k and
 * v [n x kv_dim]): one launch for the kv heads of a transformer layer. */
int vireo_kv_append_n(VireoKV *s, int layer0, int n, int pos, const float *k, const float *v, void *stream);
/* kv_attend (src/kvstore.h:62-64): out [kv_dim] = attention of q [kv_dim]
 * over `layer`'s selected tokens. */
int vireo_kv_attend(VireoKV *s, int layer, const float *q, float *out, void *stream);
/* Grouped-query attention of n_heads query heads (q, out [n_heads x
 * kv_dim]); head h reads layer layer0 + h / (n_heads / n_kv_heads), as the
 * reference's forward does (src/gguf_run.c:233-235). One launch for all heads. */
int vireo_kv_attend_gqa(VireoKV *s, int layer0, int n_heads, int n_kv_heads, const float *q, float *out,
                        void *stream);
/* A dense store whose blocks for up to max_tokens tokens per layer are
 * allocated at once, every layer's blocks consecutive, so a block's address
 * follows from the position: besides the calls above (host positions) it
 * takes the two calls below, which read the position from device memory and
 * so can be captured in a HIP graph with a device-side position counter.
 * Results equal vireo_kv_create_dense's bit for bit. Once a device-position
 * append has been made, a store takes only device-position calls (the host
 * does not track those tokens; vireo_kv_stats counts the host-position ones).
 * NULL on failure. No counterpart in the reference (its stores grow by host
 * calls). */
VireoKV *vireo_kv_create_contiguous(VireoKVConfig cfg, int max_tokens);
/* vireo_kv_append_n at the position *pos (device int32); nothing is written
 * for a position outside [0, max_tokens). */
int vireo_kv_append_pos(VireoKV *s, int layer0, int n, const int32_t *pos, const float *k, const float *v,
                        void *stream);
/* vireo_kv_attend_gqa over tokens 0 .. *pos of each kv head (n_heads /
 * n_kv_heads in {1, 2, 4, 8}; q 16-byte aligned). The first call on a store
 * sizes its buffers (synchronizing the stream): capture after one call. */
int vireo_kv_attend_gqa_pos(VireoKV *s, int layer0, int n_heads, int n_kv_heads, const int32_t *pos, const float *q,
                            float *out, void *stream);
/* kv_stats (src/kvstore.h:65) */
void vireo_kv_stats(const VireoKV *s, VireoKVStats *out);
/* kv_destroy (src/kvstore.h:66-68); waits for the store's work first */
void vireo_kv_destroy(VireoKV *s);

#ifdef __cplusplus
}
#endif
#endif /* VIREO_KV_H */
