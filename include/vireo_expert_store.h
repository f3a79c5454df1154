/* ExpertStore with its resident pool in HBM.
 *
 * Same API and semantics as the reference's src/expert_store.h:22-52 (lease
 * LRU over (layer, expert) -> {gate, up, down} slices, paged from an open
 * file with pread), and the same include guard, so it replaces that header
 * one for one. The difference is where resident slices live: here in device
 * memory, so ExpertView pointers are device pointers that the vireo-hip
 * kernels read directly. Budget, eviction order, lease pinning and the
 * ExpertStats counters follow src/expert_store.c:52-105.
 *
 * Errors: lookup returns 0 on success and -1 for an unregistered expert (as
 * the reference does, src/expert_store.c:75); where the reference ignores a
 * failure this store reports it instead: -EIO for a short read from the
 * backing file, -ENOMEM when device memory runs out.
 *
 * Threading: like the reference, a store is not locked; use it from one host
 * thread at a time. Inside, an expert of 256 KiB or more is read from the
 * file by eight threads at once (seven workers the store starts on its first
 * such read and joins in expert_store_destroy), since one thread's copy out of
 * the page cache runs at about half the host-to-device link. The workers
 * inherit the CPU affinity of the thread that starts them: a program that has
 * bound that thread to one core (OpenMP's OMP_PROC_BIND does so once its
 * runtime starts) runs all eight readers on that core. */
#ifndef VIREO_EXPERT_STORE_H
#define VIREO_EXPERT_STORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint64_t requests, hits, misses, bytes_read;
    uint64_t resident_bytes, capacity_bytes, experts_resident;
} ExpertStats;

/* Where one expert's three weight slices live in the backing file. */
typedef struct {
    uint64_t gate_off, up_off, down_off;      /* absolute byte offsets        */
    uint32_t gate_bytes, up_bytes, down_bytes;
} ExpertSlices;

/* A leased view of one resident expert. Valid until release(). The three
 * pointers are device addresses. */
typedef struct {
    const void *gate, *up, *down;
    void *slot;        /* opaque lease handle; do not touch */
} ExpertView;

typedef struct ExpertStore ExpertStore;

/* src/expert_store.h:43. fd: the open backing file (a GGUF file or any file
 * holding the slices). capacity_bytes: HBM budget for resident experts
 * (0 = unbounded). Returns NULL on failure. */
ExpertStore *expert_store_create(int fd, uint64_t capacity_bytes,
                                 int n_layers, int n_experts);
/* src/expert_store.h:45 */
void expert_store_register(ExpertStore *s, int layer, int expert,
                           const ExpertSlices *loc);
/* src/expert_store.h:49. Loads the expert into HBM if not resident (evicting
 * the coldest unleased one if over budget), leases it, and fills view.
 * Returns 0 on success. */
int  expert_store_lookup(ExpertStore *s, int layer, int expert, ExpertView *view);
/* src/expert_store.h:50 */
void expert_store_release(ExpertStore *s, ExpertView *view);
/* src/expert_store.h:51. The reference's counters for the same work: direct
 * lookups, plus one lookup per (token, routed expert) of every MoE call that
 * was not captured in a graph, replayed through the reference's policy and
 * budget (so they equal what src/expert_store.c reports for the same tokens,
 * however the HBM pool pins or batches; expert_store_hbm_stats in vireo_hip.h
 * reports the pool). Waits for the routing copies of calls still in flight. */
void expert_store_stats(const ExpertStore *s, ExpertStats *out);
/* src/expert_store.h:52 */
void expert_store_destroy(ExpertStore *s);

#ifdef __cplusplus
}
#endif
#endif
