/* ExpertStore with an HBM resident pool (API: include/vireo_expert_store.h,
 * extensions in include/vireo_hip.h).
 *
 * Two books are kept for every store.
 *
 * The pool (what is in HBM). A resident expert is one device allocation
 * holding gate | up | down, each at a 256-byte boundary, paged in by pread
 * into pinned host staging and a copy to HBM; a store created over a device
 * buffer (expert_store_create_device) makes slices resident by pointing into
 * that buffer, with no copy. The pool follows the reference's policy
 * (src/expert_store.c:52-105): a miss evicts unleased residents in
 * least-recently-used order until the expert fits and stays over budget when
 * everything resident is leased; every lookup takes a lease. The library's
 * own lookups (pinned layers, paged MoE calls, prefetches) only touch this
 * book; expert_store_hbm_stats reports it.
 *
 * The reference's statistics (what expert_store_stats reports): the counters
 * src/expert_store.c would hold after the lookups the reference makes for the
 * same work - every direct expert_store_lookup, and for every MoE call one
 * lookup per (token, routed expert) in token order and selection order, each
 * released before the next, as moe_ffn does (src/gguf_run.c:193-213). This
 * book replays the reference's own residency, LRU order and budget on the
 * host (per-slot ref_* fields), so it does not depend on how the pool pins or
 * batches. The MoE kernels choose the experts on the device; their routing
 * reaches this book through an asynchronous copy into pinned host memory
 * (vh_store_note_routing), which is applied once the copy has landed, so the
 * decode path never waits for it. Calls captured in a HIP graph are not
 * counted (the host does not see replays). */
#define _POSIX_C_SOURCE 200809L
#define __HIP_PLATFORM_AMD__ 1
#include <errno.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <hip/hip_runtime_api.h>
#include "vireo_hip.h"

typedef struct {
    ExpertSlices loc;
    void *dev;            /* device block, NULL when not resident (or aliased) */
    const uint8_t *gate, *up, *down;
    uint64_t bytes;       /* gate + up + down, the budget unit */
    uint64_t alloc;       /* size of dev */
    int resident, lease, registered, pinned;
    uint64_t last_used;
    hipEvent_t busy;      /* after the last kernels enqueued on this block (async paging), or NULL */
    int busy_set;
    /* the reference's book */
    int ref_resident, ref_lease;
    uint64_t ref_last_used;
} Slot;

typedef struct { void *ptr; uint64_t size; hipEvent_t busy; int busy_set; } FreeBlock;

/* A routing copy in flight: idx [T x k] of one MoE call on `layer`. */
typedef struct {
    int layer, T, k, used;
    int32_t *host;        /* pinned */
    size_t cap;           /* entries */
    hipEvent_t ev;
} Note;
#define VH_NOTES 64

/* Staging buffers for asynchronous page-in: pread fills one, an H2D copy on
 * the copy stream drains it; `done` marks when it may be filled again. */
#define VH_STAGES 8
typedef struct { void *buf; size_t bytes; hipEvent_t done; int done_set; } Stage;

/* First word of every store made here. A store handed in by a program that
 * still links the reference's CPU src/expert_store.c starts with its int fd
 * and n_layers instead, so the GPU entry points can refuse it rather than
 * read host pointers from a foreign layout. */
#define VH_STORE_MAGIC 0x4d42485f4f455256ull /* "VREO_HBM" */

struct ExpertStore {
    uint64_t magic;
    int fd;
    const uint8_t *dev_base;   /* device-resident backing, or NULL */
    uint64_t dev_size;
    int n_layers, n_experts, n_slots;
    Slot *slots;
    /* the pool */
    uint64_t tick, resident_bytes, capacity_bytes;
    ExpertStats hbm;
    void *stage;               /* pinned staging for synchronous pread */
    size_t stage_bytes;
    void **tables;             /* per layer: device [n_experts x 3] pointer table */
    FreeBlock *freel;          /* device blocks of evicted experts, kept for reuse */
    int nfree, capfree;
    Stage ring[VH_STAGES];     /* asynchronous page-in */
    int ring_next;
    hipEvent_t copied;         /* after the last asynchronous page-in copy */
    /* the reference's book */
    uint64_t ref_tick, ref_resident_bytes;
    ExpertStats ref;
    Note notes[VH_NOTES];
    int nhead, ncount;
};

static uint64_t al256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

static int store_ok(const ExpertStore *s) { return s && s->magic == VH_STORE_MAGIC; }

static Slot *slot_at(ExpertStore *s, int layer, int expert) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || expert < 0 || expert >= s->n_experts) return NULL;
    return &s->slots[(size_t)layer * s->n_experts + expert];
}

static ExpertStore *store_new(int n_layers, int n_experts, uint64_t capacity_bytes) {
    if (n_layers <= 0 || n_experts <= 0 || (int64_t)n_layers * n_experts > (1 << 26)) return NULL;
    ExpertStore *s = calloc(1, sizeof *s);
    if (!s) return NULL;
    s->magic = VH_STORE_MAGIC;
    s->fd = -1;
    s->n_layers = n_layers;
    s->n_experts = n_experts;
    s->n_slots = n_layers * n_experts;
    s->slots = calloc((size_t)s->n_slots, sizeof(Slot));
    s->tables = calloc((size_t)n_layers, sizeof(void *));
    if (!s->slots || !s->tables) { free(s->slots); free(s->tables); free(s); return NULL; }
    s->capacity_bytes = capacity_bytes;
    return s;
}

ExpertStore *expert_store_create(int fd, uint64_t capacity_bytes, int n_layers, int n_experts) {
    ExpertStore *s = store_new(n_layers, n_experts, capacity_bytes);
    if (s) s->fd = fd;
    return s;
}

ExpertStore *expert_store_create_device(const void *dev_base, uint64_t size, uint64_t capacity_bytes, int n_layers,
                                        int n_experts) {
    if (!dev_base) return NULL;
    ExpertStore *s = store_new(n_layers, n_experts, capacity_bytes);
    if (s) { s->dev_base = (const uint8_t *)dev_base; s->dev_size = size; }
    return s;
}

void expert_store_register(ExpertStore *s, int layer, int expert, const ExpertSlices *loc) {
    Slot *sl = slot_at(s, layer, expert);
    if (!sl || !loc) return;
    sl->loc = *loc;
    sl->bytes = (uint64_t)loc->gate_bytes + loc->up_bytes + loc->down_bytes;
    sl->registered = 1;
}

/* ------------------------------------------------------------------ the reference's book */

/* src/expert_store.c:52-63 on the replayed residency */
static void ref_make_room(ExpertStore *s, uint64_t need) {
    if (!s->capacity_bytes) return;
    while (s->ref_resident_bytes + need > s->capacity_bytes) {
        Slot *victim = NULL;
        for (int i = 0; i < s->n_slots; i++) {
            Slot *c = &s->slots[i];
            if (c->ref_resident && !c->ref_lease && (!victim || c->ref_last_used < victim->ref_last_used)) victim = c;
        }
        if (!victim) break;
        victim->ref_resident = 0;
        s->ref_resident_bytes -= victim->bytes;
        s->ref.experts_resident--;
    }
}

/* src/expert_store.c:72-92 on the replayed residency; returns -1 for an
 * unregistered expert, else takes a lease (lease != 0) or not. */
static int ref_lookup(ExpertStore *s, Slot *sl, int lease) {
    s->ref.requests++;
    if (!sl->registered) return -1;
    if (sl->ref_resident) {
        s->ref.hits++;
    } else {
        s->ref.misses++;
        ref_make_room(s, sl->bytes);
        s->ref.bytes_read += sl->bytes;
        sl->ref_resident = 1;
        s->ref_resident_bytes += sl->bytes;
        s->ref.experts_resident++;
    }
    sl->ref_last_used = ++s->ref_tick;
    if (lease) sl->ref_lease++;
    return 0;
}

static void apply_note(ExpertStore *s, const Note *n) {
    for (int t = 0; t < n->T; t++)
        for (int j = 0; j < n->k; j++) {
            Slot *sl = slot_at(s, n->layer, n->host[(size_t)t * n->k + j]);
            if (sl) (void)ref_lookup(s, sl, 0);  /* looked up, used, released (src/gguf_run.c:201-210) */
            else s->ref.requests++;
        }
}

/* Apply the routing copies that have landed, in call order; with wait, all. */
static int drain_notes(ExpertStore *s, int wait) {
    int rc = 0;
    while (s->ncount) {
        Note *n = &s->notes[s->nhead];
        if (wait) {
            if (hipEventSynchronize(n->ev) != hipSuccess) rc = -EIO;
        } else if (hipEventQuery(n->ev) != hipSuccess) {
            break;
        }
        apply_note(s, n);
        n->used = 0;
        s->nhead = (s->nhead + 1) % VH_NOTES;
        s->ncount--;
    }
    return rc;
}

/* Record the routing of an MoE call (idx_dev: device [T x k]) for the
 * reference's book: copied to pinned host memory on `stream` and applied
 * after it lands. Nothing is recorded while the stream is being captured. */
int vh_store_note_routing(ExpertStore *s, int layer, const int32_t *idx_dev, int T, int k, hipStream_t stream) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || T <= 0 || k <= 0 || !idx_dev) return -EINVAL;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return -EIO;
    if (cs != hipStreamCaptureStatusNone) return 0;
    (void)drain_notes(s, 0);
    if (s->ncount == VH_NOTES) {  /* the oldest copy must land before its slot is reused */
        Note *o = &s->notes[s->nhead];
        if (hipEventSynchronize(o->ev) != hipSuccess) return -EIO;
        (void)drain_notes(s, 0);
    }
    Note *n = &s->notes[(s->nhead + s->ncount) % VH_NOTES];
    const size_t need = (size_t)T * (size_t)k;
    if (need > n->cap) {
        if (n->host) (void)hipHostFree(n->host);
        n->host = NULL;
        n->cap = 0;
        size_t c = need < 4096 ? 4096 : need;
        if (hipHostMalloc((void **)&n->host, c * sizeof(int32_t), 0) != hipSuccess) { n->host = NULL; return -ENOMEM; }
        n->cap = c;
    }
    if (!n->ev && hipEventCreateWithFlags(&n->ev, hipEventDisableTiming) != hipSuccess) { n->ev = NULL; return -EIO; }
    if (hipMemcpyAsync(n->host, idx_dev, need * sizeof(int32_t), hipMemcpyDeviceToHost, stream) != hipSuccess)
        return -EIO;
    if (hipEventRecord(n->ev, stream) != hipSuccess) return -EIO;
    n->layer = layer;
    n->T = T;
    n->k = k;
    n->used = 1;
    s->ncount++;
    return 0;
}

/* The same for routing the host already holds (the paged plan copies it). */
void vh_store_note_routing_host(ExpertStore *s, int layer, const int32_t *idx, int T, int k) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || !idx) return;
    (void)drain_notes(s, 1);
    Note n = {layer, T, k, 1, (int32_t *)idx, (size_t)T * k, NULL};
    apply_note(s, &n);
}

/* ------------------------------------------------------------------ the pool */

static void release_block(ExpertStore *s, Slot *v) {
    if (v->dev) {
        if (s->nfree == s->capfree) {
            int nc = s->capfree ? 2 * s->capfree : 64;
            FreeBlock *nf = realloc(s->freel, (size_t)nc * sizeof *nf);
            if (nf) { s->freel = nf; s->capfree = nc; }
        }
        if (s->nfree < s->capfree) {
            /* the block keeps the event of the last kernels that read it: a
             * later asynchronous copy into it waits for them */
            s->freel[s->nfree++] = (FreeBlock){v->dev, v->alloc, v->busy_set ? v->busy : NULL, v->busy_set};
            v->busy = NULL;
            v->busy_set = 0;
        } else {
            if (v->busy_set) (void)hipEventSynchronize(v->busy);
            (void)hipFree(v->dev);
        }
    }
    v->dev = NULL;
    v->gate = v->up = v->down = NULL;
}

static void evict_one(ExpertStore *s, Slot *v) {
    release_block(s, v);
    v->resident = 0;
    s->resident_bytes -= v->bytes;
    s->hbm.experts_resident--;
}

/* src/expert_store.c:52-63 */
static void make_room(ExpertStore *s, uint64_t need) {
    if (!s->capacity_bytes) return;
    while (s->resident_bytes + need > s->capacity_bytes) {
        Slot *victim = NULL;
        for (int i = 0; i < s->n_slots; i++) {
            Slot *c = &s->slots[i];
            if (c->resident && !c->lease && (!victim || c->last_used < victim->last_used)) victim = c;
        }
        if (!victim) break; /* everything resident is leased: stay over budget */
        evict_one(s, victim);
    }
}

/* A device block of `size` bytes: a cached one (with the event its last
 * readers left, to be waited on before it is overwritten) or a new one. */
static void *take_block(ExpertStore *s, uint64_t size, hipEvent_t *busy, int *busy_set) {
    *busy = NULL;
    *busy_set = 0;
    for (int i = 0; i < s->nfree; i++)
        if (s->freel[i].size == size) {
            void *p = s->freel[i].ptr;
            *busy = s->freel[i].busy;
            *busy_set = s->freel[i].busy_set;
            s->freel[i] = s->freel[--s->nfree];
            return p;
        }
    void *p = NULL;
    if (hipMalloc(&p, size) != hipSuccess) {
        /* drop cached blocks and retry once */
        for (int i = 0; i < s->nfree; i++) {
            if (s->freel[i].busy_set) (void)hipEventSynchronize(s->freel[i].busy);
            if (s->freel[i].busy) (void)hipEventDestroy(s->freel[i].busy);
            (void)hipFree(s->freel[i].ptr);
        }
        s->nfree = 0;
        if (hipMalloc(&p, size) != hipSuccess) return NULL;
    }
    return p;
}

static int pread_all(int fd, void *dst, uint32_t bytes, uint64_t off) {
    uint8_t *b = (uint8_t *)dst;
    uint64_t done = 0;
    while (done < bytes) {
        ssize_t r = pread(fd, b + done, bytes - done, (off_t)(off + done));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return -EIO;  /* read error, or the file ends before the slice does */
        done += (uint64_t)r;
    }
    return 0;
}

static int read_slice(ExpertStore *s, uint64_t off, uint32_t bytes, void *dst) {
    if ((size_t)bytes > s->stage_bytes) {
        if (s->stage) (void)hipHostFree(s->stage);
        s->stage = NULL;
        s->stage_bytes = 0;
        size_t nb = bytes < (1u << 20) ? (1u << 20) : bytes;
        if (hipHostMalloc(&s->stage, nb, 0) != hipSuccess) { s->stage = NULL; return -ENOMEM; }
        s->stage_bytes = nb;
    }
    if (pread_all(s->fd, s->stage, bytes, off)) return -EIO;
    if (hipMemcpy(dst, s->stage, bytes, hipMemcpyHostToDevice) != hipSuccess) return -EIO;
    return 0;
}

/* The same through the staging ring: pread into the next buffer (once the
 * copy that last drained it has finished), then an H2D copy on `cs`. The
 * host reads the next slice while earlier copies and kernels run. */
static int read_slice_async(ExpertStore *s, uint64_t off, uint32_t bytes, void *dst, hipStream_t cs) {
    Stage *st = &s->ring[s->ring_next];
    s->ring_next = (s->ring_next + 1) % VH_STAGES;
    if (st->done_set && hipEventSynchronize(st->done) != hipSuccess) return -EIO;
    st->done_set = 0;
    if ((size_t)bytes > st->bytes) {
        if (st->buf) (void)hipHostFree(st->buf);
        st->buf = NULL;
        st->bytes = 0;
        size_t nb = bytes < (2u << 20) ? (2u << 20) : bytes;
        if (hipHostMalloc(&st->buf, nb, 0) != hipSuccess) { st->buf = NULL; return -ENOMEM; }
        st->bytes = nb;
    }
    if (!st->done && hipEventCreateWithFlags(&st->done, hipEventDisableTiming) != hipSuccess) {
        st->done = NULL;
        return -EIO;
    }
    if (pread_all(s->fd, st->buf, bytes, off)) return -EIO;
    if (hipMemcpyAsync(dst, st->buf, bytes, hipMemcpyHostToDevice, cs) != hipSuccess) return -EIO;
    if (hipEventRecord(st->done, cs) != hipSuccess) return -EIO;
    st->done_set = 1;
    return 0;
}

/* Make sl resident: alias the device backing, or allocate HBM and page in
 * (synchronously, or on the copy stream cs). */
static int page_in(ExpertStore *s, Slot *sl, hipStream_t cs) {
    const ExpertSlices *L = &sl->loc;
    const uint64_t total = (uint64_t)L->gate_bytes + L->up_bytes + L->down_bytes;
    if (s->dev_base) {
        uint64_t ends[3] = {L->gate_off + L->gate_bytes, L->up_off + L->up_bytes, L->down_off + L->down_bytes};
        for (int i = 0; i < 3; i++) if (ends[i] > s->dev_size) return -EINVAL;
        sl->gate = s->dev_base + L->gate_off;
        sl->up = s->dev_base + L->up_off;
        sl->down = s->dev_base + L->down_off;
        s->hbm.bytes_read += total;
        return 0;
    }
    uint64_t og = 0, ou = al256(L->gate_bytes), od = ou + al256(L->up_bytes);
    uint64_t size = od + al256(L->down_bytes);
    hipEvent_t busy;
    int busy_set;
    uint8_t *blk = take_block(s, size, &busy, &busy_set);
    if (!blk) return -ENOMEM;
    int rc = 0;
    if (busy_set) {  /* kernels that read the block under its last owner come first */
        if (cs) rc = hipStreamWaitEvent(cs, busy, 0) == hipSuccess ? 0 : -EIO;
        else rc = hipEventSynchronize(busy) == hipSuccess ? 0 : -EIO;
    }
    if (busy) {  /* the event object is reused for the new owner */
        if (sl->busy) (void)hipEventDestroy(sl->busy);
        sl->busy = busy;
        sl->busy_set = 0;
    }
    const uint64_t offs[3] = {L->gate_off, L->up_off, L->down_off};
    const uint32_t lens[3] = {L->gate_bytes, L->up_bytes, L->down_bytes};
    const uint64_t dsts[3] = {og, ou, od};
    for (int i = 0; i < 3 && !rc; i++)
        rc = cs ? read_slice_async(s, offs[i], lens[i], blk + dsts[i], cs) : read_slice(s, offs[i], lens[i], blk + dsts[i]);
    if (rc) {
        if (cs) (void)hipStreamSynchronize(cs);  /* no copy may still target the block */
        Slot tmp = *sl;
        tmp.dev = blk;
        tmp.alloc = size;
        tmp.busy = NULL;
        tmp.busy_set = 0;
        release_block(s, &tmp);
        return rc;
    }
    s->hbm.bytes_read += total;
    sl->dev = blk;
    sl->alloc = size;
    sl->gate = blk + og;
    sl->up = blk + ou;
    sl->down = blk + od;
    return 0;
}

/* The pool's lookup (src/expert_store.c:72-92): hit, or miss + make room +
 * page in; takes a lease. -1 for an unregistered expert. */
static int pool_lookup(ExpertStore *s, Slot *sl, ExpertView *view, hipStream_t cs) {
    s->hbm.requests++;
    if (!sl->registered) { memset(view, 0, sizeof *view); return -1; }
    if (sl->resident) {
        s->hbm.hits++;
    } else {
        s->hbm.misses++;
        make_room(s, sl->bytes);
        int rc = page_in(s, sl, cs);
        if (rc) { memset(view, 0, sizeof *view); return rc; }
        sl->resident = 1;
        s->resident_bytes += sl->bytes;
        s->hbm.experts_resident++;
    }
    sl->last_used = ++s->tick;
    sl->lease++;
    view->gate = sl->gate;
    view->up = sl->up;
    view->down = sl->down;
    view->slot = sl;
    return 0;
}

int expert_store_lookup(ExpertStore *s, int layer, int expert, ExpertView *view) {
    if (!view) return -EINVAL;
    Slot *sl = slot_at(s, layer, expert);
    if (!sl) { memset(view, 0, sizeof *view); return -EINVAL; }
    if (s->ncount) (void)drain_notes(s, 1);  /* earlier MoE calls' lookups come first */
    (void)ref_lookup(s, sl, 1);
    return pool_lookup(s, sl, view, NULL);
}

void expert_store_release(ExpertStore *s, ExpertView *view) {
    (void)s;
    if (view && view->slot) {
        Slot *sl = (Slot *)view->slot;
        if (sl->lease > 0) sl->lease--;
        if (sl->ref_lease > 0) sl->ref_lease--;
    }
    if (view) memset(view, 0, sizeof *view);
}

void expert_store_stats(const ExpertStore *cs, ExpertStats *out) {
    ExpertStore *s = (ExpertStore *)cs;  /* applying landed routing copies is not a visible change */
    if (!store_ok(s) || !out) return;
    (void)drain_notes(s, 1);
    *out = s->ref;
    out->resident_bytes = s->ref_resident_bytes;
    out->capacity_bytes = s->capacity_bytes;
}

void expert_store_hbm_stats(const ExpertStore *s, ExpertStats *out) {
    if (!store_ok(s) || !out) return;
    *out = s->hbm;
    out->resident_bytes = s->resident_bytes;
    out->capacity_bytes = s->capacity_bytes;
}

int expert_store_pin_layer(ExpertStore *s, int layer, const void *const **dev_table) {
    if (!store_ok(s) || !dev_table || layer < 0 || layer >= s->n_layers) return -EINVAL;
    if (s->tables[layer]) { *dev_table = (const void *const *)s->tables[layer]; return 0; }
    const int E = s->n_experts;
    uint64_t need = 0, all = 0;
    for (int e = 0; e < E; e++) {
        Slot *sl = slot_at(s, layer, e);
        if (sl->registered && !sl->resident) need += sl->bytes;
        if (sl->registered) all += sl->bytes;
    }
    /* a layer larger than the store never fits: say so before evicting anything */
    if (s->capacity_bytes && all > s->capacity_bytes) return -ENOSPC;
    if (s->capacity_bytes && s->resident_bytes + need > s->capacity_bytes) {
        /* evict what can go; the layer must then fit entirely */
        make_room(s, need);
        if (s->resident_bytes + need > s->capacity_bytes) return -ENOSPC;
    }
    const void **host = calloc((size_t)E * 3, sizeof(void *));
    if (!host) return -ENOMEM;
    int rc = 0, e;
    for (e = 0; e < E && !rc; e++) {
        Slot *sl = slot_at(s, layer, e);
        if (!sl->registered) continue;
        ExpertView v;
        rc = pool_lookup(s, sl, &v, NULL);
        if (rc) break;
        sl->pinned = 1;
        if (((uintptr_t)v.gate | (uintptr_t)v.up | (uintptr_t)v.down) & 15u) rc = -EINVAL;
        host[3 * e + 0] = v.gate;
        host[3 * e + 1] = v.up;
        host[3 * e + 2] = v.down;
    }
    void *tab = NULL;
    if (!rc && hipMalloc(&tab, (size_t)E * 3 * sizeof(void *)) != hipSuccess) rc = -ENOMEM;
    if (!rc && hipMemcpy(tab, host, (size_t)E * 3 * sizeof(void *), hipMemcpyHostToDevice) != hipSuccess) rc = -EIO;
    free(host);
    if (rc) {
        if (tab) (void)hipFree(tab);
        for (int j = 0; j < E; j++) {
            Slot *sl = slot_at(s, layer, j);
            if (sl->pinned) { sl->pinned = 0; if (sl->lease > 0) sl->lease--; }
        }
        return rc;
    }
    s->tables[layer] = tab;
    *dev_table = (const void *const *)tab;
    return 0;
}

int expert_store_unpin_layer(ExpertStore *s, int layer) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers) return -EINVAL;
    if (!s->tables[layer]) return 0;
    if (hipDeviceSynchronize() != hipSuccess) return -EIO;
    (void)hipFree(s->tables[layer]);
    s->tables[layer] = NULL;
    for (int e = 0; e < s->n_experts; e++) {
        Slot *sl = slot_at(s, layer, e);
        if (sl->pinned) { sl->pinned = 0; if (sl->lease > 0) sl->lease--; }
    }
    return 0;
}

void expert_store_destroy(ExpertStore *s) {
    if (!store_ok(s)) return;
    s->magic = 0;
    (void)hipDeviceSynchronize();
    for (int l = 0; l < s->n_layers; l++) if (s->tables[l]) (void)hipFree(s->tables[l]);
    for (int i = 0; i < s->n_slots; i++) {
        if (s->slots[i].dev) (void)hipFree(s->slots[i].dev);
        if (s->slots[i].busy) (void)hipEventDestroy(s->slots[i].busy);
    }
    for (int i = 0; i < s->nfree; i++) {
        (void)hipFree(s->freel[i].ptr);
        if (s->freel[i].busy) (void)hipEventDestroy(s->freel[i].busy);
    }
    for (int i = 0; i < VH_NOTES; i++) {
        if (s->notes[i].host) (void)hipHostFree(s->notes[i].host);
        if (s->notes[i].ev) (void)hipEventDestroy(s->notes[i].ev);
    }
    for (int i = 0; i < VH_STAGES; i++) {
        if (s->ring[i].buf) (void)hipHostFree(s->ring[i].buf);
        if (s->ring[i].done) (void)hipEventDestroy(s->ring[i].done);
    }
    if (s->copied) (void)hipEventDestroy(s->copied);
    if (s->stage) (void)hipHostFree(s->stage);
    free(s->freel);
    free(s->tables);
    free(s->slots);
    free(s);
}

/* ------------------------------------------------------------------ helpers for the MoE plans */

/* Bytes an expert takes in the pool (0 if unregistered), and the pool's
 * capacity (0 = unbounded), for callers that page experts in batches. */
uint64_t vh_store_expert_bytes(const ExpertStore *s, int layer, int expert) {
    const Slot *sl = (store_ok(s) && layer >= 0 && layer < s->n_layers && expert >= 0 && expert < s->n_experts)
                         ? &s->slots[(size_t)layer * (size_t)s->n_experts + (size_t)expert]
                         : NULL;
    return sl && sl->registered ? sl->bytes : 0;
}
uint64_t vh_store_capacity(const ExpertStore *s) { return store_ok(s) ? s->capacity_bytes : 0; }
/* 1 for a store made by this library, 0 for NULL or a foreign layout. */
int vh_store_valid(const ExpertStore *s) { return store_ok(s); }

/* The device table of a pinned layer, or NULL (never allocates). */
const void *const *vh_store_layer_table(const ExpertStore *s, int layer) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers) return NULL;
    return (const void *const *)s->tables[layer];
}

/* 1 when every registered expert of every layer fits the capacity at once:
 * only then does the MoE path pin whole layers. */
int vh_store_fits_all(const ExpertStore *s) {
    if (!store_ok(s)) return 0;
    if (!s->capacity_bytes) return 1;
    uint64_t all = 0;
    for (int i = 0; i < s->n_slots; i++)
        if (s->slots[i].registered) all += s->slots[i].bytes;
    return all <= s->capacity_bytes;
}

/* Bytes of resident experts that hold a lease (pinned layers, a caller's
 * open lookups): what a paged call cannot evict. */
uint64_t vh_store_leased_bytes(const ExpertStore *s) {
    if (!store_ok(s)) return 0;
    uint64_t b = 0;
    for (int i = 0; i < s->n_slots; i++)
        if (s->slots[i].resident && s->slots[i].lease) b += s->slots[i].bytes;
    return b;
}

/* The pool's lookup for a paged call: misses are paged in on the copy
 * stream cs (vh_store_copy_fence orders them before the kernels). */
int vh_store_acquire(ExpertStore *s, int layer, int expert, ExpertView *view, hipStream_t cs) {
    Slot *sl = slot_at(s, layer, expert);
    if (!view) return -EINVAL;
    if (!sl) { memset(view, 0, sizeof *view); return -EINVAL; }
    return pool_lookup(s, sl, view, cs);
}

/* The kernels enqueued on `stream` so far read view's block: a later copy into
 * that block (after eviction) waits for them. Then the lease is dropped. */
int vh_store_drop(ExpertStore *s, ExpertView *view, hipStream_t stream) {
    int rc = 0;
    if (view && view->slot) {
        Slot *sl = (Slot *)view->slot;
        if (sl->dev) {
            if (!sl->busy && hipEventCreateWithFlags(&sl->busy, hipEventDisableTiming) != hipSuccess) {
                sl->busy = NULL;
                rc = -EIO;
            }
            if (sl->busy) {
                if (hipEventRecord(sl->busy, stream) == hipSuccess) sl->busy_set = 1;
                else rc = -EIO;
            }
            if (rc) (void)hipStreamSynchronize(stream);
        }
        if (sl->lease > 0) sl->lease--;
    }
    if (view) memset(view, 0, sizeof *view);
    (void)s;
    return rc;
}

/* Make `stream` wait for every page-in copy issued on cs so far. */
int vh_store_copy_fence(ExpertStore *s, hipStream_t cs, hipStream_t stream) {
    if (!store_ok(s)) return -EINVAL;
    if (!s->copied && hipEventCreateWithFlags(&s->copied, hipEventDisableTiming) != hipSuccess) {
        s->copied = NULL;
        return -EIO;
    }
    if (hipEventRecord(s->copied, cs) != hipSuccess) return -EIO;
    return hipStreamWaitEvent(stream, s->copied, 0) == hipSuccess ? 0 : -EIO;
}

/* The store's own file descriptor, for callers that need to know whether
 * page-ins read a file (-1 for a device-backed store). */
int vh_store_fd(const ExpertStore *s) { return store_ok(s) && !s->dev_base ? s->fd : -1; }
