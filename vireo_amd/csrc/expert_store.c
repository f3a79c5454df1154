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
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <hip/hip_runtime_api.h>
#include "vireo_hip.h"

void vh_store_packed_abort(ExpertStore *s, int layer, int kind);

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
    /* places in the two books' LRU lists (slot indices, -1 at the ends) */
    int lru_prev, lru_next, ref_prev, ref_next;
    int prefetched;       /* paged in ahead of use and not yet looked up */
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

/* Staging buffers for asynchronous page-in: one expert's three slices are
 * read into one buffer, laid out as its HBM block, and one H2D copy on the
 * copy stream drains it; `done` marks when it may be filled again. */
#define VH_STAGES 8
typedef struct { void *buf; size_t bytes; hipEvent_t done; int done_set; } Stage;

/* Where one read puts a slice: file offset, length, offset in the buffer. */
typedef struct { uint64_t off; uint32_t len; uint64_t at; } Span;

/* Parallel reads: an expert of at least VH_PAR_MIN bytes is read by
 * VH_READERS threads at once, each pread-ing a 4 KiB-aligned piece of its
 * slices laid end to end - one thread's copy out of the page cache runs at
 * about half the host-to-device link. The workers start with the store's
 * first large read and stop in expert_store_destroy; a store that cannot
 * start them reads serially. */
#define VH_READERS 8
#define VH_PAR_MIN (256u << 10)
typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    pthread_t th[VH_READERS - 1];
    int nth, quit;
    unsigned gen;              /* job number: workers run each job once */
    int pending, err;          /* workers still reading the job; the first error */
    int fd;
    uint8_t *dst;
    Span sp[3];
    int nsp;
    uint64_t total;
} ReadPool;

/* First word of every store made here. A store handed in by a program that
 * still links the reference's CPU src/expert_store.c starts with its int fd
 * and n_layers instead, so the GPU entry points can refuse it rather than
 * read host pointers from a foreign layout. */
#define VH_STORE_MAGIC 0x4d42485f4f455256ull /* "VREO_HBM" */
#define VH_PACK_KINDS 2 /* decode-batch 16-row tiles; prefill Q8_0 row octets */

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
    void **ptables, **pbufs;   /* per kind and pinned layer: a reordered copy of its experts and its table */
    uint64_t *pbytes;          /* the copies' sizes; they count against the capacity */
    uint64_t packed_bytes;     /* their sum */
    FreeBlock *freel;          /* device blocks of evicted experts, kept for reuse */
    int nfree, capfree;
    uint8_t *arena;            /* one allocation the pool's blocks are cut from (bounded pools) */
    uint64_t arena_size, arena_used;
    int arena_failed;
    Stage ring[VH_STAGES];     /* asynchronous page-in */
    ReadPool *readers;         /* parallel pread workers (NULL until the first large read) */
    int readers_failed;
    int ring_next;
    hipEvent_t copied;         /* after the last asynchronous page-in copy */
    /* the reference's book */
    uint64_t ref_tick, ref_resident_bytes;
    ExpertStats ref;
    Note notes[VH_NOTES];
    int nhead, ncount;
    /* Resident slots from least to most recently used, one list per book:
     * the eviction victim of src/expert_store.c:52-63 (the resident expert
     * without a lease used longest ago) is the first unleased slot of its
     * list, as every use moves a slot to the end. */
    int lru_head, lru_tail, ref_head, ref_tail;
    uint64_t registered_bytes;
    /* prefetch: the experts of one layer expected next, most likely first */
    int hint_layer, hint_n, hint_pos, prefetch_off;
    int32_t hint[64];
    uint64_t pf_issued, pf_used, pf_bytes;
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
    s->ptables = calloc((size_t)n_layers * VH_PACK_KINDS, sizeof(void *));
    s->pbufs = calloc((size_t)n_layers * VH_PACK_KINDS, sizeof(void *));
    s->pbytes = calloc((size_t)n_layers * VH_PACK_KINDS, sizeof(uint64_t));
    if (!s->slots || !s->tables || !s->ptables || !s->pbufs || !s->pbytes) {
        free(s->slots); free(s->tables); free(s->ptables); free(s->pbufs); free(s->pbytes); free(s);
        return NULL;
    }
    s->capacity_bytes = capacity_bytes;
    for (int i = 0; i < s->n_slots; i++)
        s->slots[i].lru_prev = s->slots[i].lru_next = s->slots[i].ref_prev = s->slots[i].ref_next = -1;
    s->lru_head = s->lru_tail = s->ref_head = s->ref_tail = -1;
    s->hint_layer = -1;
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
    if (sl->registered) s->registered_bytes -= sl->bytes;
    sl->loc = *loc;
    sl->bytes = (uint64_t)loc->gate_bytes + loc->up_bytes + loc->down_bytes;
    sl->registered = 1;
    s->registered_bytes += sl->bytes;
}

/* ------------------------------------------------------------------ LRU lists */

/* book 0: the pool's residency; book 1: the reference's replayed one */
static int *link_prev(Slot *sl, int book) { return book ? &sl->ref_prev : &sl->lru_prev; }
static int *link_next(Slot *sl, int book) { return book ? &sl->ref_next : &sl->lru_next; }

static void lru_unlink(ExpertStore *s, Slot *sl, int book) {
    int *head = book ? &s->ref_head : &s->lru_head, *tail = book ? &s->ref_tail : &s->lru_tail;
    const int p = *link_prev(sl, book), n = *link_next(sl, book);
    if (p >= 0) *link_next(&s->slots[p], book) = n;
    else *head = n;
    if (n >= 0) *link_prev(&s->slots[n], book) = p;
    else *tail = p;
    *link_prev(sl, book) = *link_next(sl, book) = -1;
}

/* sl has just been used: to the end of the list (linked in if new) */
static void lru_touch(ExpertStore *s, Slot *sl, int book, int linked) {
    int *head = book ? &s->ref_head : &s->lru_head, *tail = book ? &s->ref_tail : &s->lru_tail;
    const int i = (int)(sl - s->slots);
    if (linked) {
        if (*tail == i) return;
        lru_unlink(s, sl, book);
    }
    *link_prev(sl, book) = *tail;
    *link_next(sl, book) = -1;
    if (*tail >= 0) *link_next(&s->slots[*tail], book) = i;
    else *head = i;
    *tail = i;
}

/* ------------------------------------------------------------------ the reference's book */

/* src/expert_store.c:52-63 on the replayed residency */
static void ref_make_room(ExpertStore *s, uint64_t need) {
    if (!s->capacity_bytes) return;
    while (s->ref_resident_bytes + need > s->capacity_bytes) {
        Slot *victim = NULL;
        for (int i = s->ref_head; i >= 0 && !victim; i = s->slots[i].ref_next)
            if (!s->slots[i].ref_lease) victim = &s->slots[i];
        if (!victim) break;
        lru_unlink(s, victim, 1);
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
    const int was = sl->ref_resident;
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
    lru_touch(s, sl, 1, was);
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

/* Free a device block: blocks cut from the arena go back with the arena. */
static void block_free(ExpertStore *s, void *p) {
    const uint8_t *b = (const uint8_t *)p;
    if (s->arena && b >= s->arena && b < s->arena + s->arena_size) return;
    (void)hipFree(p);
}

static void release_block(ExpertStore *s, Slot *v) {
    if (v->dev) {
        if (s->nfree == s->capfree) {
            int nc = s->capfree ? 2 * s->capfree : 64;
            FreeBlock *nf = realloc(s->freel, (size_t)nc * sizeof *nf);
            if (nf) { s->freel = nf; s->capfree = nc; }
        }
        if (s->nfree < s->capfree) {
            /* the block keeps the event of the last kernels that read it: a
             * later asynchronous copy into it waits for them (an event never
             * recorded goes along too, for the next owner to reuse) */
            s->freel[s->nfree++] = (FreeBlock){v->dev, v->alloc, v->busy, v->busy_set};
            v->busy = NULL;
            v->busy_set = 0;
        } else {
            if (v->busy_set) (void)hipEventSynchronize(v->busy);
            block_free(s, v->dev);
        }
    }
    v->dev = NULL;
    v->gate = v->up = v->down = NULL;
}

static void evict_one(ExpertStore *s, Slot *v) {
    release_block(s, v);
    lru_unlink(s, v, 0);
    v->prefetched = 0;  /* read ahead for nothing */
    v->resident = 0;
    s->resident_bytes -= v->bytes;
    s->hbm.experts_resident--;
}

/* src/expert_store.c:52-63 */
static void make_room(ExpertStore *s, uint64_t need) {
    if (!s->capacity_bytes) return;
    while (s->resident_bytes + s->packed_bytes + need > s->capacity_bytes) {
        Slot *victim = NULL;
        for (int i = s->lru_head; i >= 0 && !victim; i = s->slots[i].lru_next)
            if (!s->slots[i].lease) victim = &s->slots[i];
        if (!victim) break; /* everything resident is leased: stay over budget */
        evict_one(s, victim);
    }
}

/* A device block of `size` bytes: a cached one (with the event its last
 * readers left, to be waited on before it is overwritten) or a new one. A
 * bounded pool cuts new blocks from one allocation of its capacity (plus
 * 1/32 for the 256-byte padding of slices), made on its first page-in, so
 * filling the pool costs no allocation per expert; past it (a pool over
 * budget because every resident expert is leased, or blocks of several
 * sizes) a block is allocated on its own. */
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
    if (s->capacity_bytes && s->capacity_bytes <= (1ull << 44) && !s->arena && !s->arena_failed) {
        const uint64_t want = s->capacity_bytes + (s->capacity_bytes >> 5);
        void *a = NULL;
        if (hipMalloc(&a, want) == hipSuccess) {
            s->arena = (uint8_t *)a;
            s->arena_size = want;
            s->arena_used = 0;
        } else {
            (void)hipGetLastError();
            s->arena_failed = 1;
        }
    }
    if (s->arena && s->arena_size - s->arena_used >= size) {
        void *p = s->arena + s->arena_used;
        s->arena_used += (size + 255u) & ~(uint64_t)255u;
        if (s->arena_used > s->arena_size) s->arena_used = s->arena_size;
        return p;
    }
    void *p = NULL;
    if (hipMalloc(&p, size) != hipSuccess) {
        /* drop cached blocks and retry once */
        for (int i = 0; i < s->nfree; i++) {
            if (s->freel[i].busy_set) (void)hipEventSynchronize(s->freel[i].busy);
            if (s->freel[i].busy) (void)hipEventDestroy(s->freel[i].busy);
            block_free(s, s->freel[i].ptr);
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

/* Piece `id` of VH_READERS of a job: bytes [lo, hi) of its spans laid end to
 * end, each part pread into its place in dst. */
static int read_piece(int fd, uint8_t *dst, const Span *sp, int nsp, uint64_t total, int id) {
    uint64_t per = (total + VH_READERS - 1) / VH_READERS;
    per = (per + 4095u) & ~(uint64_t)4095u;
    const uint64_t lo = per * (uint64_t)id < total ? per * (uint64_t)id : total;
    const uint64_t hi = lo + per < total ? lo + per : total;
    uint64_t base = 0;
    for (int i = 0; i < nsp && lo < hi; i++) {
        const uint64_t a = base, b = base + sp[i].len;
        const uint64_t x = a > lo ? a : lo, y = b < hi ? b : hi;
        if (x < y && pread_all(fd, dst + sp[i].at + (x - a), (uint32_t)(y - x), sp[i].off + (x - a))) return -EIO;
        base = b;
    }
    return 0;
}

typedef struct { ReadPool *p; int id; } ReaderArg;

static void *reader_main(void *arg) {
    ReaderArg a = *(ReaderArg *)arg;
    free(arg);
    ReadPool *p = a.p;
    unsigned seen = 0;
    pthread_mutex_lock(&p->mu);
    for (;;) {
        while (!p->quit && p->gen == seen) pthread_cond_wait(&p->go, &p->mu);
        if (p->quit) break;
        seen = p->gen;
        Span sp[3];
        memcpy(sp, p->sp, sizeof sp);
        const int fd = p->fd, nsp = p->nsp;
        uint8_t *dst = p->dst;
        const uint64_t total = p->total;
        pthread_mutex_unlock(&p->mu);
        const int rc = read_piece(fd, dst, sp, nsp, total, a.id);
        pthread_mutex_lock(&p->mu);
        if (rc && !p->err) p->err = rc;
        if (--p->pending == 0) pthread_cond_signal(&p->done);
    }
    pthread_mutex_unlock(&p->mu);
    return NULL;
}

static void readers_stop(ExpertStore *s) {
    ReadPool *p = s->readers;
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->nth; i++) pthread_join(p->th[i], NULL);
    pthread_cond_destroy(&p->go);
    pthread_cond_destroy(&p->done);
    pthread_mutex_destroy(&p->mu);
    free(p);
    s->readers = NULL;
}

static int readers_start(ExpertStore *s) {
    if (s->readers) return 0;
    if (s->readers_failed) return -1;
    ReadPool *p = (ReadPool *)calloc(1, sizeof(ReadPool));
    if (!p) { s->readers_failed = 1; return -1; }
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->go, NULL);
    pthread_cond_init(&p->done, NULL);
    s->readers = p;
    for (int i = 0; i < VH_READERS - 1; i++) {
        ReaderArg *a = (ReaderArg *)malloc(sizeof(ReaderArg));
        if (!a) break;
        a->p = p;
        a->id = i + 1;
        if (pthread_create(&p->th[i], NULL, reader_main, a) != 0) { free(a); break; }
        p->nth++;
    }
    if (p->nth != VH_READERS - 1) {  /* all or nothing: the pieces assume every worker */
        readers_stop(s);
        s->readers_failed = 1;
        return -1;
    }
    return 0;
}

/* Read the spans into dst: by the reader pool when they are large (the
 * calling thread reads piece 0 and waits for the rest), else in turn. */
static int read_spans(ExpertStore *s, uint8_t *dst, const Span *sp, int nsp) {
    uint64_t total = 0;
    for (int i = 0; i < nsp; i++) total += sp[i].len;
    if (total < VH_PAR_MIN || readers_start(s)) {
        for (int i = 0; i < nsp; i++)
            if (pread_all(s->fd, dst + sp[i].at, sp[i].len, sp[i].off)) return -EIO;
        return 0;
    }
    ReadPool *p = s->readers;
    pthread_mutex_lock(&p->mu);
    p->fd = s->fd;
    p->dst = dst;
    memcpy(p->sp, sp, (size_t)nsp * sizeof(Span));
    p->nsp = nsp;
    p->total = total;
    p->err = 0;
    p->pending = VH_READERS - 1;
    p->gen++;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    int rc = read_piece(s->fd, dst, sp, nsp, total, 0);
    pthread_mutex_lock(&p->mu);
    while (p->pending > 0) pthread_cond_wait(&p->done, &p->mu);
    if (!rc) rc = p->err;
    pthread_mutex_unlock(&p->mu);
    return rc;
}

/* A pinned buffer of at least `bytes` in *buf (grown as needed). */
static int stage_fit(void **buf, size_t *have, size_t bytes) {
    if (bytes <= *have) return 0;
    if (*buf) (void)hipHostFree(*buf);
    *buf = NULL;
    *have = 0;
    const size_t nb = bytes < (4u << 20) ? (4u << 20) : bytes;
    if (hipHostMalloc(buf, nb, 0) != hipSuccess) { *buf = NULL; return -ENOMEM; }
    *have = nb;
    return 0;
}

/* Read one expert's slices from the file into the device block `blk` (at
 * offsets sp[i].at, `len` bytes in all): through pinned staging and a
 * synchronous copy, or through the next buffer of the staging ring (once the
 * copy that last drained it has finished) and a copy on `cs`, so the host
 * reads the next expert while earlier copies and kernels run. */
static int read_block(ExpertStore *s, const Span *sp, uint64_t len, uint8_t *blk, hipStream_t cs) {
    if (!cs) {
        if (stage_fit(&s->stage, &s->stage_bytes, len)) return -ENOMEM;
        if (read_spans(s, (uint8_t *)s->stage, sp, 3)) return -EIO;
        return hipMemcpy(blk, s->stage, len, hipMemcpyHostToDevice) == hipSuccess ? 0 : -EIO;
    }
    Stage *st = &s->ring[s->ring_next];
    s->ring_next = (s->ring_next + 1) % VH_STAGES;
    if (st->done_set && hipEventSynchronize(st->done) != hipSuccess) return -EIO;
    st->done_set = 0;
    if (stage_fit(&st->buf, &st->bytes, len)) return -ENOMEM;
    if (!st->done && hipEventCreateWithFlags(&st->done, hipEventDisableTiming) != hipSuccess) {
        st->done = NULL;
        return -EIO;
    }
    if (read_spans(s, (uint8_t *)st->buf, sp, 3)) return -EIO;
    if (hipMemcpyAsync(blk, st->buf, len, hipMemcpyHostToDevice, cs) != hipSuccess) return -EIO;
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
    const Span sp[3] = {{L->gate_off, L->gate_bytes, og}, {L->up_off, L->up_bytes, ou}, {L->down_off, L->down_bytes, od}};
    if (!rc) rc = read_block(s, sp, od + L->down_bytes, blk, cs);
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
    const int was = sl->resident;
    if (sl->resident) {
        s->hbm.hits++;
        if (sl->prefetched) { s->pf_used++; sl->prefetched = 0; }
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
    lru_touch(s, sl, 0, was);
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
    out->resident_bytes = s->resident_bytes + s->packed_bytes;
    out->capacity_bytes = s->capacity_bytes;
}

uint64_t expert_store_packed_bytes(const ExpertStore *s) { return store_ok(s) ? s->packed_bytes : 0; }

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
    if (s->capacity_bytes && s->resident_bytes + s->packed_bytes + need > s->capacity_bytes) {
        /* evict what can go; the layer must then fit entirely */
        make_room(s, need);
        if (s->resident_bytes + s->packed_bytes + need > s->capacity_bytes) return -ENOSPC;
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
    for (int kd = 0; kd < VH_PACK_KINDS; kd++) {
        if (s->ptables[(size_t)kd * s->n_layers + layer])
            (void)hipFree(s->ptables[(size_t)kd * s->n_layers + layer]);
        s->ptables[(size_t)kd * s->n_layers + layer] = NULL;
        vh_store_packed_abort(s, layer, kd);
    }
    for (int e = 0; e < s->n_experts; e++) {
        Slot *sl = slot_at(s, layer, e);
        if (sl->pinned) { sl->pinned = 0; if (sl->lease > 0) sl->lease--; }
    }
    return 0;
}

void expert_store_destroy(ExpertStore *s) {
    if (!store_ok(s)) return;
    s->magic = 0;
    readers_stop(s);
    (void)hipDeviceSynchronize();
    for (int l = 0; l < s->n_layers; l++) {
        if (s->tables[l]) (void)hipFree(s->tables[l]);
        for (int kd = 0; kd < VH_PACK_KINDS; kd++) {
            const size_t i = (size_t)kd * s->n_layers + l;
            if (s->ptables[i]) (void)hipFree(s->ptables[i]);
            if (s->pbufs[i]) block_free(s, s->pbufs[i]);
        }
    }
    for (int i = 0; i < s->n_slots; i++) {
        if (s->slots[i].dev) block_free(s, s->slots[i].dev);
        if (s->slots[i].busy) (void)hipEventDestroy(s->slots[i].busy);
    }
    for (int i = 0; i < s->nfree; i++) {
        block_free(s, s->freel[i].ptr);
        if (s->freel[i].busy) (void)hipEventDestroy(s->freel[i].busy);
    }
    if (s->arena) (void)hipFree(s->arena);
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
    free(s->ptables);
    free(s->pbufs);
    free(s->pbytes);
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

/* A pinned layer's experts reordered for a kernel (kind 0: the matrix-core
 * decode batch's 16-row tiles, 1: the prefill GEMMs' Q8_0 row octets): their
 * device table, or NULL (never allocates). A copy counts against the
 * capacity like resident experts: vh_store_packed_begin gives a device
 * block of `bytes` for one only while resident experts and copies fit the
 * capacity with it (else NULL, and the caller reads the GGUF rows), cut
 * from the pool's arena when it has room; vh_store_set_packed then hands
 * the store the copy's device [n_experts x 3] table, or vh_store_packed_abort
 * takes the block back. The store frees both when the layer is unpinned or
 * the store destroyed. */
const void *const *vh_store_packed_table(const ExpertStore *s, int layer, int kind) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || kind < 0 || kind >= VH_PACK_KINDS || !s->tables[layer])
        return NULL;
    return (const void *const *)s->ptables[(size_t)kind * s->n_layers + layer];
}
void *vh_store_packed_begin(ExpertStore *s, int layer, int kind, uint64_t bytes) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || kind < 0 || kind >= VH_PACK_KINDS || !s->tables[layer] ||
        !bytes)
        return NULL;
    const size_t i = (size_t)kind * s->n_layers + layer;
    if (s->ptables[i] || s->pbufs[i]) return NULL;
    if (s->capacity_bytes && s->resident_bytes + s->packed_bytes + bytes > s->capacity_bytes) return NULL;
    void *p = NULL;
    for (int j = 0; j < s->nfree && !p; j++)
        if (s->freel[j].size == bytes) {
            /* a block of this size: the layer's own copy, dropped at an unpin
             * that waited for the device */
            p = s->freel[j].ptr;
            if (s->freel[j].busy_set) (void)hipEventSynchronize(s->freel[j].busy);
            if (s->freel[j].busy) (void)hipEventDestroy(s->freel[j].busy);
            s->freel[j] = s->freel[--s->nfree];
        }
    if (!p && s->arena && s->arena_size - s->arena_used >= bytes) {
        p = s->arena + s->arena_used;
        s->arena_used += (bytes + 255u) & ~(uint64_t)255u;
        if (s->arena_used > s->arena_size) s->arena_used = s->arena_size;
    }
    if (!p && hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return NULL;
    }
    s->pbufs[i] = p;
    s->pbytes[i] = bytes;
    s->packed_bytes += bytes;
    return p;
}

int vh_store_set_packed(ExpertStore *s, int layer, int kind, void *tab) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || kind < 0 || kind >= VH_PACK_KINDS || !s->tables[layer])
        return -EINVAL;
    const size_t i = (size_t)kind * s->n_layers + layer;
    if (s->ptables[i] || !s->pbufs[i]) return -EINVAL;
    s->ptables[i] = tab;
    return 0;
}

/* The block of a copy goes back to the free list (the arena's memory stays
 * with the arena; a re-pinned layer packs into it again). The caller has
 * waited for the kernels that wrote or read it. */
void vh_store_packed_abort(ExpertStore *s, int layer, int kind) {
    if (!store_ok(s) || layer < 0 || layer >= s->n_layers || kind < 0 || kind >= VH_PACK_KINDS) return;
    const size_t i = (size_t)kind * s->n_layers + layer;
    if (!s->pbufs[i]) return;
    if (s->nfree == s->capfree) {
        int nc = s->capfree ? 2 * s->capfree : 64;
        FreeBlock *nf = realloc(s->freel, (size_t)nc * sizeof *nf);
        if (nf) { s->freel = nf; s->capfree = nc; }
    }
    if (s->nfree < s->capfree) s->freel[s->nfree++] = (FreeBlock){s->pbufs[i], s->pbytes[i], NULL, 0};
    else block_free(s, s->pbufs[i]);
    s->packed_bytes -= s->pbytes[i];
    s->pbufs[i] = NULL;
    s->pbytes[i] = 0;
}

/* 1 when every registered expert of every layer fits the capacity at once:
 * only then does the MoE path pin whole layers. */
int vh_store_fits_all(const ExpertStore *s) {
    if (!store_ok(s)) return 0;
    return !s->capacity_bytes || s->registered_bytes <= s->capacity_bytes;
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

/* ------------------------------------------------------------------ prefetch */

/* The experts of `layer` that the next call on it is expected to route to,
 * most likely first (up to 64; ids not registered are skipped when read). */
void vh_store_hint(ExpertStore *s, int layer, const int32_t *ids, int n) {
    if (!store_ok(s)) return;
    if (n > 64) n = 64;
    s->hint_layer = n > 0 ? layer : -1;
    s->hint_n = n > 0 ? n : 0;
    s->hint_pos = 0;
    if (n > 0) memcpy(s->hint, ids, (size_t)n * sizeof(int32_t));
}

/* Read the next hinted expert of `layer` that is not resident into the pool,
 * without a lease, its copy on cs: 1 after a read, 0 when none is left (or
 * the hint is for another layer, the store is device-backed, prefetch is off,
 * or the pool has no room without going over its capacity), < 0 on a failed
 * read. The pool's requests, hits and misses do not count it; its
 * bytes_read does, and a later lookup of it counts as a hit. */
int vh_store_prefetch_next(ExpertStore *s, int layer, hipStream_t cs) {
    if (!store_ok(s) || s->prefetch_off || s->dev_base || !cs || layer != s->hint_layer) return 0;
    while (s->hint_pos < s->hint_n) {
        Slot *sl = slot_at(s, layer, s->hint[s->hint_pos++]);
        if (!sl || !sl->registered || sl->resident) continue;
        if (s->capacity_bytes) {
            make_room(s, sl->bytes);
            if (s->resident_bytes + s->packed_bytes + sl->bytes > s->capacity_bytes) { s->hint_pos = s->hint_n; return 0; }
        }
        const int rc = page_in(s, sl, cs);
        if (rc) return rc;
        sl->resident = 1;
        s->resident_bytes += sl->bytes;
        s->hbm.experts_resident++;
        sl->last_used = ++s->tick;
        lru_touch(s, sl, 0, 0);
        sl->prefetched = 1;
        s->pf_issued++;
        s->pf_bytes += sl->bytes;
        return 1;
    }
    return 0;
}

/* 1 when paged calls may read hinted experts ahead (a store reading a file
 * with prefetch on). */
int vh_store_prefetching(const ExpertStore *s) { return store_ok(s) && !s->dev_base && !s->prefetch_off; }

int expert_store_set_prefetch(ExpertStore *s, int on) {
    if (!store_ok(s)) return -EINVAL;
    s->prefetch_off = !on;
    if (!on) s->hint_layer = -1;
    return 0;
}

void expert_store_prefetch_stats(const ExpertStore *s, uint64_t out[3]) {
    if (!out) return;
    out[0] = out[1] = out[2] = 0;
    if (!store_ok(s)) return;
    out[0] = s->pf_issued;
    out[1] = s->pf_used;
    out[2] = s->pf_bytes;
}

/* The store's own file descriptor, for callers that need to know whether
 * page-ins read a file (-1 for a device-backed store). */
int vh_store_fd(const ExpertStore *s) { return store_ok(s) && !s->dev_base ? s->fd : -1; }
