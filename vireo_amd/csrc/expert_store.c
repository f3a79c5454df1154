/* ExpertStore with an HBM resident pool (API: include/vireo_expert_store.h,
 * extensions in include/vireo_hip.h).
 *
 * Paging policy, budget accounting and statistics follow the reference
 * src/expert_store.c:
 *   - lookup of an unregistered expert returns -1 with a zeroed view (:75);
 *   - a hit bumps `hits`; a miss bumps `misses`, evicts unleased residents in
 *     least-recently-used order until the expert fits, and stays over budget if
 *     everything resident is leased (:52-63); bytes_read grows by each slice
 *     read (:65-70);
 *   - every lookup sets last_used = ++tick and takes a lease (:88-90);
 *     release drops one lease and zeroes the view (:94-98).
 * What differs is where a resident expert lives: one device allocation holding
 * gate | up | down, each at a 256-byte boundary, filled by pread into pinned
 * host staging and a copy to HBM. A store created over a device buffer
 * (expert_store_create_device) makes slices resident by pointing into that
 * buffer, with no copy. */
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
} Slot;

typedef struct { void *ptr; uint64_t size; } FreeBlock;

struct ExpertStore {
    int fd;
    const uint8_t *dev_base;   /* device-resident backing, or NULL */
    uint64_t dev_size;
    int n_layers, n_experts, n_slots;
    Slot *slots;
    uint64_t tick, resident_bytes, capacity_bytes;
    ExpertStats st;
    void *stage;               /* pinned staging for pread */
    size_t stage_bytes;
    void **tables;             /* per layer: device [n_experts x 3] pointer table */
    FreeBlock *freel;          /* device blocks of evicted experts, kept for reuse */
    int nfree, capfree;
};

static uint64_t al256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

static Slot *slot_at(ExpertStore *s, int layer, int expert) {
    if (!s || layer < 0 || layer >= s->n_layers || expert < 0 || expert >= s->n_experts) return NULL;
    return &s->slots[(size_t)layer * s->n_experts + expert];
}

static ExpertStore *store_new(int n_layers, int n_experts, uint64_t capacity_bytes) {
    if (n_layers <= 0 || n_experts <= 0) return NULL;
    ExpertStore *s = calloc(1, sizeof *s);
    if (!s) return NULL;
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

static void release_block(ExpertStore *s, Slot *v) {
    if (v->dev) {
        if (s->nfree == s->capfree) {
            int nc = s->capfree ? 2 * s->capfree : 64;
            FreeBlock *nf = realloc(s->freel, (size_t)nc * sizeof *nf);
            if (nf) { s->freel = nf; s->capfree = nc; }
        }
        if (s->nfree < s->capfree) s->freel[s->nfree++] = (FreeBlock){v->dev, v->alloc};
        else (void)hipFree(v->dev);
    }
    v->dev = NULL;
    v->gate = v->up = v->down = NULL;
}

static void evict_one(ExpertStore *s, Slot *v) {
    release_block(s, v);
    v->resident = 0;
    s->resident_bytes -= v->bytes;
    s->st.experts_resident--;
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

static void *take_block(ExpertStore *s, uint64_t size) {
    for (int i = 0; i < s->nfree; i++)
        if (s->freel[i].size == size) {
            void *p = s->freel[i].ptr;
            s->freel[i] = s->freel[--s->nfree];
            return p;
        }
    void *p = NULL;
    if (hipMalloc(&p, size) != hipSuccess) {
        /* drop cached blocks and retry once */
        for (int i = 0; i < s->nfree; i++) (void)hipFree(s->freel[i].ptr);
        s->nfree = 0;
        if (hipMalloc(&p, size) != hipSuccess) return NULL;
    }
    return p;
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
    uint8_t *b = (uint8_t *)s->stage;
    uint64_t done = 0;
    while (done < bytes) {
        ssize_t r = pread(s->fd, b + done, bytes - done, (off_t)(off + done));
        if (r <= 0) return -EIO;
        done += (uint64_t)r;
    }
    if (hipMemcpy(dst, s->stage, bytes, hipMemcpyHostToDevice) != hipSuccess) return -EIO;
    return 0;
}

/* Make sl resident: alias the device backing, or allocate HBM and page in. */
static int page_in(ExpertStore *s, Slot *sl) {
    const ExpertSlices *L = &sl->loc;
    if (s->dev_base) {
        uint64_t ends[3] = {L->gate_off + L->gate_bytes, L->up_off + L->up_bytes, L->down_off + L->down_bytes};
        for (int i = 0; i < 3; i++) if (ends[i] > s->dev_size) return -EINVAL;
        sl->gate = s->dev_base + L->gate_off;
        sl->up = s->dev_base + L->up_off;
        sl->down = s->dev_base + L->down_off;
        s->st.bytes_read += (uint64_t)L->gate_bytes + L->up_bytes + L->down_bytes;
        return 0;
    }
    uint64_t og = 0, ou = al256(L->gate_bytes), od = ou + al256(L->up_bytes);
    uint64_t size = od + al256(L->down_bytes);
    uint8_t *blk = take_block(s, size);
    if (!blk) return -ENOMEM;
    int rc = read_slice(s, L->gate_off, L->gate_bytes, blk + og);
    if (!rc) rc = read_slice(s, L->up_off, L->up_bytes, blk + ou);
    if (!rc) rc = read_slice(s, L->down_off, L->down_bytes, blk + od);
    if (rc) {
        Slot tmp = *sl;
        tmp.dev = blk; tmp.alloc = size;
        release_block(s, &tmp);
        return rc;
    }
    s->st.bytes_read += (uint64_t)L->gate_bytes + L->up_bytes + L->down_bytes;
    sl->dev = blk;
    sl->alloc = size;
    sl->gate = blk + og;
    sl->up = blk + ou;
    sl->down = blk + od;
    return 0;
}

int expert_store_lookup(ExpertStore *s, int layer, int expert, ExpertView *view) {
    if (!view) return -EINVAL;
    Slot *sl = slot_at(s, layer, expert);
    if (!sl) { memset(view, 0, sizeof *view); return -EINVAL; }
    s->st.requests++;
    if (!sl->registered) { memset(view, 0, sizeof *view); return -1; }
    if (sl->resident) {
        s->st.hits++;
    } else {
        s->st.misses++;
        make_room(s, sl->bytes);
        int rc = page_in(s, sl);
        if (rc) { memset(view, 0, sizeof *view); return rc; }
        sl->resident = 1;
        s->resident_bytes += sl->bytes;
        s->st.experts_resident++;
    }
    sl->last_used = ++s->tick;
    sl->lease++;
    view->gate = sl->gate;
    view->up = sl->up;
    view->down = sl->down;
    view->slot = sl;
    return 0;
}

void expert_store_release(ExpertStore *s, ExpertView *view) {
    (void)s;
    if (view && view->slot) {
        Slot *sl = (Slot *)view->slot;
        if (sl->lease > 0) sl->lease--;
    }
    if (view) memset(view, 0, sizeof *view);
}

void expert_store_stats(const ExpertStore *s, ExpertStats *out) {
    if (!s || !out) return;
    *out = s->st;
    out->resident_bytes = s->resident_bytes;
    out->capacity_bytes = s->capacity_bytes;
    out->experts_resident = s->st.experts_resident;
}

int expert_store_pin_layer(ExpertStore *s, int layer, const void *const **dev_table) {
    if (!s || !dev_table || layer < 0 || layer >= s->n_layers) return -EINVAL;
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
        rc = expert_store_lookup(s, layer, e, &v);
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
    if (!s || layer < 0 || layer >= s->n_layers) return -EINVAL;
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
    if (!s) return;
    (void)hipDeviceSynchronize();
    for (int l = 0; l < s->n_layers; l++) if (s->tables[l]) (void)hipFree(s->tables[l]);
    for (int i = 0; i < s->n_slots; i++) if (s->slots[i].dev) (void)hipFree(s->slots[i].dev);
    for (int i = 0; i < s->nfree; i++) (void)hipFree(s->freel[i].ptr);
    if (s->stage) (void)hipHostFree(s->stage);
    free(s->freel);
    free(s->tables);
    free(s->slots);
    free(s);
}

/* Bytes an expert takes in the pool (0 if unregistered), and the pool's
 * capacity (0 = unbounded), for callers that page experts in batches. */
uint64_t vh_store_expert_bytes(const ExpertStore *s, int layer, int expert) {
    const Slot *sl = (s && layer >= 0 && layer < s->n_layers && expert >= 0 && expert < s->n_experts)
                         ? &s->slots[(size_t)layer * (size_t)s->n_experts + (size_t)expert]
                         : NULL;
    return sl && sl->registered ? sl->bytes : 0;
}
uint64_t vh_store_capacity(const ExpertStore *s) { return s ? s->capacity_bytes : 0; }
