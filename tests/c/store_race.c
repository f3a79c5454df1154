/* The HBM ExpertStore's paging under the sanitizers (tests/test_store_sanitizers.py):
 * a file-backed store smaller than the model serves routed experts layer
 * after layer the way the paged MoE plan does - page-ins on a copy stream
 * (parallel pread workers, the pinned staging ring), a copy fence into the
 * compute stream, "kernels" on that stream that read every byte of each view
 * and check it against the file, leases dropped behind them (the event that
 * guards a block's reuse), the next layer's guess read ahead, routing notes
 * copied back from the "device", and synchronous lookups on the null stream
 * in between. Built with hip_host_stub.c against expert_store.c; exits 0 when
 * every byte read matched and every call succeeded. */
#include <hip/hip_runtime_api.h>
#include <errno.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "vireo_expert_store.h"

int vh_store_acquire(ExpertStore *s, int layer, int expert, ExpertView *view, hipStream_t cs);
int vh_store_drop(ExpertStore *s, ExpertView *view, hipStream_t stream);
int vh_store_copy_fence(ExpertStore *s, hipStream_t cs, hipStream_t stream);
void vh_store_hint(ExpertStore *s, int layer, const int32_t *ids, int n);
int vh_store_prefetch_next(ExpertStore *s, int layer, hipStream_t cs);
int vh_store_note_routing(ExpertStore *s, int layer, const int32_t *idx_dev, int T, int k, hipStream_t stream);
void expert_store_hbm_stats(const ExpertStore *s, ExpertStats *out);
void stub_launch(hipStream_t s, void (*fn)(void *), void *arg);

enum { NL = 3, NE = 8, K = 3, ITERS = 48 };
static const uint32_t SZ[3] = {300 * 1024 + 36, 300 * 1024 + 36, 200 * 1024 + 10};  /* gate, up, down */

static uint8_t pattern(uint64_t off) { return (uint8_t)((off * 2654435761u) >> 13); }

static pthread_mutex_t g_bad_mu = PTHREAD_MUTEX_INITIALIZER;
static long g_bad;

typedef struct {
    const uint8_t *p[3];
    uint64_t off[3];
} Check;

/* a "kernel": every byte of a view against the file */
static void check_view(void *arg) {
    Check *c = (Check *)arg;
    long bad = 0;
    for (int i = 0; i < 3; i++)
        for (uint32_t j = 0; j < SZ[i]; j++)
            if (c->p[i][j] != pattern(c->off[i] + j)) bad++;
    pthread_mutex_lock(&g_bad_mu);
    g_bad += bad;
    pthread_mutex_unlock(&g_bad_mu);
    free(c);
}

typedef struct {
    int32_t *dst;
    int32_t ids[K];
} SetIdx;

/* a "kernel" that writes the routing the note copies back */
static void set_idx(void *arg) {
    SetIdx *a = (SetIdx *)arg;
    memcpy(a->dst, a->ids, sizeof a->ids);
    free(a);
}

static uint64_t slice_off(int l, int e, int i) {
    uint64_t o = 4096 + ((uint64_t)l * NE + e) * (SZ[0] + SZ[1] + SZ[2]);
    for (int j = 0; j < i; j++) o += SZ[j];
    return o;
}

static void enqueue_check(hipStream_t ks, const ExpertView *v, int l, int e) {
    Check *c = (Check *)malloc(sizeof *c);
    if (!c) abort();
    c->p[0] = (const uint8_t *)v->gate;
    c->p[1] = (const uint8_t *)v->up;
    c->p[2] = (const uint8_t *)v->down;
    for (int i = 0; i < 3; i++) c->off[i] = slice_off(l, e, i);
    stub_launch(ks, check_view, c);
}

#define CK(x)                                                                         \
    do {                                                                              \
        int rc_ = (x);                                                                \
        if (rc_ < 0) {                                                                \
            fprintf(stderr, "%s failed: %d (line %d)\n", #x, rc_, __LINE__);          \
            return 1;                                                                 \
        }                                                                             \
    } while (0)

int main(void) {
    char path[] = "/tmp/vireo_store_race_XXXXXX";
    const int fd = mkstemp(path);
    if (fd < 0) return 1;
    unlink(path);
    const uint64_t total = slice_off(NL - 1, NE - 1, 3);
    uint8_t *buf = (uint8_t *)malloc(total);
    if (!buf) return 1;
    for (uint64_t o = 0; o < total; o++) buf[o] = pattern(o);
    if (pwrite(fd, buf, total, 0) != (ssize_t)total) return 1;
    free(buf);

    const uint64_t eb = (uint64_t)SZ[0] + SZ[1] + SZ[2];
    ExpertStore *s = expert_store_create(fd, 5 * eb, NL, NE);  /* five experts of 24 */
    if (!s) return 1;
    for (int l = 0; l < NL; l++)
        for (int e = 0; e < NE; e++) {
            ExpertSlices sl = {slice_off(l, e, 0), slice_off(l, e, 1), slice_off(l, e, 2), SZ[0], SZ[1], SZ[2]};
            expert_store_register(s, l, e, &sl);
        }
    hipStream_t cs, ks;
    if (hipStreamCreate(&cs) != hipSuccess || hipStreamCreate(&ks) != hipSuccess) return 1;
    int32_t *idx_dev;
    if (hipMalloc((void **)&idx_dev, K * sizeof(int32_t)) != hipSuccess) return 1;

    uint32_t rng = 12345u;
    for (int it = 0; it < ITERS; it++) {
        const int l = it % NL, nl = (l + 1) % NL;
        int ids[K];
        for (int j = 0; j < K; j++) {  /* K distinct experts */
            int e;
            int again;
            do {
                rng = rng * 1664525u + 1013904223u;
                e = (int)((rng >> 16) % NE);
                again = 0;
                for (int q = 0; q < j; q++) again |= ids[q] == e;
            } while (again);
            ids[j] = e;
        }
        ExpertView v[K];
        for (int j = 0; j < K; j++) CK(vh_store_acquire(s, l, ids[j], &v[j], cs));
        CK(vh_store_copy_fence(s, cs, ks));
        for (int j = 0; j < K; j++) enqueue_check(ks, &v[j], l, ids[j]);
        SetIdx *si = (SetIdx *)malloc(sizeof *si);
        if (!si) return 1;
        si->dst = idx_dev;
        memcpy(si->ids, ids, sizeof si->ids);
        stub_launch(ks, set_idx, si);
        CK(vh_store_note_routing(s, l, idx_dev, 1, K, ks));
        /* the next layer's guess, read ahead while the checks run */
        int32_t guess[K] = {(ids[0] + 1) % NE, (ids[1] + 3) % NE, (ids[2] + 5) % NE};
        vh_store_hint(s, nl, guess, K);
        CK(vh_store_prefetch_next(s, nl, cs));
        CK(vh_store_prefetch_next(s, nl, cs));
        for (int j = 0; j < K; j++) CK(vh_store_drop(s, &v[j], ks));
        if (it % 7 == 3) {  /* the reference's synchronous lookup on the null stream */
            ExpertView w;
            const int e = (it * 5) % NE;
            CK(expert_store_lookup(s, nl, e, &w));
            enqueue_check(NULL, &w, nl, e);
            expert_store_release(s, &w);
        }
    }
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    ExpertStats st;
    expert_store_hbm_stats(s, &st);
    expert_store_stats(s, &st);
    expert_store_destroy(s);
    hipFree(idx_dev);
    hipStreamDestroy(cs);
    hipStreamDestroy(ks);
    close(fd);
    if (g_bad) {
        fprintf(stderr, "%ld bytes read from the store differ from the file\n", g_bad);
        return 1;
    }
    printf("store_race: %d iterations, every byte read matched\n", ITERS);
    return 0;
}
