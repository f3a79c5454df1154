/* A host-memory stand-in for the HIP runtime calls that vireo_amd/csrc/
 * expert_store.c makes, for running the store under ThreadSanitizer and
 * AddressSanitizer on a machine without a GPU (tests/test_store_sanitizers.py).
 *
 * "Device" memory is host memory. Every stream made by hipStreamCreate runs
 * its work (copies, event records, event waits, and the test's own "kernels"
 * from stub_launch) in order on a thread of its own, so asynchronous copies
 * really overlap the caller, as they do on a GPU. The null stream is the
 * legacy default stream: its work runs in the calling thread after every
 * other stream has drained. One mutex and one condition variable guard all
 * of the stand-in's state, so the sanitizers see every hand-off between the
 * caller and the stream threads through them. */
#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OP_COPY, OP_RECORD, OP_WAIT, OP_FN };

typedef struct Op {
    int kind;
    void *dst;
    const void *src;
    size_t n;
    hipEvent_t ev;
    uint64_t gen;
    void (*fn)(void *);
    void *arg;
    struct Op *next;
} Op;

struct ihipStream_t {
    pthread_t th;
    Op *head, *tail;
    int busy, quit;
    struct ihipStream_t *next_all;
};

struct ihipEvent_t {
    uint64_t recorded, done;
    int refs, dead;  /* queued records and waits naming it; destroyed while some were queued */
};

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_cv = PTHREAD_COND_INITIALIZER;
static struct ihipStream_t *g_streams;

static void *worker(void *p) {
    struct ihipStream_t *s = (struct ihipStream_t *)p;
    pthread_mutex_lock(&g_mu);
    for (;;) {
        while (!s->head && !s->quit) pthread_cond_wait(&g_cv, &g_mu);
        if (!s->head) break;
        Op *op = s->head;
        if (op->kind == OP_WAIT)
            while (op->ev->done < op->gen) pthread_cond_wait(&g_cv, &g_mu);
        s->busy = 1;
        pthread_mutex_unlock(&g_mu);
        if (op->kind == OP_COPY) memcpy(op->dst, op->src, op->n);
        if (op->kind == OP_FN) op->fn(op->arg);
        pthread_mutex_lock(&g_mu);
        if (op->kind == OP_RECORD && op->ev->done < op->gen) op->ev->done = op->gen;
        if ((op->kind == OP_RECORD || op->kind == OP_WAIT) && --op->ev->refs == 0 && op->ev->dead) free(op->ev);
        s->head = op->next;
        if (!s->head) s->tail = NULL;
        s->busy = 0;
        free(op);
        pthread_cond_broadcast(&g_cv);
    }
    pthread_mutex_unlock(&g_mu);
    return NULL;
}

/* with g_mu held: every stream idle */
static void drain_all_locked(void) {
    for (;;) {
        int idle = 1;
        for (struct ihipStream_t *s = g_streams; s; s = s->next_all)
            if (s->head || s->busy) idle = 0;
        if (idle) return;
        pthread_cond_wait(&g_cv, &g_mu);
    }
}

static void drain_all(void) {
    pthread_mutex_lock(&g_mu);
    drain_all_locked();
    pthread_mutex_unlock(&g_mu);
}

static hipError_t enqueue(hipStream_t s, Op *op) {
    op->next = NULL;
    pthread_mutex_lock(&g_mu);
    if (s->tail) s->tail->next = op;
    else s->head = op;
    s->tail = op;
    pthread_cond_broadcast(&g_cv);
    pthread_mutex_unlock(&g_mu);
    return hipSuccess;
}

static Op *new_op(int kind) {
    Op *op = (Op *)calloc(1, sizeof(Op));
    if (op) op->kind = kind;
    return op;
}

hipError_t hipStreamCreate(hipStream_t *out) {
    struct ihipStream_t *s = (struct ihipStream_t *)calloc(1, sizeof *s);
    if (!s) return hipErrorOutOfMemory;
    pthread_mutex_lock(&g_mu);
    s->next_all = g_streams;
    g_streams = s;
    pthread_mutex_unlock(&g_mu);
    if (pthread_create(&s->th, NULL, worker, s) != 0) return hipErrorOutOfMemory;
    *out = s;
    return hipSuccess;
}

hipError_t hipStreamDestroy(hipStream_t s) {
    pthread_mutex_lock(&g_mu);
    s->quit = 1;
    pthread_cond_broadcast(&g_cv);
    pthread_mutex_unlock(&g_mu);
    pthread_join(s->th, NULL);
    pthread_mutex_lock(&g_mu);
    for (struct ihipStream_t **p = &g_streams; *p; p = &(*p)->next_all)
        if (*p == s) {
            *p = s->next_all;
            break;
        }
    pthread_mutex_unlock(&g_mu);
    free(s);
    return hipSuccess;
}

hipError_t hipMalloc(void **p, size_t n) {
    *p = aligned_alloc(256, (n + 255) & ~(size_t)255);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void *p) {
    free(p);
    return hipSuccess;
}
hipError_t hipHostMalloc(void **p, size_t n, unsigned int flags) {
    (void)flags;
    *p = aligned_alloc(4096, (n + 4095) & ~(size_t)4095);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void *p) {
    free(p);
    return hipSuccess;
}

hipError_t hipMemcpy(void *dst, const void *src, size_t n, hipMemcpyKind kind) {
    (void)kind;
    drain_all();
    memcpy(dst, src, n);
    return hipSuccess;
}

hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind kind, hipStream_t s) {
    (void)kind;
    if (!s) return hipMemcpy(dst, src, n, kind);
    Op *op = new_op(OP_COPY);
    if (!op) return hipErrorOutOfMemory;
    op->dst = dst;
    op->src = src;
    op->n = n;
    return enqueue(s, op);
}

hipError_t hipEventCreateWithFlags(hipEvent_t *ev, unsigned flags) {
    (void)flags;
    *ev = (hipEvent_t)calloc(1, sizeof(struct ihipEvent_t));
    return *ev ? hipSuccess : hipErrorOutOfMemory;
}

hipError_t hipEventRecord(hipEvent_t ev, hipStream_t s) {
    if (!s) {
        pthread_mutex_lock(&g_mu);
        drain_all_locked();
        ev->done = ++ev->recorded;
        pthread_cond_broadcast(&g_cv);
        pthread_mutex_unlock(&g_mu);
        return hipSuccess;
    }
    Op *op = new_op(OP_RECORD);
    if (!op) return hipErrorOutOfMemory;
    op->ev = ev;
    pthread_mutex_lock(&g_mu);
    op->gen = ++ev->recorded;
    ev->refs++;
    pthread_mutex_unlock(&g_mu);
    return enqueue(s, op);
}

hipError_t hipEventSynchronize(hipEvent_t ev) {
    pthread_mutex_lock(&g_mu);
    const uint64_t target = ev->recorded;
    while (ev->done < target) pthread_cond_wait(&g_cv, &g_mu);
    pthread_mutex_unlock(&g_mu);
    return hipSuccess;
}

hipError_t hipEventQuery(hipEvent_t ev) {
    pthread_mutex_lock(&g_mu);
    const int done = ev->done >= ev->recorded;
    pthread_mutex_unlock(&g_mu);
    return done ? hipSuccess : hipErrorNotReady;
}

/* as on a GPU, work already queued that names the event still completes:
 * the memory goes when the last such record or wait has run */
hipError_t hipEventDestroy(hipEvent_t ev) {
    pthread_mutex_lock(&g_mu);
    if (ev->refs == 0) free(ev);
    else ev->dead = 1;
    pthread_mutex_unlock(&g_mu);
    return hipSuccess;
}

hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t ev, unsigned int flags) {
    (void)flags;
    if (!s) return hipEventSynchronize(ev);
    Op *op = new_op(OP_WAIT);
    if (!op) return hipErrorOutOfMemory;
    op->ev = ev;
    pthread_mutex_lock(&g_mu);
    op->gen = ev->recorded;
    ev->refs++;
    pthread_mutex_unlock(&g_mu);
    return enqueue(s, op);
}

hipError_t hipStreamSynchronize(hipStream_t s) {
    pthread_mutex_lock(&g_mu);
    if (!s) drain_all_locked();
    else
        while (s->head || s->busy) pthread_cond_wait(&g_cv, &g_mu);
    pthread_mutex_unlock(&g_mu);
    return hipSuccess;
}

hipError_t hipDeviceSynchronize(void) {
    drain_all();
    return hipSuccess;
}

hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus *st) {
    (void)s;
    *st = hipStreamCaptureStatusNone;
    return hipSuccess;
}

hipError_t hipGetLastError(void) { return hipSuccess; }

/* The test's "kernel": fn(arg) runs in stream order (on the null stream: now,
 * after every stream has drained). */
void stub_launch(hipStream_t s, void (*fn)(void *), void *arg) {
    if (!s) {
        drain_all();
        fn(arg);
        return;
    }
    Op *op = new_op(OP_FN);
    if (!op) abort();
    op->fn = fn;
    op->arg = arg;
    enqueue(s, op);
}
