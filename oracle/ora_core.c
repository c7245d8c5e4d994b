/*
 * oracle/ora_core.c -- CPU oracle (test infrastructure): arena, globals,
 * tensor lifetime, xorshift32 generators, broadcasting, graph walk, thread pool.
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <threads.h>

#include "ora.h"
#include "ora_internal.h"

/* ------------------------------------------------------------------ globals */
/* pico_init picks AVX2 (src/global.c:21-23,35); with that level the matmul
 * dispatch has no AVX2 case and falls to the scalar kernel (cpu_kernels.h:46-55). */
SimdLevel g_simd_level = SIMD_NONE;
uint32_t x_state = 123456789u; /* src/global.c:13 */
static int g_initialized = 0;

void pico_init(void) {
    /* src/global.c:29-69.  The reference also reseeds x_state from time() and
     * prints a banner; the oracle keeps the generator deterministic. */
    if(g_initialized) return;
    g_simd_level = SIMD_AVX2;
    g_initialized = 1;
    ora_pool_start(8); /* src/global.c:62: 8 workers */
}

void pico_shutdown(void) {
    ora_pool_stop();
    g_initialized = 0;
}

void ora_set_seed(uint32_t seed) { x_state = seed ? seed : 123456789u; }
void ora_set_simd(int level) { g_simd_level = (SimdLevel)level; }
int ora_get_simd(void) { return (int)g_simd_level; }

/* -------------------------------------------------------------------- arena
 * src/arena.h:38-169.  One deliberate difference: a growth block is sized
 * max(first block, request) so one oversized tensor cannot fail (the
 * reference reuses the first block's capacity, arena.h:81,113). */
static thread_local struct Arena* ctx_stack[16];
static thread_local int ctx_top = -1;

static struct ArenaBlock* block_new(size_t bytes) {
    struct ArenaBlock* b = (struct ArenaBlock*)malloc(sizeof(*b));
    if(!b) return NULL;
    b->bottom = (unsigned char*)malloc(bytes ? bytes : 1);
    if(!b->bottom) {
        free(b);
        return NULL;
    }
    b->curr = b->bottom;
    b->capacity = bytes;
    b->next = NULL;
    return b;
}

struct Arena* arena_init(size_t bytes) {
    struct Arena* a = (struct Arena*)malloc(sizeof(*a));
    if(!a) return NULL;
    a->begin = a->end = block_new(bytes);
    if(!a->begin) {
        free(a);
        return NULL;
    }
    return a;
}

void* arena_alloc(struct Arena* a, size_t size) {
    size = (size + 15) & ~(size_t)15;
    struct ArenaBlock* b = a->end;
    if((size_t)(b->curr - b->bottom) + size > b->capacity) {
        size_t cap = a->begin->capacity > size ? a->begin->capacity : size;
        struct ArenaBlock* nb = block_new(cap);
        if(!nb) {
            fprintf(stderr, "Memory allocation failed!\n");
            exit(1);
        }
        b->next = nb;
        a->end = b = nb;
    }
    void* p = b->curr;
    b->curr += size;
    return p;
}

void arena_reset(struct Arena* a) {
    struct ArenaBlock* c = a->begin->next;
    while(c) {
        struct ArenaBlock* n = c->next;
        free(c->bottom);
        free(c);
        c = n;
    }
    a->begin->curr = a->begin->bottom;
    a->begin->next = NULL;
    a->end = a->begin;
}

void arena_destroy(struct Arena* a) {
    struct ArenaBlock* c = a->begin;
    while(c) {
        struct ArenaBlock* n = c->next;
        free(c->bottom);
        free(c);
        c = n;
    }
    free(a);
}

void arena_ctx_push(struct Arena* a) { ctx_stack[++ctx_top] = a; }
void arena_ctx_pop(void) { ctx_top--; }
struct Arena* arena_ctx_current(void) {
    if(ctx_top < 0 || ctx_top >= 16) return NULL;
    return ctx_stack[ctx_top];
}

/* ------------------------------------------------------------------ tensors */
void ora_contig_strides(const int64_t* shape, int ndim, int64_t* strides) {
    int64_t s = 1;
    for(int d = ndim - 1; d >= 0; d--) {
        strides[d] = s;
        s *= shape[d];
    }
}

static int64_t numel_of(const int64_t* shape, int ndim) {
    int64_t n = 1;
    for(int d = 0; d < ndim; d++) n *= shape[d];
    return n;
}

struct PicoTensor* pico_param(int64_t* shape, uint8_t ndim) {
    /* src/tensor.c:44-84: calloc'd, persistent, zeroed data and grad */
    struct PicoTensor* t = (struct PicoTensor*)calloc(1, sizeof(*t));
    if(!t) return NULL;
    t->ndim = ndim;
    t->is_persistent = 1;
    t->numel = numel_of(shape, ndim);
    t->shape = (int64_t*)calloc(ndim, sizeof(int64_t));
    t->strides = (int64_t*)calloc(ndim, sizeof(int64_t));
    t->data = (float*)calloc((size_t)t->numel, sizeof(float));
    t->grad = (float*)calloc((size_t)t->numel, sizeof(float));
    if(!t->shape || !t->strides || !t->data || !t->grad) {
        free(t->shape);
        free(t->strides);
        free(t->data);
        free(t->grad);
        free(t);
        return NULL;
    }
    memcpy(t->shape, shape, ndim * sizeof(int64_t));
    ora_contig_strides(shape, ndim, t->strides);
    return t;
}

struct PicoTensor* pico_create_tensor(struct Arena* arena, int64_t* shape, uint8_t ndim) {
    /* src/tensor.c:86-134: arena-backed, data and grad zeroed, backend CPU */
    struct PicoTensor* t = (struct PicoTensor*)arena_alloc(arena, sizeof(*t));
    memset(t, 0, sizeof(*t));
    t->ndim = ndim;
    t->backend = CPU;
    t->numel = numel_of(shape, ndim);
    t->shape = (int64_t*)arena_alloc(arena, ndim * sizeof(int64_t));
    t->strides = (int64_t*)arena_alloc(arena, ndim * sizeof(int64_t));
    memcpy(t->shape, shape, ndim * sizeof(int64_t));
    ora_contig_strides(shape, ndim, t->strides);
    t->data = (float*)arena_alloc(arena, (size_t)t->numel * sizeof(float));
    t->grad = (float*)arena_alloc(arena, (size_t)t->numel * sizeof(float));
    memset(t->data, 0, (size_t)t->numel * sizeof(float));
    memset(t->grad, 0, (size_t)t->numel * sizeof(float));
    return t;
}

struct PicoTensor* pico_tensor_from_scalar(float value) {
    struct Arena* ar = arena_ctx_current();
    if(!ar) {
        fprintf(stderr, "[Pico] Error: No current arena in context!\n");
        return NULL;
    }
    int64_t s[1] = {1};
    struct PicoTensor* t = pico_create_tensor(ar, s, 1);
    t->data[0] = value;
    return t;
}

void pico_free(struct PicoTensor* t) {
    /* src/tensor.c:136-168: no-op for arena tensors */
    if(!t || !t->is_persistent) return;
    free(t->shape);
    free(t->strides);
    free(t->data);
    free(t->grad);
    free(t->parents);
    free(t);
}

void pico_transpose_2d(struct PicoTensor* t) {
    /* src/tensor.c:230-244: swap shape and strides, data untouched */
    if(t->ndim != 2) {
        fprintf(stderr, "Error: This is not a rank 2 tensor!\n");
        return;
    }
    int64_t s = t->shape[0];
    t->shape[0] = t->shape[1];
    t->shape[1] = s;
    s = t->strides[0];
    t->strides[0] = t->strides[1];
    t->strides[1] = s;
}

/* -------------------------------------------------------------- generators */
/* xorshift32 with shifts (13, 17, 5), src/tensor.c:249-256 */
static inline uint32_t xs32(uint32_t* s) {
    uint32_t x = *s;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return *s = x;
}

/* [0,1) from the top 23 bits through the [1,2) exponent trick, src/tensor.c:259-266 */
static inline float u01(uint32_t r) {
    uint32_t bits = (r >> 9) | 0x3F800000u;
    float f;
    memcpy(&f, &bits, 4);
    return f - 1.0f;
}

void ora_fill_pico_rand(float* out, int64_t n, uint32_t seed) {
    uint32_t s = seed ? seed : 123456789u;
    for(int64_t i = 0; i < n; i++) out[i] = u01(xs32(&s));
}

void ora_fill_uniform(float* out, int64_t n, uint32_t seed, float lo, float hi) {
    uint32_t s = seed ? seed : 123456789u;
    for(int64_t i = 0; i < n; i++) out[i] = lo + (hi - lo) * u01(xs32(&s));
}

/* flat Box-Muller over the whole buffer; u1 in (0,1] so log never sees 0.
 * (pico_randn, src/tensor.c:348-367, halves only the last dim and can hit log(0);
 * the seeded inputs of every config use this flat form instead.) */
void ora_fill_normal(float* out, int64_t n, uint32_t seed, float mean, float std) {
    uint32_t s = seed ? seed : 123456789u;
    for(int64_t i = 0; i < n; i += 2) {
        double u1 = 1.0 - (double)u01(xs32(&s));
        double u2 = (double)u01(xs32(&s));
        double r = sqrt(-2.0 * log(u1));
        double a = 6.283185307179586 * u2;
        out[i] = (float)(mean + std * r * cos(a));
        if(i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(a));
    }
}

void ora_fill_labels(int32_t* out, int64_t n, uint32_t seed, int32_t vocab) {
    uint32_t s = seed ? seed : 123456789u;
    for(int64_t i = 0; i < n; i++) out[i] = (int32_t)(xs32(&s) % (uint32_t)vocab);
}

struct PicoTensor* pico_rand(struct Arena* arena, int64_t* shape, uint8_t ndim) {
    struct PicoTensor* t = pico_create_tensor(arena, shape, ndim);
    for(int64_t i = 0; i < t->numel; i++) t->data[i] = u01(xs32(&x_state));
    return t;
}

/* ------------------------------------------------------------- broadcasting */
uint8_t pico_check_broadcast_compatibility(struct PicoTensor* a, struct PicoTensor* b) {
    /* src/tensor.c:371-397: right-aligned, equal or one of them 1 */
    for(int i = a->ndim - 1, j = b->ndim - 1; i >= 0 && j >= 0; i--, j--) {
        if(a->shape[i] != b->shape[j] && a->shape[i] != 1 && b->shape[j] != 1) return 0;
    }
    return 1;
}

/* src/tensor.h:122-138: flat output index -> flat index into a broadcast input */
int64_t ora_map_index(int64_t gi, const int64_t* t_shape, const int64_t* t_strides, int t_ndim,
                      const int64_t* out_strides, int out_ndim) {
    int64_t idx = 0, rem = gi;
    int diff = out_ndim - t_ndim;
    for(int d = 0; d < out_ndim; d++) {
        int64_t c = rem / out_strides[d];
        rem %= out_strides[d];
        int sd = d - diff;
        if(sd >= 0 && t_shape[sd] > 1) idx += c * t_strides[sd];
    }
    return idx;
}

/* --------------------------------------------------------------- graph walk */
struct NodeList {
    struct PicoTensor** v;
    int n, cap;
};
static void nl_push(struct NodeList* l, struct PicoTensor* t) {
    if(l->n == l->cap) {
        l->cap = l->cap ? 2 * l->cap : 32;
        l->v = (struct PicoTensor**)realloc(l->v, l->cap * sizeof(*l->v));
    }
    l->v[l->n++] = t;
}
static int nl_has(struct NodeList* l, struct PicoTensor* t) {
    for(int i = 0; i < l->n; i++)
        if(l->v[i] == t) return 1;
    return 0;
}
static void postorder(struct PicoTensor* t, struct NodeList* order, struct NodeList* seen) {
    if(!t || nl_has(seen, t)) return;
    nl_push(seen, t);
    for(int i = 0; i < t->num_parents; i++) postorder(t->parents[i], order, seen);
    nl_push(order, t);
}

void pico_backward(struct Arena* arena, struct PicoTensor* entry) {
    /* src/tensor.c:15-42: post-order DFS, seed entry grad with 1 over all
     * elements, then call each _backward from the entry towards the leaves. */
    (void)arena;
    struct NodeList order = {0}, seen = {0};
    postorder(entry, &order, &seen);
    if(order.n == 0) return;
    struct PicoTensor* e = order.v[order.n - 1];
    for(int64_t i = 0; i < e->numel; i++) e->grad[i] = 1.0f;
    for(int i = order.n - 1; i >= 0; i--)
        if(order.v[i]->_backward) order.v[i]->_backward(order.v[i]);
    free(order.v);
    free(seen.v);
}

/* --------------------------------------------------------------- thread pool
 * A fixed set of workers pulling jobs from a FIFO under one mutex; wait() is a
 * barrier on "queue empty and nobody working" (the contract of src/tpool.h:98-368). */
struct Job {
    void (*fn)(void*);
    void* arg;
    struct Job* next;
};
static struct {
    pthread_mutex_t mu;
    pthread_cond_t ready, done;
    struct Job *head, *tail;
    pthread_t* th;
    int nthreads, busy, stop, started;
} pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER};
static int g_matmul_threads = 8;

static void* worker(void* unused) {
    (void)unused;
    pthread_mutex_lock(&pool.mu);
    for(;;) {
        while(!pool.head && !pool.stop) pthread_cond_wait(&pool.ready, &pool.mu);
        if(pool.stop && !pool.head) break;
        struct Job* j = pool.head;
        pool.head = j->next;
        if(!pool.head) pool.tail = NULL;
        pool.busy++;
        pthread_mutex_unlock(&pool.mu);
        j->fn(j->arg);
        free(j);
        pthread_mutex_lock(&pool.mu);
        pool.busy--;
        if(!pool.head && pool.busy == 0) pthread_cond_broadcast(&pool.done);
    }
    pthread_mutex_unlock(&pool.mu);
    return NULL;
}

void ora_pool_start(int n) {
    if(pool.started) return;
    pool.stop = 0;
    pool.nthreads = n;
    pool.th = (pthread_t*)calloc(n, sizeof(pthread_t));
    for(int i = 0; i < n; i++) pthread_create(&pool.th[i], NULL, worker, NULL);
    pool.started = 1;
}

void ora_pool_stop(void) {
    if(!pool.started) return;
    pthread_mutex_lock(&pool.mu);
    pool.stop = 1;
    pthread_cond_broadcast(&pool.ready);
    pthread_mutex_unlock(&pool.mu);
    for(int i = 0; i < pool.nthreads; i++) pthread_join(pool.th[i], NULL);
    free(pool.th);
    pool.th = NULL;
    pool.started = 0;
}

void ora_pool_add(void (*fn)(void*), void* arg) {
    struct Job* j = (struct Job*)malloc(sizeof(*j));
    j->fn = fn;
    j->arg = arg;
    j->next = NULL;
    pthread_mutex_lock(&pool.mu);
    if(pool.tail)
        pool.tail->next = j;
    else
        pool.head = j;
    pool.tail = j;
    pthread_cond_broadcast(&pool.ready);
    pthread_mutex_unlock(&pool.mu);
}

void ora_pool_wait(void) {
    pthread_mutex_lock(&pool.mu);
    while(pool.head || pool.busy) pthread_cond_wait(&pool.done, &pool.mu);
    pthread_mutex_unlock(&pool.mu);
}

void ora_set_threads(int n) {
    if(n < 1) n = 1;
    if(pool.started && n > pool.nthreads) {
        ora_pool_stop();
        ora_pool_start(n);
    } else if(!pool.started) {
        ora_pool_start(n > 8 ? n : 8);
    }
    g_matmul_threads = n;
}
int ora_matmul_threads(void) { return g_matmul_threads; }

/* run fn(i) for i in [0,n) over the pool, in contiguous chunks */
struct RangeJob {
    void (*fn)(void*, int64_t, int64_t);
    void* ctx;
    int64_t lo, hi;
};
static void range_entry(void* p) {
    struct RangeJob* j = (struct RangeJob*)p;
    j->fn(j->ctx, j->lo, j->hi);
}
void ora_parallel_for(int64_t n, void (*fn)(void*, int64_t, int64_t), void* ctx) {
    if(!pool.started) ora_pool_start(8);
    int nt = pool.nthreads;
    if(n < 2 * nt) {
        fn(ctx, 0, n);
        return;
    }
    struct RangeJob* jobs = (struct RangeJob*)malloc(nt * sizeof(*jobs));
    for(int t = 0; t < nt; t++) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].lo = n * t / nt;
        jobs[t].hi = n * (t + 1) / nt;
        ora_pool_add(range_entry, &jobs[t]);
    }
    ora_pool_wait();
    free(jobs);
}
