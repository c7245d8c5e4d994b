/*
 * tests/host/registry_host_test.c -- host-only test of pico_amd/host/arena.c,
 * built with AddressSanitizer on the CPU (tests/test_registry_host.py).
 *
 * It checks that tensors and arenas allocated the way pico allocates them
 * (a calloc'd 64-byte PicoTensor, tensors packed back to back in one block, a
 * malloc'd 16-byte two-pointer Arena) go through the node lookup and the
 * device-arena calls without a byte read or written outside them, and that
 * the registry finds exactly the nodes this library registered.  Eight
 * threads then check what pico's tests/test_arena.c:160-247 checks of the
 * arena context stack (each thread has its own, the main thread's survives
 * the workers' pushes) while they register, look up and drop nodes in the
 * shared registry at the same time.
 */
#include <pthread.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

/* host stand-ins for runtime.c's device helpers: this test has no GPU */
void* pkh_device_alloc(size_t bytes) { return malloc(bytes); }
void pkh_device_free(void* p) { free(p); }
int pkh_sync(void) { return 0; }

static int g_fail = 0;
#define CHECK(c)                                                        \
    do {                                                                \
        if(!(c)) {                                                      \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            g_fail = 1;                                                 \
        }                                                               \
    } while(0)

/* pico's pico_create_tensor / pico_param: exactly one PicoTensor */
static struct PicoTensor* pico_style_tensor(void) {
    return (struct PicoTensor*)calloc(1, sizeof(struct PicoTensor));
}

/* pico's arena_init (src/arena.h:38-64): a 16-byte arena and its first block */
static struct Arena* pico_style_arena(size_t bytes) {
    struct Arena* a = (struct Arena*)malloc(sizeof(struct Arena));
    struct ArenaBlock* b = (struct ArenaBlock*)malloc(sizeof(struct ArenaBlock));
    b->bottom = (unsigned char*)malloc(bytes);
    b->curr = b->bottom;
    b->capacity = bytes;
    b->next = NULL;
    a->begin = a->end = b;
    return a;
}

static void pico_style_arena_free(struct Arena* a) {
    free(a->begin->bottom);
    free(a->begin);
    free(a);
}

/* one worker: its own arena on its own context stack, which must stay the
 * current one whatever the other threads do; meanwhile it churns the shared
 * node registry (src/arena.h:155-169 for the stack) */
enum { CTX_THREADS = 8, CTX_SPINS = 2000, CTX_NODES = 256 };
static void* ctx_worker(void* arg) {
    int* ok = (int*)arg;
    *ok = 0;
    if(arena_ctx_current() != NULL) return NULL;  /* a fresh thread's stack is empty */
    struct Arena* mine = arena_init(1 << 12);
    if(!mine) return NULL;
    arena_ctx_push(mine);
    struct PkNode* nodes[CTX_NODES];
    int good = 1;
    for(int i = 0; i < CTX_NODES; i++) {
        nodes[i] = (struct PkNode*)calloc(1, sizeof(struct PkNode));
        good &= pkh_node_register(nodes[i], NULL) == 0;
    }
    for(int i = 0; i < CTX_SPINS; i++) {
        if(arena_ctx_current() != mine) good = 0;
        if(pkh_node(&nodes[i % CTX_NODES]->t) == NULL) good = 0;
        sched_yield();
    }
    for(int i = 0; i < CTX_NODES; i++) {
        pkh_node_unregister(nodes[i]);
        if(pkh_node(&nodes[i]->t) != NULL) good = 0;
        free(nodes[i]);
    }
    arena_ctx_pop();
    if(arena_ctx_current() != NULL) good = 0;
    arena_destroy(mine);
    *ok = good;
    return NULL;
}

static void ctx_threads_test(void) {
    struct Arena* main_arena = arena_init(1 << 12);
    CHECK(main_arena != NULL);
    arena_ctx_push(main_arena);
    pthread_t th[CTX_THREADS];
    int ok[CTX_THREADS];
    for(int i = 0; i < CTX_THREADS; i++) CHECK(pthread_create(&th[i], NULL, ctx_worker, &ok[i]) == 0);
    for(int i = 0; i < CTX_THREADS; i++) CHECK(pthread_join(th[i], NULL) == 0);
    for(int i = 0; i < CTX_THREADS; i++) CHECK(ok[i] == 1);
    CHECK(arena_ctx_current() == main_arena);  /* the workers never touched this stack */
    arena_ctx_pop();
    CHECK(arena_ctx_current() == NULL);
    arena_destroy(main_arena);
}

int main(void) {
    CHECK(sizeof(struct PicoTensor) == 64);
    CHECK(sizeof(struct Arena) == 16);

    /* a foreign tensor of exactly sizeof(struct PicoTensor) bytes */
    struct PicoTensor* ft = pico_style_tensor();
    CHECK(pkh_node(ft) == NULL);
    CHECK(pkh_node(NULL) == NULL);

    /* foreign tensors packed back to back, as in pico's arena blocks; the
     * last one ends exactly at the end of its allocation */
    struct PicoTensor* packed = (struct PicoTensor*)malloc(4 * sizeof(struct PicoTensor));
    memset(packed, 0xAB, 4 * sizeof(struct PicoTensor));
    for(int i = 0; i < 4; i++) CHECK(pkh_node(&packed[i]) == NULL);

    /* this library's nodes: arena nodes are forgotten at reset and destroy */
    struct Arena* own = arena_init(1 << 16);
    CHECK(own != NULL);
    struct PkNode* n1 = (struct PkNode*)arena_alloc(own, sizeof(struct PkNode));
    memset(n1, 0, sizeof(*n1));
    CHECK(pkh_node_register(n1, own) == 0);
    CHECK(pkh_node(&n1->t) == n1);
    CHECK(pkh_node(ft) == NULL);
    void* d1 = arena_alloc_device(own, 1000);
    CHECK(d1 != NULL && ((uintptr_t)d1 % 256) == 0);
    arena_reset(own);
    CHECK(pkh_node(&n1->t) == NULL);
    CHECK(arena_alloc_device(own, 1000) == d1); /* rewound, block kept */
    struct PkNode* n2 = (struct PkNode*)arena_alloc(own, sizeof(struct PkNode));
    memset(n2, 0, sizeof(*n2));
    CHECK(pkh_node_register(n2, own) == 0);
    CHECK(pkh_node(&n2->t) == n2);
    arena_destroy(own);
    CHECK(pkh_node(&n2->t) == NULL);

    /* a param node: registered without an arena, forgotten on unregister */
    struct PkNode* pn = (struct PkNode*)calloc(1, sizeof(struct PkNode));
    CHECK(pkh_node_register(pn, NULL) == 0);
    CHECK(pkh_node(&pn->t) == pn);
    pkh_node_unregister(pn);
    CHECK(pkh_node(&pn->t) == NULL);
    free(pn);

    /* an arena pico allocated itself (16 bytes) through the device calls */
    struct Arena* fa = pico_style_arena(1 << 12);
    unsigned char* p1 = (unsigned char*)arena_alloc_device(fa, 1000);
    unsigned char* p2 = (unsigned char*)arena_alloc_device(fa, 24);
    CHECK(p1 && p2 && p2 == p1 + 1024);
    memset(p1, 1, 1000); /* the memory is usable as the sizes say */
    unsigned char* big = (unsigned char*)arena_alloc_device(fa, (size_t)3 << 20);
    CHECK(big != NULL);
    memset(big, 2, (size_t)3 << 20);
    arena_device_reset(fa);
    CHECK(arena_alloc_device(fa, 1000) == p1);
    arena_device_release(fa);
    arena_device_release(fa); /* a second release is a no-op */
    CHECK(fa->begin != NULL && fa->begin == fa->end); /* pico's fields untouched */
    pico_style_arena_free(fa);

    /* the hash set under many inserts and deletions in mixed order */
    enum { N = 50000 };
    struct PkNode** many = (struct PkNode**)malloc(N * sizeof(*many));
    for(int i = 0; i < N; i++) {
        many[i] = (struct PkNode*)calloc(1, sizeof(struct PkNode));
        CHECK(pkh_node_register(many[i], NULL) == 0);
    }
    for(int i = 0; i < N; i += 2) pkh_node_unregister(many[(i * 7919) % N]);
    /* 7919 is invertible mod N, so j -> (j * 7919) % N visits every index
     * once: exactly the even j's nodes are gone */
    int found = 0;
    for(int i = 0; i < N; i++) found += pkh_node(&many[i]->t) != NULL;
    CHECK(found == N / 2);
    for(int j = 0; j < N; j += 2) CHECK(pkh_node(&many[(j * 7919) % N]->t) == NULL);
    for(int j = 1; j < N; j += 2) CHECK(pkh_node(&many[(j * 7919) % N]->t) != NULL);
    for(int i = 0; i < N; i++) {
        pkh_node_unregister(many[i]);
        free(many[i]);
    }
    free(many);
    ctx_threads_test();
    pkh_registry_clear();

    free(ft);
    free(packed);
    if(g_fail) return 1;
    printf("registry host test ok\n");
    return 0;
}
