/*
 * pico_amd/host/arena.c -- arenas, their device twins, and the registry of
 * tensor nodes this library made.  Host code only: device memory comes from
 * pkh_device_alloc / pkh_device_free, so this file also builds and runs on a
 * machine without a GPU (the CPU sanitizer test links it against host stubs).
 *
 * struct Arena keeps pico's two-pointer layout (src/arena.h:27-29).  What this
 * library adds to an arena -- its device blocks and the list of nodes made in
 * it -- lives in a side table keyed by the arena's address, never inside the
 * struct, so an arena that pico itself allocated (16 bytes) can be handed to
 * arena_alloc_device without anything being read or written past its end.
 *
 * Likewise a PicoTensor is recognised as one of this library's nodes by a
 * lookup of its address in a hash set, never by reading fields beyond
 * sizeof(struct PicoTensor): pico's tensors are exactly that size, calloc'd or
 * packed back to back in its arena blocks (src/tensor.c:44-134).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

#define DEV_ALIGN 256
#define HOST_ALIGN 16
#define MAX_ARENA_STACK 16

/* ------------------------------------------------------- pointer hash map */
/* Open addressing with linear probing and backward-shift deletion (no
 * tombstones), keys are addresses (never NULL), load factor <= 1/2. */
struct PtrMap {
    uintptr_t* keys;
    void** vals;
    size_t cap; /* power of two, or 0 */
    size_t n;
};

static size_t ptr_hash(uintptr_t k, size_t mask) {
    uint64_t x = (uint64_t)k;
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33;
    return (size_t)x & mask;
}

static int map_grow(struct PtrMap* m) {
    size_t cap = m->cap ? 2 * m->cap : 1024;
    uintptr_t* keys = (uintptr_t*)calloc(cap, sizeof(uintptr_t));
    void** vals = (void**)calloc(cap, sizeof(void*));
    if(!keys || !vals) {
        free(keys);
        free(vals);
        return -1;
    }
    for(size_t i = 0; i < m->cap; i++) {
        if(!m->keys[i]) continue;
        size_t j = ptr_hash(m->keys[i], cap - 1);
        while(keys[j]) j = (j + 1) & (cap - 1);
        keys[j] = m->keys[i];
        vals[j] = m->vals[i];
    }
    free(m->keys);
    free(m->vals);
    m->keys = keys;
    m->vals = vals;
    m->cap = cap;
    return 0;
}

static int map_put(struct PtrMap* m, const void* key, void* val) {
    if(2 * (m->n + 1) > m->cap && map_grow(m)) return -1;
    const uintptr_t k = (uintptr_t)key;
    size_t j = ptr_hash(k, m->cap - 1);
    while(m->keys[j] && m->keys[j] != k) j = (j + 1) & (m->cap - 1);
    if(!m->keys[j]) m->n++;
    m->keys[j] = k;
    m->vals[j] = val;
    return 0;
}

/* returns the slot of key, or -1 */
static long map_find(const struct PtrMap* m, const void* key) {
    if(!m->cap || !key) return -1;
    const uintptr_t k = (uintptr_t)key;
    size_t j = ptr_hash(k, m->cap - 1);
    while(m->keys[j]) {
        if(m->keys[j] == k) return (long)j;
        j = (j + 1) & (m->cap - 1);
    }
    return -1;
}

static void map_del(struct PtrMap* m, const void* key) {
    long s = map_find(m, key);
    if(s < 0) return;
    const size_t mask = m->cap - 1;
    size_t i = (size_t)s;
    m->keys[i] = 0;
    m->vals[i] = NULL;
    m->n--;
    /* shift back the entries of the probe run that follows the hole */
    for(size_t j = (i + 1) & mask; m->keys[j]; j = (j + 1) & mask) {
        size_t home = ptr_hash(m->keys[j], mask);
        /* the entry at j may move to the hole at i when its home slot does
         * not lie cyclically in (i, j] */
        int stays = (i <= j) ? (home > i && home <= j) : (home > i || home <= j);
        if(stays) continue;
        m->keys[i] = m->keys[j];
        m->vals[i] = m->vals[j];
        m->keys[j] = 0;
        m->vals[j] = NULL;
        i = j;
    }
}

static void map_free(struct PtrMap* m) {
    free(m->keys);
    free(m->vals);
    memset(m, 0, sizeof(*m));
}

/* ------------------------------------------------ arena side-table entries */
struct PicoDeviceBlock {
    struct PicoDeviceBlock* next;
    size_t capacity;
    size_t used;
    unsigned char* bottom; /* device memory */
};

struct PkArenaState {
    struct PicoDeviceBlock *dev_begin, *dev_end;
    size_t dev_block_bytes;
    struct PkNode** nodes; /* nodes made in this arena, unregistered at reset */
    size_t n_nodes, cap_nodes;
};

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static struct PtrMap g_nodes;  /* node address -> its arena's state (NULL: a param) */
static struct PtrMap g_arenas; /* arena address -> struct PkArenaState* */

/* the state of arena a (created for an arena this library has not seen: one
 * pico allocated itself); caller holds g_lock */
static struct PkArenaState* arena_state_locked(struct Arena* a, int create) {
    long s = map_find(&g_arenas, a);
    if(s >= 0) return (struct PkArenaState*)g_arenas.vals[s];
    if(!create) return NULL;
    struct PkArenaState* st = (struct PkArenaState*)calloc(1, sizeof(*st));
    if(!st) return NULL;
    /* pico sizes an arena by its first block (src/arena.h:38-64); the device
     * blocks of a foreign arena follow that size, at least 1 MiB.  Reading
     * begin->capacity stays inside pico's ArenaBlock (same layout as here). */
    size_t cap = a->begin ? a->begin->capacity : 0;
    st->dev_block_bytes = cap < ((size_t)1 << 20) ? ((size_t)1 << 20) : cap;
    if(map_put(&g_arenas, a, st)) {
        free(st);
        return NULL;
    }
    return st;
}

/* unregisters the nodes made in st's arena; caller holds g_lock */
static void forget_nodes_locked(struct PkArenaState* st) {
    for(size_t i = 0; i < st->n_nodes; i++) map_del(&g_nodes, st->nodes[i]);
    st->n_nodes = 0;
}

/* ----------------------------------------------------------- node registry */
int pkh_node_register(struct PkNode* n, struct Arena* a) {
    pthread_mutex_lock(&g_lock);
    struct PkArenaState* st = a ? arena_state_locked(a, 1) : NULL;
    int rc = (a && !st) ? -1 : 0;
    if(!rc && st && st->n_nodes == st->cap_nodes) {
        size_t cap = st->cap_nodes ? 2 * st->cap_nodes : 256;
        struct PkNode** v = (struct PkNode**)realloc(st->nodes, cap * sizeof(*v));
        if(v) {
            st->nodes = v;
            st->cap_nodes = cap;
        } else {
            rc = -1;
        }
    }
    if(!rc) rc = map_put(&g_nodes, n, st);
    if(!rc && st) st->nodes[st->n_nodes++] = n;
    pthread_mutex_unlock(&g_lock);
    if(rc) PKH_ERR("out of host memory registering a tensor!\n");
    return rc;
}

void pkh_node_unregister(const struct PkNode* n) {
    pthread_mutex_lock(&g_lock);
    map_del(&g_nodes, n);
    pthread_mutex_unlock(&g_lock);
}

struct PkNode* pkh_node(const struct PicoTensor* t) {
    if(!t) return NULL;
    pthread_mutex_lock(&g_lock);
    long s = map_find(&g_nodes, t);
    pthread_mutex_unlock(&g_lock);
    return s >= 0 ? (struct PkNode*)t : NULL;
}

/* ------------------------------------------------------------------ arena */
static _Thread_local struct Arena* g_arena_stack[MAX_ARENA_STACK];
static _Thread_local int g_arena_top = -1;

static struct ArenaBlock* host_block_new(size_t bytes) {
    struct ArenaBlock* b = (struct ArenaBlock*)malloc(sizeof(*b));
    if(!b) return NULL;
    b->bottom = (unsigned char*)malloc(bytes);
    if(!b->bottom) {
        free(b);
        return NULL;
    }
    b->curr = b->bottom;
    b->capacity = bytes;
    b->next = NULL;
    return b;
}

/* src/arena.h:38-64.  `bytes` sizes both the first host block and each device
 * block; host blocks hold only structs, shapes and parent lists, so they are
 * capped at 4 MiB and grow on demand. */
struct Arena* arena_init(size_t bytes) {
    struct Arena* a = (struct Arena*)calloc(1, sizeof(*a));
    if(!a) return NULL;
    size_t hb = bytes < ((size_t)4 << 20) ? bytes : ((size_t)4 << 20);
    if(hb < 4096) hb = 4096;
    a->begin = host_block_new(hb);
    if(!a->begin) {
        free(a);
        return NULL;
    }
    a->end = a->begin;
    pthread_mutex_lock(&g_lock);
    struct PkArenaState* st = arena_state_locked(a, 1);
    if(st) st->dev_block_bytes = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    pthread_mutex_unlock(&g_lock);
    if(!st) {
        free(a->begin->bottom);
        free(a->begin);
        free(a);
        return NULL;
    }
    return a;
}

/* src/arena.h:105-116; a request larger than the block size gets a block of
 * its own size instead of failing */
void* arena_alloc(struct Arena* a, size_t size) {
    size = (size + HOST_ALIGN - 1) & ~(size_t)(HOST_ALIGN - 1);
    struct ArenaBlock* b = a->end;
    if((size_t)(b->curr - b->bottom) + size > b->capacity) {
        size_t cap = a->begin->capacity > size ? a->begin->capacity : size;
        struct ArenaBlock* nb = host_block_new(cap);
        if(!nb) {
            printf("Memory allocation failed!\n");
            exit(1);
        }
        b->next = nb;
        a->end = nb;
        b = nb;
    }
    void* p = b->curr;
    b->curr += size;
    return p;
}

void* arena_alloc_device(struct Arena* a, size_t size) {
    if(!a) return NULL;
    size = (size + DEV_ALIGN - 1) & ~(size_t)(DEV_ALIGN - 1);
    if(size == 0) size = DEV_ALIGN;
    pthread_mutex_lock(&g_lock);
    struct PkArenaState* st = arena_state_locked(a, 1);
    pthread_mutex_unlock(&g_lock);
    if(!st) return NULL;
    /* the state of one arena is touched only by the thread using it (pico's
     * ops are single-threaded per arena, src/arena.h:31-36) */
    struct PicoDeviceBlock* b = st->dev_end;
    while(b && b->used + size > b->capacity) b = b->next;
    if(!b) {
        size_t cap = st->dev_block_bytes > size ? st->dev_block_bytes : size;
        struct PicoDeviceBlock* nb = (struct PicoDeviceBlock*)calloc(1, sizeof(*nb));
        if(!nb) return NULL;
        nb->bottom = (unsigned char*)pkh_device_alloc(cap);
        if(!nb->bottom) {
            free(nb);
            PKH_ERR("arena: device memory exhausted (%zu bytes requested)\n", size);
            return NULL;
        }
        nb->capacity = cap;
        if(!st->dev_begin) {
            st->dev_begin = nb;
        } else {
            struct PicoDeviceBlock* last = st->dev_begin;
            while(last->next) last = last->next;
            last->next = nb;
        }
        b = nb;
    }
    st->dev_end = b;
    void* p = b->bottom + b->used;
    b->used += size;
    return p;
}

/* rewinds a's device blocks and forgets the nodes made in it; the blocks are
 * kept, so a training loop allocates device memory only in its first step */
void arena_device_reset(struct Arena* a) {
    if(!a) return;
    pthread_mutex_lock(&g_lock);
    struct PkArenaState* st = arena_state_locked(a, 0);
    if(st) {
        forget_nodes_locked(st);
        for(struct PicoDeviceBlock* d = st->dev_begin; d; d = d->next) d->used = 0;
        st->dev_end = st->dev_begin;
    }
    pthread_mutex_unlock(&g_lock);
}

/* frees a's device blocks and its side-table entry (the arena struct and its
 * host blocks stay with whoever allocated them) */
void arena_device_release(struct Arena* a) {
    if(!a) return;
    pthread_mutex_lock(&g_lock);
    struct PkArenaState* st = arena_state_locked(a, 0);
    if(st) {
        forget_nodes_locked(st);
        map_del(&g_arenas, a);
    }
    pthread_mutex_unlock(&g_lock);
    if(!st) return;
    if(st->dev_begin) pkh_sync();
    struct PicoDeviceBlock* d = st->dev_begin;
    while(d) {
        struct PicoDeviceBlock* n = d->next;
        pkh_device_free(d->bottom);
        free(d);
        d = n;
    }
    free(st->nodes);
    free(st);
}

/* src/arena.h:123-136: the host side frees its extra blocks as pico does; the
 * device twin is rewound (arena_device_reset) */
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
    arena_device_reset(a);
}

void arena_destroy(struct Arena* a) {
    if(!a) return;
    arena_device_release(a);
    struct ArenaBlock* c = a->begin;
    while(c) {
        struct ArenaBlock* n = c->next;
        free(c->bottom);
        free(c);
        c = n;
    }
    free(a);
}

/* src/arena.h:155-169 */
void arena_ctx_push(struct Arena* a) {
    if(g_arena_top + 1 >= MAX_ARENA_STACK) {
        PKH_ERR("arena context stack overflow (max %d)\n", MAX_ARENA_STACK);
        return;
    }
    g_arena_stack[++g_arena_top] = a;
}
void arena_ctx_pop(void) {
    if(g_arena_top >= 0) g_arena_top--;
}
struct Arena* arena_ctx_current(void) {
    if(g_arena_top < 0 || g_arena_top >= MAX_ARENA_STACK) return NULL;
    return g_arena_stack[g_arena_top];
}

struct Arena* pkh_need_arena(void) {
    struct Arena* a = arena_ctx_current();
    if(!a) PKH_ERR("No current arena in context!\n");
    return a;
}

/* drops every side-table entry (pico_shutdown after all arenas are gone) */
void pkh_registry_clear(void) {
    pthread_mutex_lock(&g_lock);
    if(g_arenas.n == 0) map_free(&g_arenas);
    if(g_nodes.n == 0) map_free(&g_nodes);
    pthread_mutex_unlock(&g_lock);
}
