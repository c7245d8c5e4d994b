/*
 * pico_amd/host/tensor.c -- arenas, GPU tensor creation, the backward walk,
 * seeded generators and host<->device copies for libpico_amd.so.
 *
 * Follows the reference's contracts (docs/contracts/01-allocation-and-
 * ownership.md): params are persistent and freed by pico_free; everything
 * else lives in the current arena until arena_reset / arena_destroy.  Struct
 * metadata stays in the arena's host blocks, tensor data goes to its device
 * twin (arena.c).  Every node made here is registered (pkh_node_register),
 * which is how pkh_node tells this library's tensors from pico's own.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

#define DEV_ALIGN 256

/* ---------------------------------------------------------------- tensors */
static int64_t numel_of(const int64_t* shape, int ndim) {
    int64_t n = 1;
    for(int i = 0; i < ndim; i++) n *= shape[i];
    return n;
}

static void contig_strides(const int64_t* shape, int ndim, int64_t* st) {
    int64_t s = 1;
    for(int i = ndim - 1; i >= 0; i--) {
        st[i] = s;
        s *= shape[i];
    }
}

int pkh_is_gpu(const struct PicoTensor* t) { return t && t->backend == GPU; }

struct PicoTensor* pkh_new_tensor(struct Arena* a, const int64_t* shape, int ndim) {
    if(pkh_init()) return NULL;
    if(ndim < 1 || ndim > 255) {
        PKH_ERR("tensor rank %d not supported\n", ndim);
        return NULL;
    }
    struct PkNode* n = (struct PkNode*)arena_alloc(a, sizeof(struct PkNode));
    memset(n, 0, sizeof(*n));
    if(pkh_node_register(n, a)) return NULL;
    struct PicoTensor* t = &n->t;
    t->ndim = (uint8_t)ndim;
    t->shape = (int64_t*)arena_alloc(a, sizeof(int64_t) * ndim);
    t->strides = (int64_t*)arena_alloc(a, sizeof(int64_t) * ndim);
    memcpy(t->shape, shape, sizeof(int64_t) * ndim);
    contig_strides(t->shape, ndim, t->strides);
    t->numel = numel_of(shape, ndim);
    t->backend = GPU;
    t->data = (float*)arena_alloc_device(a, sizeof(float) * (size_t)t->numel);
    t->grad = (float*)arena_alloc_device(a, sizeof(float) * (size_t)t->numel);
    if(!t->data || !t->grad) return NULL;
    return t;
}

/* src/tensor.c:86-134: data zeroed (a fill kernel), grad lazily zero */
struct PicoTensor* pico_create_tensor(struct Arena* arena, int64_t* shape, uint8_t ndim) {
    if(!arena) {
        PKH_ERR("No current arena in context!\n");
        return NULL;
    }
    struct PicoTensor* t = pkh_new_tensor(arena, shape, ndim);
    if(!t) return NULL;
    if(pkh_status("pico_create_tensor", pk_fill_f32(t->numel, 0.0f, t->data, pkh_stream())))
        return NULL;
    return t;
}

/* src/tensor.c:44-84: persistent, zeroed; data and grad share one allocation */
struct PicoTensor* pico_param(int64_t* shape, uint8_t ndim) {
    if(pkh_init()) return NULL;
    pkh_params_changed(); /* a new parameter may take a freed one's address */
    if(ndim < 1) {
        PKH_ERR("pico_param needs ndim >= 1\n");
        return NULL;
    }
    struct PkNode* n = (struct PkNode*)calloc(1, sizeof(struct PkNode));
    if(!n) {
        printf("Memory allocation failed!\n");
        return NULL;
    }
    struct PicoTensor* t = &n->t;
    t->ndim = ndim;
    t->is_persistent = 1;
    t->backend = GPU;
    t->shape = (int64_t*)calloc(ndim, sizeof(int64_t));
    t->strides = (int64_t*)calloc(ndim, sizeof(int64_t));
    if(!t->shape || !t->strides) {
        free(t->shape);
        free(t->strides);
        free(n);
        return NULL;
    }
    memcpy(t->shape, shape, sizeof(int64_t) * ndim);
    contig_strides(t->shape, ndim, t->strides);
    t->numel = numel_of(shape, ndim);
    size_t half = ((size_t)t->numel * sizeof(float) + DEV_ALIGN - 1) & ~(size_t)(DEV_ALIGN - 1);
    if(half == 0) half = DEV_ALIGN;
    unsigned char* base = (unsigned char*)pkh_device_alloc(2 * half);
    if(!base) {
        free(t->shape);
        free(t->strides);
        free(n);
        return NULL;
    }
    t->data = (float*)base;
    t->grad = (float*)(base + half);
    if(pkh_status("pico_param", pk_fill_f32(t->numel, 0.0f, t->data, pkh_stream())) ||
       pkh_node_register(n, NULL)) {
        pkh_device_free(base);
        free(t->shape);
        free(t->strides);
        free(n);
        return NULL;
    }
    return t;
}

/* src/tensor.c:136-168 */
void pico_free(struct PicoTensor* t) {
    if(!t || t->is_persistent == 0) return;
    pkh_params_changed();
    struct PkNode* n = pkh_node(t);
    if(!n) {
        PKH_ERR("pico_free: not a tensor of this library!\n");
        return;
    }
    pkh_node_unregister(n);
    pkh_sync();
    free(t->shape);
    free(t->strides);
    pkh_device_free(t->data); /* data and grad are one allocation */
    free(t->parents);
    free(t);
}

/* src/tensor.c:173-188 */
struct PicoTensor* pico_tensor_from_scalar(float value) {
    struct Arena* a = pkh_need_arena();
    if(!a) return NULL;
    int64_t shape[1] = {1};
    struct PicoTensor* t = pkh_new_tensor(a, shape, 1);
    if(!t) return NULL;
    if(pkh_status("pico_tensor_from_scalar", pk_fill_f32(1, value, t->data, pkh_stream())))
        return NULL;
    return t;
}

/* src/tensor.c:230-244 */
void pico_transpose_2d(struct PicoTensor* t) {
    if(t->ndim != 2) {
        fprintf(stderr, "Error: This is not a rank 2 tensor!\n");
        return;
    }
    int64_t c = t->shape[1];
    t->shape[1] = t->shape[0];
    t->shape[0] = c;
    int64_t sc = t->strides[1];
    t->strides[1] = t->strides[0];
    t->strides[0] = sc;
}

/* src/tensor.c:371-397 */
uint8_t pico_check_broadcast_compatibility(struct PicoTensor* a, struct PicoTensor* b) {
    for(int i = a->ndim - 1, j = b->ndim - 1; i >= 0 && j >= 0; i--, j--) {
        int64_t da = a->shape[i], db = b->shape[j];
        if(da != db && da != 1 && db != 1) return 0;
    }
    return 1;
}

void pkh_set_parents(struct Arena* a, struct PicoTensor* out, int n, struct PicoTensor* const* ps,
                     void (*bw)(struct PicoTensor*)) {
    out->parents = (struct PicoTensor**)arena_alloc(a, sizeof(struct PicoTensor*) * n);
    for(int i = 0; i < n; i++) out->parents[i] = ps[i];
    out->num_parents = (uint8_t)n;
    out->_backward = bw;
}

const float* pkh_upstream(struct PicoTensor* self) {
    return pkh_grad_is_live(self) ? self->grad : NULL;
}

/* ---------------------------------------------------------- grad aliases */
int pkh_grad_alias(struct PicoTensor* t, const struct PicoTensor* src) {
    struct PkNode* n = pkh_node(t);
    struct PkNode* sn = pkh_node(src);
    if(!n || !sn || t == src || t->is_persistent || n->base || n->n_views || n->own_grad ||
       sn->base || t->numel != src->numel || !pkh_grad_is_live(src) || pkh_node_live(n))
        return 0;
    pkh_grad_on_main(n);
    n->own_grad = t->grad;
    t->grad = src->grad;
    n->grad_live = 1;
    return 1;
}

void pkh_grad_unalias(struct PkNode* n, int copy) {
    if(!n->own_grad) return;
    float* own = n->own_grad;
    /* a failed copy is reported (the error is recorded); the tensor gets its
     * own buffer back either way, so no later write reaches the shared grad */
    if(copy) pkh_copy_d2d_async(own, n->t.grad, sizeof(float) * (size_t)n->t.numel);
    n->t.grad = own;
    n->own_grad = NULL;
}

/* ------------------------------------------------------ column-block views */
void pkh_grad_complete(struct PkNode* n) {
    int any = 0;
    for(uint32_t i = 0; i < n->n_views; i++) any |= pkh_node(n->views[i])->grad_live != 0;
    if(!any) return; /* nothing written: the grad stays empty */
    for(uint32_t i = 0; i < n->n_views; i++) {
        struct PicoTensor* v = n->views[i];
        struct PkNode* vn = pkh_node(v);
        if(vn->grad_live) continue;
        if(pkh_status("pico_split_cols (zero grad)",
                      pk_fill2d_f32(v->shape[0], v->shape[1], 0.0f, v->grad, v->strides[0],
                                    pkh_stream())))
            return;
        vn->grad_live = 1;
    }
    n->grad_live = 1;
}

/* no reference counterpart (the reference's only view is pico_transpose_2d):
 * views share t's data and grad, so nothing is copied either way */
int pico_split_cols(struct PicoTensor* t, int n, struct PicoTensor** outs) {
    struct PkNode* tn = pkh_node(t);
    if(!t || !tn || !pkh_is_gpu(t) || !outs || n < 1) {
        PKH_ERR("pico_split_cols: expects a GPU tensor of this library and n >= 1!\n");
        return PK_EINVAL;
    }
    if(t->ndim != 2 || t->strides[1] != 1 || t->strides[0] != t->shape[1] ||
       t->shape[1] % n || tn->base || tn->n_views || t->is_persistent) {
        PKH_ERR("pico_split_cols: expects a contiguous, unsplit, non-parameter [M, n*C] tensor!\n");
        return PK_EINVAL;
    }
    struct Arena* a = pkh_need_arena();
    if(!a) return PK_EINVAL;
    const int64_t M = t->shape[0], C = t->shape[1] / n;
    struct PicoTensor** vs = (struct PicoTensor**)arena_alloc(a, sizeof(*vs) * (size_t)n);
    if(!vs) return PK_EINVAL;
    for(int i = 0; i < n; i++) {
        struct PkNode* vn = (struct PkNode*)arena_alloc(a, sizeof(struct PkNode));
        int64_t* shape = (int64_t*)arena_alloc(a, sizeof(int64_t) * 2);
        int64_t* strides = (int64_t*)arena_alloc(a, sizeof(int64_t) * 2);
        if(!vn || !shape || !strides) return PK_EINVAL;
        memset(vn, 0, sizeof(*vn));
        if(pkh_node_register(vn, a)) return PK_EINVAL;
        vn->base = t;
        struct PicoTensor* v = &vn->t;
        shape[0] = M;
        shape[1] = C;
        strides[0] = t->shape[1];
        strides[1] = 1;
        v->shape = shape;
        v->strides = strides;
        v->ndim = 2;
        v->numel = M * C;
        v->backend = GPU;
        v->data = t->data + i * C;
        v->grad = t->grad + i * C;
        pkh_set_parents(a, v, 1, &t, NULL);
        vs[i] = v;
    }
    tn->views = vs;
    tn->n_views = (uint32_t)n;
    for(int i = 0; i < n; i++) outs[i] = vs[i];
    return 0;
}

/* ------------------------------------------------------------ pico_rand/n */
static inline uint32_t xorshift32(void) {
    uint32_t x = x_state;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return x_state = x;
}

static inline float unit_from_bits(uint32_t r) {
    uint32_t bits = (r >> 9) | 0x3F800000u; /* [1, 2) */
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f - 1.0f;
}

static struct PicoTensor* tensor_from_host_values(struct Arena* a, const int64_t* shape, int ndim,
                                                  float* host) {
    struct PicoTensor* t = pkh_new_tensor(a, shape, ndim);
    if(!t) return NULL;
    if(pkh_copy_h2d(t->data, host, sizeof(float) * (size_t)t->numel)) return NULL;
    return t;
}

/* src/tensor.c:249-273: the same xorshift32 stream and bit construction */
struct PicoTensor* pico_rand(struct Arena* arena, int64_t* shape, uint8_t ndim) {
    int64_t n = numel_of(shape, ndim);
    float* h = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    if(!h) return NULL;
    for(int64_t i = 0; i < n; i++) h[i] = unit_from_bits(xorshift32());
    struct PicoTensor* t = tensor_from_host_values(arena, shape, ndim, h);
    free(h);
    return t;
}

struct PicoTensor* pico_randn(struct Arena* arena, int64_t* shape, uint8_t ndim) {
    int64_t n = numel_of(shape, ndim);
    float* h = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    if(!h) return NULL;
    const double two_pi = 6.283185307179586;
    for(int64_t i = 0; i < n; i += 2) {
        double u1 = 1.0 - (double)unit_from_bits(xorshift32()); /* (0, 1] */
        double u2 = (double)unit_from_bits(xorshift32());
        double r = sqrt(-2.0 * log(u1));
        h[i] = (float)(r * cos(two_pi * u2));
        if(i + 1 < n) h[i + 1] = (float)(r * sin(two_pi * u2));
    }
    struct PicoTensor* t = tensor_from_host_values(arena, shape, ndim, h);
    free(h);
    return t;
}

/* ------------------------------------------------------------- backward */
static uint64_t g_visit_epoch = 0;

struct NodeVec {
    struct PicoTensor** v;
    int64_t n, cap;
};
static int nv_push(struct NodeVec* l, struct PicoTensor* t) {
    if(l->n == l->cap) {
        int64_t cap = l->cap ? 2 * l->cap : 64;
        struct PicoTensor** nv = (struct PicoTensor**)realloc(l->v, sizeof(*nv) * cap);
        if(!nv) return -1;
        l->v = nv;
        l->cap = cap;
    }
    l->v[l->n++] = t;
    return 0;
}

/* src/tensor.c:15-42, 399-415.  The same post-order as the reference's
 * recursive DFS (mark on entry, parents in order, append after them), walked
 * with an explicit stack and an epoch mark per node instead of a linear
 * visited scan. */
void pico_backward(struct Arena* arena, struct PicoTensor* entry) {
    (void)arena;
    if(!entry) return;
    if(!pkh_node(entry) || !pkh_is_gpu(entry)) {
        PKH_ERR("pico_backward: entry is not a GPU tensor of this library!\n");
        return;
    }
    uint64_t epoch = ++g_visit_epoch;
    struct NodeVec order = {0}, stack = {0};
    int64_t* next = NULL;
    int64_t next_cap = 0;
    pkh_node(entry)->visit = epoch;
    nv_push(&stack, entry);
    next_cap = 64;
    next = (int64_t*)calloc(next_cap, sizeof(int64_t));
    while(stack.n > 0) {
        struct PicoTensor* top = stack.v[stack.n - 1];
        int64_t* idx = &next[stack.n - 1];
        if(*idx < top->num_parents) {
            struct PicoTensor* p = top->parents[(*idx)++];
            if(!p) continue;
            struct PkNode* pn = pkh_node(p);
            if(!pn) {
                PKH_ERR("pico_backward: graph holds a tensor this library did not make!\n");
                goto done;
            }
            if(pn->visit == epoch) continue;
            pn->visit = epoch;
            if(stack.n == next_cap) {
                next_cap *= 2;
                next = (int64_t*)realloc(next, sizeof(int64_t) * next_cap);
            }
            next[stack.n] = 0;
            nv_push(&stack, p);
        } else {
            stack.n--;
            nv_push(&order, top);
        }
    }
    /* a graph run a second time: its aliased grads get their own buffers
     * back before anything accumulates into them */
    for(int64_t i = 0; i < order.n; i++) pkh_grad_unalias(pkh_node(order.v[i]), 1);
    /* seed dL/dentry = 1 over every element (tensor.c:27-30) */
    if(pkh_status("pico_backward", pk_fill_f32(entry->numel, 1.0f, entry->grad, pkh_stream())))
        goto done;
    pkh_grad_mark(entry);
    pkh_node(entry)->seed_one = 1;
    /* a hook that fails records an error and leaves its parents' grads
     * unwritten: stop there rather than propagate from partial grads */
    const uint64_t errors = pkh_error_count();
    for(int64_t i = order.n - 1; i >= 0; i--) {
        struct PicoTensor* t = order.v[i];
        if(t->_backward) t->_backward(t);
        if(pkh_error_count() != errors) {
            PKH_ERR("pico_backward: stopped at a failed backward hook (%s)\n", pico_gpu_last_error());
            break;
        }
    }
    pkh_side_join(); /* weight gradients computed on the side stream are in */
    pkh_node(entry)->seed_one = 0;
done:
    free(order.v);
    free(stack.v);
    free(next);
}

/* ----------------------------------------------------------------- copies */
int pico_tensor_copy_from_host(struct PicoTensor* t, const float* src) {
    if(!t || !pkh_is_gpu(t)) return PK_EINVAL;
    return pkh_copy_h2d(t->data, src, sizeof(float) * (size_t)t->numel);
}

int pico_tensor_copy_to_host(const struct PicoTensor* t, float* dst) {
    if(!t || !pkh_is_gpu(t)) return PK_EINVAL;
    return pkh_copy_d2h(dst, t->data, sizeof(float) * (size_t)t->numel);
}

int pico_tensor_grad_to_host(const struct PicoTensor* t, float* dst) {
    if(!t || !pkh_is_gpu(t)) return PK_EINVAL;
    if(!pkh_grad_is_live(t)) {
        memset(dst, 0, sizeof(float) * (size_t)t->numel);
        return 0;
    }
    return pkh_copy_d2h(dst, t->grad, sizeof(float) * (size_t)t->numel);
}

int pico_tensor_grad_from_host(struct PicoTensor* t, const float* src) {
    if(!t || !pkh_is_gpu(t)) return PK_EINVAL;
    pkh_grad_unalias(pkh_node(t), 0);
    int rc = pkh_copy_h2d(t->grad, src, sizeof(float) * (size_t)t->numel);
    if(rc == 0) pkh_grad_mark(t);
    return rc;
}

int32_t* pico_ids_to_device(const int32_t* host_ids, int64_t n) {
    struct Arena* a = pkh_need_arena();
    if(!a || n < 0) return NULL;
    int32_t* d = (int32_t*)arena_alloc_device(a, sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
    if(!d) return NULL;
    if(n > 0 && pkh_copy_h2d(d, host_ids, sizeof(int32_t) * (size_t)n)) return NULL;
    return d;
}

int pico_ids_update(int32_t* device_ids, const int32_t* host_ids, int64_t n) {
    if(n < 0 || (n > 0 && (!device_ids || !host_ids))) {
        pkh_set_error("pico_ids_update: bad arguments");
        return PK_EINVAL;
    }
    return pkh_copy_h2d(device_ids, host_ids, sizeof(int32_t) * (size_t)n);
}

const int32_t* pkh_ids_on_device(const int32_t* ids, int64_t n) {
    if(!ids) return NULL;
    if(pkh_is_device_ptr(ids)) return ids;
    return pico_ids_to_device(ids, n);
}

/* src/tensor.c:190-228, reading the device data back first */
static void print_rec(const struct PicoTensor* t, const float* h, int dim, int64_t off) {
    if(dim == t->ndim - 1) {
        printf("[");
        for(int64_t i = 0; i < t->shape[dim]; i++) {
            printf("%g", h[off + i * t->strides[dim]]);
            if(i != t->shape[dim] - 1) printf(", ");
        }
        printf("]");
        return;
    }
    printf("[");
    for(int64_t i = 0; i < t->shape[dim]; i++) {
        print_rec(t, h, dim + 1, off + i * t->strides[dim]);
        if(i != t->shape[dim] - 1) printf(",\n ");
    }
    printf("]");
}

void pico_tensor_print(struct PicoTensor* t) {
    if(!t) {
        printf("PicoTensor(NULL)\n");
        return;
    }
    printf("PicoTensor(shape=[");
    for(int i = 0; i < t->ndim; i++) {
        printf("%ld", (long)t->shape[i]);
        if(i != t->ndim - 1) printf(", ");
    }
    printf("], numel=%ld)\n", (long)t->numel);
    if(t->ndim == 0 || !t->data) {
        printf("(no data)\n");
        return;
    }
    float* h = (float*)malloc(sizeof(float) * (size_t)(t->numel > 0 ? t->numel : 1));
    if(!h || pico_tensor_copy_to_host(t, h)) {
        free(h);
        printf("(device read failed)\n");
        return;
    }
    print_rec(t, h, 0, 0);
    printf("\n");
    free(h);
}
