/*
 * pico_amd/host/pk_host.h -- internals shared by the C11 host side of the
 * MI355X backend (libpico_amd.so): the node that carries every tensor this
 * library makes, lazy-grad bookkeeping, error reporting, device workspace.
 */
#pragma once

#include <stdint.h>
#include <stdio.h>

#include "pico_amd.h"
#include "pico_hip.h"

/* everything declared below is internal to libpico_amd.so */
#pragma GCC visibility push(hidden)

#define PKH_MAX_SAVED 4

/* Every tensor made by this library is the first member of a node.  The node
 * adds what pico's struct has no room for: whether the grad buffer holds
 * values yet (lazy zeroing), a traversal mark for pico_backward, and the
 * state an op's backward needs (saved device buffers and sizes). */
struct PkNode {
    struct PicoTensor t;
    uint32_t grad_live;
    uint64_t visit;
    uint32_t seed_one; /* this node is the entry pico_backward seeded with 1 */
    uint32_t n_views;  /* column-block views made of this tensor (pico_split_cols) */
    uint64_t side_seq; /* the side-stream fork that last wrote this grad (0: none) */
    struct PicoTensor* base;    /* a view: the tensor whose data and grad it shares */
    struct PicoTensor** views;  /* a split tensor: its views */
    float* own_grad; /* non-NULL: grad points at another tensor's final grad (an alias),
                      * this is the tensor's own buffer */
    void* saved[PKH_MAX_SAVED];
    int64_t ival[PKH_MAX_SAVED];
    float fval[PKH_MAX_SAVED];
};

/* Node registry (arena.c).  pkh_node(t) is t's node when this library made t,
 * else NULL; it looks t's address up in a hash set and reads nothing of *t,
 * so a tensor pico allocated itself (exactly sizeof(struct PicoTensor) bytes)
 * is safe to pass.  Nodes made in an arena are registered with it and
 * forgotten at arena_reset / arena_destroy; params (arena NULL) at pico_free. */
struct PkNode* pkh_node(const struct PicoTensor* t);
int pkh_node_register(struct PkNode* n, struct Arena* arena);
void pkh_node_unregister(const struct PkNode* n);
void pkh_registry_clear(void);

/* runtime (runtime.c) */
int pkh_init(void);              /* 0 once the device and stream are up */
pk_stream_t pkh_stream(void);
void pkh_set_error(const char* fmt, ...);
uint64_t pkh_error_count(void); /* errors recorded so far (pico_backward stops on a new one) */
/* maps a launcher status to the pico convention: prints "[Pico] Error: op: msg"
 * and records it; returns status */
int pkh_status(const char* op, int status);
int pkh_sync(void);
int pkh_capturing(void); /* a graph capture is in progress */

/* The side stream: weight gradients (dW = X^T.dY of a parameter) run there,
 * concurrently with the rest of the backward on the library's stream.
 * pkh_side_fork() makes it wait for everything issued so far on the main
 * stream and returns it (NULL if it cannot be created: run on the main
 * stream then); each fork gets a sequence number (pkh_side_seq).
 * pkh_side_join() makes the main stream wait for everything issued on the
 * side stream; pkh_side_joined() is the last sequence number a join covers.
 * Any main-stream access to a grad written on the side stream joins first
 * (pkh_grad_flag / pkh_grad_is_live do it), pico_backward joins at its end,
 * and so do synchronisation and copies. */
pk_stream_t pkh_side_fork(void);
/* Under graph capture only (else they do nothing and return 0):
 * pkh_side_prepare() records the next fork's point on the main stream now, so
 * that the caller can issue a main-stream kernel before the pkh_side_fork()
 * whose side work must not wait for it; pkh_side_defer() queues side work
 * (fn(args, side) with a copy of n <= PKH_SIDE_JOB_ARGS bytes of args) to be
 * issued at the next fork or join, and returns 1 when it did.  A deferred job
 * must leave its tensor's side_seq at pkh_side_seq() + 1 (the fork that
 * issues it), so a main-stream access joins, and so issues it, first. */
int pkh_side_prepare(void);
#define PKH_SIDE_JOB_ARGS 96
typedef void (*pkh_side_job_fn)(const void* args, pk_stream_t side);
int pkh_side_defer(pkh_side_job_fn fn, const void* args, size_t n);
uint64_t pkh_side_seq(void);
uint64_t pkh_side_joined(void);
void pkh_side_join(void);
/* the side stream's own scratch buffer (pkh_workspace is the main stream's) */
void* pkh_side_workspace(size_t bytes);
/* the same for a caller with a fallback (an unsplit product): NULL without a
 * recorded error when the buffer cannot be had */
void* pkh_side_workspace_opt(size_t bytes);

/* AdamW state, for checkpoints (optim.c) */
int pkh_adamw_moments(const struct PicoOptimAdamW* o, const struct PicoTensor* p, float** m,
                      float** v);
int pkh_adamw_sync_step(struct PicoOptimAdamW* o);
int pkh_adamw_step(const struct PicoOptimAdamW* o);
int pkh_adamw_set_step(struct PicoOptimAdamW* o, int step);
void pkh_adamw_hparams(const struct PicoOptimAdamW* o, float* lr, float* b1, float* b2,
                       float* eps, float* wd);
void* pkh_device_alloc(size_t bytes); /* hipMalloc; NULL + message on failure */
void pkh_device_free(void* p);
/* a device scratch buffer of at least `bytes`, reused across calls (the
 * previous contents are not preserved); valid until the next call */
void* pkh_workspace(size_t bytes);
void* pkh_workspace_opt(size_t bytes); /* optional: NULL without a recorded error */
int pkh_is_device_ptr(const void* p);
int pkh_copy_h2d(void* dst, const void* src, size_t bytes);
int pkh_copy_d2h(void* dst, const void* src, size_t bytes);
/* device-to-device on the library's stream, not waited for */
int pkh_copy_d2d_async(void* dst, const void* src, size_t bytes);

/* x . W + bias as one node (ops.c): pico's Linear forward in one product */
struct PicoTensor* pkh_linear(struct PicoTensor* x, struct PicoTensor* w, struct PicoTensor* bias);

/* tensors (tensor.c) */
/* a GPU tensor node in `arena` with uninitialised device data and a
 * not-yet-live grad; `node_bytes` >= sizeof(struct PkNode) */
struct PicoTensor* pkh_new_tensor(struct Arena* arena, const int64_t* shape, int ndim);
struct Arena* pkh_need_arena(void);
int pkh_is_gpu(const struct PicoTensor* t);
/* flags for a write into t->grad: PK_ACCUM if it already holds values; the
 * caller marks it live after a successful launch */
/* before the main stream touches t's grad: wait for side-stream writes to it */
static inline void pkh_grad_on_main(const struct PkNode* n) {
    if(n && n->side_seq > pkh_side_joined()) pkh_side_join();
}
/* A split tensor's grad is the union of its views' grads.  Before it is used
 * whole: if some views hold values, the columns of those that do not are
 * zero-filled and the whole grad becomes live (tensor.c). */
void pkh_grad_complete(struct PkNode* n);
/* does t's grad hold values (for a view: its columns, written through it or
 * through its base; for a split tensor: completed first) */
static inline int pkh_node_live(struct PkNode* n) {
    if(n->n_views && !n->grad_live) pkh_grad_complete(n);
    if(n->grad_live) return 1;
    struct PkNode* b = n->base ? pkh_node(n->base) : NULL;
    return b ? (int)b->grad_live : 0;
}
/* Gradient aliases.  Where an op's backward would copy its upstream gradient
 * unchanged into an operand's empty grad (the operands of c = a + b), the
 * operand's grad pointer is set to c's grad instead (pkh_grad_alias): c's grad
 * is final by then, and the operand reads the same values through it.  The
 * first write into an aliased grad gives the tensor its own buffer back:
 * pkh_grad_flag copies the aliased values into it and returns PK_ACCUM;
 * pkh_grad_base returns the aliased buffer as the source of the accumulated
 * term, for a kernel that writes own = source + contribution without the
 * copy.  pico_backward restores the own buffers of the graph it is about to
 * run, so a second backward over the same graph writes nothing shared. */
int pkh_grad_alias(struct PicoTensor* t, const struct PicoTensor* src); /* 1: aliased */
void pkh_grad_unalias(struct PkNode* n, int copy);
static inline int pkh_grad_flag(const struct PicoTensor* t) {
    struct PkNode* n = pkh_node(t);
    pkh_grad_on_main(n);
    if(n && n->own_grad) pkh_grad_unalias(n, 1);
    return (n && !pkh_node_live(n)) ? 0 : PK_ACCUM;
}
/* for a write t->grad = source + contribution: the source of the accumulated
 * term (t's grad itself, an aliased grad, or NULL when t's grad is empty) */
static inline const float* pkh_grad_base(struct PicoTensor* t) {
    struct PkNode* n = pkh_node(t);
    if(n && n->own_grad) {
        const float* src = t->grad;
        pkh_grad_unalias(n, 0);
        return src;
    }
    return pkh_grad_flag(t) ? t->grad : NULL;
}
static inline void pkh_grad_mark(struct PicoTensor* t) {
    struct PkNode* n = pkh_node(t);
    if(n) n->grad_live = 1;
}
static inline int pkh_grad_is_live(const struct PicoTensor* t) {
    struct PkNode* n = pkh_node(t);
    pkh_grad_on_main(n);
    return n ? pkh_node_live(n) : 1;
}
void pkh_set_parents(struct Arena* arena, struct PicoTensor* out, int n,
                     struct PicoTensor* const* ps, void (*bw)(struct PicoTensor*));
/* the grad of `self` as the upstream gradient; NULL (nothing to propagate)
 * when it holds no values */
const float* pkh_upstream(struct PicoTensor* self);
/* int32 ids/labels on the device: device pointers pass through, host arrays
 * are copied into the current arena */
const int32_t* pkh_ids_on_device(const int32_t* ids, int64_t n);

/* matrix view of a 2-D tensor for the GEMM launcher: 'N' when rows are
 * contiguous (strides[1] == 1), 'T' when columns are (strides[0] == 1) */
struct PkMat {
    const float* p;
    char t;
    int64_t ld;
    int persist; /* p is a parameter's data, read as itself (its casts can be kept) */
};
int pkh_mat_view(const struct PicoTensor* x, const float* base, struct PkMat* m);
/* C (+)= A . B for logical matrices A [M,K], B [K,N]; C is stored as the
 * view `c` describes (a transposed C is produced as C^T = B^T A^T) */
int pkh_gemm(struct PkMat A, struct PkMat B, int64_t M, int64_t N, int64_t K, float* C, char tc,
             int64_t ldc, int flags);

/* fp8 products (mx8.c): C [M, N] (not transposed) = op(A).op(B) + beta X
 * through MX8 operands; the side flag picks the side stream's workspace */
int pkh_mx8_product(struct PkMat A, struct PkMat B, int64_t M, int64_t N, int64_t K, float* C,
                    int64_t ldc, float beta, const float* X, int64_t ldx, pk_stream_t st,
                    int side);
/* both casts of a backward's upstream gradient g [M, N] (row stride N), used
 * by the products issued until pkh_mx8_grad_casts_done() */
int pkh_mx8_grad_casts(const float* g, int64_t M, int64_t N, pk_stream_t st);
void pkh_mx8_grad_casts_done(void);
/* parameters may have changed: casts kept from before are redone at next use */
void pkh_params_changed(void);
void pkh_mx8_release(void);

#pragma GCC visibility pop

#define PKH_ERR(...) fprintf(stderr, "[Pico] Error: " __VA_ARGS__)
