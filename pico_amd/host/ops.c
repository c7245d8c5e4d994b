/*
 * pico_amd/host/ops.c -- pico's op layer for GPU tensors: add/sub/mul with
 * broadcasting, 2-D matmul, unary math, relu, their backward hooks, and the
 * GPU twins of the op seam the reference leaves as commented-out stubs
 * (src/ops.c:42-44, 86-88, 130-132).
 *
 * Each op keeps the reference's template (src/ops.c:12-54): validate in the
 * same order with the same messages, take the current arena, allocate the
 * output there, launch, wire parents and _backward.  The launches go to the
 * pk_* layer (include/pico_hip.h); nothing here touches device data.
 */
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

enum { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2 };
enum { U_SQRT = 0, U_SIN, U_COS, U_TAN, U_TANH, U_LOG };

static int refuse_cpu(const char* op, const struct PicoTensor* a) {
    if(pkh_is_gpu(a)) return 0;
    PKH_ERR("%s: this library runs backend GPU; CPU tensors belong to pico's CPU library!\n", op);
    return 1;
}

/* strides of t mapped onto an ndim-dim output (0 where t is broadcast), the
 * map pico's map_index applies per element (src/tensor.h:122-138) */
static void mapped_strides(const struct PicoTensor* t, int ndim, int64_t* out) {
    int diff = ndim - t->ndim;
    for(int d = 0; d < ndim; d++) {
        int sd = d - diff;
        out[d] = (sd >= 0 && t->shape[sd] > 1) ? t->strides[sd] : 0;
    }
}

/* t has self's shape and is stored row-major, so its grad and self's index
 * alike */
static int same_layout(const struct PicoTensor* t, const struct PicoTensor* self) {
    if(t->ndim != self->ndim) return 0;
    int64_t stride = 1;
    for(int d = t->ndim - 1; d >= 0; d--) {
        if(t->shape[d] != self->shape[d]) return 0;
        if(t->shape[d] > 1 && t->strides[d] != stride) return 0;
        stride *= t->shape[d];
    }
    return 1;
}

/* ---------------------------------------------------- binary: seam twins */
/* The seam twins may be called by pico itself (its ops.c with the GPU stubs
 * filled in) on tensors it allocated: nothing here assumes they are this
 * library's nodes, only that data and grad are device memory. */
static int twin_refuses(const char* op, const struct PicoTensor* a, const struct PicoTensor* b,
                        const struct PicoTensor* out) {
    if(pkh_init()) return PK_EINVAL;
    const char* why = (!a || !b || !out) ? "NULL tensor"
                      : (!pkh_is_gpu(a) || !pkh_is_gpu(b) || !pkh_is_gpu(out))
                          ? "expects tensors whose backend is GPU (device data and grad)"
                          : NULL;
    if(!why) return 0;
    pkh_set_error("%s: %s", op, why);
    PKH_ERR("%s: %s!\n", op, why);
    return PK_EINVAL;
}

static int binary_gpu(int op, struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out) {
    int64_t sa[256], sb[256];
    int nd = out->ndim;
    mapped_strides(a, nd, sa);
    mapped_strides(b, nd, sb);
    return pk_binary_f32(op, nd, out->shape, sa, sb, a->data, b->data, out->data, pkh_stream());
}

int pico_add_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out) {
    if(twin_refuses("pico_add_gpu", a, b, out)) return PK_EINVAL;
    return pkh_status("pico_add", binary_gpu(OP_ADD, a, b, out));
}
int pico_sub_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out) {
    if(twin_refuses("pico_sub_gpu", a, b, out)) return PK_EINVAL;
    return pkh_status("pico_sub", binary_gpu(OP_SUB, a, b, out));
}
int pico_mul_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out) {
    if(twin_refuses("pico_mul_gpu", a, b, out)) return PK_EINVAL;
    return pkh_status("pico_mul", binary_gpu(OP_MUL, a, b, out));
}

/* src/autograd.h:53-94: a.grad += g (or g*b), b.grad += g (-g, g*a), summed
 * over each operand's broadcast dims */
static void binary_backward(int op, struct PicoTensor* self) {
    if(pkh_init()) return;
    struct PicoTensor *a = self->parents[0], *b = self->parents[1];
    const float* g = pkh_upstream(self);
    if(!g) return;
    int64_t sa[256], sb[256];
    int nd = self->ndim;
    mapped_strides(a, nd, sa);
    mapped_strides(b, nd, sb);
    static const char* names[3] = {"pico_add_backward", "pico_sub_backward", "pico_mul_backward"};
    /* d(a+b)/da = d(a+b)/db = 1: an operand of self's shape whose grad is empty
     * takes self's grad as it is (an alias) instead of a copy of it */
    if(!(op == OP_ADD && same_layout(a, self) && pkh_grad_alias(a, self))) {
        int st = pk_binary_bwd_f32(op, 0, nd, self->shape, sa, sb, a->numel, g, b->data, a->grad,
                                   pkh_grad_flag(a), pkh_stream());
        if(pkh_status(names[op], st)) return;
        pkh_grad_mark(a);
    }
    if(!(op == OP_ADD && same_layout(b, self) && pkh_grad_alias(b, self))) {
        int st = pk_binary_bwd_f32(op, 1, nd, self->shape, sb, sa, b->numel, g, a->data, b->grad,
                                   pkh_grad_flag(b), pkh_stream());
        if(pkh_status(names[op], st)) return;
        pkh_grad_mark(b);
    }
}
void pico_add_backward_gpu(struct PicoTensor* self) { binary_backward(OP_ADD, self); }
void pico_sub_backward_gpu(struct PicoTensor* self) { binary_backward(OP_SUB, self); }
void pico_mul_backward_gpu(struct PicoTensor* self) { binary_backward(OP_MUL, self); }

/* src/ops.c:12-142 */
static struct PicoTensor* binary_op(int op, const char* name, struct PicoTensor* a,
                                    struct PicoTensor* b, void (*bw)(struct PicoTensor*)) {
    if(!a || !b) {
        PKH_ERR("%s: NULL tensor!\n", name);
        return NULL;
    }
    if(!pico_check_broadcast_compatibility(a, b)) {
        PKH_ERR("Shapes are not broadcastable!\n");
        return NULL;
    }
    if(a->backend != b->backend) {
        PKH_ERR("PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(refuse_cpu(name, a)) return NULL;
    int ndim = a->ndim > b->ndim ? a->ndim : b->ndim;
    int64_t shape[256];
    for(int i = 0; i < ndim; i++) {
        int ia = i - (ndim - a->ndim), ib = i - (ndim - b->ndim);
        int64_t da = ia >= 0 ? a->shape[ia] : 1, db = ib >= 0 ? b->shape[ib] : 1;
        shape[i] = da > db ? da : db;
    }
    struct PicoTensor* out = pkh_new_tensor(arena, shape, ndim);
    if(!out) return NULL;
    if(pkh_status(name, binary_gpu(op, a, b, out))) return NULL;
    struct PicoTensor* ps[2] = {a, b};
    pkh_set_parents(arena, out, 2, ps, bw);
    return out;
}

struct PicoTensor* pico_add(struct PicoTensor* a, struct PicoTensor* b) {
    return binary_op(OP_ADD, "pico_add", a, b, pico_add_backward_gpu);
}
struct PicoTensor* pico_sub(struct PicoTensor* a, struct PicoTensor* b) {
    return binary_op(OP_SUB, "pico_sub", a, b, pico_sub_backward_gpu);
}
struct PicoTensor* pico_mul(struct PicoTensor* a, struct PicoTensor* b) {
    return binary_op(OP_MUL, "pico_mul", a, b, pico_mul_backward_gpu);
}

/* ------------------------------------------------------------------ GEMM */
/* 'N' when rows are contiguous (strides[1] == 1, ld = strides[0]); 'T' when
 * columns are (strides[0] == 1, ld = strides[1]).  With a single row (or
 * column) the leading dimension is never stepped and only has to satisfy the
 * launcher's minimum. */
int pkh_mat_view(const struct PicoTensor* x, const float* base, struct PkMat* m) {
    if(x->ndim != 2) return PK_EINVAL;
    int64_t rows = x->shape[0], cols = x->shape[1], s0 = x->strides[0], s1 = x->strides[1];
    m->p = base;
    if(s1 == 1 && (rows <= 1 || s0 >= cols)) {
        m->t = 'N';
        m->ld = s0 > cols ? s0 : cols;
    } else if(s0 == 1 && (cols <= 1 || s1 >= rows)) {
        m->t = 'T';
        m->ld = s1 > rows ? s1 : rows;
    } else {
        return PK_EINVAL;
    }
    if(m->ld < 1) m->ld = 1;
    m->persist = x->is_persistent && base == x->data;
    return 0;
}

static inline char flip(char t) { return t == 'N' ? 'T' : 'N'; }

/* precision of pico_matmul's products and of their gradients */
static int g_matmul_precision = PICO_MATMUL_FP32;

int pico_set_matmul_precision(int precision) {
    if(precision != PICO_MATMUL_FP32 && precision != PICO_MATMUL_BF16 &&
       precision != PICO_MATMUL_BF16X3 && precision != PICO_MATMUL_FP8) {
        PKH_ERR("pico_set_matmul_precision: unknown precision %d!\n", precision);
        return PK_EINVAL;
    }
    g_matmul_precision = precision;
    return 0;
}

int pico_get_matmul_precision(void) { return g_matmul_precision; }

/* products with too few output tiles (weight gradients) split K through a
 * workspace; see pk_gemm_ex_f32.  On the side stream (side != 0) the product
 * uses the side stream's own workspace.  fp8 products go through MX8
 * operands (mx8.c). */
static int gemm_add_on(struct PkMat A, struct PkMat B, int64_t M, int64_t N, int64_t K, float* C,
                       char tc, int64_t ldc, float beta, const float* X, int64_t ldx,
                       pk_stream_t st, int side) {
    /* C stored transposed: produce C^T [N, M] = B^T . A^T (X is C itself here) */
    struct PkMat BT = {B.p, flip(B.t), B.ld, B.persist}, AT = {A.p, flip(A.t), A.ld, A.persist};
    if(g_matmul_precision == PICO_MATMUL_FP8)
        return tc == 'N' ? pkh_mx8_product(A, B, M, N, K, C, ldc, beta, X, ldx, st, side)
                         : pkh_mx8_product(BT, AT, N, M, K, C, ldc, beta, C, ldc, st, side);
    size_t ws_bytes = pk_gemm_workspace_f32(M, N, K);
    /* split-K scratch is optional (the product runs unsplit without it) */
    void* ws = NULL;
    if(ws_bytes) ws = side ? pkh_side_workspace_opt(ws_bytes) : pkh_workspace_opt(ws_bytes);
    if(!ws) ws_bytes = 0;
    if(tc == 'N')
        return pk_gemm_add_f32(A.t, B.t, M, N, K, 1.0f, A.p, A.ld, B.p, B.ld, beta, X, ldx, C, ldc,
                               g_matmul_precision, NULL, ws, ws_bytes, st);
    return pk_gemm_add_f32(BT.t, AT.t, N, M, K, 1.0f, B.p, B.ld, A.p, A.ld, beta, C, ldc, C, ldc,
                           g_matmul_precision, NULL, ws, ws_bytes, st);
}

static int gemm_on(struct PkMat A, struct PkMat B, int64_t M, int64_t N, int64_t K, float* C,
                   char tc, int64_t ldc, int flags, pk_stream_t st, int side) {
    const float beta = (flags & PK_ACCUM) ? 1.0f : 0.0f;
    return gemm_add_on(A, B, M, N, K, C, tc, ldc, beta, C, ldc, st, side);
}

int pkh_gemm(struct PkMat A, struct PkMat B, int64_t M, int64_t N, int64_t K, float* C, char tc,
             int64_t ldc, int flags) {
    return gemm_on(A, B, M, N, K, C, tc, ldc, flags, pkh_stream(), 0);
}

static int matmul_views(struct PicoTensor* a, struct PicoTensor* b, struct PkMat* va,
                        struct PkMat* vb) {
    if(pkh_mat_view(a, a->data, va) || pkh_mat_view(b, b->data, vb)) {
        pkh_set_error("pico_matmul: operands must have a unit stride along one dimension");
        PKH_ERR("pico_matmul: operands must have a unit stride along one dimension!\n");
        return PK_EINVAL;
    }
    return 0;
}

/* out = a . b, out contiguous [rows(a), cols(b)] (pico's kernels += into a
 * zeroed out, src/kernels/cpu/cpu_scalar.h:39-54; here it is overwritten) */
int pico_matmul_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out) {
    if(twin_refuses("pico_matmul_gpu", a, b, out)) return PK_EINVAL;
    struct PkMat va, vb;
    if(matmul_views(a, b, &va, &vb)) return PK_EINVAL;
    int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    return pkh_status("pico_matmul",
                      pkh_gemm(va, vb, M, N, K, out->data, 'N', N > 0 ? N : 1, 0));
}

/* The two products of a matmul's backward (src/autograd.h:96-130) for
 * self = A.B (+ ...) with upstream gradient g [M, N]: the input gradient
 * (dA (+)= g.B^T, issued by dA_fn) and the weight gradient dB (+)= A^T.g,
 * each laid out with its tensor's strides, so a transposed view's grad is
 * produced transposed.  A is given as a matrix view of its data, since a
 * fused op's A may be a buffer the op saved rather than a graph tensor.
 *
 * When B is a parameter (persistent) and A is not, dB -- a weight gradient,
 * read only once the backward is over -- goes to the side stream and runs
 * concurrently with the rest of the backward; the main stream waits for it
 * before it next touches B's grad and at the end of pico_backward.  Writes to
 * one grad keep their program order either way, so results are bit for bit
 * those of a single stream.
 *
 * Eagerly, dB is forked before dA is issued, so that it runs beside dA
 * rather than beside the memory-bound kernels that follow dA (config 5: about
 * 1.3 ms less per step).  Under graph capture dA is captured first and dB
 * after it, waiting for the same point before dA (pkh_side_prepare): a
 * replay continues each stream with a node's first captured child, so dA's
 * chain stays on the main stream.  Either way the side stream orders dB's
 * write after every earlier write to B's grad: main-stream ones through the
 * fork, side ones by issue order. */
static void matmul_backward_body(struct PkMat va, int a_param, struct PicoTensor* b,
                                 const float* g, int64_t M, int64_t K, int64_t N,
                                 int (*dA_fn)(void*), void* ctx) {
    struct PkMat vb;
    if(pkh_mat_view(b, b->data, &vb)) {
        pkh_status("pico_matmul_backward", PK_EINVAL);
        return;
    }
    struct PkMat dC = {g, 'N', N > 0 ? N : 1, 0};
    struct PkMat AT = {va.p, flip(va.t), va.ld, va.persist};
    struct PkNode* nb = pkh_node(b);
    const int to_side = nb && b->is_persistent && !a_param && va.p != b->data;
    const int db_first = to_side && !pkh_capturing();
    pk_stream_t side = db_first ? pkh_side_fork() : NULL;
    int st;
    if(side) {
        st = gemm_on(AT, dC, K, N, M, b->grad, vb.t, vb.ld, nb->grad_live ? PK_ACCUM : 0, side, 1);
        nb->side_seq = pkh_side_seq();
        if(pkh_status("pico_matmul_backward", st)) return;
        pkh_grad_mark(b);
    }
    /* under capture: dA is captured before dB, and dB waits for the point
     * before dA (as eagerly), so a replay keeps dA's chain on the main stream */
    if(to_side && !side) pkh_side_prepare();
    if(dA_fn(ctx)) return;
    if(side) return;
    side = to_side ? pkh_side_fork() : NULL;
    if(side) {
        st = gemm_on(AT, dC, K, N, M, b->grad, vb.t, vb.ld, nb->grad_live ? PK_ACCUM : 0, side, 1);
        nb->side_seq = pkh_side_seq();
    } else {
        st = pkh_gemm(AT, dC, K, N, M, b->grad, vb.t, vb.ld, pkh_grad_flag(b));
    }
    if(pkh_status("pico_matmul_backward", st)) return;
    pkh_grad_mark(b);
}

/* fp8: both products read g, cast once for both (mx8.c) */
static void matmul_backward_with(struct PkMat va, int a_param, struct PicoTensor* b,
                                 const float* g, int64_t M, int64_t K, int64_t N,
                                 int (*dA_fn)(void*), void* ctx) {
    if(g_matmul_precision == PICO_MATMUL_FP8 &&
       pkh_status("pico_matmul_backward", pkh_mx8_grad_casts(g, M, N, pkh_stream())))
        return;
    matmul_backward_body(va, a_param, b, g, M, K, N, dA_fn, ctx);
    pkh_mx8_grad_casts_done();
}

/* dA (+)= g . B^T into a tensor's grad (the plain matmul's input gradient) */
struct DaPlain {
    struct PicoTensor *a, *b;
    const float* g;
    int64_t M, K, N;
};
static int da_plain(void* ctx) {
    struct DaPlain* c = (struct DaPlain*)ctx;
    struct PkMat va, vb;
    if(matmul_views(c->a, c->b, &va, &vb)) return PK_EINVAL;
    struct PkMat dC = {c->g, 'N', c->N > 0 ? c->N : 1, 0};
    struct PkMat BT = {c->b->data, flip(vb.t), vb.ld, vb.persist};
    int st = pkh_gemm(dC, BT, c->M, c->K, c->N, c->a->grad, va.t, va.ld, pkh_grad_flag(c->a));
    if(pkh_status("pico_matmul_backward", st)) return st;
    pkh_grad_mark(c->a);
    return 0;
}

void pico_matmul_backward_gpu(struct PicoTensor* self) {
    if(pkh_init()) return;
    struct PicoTensor *a = self->parents[0], *b = self->parents[1];
    const float* g = pkh_upstream(self);
    if(!g) return;
    struct PkMat va, vb;
    if(matmul_views(a, b, &va, &vb)) return;
    int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    struct DaPlain ctx = {a, b, g, M, K, N};
    matmul_backward_with(va, a->is_persistent || a == b, b, g, M, K, N, da_plain, &ctx);
}

/* src/ops.c:144-190 (checks in the reference's order) */
struct PicoTensor* pico_matmul(struct PicoTensor* a, struct PicoTensor* b) {
    if(!a || !b) {
        PKH_ERR("pico_matmul: NULL tensor!\n");
        return NULL;
    }
    if(a->shape[a->ndim - 1] != b->shape[0]) {
        PKH_ERR("2 matmuls matrices must be compatible\n");
        return NULL;
    }
    if(a->ndim != 2 || b->ndim != 2) {
        PKH_ERR("2d matmul matrices must be compatible\n");
        return NULL;
    }
    if(a->backend != b->backend) {
        PKH_ERR("PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(refuse_cpu("pico_matmul", a)) return NULL;
    int64_t shape[2] = {a->shape[0], b->shape[1]};
    struct PicoTensor* out = pkh_new_tensor(arena, shape, 2);
    if(!out) return NULL;
    if(pico_matmul_gpu(a, b, out)) return NULL;
    struct PicoTensor* ps[2] = {a, b};
    pkh_set_parents(arena, out, 2, ps, pico_matmul_backward_gpu);
    return out;
}

/* ----------------------------------------------------------- fused ops
 * No reference counterpart: pico runs a matmul and the op that consumes it as
 * two passes over memory.  These produce the same values as the composed ops
 * (the fused epilogue rounds exactly as the separate kernels do), with one
 * pass fewer and no intermediate tensor in the graph. */

/* a residual matrix added in the product's epilogue: the output's shape,
 * contiguous */
static int residual_ok(const struct PicoTensor* c, int64_t M, int64_t N) {
    return c->ndim == 2 && c->shape[0] == M && c->shape[1] == N && c->strides[1] == 1 &&
           (c->strides[0] == N || M <= 1);
}

/* d(out)/dc = 1: an empty grad takes out's grad by pointer (an alias),
 * otherwise out's grad is added to it */
static int residual_backward(struct PicoTensor* self, struct PicoTensor* c, const float* g) {
    if(same_layout(c, self) && pkh_grad_alias(c, self)) return 0;
    int st = pk_axpy_f32(c->numel, 1.0f, NULL, g, c->grad, pkh_grad_flag(c), pkh_stream());
    if(pkh_status("pico_matmul_add_backward", st)) return st;
    pkh_grad_mark(c);
    return 0;
}

static void matmul_add_backward(struct PicoTensor* self) {
    if(pkh_init()) return;
    struct PicoTensor *a = self->parents[0], *b = self->parents[1], *c = self->parents[2];
    const float* g = pkh_upstream(self);
    if(!g) return;
    if(residual_backward(self, c, g)) return;
    struct PkMat va, vb;
    if(matmul_views(a, b, &va, &vb)) return;
    int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    struct DaPlain ctx = {a, b, g, M, K, N};
    matmul_backward_with(va, a->is_persistent || a == b, b, g, M, K, N, da_plain, &ctx);
}

/* out = c + a . b in one pass: the product's epilogue adds c (a residual
 * connection, x + attn.Wo) */
struct PicoTensor* pico_matmul_add(struct PicoTensor* a, struct PicoTensor* b,
                                   struct PicoTensor* c) {
    if(!a || !b || !c) {
        PKH_ERR("pico_matmul_add: NULL tensor!\n");
        return NULL;
    }
    if(a->ndim != 2 || b->ndim != 2 || a->shape[1] != b->shape[0]) {
        PKH_ERR("2d matmul matrices must be compatible\n");
        return NULL;
    }
    if(a->backend != b->backend || a->backend != c->backend) {
        PKH_ERR("PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(refuse_cpu("pico_matmul_add", a)) return NULL;
    int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    if(!residual_ok(c, M, N)) {
        PKH_ERR("pico_matmul_add: the added tensor must be a contiguous [rows(a), cols(b)]!\n");
        return NULL;
    }
    struct PkMat va, vb;
    if(matmul_views(a, b, &va, &vb)) return NULL;
    int64_t shape[2] = {M, N};
    struct PicoTensor* out = pkh_new_tensor(arena, shape, 2);
    if(!out) return NULL;
    int st = gemm_add_on(va, vb, M, N, K, out->data, 'N', N > 0 ? N : 1, 1.0f, c->data,
                         c->strides[0], pkh_stream(), 0);
    if(pkh_status("pico_matmul_add", st)) return NULL;
    struct PicoTensor* ps[3] = {a, b, c};
    pkh_set_parents(arena, out, 3, ps, matmul_add_backward);
    return out;
}

/* ------------------------------------------------- Linear in one product
 * pico's Linear forward is pico_matmul then pico_add of the bias row
 * (src/nn/linear.c:57-64): two nodes, two passes.  Here one node x.W + b: the
 * product's epilogue adds the bias row (pk_gemm_add_f32 with ldx = 0), which
 * rounds exactly as the separate add does (the product is the same fp32
 * accumulator, then one rounding of its sum with b).  Its backward gives the
 * same gradients as the two nodes': db is the broadcast add's column sums in
 * pico's order (src/autograd.h:53-65), dx and dW the matmul's products. */

/* db (+)= the column sums of g [M, N]; on the side stream with the weight
 * gradient when the layer's input is not a parameter (a bias is read only
 * once the backward is over) */
struct BiasJob {
    int64_t shape[2], sb[2], sg[2], numel;
    const float* g;
    float* grad;
    int flag;
};
static void bias_job(const void* args, pk_stream_t side) {
    const struct BiasJob* j = (const struct BiasJob*)args;
    pkh_status("pico_add_backward", pk_binary_bwd_f32(OP_ADD, 1, 2, j->shape, j->sb, j->sg,
                                                      j->numel, j->g, j->g, j->grad, j->flag, side));
}

static int bias_backward(struct PicoTensor* self, struct PicoTensor* bias, const float* g,
                         int input_param) {
    int64_t sb[2], sg[2] = {self->strides[0], self->strides[1]};
    mapped_strides(bias, 2, sb);
    struct PkNode* nb = pkh_node(bias);
    const int to_side = nb && bias->is_persistent && !input_param;
    if(to_side && pkh_capturing()) {
        /* captured, the side work waits for the next fork (after the main
         * stream's next kernel), so a replay keeps the main chain on its stream */
        struct BiasJob j = {{self->shape[0], self->shape[1]}, {sb[0], sb[1]}, {sg[0], sg[1]},
                            bias->numel, g, bias->grad, nb->grad_live ? PK_ACCUM : 0};
        if(pkh_side_defer(bias_job, &j, sizeof(j))) {
            nb->side_seq = pkh_side_seq() + 1;
            pkh_grad_mark(bias);
            return 0;
        }
    }
    pk_stream_t side = to_side ? pkh_side_fork() : NULL;
    const int flag = side ? (nb->grad_live ? PK_ACCUM : 0) : pkh_grad_flag(bias);
    int st = pk_binary_bwd_f32(OP_ADD, 1, 2, self->shape, sb, sg, bias->numel, g, g, bias->grad,
                               flag, side ? side : pkh_stream());
    if(side) nb->side_seq = pkh_side_seq();
    if(pkh_status("pico_add_backward", st)) return st;
    pkh_grad_mark(bias);
    return 0;
}

static void linear_backward(struct PicoTensor* self) {
    if(pkh_init()) return;
    struct PicoTensor *a = self->parents[0], *b = self->parents[1], *bias = self->parents[2];
    const float* g = pkh_upstream(self);
    if(!g) return;
    const int a_param = a->is_persistent || a == b;
    if(bias_backward(self, bias, g, a_param)) return;
    struct PkMat va, vb;
    if(matmul_views(a, b, &va, &vb)) return;
    int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    struct DaPlain ctx = {a, b, g, M, K, N};
    matmul_backward_with(va, a_param, b, g, M, K, N, da_plain, &ctx);
}

/* x . W + bias with the checks of pico_matmul then pico_add (bias [N] or
 * [1, N]); NULL (with the reference's message) where either would refuse */
struct PicoTensor* pkh_linear(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* bias) {
    if(!a || !b || !bias) {
        PKH_ERR("pico_matmul: NULL tensor!\n");
        return NULL;
    }
    if(a->shape[a->ndim - 1] != b->shape[0]) {
        PKH_ERR("2 matmuls matrices must be compatible\n");
        return NULL;
    }
    if(a->ndim != 2 || b->ndim != 2) {
        PKH_ERR("2d matmul matrices must be compatible\n");
        return NULL;
    }
    if(a->backend != b->backend || a->backend != bias->backend) {
        PKH_ERR("PicoTensor backends are not compatible!\n");
        return NULL;
    }
    int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    const int row = (bias->ndim == 1 && bias->shape[0] == N) ||
                    (bias->ndim == 2 && bias->shape[0] == 1 && bias->shape[1] == N);
    if(!row || bias->strides[bias->ndim - 1] != 1) {
        /* another broadcast: the two ops */
        struct PicoTensor* prod = pico_matmul(a, b);
        return prod ? pico_add(prod, bias) : NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(refuse_cpu("pico_matmul", a)) return NULL;
    struct PkMat va, vb;
    if(matmul_views(a, b, &va, &vb)) return NULL;
    int64_t shape[2] = {M, N};
    struct PicoTensor* out = pkh_new_tensor(arena, shape, 2);
    if(!out) return NULL;
    int st = gemm_add_on(va, vb, M, N, K, out->data, 'N', N > 0 ? N : 1, 1.0f, bias->data, 0,
                         pkh_stream(), 0);
    if(pkh_status("pico_matmul", st)) return NULL;
    struct PicoTensor* ps[3] = {a, b, bias};
    pkh_set_parents(arena, out, 3, ps, linear_backward);
    return out;
}

/* The gate/up projection of a SwiGLU block (no reference counterpart): out =
 * a . w for w = [W1 | W3] (two column halves), a matmul to autograd.  Its
 * product also writes h = silu(out[:, :F]) * out[:, F:] from the tiles
 * (pk_gemm_swiglu_fwd_f32: each tile holds matching gate and up columns), and
 * the node keeps h: pico_swiglu_matmul_add over the two column views of out
 * (pico_split_cols(out, 2)) takes it instead of running the SwiGLU kernel.
 * Shapes the paired product does not take (a transposed view, F not a
 * multiple of 32) run the plain product and keep nothing. */
enum { GU_H = 0 };
enum { GU_MARK = 0 };
#define PKH_GU_MARK 0x53574947 /* "GIWS": this node holds h */

struct PicoTensor* pico_matmul_gate_up(struct PicoTensor* a, struct PicoTensor* w) {
    if(!a || !w) {
        PKH_ERR("pico_matmul_gate_up: NULL tensor!\n");
        return NULL;
    }
    if(a->ndim != 2 || w->ndim != 2 || a->shape[1] != w->shape[0]) {
        PKH_ERR("2d matmul matrices must be compatible\n");
        return NULL;
    }
    if(a->backend != w->backend) {
        PKH_ERR("PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(refuse_cpu("pico_matmul_gate_up", a)) return NULL;
    const int64_t M = a->shape[0], K = a->shape[1], N = w->shape[1], F = N / 2;
    if(N % 2) {
        PKH_ERR("pico_matmul_gate_up: w must have an even number of columns [W1 | W3]!\n");
        return NULL;
    }
    struct PkMat va, vw;
    if(matmul_views(a, w, &va, &vw)) return NULL;
    int64_t shape[2] = {M, N};
    struct PicoTensor* out = pkh_new_tensor(arena, shape, 2);
    if(!out) return NULL;
    float* h = NULL;
    /* the paired product never splits K and runs on the tiled kernels; where
     * the plain product would split K or run on the small-product kernels, the
     * plain product runs, so both ways sum k in the same order.  fp8 products
     * (MX8) run the plain product too. */
    if(va.t == 'N' && vw.t == 'N' && F % 32 == 0 && M > 0 && K > 0 && F > 0 &&
       g_matmul_precision != PICO_MATMUL_FP8 && pk_gemm_workspace_f32(M, N, K) == 0 &&
       !pk_gemm_small_product_f32(M, N, K)) {
        h = (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(M * F));
        if(!h) return NULL;
        int st = pk_gemm_swiglu_fwd_f32('N', 'N', M, N, K, 1.0f, va.p, va.ld, vw.p, vw.ld,
                                        out->data, N, h, F, g_matmul_precision, NULL,
                                        pkh_stream());
        if(pkh_status("pico_matmul_gate_up", st)) return NULL;
    } else if(pico_matmul_gpu(a, w, out)) {
        return NULL;
    }
    struct PkNode* n = pkh_node(out);
    n->saved[GU_H] = h;
    n->ival[GU_MARK] = h ? PKH_GU_MARK : 0;
    struct PicoTensor* ps[2] = {a, w};
    pkh_set_parents(arena, out, 2, ps, pico_matmul_backward_gpu);
    return out;
}

/* h that pico_matmul_gate_up kept for exactly these two column views, else NULL */
static const float* gate_up_h(struct PicoTensor* gate, struct PicoTensor* up) {
    struct PkNode *gn = pkh_node(gate), *un = pkh_node(up);
    if(!gn || !un || !gn->base || gn->base != un->base) return NULL;
    struct PicoTensor* src = gn->base;
    struct PkNode* sn = pkh_node(src);
    const int64_t F = gate->shape[1];
    if(!sn || sn->ival[GU_MARK] != PKH_GU_MARK || !sn->saved[GU_H] || src->ndim != 2 ||
       src->shape[1] != 2 * F || src->shape[0] != gate->shape[0] || gate->data != src->data ||
       up->data != src->data + F)
        return NULL;
    return (const float*)sn->saved[GU_H];
}

/* SwiGLU then a product: out = (c +) swiglu(gate, up) . w.  h = silu(gate) *
 * up is kept in the arena for the weight gradient (or taken from
 * pico_matmul_gate_up, which made it); the backward never stores dh: the
 * input-gradient product dY . w^T writes the gate and up gradients straight
 * from its tiles (pk_gemm_swiglu_bwd_f32). */
enum { SM_H = 0 };
enum { SM_LD = 0, SM_RESID = 1 };

struct DaSwiglu {
    struct PicoTensor *gate, *up, *w;
    const float* g;
    int64_t M, F, N, ld;
};
static int da_swiglu(void* ctx) {
    struct DaSwiglu* c = (struct DaSwiglu*)ctx;
    const int flags = (pkh_grad_flag(c->gate) ? PK_ACCUM : 0) | (pkh_grad_flag(c->up) ? PK_ACCUM2 : 0);
    struct PkMat g = {c->g, 'N', c->N > 0 ? c->N : 1, 0},
                 wt = {c->w->data, 'T', c->w->strides[0], c->w->is_persistent};
    if((g_matmul_precision == PICO_MATMUL_FP32 && pk_gemm_small_product_f32(c->M, c->F, c->N)) ||
       g_matmul_precision == PICO_MATMUL_FP8) {
        /* a small product, or an fp8 one (MX8): dh into the arena, then
         * SwiGLU's backward row kernel, as the composed ops compute it */
        struct Arena* arena = pkh_need_arena();
        float* dh = arena ? (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(c->M * c->F))
                          : NULL;
        if(!dh) return pkh_status("pico_swiglu_matmul_add_backward", PK_EINVAL);
        int st = pkh_gemm(g, wt, c->M, c->F, c->N, dh, 'N', c->F, 0);
        if(!st)
            st = pk_swiglu_bwd_f32(c->M, c->F, c->gate->data, c->ld, c->up->data, c->ld, dh, c->F,
                                   c->gate->grad, c->up->grad, c->ld, flags, pkh_stream());
        if(pkh_status("pico_swiglu_matmul_add_backward", st)) return st;
        pkh_grad_mark(c->gate);
        pkh_grad_mark(c->up);
        return 0;
    }
    /* dh = g [M, N] . w^T, w [F, N] row-major */
    int st = pk_gemm_swiglu_bwd_f32('N', 'T', c->M, c->F, c->N, 1.0f, g.p, g.ld, wt.p, wt.ld,
                                    c->gate->data, c->ld, c->up->data, c->ld, c->gate->grad,
                                    c->up->grad, c->ld, flags, g_matmul_precision, NULL,
                                    pkh_stream());
    if(pkh_status("pico_swiglu_matmul_add_backward", st)) return st;
    pkh_grad_mark(c->gate);
    pkh_grad_mark(c->up);
    return 0;
}

static void swiglu_matmul_backward(struct PicoTensor* self) {
    if(pkh_init()) return;
    struct PkNode* n = pkh_node(self);
    struct PicoTensor *gate = self->parents[0], *up = self->parents[1], *w = self->parents[2];
    const float* g = pkh_upstream(self);
    if(!g) return;
    if(n->ival[SM_RESID] && residual_backward(self, self->parents[3], g)) return;
    const int64_t M = gate->shape[0], F = gate->shape[1], N = w->shape[1];
    struct PkMat vh = {(const float*)n->saved[SM_H], 'N', F > 0 ? F : 1, 0};
    struct DaSwiglu ctx = {gate, up, w, g, M, F, N, n->ival[SM_LD]};
    matmul_backward_with(vh, 0, w, g, M, F, N, da_swiglu, &ctx);
}

struct PicoTensor* pico_swiglu_matmul_add(struct PicoTensor* gate, struct PicoTensor* up,
                                          struct PicoTensor* w, struct PicoTensor* c) {
    if(!gate || !up || !w) {
        PKH_ERR("pico_swiglu_matmul_add: NULL tensor!\n");
        return NULL;
    }
    if(gate->backend != up->backend || gate->backend != w->backend ||
       (c && c->backend != gate->backend)) {
        PKH_ERR("PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(refuse_cpu("pico_swiglu_matmul_add", gate)) return NULL;
    if(gate->ndim != 2 || up->ndim != 2 || gate->shape[0] != up->shape[0] ||
       gate->shape[1] != up->shape[1] || gate->strides[1] != 1 || up->strides[1] != 1 ||
       gate->strides[0] != up->strides[0] || gate->strides[0] < gate->shape[1] || gate == up) {
        PKH_ERR("pico_swiglu_matmul_add: gate and up must be distinct [M, F] tensors with unit "
                "columns and one row stride!\n");
        return NULL;
    }
    const int64_t M = gate->shape[0], F = gate->shape[1];
    if(w->ndim != 2 || w->shape[0] != F || w->strides[1] != 1 || w->strides[0] < w->shape[1]) {
        PKH_ERR("pico_swiglu_matmul_add: w must be a row-contiguous [F, N] tensor!\n");
        return NULL;
    }
    const int64_t N = w->shape[1], ld = gate->strides[0];
    if(c && !residual_ok(c, M, N)) {
        PKH_ERR("pico_swiglu_matmul_add: the added tensor must be a contiguous [M, N]!\n");
        return NULL;
    }
    float* h = (float*)gate_up_h(gate, up);
    int64_t shape[2] = {M, N};
    struct PicoTensor* out = pkh_new_tensor(arena, shape, 2);
    if(!out) return NULL;
    int st;
    if(!h) {
        h = (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(M * F > 0 ? M * F : 1));
        if(!h) return NULL;
        st = pk_swiglu_fwd_f32(M, F, gate->data, ld, up->data, ld, h, F, pkh_stream());
        if(pkh_status("pico_swiglu_matmul_add", st)) return NULL;
    }
    struct PkMat vh = {h, 'N', F > 0 ? F : 1, 0},
                 vw = {w->data, 'N', w->strides[0], w->is_persistent};
    st = gemm_add_on(vh, vw, M, N, F, out->data, 'N', N > 0 ? N : 1, c ? 1.0f : 0.0f,
                     c ? c->data : NULL, c ? c->strides[0] : 0, pkh_stream(), 0);
    if(pkh_status("pico_swiglu_matmul_add", st)) return NULL;
    struct PkNode* n = pkh_node(out);
    n->saved[SM_H] = h;
    n->ival[SM_LD] = ld;
    n->ival[SM_RESID] = c != NULL;
    struct PicoTensor* ps[4] = {gate, up, w, c};
    pkh_set_parents(arena, out, c ? 4 : 3, ps, swiglu_matmul_backward);
    return out;
}

/* ----------------------------------------------------------------- unary */
/* src/ops.c:198-328 / src/autograd.h:132-176: elementwise over the flat
 * buffer, output contiguous in the input's shape */
static void unary_backward(int op, struct PicoTensor* self) {
    struct PicoTensor* a = self->parents[0];
    const float* g = pkh_upstream(self);
    if(!g) return;
    int st = pk_unary_bwd_f32(op, self->numel, a->data, self->data, g, a->grad, pkh_grad_flag(a),
                              pkh_stream());
    if(pkh_status("pico_tensor_unary_backward", st)) return;
    pkh_grad_mark(a);
}
static void sqrt_bw(struct PicoTensor* s) { unary_backward(U_SQRT, s); }
static void sin_bw(struct PicoTensor* s) { unary_backward(U_SIN, s); }
static void cos_bw(struct PicoTensor* s) { unary_backward(U_COS, s); }
static void tan_bw(struct PicoTensor* s) { unary_backward(U_TAN, s); }
static void tanh_bw(struct PicoTensor* s) { unary_backward(U_TANH, s); }
static void log_bw(struct PicoTensor* s) { unary_backward(U_LOG, s); }

static struct PicoTensor* unary_op(int op, const char* name, struct PicoTensor* a,
                                   void (*bw)(struct PicoTensor*)) {
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(!a) {
        PKH_ERR("%s: NULL tensor!\n", name);
        return NULL;
    }
    if(refuse_cpu(name, a)) return NULL;
    struct PicoTensor* out = pkh_new_tensor(arena, a->shape, a->ndim);
    if(!out) return NULL;
    if(pkh_status(name, pk_unary_f32(op, a->numel, a->data, out->data, pkh_stream())))
        return NULL;
    pkh_set_parents(arena, out, 1, &a, bw);
    return out;
}

struct PicoTensor* pico_tensor_sqrt(struct PicoTensor* a) {
    return unary_op(U_SQRT, "pico_tensor_sqrt", a, sqrt_bw);
}
struct PicoTensor* pico_tensor_sin(struct PicoTensor* a) {
    return unary_op(U_SIN, "pico_tensor_sin", a, sin_bw);
}
struct PicoTensor* pico_tensor_cos(struct PicoTensor* a) {
    return unary_op(U_COS, "pico_tensor_cos", a, cos_bw);
}
struct PicoTensor* pico_tensor_tan(struct PicoTensor* a) {
    return unary_op(U_TAN, "pico_tensor_tan", a, tan_bw);
}
struct PicoTensor* pico_tensor_tanh(struct PicoTensor* a) {
    return unary_op(U_TANH, "pico_tensor_tanh", a, tanh_bw);
}
struct PicoTensor* pico_tensor_log(struct PicoTensor* a) {
    return unary_op(U_LOG, "pico_tensor_log", a, log_bw);
}

/* ------------------------------------------------------------------ relu */
/* src/act/autograd.h:9-17: parent.grad += g * (y > 0) */
void pico_relu_backward_gpu(struct PicoTensor* self) {
    if(pkh_init()) return;
    struct PicoTensor* x = self->parents[0];
    const float* g = pkh_upstream(self);
    if(!g) return;
    int st = pk_relu_bwd_f32(x->numel, self->data, g, x->grad, pkh_grad_flag(x), pkh_stream());
    if(pkh_status("pico_relu_backward", st)) return;
    pkh_grad_mark(x);
}

/* src/act/activations.c:8-26 (the output is GPU-backed like its input; the
 * reference leaves relu's output on the CPU backend) */
struct PicoTensor* pico_relu(struct PicoTensor* x) {
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    if(!x) {
        PKH_ERR("pico_relu: NULL tensor!\n");
        return NULL;
    }
    if(refuse_cpu("pico_relu", x)) return NULL;
    struct PicoTensor* out = pkh_new_tensor(arena, x->shape, x->ndim);
    if(!out) return NULL;
    if(pkh_status("pico_relu", pk_relu_f32(x->numel, x->data, out->data, pkh_stream())))
        return NULL;
    pkh_set_parents(arena, out, 1, &x, pico_relu_backward_gpu);
    return out;
}
