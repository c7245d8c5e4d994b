/*
 * oracle/ora_ops.c -- CPU oracle (test infrastructure): pico's op layer,
 * autograd hooks, relu, Linear and SGD restated, plus AdamW.
 *
 * Op template (src/ops.c:12-54): validate -> arena of the current context ->
 * output tensor (zeroed) -> CPU kernel -> wire parents and _backward.
 * Validation failures print "[Pico] Error: ..." and return NULL.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ora.h"
#include "ora_internal.h"

static struct Arena* need_arena(void) {
    struct Arena* ar = arena_ctx_current();
    if(!ar) fprintf(stderr, "[Pico] Error: No current arena in context!\n");
    return ar;
}

static void wire(struct Arena* ar, struct PicoTensor* out, struct PicoTensor* a,
                 struct PicoTensor* b, void (*bw)(struct PicoTensor*)) {
    int n = b ? 2 : 1;
    out->parents = (struct PicoTensor**)arena_alloc(ar, sizeof(struct PicoTensor*) * n);
    out->parents[0] = a;
    if(b) out->parents[1] = b;
    out->num_parents = (uint8_t)n;
    out->_backward = bw;
}

/* ----------------------------------------------------------- binary ops */
enum { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2 };

static inline float bin_apply(int op, float x, float y) {
    switch(op) {
        case OP_ADD: return x + y;
        case OP_SUB: return x - y;
        default: return x * y;
    }
}

/* src/kernels/cpu/cpu_scalar.h:12-30 and cpu_avx_2.h:15-42 (same-shape fast path
 * gives the same bits: each element is one rounding of a op b) */
static void k_binary(int op, const struct PicoTensor* a, const struct PicoTensor* b,
                     struct PicoTensor* out) {
    for(int64_t i = 0; i < out->numel; i++) {
        int64_t ia = ora_map_index(i, a->shape, a->strides, a->ndim, out->strides, out->ndim);
        int64_t ib = ora_map_index(i, b->shape, b->strides, b->ndim, out->strides, out->ndim);
        out->data[i] = bin_apply(op, a->data[ia], b->data[ib]);
    }
}

/* src/autograd.h:53-94: one pass over the output, += into each parent's grad
 * at the broadcast source index (so stretched dims are summed in index order) */
static void k_binary_bwd(int op, struct PicoTensor* self) {
    struct PicoTensor *a = self->parents[0], *b = self->parents[1];
    for(int64_t i = 0; i < self->numel; i++) {
        int64_t ia = ora_map_index(i, a->shape, a->strides, a->ndim, self->strides, self->ndim);
        int64_t ib = ora_map_index(i, b->shape, b->strides, b->ndim, self->strides, self->ndim);
        float g = self->grad[i];
        switch(op) {
            case OP_ADD:
                a->grad[ia] += g;
                b->grad[ib] += g;
                break;
            case OP_SUB:
                a->grad[ia] += g;
                b->grad[ib] -= g;
                break;
            default: {
                float ga = g * b->data[ib];
                a->grad[ia] += ga;
                float gb = g * a->data[ia];
                b->grad[ib] += gb;
            }
        }
    }
}
static void add_bw(struct PicoTensor* s) { k_binary_bwd(OP_ADD, s); }
static void sub_bw(struct PicoTensor* s) { k_binary_bwd(OP_SUB, s); }
static void mul_bw(struct PicoTensor* s) { k_binary_bwd(OP_MUL, s); }

static struct PicoTensor* binary_op(int op, struct PicoTensor* a, struct PicoTensor* b) {
    if(!pico_check_broadcast_compatibility(a, b)) {
        fprintf(stderr, "[Pico] Error: Shapes are not broadcastable!\n");
        return NULL;
    }
    if(a->backend != b->backend) {
        fprintf(stderr, "[Pico] Error: PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    int nd = ORA_MAX(a->ndim, b->ndim);
    int64_t shape[16];
    for(int d = 0; d < nd; d++) {
        int da = d - (nd - a->ndim), db = d - (nd - b->ndim);
        int64_t sa = da >= 0 ? a->shape[da] : 1, sb = db >= 0 ? b->shape[db] : 1;
        shape[d] = ORA_MAX(sa, sb);
    }
    struct PicoTensor* out = pico_create_tensor(ar, shape, (uint8_t)nd);
    out->backend = a->backend;
    k_binary(op, a, b, out);
    wire(ar, out, a, b, op == OP_ADD ? add_bw : op == OP_SUB ? sub_bw : mul_bw);
    return out;
}
struct PicoTensor* pico_add(struct PicoTensor* a, struct PicoTensor* b) { return binary_op(OP_ADD, a, b); }
struct PicoTensor* pico_sub(struct PicoTensor* a, struct PicoTensor* b) { return binary_op(OP_SUB, a, b); }
struct PicoTensor* pico_mul(struct PicoTensor* a, struct PicoTensor* b) { return binary_op(OP_MUL, a, b); }

/* ----------------------------------------------------------------- matmul */
static void matmul_bw(struct PicoTensor* s) { ora_k_matmul_backward(s); }

struct PicoTensor* pico_matmul(struct PicoTensor* a, struct PicoTensor* b) {
    /* src/ops.c:144-190: inner dims checked first, then 2-D, then backend */
    if(a->shape[a->ndim - 1] != b->shape[0]) {
        fprintf(stderr, "[Pico] Error: 2 matmuls matrices must be compatible\n");
        return NULL;
    }
    if(a->ndim != 2 || b->ndim != 2) {
        fprintf(stderr, "[Pico] Error: 2d matmul matrices must be compatible\n");
        return NULL;
    }
    if(a->backend != b->backend) {
        fprintf(stderr, "[Pico] Error: PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    int64_t shape[2] = {a->shape[0], b->shape[1]};
    struct PicoTensor* out = pico_create_tensor(ar, shape, 2);
    out->backend = a->backend;
    /* dispatch of src/kernels/cpu_kernels.h:46-55: only SIMD_AVX takes the AVX path */
    if(g_simd_level == SIMD_AVX)
        ora_k_matmul_avx(a, b, out);
    else
        ora_k_matmul_scalar(a, b, out);
    wire(ar, out, a, b, matmul_bw);
    return out;
}

/* ------------------------------------------------------------------ unary */
enum { U_SQRT = 0, U_SIN, U_COS, U_TAN, U_TANH, U_LOG };

/* src/kernels/cpu/cpu_scalar.h:32-37: sqrtf/logf in float; sin/cos/tan/tanh
 * through the double libm routines, narrowed on store */
static inline float un_apply(int op, float x) {
    switch(op) {
        case U_SQRT: return sqrtf(x);
        case U_SIN: return (float)sin((double)x);
        case U_COS: return (float)cos((double)x);
        case U_TAN: return (float)tan((double)x);
        case U_TANH: return (float)tanh((double)x);
        default: return logf(x);
    }
}

/* src/autograd.h:132-176, with the reference's evaluation types:
 *   sqrt: g * (1 / (2*y))                    float
 *   sin:  grad + g*cos(x)                    double, narrowed
 *   cos:  grad - g*sin(x)                    double, narrowed
 *   tan:  g * powf((float)sec(x), 2)         float
 *   tanh: g*1 - y*y   (the reference omits the parentheses around 1 - y^2)
 *   log:  (g*1) / x                          float                              */
static inline float un_bwd_apply(int op, float gx, float x, float y, float g) {
    switch(op) {
        case U_SQRT: return gx + g * (1.0f / (2.0f * y));
        case U_SIN: return (float)((double)gx + (double)g * cos((double)x));
        case U_COS: return (float)((double)gx - (double)g * sin((double)x));
        case U_TAN: {
            float sec = (float)(1.0 / cos((double)x));
            return gx + g * powf(sec, 2.0f);
        }
        case U_TANH: {
            float yy = powf(y, 2.0f);
            return gx + (g * 1.0f - yy);
        }
        default: return gx + g * 1.0f / x;
    }
}

static void unary_bw_common(struct PicoTensor* s, int op) {
    struct PicoTensor* a = s->parents[0];
    for(int64_t i = 0; i < s->numel; i++)
        a->grad[i] = un_bwd_apply(op, a->grad[i], a->data[i], s->data[i], s->grad[i]);
}
static void sqrt_bw(struct PicoTensor* s) { unary_bw_common(s, U_SQRT); }
static void sin_bw(struct PicoTensor* s) { unary_bw_common(s, U_SIN); }
static void cos_bw(struct PicoTensor* s) { unary_bw_common(s, U_COS); }
static void tan_bw(struct PicoTensor* s) { unary_bw_common(s, U_TAN); }
static void tanh_bw(struct PicoTensor* s) { unary_bw_common(s, U_TANH); }
static void log_bw(struct PicoTensor* s) { unary_bw_common(s, U_LOG); }

static struct PicoTensor* unary_op(int op, struct PicoTensor* a) {
    static void (*const bws[6])(struct PicoTensor*) = {sqrt_bw, sin_bw, cos_bw,
                                                       tan_bw,  tanh_bw, log_bw};
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    struct PicoTensor* out = pico_create_tensor(ar, a->shape, a->ndim);
    out->backend = a->backend;
    for(int64_t i = 0; i < out->numel; i++) out->data[i] = un_apply(op, a->data[i]);
    wire(ar, out, a, NULL, bws[op]);
    return out;
}
struct PicoTensor* pico_tensor_sqrt(struct PicoTensor* a) { return unary_op(U_SQRT, a); }
struct PicoTensor* pico_tensor_sin(struct PicoTensor* a) { return unary_op(U_SIN, a); }
struct PicoTensor* pico_tensor_cos(struct PicoTensor* a) { return unary_op(U_COS, a); }
struct PicoTensor* pico_tensor_tan(struct PicoTensor* a) { return unary_op(U_TAN, a); }
struct PicoTensor* pico_tensor_tanh(struct PicoTensor* a) { return unary_op(U_TANH, a); }
struct PicoTensor* pico_tensor_log(struct PicoTensor* a) { return unary_op(U_LOG, a); }

/* ------------------------------------------------------------------- relu */
/* src/act/activations.c:8-26: y = MAX(x, 0) (NaN and -0 map to +0);
 * src/act/autograd.h:9-17: grad += g * (y > 0) */
static inline float relu_f(float x) { return x > 0.0f ? x : 0.0f; }
static void relu_bw(struct PicoTensor* s) {
    struct PicoTensor* p = s->parents[0];
    for(int64_t i = 0; i < p->numel; i++) {
        float gate = (float)(s->data[i] > 0.0f);
        p->grad[i] += s->grad[i] * gate;
    }
}
struct PicoTensor* pico_relu(struct PicoTensor* x) {
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    struct PicoTensor* out = pico_create_tensor(ar, x->shape, x->ndim);
    for(int64_t i = 0; i < x->numel; i++) out->data[i] = relu_f(x->data[i]);
    wire(ar, out, x, NULL, relu_bw);
    return out;
}

/* ----------------------------------------------------------------- Linear */
struct PicoLinear* pico_nn_linear_init(int in_features, int out_features, bool bias) {
    /* src/nn/linear.c:9-38: W [in,out] and b [out], zero-filled params */
    int64_t ws[2] = {in_features, out_features}, bs[1] = {out_features};
    struct PicoLinear* l = (struct PicoLinear*)malloc(sizeof(*l));
    l->in_features = in_features;
    l->out_features = out_features;
    l->weights = pico_param(ws, 2);
    l->bias = bias ? pico_param(bs, 1) : NULL;
    return l;
}
struct PicoTensor* pico_nn_linear_forward(struct PicoLinear* layer, struct PicoTensor* input) {
    /* src/nn/linear.c:40-67 */
    if(input->shape[input->ndim - 1] != layer->weights->shape[0]) {
        fprintf(stderr, "[Pico] Error:  In Linear - 2 matmuls matrices must be compatible\n");
        return NULL;
    }
    if(layer->weights->backend != input->backend) {
        fprintf(stderr, "[Pico] Error: In Linear - PicoTensor backends are not compatible!\n");
        return NULL;
    }
    struct PicoTensor* out = pico_matmul(input, layer->weights);
    if(out && layer->bias) out = pico_add(out, layer->bias);
    return out;
}
void pico_nn_linear_free(struct PicoLinear* l) {
    if(!l) return;
    pico_free(l->weights);
    pico_free(l->bias);
    free(l);
}

/* -------------------------------------------------------------------- SGD */
struct ParamList {
    struct PicoTensor** v;
    int n, cap;
};
static void pl_push(struct ParamList* l, struct PicoTensor* t) {
    if(l->n == l->cap) {
        l->cap = l->cap ? 2 * l->cap : 16;
        l->v = (struct PicoTensor**)realloc(l->v, l->cap * sizeof(*l->v));
    }
    l->v[l->n++] = t;
}

struct PicoOptimSGD {
    struct ParamList params;
    float lr;
};
struct PicoOptimSGD* pico_optim_sgd_init(float lr) {
    struct PicoOptimSGD* o = (struct PicoOptimSGD*)calloc(1, sizeof(*o));
    o->lr = lr;
    return o;
}
void pico_optim_sgd_add(struct PicoOptimSGD* o, struct PicoTensor* p) { pl_push(&o->params, p); }
void ora_sgd(int64_t n, float lr, float* p, const float* g) {
    /* src/optim/SGD.c:29-37: p -= lr*g, product rounded before the subtract */
    for(int64_t j = 0; j < n; j++) {
        float step = lr * g[j];
        p[j] -= step;
    }
}
void pico_optim_sgd_step(struct PicoOptimSGD* o) {
    for(int i = 0; i < o->params.n; i++)
        ora_sgd(o->params.v[i]->numel, o->lr, o->params.v[i]->data, o->params.v[i]->grad);
}
void pico_optim_sgd_zero_grad(struct PicoOptimSGD* o) {
    for(int i = 0; i < o->params.n; i++)
        memset(o->params.v[i]->grad, 0, sizeof(float) * o->params.v[i]->numel);
}
void pico_optim_sgd_free(struct PicoOptimSGD* o) {
    free(o->params.v);
    free(o);
}

/* ------------------------------------------------------------------ AdamW
 * No reference code (src/optim/optim.h:19-23 is a placeholder).  Decoupled
 * weight decay, bias-corrected moments:
 *   p <- p*(1 - lr*wd);  m <- b1*m + (1-b1)*g;  v <- b2*v + (1-b2)*g*g
 *   p <- p - (lr/(1-b1^t)) * m / (sqrt(v)/sqrt(1-b2^t) + eps)           */
void ora_adamw(int64_t n, float lr, float beta1, float beta2, float eps, float wd, int step,
               float* p, const float* g, float* m, float* v) {
    double bc1 = 1.0 - pow((double)beta1, (double)step);
    double bc2 = 1.0 - pow((double)beta2, (double)step);
    float step_size = (float)((double)lr / bc1);
    float bc2_sqrt = (float)sqrt(bc2);
    float decay = 1.0f - lr * wd;
    for(int64_t j = 0; j < n; j++) {
        float gj = g ? g[j] : 0.0f;
        float pj = p[j] * decay;
        float mj = beta1 * m[j] + (1.0f - beta1) * gj;
        float vj = beta2 * v[j] + (1.0f - beta2) * gj * gj;
        float denom = sqrtf(vj) / bc2_sqrt + eps;
        p[j] = pj - step_size * (mj / denom);
        m[j] = mj;
        v[j] = vj;
    }
}

struct PicoOptimAdamW {
    struct ParamList params;
    float **m, **v;
    float lr, beta1, beta2, eps, wd;
    int t;
};
struct PicoOptimAdamW* pico_optim_adamw_init(float lr, float beta1, float beta2, float eps,
                                             float weight_decay) {
    struct PicoOptimAdamW* o = (struct PicoOptimAdamW*)calloc(1, sizeof(*o));
    o->lr = lr;
    o->beta1 = beta1;
    o->beta2 = beta2;
    o->eps = eps;
    o->wd = weight_decay;
    return o;
}
void pico_optim_adamw_add(struct PicoOptimAdamW* o, struct PicoTensor* p) {
    pl_push(&o->params, p);
    o->m = (float**)realloc(o->m, o->params.cap * sizeof(float*));
    o->v = (float**)realloc(o->v, o->params.cap * sizeof(float*));
    o->m[o->params.n - 1] = (float*)calloc((size_t)p->numel, sizeof(float));
    o->v[o->params.n - 1] = (float*)calloc((size_t)p->numel, sizeof(float));
}
void pico_optim_adamw_step(struct PicoOptimAdamW* o) {
    o->t++;
    for(int i = 0; i < o->params.n; i++) {
        struct PicoTensor* p = o->params.v[i];
        ora_adamw(p->numel, o->lr, o->beta1, o->beta2, o->eps, o->wd, o->t, p->data, p->grad,
                  o->m[i], o->v[i]);
    }
}
void pico_optim_adamw_zero_grad(struct PicoOptimAdamW* o) {
    for(int i = 0; i < o->params.n; i++)
        memset(o->params.v[i]->grad, 0, sizeof(float) * o->params.v[i]->numel);
}
void pico_optim_adamw_free(struct PicoOptimAdamW* o) {
    for(int i = 0; i < o->params.n; i++) {
        free(o->m[i]);
        free(o->v[i]);
    }
    free(o->m);
    free(o->v);
    free(o->params.v);
    free(o);
}

/* ------------------------------------------------------ flat entry points */
static void fill_view(struct PicoTensor* t, int64_t* shape, int64_t* strides, int ndim,
                      const float* data) {
    memset(t, 0, sizeof(*t));
    t->shape = shape;
    t->strides = strides;
    t->ndim = (uint8_t)ndim;
    t->data = (float*)data;
    ora_contig_strides(shape, ndim, strides);
    t->numel = 1;
    for(int d = 0; d < ndim; d++) t->numel *= shape[d];
}

void ora_binary(int op, int ndim, const int64_t* out_shape, const float* a, int a_ndim,
                const int64_t* a_shape, const float* b, int b_ndim, const int64_t* b_shape,
                float* out) {
    int64_t os[16], ost[16], as[16], ast[16], bs[16], bst[16];
    struct PicoTensor ta, tb, to;
    memcpy(os, out_shape, ndim * sizeof(int64_t));
    memcpy(as, a_shape, a_ndim * sizeof(int64_t));
    memcpy(bs, b_shape, b_ndim * sizeof(int64_t));
    fill_view(&ta, as, ast, a_ndim, a);
    fill_view(&tb, bs, bst, b_ndim, b);
    fill_view(&to, os, ost, ndim, out);
    k_binary(op, &ta, &tb, &to);
}

void ora_binary_bwd(int op, int ndim, const int64_t* out_shape, const float* a, int a_ndim,
                    const int64_t* a_shape, const float* b, int b_ndim, const int64_t* b_shape,
                    const float* gout, float* ga, float* gb) {
    int64_t os[16], ost[16], as[16], ast[16], bs[16], bst[16];
    struct PicoTensor ta, tb, to;
    memcpy(os, out_shape, ndim * sizeof(int64_t));
    memcpy(as, a_shape, a_ndim * sizeof(int64_t));
    memcpy(bs, b_shape, b_ndim * sizeof(int64_t));
    fill_view(&ta, as, ast, a_ndim, a);
    fill_view(&tb, bs, bst, b_ndim, b);
    fill_view(&to, os, ost, ndim, NULL);
    ta.grad = ga;
    tb.grad = gb;
    to.grad = (float*)gout;
    struct PicoTensor* parents[2] = {&ta, &tb};
    to.parents = parents;
    to.num_parents = 2;
    k_binary_bwd(op, &to);
}

void ora_unary(int op, int64_t n, const float* x, float* y) {
    for(int64_t i = 0; i < n; i++) y[i] = un_apply(op, x[i]);
}
void ora_unary_bwd(int op, int64_t n, const float* x, const float* y, const float* gy, float* gx) {
    for(int64_t i = 0; i < n; i++) gx[i] = un_bwd_apply(op, gx[i], x[i], y[i], gy[i]);
}
void ora_relu(int64_t n, const float* x, float* y) {
    for(int64_t i = 0; i < n; i++) y[i] = relu_f(x[i]);
}
void ora_relu_bwd(int64_t n, const float* y, const float* gy, float* gx) {
    for(int64_t i = 0; i < n; i++) {
        float gate = (float)(y[i] > 0.0f);
        gx[i] += gy[i] * gate;
    }
}
