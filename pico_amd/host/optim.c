/*
 * pico_amd/host/optim.c -- SGD (src/optim/SGD.c:16-52) and AdamW over GPU
 * params, and pico's Linear layer (src/nn/linear.c:9-77).
 *
 * The optimizers mutate params in place, as the reference's contract says
 * (docs/contracts/01-allocation-and-ownership.md:43-46).  zero_grad marks each
 * grad as holding nothing (it then reads as zeros and the next contribution
 * overwrites it), which is what the reference's zero-fill achieves, without
 * a pass over memory.
 */
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

struct ParamList {
    struct PicoTensor** v;
    int n, cap;
};

static int pl_push(struct ParamList* l, struct PicoTensor* t) {
    if(l->n == l->cap) {
        int cap = l->cap ? 2 * l->cap : 16;
        struct PicoTensor** nv = (struct PicoTensor**)realloc(l->v, sizeof(*nv) * cap);
        if(!nv) return -1;
        l->v = nv;
        l->cap = cap;
    }
    l->v[l->n++] = t;
    return 0;
}

static void zero_grads(struct ParamList* l) {
    for(int i = 0; i < l->n; i++) {
        struct PkNode* n = pkh_node(l->v[i]);
        if(n) n->grad_live = 0;
    }
}

/* ----------------------------------------------------------------- SGD */
struct PicoOptimSGD {
    struct ParamList params;
    float lr;
};

struct PicoOptimSGD* pico_optim_sgd_init(float lr) {
    struct PicoOptimSGD* o = (struct PicoOptimSGD*)calloc(1, sizeof(*o));
    if(o) o->lr = lr;
    return o;
}

void pico_optim_sgd_add(struct PicoOptimSGD* o, struct PicoTensor* p) {
    if(!o || !p) return;
    if(!pkh_node(p) || !pkh_is_gpu(p)) {
        PKH_ERR("SGD: param is not a GPU tensor of this library!\n");
        return;
    }
    pl_push(&o->params, p);
}

/* p -= lr * g (src/optim/SGD.c:29-37) for every param in one launch; a grad
 * holding nothing is zero, and p - lr*0 == p, so such params are skipped */
void pico_optim_sgd_step(struct PicoOptimSGD* o) {
    enum { BATCH = 32 };
    float* ps[BATCH];
    const float* gs[BATCH];
    int64_t ns[BATCH];
    int k = 0;
    for(int i = 0; i <= o->params.n; i++) {
        if(i < o->params.n) {
            struct PicoTensor* p = o->params.v[i];
            if(!pkh_grad_is_live(p)) continue;
            ps[k] = p->data;
            gs[k] = p->grad;
            ns[k] = p->numel;
            k++;
        }
        if(k == BATCH || (i == o->params.n && k > 0)) {
            pkh_status("pico_optim_sgd_step", pk_sgd_multi_f32(k, ps, gs, ns, o->lr, pkh_stream()));
            k = 0;
        }
    }
    pkh_params_changed();
}

void pico_optim_sgd_zero_grad(struct PicoOptimSGD* o) { zero_grads(&o->params); }

void pico_optim_sgd_free(struct PicoOptimSGD* o) {
    if(!o) return;
    free(o->params.v);
    free(o);
}

/* --------------------------------------------------------------- AdamW */
/*
 * One step is two launches whatever the number of params: a one-thread
 * kernel advances the step counter held in device memory and writes the two
 * bias corrections, then one multi-tensor kernel updates every param, one
 * workgroup per chunk of up to PK_ADAMW_CHUNK elements.  Nothing in the
 * launches changes between steps, so a step can be captured in a graph and
 * replayed.  The chunk table lives in device memory and is rebuilt (a
 * synchronous upload) only when the params or the set of params holding a
 * gradient change.
 */
struct PicoOptimAdamW {
    struct ParamList params;
    float** m; /* device moment buffers, one allocation per param (m then v) */
    float lr, beta1, beta2, eps, wd;
    int t;
    void* state;          /* device: int32 step count, then 2 floats of coefficients */
    PkAdamwChunk* table;  /* device chunk table */
    int64_t nchunks, table_cap;
    unsigned char* built; /* per param: 1 + grad_live when the table was built, 0 = stale */
    int built_n;
};

struct PicoOptimAdamW* pico_optim_adamw_init(float lr, float beta1, float beta2, float eps,
                                             float weight_decay) {
    struct PicoOptimAdamW* o = (struct PicoOptimAdamW*)calloc(1, sizeof(*o));
    if(!o) return NULL;
    o->lr = lr;
    o->beta1 = beta1;
    o->beta2 = beta2;
    o->eps = eps;
    o->wd = weight_decay;
    o->state = pkh_device_alloc(256);
    if(!o->state) {
        free(o);
        return NULL;
    }
    /* step count 0 and zero coefficients: all-zero bits */
    pkh_status("pico_optim_adamw_init", pk_fill_f32(3, 0.0f, (float*)o->state, pkh_stream()));
    return o;
}

void pico_optim_adamw_add(struct PicoOptimAdamW* o, struct PicoTensor* p) {
    if(!o || !p) return;
    if(!pkh_node(p) || !pkh_is_gpu(p)) {
        PKH_ERR("AdamW: param is not a GPU tensor of this library!\n");
        return;
    }
    if(pl_push(&o->params, p)) return;
    float** nm = (float**)realloc(o->m, sizeof(float*) * o->params.cap);
    if(!nm) return;
    o->m = nm;
    size_t half = ((size_t)p->numel * sizeof(float) + 255) & ~(size_t)255;
    float* buf = (float*)pkh_device_alloc(2 * (half ? half : 256));
    o->m[o->params.n - 1] = buf;
    if(buf)
        pkh_status("pico_optim_adamw_add",
                   pk_fill_f32((int64_t)(2 * half / sizeof(float)), 0.0f, buf, pkh_stream()));
}

/* the chunk table for the current params and their gradient state */
static int adamw_table(struct PicoOptimAdamW* o) {
    const int n = o->params.n;
    int stale = o->built_n != n || !o->built;
    for(int i = 0; i < n && !stale; i++)
        stale = o->built[i] != (unsigned char)(1 + (pkh_grad_is_live(o->params.v[i]) ? 1 : 0));
    if(!stale) return 0;
    int64_t count = 0;
    for(int i = 0; i < n; i++)
        if(o->m[i]) count += (o->params.v[i]->numel + PK_ADAMW_CHUNK - 1) / PK_ADAMW_CHUNK;
    PkAdamwChunk* h = (PkAdamwChunk*)malloc(sizeof(PkAdamwChunk) * (size_t)(count ? count : 1));
    unsigned char* built = (unsigned char*)realloc(o->built, (size_t)(n > 0 ? n : 1));
    if(!h || !built) {
        free(h);
        if(built) o->built = built;
        pkh_set_error("AdamW: out of host memory");
        return -1;
    }
    o->built = built;
    int64_t c = 0;
    for(int i = 0; i < n; i++) {
        struct PicoTensor* p = o->params.v[i];
        const int live = pkh_grad_is_live(p);
        built[i] = (unsigned char)(1 + (live ? 1 : 0));
        float* m = o->m[i];
        if(!m) continue;
        size_t half = ((size_t)p->numel * sizeof(float) + 255) & ~(size_t)255;
        float* v = (float*)((unsigned char*)m + half);
        for(int64_t off = 0; off < p->numel; off += PK_ADAMW_CHUNK, c++) {
            h[c].p = p->data + off;
            h[c].g = live ? p->grad + off : NULL;
            h[c].m = m + off;
            h[c].v = v + off;
            h[c].n = p->numel - off < PK_ADAMW_CHUNK ? p->numel - off : PK_ADAMW_CHUNK;
        }
    }
    int rc = 0;
    if(count > o->table_cap) {
        if(o->table) {
            pkh_sync();
            pkh_device_free(o->table);
        }
        o->table = (PkAdamwChunk*)pkh_device_alloc(sizeof(PkAdamwChunk) * (size_t)count);
        o->table_cap = o->table ? count : 0;
        if(!o->table) rc = -1;
    }
    if(rc == 0 && count > 0) rc = pkh_copy_h2d(o->table, h, sizeof(PkAdamwChunk) * (size_t)count);
    free(h);
    o->nchunks = rc == 0 ? count : 0;
    o->built_n = rc == 0 ? n : -1;
    return rc;
}

void pico_optim_adamw_step(struct PicoOptimAdamW* o) {
    if(!o) return;
    pkh_side_join(); /* the grads are read on the main stream */
    if(adamw_table(o)) return; /* the failing call recorded the error */
    o->t++;
    int32_t* step = (int32_t*)o->state;
    float* coef = (float*)o->state + 1;
    if(pkh_status("pico_optim_adamw_step",
                  pk_adamw_prep_f32(step, o->lr, o->beta1, o->beta2, coef, pkh_stream())))
        return;
    pkh_status("pico_optim_adamw_step",
               pk_adamw_multi_f32(o->nchunks, o->table, o->lr, o->beta1, o->beta2, o->eps, o->wd,
                                  coef, pkh_stream()));
    pkh_params_changed();
}

void pico_optim_adamw_zero_grad(struct PicoOptimAdamW* o) { zero_grads(&o->params); }

/* ---- state access for checkpoints ---- */
int pkh_adamw_moments(const struct PicoOptimAdamW* o, const struct PicoTensor* p, float** m,
                      float** v) {
    for(int i = 0; i < o->params.n; i++) {
        if(o->params.v[i] != p || !o->m[i]) continue;
        size_t half = ((size_t)p->numel * sizeof(float) + 255) & ~(size_t)255;
        *m = o->m[i];
        *v = (float*)((unsigned char*)o->m[i] + half);
        return 1;
    }
    return 0;
}

/* the device's step count is authoritative (graph replays advance only it) */
int pkh_adamw_sync_step(struct PicoOptimAdamW* o) {
    int32_t t = 0;
    if(pkh_copy_d2h(&t, o->state, sizeof(t))) return -1;
    o->t = t;
    return 0;
}

int pkh_adamw_step(const struct PicoOptimAdamW* o) { return o->t; }

int pkh_adamw_set_step(struct PicoOptimAdamW* o, int step) {
    int32_t t = step;
    if(step < 0) {
        pkh_set_error("AdamW: negative step count %d", step);
        return PK_EINVAL;
    }
    if(pkh_copy_h2d(o->state, &t, sizeof(t))) return PK_EINVAL;
    o->t = step;
    return 0;
}

void pkh_adamw_hparams(const struct PicoOptimAdamW* o, float* lr, float* b1, float* b2,
                       float* eps, float* wd) {
    *lr = o->lr;
    *b1 = o->beta1;
    *b2 = o->beta2;
    *eps = o->eps;
    *wd = o->wd;
}

void pico_optim_adamw_free(struct PicoOptimAdamW* o) {
    if(!o) return;
    pkh_sync();
    for(int i = 0; i < o->params.n; i++) pkh_device_free(o->m[i]);
    pkh_device_free(o->table);
    pkh_device_free(o->state);
    free(o->built);
    free(o->m);
    free(o->params.v);
    free(o);
}

/* -------------------------------------------------------------- Linear */
/* src/nn/linear.c:9-38: W [in, out] and b [out], both zero-initialised */
struct PicoLinear* pico_nn_linear_init(int in_features, int out_features, bool bias) {
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    int64_t wshape[2] = {in_features, out_features};
    int64_t bshape[1] = {out_features};
    struct PicoTensor* w = pico_param(wshape, 2);
    struct PicoTensor* b = bias ? pico_param(bshape, 1) : NULL;
    struct PicoLinear* l = (struct PicoLinear*)malloc(sizeof(*l));
    if(!l || !w || (bias && !b)) {
        pico_free(w);
        pico_free(b);
        free(l);
        return NULL;
    }
    l->weights = w;
    l->bias = b;
    l->in_features = in_features;
    l->out_features = out_features;
    return l;
}

/* src/nn/linear.c:40-67: x . W, then + b broadcast over rows, as one node
 * whose product adds the bias in its epilogue (pkh_linear) */
struct PicoTensor* pico_nn_linear_forward(struct PicoLinear* layer, struct PicoTensor* input) {
    if(!layer || !input) {
        PKH_ERR("In Linear - NULL layer or input!\n");
        return NULL;
    }
    if(input->shape[input->ndim - 1] != layer->weights->shape[0]) {
        PKH_ERR(" In Linear - 2 matmuls matrices must be compatible\n");
        return NULL;
    }
    if(layer->weights->backend != input->backend) {
        PKH_ERR("In Linear - PicoTensor backends are not compatible!\n");
        return NULL;
    }
    if(!arena_ctx_current()) {
        PKH_ERR("In Linear - No current arena in context!\n");
        return NULL;
    }
    if(layer->bias) return pkh_linear(input, layer->weights, layer->bias);
    return pico_matmul(input, layer->weights);
}

void pico_nn_linear_free(struct PicoLinear* l) {
    if(!l) return;
    pico_free(l->weights);
    pico_free(l->bias);
    free(l);
}
