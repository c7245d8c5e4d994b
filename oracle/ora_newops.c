/*
 * oracle/ora_newops.c -- CPU oracle (test infrastructure) for the hot-path ops
 * the reference does not implement: fused softmax cross-entropy, RMSNorm,
 * SwiGLU, causal attention, embedding, argmax.
 *
 * No reference implementation exists for these (the only trace is the softmax
 * Jacobian comment at src/autograd.h:38-40 and the plan at todo.md:95), so they
 * are written from their mathematical definitions, accumulate in double, and
 * are pinned in tests/ by torch-CPU golden vectors, closed forms and central
 * finite differences.  The pico-style ops follow the op template of
 * src/ops.c:12-54 and the += backward contract of src/autograd.h:25-29.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ora.h"
#include "ora_internal.h"

/* ------------------------------------------------------------ flat kernels */
void ora_xent_fwd_bwd(int64_t R, int64_t V, const float* logits, const int32_t* labels,
                      float* loss_rows, float* dlogits, float scale) {
    /* loss_r = logsumexp(z_r) - z_r[y_r];  dz_r = scale * (softmax(z_r) - onehot(y_r)).
     * A label outside [0, V) gives loss NaN and a zero gradient row. */
    for(int64_t r = 0; r < R; r++) {
        const float* z = logits + r * V;
        int32_t y = labels[r];
        double m = -INFINITY;
        for(int64_t j = 0; j < V; j++) m = z[j] > m ? z[j] : m;
        double s = 0.0;
        for(int64_t j = 0; j < V; j++) s += exp((double)z[j] - m);
        double lse = m + log(s);
        int ok = y >= 0 && y < V;
        if(loss_rows) loss_rows[r] = ok ? (float)(lse - (double)z[y]) : NAN;
        if(dlogits) {
            float* dz = dlogits + r * V;
            for(int64_t j = 0; j < V; j++) {
                double p = exp((double)z[j] - lse);
                dz[j] = ok ? (float)((double)scale * (p - (j == y ? 1.0 : 0.0))) : 0.0f;
            }
        }
    }
}

void ora_argmax(int64_t R, int64_t V, const float* x, int32_t* idx) {
    /* first maximum wins; a NaN counts as the maximum (first NaN wins) */
    for(int64_t r = 0; r < R; r++) {
        const float* z = x + r * V;
        int64_t best = 0;
        float bv = z[0];
        for(int64_t j = 1; j < V; j++) {
            if(isnan(bv)) break;
            if(isnan(z[j]) || z[j] > bv) {
                bv = z[j];
                best = j;
            }
        }
        idx[r] = (int32_t)best;
    }
}

void ora_rmsnorm_fwd(int64_t R, int64_t C, float eps, const float* x, const float* g, float* y,
                     float* rstd) {
    /* y = x * rstd * g,  rstd = 1/sqrt(mean(x^2) + eps) */
    for(int64_t r = 0; r < R; r++) {
        const float* xr = x + r * C;
        double ss = 0.0;
        for(int64_t c = 0; c < C; c++) ss += (double)xr[c] * xr[c];
        double rs = 1.0 / sqrt(ss / (double)C + (double)eps);
        if(rstd) rstd[r] = (float)rs;
        for(int64_t c = 0; c < C; c++) y[r * C + c] = (float)((double)xr[c] * rs * g[c]);
    }
}

void ora_rmsnorm_bwd(int64_t R, int64_t C, const float* x, const float* g, const float* rstd,
                     const float* dy, float* dx, float* dg) {
    /* dx += rstd*(g*dy) - x*rstd^3*mean(g*dy*x);  dg += sum_r dy*x*rstd.
     * rstd is the saved forward value (float), as the GPU path reads it. */
    double* dga = dg ? (double*)calloc((size_t)C, sizeof(double)) : NULL;
    for(int64_t r = 0; r < R; r++) {
        const float *xr = x + r * C, *dyr = dy + r * C;
        double rs = rstd[r];
        double dot = 0.0;
        for(int64_t c = 0; c < C; c++) dot += (double)g[c] * dyr[c] * xr[c];
        double k = rs * rs * rs * dot / (double)C;
        if(dx)
            for(int64_t c = 0; c < C; c++)
                dx[r * C + c] += (float)(rs * g[c] * dyr[c] - (double)xr[c] * k);
        if(dga)
            for(int64_t c = 0; c < C; c++) dga[c] += (double)dyr[c] * xr[c] * rs;
    }
    if(dga) {
        for(int64_t c = 0; c < C; c++) dg[c] += (float)dga[c];
        free(dga);
    }
}

void ora_swiglu_fwd(int64_t n, const float* a, const float* u, float* h) {
    /* h = silu(a) * u,  silu(a) = a * sigmoid(a) */
    for(int64_t i = 0; i < n; i++) {
        double s = 1.0 / (1.0 + exp(-(double)a[i]));
        h[i] = (float)((double)a[i] * s * u[i]);
    }
}

void ora_swiglu_bwd(int64_t n, const float* a, const float* u, const float* dh, float* da,
                    float* du) {
    /* da += dh*u*s*(1 + a*(1-s));  du += dh*a*s   (s = sigmoid(a)) */
    for(int64_t i = 0; i < n; i++) {
        double s = 1.0 / (1.0 + exp(-(double)a[i]));
        double av = a[i];
        if(da) da[i] += (float)((double)dh[i] * u[i] * s * (1.0 + av * (1.0 - s)));
        if(du) du[i] += (float)((double)dh[i] * av * s);
    }
}

/* q, k, v, o are token-major [B*T, H*hd]; head h of batch b owns columns
 * h*hd .. h*hd+hd-1 of rows b*T .. b*T+T-1.  lse is [B*H, T]. */
struct AttnCtx {
    int B, H, T, hd;
    float scale;
    const float *q, *k, *v, *o, *lse, *dout;
    float *out, *lse_out, *dq, *dk, *dv;
};

static void attn_fwd_heads(void* p, int64_t lo, int64_t hi) {
    struct AttnCtx* c = (struct AttnCtx*)p;
    const int T = c->T, hd = c->hd, D = c->H * c->hd;
    double* s = (double*)malloc(sizeof(double) * T);
    double* acc = (double*)malloc(sizeof(double) * hd);
    for(int64_t bh = lo; bh < hi; bh++) {
        int64_t b = bh / c->H, h = bh % c->H;
        const float* Q = c->q + b * T * D + h * hd;
        const float* K = c->k + b * T * D + h * hd;
        const float* Vv = c->v + b * T * D + h * hd;
        float* O = c->out + b * T * D + h * hd;
        for(int i = 0; i < T; i++) {
            double m = -INFINITY;
            for(int j = 0; j <= i; j++) {
                double d = 0.0;
                for(int e = 0; e < hd; e++) d += (double)Q[i * D + e] * K[j * D + e];
                s[j] = d * c->scale;
                m = s[j] > m ? s[j] : m;
            }
            double sum = 0.0;
            for(int j = 0; j <= i; j++) sum += exp(s[j] - m);
            double lse = m + log(sum);
            if(c->lse_out) c->lse_out[bh * T + i] = (float)lse;
            for(int e = 0; e < hd; e++) acc[e] = 0.0;
            for(int j = 0; j <= i; j++) {
                double pj = exp(s[j] - lse);
                for(int e = 0; e < hd; e++) acc[e] += pj * Vv[j * D + e];
            }
            for(int e = 0; e < hd; e++) O[i * D + e] = (float)acc[e];
        }
    }
    free(s);
    free(acc);
}

void ora_attn_causal_fwd(int B, int H, int T, int hd, float scale, const float* q, const float* k,
                         const float* v, float* o, float* lse) {
    struct AttnCtx c = {B, H, T, hd, scale, q, k, v, NULL, NULL, NULL, o, lse, NULL, NULL, NULL};
    ora_parallel_for((int64_t)B * H, attn_fwd_heads, &c);
}

static void attn_bwd_heads(void* p, int64_t lo, int64_t hi) {
    /* P_ij = exp(scale*q_i.k_j - lse_i) for j <= i
     * dV_j += sum_i P_ij dO_i ;  dP_ij = dO_i . v_j ;  D_i = dO_i . O_i
     * dS_ij = P_ij (dP_ij - D_i) ;  dQ_i += scale sum_j dS_ij k_j ;  dK_j += scale sum_i dS_ij q_i */
    struct AttnCtx* c = (struct AttnCtx*)p;
    const int T = c->T, hd = c->hd, D = c->H * c->hd;
    double* dQ = (double*)malloc(sizeof(double) * T * hd);
    double* dK = (double*)malloc(sizeof(double) * T * hd);
    double* dV = (double*)malloc(sizeof(double) * T * hd);
    for(int64_t bh = lo; bh < hi; bh++) {
        int64_t b = bh / c->H, h = bh % c->H;
        int64_t base = b * T * D + h * hd;
        const float *Q = c->q + base, *K = c->k + base, *Vv = c->v + base, *O = c->o + base,
                    *dO = c->dout + base;
        memset(dQ, 0, sizeof(double) * T * hd);
        memset(dK, 0, sizeof(double) * T * hd);
        memset(dV, 0, sizeof(double) * T * hd);
        for(int i = 0; i < T; i++) {
            double Di = 0.0;
            for(int e = 0; e < hd; e++) Di += (double)dO[i * D + e] * O[i * D + e];
            double lse = c->lse[bh * T + i];
            for(int j = 0; j <= i; j++) {
                double sdot = 0.0, dp = 0.0;
                for(int e = 0; e < hd; e++) {
                    sdot += (double)Q[i * D + e] * K[j * D + e];
                    dp += (double)dO[i * D + e] * Vv[j * D + e];
                }
                double P = exp(sdot * c->scale - lse);
                double dS = P * (dp - Di);
                for(int e = 0; e < hd; e++) {
                    dV[j * hd + e] += P * dO[i * D + e];
                    dQ[i * hd + e] += c->scale * dS * K[j * D + e];
                    dK[j * hd + e] += c->scale * dS * Q[i * D + e];
                }
            }
        }
        for(int i = 0; i < T; i++)
            for(int e = 0; e < hd; e++) {
                if(c->dq) c->dq[base + i * D + e] += (float)dQ[i * hd + e];
                if(c->dk) c->dk[base + i * D + e] += (float)dK[i * hd + e];
                if(c->dv) c->dv[base + i * D + e] += (float)dV[i * hd + e];
            }
    }
    free(dQ);
    free(dK);
    free(dV);
}

void ora_attn_causal_bwd(int B, int H, int T, int hd, float scale, const float* q, const float* k,
                         const float* v, const float* o, const float* lse, const float* dout,
                         float* dq, float* dk, float* dv) {
    struct AttnCtx c = {B, H, T, hd, scale, q, k, v, o, lse, dout, NULL, NULL, dq, dk, dv};
    ora_parallel_for((int64_t)B * H, attn_bwd_heads, &c);
}

void ora_embed_fwd(int64_t n, int64_t d, const int32_t* ids, const float* table, float* out) {
    for(int64_t i = 0; i < n; i++) memcpy(out + i * d, table + (int64_t)ids[i] * d, d * 4);
}

void ora_embed_bwd(int64_t n, int64_t d, const int32_t* ids, const float* dout, float* dtable) {
    for(int64_t i = 0; i < n; i++)
        for(int64_t e = 0; e < d; e++) dtable[(int64_t)ids[i] * d + e] += dout[i * d + e];
}

/* --------------------------------------------------------- pico-style ops
 * Each op node is a PicoTensor followed by its saved state in the arena; the
 * backward hook recovers the state from the tensor's address. */
static struct Arena* need_arena(void) {
    struct Arena* ar = arena_ctx_current();
    if(!ar) fprintf(stderr, "[Pico] Error: No current arena in context!\n");
    return ar;
}

static struct PicoTensor* node_new(struct Arena* ar, size_t node_bytes, int64_t* shape,
                                   int ndim) {
    /* node_bytes >= sizeof(PicoTensor); the tensor is the node's first member */
    struct PicoTensor* t = pico_create_tensor(ar, shape, (uint8_t)ndim);
    struct PicoTensor* n = (struct PicoTensor*)arena_alloc(ar, node_bytes);
    memset(n, 0, node_bytes);
    *n = *t;
    return n;
}

static void set_parents(struct Arena* ar, struct PicoTensor* out, int n, struct PicoTensor** ps,
                        void (*bw)(struct PicoTensor*)) {
    out->parents = (struct PicoTensor**)arena_alloc(ar, sizeof(struct PicoTensor*) * n);
    for(int i = 0; i < n; i++) out->parents[i] = ps[i];
    out->num_parents = (uint8_t)n;
    out->_backward = bw;
}

/* softmax cross-entropy: loss [1] = mean_r (lse_r - z[r, y_r]) */
struct XentNode {
    struct PicoTensor t;
    const int32_t* labels;
};
static void xent_bw(struct PicoTensor* self) {
    struct XentNode* n = (struct XentNode*)self;
    struct PicoTensor* z = self->parents[0];
    int64_t R = z->shape[0], V = z->shape[1];
    float* tmp = (float*)malloc(sizeof(float) * R * V);
    ora_xent_fwd_bwd(R, V, z->data, n->labels, NULL, tmp, self->grad[0] / (float)R);
    for(int64_t i = 0; i < R * V; i++) z->grad[i] += tmp[i];
    free(tmp);
}
struct PicoTensor* pico_softmax_xent(struct PicoTensor* logits, const int32_t* labels) {
    if(logits->ndim != 2) {
        fprintf(stderr, "[Pico] Error: softmax_xent expects 2-D logits [rows, classes]!\n");
        return NULL;
    }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    int64_t one[1] = {1};
    struct XentNode* n = (struct XentNode*)node_new(ar, sizeof(struct XentNode), one, 1);
    n->t.backend = logits->backend;
    n->labels = labels;
    int64_t R = logits->shape[0], V = logits->shape[1];
    float* rows = (float*)malloc(sizeof(float) * R);
    ora_xent_fwd_bwd(R, V, logits->data, labels, rows, NULL, 0.0f);
    double s = 0.0;
    for(int64_t r = 0; r < R; r++) s += rows[r];
    free(rows);
    n->t.data[0] = (float)(s / (double)R);
    set_parents(ar, &n->t, 1, &logits, xent_bw);
    return &n->t;
}

/* RMSNorm over the last dim of a 2-D x, gain [C] */
struct RmsNode {
    struct PicoTensor t;
    float* rstd;
};
static void rms_bw(struct PicoTensor* self) {
    struct RmsNode* n = (struct RmsNode*)self;
    struct PicoTensor *x = self->parents[0], *g = self->parents[1];
    ora_rmsnorm_bwd(x->shape[0], x->shape[1], x->data, g->data, n->rstd, self->grad, x->grad,
                    g->grad);
}
struct PicoTensor* pico_rmsnorm(struct PicoTensor* x, struct PicoTensor* gain, float eps) {
    if(x->ndim != 2 || gain->numel != x->shape[1]) {
        fprintf(stderr, "[Pico] Error: rmsnorm expects x [rows, C] and gain [C]!\n");
        return NULL;
    }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    struct RmsNode* n = (struct RmsNode*)node_new(ar, sizeof(struct RmsNode), x->shape, 2);
    n->t.backend = x->backend;
    n->rstd = (float*)arena_alloc(ar, sizeof(float) * x->shape[0]);
    ora_rmsnorm_fwd(x->shape[0], x->shape[1], eps, x->data, gain->data, n->t.data, n->rstd);
    struct PicoTensor* ps[2] = {x, gain};
    set_parents(ar, &n->t, 2, ps, rms_bw);
    return &n->t;
}

static void swiglu_bw(struct PicoTensor* self) {
    struct PicoTensor *a = self->parents[0], *u = self->parents[1];
    ora_swiglu_bwd(self->numel, a->data, u->data, self->grad, a->grad, u->grad);
}
struct PicoTensor* pico_swiglu(struct PicoTensor* a, struct PicoTensor* u) {
    if(a->numel != u->numel || a->ndim != u->ndim) {
        fprintf(stderr, "[Pico] Error: swiglu expects gate and up of the same shape!\n");
        return NULL;
    }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    struct PicoTensor* out = pico_create_tensor(ar, a->shape, a->ndim);
    out->backend = a->backend;
    ora_swiglu_fwd(a->numel, a->data, u->data, out->data);
    struct PicoTensor* ps[2] = {a, u};
    set_parents(ar, out, 2, ps, swiglu_bw);
    return out;
}

struct AttnNode {
    struct PicoTensor t;
    float* lse;
    int B, H;
};
static void attn_bw(struct PicoTensor* self) {
    struct AttnNode* n = (struct AttnNode*)self;
    struct PicoTensor *q = self->parents[0], *k = self->parents[1], *v = self->parents[2];
    int T = (int)(q->shape[0] / n->B), D = (int)q->shape[1], hd = D / n->H;
    ora_attn_causal_bwd(n->B, n->H, T, hd, 1.0f / sqrtf((float)hd), q->data, k->data, v->data,
                        self->data, n->lse, self->grad, q->grad, k->grad, v->grad);
}
struct PicoTensor* pico_attention_causal(struct PicoTensor* q, struct PicoTensor* k,
                                         struct PicoTensor* v, int batch, int n_heads) {
    if(q->ndim != 2 || !pico_check_broadcast_compatibility(q, k) || q->numel != k->numel ||
       q->numel != v->numel || batch <= 0 || n_heads <= 0 || q->shape[0] % batch ||
       q->shape[1] % n_heads) {
        fprintf(stderr, "[Pico] Error: attention expects q, k, v [batch*T, heads*hd]!\n");
        return NULL;
    }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    struct AttnNode* n = (struct AttnNode*)node_new(ar, sizeof(struct AttnNode), q->shape, 2);
    n->t.backend = q->backend;
    int T = (int)(q->shape[0] / batch), D = (int)q->shape[1], hd = D / n_heads;
    n->B = batch;
    n->H = n_heads;
    n->lse = (float*)arena_alloc(ar, sizeof(float) * (size_t)batch * n_heads * T);
    ora_attn_causal_fwd(batch, n_heads, T, hd, 1.0f / sqrtf((float)hd), q->data, k->data,
                        v->data, n->t.data, n->lse);
    struct PicoTensor* ps[3] = {q, k, v};
    set_parents(ar, &n->t, 3, ps, attn_bw);
    return &n->t;
}

struct EmbNode {
    struct PicoTensor t;
    const int32_t* ids;
};
static void emb_bw(struct PicoTensor* self) {
    struct EmbNode* n = (struct EmbNode*)self;
    struct PicoTensor* tab = self->parents[0];
    ora_embed_bwd(self->shape[0], self->shape[1], n->ids, self->grad, tab->grad);
}
struct PicoTensor* pico_embedding(struct PicoTensor* table, const int32_t* ids, int64_t n_ids) {
    if(table->ndim != 2) {
        fprintf(stderr, "[Pico] Error: embedding expects a 2-D table [vocab, d]!\n");
        return NULL;
    }
    for(int64_t i = 0; i < n_ids; i++)
        if(ids[i] < 0 || ids[i] >= table->shape[0]) {
            fprintf(stderr, "[Pico] Error: embedding id out of range!\n");
            return NULL;
        }
    struct Arena* ar = need_arena();
    if(!ar) return NULL;
    int64_t shape[2] = {n_ids, table->shape[1]};
    struct EmbNode* n = (struct EmbNode*)node_new(ar, sizeof(struct EmbNode), shape, 2);
    n->t.backend = table->backend;
    n->ids = ids;
    ora_embed_fwd(n_ids, table->shape[1], ids, table->data, n->t.data);
    set_parents(ar, &n->t, 1, &table, emb_bw);
    return &n->t;
}
