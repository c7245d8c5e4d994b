/*
 * pico_amd/host/newops.c -- the hot-path ops pico does not have, in pico's op
 * style (src/ops.c:12-54) over GPU tensors: fused softmax cross-entropy,
 * RMSNorm, SwiGLU, causal attention, embedding, argmax.
 *
 * No reference code exists for these (the only traces are the softmax
 * Jacobian comment at src/autograd.h:38-40 and the plan at todo.md:95).
 * Their backward hooks keep the += contract of src/autograd.h:25-29.  Saved
 * state (rstd, lse, probabilities, staged labels) lives in the node and in
 * the arena's device memory, so it is released by arena_reset.
 */
#include <stdlib.h>
#include <math.h>
#include <string.h>

#include "pk_host.h"

static int need_gpu(const char* op, const struct PicoTensor* t) {
    if(!t) {
        PKH_ERR("%s: NULL tensor!\n", op);
        return 1;
    }
    if(!pkh_is_gpu(t)) {
        PKH_ERR("%s: this library runs backend GPU; CPU tensors belong to pico's CPU library!\n",
                op);
        return 1;
    }
    return 0;
}

/* ------------------------------------------------ softmax cross-entropy
 * loss [1] = mean_r (logsumexp(z_r) - z_r[y_r]).  The forward pass reads the
 * logits once and, when the logits' grad holds nothing yet, also writes the
 * gradient of the mean, (softmax - onehot)/R, into that grad buffer.  If the
 * backward then finds the upstream gradient is exactly pico_backward's seed
 * of 1 and the buffer still untouched, it only marks it live: one pass over
 * the logits instead of two.  Otherwise it recomputes, scaled by the upstream
 * gradient on the device. */
enum { XS_LABELS = 0, XS_ROWS = 1 };
enum { XI_PRECOMPUTED = 0 };

static void xent_backward(struct PicoTensor* self) {
    struct PkNode* n = pkh_node(self);
    struct PicoTensor* z = self->parents[0];
    const float* g = pkh_upstream(self);
    if(!g) return;
    int64_t R = z->shape[0], V = z->shape[1];
    if(n->ival[XI_PRECOMPUTED] && n->seed_one && !pkh_grad_is_live(z)) {
        n->ival[XI_PRECOMPUTED] = 0;
        pkh_grad_mark(z);
        return;
    }
    n->ival[XI_PRECOMPUTED] = 0;
    int st = pk_xent_fwd_bwd_f32(R, V, z->data, V, (const int32_t*)n->saved[XS_LABELS], NULL,
                                 z->grad, V, 1.0f / (float)R, g, pkh_grad_flag(z), pkh_stream());
    if(pkh_status("pico_softmax_xent_backward", st)) return;
    pkh_grad_mark(z);
}

struct PicoTensor* pico_softmax_xent(struct PicoTensor* logits, const int32_t* labels) {
    if(need_gpu("pico_softmax_xent", logits)) return NULL;
    if(logits->ndim != 2 || logits->strides[1] != 1 || logits->strides[0] != logits->shape[1]) {
        PKH_ERR("softmax_xent expects contiguous 2-D logits [rows, classes]!\n");
        return NULL;
    }
    if(!labels) {
        PKH_ERR("softmax_xent: NULL labels!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    int64_t R = logits->shape[0], V = logits->shape[1];
    const int32_t* dl = pkh_ids_on_device(labels, R);
    if(!dl) return NULL;
    int64_t one[1] = {1};
    struct PicoTensor* out = pkh_new_tensor(arena, one, 1);
    if(!out) return NULL;
    struct PkNode* n = pkh_node(out);
    float* rows = (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(R > 0 ? R : 1));
    if(!rows) return NULL;
    n->saved[XS_LABELS] = (void*)dl;
    n->saved[XS_ROWS] = rows;
    int pre = !pkh_grad_is_live(logits);
    /* the loss rows, their gradient and the mean (one launch for a small head) */
    const float inv = 1.0f / (float)(R > 0 ? R : 1);
    int st = pk_xent_mean_f32(R, V, logits->data, V, dl, rows, pre ? logits->grad : NULL, V, inv, 0, inv,
                              out->data, pkh_stream());
    if(pkh_status("pico_softmax_xent", st)) return NULL;
    n->ival[XI_PRECOMPUTED] = pre;
    pkh_set_parents(arena, out, 1, &logits, xent_backward);
    return out;
}

/* ---------------------------------------------------------------- RMSNorm
 * y = x * rstd * gain over the last dim; the backward reads the saved rstd */
enum { RS_RSTD = 0, RS_PARTS = 1 };

struct RmsDgJob {
    int64_t R, C;
    const void* parts;
    size_t bytes;
    float* grad;
    int flag;
};
static void rms_dg_job(const void* args, pk_stream_t side) {
    const struct RmsDgJob* j = (const struct RmsDgJob*)args;
    pkh_status("pico_rmsnorm_backward",
               pk_rmsnorm_dg_reduce_f32(j->R, j->C, j->parts, j->bytes, j->grad, j->flag, side));
}

static void rms_backward(struct PicoTensor* self) {
    struct PkNode* n = pkh_node(self);
    struct PicoTensor *x = self->parents[0], *gain = self->parents[1];
    const float* dy = pkh_upstream(self);
    if(!dy) return;
    int64_t C = x->shape[x->ndim - 1], R = C ? x->numel / C : 0;
    size_t ws_bytes = pk_rmsnorm_bwd_workspace(R, C);
    void* parts = n->saved[RS_PARTS];
    void* ws = parts ? parts : pkh_workspace(ws_bytes);
    if(!ws && ws_bytes) return;
    const float* dx_in = pkh_grad_base(x);
    const float* rstd = (const float*)n->saved[RS_RSTD];
    if(parts) {
        /* dgain like a weight gradient: the rows kernel leaves its partial
         * sums in a buffer of this node, and the side stream reduces them */
        int st = pk_rmsnorm_bwd_into_f32(R, C, x->data, gain->data, rstd, dy, dx_in, x->grad, NULL,
                                         PK_RMS_KEEP_PARTIALS, parts, ws_bytes, pkh_stream());
        if(pkh_status("pico_rmsnorm_backward", st)) return;
        pkh_grad_mark(x);
        struct PkNode* ng = pkh_node(gain);
        if(pkh_capturing()) {
            /* captured, the reduction waits for the next fork (after the main
             * stream's next kernel), so a replay keeps the main chain on its
             * stream */
            struct RmsDgJob j = {R, C, parts, ws_bytes, gain->grad, ng->grad_live ? PK_ACCUM : 0};
            if(pkh_side_defer(rms_dg_job, &j, sizeof(j))) {
                ng->side_seq = pkh_side_seq() + 1;
                pkh_grad_mark(gain);
                return;
            }
        }
        pk_stream_t side = pkh_side_fork();
        if(side) {
            st = pk_rmsnorm_dg_reduce_f32(R, C, parts, ws_bytes, gain->grad,
                                          ng->grad_live ? PK_ACCUM : 0, side);
            ng->side_seq = pkh_side_seq();
        } else {
            st = pk_rmsnorm_dg_reduce_f32(R, C, parts, ws_bytes, gain->grad,
                                          pkh_grad_flag(gain), pkh_stream());
        }
        if(pkh_status("pico_rmsnorm_backward", st)) return;
        pkh_grad_mark(gain);
        return;
    }
    int flags = pkh_grad_flag(gain) ? PK_ACCUM2 : 0;
    int st = pk_rmsnorm_bwd_into_f32(R, C, x->data, gain->data, rstd, dy, dx_in, x->grad,
                                     gain->grad, flags, ws, ws_bytes, pkh_stream());
    if(pkh_status("pico_rmsnorm_backward", st)) return;
    pkh_grad_mark(x);
    pkh_grad_mark(gain);
}

struct PicoTensor* pico_rmsnorm(struct PicoTensor* x, struct PicoTensor* gain, float eps) {
    if(need_gpu("pico_rmsnorm", x) || need_gpu("pico_rmsnorm", gain)) return NULL;
    if(x->ndim < 1 || gain->numel != x->shape[x->ndim - 1] || x == gain) {
        PKH_ERR("rmsnorm expects x [rows, C] and gain [C]!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    int64_t C = x->shape[x->ndim - 1], R = C ? x->numel / C : 0;
    struct PicoTensor* out = pkh_new_tensor(arena, x->shape, x->ndim);
    if(!out) return NULL;
    struct PkNode* n = pkh_node(out);
    float* rstd = (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(R > 0 ? R : 1));
    if(!rstd) return NULL;
    n->saved[RS_RSTD] = rstd;
    n->fval[0] = eps;
    /* a learned gain of an activation: its gradient's partial sums get a
     * buffer of their own, so the reduction can run on the side stream */
    if(gain->is_persistent && !x->is_persistent && R > 0) {
        n->saved[RS_PARTS] = arena_alloc_device(arena, pk_rmsnorm_bwd_workspace(R, C));
        if(!n->saved[RS_PARTS]) return NULL;
    }
    int st = pk_rmsnorm_fwd_f32(R, C, eps, x->data, gain->data, out->data, rstd, pkh_stream());
    if(pkh_status("pico_rmsnorm", st)) return NULL;
    struct PicoTensor* ps[2] = {x, gain};
    pkh_set_parents(arena, out, 2, ps, rms_backward);
    return out;
}

/* ----------------------------------------------------------------- SwiGLU
 * gate and up are contiguous, or 2-D with unit column stride and one shared
 * row stride (the two halves of a fused [R, 2F] projection) */
static int64_t swiglu_ld(const struct PicoTensor* t) {
    const int64_t F = t->shape[t->ndim - 1];
    if(t->ndim == 2 && t->strides[1] == 1 && t->strides[0] >= F) return t->strides[0];
    int64_t s = 1;
    for(int i = t->ndim - 1; i >= 0; i--) {
        if(t->shape[i] > 1 && t->strides[i] != s) return -1;
        s *= t->shape[i];
    }
    return F;
}

static void swiglu_backward(struct PicoTensor* self) {
    struct PicoTensor *a = self->parents[0], *u = self->parents[1];
    const float* dh = pkh_upstream(self);
    if(!dh) return;
    int64_t F = a->shape[a->ndim - 1], R = F ? a->numel / F : 0;
    const int64_t ld = swiglu_ld(a);
    if(a == u) {
        /* h = silu(a)*a: two passes so the second accumulates onto the first */
        int st = pk_swiglu_bwd_f32(R, F, a->data, ld, u->data, ld, dh, F, a->grad, NULL, ld,
                                   pkh_grad_flag(a), pkh_stream());
        if(pkh_status("pico_swiglu_backward", st)) return;
        pkh_grad_mark(a);
        st = pk_swiglu_bwd_f32(R, F, a->data, ld, u->data, ld, dh, F, NULL, u->grad, ld,
                               PK_ACCUM2, pkh_stream());
        pkh_status("pico_swiglu_backward", st);
        return;
    }
    int flags = (pkh_grad_flag(a) ? PK_ACCUM : 0) | (pkh_grad_flag(u) ? PK_ACCUM2 : 0);
    int st = pk_swiglu_bwd_f32(R, F, a->data, ld, u->data, ld, dh, F, a->grad, u->grad, ld, flags,
                               pkh_stream());
    if(pkh_status("pico_swiglu_backward", st)) return;
    pkh_grad_mark(a);
    pkh_grad_mark(u);
}

struct PicoTensor* pico_swiglu(struct PicoTensor* a, struct PicoTensor* u) {
    if(need_gpu("pico_swiglu", a) || need_gpu("pico_swiglu", u)) return NULL;
    if(a->numel != u->numel || a->ndim != u->ndim ||
       memcmp(a->shape, u->shape, sizeof(int64_t) * a->ndim) != 0) {
        PKH_ERR("swiglu expects gate and up of the same shape!\n");
        return NULL;
    }
    const int64_t ld = swiglu_ld(a);
    if(ld < 0 || swiglu_ld(u) != ld) {
        PKH_ERR("swiglu expects gate and up contiguous or with one row stride!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    int64_t F = a->shape[a->ndim - 1], R = F ? a->numel / F : 0;
    struct PicoTensor* out = pkh_new_tensor(arena, a->shape, a->ndim);
    if(!out) return NULL;
    int st = pk_swiglu_fwd_f32(R, F, a->data, ld, u->data, ld, out->data, F, pkh_stream());
    if(pkh_status("pico_swiglu", st)) return NULL;
    struct PicoTensor* ps[2] = {a, u};
    pkh_set_parents(arena, out, 2, ps, swiglu_backward);
    return out;
}

/* -------------------------------------------------------- causal attention
 * q, k, v token-major [batch*T, heads*hd] with unit column stride and one
 * shared row stride (contiguous, or column blocks of one fused projection);
 * out contiguous [batch*T, heads*hd].  For head size 64 (any T) the fused
 * kernels run (pk_flash_attn_*): only lse
 * [B*H*T] is saved, and the forward never writes scores or probabilities;
 * the backward passes dS from its dK/dV kernel to its dQ kernel as 32x32 tiles
 * of each head's causal triangle in a workspace of about 2*B*H*T^2 bytes.  Above
 * attn_ds_cap() bytes of tiles the fp32 backward recomputes dQ's scores
 * instead (PK_FLASH_RECOMPUTE: a workspace of 8*B*H*T bytes, the same
 * results).  Otherwise the chain of
 * batched GEMMs and causal-softmax kernels runs and saves the probabilities
 * P [B*H, T, T] (arena device memory). */
enum { AS_LSE = 0, AS_P = 1 };
/* largest dS-tile workspace the fused backward takes: 4 GiB (B*H*T^2 up to
 * about 2^31; 8 x 12 heads at T 8192 recompute), or PICO_ATTN_DS_CAP bytes
 * from the environment */
static size_t attn_ds_cap(void) {
    const char* e = getenv("PICO_ATTN_DS_CAP");
    if(e && *e) {
        char* end = NULL;
        unsigned long long v = strtoull(e, &end, 10);
        if(end && *end == '\0') return (size_t)v;
    }
    return (size_t)4 << 30;
}
/* AI_PREC: the products' precision, 0 fp32, 1 bf16, 2 fp8 (flash only); an
 * fp8 node keeps max|q|, max|k|, max|v| for the backward in saved[AS_P] */
enum { AI_B = 0, AI_H = 1, AI_FLASH = 2, AI_PREC = 3 };
enum { ATTN_F32 = 0, ATTN_BF16 = 1, ATTN_FP8 = 2, ATTN_BF16X3 = 3 };

static void attn_backward(struct PicoTensor* self) {
    struct PkNode* n = pkh_node(self);
    struct PicoTensor *q = self->parents[0], *k = self->parents[1], *v = self->parents[2];
    const float* dout = pkh_upstream(self);
    if(!dout) return;
    int64_t B = n->ival[AI_B], H = n->ival[AI_H];
    int64_t T = q->shape[0] / B, hd = q->shape[1] / H, ld = q->strides[0];
    const int flash = (int)n->ival[AI_FLASH], prec = flash ? (int)n->ival[AI_PREC] : ATTN_F32;
    size_t ws_bytes = flash ? pk_flash_attn_bwd_workspace(B, H, T)
                            : sizeof(float) * (size_t)(B * H * T * T);
    const int recompute = flash && prec == ATTN_F32 && ws_bytes > attn_ds_cap();
    if(recompute) ws_bytes = pk_flash_attn_bwd_workspace_recompute(B, H, T);
    void* ws = pkh_workspace(ws_bytes);
    if(!ws) {
        pkh_set_error("pico_attention_causal_backward: no device workspace of %zu bytes; the q, "
                      "k and v grads are not written",
                      ws_bytes);
        PKH_ERR("%s\n", pico_gpu_last_error());
        return;
    }
    /* aliased grads (q, k or v the same tensor) accumulate when each write
     * after the first carries its accumulate bit; the write order is dv, dk,
     * dq (fused) or dv, dq, dk (chain) */
    struct PicoTensor* order[3] = {v, flash ? k : q, flash ? q : k};
    const int bit[3] = {PK_ACCUM3, flash ? PK_ACCUM2 : PK_ACCUM, flash ? PK_ACCUM : PK_ACCUM2};
    int flags = recompute ? PK_FLASH_RECOMPUTE : 0;
    for(int i = 0; i < 3; i++) {
        if(pkh_grad_flag(order[i])) flags |= bit[i];
        pkh_grad_mark(order[i]);
    }
    int st;
    if(flash && prec == ATTN_FP8)
        st = pk_flash_attn_bwd_fp8_f32(B, H, T, hd, ld, n->fval[0], q->data, k->data, v->data,
                                       self->data, (const float*)n->saved[AS_LSE], dout, q->grad,
                                       k->grad, v->grad, (float*)n->saved[AS_P], ws, ws_bytes,
                                       flags, pkh_stream());
    else if(flash)
        st = (prec == ATTN_BF16     ? pk_flash_attn_bwd_bf16_f32
              : prec == ATTN_BF16X3 ? pk_flash_attn_bwd_bf16x3_f32
                                    : pk_flash_attn_bwd_f32)(
            B, H, T, hd, ld, n->fval[0], q->data, k->data, v->data, self->data,
            (const float*)n->saved[AS_LSE], dout, q->grad, k->grad, v->grad, ws, ws_bytes, flags,
            pkh_stream());
    else
        st = pk_attn_causal_bwd_f32(B, H, T, hd, ld, n->fval[0], q->data, k->data, v->data,
                                    (const float*)n->saved[AS_P], dout, q->grad, k->grad, v->grad,
                                    (float*)ws, flags, pkh_stream());
    pkh_status("pico_attention_causal_backward", st);
}

struct PicoTensor* pico_attention_causal(struct PicoTensor* q, struct PicoTensor* k,
                                         struct PicoTensor* v, int batch, int n_heads) {
    if(need_gpu("pico_attention_causal", q) || need_gpu("pico_attention_causal", k) ||
       need_gpu("pico_attention_causal", v))
        return NULL;
    int layout_ok = 1;
    struct PicoTensor* xs[3] = {q, k, v};
    for(int i = 0; i < 3; i++)
        if(xs[i]->ndim != 2 || xs[i]->strides[1] != 1 || xs[i]->strides[0] != q->strides[0] ||
           xs[i]->strides[0] < xs[i]->shape[1] || xs[i]->strides[0] % 4)
            layout_ok = 0;
    if(!layout_ok || q->shape[0] != k->shape[0] || q->shape[1] != k->shape[1] ||
       q->shape[0] != v->shape[0] || q->shape[1] != v->shape[1] || batch <= 0 || n_heads <= 0 ||
       q->shape[0] % batch || q->shape[1] % n_heads) {
        PKH_ERR("attention expects q, k, v [batch*T, heads*hd] with one row stride (a "
                "multiple of 4) and unit columns!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    int64_t B = batch, H = n_heads, T = q->shape[0] / batch, hd = q->shape[1] / n_heads;
    const int64_t ld = q->strides[0];
    struct PicoTensor* out = pkh_new_tensor(arena, q->shape, 2);
    if(!out) return NULL;
    struct PkNode* n = pkh_node(out);
    const int flash = pk_flash_attn_supported(T, hd);
    /* the matmul precision switch covers attention's products too; the
     * backward uses the precision the forward ran in */
    const int mp = pico_get_matmul_precision();
    const int prec = !flash                     ? ATTN_F32
                     : mp == PICO_MATMUL_FP8    ? ATTN_FP8
                     : mp == PICO_MATMUL_BF16   ? ATTN_BF16
                     : mp == PICO_MATMUL_BF16X3 ? ATTN_BF16X3
                                                : ATTN_F32;
    float* lse = (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(B * H * T));
    /* P for the unfused chain; fp8's max|q|, max|k|, max|v|, max|dout| */
    float* P = !flash ? (float*)arena_alloc_device(arena, sizeof(float) * (size_t)(B * H * T * T))
                      : prec == ATTN_FP8 ? (float*)arena_alloc_device(arena, 4 * sizeof(float))
                                         : NULL;
    if(!lse || ((!flash || prec == ATTN_FP8) && !P)) return NULL;
    n->saved[AS_LSE] = lse;
    n->saved[AS_P] = P;
    n->ival[AI_B] = B;
    n->ival[AI_H] = H;
    n->ival[AI_FLASH] = flash;
    n->ival[AI_PREC] = prec;
    n->fval[0] = 1.0f / sqrtf((float)hd);
    int st;
    if(prec == ATTN_FP8)
        st = pk_flash_attn_fwd_fp8_f32(B, H, T, hd, ld, n->fval[0], q->data, k->data, v->data,
                                       out->data, lse, P, pkh_stream());
    else if(flash)
        st = (prec == ATTN_BF16     ? pk_flash_attn_fwd_bf16_f32
              : prec == ATTN_BF16X3 ? pk_flash_attn_fwd_bf16x3_f32
                                    : pk_flash_attn_fwd_f32)(
            B, H, T, hd, ld, n->fval[0], q->data, k->data, v->data, out->data, lse, pkh_stream());
    else
        st = pk_attn_causal_fwd_f32(B, H, T, hd, ld, n->fval[0], q->data, k->data, v->data,
                                    out->data, lse, P, pkh_stream());
    if(pkh_status("pico_attention_causal", st)) return NULL;
    pkh_set_parents(arena, out, 3, xs, attn_backward);
    return out;
}

/* -------------------------------------------------------------- embedding
 * out [n, d] = table[ids]; the backward scatter-adds rows into table.grad */
enum { ES_IDS = 0 };

static void emb_backward(struct PicoTensor* self) {
    struct PkNode* n = pkh_node(self);
    struct PicoTensor* tab = self->parents[0];
    const float* g = pkh_upstream(self);
    if(!g) return;
    int64_t V = tab->shape[0], d = tab->shape[1];
    if(!pkh_grad_flag(tab)) {
        /* rows no id touches must read as zero */
        if(pkh_status("pico_embedding_backward", pk_fill_f32(tab->numel, 0.0f, tab->grad,
                                                               pkh_stream())))
            return;
        pkh_grad_mark(tab);
    }
    const size_t need = pk_embed_bwd_workspace(self->shape[0]);
    void* ws = pkh_workspace(need);
    if(!ws) return;
    int st = pk_embed_bwd_f32(self->shape[0], d, V, (const int32_t*)n->saved[ES_IDS], g,
                              tab->grad, ws, need, pkh_stream());
    pkh_status("pico_embedding_backward", st);
}

struct PicoTensor* pico_embedding(struct PicoTensor* table, const int32_t* ids, int64_t n_ids) {
    if(need_gpu("pico_embedding", table)) return NULL;
    if(table->ndim != 2 || table->strides[1] != 1 || table->strides[0] != table->shape[1]) {
        PKH_ERR("embedding expects a contiguous 2-D table [vocab, d]!\n");
        return NULL;
    }
    if(!ids || n_ids < 0) {
        PKH_ERR("embedding: NULL ids or negative count!\n");
        return NULL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return NULL;
    const int32_t* dids = pkh_ids_on_device(ids, n_ids);
    if(!dids && n_ids) return NULL;
    int64_t shape[2] = {n_ids, table->shape[1]};
    struct PicoTensor* out = pkh_new_tensor(arena, shape, 2);
    if(!out) return NULL;
    pkh_node(out)->saved[ES_IDS] = (void*)dids;
    int st = pk_embed_fwd_f32(n_ids, table->shape[1], table->shape[0], dids, table->data, out->data,
                              pkh_stream());
    if(pkh_status("pico_embedding", st)) return NULL;
    pkh_set_parents(arena, out, 1, &table, emb_backward);
    return out;
}

/* ----------------------------------------------------------------- argmax */
int pico_argmax(struct PicoTensor* x, int32_t* idx) {
    if(need_gpu("pico_argmax", x)) return PK_EINVAL;
    if(x->ndim != 2 || x->strides[1] != 1 || !idx) {
        PKH_ERR("argmax expects 2-D x [rows, V] with contiguous rows and an output array!\n");
        return PK_EINVAL;
    }
    struct Arena* arena = pkh_need_arena();
    if(!arena) return PK_EINVAL;
    int64_t R = x->shape[0], V = x->shape[1];
    if(R == 0) return 0;
    int32_t* d = (int32_t*)arena_alloc_device(arena, sizeof(int32_t) * (size_t)R);
    if(!d) return PK_EINVAL;
    int st = pk_argmax_f32(R, V, x->data, x->strides[0], d, pkh_stream());
    if(pkh_status("pico_argmax", st)) return st;
    return pkh_copy_d2h(idx, d, sizeof(int32_t) * (size_t)R);
}
