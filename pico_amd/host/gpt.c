/*
 * pico_amd/host/gpt.c -- a pre-norm decoder-only transformer written only
 * with pico's public API (include/pico_amd.h), the way a pico user writes a
 * model (compare examples/02_relu_mlp/main.c:64-130 for the MLP).  It is the
 * training step of the benchmark configurations; the ops it calls are the
 * hot path.
 *
 * The projections that read the same input are one product each:
 * wqkv = [Wq | Wk | Wv] (d x 3d) and w13 = [W1 | W3] (d x 2F), whose output
 * pico_split_cols turns into the q, k, v (gate, up) column views that
 * attention (SwiGLU) reads.  The math is that of separate Wq, Wk, Wv, W1, W3;
 * one [8192, 2304] product replaces three [8192, 768] ones, and the
 * backward's dX = dQKV . Wqkv^T is one K = 2304 product instead of three
 * accumulating K = 768 ones.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

struct PicoGPTLayer {
    struct PicoTensor *g_attn, *wqkv, *wo, *g_ffn, *w13, *w2;
};

enum { PER_LAYER = 6 };

struct PicoGPT {
    struct PicoGPTConfig cfg;
    struct PicoTensor* emb;
    struct PicoGPTLayer* layers;
    struct PicoTensor *g_final, *wlm;
    struct PicoTensor** params;
    char** names;
    int n_params;
};

static struct PicoTensor* new_param(struct PicoGPT* m, int64_t r, int64_t c, int is_gain,
                                    uint64_t seed) {
    int64_t shape[2] = {r, c};
    struct PicoTensor* t = is_gain ? pico_param(&shape[1], 1) : pico_param(shape, 2);
    if(!t) return NULL;
    int st = is_gain ? pk_fill_f32(t->numel, 1.0f, t->data, pkh_stream())
                     : pk_fill_normal_f32(t->numel, seed, 0.0f, m->cfg.init_std, t->data,
                                          pkh_stream());
    if(pkh_status("pico_gpt_init", st)) {
        pico_free(t);
        return NULL;
    }
    m->params[m->n_params++] = t;
    return t;
}

static int name_params(struct PicoGPT* m);

struct PicoGPT* pico_gpt_init(const struct PicoGPTConfig* cfg, uint64_t seed) {
    if(!cfg || cfg->vocab < 1 || cfg->d_model < 1 || cfg->n_layers < 0 || cfg->n_heads < 1 ||
       cfg->d_ff < 1 || cfg->batch < 1 || cfg->seq_len < 1 || cfg->d_model % cfg->n_heads) {
        PKH_ERR("pico_gpt_init: invalid configuration!\n");
        return NULL;
    }
    if(pkh_init()) return NULL;
    struct PicoGPT* m = (struct PicoGPT*)calloc(1, sizeof(*m));
    if(!m) return NULL;
    m->cfg = *cfg;
    int total = 3 + PER_LAYER * cfg->n_layers;
    m->params = (struct PicoTensor**)calloc(total, sizeof(struct PicoTensor*));
    m->layers = (struct PicoGPTLayer*)calloc(cfg->n_layers ? cfg->n_layers : 1, sizeof(*m->layers));
    if(!m->params || !m->layers) {
        pico_gpt_free(m);
        return NULL;
    }
    const int64_t V = cfg->vocab, d = cfg->d_model, F = cfg->d_ff;
    uint64_t s = seed * 1000003ull;
    int ok = (m->emb = new_param(m, V, d, 0, s++)) != NULL;
    for(int l = 0; ok && l < cfg->n_layers; l++) {
        struct PicoGPTLayer* L = &m->layers[l];
        ok = (L->g_attn = new_param(m, 1, d, 1, 0)) &&
             (L->wqkv = new_param(m, d, 3 * d, 0, s++)) && (L->wo = new_param(m, d, d, 0, s++)) &&
             (L->g_ffn = new_param(m, 1, d, 1, 0)) && (L->w13 = new_param(m, d, 2 * F, 0, s++)) &&
             (L->w2 = new_param(m, F, d, 0, s++));
    }
    ok = ok && (m->g_final = new_param(m, 1, d, 1, 0)) && (m->wlm = new_param(m, d, V, 0, s++));
    ok = ok && name_params(m) == 0;
    if(!ok) {
        pico_gpt_free(m);
        return NULL;
    }
    return m;
}

struct PicoTensor* pico_gpt_loss(struct PicoGPT* m, const int32_t* tokens,
                                 const int32_t* targets) {
    if(!m || !tokens || !targets) {
        PKH_ERR("pico_gpt_loss: NULL model or batch!\n");
        return NULL;
    }
    const struct PicoGPTConfig* c = &m->cfg;
    const int64_t n = (int64_t)c->batch * c->seq_len;
    const float eps = c->norm_eps;
    struct PicoTensor* x = pico_embedding(m->emb, tokens, n);
    for(int l = 0; x && l < c->n_layers; l++) {
        struct PicoGPTLayer* L = &m->layers[l];
        struct PicoTensor* h = pico_rmsnorm(x, L->g_attn, eps);
        if(!h) return NULL;
        struct PicoTensor* qkv = pico_matmul(h, L->wqkv);
        struct PicoTensor* qkv3[3];
        if(!qkv || pico_split_cols(qkv, 3, qkv3)) return NULL;
        struct PicoTensor* a =
            pico_attention_causal(qkv3[0], qkv3[1], qkv3[2], c->batch, c->n_heads);
        if(!a) return NULL;
        x = pico_matmul_add(a, L->wo, x); /* x + a.Wo in the product's epilogue */
        if(!x) return NULL;
        h = pico_rmsnorm(x, L->g_ffn, eps);
        if(!h) return NULL;
        /* [gate | up] = h.W13; the product also writes silu(gate) * up */
        struct PicoTensor* gu = pico_matmul_gate_up(h, L->w13);
        struct PicoTensor* gu2[2];
        if(!gu || pico_split_cols(gu, 2, gu2)) return NULL;
        /* x + swiglu(gate, up).W2; the backward's dY.W2^T writes d(gate), d(up) */
        x = pico_swiglu_matmul_add(gu2[0], gu2[1], L->w2, x);
    }
    if(!x) return NULL;
    struct PicoTensor* hf = pico_rmsnorm(x, m->g_final, eps);
    if(!hf) return NULL;
    struct PicoTensor* logits = pico_matmul(hf, m->wlm);
    if(!logits) return NULL;
    return pico_softmax_xent(logits, targets);
}

int pico_gpt_num_params(const struct PicoGPT* m) { return m ? m->n_params : 0; }

struct PicoTensor* pico_gpt_param(struct PicoGPT* m, int i) {
    return (m && i >= 0 && i < m->n_params) ? m->params[i] : NULL;
}

const char* pico_gpt_param_name(const struct PicoGPT* m, int i) {
    return (m && m->names && i >= 0 && i < m->n_params) ? m->names[i] : NULL;
}

/* "emb", "layers.<l>.<part>", "final_norm", "lm_head", in param order */
static int name_params(struct PicoGPT* m) {
    static const char* const parts[PER_LAYER] = {"attn_norm", "wqkv", "wo",
                                                 "ffn_norm", "w13", "w2"};
    m->names = (char**)calloc((size_t)m->n_params, sizeof(char*));
    if(!m->names) return -1;
    for(int i = 0; i < m->n_params; i++) {
        char buf[48];
        if(i == 0)
            snprintf(buf, sizeof(buf), "emb");
        else if(i == m->n_params - 2)
            snprintf(buf, sizeof(buf), "final_norm");
        else if(i == m->n_params - 1)
            snprintf(buf, sizeof(buf), "lm_head");
        else
            snprintf(buf, sizeof(buf), "layers.%d.%s", (i - 1) / PER_LAYER,
                     parts[(i - 1) % PER_LAYER]);
        m->names[i] = (char*)malloc(strlen(buf) + 1);
        if(!m->names[i]) return -1;
        memcpy(m->names[i], buf, strlen(buf) + 1);
    }
    return 0;
}

void pico_gpt_free(struct PicoGPT* m) {
    if(!m) return;
    for(int i = 0; i < m->n_params; i++) pico_free(m->params[i]);
    if(m->names)
        for(int i = 0; i < m->n_params; i++) free(m->names[i]);
    free(m->names);
    free(m->params);
    free(m->layers);
    free(m);
}
