/*
 * pico_amd/host/mx8.c -- pico_matmul's fp8 products (PICO_MATMUL_FP8; no
 * reference counterpart: pico is fp32 only, src/tensor.h:14-15).
 *
 * A product C = op(A).op(B) (+ beta X) runs as pk_gemm_mx8_f32 over MX8
 * operands: e4m3 values with a power-of-two scale per 32 values along K
 * (pk_mx8_quantize_f32), so each operand is cast in one pass over it, with no
 * tensor-wide maximum to find first.  op(A) is cast as [M, K] and op(B)^T as
 * [N, K], into the stream's workspace, followed there by the partial planes
 * of a product that splits K (pk_gemm_mx8_ex_f32).
 *
 * A parameter read as itself (a weight) is cast once per change instead: its
 * casts -- W^T for x.W, W for the input gradient dY.W^T -- are kept, tagged
 * with the parameter epoch they were made in.  pkh_params_changed() starts a
 * new epoch wherever parameters may change behind the library's back or by
 * its own hand: optimizer steps, host-to-device copies, new and freed
 * parameters, checkpoint loads, graph capture and every graph replay.  A
 * cast from an earlier epoch is redone, in place, at its next use; so within
 * a training step each weight is cast at most twice (once per layout), and a
 * captured step recasts its weights on every replay.
 *
 * A matmul's backward reads its upstream gradient g in both layouts: g [M, N]
 * for the input gradient, g^T [N, M] for the weight gradient.  Both casts come
 * from one read of g (pk_mx8_quantize2_f32), issued on the main stream before
 * the weight gradient forks to the side stream, and live in the arena, which
 * no later op reuses before the arena is reset.
 */
#include <stdint.h>
#include <string.h>

#include "pk_host.h"

#define MX8_CACHE_MAX 512

struct Mx8Cast {
    const float* p;
    int64_t rows, k, ld;
    int trans;
    uint64_t epoch;
    void* q;
};

static struct Mx8Cast g_casts[MX8_CACHE_MAX];
static int g_ncasts;
static uint64_t g_epoch = 1;

void pkh_params_changed(void) { g_epoch++; }

/* the upstream gradient of the matmul whose backward is running, cast both
 * ways by one pass over it (pkh_mx8_grad_casts) into the current arena, so
 * that its input gradient (g as [M, N]) and its weight gradient (g^T as
 * [N, M], on the side stream) read it without casting it again */
static struct Mx8Cast g_grad[2];

int pkh_mx8_grad_casts(const float* g, int64_t M, int64_t N, pk_stream_t st) {
    memset(g_grad, 0, sizeof(g_grad));
    struct Arena* arena = pkh_need_arena();
    if(!arena || M <= 0 || N <= 0) return 0;
    void* qr = arena_alloc_device(arena, pk_mx8_bytes(M, N));
    void* qt = qr ? arena_alloc_device(arena, pk_mx8_bytes(N, M)) : NULL;
    if(!qt) return 0; /* the products cast g themselves */
    int s = pk_mx8_quantize2_f32(M, N, g, N, qr, qt, st);
    if(s) return s;
    g_grad[0] = (struct Mx8Cast){g, M, N, N, 0, 0, qr};
    g_grad[1] = (struct Mx8Cast){g, N, M, N, 1, 0, qt};
    return 0;
}

void pkh_mx8_grad_casts_done(void) { memset(g_grad, 0, sizeof(g_grad)); }

void pkh_mx8_release(void) {
    for(int i = 0; i < g_ncasts; i++) pkh_device_free(g_casts[i].q);
    memset(g_casts, 0, sizeof(g_casts));
    g_ncasts = 0;
}

/* the kept cast of a parameter's op(m) [rows, k] (trans: m stored [k, rows]),
 * refreshed if stale; NULL when the operand is not kept (not a parameter, the
 * side stream, a full table, or a capture that would have to allocate) */
static const void* kept_cast(struct PkMat m, int64_t rows, int64_t k, int trans, pk_stream_t st,
                             int side, int* status) {
    *status = 0;
    for(int i = 0; i < 2; i++) {
        const struct Mx8Cast* e = &g_grad[i];
        if(e->q && e->p == m.p && e->rows == rows && e->k == k && e->ld == m.ld && e->trans == trans)
            return e->q;
    }
    if(!m.persist || side) return NULL;
    struct Mx8Cast* c = NULL;
    for(int i = 0; i < g_ncasts; i++) {
        struct Mx8Cast* e = &g_casts[i];
        if(e->p == m.p && e->rows == rows && e->k == k && e->ld == m.ld && e->trans == trans) {
            c = e;
            break;
        }
    }
    if(!c) {
        if(g_ncasts == MX8_CACHE_MAX || pkh_capturing()) return NULL;
        void* q = pkh_device_alloc(pk_mx8_bytes(rows, k));
        if(!q) return NULL;
        c = &g_casts[g_ncasts++];
        c->p = m.p;
        c->rows = rows;
        c->k = k;
        c->ld = m.ld;
        c->trans = trans;
        c->epoch = 0;
        c->q = q;
    }
    if(c->epoch != g_epoch) {
        *status = pk_mx8_quantize_f32(rows, k, m.p, m.ld, trans, c->q, st);
        if(*status) return NULL;
        c->epoch = g_epoch;
    }
    return c->q;
}

int pkh_mx8_product(struct PkMat A, struct PkMat B, int64_t M, int64_t N, int64_t K, float* C,
                    int64_t ldc, float beta, const float* X, int64_t ldx, pk_stream_t st,
                    int side) {
    if(M <= 0 || N <= 0) return 0;
    if(K <= 0) {
        /* C = beta X: the product's epilogue with no slices to multiply */
        return pk_gemm_mx8_f32(M, N, 0, 1.0f, NULL, NULL, beta, X, ldx, C, ldc, st);
    }
    /* op(A) [M, K] is A itself ('N') or A^T; op(B)^T [N, K] is B^T ('N') or B */
    const int ta = A.t == 'T', tb = B.t == 'N';
    int s = 0;
    const void* qa = kept_cast(A, M, K, ta, st, side, &s);
    if(s) return s;
    const void* qb = kept_cast(B, N, K, tb, st, side, &s);
    if(s) return s;
    /* the casts, then a K split's partial planes (MX8 sizes keep 256-byte alignment) */
    const size_t ba = qa ? 0 : pk_mx8_bytes(M, K), bb = qb ? 0 : pk_mx8_bytes(N, K);
    const size_t bs = pk_gemm_mx8_workspace(M, N, K);
    unsigned char* ws = NULL;
    if(ba + bb + bs) {
        ws = (unsigned char*)(side ? pkh_side_workspace(ba + bb + bs) : pkh_workspace(ba + bb + bs));
        if(!ws) return PK_EINVAL;
    }
    if(!qa) {
        if((s = pk_mx8_quantize_f32(M, K, A.p, A.ld, ta, ws, st))) return s;
        qa = ws;
    }
    if(!qb) {
        if((s = pk_mx8_quantize_f32(N, K, B.p, B.ld, tb, ws + ba, st))) return s;
        qb = ws + ba;
    }
    return pk_gemm_mx8_ex_f32(M, N, K, 1.0f, qa, qb, beta, X, ldx, C, ldc,
                              bs ? ws + ba + bb : NULL, bs, st);
}
