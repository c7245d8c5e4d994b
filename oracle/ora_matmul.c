/*
 * oracle/ora_matmul.c -- CPU oracle (test infrastructure): pico's matmul
 * kernels restated.
 *
 *  - scalar i-k-j, out += a*b with separate multiply and add
 *      (src/kernels/cpu/cpu_scalar.h:39-54)
 *  - AVX+FMA R x 8 register tiles, R in {8,4,2,1}; per C element the k loop is
 *    a chain of fused multiply-adds starting from the loaded C value; columns
 *    past the last multiple of 8 use separate multiply and add
 *      (src/kernels/cpu/cpu_avx.h:22-129)
 *  - rows >= 512 are split into min(8, ceil(rows/64)) contiguous chunks, the
 *    remainder going to the last chunk (src/kernels/cpu/cpu_avx.h:151-205)
 *  - backward: dA[i,k] += sum_j dC[i,j]*B[k,j]; dB[k,j] += sum_i A[i,k]*dC[i,j],
 *    each with a float accumulator summed in index order, then one += into the
 *    grad (src/autograd.h:96-130).  Cells are independent, so splitting the
 *    cells over threads leaves every result bit unchanged.
 */
#include <immintrin.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ora.h"
#include "ora_internal.h"

#define THREAD_MIN_ROWS 512
#define THREAD_ROW_MAX 64

void ora_k_matmul_scalar(const struct PicoTensor* a, const struct PicoTensor* b,
                         struct PicoTensor* out) {
    const int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    for(int64_t i = 0; i < M; i++) {
        for(int64_t k = 0; k < K; k++) {
            const float av = a->data[i * a->strides[0] + k * a->strides[1]];
            for(int64_t j = 0; j < N; j++) {
                float prod = av * b->data[k * b->strides[0] + j * b->strides[1]];
                out->data[i * out->strides[0] + j * out->strides[1]] += prod;
            }
        }
    }
}

/* R x 8 tile at (i, j): acc rows loaded from C, FMA chain over k, stored back */
#define DEFINE_TILE(R)                                                                      \
    __attribute__((target("avx2,fma"))) static void tile_##R##x8(                           \
        const struct PicoTensor* a, const struct PicoTensor* b, struct PicoTensor* o,       \
        int64_t K, int64_t i, int64_t j) {                                                  \
        __m256 acc[R];                                                                      \
        for(int r = 0; r < R; r++)                                                          \
            acc[r] = _mm256_loadu_ps(o->data + (i + r) * o->strides[0] + j * o->strides[1]); \
        for(int64_t k = 0; k < K; k++) {                                                    \
            __m256 bv = _mm256_loadu_ps(b->data + k * b->strides[0] + j * b->strides[1]);   \
            for(int r = 0; r < R; r++) {                                                    \
                __m256 av = _mm256_set1_ps(a->data[(i + r) * a->strides[0] + k * a->strides[1]]); \
                acc[r] = _mm256_fmadd_ps(av, bv, acc[r]);                                   \
            }                                                                               \
        }                                                                                   \
        for(int r = 0; r < R; r++)                                                          \
            _mm256_storeu_ps(o->data + (i + r) * o->strides[0] + j * o->strides[1], acc[r]); \
    }
DEFINE_TILE(8)
DEFINE_TILE(4)
DEFINE_TILE(2)
DEFINE_TILE(1)

/* a column that does not fill 8 lanes: R rows, separate multiply and add */
static void tail_column(const struct PicoTensor* a, const struct PicoTensor* b,
                        struct PicoTensor* o, int64_t K, int64_t i, int64_t j, int R) {
    for(int64_t k = 0; k < K; k++) {
        const float bv = b->data[k * b->strides[0] + j * b->strides[1]];
        for(int r = 0; r < R; r++) {
            float prod = a->data[(i + r) * a->strides[0] + k * a->strides[1]] * bv;
            o->data[(i + r) * o->strides[0] + j * o->strides[1]] += prod;
        }
    }
}

static void avx_rows(const struct PicoTensor* a, const struct PicoTensor* b, struct PicoTensor* o,
                     int64_t row0, int64_t row1) {
    const int64_t K = a->shape[1], N = b->shape[1];
    int64_t i = row0;
    static const int rolls[4] = {8, 4, 2, 1};
    for(int ri = 0; ri < 4; ri++) {
        const int R = rolls[ri];
        for(; i + R <= row1; i += R) {
            int64_t j = 0;
            for(; j + 8 <= N; j += 8) {
                switch(R) {
                    case 8: tile_8x8(a, b, o, K, i, j); break;
                    case 4: tile_4x8(a, b, o, K, i, j); break;
                    case 2: tile_2x8(a, b, o, K, i, j); break;
                    default: tile_1x8(a, b, o, K, i, j); break;
                }
            }
            for(; j < N; j++) tail_column(a, b, o, K, i, j, R);
        }
    }
}

struct AvxChunk {
    const struct PicoTensor *a, *b;
    struct PicoTensor* o;
    int64_t r0, r1;
};
static void avx_chunk_entry(void* p) {
    struct AvxChunk* c = (struct AvxChunk*)p;
    avx_rows(c->a, c->b, c->o, c->r0, c->r1);
}

void ora_k_matmul_avx(const struct PicoTensor* a, const struct PicoTensor* b,
                      struct PicoTensor* out) {
    const int64_t M = a->shape[0];
    if(M < THREAD_MIN_ROWS) {
        avx_rows(a, b, out, 0, M);
        return;
    }
    int64_t chunks = (M + THREAD_ROW_MAX - 1) / THREAD_ROW_MAX;
    int nt = ora_matmul_threads();
    int tc = (int)(chunks < nt ? chunks : nt);
    struct AvxChunk* jobs = (struct AvxChunk*)malloc(tc * sizeof(*jobs));
    int64_t per = M / tc, tail = M % tc, r = 0;
    for(int t = 0; t < tc; t++) {
        int64_t n = per + (t == tc - 1 ? tail : 0);
        jobs[t].a = a;
        jobs[t].b = b;
        jobs[t].o = out;
        jobs[t].r0 = r;
        jobs[t].r1 = r + n;
        r += n;
        ora_pool_add(avx_chunk_entry, &jobs[t]);
    }
    ora_pool_wait();
    free(jobs);
}

/* ---------------------------------------------------------------- backward */
struct BwdCtx {
    const struct PicoTensor *a, *b, *self;
    int64_t M, K, N;
};

static void bwd_da_rows(void* p, int64_t lo, int64_t hi) {
    struct BwdCtx* c = (struct BwdCtx*)p;
    const struct PicoTensor *a = c->a, *b = c->b, *s = c->self;
    for(int64_t i = lo; i < hi; i++)
        for(int64_t k = 0; k < c->K; k++) {
            float acc = 0.0f;
            for(int64_t j = 0; j < c->N; j++) {
                float prod = s->grad[i * s->strides[0] + j * s->strides[1]] *
                             b->data[k * b->strides[0] + j * b->strides[1]];
                acc += prod;
            }
            a->grad[i * a->strides[0] + k * a->strides[1]] += acc;
        }
}

static void bwd_db_rows(void* p, int64_t lo, int64_t hi) {
    struct BwdCtx* c = (struct BwdCtx*)p;
    const struct PicoTensor *a = c->a, *b = c->b, *s = c->self;
    for(int64_t k = lo; k < hi; k++)
        for(int64_t j = 0; j < c->N; j++) {
            float acc = 0.0f;
            for(int64_t i = 0; i < c->M; i++) {
                float prod = a->data[i * a->strides[0] + k * a->strides[1]] *
                             s->grad[i * s->strides[0] + j * s->strides[1]];
                acc += prod;
            }
            b->grad[k * b->strides[0] + j * b->strides[1]] += acc;
        }
}

void ora_k_matmul_backward(struct PicoTensor* self) {
    struct BwdCtx c = {self->parents[0], self->parents[1], self, self->parents[0]->shape[0],
                       self->parents[0]->shape[1], self->parents[1]->shape[1]};
    /* dA first, then dB: matters when A and B are the same tensor */
    ora_parallel_for(c.M, bwd_da_rows, &c);
    ora_parallel_for(c.K, bwd_db_rows, &c);
}

/* -------------------------------------------------------- flat entry points */
void ora_matmul_scalar(int M, int N, int K, const float* A, int64_t sa0, int64_t sa1,
                       const float* B, int64_t sb0, int64_t sb1, float* C, int64_t sc0,
                       int64_t sc1) {
    struct OraView va, vb, vc;
    ora_k_matmul_scalar(ora_view2(&va, A, M, K, sa0, sa1), ora_view2(&vb, B, K, N, sb0, sb1),
                        ora_view2(&vc, C, M, N, sc0, sc1));
}

void ora_matmul_avx(int M, int N, int K, const float* A, int64_t sa0, int64_t sa1,
                    const float* B, int64_t sb0, int64_t sb1, float* C, int64_t sc0, int64_t sc1) {
    struct OraView va, vb, vc;
    ora_k_matmul_avx(ora_view2(&va, A, M, K, sa0, sa1), ora_view2(&vb, B, K, N, sb0, sb1),
                     ora_view2(&vc, C, M, N, sc0, sc1));
}

void ora_matmul_backward(int M, int K, int N, const float* A, const float* B, const float* dC,
                         float* dA, float* dB) {
    struct OraView va, vb, vs;
    struct PicoTensor* a = ora_view2(&va, A, M, K, K, 1);
    struct PicoTensor* b = ora_view2(&vb, B, K, N, N, 1);
    struct PicoTensor* s = ora_view2(&vs, NULL, M, N, N, 1);
    a->grad = dA;
    b->grad = dB;
    s->grad = (float*)dC;
    struct PicoTensor* parents[2] = {a, b};
    s->parents = parents;
    s->num_parents = 2;
    ora_k_matmul_backward(s);
}

/* C += op(A).op(B): float accumulator per cell in k order, then one add */
struct PoCtx {
    char ta, tb;
    int M, N, K;
    const float *A, *B;
    int64_t lda, ldb, ldc;
    float* C;
};
static void po_rows(void* p, int64_t lo, int64_t hi) {
    struct PoCtx* c = (struct PoCtx*)p;
    for(int64_t i = lo; i < hi; i++)
        for(int64_t j = 0; j < c->N; j++) {
            float acc = 0.0f;
            for(int64_t k = 0; k < c->K; k++) {
                float av = c->ta == 'T' ? c->A[k * c->lda + i] : c->A[i * c->lda + k];
                float bv = c->tb == 'T' ? c->B[j * c->ldb + k] : c->B[k * c->ldb + j];
                float prod = av * bv;
                acc += prod;
            }
            c->C[i * c->ldc + j] += acc;
        }
}
void ora_gemm_pico_order(char ta, char tb, int M, int N, int K, const float* A, int64_t lda,
                         const float* B, int64_t ldb, float* C, int64_t ldc) {
    struct PoCtx c = {ta, tb, M, N, K, A, B, lda, ldb, ldc, C};
    ora_parallel_for(M, po_rows, &c);
}

/* fp64-accumulated GEMM for checking large products */
struct RefCtx {
    char ta, tb;
    int M, N, K;
    float alpha, beta;
    const float *A, *B;
    int64_t lda, ldb, ldc;
    float* C;
};
static void ref_rows(void* p, int64_t lo, int64_t hi) {
    struct RefCtx* c = (struct RefCtx*)p;
    double* row = (double*)malloc(sizeof(double) * c->N);
    for(int64_t i = lo; i < hi; i++) {
        for(int j = 0; j < c->N; j++) row[j] = 0.0;
        for(int64_t k = 0; k < c->K; k++) {
            double av = c->ta == 'T' ? c->A[k * c->lda + i] : c->A[i * c->lda + k];
            if(c->tb == 'T') {
                for(int j = 0; j < c->N; j++) row[j] += av * (double)c->B[j * c->ldb + k];
            } else {
                const float* br = c->B + k * c->ldb;
                for(int j = 0; j < c->N; j++) row[j] += av * (double)br[j];
            }
        }
        for(int j = 0; j < c->N; j++) {
            double prev = c->beta != 0.0f ? (double)c->beta * c->C[i * c->ldc + j] : 0.0;
            c->C[i * c->ldc + j] = (float)((double)c->alpha * row[j] + prev);
        }
    }
    free(row);
}
void ora_gemm_ref_f64(char ta, char tb, int M, int N, int K, float alpha, const float* A,
                      int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc) {
    struct RefCtx c = {ta, tb, M, N, K, alpha, beta, A, B, lda, ldb, ldc, C};
    ora_parallel_for(M, ref_rows, &c);
}
