/* oracle/ora_internal.h -- shared helpers of the CPU oracle (test infrastructure). */
#pragma once
#include <stdint.h>

#include "ora.h"

#define ORA_MAX(a, b) (((a) > (b)) ? (a) : (b))
#define ORA_MIN(a, b) (((a) < (b)) ? (a) : (b))

void ora_contig_strides(const int64_t* shape, int ndim, int64_t* strides);
int64_t ora_map_index(int64_t gi, const int64_t* t_shape, const int64_t* t_strides, int t_ndim,
                      const int64_t* out_strides, int out_ndim);

void ora_pool_start(int n);
void ora_pool_stop(void);
void ora_pool_add(void (*fn)(void*), void* arg);
void ora_pool_wait(void);
int ora_matmul_threads(void);
void ora_parallel_for(int64_t n, void (*fn)(void*, int64_t, int64_t), void* ctx);

/* matmul kernels over strided views (out += a.b) */
void ora_k_matmul_scalar(const struct PicoTensor* a, const struct PicoTensor* b,
                         struct PicoTensor* out);
void ora_k_matmul_avx(const struct PicoTensor* a, const struct PicoTensor* b,
                      struct PicoTensor* out);
void ora_k_matmul_backward(struct PicoTensor* self);

/* a stack-resident 2-D view over a raw buffer */
struct OraView {
    struct PicoTensor t;
    int64_t shape[2];
    int64_t strides[2];
};
static inline struct PicoTensor* ora_view2(struct OraView* v, const float* data, int64_t r,
                                           int64_t c, int64_t s0, int64_t s1) {
    v->shape[0] = r;
    v->shape[1] = c;
    v->strides[0] = s0;
    v->strides[1] = s1;
    v->t.shape = v->shape;
    v->t.strides = v->strides;
    v->t.data = (float*)data;
    v->t.grad = 0;
    v->t._backward = 0;
    v->t.parents = 0;
    v->t.numel = r * c;
    v->t.backend = CPU;
    v->t.ndim = 2;
    v->t.num_parents = 0;
    v->t.is_persistent = 0;
    return &v->t;
}
