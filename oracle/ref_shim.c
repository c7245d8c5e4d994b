/*
 * oracle/ref_shim.c -- compiled together with pico's own sources (see Makefile)
 * into oracle/_ref/libpicoref.so.  pico's CPU kernels are static inline in its
 * headers (src/kernels/cpu/cpu_scalar.h, cpu_avx.h, src/autograd.h), so they
 * have no symbols of their own; these wrappers give them C-ABI entry points
 * over raw row-major buffers, the way the reference's benches call them
 * (bench/README.md:26-28).  Test infrastructure only.
 */
#include <stdint.h>

#include "autograd.h"
#include "global.h"
#include "kernels/cpu_kernels.h"
#include "tensor.h"

static struct PicoTensor view2(float* data, int64_t* shape, int64_t* strides, int64_t r,
                               int64_t c) {
    struct PicoTensor t = {0};
    shape[0] = r;
    shape[1] = c;
    strides[0] = c;
    strides[1] = 1;
    t.shape = shape;
    t.strides = strides;
    t.data = data;
    t.numel = r * c;
    t.ndim = 2;
    return t;
}

/* pico_init without touching stdout: the pool is what the AVX kernel needs */
void picoref_init_pool(void) {
    if(global_tp == 0) global_tp = pico_tpool_create(8);
}

void picoref_matmul_avx(int M, int N, int K, float* A, float* B, float* C) {
    int64_t s0[2], t0[2], s1[2], t1[2], s2[2], t2[2];
    struct PicoTensor a = view2(A, s0, t0, M, K), b = view2(B, s1, t1, K, N),
                      c = view2(C, s2, t2, M, N);
    picoref_init_pool();
    pico_matmul_cpu_avx(&a, &b, &c);
}

void picoref_matmul_scalar(int M, int N, int K, float* A, float* B, float* C) {
    int64_t s0[2], t0[2], s1[2], t1[2], s2[2], t2[2];
    struct PicoTensor a = view2(A, s0, t0, M, K), b = view2(B, s1, t1, K, N),
                      c = view2(C, s2, t2, M, N);
    pico_matmul_cpu_scalar(&a, &b, &c);
}

void picoref_matmul_backward(int M, int K, int N, float* A, float* B, float* dC, float* dA,
                             float* dB) {
    int64_t s0[2], t0[2], s1[2], t1[2], s2[2], t2[2];
    struct PicoTensor a = view2(A, s0, t0, M, K), b = view2(B, s1, t1, K, N),
                      c = view2(0, s2, t2, M, N);
    a.grad = dA;
    b.grad = dB;
    c.grad = dC;
    struct PicoTensor* parents[2] = {&a, &b};
    c.parents = parents;
    c.num_parents = 2;
    pico_matmul_backward(&c);
}

void picoref_set_seed(uint32_t s) { x_state = s; }

/* pico_rand's stream (src/tensor.c:249-273) into out[0..n) from seed */
void picoref_rand(uint32_t seed, int64_t n, float* out) {
    struct Arena* ar = arena_init((size_t)n * 8 + 4096);
    int64_t shape[1] = {n};
    x_state = seed;
    struct PicoTensor* t = pico_rand(ar, shape, 1);
    for(int64_t i = 0; i < n; i++) out[i] = t->data[i];
    arena_destroy(ar);
}

static struct PicoTensor view1(float* data, int64_t* shape, int64_t* strides, int64_t n) {
    struct PicoTensor t = {0};
    shape[0] = n;
    strides[0] = 1;
    t.shape = shape;
    t.strides = strides;
    t.data = data;
    t.numel = n;
    t.ndim = 1;
    return t;
}

/* pico's unary kernels (src/kernels/cpu_kernels.h:60-100), op 0..5 =
 * sqrt, sin, cos, tan, tanh, log */
void picoref_unary(int op, int64_t n, float* x, float* y) {
    int64_t s0[1], t0[1], s1[1], t1[1];
    struct PicoTensor a = view1(x, s0, t0, n), out = view1(y, s1, t1, n);
    switch(op) {
        case 0: pico_sqrt_cpu(&a, &out); break;
        case 1: pico_sin_cpu(&a, &out); break;
        case 2: pico_cos_cpu(&a, &out); break;
        case 3: pico_tan_cpu(&a, &out); break;
        case 4: pico_tanh_cpu(&a, &out); break;
        default: pico_log_cpu(&a, &out); break;
    }
}

/* their backward hooks (src/autograd.h:132-176): gx += local derivative * gy */
void picoref_unary_bwd(int op, int64_t n, float* x, float* y, float* gy, float* gx) {
    int64_t s0[1], t0[1], s1[1], t1[1];
    struct PicoTensor a = view1(x, s0, t0, n), self = view1(y, s1, t1, n);
    a.grad = gx;
    self.grad = gy;
    struct PicoTensor* parents[1] = {&a};
    self.parents = parents;
    self.num_parents = 1;
    switch(op) {
        case 0: pico_tensor_sqrt_backward(&self); break;
        case 1: pico_tensor_sin_backward(&self); break;
        case 2: pico_tensor_cos_backward(&self); break;
        case 3: pico_tensor_tan_backward(&self); break;
        case 4: pico_tensor_tanh_backward(&self); break;
        default: pico_tensor_log_backward(&self); break;
    }
}

/* pico's arena helpers are static inline in src/arena.h: entry points for the
 * ones a caller of its op API needs (the ops themselves allocate from
 * arena_ctx_current()) */
struct Arena* picoref_arena_init(size_t bytes) { return arena_init(bytes); }
void picoref_arena_destroy(struct Arena* arena) { arena_destroy(arena); }
void picoref_arena_reset(struct Arena* arena) { arena_reset(arena); }
void picoref_arena_ctx_push(struct Arena* arena) { arena_ctx_push(arena); }
void picoref_arena_ctx_pop(void) { arena_ctx_pop(); }
