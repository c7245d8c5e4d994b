/*
 * oracle/ora.h -- CPU ORACLE for the pico hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a from-scratch C11 restatement of pico's CPU path (the reference at
 * sijirama/pico) used as the checker for the HIP backend.  Only tests/, the
 * smoke entry point and bench.py's cpu_baseline leg may load it; nothing in the
 * product (pico_amd/) links, imports or calls it.
 *
 * What it restates (reference file:line it follows):
 *   - struct PicoTensor layout, strides, broadcast rules    src/tensor.h:11-23,64-138
 *   - pico_create_tensor / pico_param / pico_free           src/tensor.c:44-168
 *   - bump arena + thread-local context stack               src/arena.h:20-169
 *   - xorshift32 uniform generator                          src/tensor.c:249-273
 *   - pico_backward (post-order DFS, seed 1, reverse walk)  src/tensor.c:15-42,399-415
 *   - add/sub/mul with broadcasting, fwd + bwd              src/ops.c:12-142, src/autograd.h:53-94
 *   - matmul fwd: scalar i-k-j and AVX R x 8 microkernels   src/kernels/cpu/cpu_scalar.h:39-54,
 *     with the threaded row split                           src/kernels/cpu/cpu_avx.h:22-205
 *   - matmul backward (dA += dC.B^T, dB += A^T.dC)          src/autograd.h:96-130
 *   - unary sqrt/sin/cos/tan/tanh/log fwd + bwd             src/kernels/cpu/cpu_scalar.h:21-37,
 *                                                            src/autograd.h:132-176
 *   - relu fwd/bwd                                          src/act/activations.c:8-26, act/autograd.h:9-17
 *   - SGD step / zero_grad                                  src/optim/SGD.c:29-47
 *   - Linear (x.W + b)                                      src/nn/linear.c:9-67
 *   - a pthread pool with a global wait barrier             src/tpool.h
 * and adds CPU versions of the ops the reference lacks (no reference code
 * exists for them; they are pinned by torch-CPU golden vectors, closed forms
 * and finite differences in tests/): fused softmax cross-entropy, RMSNorm,
 * SwiGLU, causal attention, embedding, AdamW, argmax.
 *
 * Arithmetic follows the reference's compile mode (-std=c11, so no FP
 * contraction): every a*b+c outside the AVX microkernel rounds twice.
 */
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { CPU, GPU } PicoBackend;

struct PicoTensor {
    int64_t* shape;
    int64_t* strides;
    float* data;
    float* grad;
    void (*_backward)(struct PicoTensor*);
    struct PicoTensor** parents;
    int64_t numel;
    PicoBackend backend;
    uint8_t ndim;
    uint8_t num_parents;
    uint8_t is_persistent;
};

/* ---- arena (bump allocator, thread-local context stack) ---- */
struct ArenaBlock {
    struct ArenaBlock* next;
    size_t capacity;
    unsigned char* bottom;
    unsigned char* curr;
};
struct Arena {
    struct ArenaBlock *begin, *end;
};
struct Arena* arena_init(size_t bytes);
void* arena_alloc(struct Arena* arena, size_t size);
void arena_reset(struct Arena* arena);
void arena_destroy(struct Arena* arena);
void arena_ctx_push(struct Arena* arena);
void arena_ctx_pop(void);
struct Arena* arena_ctx_current(void);

/* ---- globals ---- */
typedef enum { SIMD_NONE, SIMD_SSE, SIMD_AVX, SIMD_AVX2, SIMD_AVX512 } SimdLevel;
extern SimdLevel g_simd_level;
extern uint32_t x_state;
void pico_init(void);
void pico_shutdown(void);
void ora_set_seed(uint32_t seed);
void ora_set_simd(int level);
int ora_get_simd(void);
void ora_set_threads(int n); /* pool width used by the AVX matmul (pico: 8) */

/* ---- tensors ---- */
struct PicoTensor* pico_param(int64_t* shape, uint8_t ndim);
struct PicoTensor* pico_create_tensor(struct Arena* arena, int64_t* shape, uint8_t ndim);
struct PicoTensor* pico_tensor_from_scalar(float value);
void pico_free(struct PicoTensor* t);
void pico_transpose_2d(struct PicoTensor* t);
struct PicoTensor* pico_rand(struct Arena* arena, int64_t* shape, uint8_t ndim);
uint8_t pico_check_broadcast_compatibility(struct PicoTensor* a, struct PicoTensor* b);
void pico_backward(struct Arena* arena, struct PicoTensor* entry);

/* ---- ops (pico ops.h, activations.h) ---- */
struct PicoTensor* pico_add(struct PicoTensor* a, struct PicoTensor* b);
struct PicoTensor* pico_sub(struct PicoTensor* a, struct PicoTensor* b);
struct PicoTensor* pico_mul(struct PicoTensor* a, struct PicoTensor* b);
struct PicoTensor* pico_matmul(struct PicoTensor* a, struct PicoTensor* b);
struct PicoTensor* pico_tensor_sqrt(struct PicoTensor* a);
struct PicoTensor* pico_tensor_sin(struct PicoTensor* a);
struct PicoTensor* pico_tensor_cos(struct PicoTensor* a);
struct PicoTensor* pico_tensor_tan(struct PicoTensor* a);
struct PicoTensor* pico_tensor_tanh(struct PicoTensor* a);
struct PicoTensor* pico_tensor_log(struct PicoTensor* a);
struct PicoTensor* pico_relu(struct PicoTensor* x);

/* ---- ops the reference lacks (CPU definitions of the new hot-path ops) ---- */
struct PicoTensor* pico_softmax_xent(struct PicoTensor* logits, const int32_t* labels);
struct PicoTensor* pico_rmsnorm(struct PicoTensor* x, struct PicoTensor* gain, float eps);
struct PicoTensor* pico_swiglu(struct PicoTensor* a, struct PicoTensor* u);
struct PicoTensor* pico_attention_causal(struct PicoTensor* q, struct PicoTensor* k,
                                         struct PicoTensor* v, int batch, int n_heads);
struct PicoTensor* pico_embedding(struct PicoTensor* table, const int32_t* ids, int64_t n);

/* ---- nn / optim ---- */
struct PicoLinear {
    int in_features;
    int out_features;
    struct PicoTensor* weights;
    struct PicoTensor* bias;
};
struct PicoLinear* pico_nn_linear_init(int in_features, int out_features, bool bias);
struct PicoTensor* pico_nn_linear_forward(struct PicoLinear* layer, struct PicoTensor* input);
void pico_nn_linear_free(struct PicoLinear* linear);

struct PicoOptimSGD;
struct PicoOptimSGD* pico_optim_sgd_init(float lr);
void pico_optim_sgd_add(struct PicoOptimSGD* o, struct PicoTensor* p);
void pico_optim_sgd_step(struct PicoOptimSGD* o);
void pico_optim_sgd_zero_grad(struct PicoOptimSGD* o);
void pico_optim_sgd_free(struct PicoOptimSGD* o);

struct PicoOptimAdamW;
struct PicoOptimAdamW* pico_optim_adamw_init(float lr, float beta1, float beta2, float eps,
                                             float weight_decay);
void pico_optim_adamw_add(struct PicoOptimAdamW* o, struct PicoTensor* p);
void pico_optim_adamw_step(struct PicoOptimAdamW* o);
void pico_optim_adamw_zero_grad(struct PicoOptimAdamW* o);
void pico_optim_adamw_free(struct PicoOptimAdamW* o);

/* ---- flat entry points on raw buffers (what the tests and the CPU baseline call) ----
 * Matrices are described by (rows, cols, row stride, col stride) exactly as a
 * PicoTensor view would be; C-accumulating kernels add into C. */
void ora_matmul_scalar(int M, int N, int K, const float* A, int64_t sa0, int64_t sa1,
                       const float* B, int64_t sb0, int64_t sb1, float* C, int64_t sc0,
                       int64_t sc1);
void ora_matmul_avx(int M, int N, int K, const float* A, int64_t sa0, int64_t sa1,
                    const float* B, int64_t sb0, int64_t sb1, float* C, int64_t sc0, int64_t sc1);
/* pico_matmul_backward loops: dA += dC.B^T ; dB += A^T.dC (row-major contiguous) */
void ora_matmul_backward(int M, int K, int N, const float* A, const float* B, const float* dC,
                         float* dA, float* dB);
/* cache-blocked, threaded fp64-accumulating reference GEMM for large-size checks:
 * C = alpha * op(A).op(B) + beta * C, op = transpose when t* == 'T' */
void ora_gemm_ref_f64(char ta, char tb, int M, int N, int K, float alpha, const float* A,
                      int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc);
/* C += op(A).op(B) with float accumulation in k order (the pico dA/dB loop order) */
void ora_gemm_pico_order(char ta, char tb, int M, int N, int K, const float* A, int64_t lda,
                         const float* B, int64_t ldb, float* C, int64_t ldc);

void ora_fill_uniform(float* out, int64_t n, uint32_t seed, float lo, float hi);
void ora_fill_normal(float* out, int64_t n, uint32_t seed, float mean, float std);
void ora_fill_labels(int32_t* out, int64_t n, uint32_t seed, int32_t vocab);
void ora_fill_pico_rand(float* out, int64_t n, uint32_t seed);

void ora_rmsnorm_fwd(int64_t R, int64_t C, float eps, const float* x, const float* g, float* y,
                     float* rstd);
void ora_rmsnorm_bwd(int64_t R, int64_t C, const float* x, const float* g, const float* rstd,
                     const float* dy, float* dx, float* dg);
void ora_swiglu_fwd(int64_t n, const float* a, const float* u, float* h);
void ora_swiglu_bwd(int64_t n, const float* a, const float* u, const float* dh, float* da,
                    float* du);
void ora_xent_fwd_bwd(int64_t R, int64_t V, const float* logits, const int32_t* labels,
                      float* loss_rows, float* dlogits, float scale);
void ora_argmax(int64_t R, int64_t V, const float* x, int32_t* idx);
/* q, k, v, o token-major [B*T, H*hd]; lse [B*H, T]; backward accumulates (+=) */
void ora_attn_causal_fwd(int B, int H, int T, int hd, float scale, const float* q, const float* k,
                         const float* v, float* o, float* lse);
void ora_attn_causal_bwd(int B, int H, int T, int hd, float scale, const float* q, const float* k,
                         const float* v, const float* o, const float* lse, const float* dout,
                         float* dq, float* dk, float* dv);
void ora_embed_fwd(int64_t n, int64_t d, const int32_t* ids, const float* table, float* out);
void ora_embed_bwd(int64_t n, int64_t d, const int32_t* ids, const float* dout, float* dtable);
void ora_adamw(int64_t n, float lr, float beta1, float beta2, float eps, float wd, int step,
               float* p, const float* g, float* m, float* v);
void ora_sgd(int64_t n, float lr, float* p, const float* g);
void ora_binary(int op, int ndim, const int64_t* out_shape, const float* a, int a_ndim,
                const int64_t* a_shape, const float* b, int b_ndim, const int64_t* b_shape,
                float* out);
void ora_binary_bwd(int op, int ndim, const int64_t* out_shape, const float* a, int a_ndim,
                    const int64_t* a_shape, const float* b, int b_ndim, const int64_t* b_shape,
                    const float* gout, float* ga, float* gb);
void ora_unary(int op, int64_t n, const float* x, float* y);
void ora_unary_bwd(int op, int64_t n, const float* x, const float* y, const float* gy, float* gx);
void ora_relu(int64_t n, const float* x, float* y);
void ora_relu_bwd(int64_t n, const float* y, const float* gy, float* gx);

#ifdef __cplusplus
}
#endif
