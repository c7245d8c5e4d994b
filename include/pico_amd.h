/*
 * include/pico_amd.h -- pico's public C API over MI355X (gfx950) tensors.
 *
 * libpico_amd.so implements the operator, autograd, arena, module and
 * optimizer API of pico (sijirama/pico) for tensors whose `backend` is GPU.
 * Names, signatures, argument meaning and error behaviour follow the
 * reference: an op validates its inputs, allocates its output in the calling
 * thread's current arena, launches its kernel, wires `parents` and `_backward`,
 * and returns the new tensor; a refused call prints "[Pico] Error: ..." on
 * stderr and returns NULL (src/ops.c:12-54).  Backward hooks accumulate (+=)
 * into their parents' grads (src/autograd.h:25-29).
 *
 * What differs, and why:
 *  - `data` and `grad` of every tensor made here are DEVICE pointers.  Host
 *    code must not dereference them; use pico_tensor_copy_from_host /
 *    pico_tensor_copy_to_host / pico_tensor_grad_to_host.
 *  - Every tensor made here is GPU-backed (pico_param, pico_create_tensor and
 *    the ops all produce backend == GPU).  A CPU-backed tensor passed to an
 *    op is refused with NULL: the CPU path is pico's own library, unchanged.
 *  - Grad buffers are zero-initialised lazily: a grad that has received no
 *    contribution reads as zeros (pico_tensor_grad_to_host) and the first
 *    contribution overwrites instead of adding, which is bit-identical to
 *    adding into zeros and saves one full write of every grad.
 *  - An arena has device blocks beside its host blocks: tensor structs,
 *    shapes and parent lists live in host memory, tensor data in device
 *    blocks.  struct Arena keeps pico's two-pointer layout; the device blocks
 *    are held in a side table keyed by the arena's address, so an arena pico
 *    allocated itself can be passed to arena_alloc_device.  arena_reset
 *    rewinds both and keeps the device blocks for the next step; an
 *    allocation larger than a block gets a block of its own size (the
 *    reference's growth cannot serve it, src/arena.h:78-116).
 *  - This library recognises its own tensors by address (a registry), never
 *    by reading past sizeof(struct PicoTensor): tensors pico made itself, with
 *    device data and grad, are accepted by the *_gpu twins below and treated
 *    as plain pico tensors (grads always live, every contribution += ).
 *  - Kernels run asynchronously on one HIP stream (pico_gpu_stream).  The
 *    copy helpers synchronise it.  A failed launch inside a backward hook
 *    prints "[Pico] Error: ..." and is kept for pico_gpu_last_error().
 *
 * Every declaration below cites the reference interface it replaces.
 */
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- core types: the layout of src/tensor.h:9-23 and src/arena.h:20-29 ---- */
typedef enum { CPU, GPU } PicoBackend;

struct PicoTensor {
    int64_t* shape;
    int64_t* strides;
    float* data; /* device memory */
    float* grad; /* device memory */
    void (*_backward)(struct PicoTensor*);
    struct PicoTensor** parents;
    int64_t numel;
    PicoBackend backend;
    uint8_t ndim;
    uint8_t num_parents;
    uint8_t is_persistent;
};

struct ArenaBlock {
    struct ArenaBlock* next;
    size_t capacity;
    unsigned char* bottom;
    unsigned char* curr;
};

/* pico's two-pointer arena (src/arena.h:27-29); its device blocks live in a
 * side table of this library, keyed by the arena's address */
struct Arena {
    struct ArenaBlock *begin, *end;
};

/* ---- init (src/global.c:29-75) ----
 * pico_init brings up HIP on device 0 (or $PICO_DEVICE) and creates the
 * library's stream; it is idempotent and called by every entry point that
 * needs the device. */
void pico_init(void);
void pico_shutdown(void);

/* ---- arena (src/arena.h:38-169; there they are static inline) ---- */
struct Arena* arena_init(size_t bytes);
void* arena_alloc(struct Arena* arena, size_t size);
void arena_reset(struct Arena* arena);
void arena_destroy(struct Arena* arena);
void arena_ctx_push(struct Arena* arena);
void arena_ctx_pop(void);
struct Arena* arena_ctx_current(void);
/* device memory from the arena's device blocks, 256-byte aligned (no
 * reference counterpart: the device twin of arena_alloc, src/arena.h:105-116).
 * `arena` may be one this library made or one pico made itself (its device
 * blocks are then sized like its first host block, at least 1 MiB). */
void* arena_alloc_device(struct Arena* arena, size_t size);
/* For an arena pico made itself, the two calls its arena_reset and
 * arena_destroy (src/arena.h:123-153) add: rewind the device blocks (kept for
 * the next step), and free them with the side-table entry.  This library's
 * own arena_reset / arena_destroy call them. */
void arena_device_reset(struct Arena* arena);
void arena_device_release(struct Arena* arena);

/* ---- tensors (src/tensor.h:25-57, src/tensor.c) ---- */
void pico_backward(struct Arena* arena, struct PicoTensor* entry); /* tensor.c:15-42 */
struct PicoTensor* pico_param(int64_t* shape, uint8_t ndim);       /* tensor.c:44-84 */
struct PicoTensor* pico_create_tensor(struct Arena* arena, int64_t* shape,
                                      uint8_t ndim);               /* tensor.c:86-134 */
struct PicoTensor* pico_tensor_from_scalar(float value);           /* tensor.c:173-188 */
void pico_free(struct PicoTensor* tensor);                         /* tensor.c:136-168 */
void pico_tensor_print(struct PicoTensor* t);                      /* tensor.c:210-228 */
void pico_transpose_2d(struct PicoTensor* tensor);                 /* tensor.c:230-244 */
/* n column-block views of t [M, n*C] (contiguous, in the current arena, not a
 * param): outs[i] is [M, C] with row stride n*C and shares t's data and grad
 * (no reference counterpart; the reference's only view is pico_transpose_2d).
 * One product x.[W0|W1|..] split this way feeds several consumers.  Their
 * gradients land in t's grad directly; the columns of a view that no consumer
 * wrote read as zeros.  Returns 0, or nonzero for a tensor it cannot split. */
int pico_split_cols(struct PicoTensor* t, int n, struct PicoTensor** outs);
/* uniform [0,1) from pico's xorshift32 stream (tensor.c:249-273), drawn on the
 * host in the reference's order and copied to the device */
struct PicoTensor* pico_rand(struct Arena* arena, int64_t* shape, uint8_t ndim);
/* N(0,1) over all numel elements (flat Box-Muller, u1 in (0,1]).  The
 * reference's pico_randn (tensor.c:348-367) halves the last dim and can take
 * log(0); this one returns the requested shape. */
struct PicoTensor* pico_randn(struct Arena* arena, int64_t* shape, uint8_t ndim);
uint8_t pico_check_broadcast_compatibility(struct PicoTensor* a,
                                           struct PicoTensor* b); /* tensor.c:371-397 */
/* xorshift32 state of pico_rand (src/global.c:13) */
extern uint32_t x_state;

/* ---- ops (src/ops.h:5-18, src/act/activations.h:12) ---- */
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

/* The GPU twins of the op seam the reference leaves commented out
 * (src/ops.c:42-44, 86-88, 130-132): `out` is pre-allocated by the caller with
 * the broadcast shape (matmul: [rows(a), cols(b)]), as pico's CPU kernels
 * expect (src/kernels/cpu_kernels.h:13-55).  Return 0 or a pk_* status. */
int pico_add_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
int pico_sub_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
int pico_mul_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
int pico_matmul_gpu(struct PicoTensor* a, struct PicoTensor* b, struct PicoTensor* out);
/* GPU twins of the backward hooks (src/autograd.h:53-130, act/autograd.h:9-17) */
void pico_add_backward_gpu(struct PicoTensor* self);
void pico_sub_backward_gpu(struct PicoTensor* self);
void pico_mul_backward_gpu(struct PicoTensor* self);
void pico_matmul_backward_gpu(struct PicoTensor* self);
void pico_relu_backward_gpu(struct PicoTensor* self);

/* ---- hot-path ops the reference lacks (softmax-CE, RMSNorm, SwiGLU, causal
 * attention, embedding, AdamW, argmax).  No reference code: the softmax
 * Jacobian comment at src/autograd.h:38-40 and the plan at todo.md:95 are the
 * only traces.  Same op template as src/ops.c:12-54.
 * `labels` / `ids` are int32 arrays in host or device memory; host arrays are
 * staged into the current arena's device memory. ---- */
/* loss [1] = mean_r (logsumexp(z_r) - z_r[labels[r]]) over logits [R, V] */
struct PicoTensor* pico_softmax_xent(struct PicoTensor* logits, const int32_t* labels);
/* y = x * rstd * gain over the last dim of x [R, C], rstd = (mean(x^2) + eps)^-1/2 */
struct PicoTensor* pico_rmsnorm(struct PicoTensor* x, struct PicoTensor* gain, float eps);
/* h = silu(a) * u, a and u of the same shape */
struct PicoTensor* pico_swiglu(struct PicoTensor* a, struct PicoTensor* u);
/* causal softmax(q k^T / sqrt(hd)) v per head; q, k, v token-major
 * [batch*T, n_heads*hd] */
struct PicoTensor* pico_attention_causal(struct PicoTensor* q, struct PicoTensor* k,
                                         struct PicoTensor* v, int batch, int n_heads);
/* out [n, d] = table[ids] for table [vocab, d] */
struct PicoTensor* pico_embedding(struct PicoTensor* table, const int32_t* ids, int64_t n);
/* idx[r] = first argmax of row r of x [R, V]; idx is host memory (R int32) */
int pico_argmax(struct PicoTensor* x, int32_t* idx);

/* ---- fused ops (no reference counterpart: pico runs a matmul and the op
 * that consumes it as two passes over memory).  Same template as src/ops.c
 * :144-190; each equals the composition of the ops it fuses, bit for bit.
 * pico_matmul_add(a, b, c) = c + a.b, c a contiguous [rows(a), cols(b)]
 *   (a residual connection added in the product's epilogue).
 * pico_swiglu_matmul_add(gate, up, w, c) = c + swiglu(gate, up).w, c (a
 *   contiguous [M, N]) may be NULL; gate and up distinct [M, F] with one row
 *   stride (column views of
 *   one [M, 2F] product are fine), w row-contiguous [F, N].  The backward
 *   never stores dh: the product dY.w^T writes the gate and up gradients
 *   from its tiles.
 * pico_matmul_gate_up(a, w) = a.w for w = [W1 | W3] [K, 2F]: a matmul, whose
 *   product also writes h = silu(gate) * up (gate, up the two column halves
 *   of the result) and keeps it; pico_swiglu_matmul_add over the two views
 *   pico_split_cols(result, 2) makes uses that h instead of computing it.
 *   (F not a multiple of 32, a transposed a, or a product that pico_matmul
 *   would split along K: a plain matmul.) ---- */
struct PicoTensor* pico_matmul_add(struct PicoTensor* a, struct PicoTensor* b,
                                   struct PicoTensor* c);
struct PicoTensor* pico_matmul_gate_up(struct PicoTensor* a, struct PicoTensor* w);
struct PicoTensor* pico_swiglu_matmul_add(struct PicoTensor* gate, struct PicoTensor* up,
                                          struct PicoTensor* w, struct PicoTensor* c);

/* ---- nn (src/nn/linear.h:6-15) ---- */
struct PicoLinear {
    int in_features;
    int out_features;
    struct PicoTensor* weights; /* [in, out] */
    struct PicoTensor* bias;    /* [out] */
};
struct PicoLinear* pico_nn_linear_init(int in_features, int out_features, bool bias);
struct PicoTensor* pico_nn_linear_forward(struct PicoLinear* layer, struct PicoTensor* input);
void pico_nn_linear_free(struct PicoLinear* linear);

/* ---- optim (src/optim/optim.h:7-16) ---- */
struct PicoOptimSGD;
struct PicoOptimSGD* pico_optim_sgd_init(float lr);
void pico_optim_sgd_add(struct PicoOptimSGD* optim, struct PicoTensor* param);
void pico_optim_sgd_step(struct PicoOptimSGD* optim);
void pico_optim_sgd_zero_grad(struct PicoOptimSGD* optim);
void pico_optim_sgd_free(struct PicoOptimSGD* optim);

/* AdamW with decoupled weight decay (the reference only names Adam,
 * src/optim/optim.h:19-23):  p <- p(1 - lr wd);  m <- b1 m + (1-b1) g;
 * v <- b2 v + (1-b2) g^2;  p <- p - lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps) */
struct PicoOptimAdamW;
struct PicoOptimAdamW* pico_optim_adamw_init(float lr, float beta1, float beta2, float eps,
                                             float weight_decay);
void pico_optim_adamw_add(struct PicoOptimAdamW* optim, struct PicoTensor* param);
void pico_optim_adamw_step(struct PicoOptimAdamW* optim);
void pico_optim_adamw_zero_grad(struct PicoOptimAdamW* optim);
void pico_optim_adamw_free(struct PicoOptimAdamW* optim);

/* ---- decoder-only transformer built only from the ops above (no reference
 * counterpart: pico has no sequence model; this is the training step of the
 * benchmark configurations).  Pre-norm blocks without biases:
 *   x = E[tokens]
 *   per layer: x += attn_causal(rms(x) Wq, rms(x) Wk, rms(x) Wv) Wo
 *              x += swiglu(rms(x) W1, rms(x) W3) W2
 *   loss = softmax_xent(rms(x) Wlm, targets)
 * Weights ~ N(0, init_std) from a seeded device generator, norm gains 1.
 * Parameter order: E [V,d]; per layer g_attn [d], Wq, Wk, Wv, Wo [d,d],
 * g_ffn [d], W1 [d,F], W3 [d,F], W2 [F,d]; g_final [d]; Wlm [d,V]. */
struct PicoGPTConfig {
    int vocab;
    int d_model;
    int n_layers;
    int n_heads;
    int d_ff;
    int batch;
    int seq_len;
    float norm_eps;
    float init_std;
};
struct PicoGPT;
struct PicoGPT* pico_gpt_init(const struct PicoGPTConfig* cfg, uint64_t seed);
/* mean next-token cross-entropy over batch*seq_len positions; tokens and
 * targets are int32 [batch*seq_len] (host or device).  Every intermediate is
 * allocated in the current arena. */
struct PicoTensor* pico_gpt_loss(struct PicoGPT* model, const int32_t* tokens,
                                 const int32_t* targets);
int pico_gpt_num_params(const struct PicoGPT* model);
struct PicoTensor* pico_gpt_param(struct PicoGPT* model, int index);
/* name of param `index`: "emb", "layers.<l>.{attn_norm,wq,wk,wv,wo,ffn_norm,w1,w3,w2}",
 * "final_norm", "lm_head" (NULL when out of range) */
const char* pico_gpt_param_name(const struct PicoGPT* model, int index);
void pico_gpt_free(struct PicoGPT* model);

/* ---- host <-> device (no reference counterpart: pico's data is host memory) ----
 * Each copies numel floats of the tensor's storage and synchronises the
 * stream; 0 on success. */
int pico_tensor_copy_from_host(struct PicoTensor* t, const float* src);
int pico_tensor_copy_to_host(const struct PicoTensor* t, float* dst);
int pico_tensor_grad_to_host(const struct PicoTensor* t, float* dst);
int pico_tensor_grad_from_host(struct PicoTensor* t, const float* src);
/* device copy of n int32 values in the current arena (NULL on failure) */
int32_t* pico_ids_to_device(const int32_t* host_ids, int64_t n);
/* overwrite n device ids (from pico_ids_to_device) with host values; 0 on success */
int pico_ids_update(int32_t* device_ids, const int32_t* host_ids, int64_t n);

/* ---- runtime ---- */
int pico_gpu_synchronize(void);
void* pico_gpu_stream(void);            /* the hipStream_t every launch uses */
void pico_gpu_set_stream(void* stream); /* NULL restores the library's own */
const char* pico_gpu_last_error(void);  /* "" when no error has occurred */
/* device bytes this library holds now, and the most it has held (params,
 * arena blocks, optimizer moments, scratch) */
void pico_gpu_memory(size_t* in_use, size_t* peak);
void pico_gpu_clear_error(void);
/* testing aid (no reference counterpart): the next n requests for the
 * optional split-K scratch of a matmul product are refused as if the device
 * were out of memory, so the product runs unsplit; no error is recorded for
 * them and pico_backward carries on */
void pico_gpu_fail_next_workspaces(int n);

/* ---- matmul precision (no reference counterpart: pico is fp32 only) ----
 * PICO_MATMUL_FP32 (the default): pico_matmul, the fused attention's
 * products and their gradients multiply in fp32 on the fp32 matrix cores,
 * within the fp32 parity contract.
 * PICO_MATMUL_BF16: their operands are rounded to bf16 (nearest even) and
 * multiplied on the bf16 matrix cores, accumulating in fp32; tensors, the
 * softmax statistics and every other op stay fp32.  Faster, and outside the
 * fp32 parity contract (relative error of order 2^-8 per operand).  An
 * attention node's backward uses the precision its forward ran in.
 * PICO_MATMUL_BF16X3: pico_matmul's products, the fused attention's and
 * their gradients take three bf16 products per fp32 one (pk_gemm_bf16x3_f32,
 * pk_flash_attn_*_bf16x3_f32): within about 1e-5 of fp32, inside the 1e-4
 * parity bound.
 * PICO_MATMUL_FP8: pico_matmul's products and their gradients run on MX8
 * operands (OCP e4m3 with a power-of-two scale per 32 values along the
 * contraction, pk_gemm_mx8_f32; a parameter cast once per change), the fused
 * attention on e4m3 with per-tensor power-of-two scales
 * (pk_flash_attn_*_fp8_f32), accumulating in fp32.  Relative error of order
 * 2^-4 per operand: far outside the fp32 parity contract, for experiments.
 * Returns 0, or nonzero for an unknown value. */
#define PICO_MATMUL_FP32 0
#define PICO_MATMUL_BF16 1
#define PICO_MATMUL_BF16X3 2
#define PICO_MATMUL_FP8 3
int pico_set_matmul_precision(int precision);
int pico_get_matmul_precision(void);

/* ---- checkpoints (no reference counterpart: the reference's params are plain
 * float arrays, src/tensor.h:14-15, and nothing is ever saved) ----
 * A safetensors file: 8-byte little-endian header length, a JSON header mapping
 * each name to {"dtype", "shape", "data_offsets"}, then the raw little-endian
 * bytes; any safetensors reader opens it.  tensors[i] is saved as F32 under
 * names[i] (or "param.<i>" when names is NULL).  With an AdamW optimizer, each
 * of its params also saves "<name>.adam_m" and "<name>.adam_v", plus
 * "adamw.step" (I32), and the hyper-parameters go to the header's metadata.
 * pico_checkpoint_load checks every name, dtype and shape before writing
 * anything, then restores the tensors and the optimizer's moments and step
 * count (its params must already be added), so a resumed run continues exactly
 * as the saved one.  Both return 0, or nonzero with pico_gpu_last_error() set. */
int pico_checkpoint_save(const char* path, int n, struct PicoTensor* const* tensors,
                         const char* const* names, const struct PicoOptimAdamW* adamw);
int pico_checkpoint_load(const char* path, int n, struct PicoTensor* const* tensors,
                         const char* const* names, struct PicoOptimAdamW* adamw);

/* ---- device graphs (no reference counterpart) ----
 * Record the launches of one training step once and replay them with a
 * single call.  Between pico_graph_begin() and pico_graph_end() every op,
 * pico_backward and optimizer step is recorded on the library's stream
 * instead of running.  Nothing may allocate device memory, copy to or from
 * the host, or wait on the device meanwhile, so:
 *   - run the step once eagerly first (the arena's device blocks, the GEMM
 *     workspace and the optimizer's tables then exist, and an arena_reset
 *     before capturing makes the captured step reuse the same addresses);
 *   - pass token ids as device pointers (pico_ids_to_device into an arena
 *     that outlives the graph) and refresh them with pico_ids_update;
 *   - read results (the loss tensor of the captured step) after
 *     pico_graph_launch.
 * A refused call fails the capture: pico_graph_end then returns NULL, with
 * the reason in pico_gpu_last_error().  A replay repeats the captured work
 * exactly (same kernels, same arguments, same addresses). */
struct PicoGraph;
int pico_graph_begin(void);
struct PicoGraph* pico_graph_end(void);
int pico_graph_launch(struct PicoGraph* graph);
void pico_graph_free(struct PicoGraph* graph);

#ifdef __cplusplus
}
#endif
