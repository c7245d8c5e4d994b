/*
 * include/pico_hip.h -- the C-ABI launcher layer of pico's MI355X (gfx950) backend.
 *
 * Every entry point takes raw DEVICE pointers plus sizes and layout scalars,
 * launches hand-written HIP kernels on the given stream, allocates nothing,
 * and returns a status: 0 on success, PK_EINVAL (-1) for arguments it refuses
 * (with a message available from pk_last_error()), otherwise the hipError_t
 * value of the failed launch.  Nothing here synchronises the stream.
 *
 * These are the GPU twins of pico's CPU kernel seam (src/kernels/cpu_kernels.h
 * :13-100) and of the commented-out pico_*_gpu stubs in src/ops.c:42-44,86-88,
 * 130-132; pico's op layer and backward hooks call them when a tensor's
 * backend is GPU.  Matrices are row-major, as pico's tensors are.
 *
 * "flags" arguments: bit 0 (PK_ACCUM) makes the first output accumulate
 * (out += result, the += contract of pico's backward hooks, src/autograd.h
 * :25-29); bit 1 (PK_ACCUM2) does the same for a second output.  Without the
 * bit the output is overwritten and never read.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* pk_stream_t; /* a hipStream_t; NULL is the null stream */

#define PK_OK 0
#define PK_EINVAL (-1)

#define PK_ACCUM 1
#define PK_ACCUM2 2
#define PK_ACCUM3 4
/* pk_rmsnorm_bwd_into_f32 with dg == NULL: leave dg's partial sums in the
 * workspace for pk_rmsnorm_dg_reduce_f32 */
#define PK_RMS_KEEP_PARTIALS 8
/* pk_flash_attn_bwd_f32: recompute dQ's scores instead of passing dS through
 * the workspace (which then holds only the row constants) */
#define PK_FLASH_RECOMPUTE 16

/* ---- runtime ---------------------------------------------------------- */
const char* pk_last_error(void);
/* device properties of the current device: CU count, peak clock kHz, gcnArch name */
int pk_device_info(int* cu_count, int* clock_khz, char* arch, int arch_len);

/* ---- GEMM --------------------------------------------------------------
 * C[M,N] = alpha * op(A) . op(B) + beta * C   (beta == 0: C is not read)
 * op(A) is [M,K]: ta 'N' -> A stored [M,K] (lda >= K); ta 'T' -> A stored [K,M] (lda >= M)
 * op(B) is [K,N]: tb 'N' -> B stored [K,N] (ldb >= N); tb 'T' -> B stored [N,K] (ldb >= K)
 * Replaces pico_matmul_cpu (src/kernels/cpu_kernels.h:46-55, forward C = A.B with
 * out zeroed, i.e. beta = 0) and both loops of pico_matmul_backward
 * (src/autograd.h:96-130: dA += dC.B^T is ('N','T', beta 1), dB += A^T.dC is
 * ('T','N', beta 1)); a pico_transpose_2d view (src/tensor.c:230-244) maps to 'T'. */
int pk_gemm_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                pk_stream_t stream);

/* pk_gemm_f32 with a caller-provided device workspace.  When C has too few
 * 128x128 tiles to fill the chip (a linear layer's weight gradient: M, N of the
 * order of d_model, K = tokens), K is split into slices whose partial products
 * go to the workspace and are summed by a second kernel in slice order, so the
 * result is deterministic.  pk_gemm_workspace_f32 returns the bytes a split
 * of this shape needs in any layout (0 when no layout splits it: A^T.B splits
 * wherever another layout does, while A.B and A.B^T with a long K run unsplit
 * once 64x64 tiles give every CU two); a NULL or smaller workspace runs the
 * product unsplit.  Same backward roles as pk_gemm_f32 (src/autograd.h:96-130). */
size_t pk_gemm_workspace_f32(int64_t M, int64_t N, int64_t K);
int pk_gemm_ex_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                   int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                   void* workspace, size_t workspace_bytes, pk_stream_t stream);

/* pk_gemm_ex_f32 that allocates nothing and takes no workspace.  No
 * counterpart in the reference (pico allocates freely); it is for callers that
 * cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  A product that splits K puts its
 * partial planes in a static device array of pk_gemm_noalloc_scratch_bytes()
 * (128 MiB) that each GPU holds until the process ends; a product whose
 * partials need more (in its own layout; pk_gemm_workspace_f32 is the largest
 * over layouts) is refused with PK_EINVAL and a message.  Results equal pk_gemm_ex_f32's bit for bit.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, two threads) race, so serialise them. */
size_t pk_gemm_noalloc_scratch_bytes(void);
int pk_gemm_noalloc_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                        const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                        float* C, int64_t ldc, pk_stream_t stream);

/* The same products with fp8 multiplies (no reference counterpart): op(A)
 * and op(B) are clamped to +-448 and rounded to e4m3 (OCP FP8 E4M3: bias 7, 3
 * mantissa bits, nearest even; NaN stays NaN) on their way to LDS and
 * multiplied on the fp8 matrix cores (v_mfma_f32_32x32x16_fp8_fp8),
 * accumulating in fp32.  A product of two e4m3 values is exact in fp32, so
 * the result equals the fp32 product of the rounded operands up to fp32
 * summation error.  C and the workspace contract are as in pk_gemm_f32 /
 * pk_gemm_ex_f32. */
int pk_gemm_fp8_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                    const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                    float* C, int64_t ldc, pk_stream_t stream);
int pk_gemm_ex_fp8_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                       const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                       float* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                       pk_stream_t stream);

/* Products with a fused epilogue (no reference counterpart: pico runs a matmul
 * and the op that consumes it as two passes over memory).  precision selects
 * the multiplies: 0 fp32 (as pk_gemm_ex_f32), 1 bf16 (pk_gemm_ex_bf16_f32),
 * 2 three bf16 products (pk_gemm_ex_bf16x3_f32), 3 fp8 (pk_gemm_ex_fp8_f32).
 * pk_gemm_add_f32: C = alpha * op(A).op(B) + beta * X, X [M,N] with row stride
 *   ldx (X == C with ldx == ldc is pk_gemm_ex_f32's accumulate); a residual
 *   connection x + a.W in one pass.  ldx == 0 adds the one row X [N] to every
 *   row: a Linear layer's x.W + b (src/nn/linear.c:57-64) in one pass.  Same
 *   workspace contract as pk_gemm_ex_f32.
 * pk_gemm_swiglu_bwd_f32: dh = alpha * op(A).op(B) [M,N] is the upstream
 *   gradient of h = silu(gate) * up and is never stored; each tile writes
 *   dgate (+)= dh*up*s*(1 + gate*(1-s)) (flags bit 0 accumulates) and
 *   dup (+)= dh*gate*s (bit 1), s = sigmoid(gate), with pk_swiglu_bwd_f32's
 *   arithmetic; gate, up [M,N] (row strides ldg, ldu) are read in the tile's
 *   epilogue, dgate and dup (distinct) share the row stride ldd.  In a
 *   transformer block it is the down projection's input gradient dY.W2^T
 *   turned straight into the gate/up gradients.
 * pk_gemm_swiglu_fwd_f32: ('N','N' only, batch 1) C = alpha * A.B [M, N]
 *   with N = 2F (C = [gate | up], B = [W1 | W3]) and h [M, F] (row stride
 *   ldh) = silu(gate) * up with pk_swiglu_fwd_f32's arithmetic; C holds the
 *   values pk_gemm_ex_f32 writes.  A tile takes F-aligned pairs of gate and
 *   up columns, so F must be a multiple of 32 (4 for whole-column tiles of
 *   64); refused otherwise.  The gate/up projection of a SwiGLU block and
 *   its activation in one pass. */
/* 1 when the fp32 products above (pk_gemm_f32, pk_gemm_ex_f32, pk_gemm_add_f32)
 * run an [M, N] output with inner size K (contiguous operands) on the
 * small-product kernels: an output that the tiled kernels leave short of one
 * tile per CU and one round of 32x32 tiles covers, K <= 1024.  Those split K
 * over a workgroup's waves, so their sums round differently from the tiled
 * kernels that the SwiGLU epilogues below run on; pico's fused SwiGLU ops use
 * their composition for such shapes, so fused and composed stay bit-equal. */
int pk_gemm_small_product_f32(int64_t M, int64_t N, int64_t K);
int pk_gemm_add_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                    const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                    const float* X, int64_t ldx, float* C, int64_t ldc, int precision,
                    const float* fp8_scales, void* workspace, size_t workspace_bytes,
                    pk_stream_t stream);
int pk_gemm_swiglu_bwd_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                           const float* A, int64_t lda, const float* B, int64_t ldb,
                           const float* gate, int64_t ldg, const float* up, int64_t ldu,
                           float* dgate, float* dup, int64_t ldd, int flags, int precision,
                           const float* fp8_scales, pk_stream_t stream);
int pk_gemm_swiglu_fwd_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                           const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                           int64_t ldc, float* h, int64_t ldh, int precision,
                           const float* fp8_scales, pk_stream_t stream);

/* fp8 operand scaling (no reference counterpart).  scales[0] and scales[1]
 * (device memory) receive 2^floor(log2(448 / max|A|)) and the same for B (1 for
 * an all-zero matrix): the largest powers of two that keep each operand
 * within e4m3's finite range, so small values (gradients of order 1e-5, far
 * below e4m3's smallest subnormal 2^-9) are not flushed to zero.  A [ra, ca]
 * and B [rb, cb] are given as stored, with row strides lda, ldb.  Passed as
 * fp8_scales to the fused launchers with precision 3, the operands are
 * multiplied by them before rounding and the product divided by both
 * (powers of two: exact).  NULL scales mean 1 and 1, as in pk_gemm_fp8_f32. */
int pk_fp8_scales_f32(int64_t ra, int64_t ca, const float* A, int64_t lda, int64_t rb, int64_t cb,
                      const float* B, int64_t ldb, float* scales, pk_stream_t stream);

/* Narrow-operand fp8 products (no reference counterpart): the operands are
 * quantized once into byte matrices and the product streams 1 byte per
 * element from HBM (v_mfma_scale_f32_32x32x64_f8f6f4, scales 2^0).
 * pk_fp8_quantized_bytes: bytes of the buffer pk_fp8_quantize_f32 fills for
 *   R rows of K values, and its row stride (*ld, bytes) = K rounded up to 128;
 *   rows are rounded up to a multiple of 256.
 * pk_fp8_quantize_f32: Q[r][k] = e4m3(clamp(scale * op(X)[r][k], +-448))
 *   (nearest even, NaN stays NaN) for r < R, k < K, and 0 in the padding up
 *   to ldq and to R rounded up to 256 rows; op(X) = X [R, K] (trans 0) or
 *   X^T with X [K, R] (trans 1), row stride ldx; *scale in device memory
 *   (pk_fp8_scales_f32 writes such scales).  ldq >= K rounded up to 128, a
 *   multiple of 16, Q 16-byte aligned.
 * pk_gemm_fp8q_f32: C [M, N] = alpha / (scales[0] * scales[1]) * A.B^T
 *   (+ beta * C) with A [M, K], B [N, K] e4m3 as pk_fp8_quantize_f32 writes
 *   them (row strides lda, ldb in bytes; their padding rows and columns are
 *   read and must be zero); accumulation in fp32.  For C = op(X).op(Y)
 *   quantize op(X) as A and op(Y)^T as B.  Row strides are K rounded up to
 *   128 (pk_fp8_quantized_bytes), so that a product runs an even number of
 *   64-byte slices. */
size_t pk_fp8_quantized_bytes(int64_t R, int64_t K, int64_t* ld);
int pk_fp8_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans,
                        const float* scale, uint8_t* Q, int64_t ldq, pk_stream_t stream);
int pk_gemm_fp8q_f32(int64_t M, int64_t N, int64_t K, float alpha, const uint8_t* A, int64_t lda,
                     const uint8_t* B, int64_t ldb, const float* scales, float beta, float* C,
                     int64_t ldc, pk_stream_t stream);

/* MX8 products (no reference counterpart): OCP Microscaling MXFP8, e4m3
 * values with one E8M0 power-of-two scale per 32 consecutive values of a row,
 * applied by the matrix core (v_mfma_scale_f32_32x32x64_f8f6f4).  No
 * tensor-wide maximum is needed, so an operand is quantized in one pass, and
 * each block keeps e4m3's 3 mantissa bits whatever the other blocks' sizes.
 * pk_mx8_bytes: bytes of an MX8 matrix of R rows of K values: Rp = R rounded
 *   up to 256, Kp = K rounded up to 128; Rp * Kp e4m3 bytes (row stride Kp),
 *   then the scales, Kp / 64 slices of Rp rows of 2 bytes (the scale bytes
 *   of k 0-31 and 32-63 of the slice).
 * pk_mx8_quantize_f32: Q = op(X) [R, K] (X [R, K] for trans 0, X^T with
 *   X [K, R] for trans 1, row stride ldx) as an MX8 matrix: for each block
 *   of 32 of a row with largest magnitude a, e is the smallest integer with
 *   a * 2^-e <= 448 (0 for an all-zero block; held to [-127, 127]), the
 *   scale byte is e + 127 and the values e4m3(clamp(x * 2^-e, +-448))
 *   (nearest even, NaN stays NaN); padding values are 0.  Q 16-byte aligned.
 * pk_gemm_mx8_f32: C [M, N] = alpha * A.B^T + beta * X with A [M, K] and
 *   B [N, K] MX8 matrices; fp32 accumulation.  X [M, N] has row stride ldx
 *   (X == C with ldx == ldc accumulates); ldx 0 adds the one row X [N] to
 *   every row; X is not read when beta is 0.  For C = op(P).op(R) quantize
 *   op(P) as A and op(R)^T as B. */
size_t pk_mx8_bytes(int64_t R, int64_t K);
int pk_mx8_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, void* Q,
                        pk_stream_t stream);
int pk_gemm_mx8_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                    float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                    pk_stream_t stream);
/* pk_gemm_mx8_f32 with a caller-provided device workspace: a product with
 * too few tiles to fill the chip (a weight gradient: M, N of the order of
 * d_model, K = tokens) splits K; the splits' sums go to the workspace as
 * fp32 planes and a second kernel adds them in plane order (deterministic).
 * pk_gemm_mx8_workspace returns the bytes the split needs (0: no split); a
 * NULL or smaller workspace runs the product unsplit.  pk_gemm_mx8_plan
 * reports the launch a shape gets with enough workspace: the C tile (256 x
 * 256, 256 x 128, 128 x 256 or 128 x 128) and the number of K splits. */
/* pk_mx8_quantize2_f32: both MX8 casts of one row-major X [M, N] (row stride
 * ldx) from one read of it: QR = X as an [M, N] MX8 matrix and QT = X^T as an
 * [N, M] one (pk_mx8_bytes(M, N) and pk_mx8_bytes(N, M) bytes), byte for byte
 * what pk_mx8_quantize_f32 writes for each.  A product's upstream gradient
 * needs both: dY as the input gradient's A operand, dY^T as the weight
 * gradient's B operand. */
int pk_mx8_quantize2_f32(int64_t M, int64_t N, const float* X, int64_t ldx, void* QR, void* QT,
                         pk_stream_t stream);
size_t pk_gemm_mx8_workspace(int64_t M, int64_t N, int64_t K);
int pk_gemm_mx8_ex_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                       float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                       void* workspace, size_t workspace_bytes, pk_stream_t stream);
int pk_gemm_mx8_plan(int64_t M, int64_t N, int64_t K, int* tile_m, int* tile_n, int* splits);

/* bf16 operands held in HBM (no reference counterpart: pico is fp32 only).
 * A bf16 matrix of R rows and K values per row is Rp = R rounded up to 256
 * rows of Kv = K rounded up to 64 values, 2 bytes each (row stride 2 Kv),
 * pk_bf16q_bytes(R, K) bytes: every value of op(X) rounded to nearest even,
 * zeros in the padding.  pk_bf16q_quantize_f32 writes op(X) (trans as in
 * pk_mx8_quantize_f32), pk_bf16q_quantize2_f32 both X [M, N] and X^T from one
 * read.  pk_gemm_bf16q_f32 / _ex_f32: C [M, N] = alpha * A.B^T + beta * X for
 * bf16 A [M, K] and B [N, K], on the bf16 matrix cores with fp32
 * accumulation, the MX8 product's kernel and contract (workspace, K split,
 * ldx 0 for a broadcast row).  Each product of two bf16 values is exact in
 * fp32, so the result is the fp32 product of the rounded operands up to fp32
 * summation error. */
size_t pk_bf16q_bytes(int64_t R, int64_t K);
int pk_bf16q_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, void* Q,
                          pk_stream_t stream);
int pk_bf16q_quantize2_f32(int64_t M, int64_t N, const float* X, int64_t ldx, void* QR, void* QT,
                           pk_stream_t stream);
size_t pk_gemm_bf16q_workspace(int64_t M, int64_t N, int64_t K);
int pk_gemm_bf16q_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                      float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                      pk_stream_t stream);
int pk_gemm_bf16q_ex_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                         float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                         void* workspace, size_t workspace_bytes, pk_stream_t stream);

/* Split-bf16 operands held in HBM, for fp32 products from three bf16 ones (no
 * reference counterpart: they replace the fp32 multiplies of
 * src/kernels/cpu_kernels.h:46-55 within the fp32 parity bound).  A value x is
 * kept as hi = bf16(x) and lo = bf16(x - hi), both nearest even.  A matrix of
 * R rows and K values per row is Rp = R rounded up to 256 rows of Kv = K
 * rounded up to 32 values, each row Kv / 16 groups of 64 bytes -- a group's 16
 * hi parts, then their 16 lo parts -- (row stride 4 Kv bytes,
 * pk_bf16x3q_bytes(R, K) bytes), zeros in the padding.  pk_bf16x3q_quantize_f32
 * writes op(X) (trans as in pk_mx8_quantize_f32).  pk_gemm_bf16x3q_f32 /
 * _ex_f32: C [M, N] = alpha * A.B^T + beta * X for split A [M, K] and B [N, K]
 * as ahi.bhi + ahi.blo + alo.bhi per 16 values of K on the bf16 matrix cores,
 * accumulating in fp32 (the MX8 product's kernel and contract).  That is
 * pk_gemm_bf16x3_f32's arithmetic in its order, so an unsplit product equals
 * pk_gemm_bf16x3_f32 without a workspace bit for bit: within about 1e-5 of
 * the fp32 product. */
size_t pk_bf16x3q_bytes(int64_t R, int64_t K);
int pk_bf16x3q_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, void* Q,
                            pk_stream_t stream);
size_t pk_gemm_bf16x3q_workspace(int64_t M, int64_t N, int64_t K);
int pk_gemm_bf16x3q_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                        float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                        pk_stream_t stream);
int pk_gemm_bf16x3q_ex_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                           float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                           void* workspace, size_t workspace_bytes, pk_stream_t stream);

/* The same products with bf16 multiplies (no reference counterpart: pico is
 * fp32 only): op(A) and op(B) are rounded to bf16 (nearest even) and
 * multiplied on the bf16 matrix cores, accumulating in fp32; C and the
 * workspace contract are as in pk_gemm_f32 / pk_gemm_ex_f32.  Each product
 * of two bf16 values is exact in fp32, so the result equals the fp32 product
 * of the rounded operands up to fp32 summation error. */
int pk_gemm_bf16_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                     const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                     float* C, int64_t ldc, pk_stream_t stream);
int pk_gemm_ex_bf16_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                        const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                        float* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                        pk_stream_t stream);
/* fp32 products from three bf16 ones (no reference counterpart): each operand
 * x is split as hi = bf16(x), lo = bf16(x - hi) on its way to LDS, and
 * a.b is taken as ahi.bhi + ahi.blo + alo.bhi on the bf16 matrix cores,
 * accumulating in fp32.  hi + lo is x to 2^-17, and the dropped alo.blo is
 * below 2^-16 of a.b, so the result is within about 1e-5 (norm-wise) of the
 * fp32 product, against 2^-8 for pk_gemm_bf16_f32.  C and the workspace
 * contract are as in pk_gemm_f32 / pk_gemm_ex_f32. */
int pk_gemm_bf16x3_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                       const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                       float* C, int64_t ldc, pk_stream_t stream);
int pk_gemm_ex_bf16x3_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                          const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                          float* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                          pk_stream_t stream);

/* Batched form: batch index z = outer*inner_count + inner; operand X of batch z
 * starts at X + outer*sX_outer + inner*sX_inner.  'causal' restricts work for
 * attention-shaped products (no reference counterpart: pico's matmul is 2-D
 * only, src/ops.c:150):
 *   0 dense
 *   1 only C[r,c] with c <= r is produced (tiles wholly above the diagonal are skipped)
 *   2 op(A)[r,k] is zero for k > r (the k loop stops at the tile's last row)
 *   3 op(A)[r,k] is zero for k < r (the k loop starts at the tile's first row) */
int pk_gemm_batched_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                        const float* A, int64_t lda, int64_t sA_outer, int64_t sA_inner,
                        const float* B, int64_t ldb, int64_t sB_outer, int64_t sB_inner,
                        float beta, float* C, int64_t ldc, int64_t sC_outer, int64_t sC_inner,
                        int64_t batch, int64_t inner_count, int causal, pk_stream_t stream);

/* ---- elementwise (pico ops.c:12-142, autograd.h:53-94) -----------------
 * op: 0 add, 1 sub, 2 mul.  ndim <= 8.  a_strides / b_strides are each
 * operand's element strides mapped onto the output's dims (0 on a broadcast
 * dim), the map pico's map_index computes (src/tensor.h:122-138).  out is
 * contiguous with shape out_shape. */
int pk_binary_f32(int op, int ndim, const int64_t* out_shape, const int64_t* a_strides,
                  const int64_t* b_strides, const float* a, const float* b, float* out,
                  pk_stream_t stream);
/* gradient of one operand: gx[j] (+)= sum over output elements i that read
 * x[j] of  g[i]            (add; or sub for operand a)
 *          -g[i]           (sub, operand b: which = 1)
 *          g[i] * other[i] (mul)
 * x_strides / other_strides are each operand's element strides mapped onto
 * the output dims as above (0 on a broadcast dim); gx is laid out with x's
 * strides, as pico's grads share their tensor's strides (src/autograd.h:61-63),
 * and x_numel is the number of elements x holds. */
int pk_binary_bwd_f32(int op, int which, int ndim, const int64_t* out_shape,
                      const int64_t* x_strides, const int64_t* other_strides, int64_t x_numel,
                      const float* gout, const float* other, float* gx, int flags,
                      pk_stream_t stream);
/* unary op: 0 sqrt, 1 sin, 2 cos, 3 tan, 4 tanh, 5 log (src/kernels/cpu/cpu_scalar.h:32-37) */
int pk_unary_f32(int op, int64_t n, const float* x, float* y, pk_stream_t stream);
/* gx (+)= local derivative x gy, with the reference's expressions
 * (src/autograd.h:132-176, including its tanh form g - y*y) */
int pk_unary_bwd_f32(int op, int64_t n, const float* x, const float* y, const float* gy,
                     float* gx, int flags, pk_stream_t stream);
/* y = max(x, 0) (NaN -> 0); gx (+)= gy * (y > 0)   (src/act/activations.c:16-18,
 * src/act/autograd.h:9-17) */
int pk_relu_f32(int64_t n, const float* x, float* y, pk_stream_t stream);
int pk_relu_bwd_f32(int64_t n, const float* y, const float* gy, float* gx, int flags,
                    pk_stream_t stream);
int pk_fill_f32(int64_t n, float value, float* x, pk_stream_t stream);
/* x[r*ld + c] = value for r < rows, c < cols (no reference counterpart: the
 * zeros of a column-block view's gradient that nothing wrote) */
int pk_fill2d_f32(int64_t rows, int64_t cols, float value, float* x, int64_t ld,
                  pk_stream_t stream);
/* x[i] = mean + std * z_i, z_i ~ N(0,1) from a counter-based generator: element
 * i draws two uniforms from the 64-bit mix of (seed, i) and applies Box-Muller
 * (u1 in (0,1]), so the values do not depend on the launch shape.  Seeded
 * parameter initialisation (no reference counterpart: pico_randn,
 * src/tensor.c:348-367, builds normals from graph ops on the host). */
int pk_fill_normal_f32(int64_t n, uint64_t seed, float mean, float std, float* x,
                       pk_stream_t stream);
/* y (+)= alpha * (*alpha_dev if non-NULL) * x */
int pk_axpy_f32(int64_t n, float alpha, const float* alpha_dev, const float* x, float* y,
                int flags, pk_stream_t stream);
/* out[0] (+)= scale * sum(x) */
int pk_reduce_sum_f32(int64_t n, const float* x, float scale, float* out, int flags,
                      pk_stream_t stream);

/* ---- optimizers ---------------------------------------------------------
 * SGD: p -= lr*g, product rounded first (src/optim/SGD.c:29-37).
 * AdamW: decoupled decay then bias-corrected Adam (no reference code; the
 * reference's optim.h:19-23 only names Adam).  g == NULL means a zero gradient. */
int pk_sgd_f32(int64_t n, float lr, float* p, const float* g, pk_stream_t stream);
/* pk_sgd_f32 over `count` tensors (p[i], g[i], n[i] elements) in as few
 * launches as possible (32 tensors each): the loop over an optimizer's params
 * of src/optim/SGD.c:29-37 as one launch, same arithmetic per element. */
int pk_sgd_multi_f32(int count, float* const* p, const float* const* g, const int64_t* n,
                     float lr, pk_stream_t stream);
int pk_adamw_f32(int64_t n, float lr, float beta1, float beta2, float eps, float weight_decay,
                 int step, float* p, const float* g, float* m, float* v, pk_stream_t stream);

/* AdamW over many tensors in one launch, with the step count kept on the
 * device so a captured graph replays correctly (no reference counterpart; the
 * multi-tensor form of pk_adamw_f32, same arithmetic per element).
 *   pk_adamw_prep_f32: *step += 1, then coef[0] = lr / (1 - beta1^step) and
 *     coef[1] = sqrt(1 - beta2^step) (both computed in double, rounded once).
 *   pk_adamw_multi_f32: chunks is a device array of nchunks descriptors, each
 *     at most PK_ADAMW_CHUNK elements of one tensor starting 16-byte aligned;
 *     g == NULL in a descriptor means a zero gradient. */
#define PK_ADAMW_CHUNK 65536
typedef struct PkAdamwChunk {
    float* p;
    const float* g;
    float* m;
    float* v;
    int64_t n;
} PkAdamwChunk;
int pk_adamw_prep_f32(int32_t* step, float lr, float beta1, float beta2, float* coef,
                      pk_stream_t stream);
int pk_adamw_multi_f32(int64_t nchunks, const PkAdamwChunk* chunks, float lr, float beta1,
                       float beta2, float eps, float weight_decay, const float* coef,
                       pk_stream_t stream);

/* ---- fused row kernels (no reference code; planned at todo.md:95) --------
 * softmax cross-entropy, one pass over each row of logits [R,V] (row stride ldz):
 *   loss_rows[r] = logsumexp(z_r) - z_r[labels[r]]        (if loss_rows != NULL)
 *   dlogits[r,:] (+)= s * (softmax(z_r) - onehot(y_r))     (if dlogits != NULL)
 * with s = scale * (*scale_dev) when scale_dev (a device float, e.g. the
 * upstream gradient of the loss) is non-NULL, else s = scale.
 * A label outside [0,V) gives NaN loss and a zero gradient row. */
int pk_xent_fwd_bwd_f32(int64_t R, int64_t V, const float* logits, int64_t ldz,
                        const int32_t* labels, float* loss_rows, float* dlogits, int64_t ldd,
                        float scale, const float* scale_dev, int flags, pk_stream_t stream);
/* pk_xent_fwd_bwd_f32 (scale_dev NULL) and out[0] (+)= mean_scale * sum of the
 * loss rows, summed as pk_reduce_sum_f32 sums them (flags bit 0: dlogits
 * accumulate, bit 1: out accumulates).  Up to 1024 rows of at most 64
 * classes take one launch; above that loss_rows is required and it is the
 * two calls. */
int pk_xent_mean_f32(int64_t R, int64_t V, const float* logits, int64_t ldz, const int32_t* labels,
                     float* loss_rows, float* dlogits, int64_t ldd, float scale, int flags,
                     float mean_scale, float* out, pk_stream_t stream);
/* idx[r] = argmax_j x[r,j]: first maximum wins; a NaN is the maximum (first NaN wins) */
int pk_argmax_f32(int64_t R, int64_t V, const float* x, int64_t ldx, int32_t* idx,
                  pk_stream_t stream);
/* RMSNorm over rows of x [R,C]: y = x * rstd * g, rstd = (mean(x^2) + eps)^-1/2 */
int pk_rmsnorm_fwd_f32(int64_t R, int64_t C, float eps, const float* x, const float* g, float* y,
                       float* rstd, pk_stream_t stream);
/* dx (+)= rstd*(g*dy) - x*rstd^3*mean(g*dy*x)   (flags bit 0)
 * dg (+)= sum_r dy*x*rstd                       (flags bit 1)
 * needs pk_rmsnorm_bwd_workspace(R, C) bytes of device workspace */
size_t pk_rmsnorm_bwd_workspace(int64_t R, int64_t C);
int pk_rmsnorm_bwd_f32(int64_t R, int64_t C, const float* x, const float* g, const float* rstd,
                       const float* dy, float* dx, float* dg, int flags, void* workspace,
                       size_t workspace_bytes, pk_stream_t stream);
/* as pk_rmsnorm_bwd_f32, with the accumulated term of dx read from dx_in:
 * dx = dx_in + rstd*(g*dy) - x*rstd^3*mean(g*dy*x), or without the dx_in term
 * when dx_in is NULL (dx_in == dx is pk_rmsnorm_bwd_f32's accumulate); flags
 * bit 1 accumulates dg, bit 0 is ignored.  pico's backward uses it to add the
 * residual stream's gradient without first copying it into dx. */
int pk_rmsnorm_bwd_into_f32(int64_t R, int64_t C, const float* x, const float* g,
                            const float* rstd, const float* dy, const float* dx_in, float* dx,
                            float* dg, int flags, void* workspace, size_t workspace_bytes,
                            pk_stream_t stream);
/* dg (+)= the partial sums a pk_rmsnorm_bwd_into_f32 call with dg == NULL and
 * PK_RMS_KEEP_PARTIALS left in `workspace` (same R, C); flags bit 0
 * accumulates.  The two calls may run on different streams, ordered by the
 * caller.  pico's backward runs this one on its weight-gradient stream. */
int pk_rmsnorm_dg_reduce_f32(int64_t R, int64_t C, const void* workspace, size_t workspace_bytes,
                             float* dg, int flags, pk_stream_t stream);
/* SwiGLU on [R,F] gate/up pairs (row strides lda, ldu, ldh): h = silu(a) * u */
int pk_swiglu_fwd_f32(int64_t R, int64_t F, const float* a, int64_t lda, const float* u,
                      int64_t ldu, float* h, int64_t ldh, pk_stream_t stream);
/* da (+)= dh*u*s*(1 + a*(1-s)) (bit 0), du (+)= dh*a*s (bit 1), s = sigmoid(a);
 * da and du share the row stride ldd */
int pk_swiglu_bwd_f32(int64_t R, int64_t F, const float* a, int64_t lda, const float* u,
                      int64_t ldu, const float* dh, int64_t ldh, float* da, float* du,
                      int64_t ldd, int flags, pk_stream_t stream);

/* ---- causal attention ----------------------------------------------------
 * q, k, v, o are token-major [B*T, H*hd]; head h of batch b owns columns
 * h*hd..h*hd+hd-1 of rows b*T..b*T+T-1.  q, k, v and their gradients dq, dk,
 * dv have row stride ld >= H*hd (H*hd when contiguous; larger when they are
 * column blocks of one fused projection); o and dout are contiguous.  lse is
 * [B*H, T] (log-sum-exp of each
 * score row, kept for the backward).  P is a [B*H, T, T] buffer the forward
 * fills with the probabilities (zero above the diagonal) and the backward
 * reads; dP_ws is a [B*H, T, T] scratch buffer for the backward.
 * scale is normally 1/sqrt(hd). */
int pk_attn_causal_fwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                           float scale, const float* q, const float* k, const float* v, float* o,
                           float* lse, float* P, pk_stream_t stream);
/* dq, dk, dv (+)= gradients: flags bit 0 (PK_ACCUM) accumulates dq, bit 1
 * (PK_ACCUM2) dk, bit 2 (PK_ACCUM3) dv; a NULL gradient pointer is skipped.
 * The writes happen in the order dv, dq, dk, so aliased outputs accumulate
 * correctly when the later ones carry their accumulate bit. */
int pk_attn_causal_bwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                           float scale, const float* q, const float* k, const float* v,
                           const float* P, const float* dout, float* dq, float* dk, float* dv,
                           float* dP_ws, int flags, pk_stream_t stream);
/* Fused causal attention for head size 64 (any T): the scores
 * are never written to memory.  Same layouts and lse as above; q, k, v, o,
 * dout, dq, dk, dv 16-byte aligned and ld a multiple of 4.
 * pk_flash_attn_supported(T, hd) says
 * whether these apply.  The backward needs pk_flash_attn_bwd_workspace(B, H,
 * T) bytes (per 64-query block: lse in base 2, then the row sums of dO*O)
 * and writes dv, then dk, then dq, each accumulating when its flags bit is
 * set (PK_ACCUM dq, PK_ACCUM2 dk, PK_ACCUM3 dv).  The dS tiles take about
 * 2*B*H*T^2 bytes of that workspace; with PK_FLASH_RECOMPUTE in flags (fp32
 * only) the dQ kernel recomputes the scores and dP block by block instead --
 * three products per block rather than one, the same results bit for bit --
 * and the workspace needs only pk_flash_attn_bwd_workspace_recompute(B, H, T)
 * = 8*B*H*T bytes. */
int pk_flash_attn_supported(int64_t T, int64_t hd);
int pk_flash_attn_fwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                          float scale, const float* q, const float* k, const float* v, float* o,
                          float* lse, pk_stream_t stream);
size_t pk_flash_attn_bwd_workspace(int64_t B, int64_t H, int64_t T);
size_t pk_flash_attn_bwd_workspace_recompute(int64_t B, int64_t H, int64_t T);
int pk_flash_attn_bwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                          float scale, const float* q, const float* k, const float* v,
                          const float* o, const float* lse, const float* dout, float* dq,
                          float* dk, float* dv, void* workspace, size_t workspace_bytes, int flags,
                          pk_stream_t stream);
/* The same fused attention with bf16 multiplies (no reference counterpart:
 * pico is fp32 only).  Q (pre-scaled), K, V, dO and the probabilities P and
 * dS are rounded to bf16 (nearest even) where they enter a matrix product;
 * the softmax statistics, exponentials and accumulators stay fp32, and every
 * tensor, lse and the workspace are as in the fp32 entry points. */
int pk_flash_attn_fwd_bf16_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                               float scale, const float* q, const float* k, const float* v,
                               float* o, float* lse, pk_stream_t stream);
int pk_flash_attn_bwd_bf16_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                               float scale, const float* q, const float* k, const float* v,
                               const float* o, const float* lse, const float* dout, float* dq,
                               float* dk, float* dv, void* workspace, size_t workspace_bytes,
                               int flags, pk_stream_t stream);
/* The same fused attention with fp32 products from three bf16 ones (no
 * reference counterpart; within the fp32 parity bound): every operand of a
 * product -- q, k, v, dout and the probabilities and dS formed in the kernels
 * -- as hi = bf16(x) and lo = bf16(x - hi), each product as hi.hi + hi.lo +
 * lo.hi on the bf16 matrix cores with fp32 accumulation (lo.lo, below 2^-16 of
 * a product, dropped); softmax statistics, exponentials and accumulators fp32.
 * Arguments, workspace and flags as the fp32 entry points. */
int pk_flash_attn_fwd_bf16x3_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                 float scale, const float* q, const float* k, const float* v,
                                 float* o, float* lse, pk_stream_t stream);
int pk_flash_attn_bwd_bf16x3_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                 float scale, const float* q, const float* k, const float* v,
                                 const float* o, const float* lse, const float* dout, float* dq,
                                 float* dk, float* dv, void* workspace, size_t workspace_bytes,
                                 int flags, pk_stream_t stream);
/* The same fused attention with fp8 multiplies (no reference counterpart):
 * OCP e4m3 operands on the 32x32x64 scaled matrix cores, fp32 accumulation.
 * q, k, v and dout enter as e4m3(x * 2^-e) per tensor, e the smallest
 * exponent that puts the tensor's largest magnitude (times scale*log2(e)
 * for the operand that carries the softmax scale) within 448; the products
 * undo 2^-e exactly.  P enters as e4m3(256 P), dS with a power of two per
 * 32 rows of a 64-row block (its largest magnitude within 448).  The softmax
 * statistics, exponentials and accumulators stay fp32.  amax: 4 floats of
 * device memory; the forward writes max|q|, max|k|, max|v| into amax[0..2],
 * the backward reads them (as the forward left them) and writes max|dout|
 * into amax[3].  Everything else as in the fp32 entry points
 * (PK_FLASH_RECOMPUTE is refused). */
int pk_flash_attn_fwd_fp8_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                              float scale, const float* q, const float* k, const float* v,
                              float* o, float* lse, float* amax, pk_stream_t stream);
int pk_flash_attn_bwd_fp8_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                              float scale, const float* q, const float* k, const float* v,
                              const float* o, const float* lse, const float* dout, float* dq,
                              float* dk, float* dv, float* amax, void* workspace,
                              size_t workspace_bytes, int flags, pk_stream_t stream);
/* the two row kernels inside the chain, exposed for tests:
 * P = softmax(scale*S) over j <= i, zero for j > i, lse per row (P may alias S) */
int pk_causal_softmax_fwd_f32(int64_t BH, int64_t T, float scale, const float* S, float* P,
                              float* lse, pk_stream_t stream);
/* dS = P * (dP - rowsum(dP*P)) for j <= i, zero above (dS may alias dP) */
int pk_causal_softmax_bwd_f32(int64_t BH, int64_t T, const float* P, const float* dP, float* dS,
                              pk_stream_t stream);

/* ---- embedding -------------------------------------------------------------
 * out[i,:] = table[ids[i],:]; dtable[ids[i],:] += dout[i,:], the adds into
 * one row made in increasing i (the sequential loop's order: deterministic).
 * An id outside [0,vocab) reads as a zero row and adds nothing.  The backward
 * needs pk_embed_bwd_workspace(n) bytes of device workspace; it groups equal
 * ids with a stable radix sort of (id, position) pairs (8 bits a pass), so
 * each row's adds keep their position order, then sums each run of equal ids
 * into its row. */
int pk_embed_fwd_f32(int64_t n, int64_t d, int64_t vocab, const int32_t* ids, const float* table,
                     float* out, pk_stream_t stream);
size_t pk_embed_bwd_workspace(int64_t n);
int pk_embed_bwd_f32(int64_t n, int64_t d, int64_t vocab, const int32_t* ids, const float* dout,
                     float* dtable, void* workspace, size_t workspace_bytes, pk_stream_t stream);

#ifdef __cplusplus
}
#endif
