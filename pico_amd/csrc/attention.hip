// pico_amd/csrc/attention.hip -- causal self-attention forward and backward as
// a chain of batched fp32 MFMA GEMMs and causal-softmax row kernels.
//
// Heads are addressed in place inside the token-major [B*T, H*hd] activations
// (a two-level batch: outer stride T*ld per sequence, inner stride hd per
// head), so no permute copies are made.  q, k, v and their gradients have
// row stride ld (>= H*hd: column blocks of a fused projection); o and dout
// are contiguous.  The probabilities P [B*H, T, T] are
// materialised once in the forward and reused by the backward.  Causality is
// exploited at tile granularity: score tiles wholly above the diagonal are not
// computed, and the products with P / dS stop (or start) their k loop at the
// diagonal.
//
//   S  = scale * Q K^T           gemm N,T  causal 1
//   P  = softmax_causal(S), lse  row kernel (in place)
//   O  = P V                     gemm N,N  causal 2
// backward:
//   dP = dO V^T                  gemm N,T  causal 1
//   dS = P * (dP - rowsum(P*dP)) row kernel (in place)
//   dV (+)= P^T dO               gemm T,N  causal 3
//   dQ (+)= scale * dS K         gemm N,N  causal 2
//   dK (+)= scale * dS^T Q       gemm T,N  causal 3
#include "pk_common.h"

extern "C" int pk_attn_causal_fwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                      float scale, const float* q, const float* k, const float* v,
                                      float* o, float* lse, float* P, pk_stream_t stream) {
    if(B < 0 || H < 1 || T < 0 || hd < 1) return pk::fail("pk_attn_causal_fwd_f32: bad sizes");
    if(ld < H * hd) return pk::fail("pk_attn_causal_fwd_f32: row stride below H*hd");
    if(B == 0 || T == 0) return PK_OK;
    if(!q || !k || !v || !o || !P) return pk::fail("pk_attn_causal_fwd_f32: NULL pointer");
    const int64_t D = H * hd, BH = B * H;
    int rc = pk_gemm_batched_f32('N', 'T', T, T, hd, scale, q, ld, T * ld, hd, k, ld, T * ld, hd,
                                 0.0f, P, T, H * T * T, T * T, BH, H, 1, stream);
    if(rc) return rc;
    rc = pk_causal_softmax_fwd_f32(BH, T, 1.0f, P, P, lse, stream);
    if(rc) return rc;
    return pk_gemm_batched_f32('N', 'N', T, hd, T, 1.0f, P, T, H * T * T, T * T, v, ld, T * ld,
                               hd, 0.0f, o, D, T * D, hd, BH, H, 2, stream);
}

extern "C" int pk_attn_causal_bwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                      float scale, const float* q, const float* k, const float* v,
                                      const float* P, const float* dout, float* dq, float* dk,
                                      float* dv, float* dP_ws, int flags, pk_stream_t stream) {
    if(B < 0 || H < 1 || T < 0 || hd < 1) return pk::fail("pk_attn_causal_bwd_f32: bad sizes");
    if(ld < H * hd) return pk::fail("pk_attn_causal_bwd_f32: row stride below H*hd");
    if(B == 0 || T == 0) return PK_OK;
    if(!q || !k || !v || !P || !dout || !dP_ws)
        return pk::fail("pk_attn_causal_bwd_f32: NULL input pointer");
    const int64_t D = H * hd, BH = B * H;
    const float beta_q = (flags & PK_ACCUM) ? 1.0f : 0.0f;
    const float beta_k = (flags & PK_ACCUM2) ? 1.0f : 0.0f;
    const float beta_v = (flags & PK_ACCUM3) ? 1.0f : 0.0f;
    int rc = pk_gemm_batched_f32('N', 'T', T, T, hd, 1.0f, dout, D, T * D, hd, v, ld, T * ld, hd,
                                 0.0f, dP_ws, T, H * T * T, T * T, BH, H, 1, stream);
    if(rc) return rc;
    if(dv) {
        rc = pk_gemm_batched_f32('T', 'N', T, hd, T, 1.0f, P, T, H * T * T, T * T, dout, D, T * D,
                                 hd, beta_v, dv, ld, T * ld, hd, BH, H, 3, stream);
        if(rc) return rc;
    }
    rc = pk_causal_softmax_bwd_f32(BH, T, P, dP_ws, dP_ws, stream);
    if(rc) return rc;
    if(dq) {
        rc = pk_gemm_batched_f32('N', 'N', T, hd, T, scale, dP_ws, T, H * T * T, T * T, k, ld,
                                 T * ld, hd, beta_q, dq, ld, T * ld, hd, BH, H, 2, stream);
        if(rc) return rc;
    }
    if(dk) {
        rc = pk_gemm_batched_f32('T', 'N', T, hd, T, scale, dP_ws, T, H * T * T, T * T, q, ld,
                                 T * ld, hd, beta_k, dk, ld, T * ld, hd, BH, H, 3, stream);
        if(rc) return rc;
    }
    return PK_OK;
}
