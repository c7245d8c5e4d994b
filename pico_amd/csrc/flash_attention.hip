// pico_amd/csrc/flash_attention.hip -- fused causal attention for head size 64
// on gfx950 fp32 matrix cores (no reference counterpart: pico has no attention;
// the softmax Jacobian it would need is the comment at src/autograd.h:38-40).
//
// q, k, v, o are token-major [B*T, H*64]; head h of sequence b is the column
// block h*64.. of rows b*T..; lse is [B*H, T] (natural log).  The score matrix
// is never written to memory: a workgroup keeps its 128 query (or key) rows in
// registers and streams 64-row blocks of the other operand through LDS.
//
// Layout.  v_mfma_f32_32x32x2f32 takes, from lane l, A[l%32][k] and B[k][l%32]
// for the lane's k-slot, and returns C[row][l%32] with row = 8*(r/4) +
// 4*(l/32) + r%4 in accumulator register r.  Computing S^T = K.Q^T (keys as
// rows, queries as columns) puts one query in each lane: the row max, the
// exponentials, the row sum and the rescale of the output are all lane-local
// (plus one exchange between the two 32-lane halves), and P^T sits in the
// registers in exactly the B-operand order the next product O^T += V^T.P^T
// needs, with the contraction over keys taken in the order
// kv(s, half) = 8*(s/4) + 4*half + s%4.  The backward kernels use the same
// construction: dK/dV keep one key per lane, dQ one query per lane.
//
// Scores are carried in log2 units (Q is pre-scaled by scale*log2(e)) so the
// exponentials are exp2.
#include <math.h>

#include "pk_common.h"

namespace {

constexpr int HD = 64;        // head size handled here
constexpr int ROWS = 128;     // query (or key) rows per workgroup: 4 waves x 32
constexpr int BLK = 64;       // rows of the streamed operand per LDS stage
constexpr int LDT = HD + 4;   // padded LDS row stride (floats)
constexpr int TILE = BLK * LDT;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct FlashParams {
    const float *q, *k, *v, *o, *dout, *lse, *dsum;
    float *out, *lse_out, *dq, *dk, *dv, *dsum_out;
    int64_t B, H, T, D;  // D = H*64, the row stride
    float scale;         // softmax scale (normally 1/8)
    int flags;
};

__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for(int r = 0; r < 16; ++r) z[r] = 0.0f;
    return z;
}

// row offset (within a 32-row sub-block) of accumulator register r for lane half h
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// 32 consecutive floats of one row: the lane's k-slots 32*h .. 32*h+31
__device__ __forceinline__ void load_frag32(const float* __restrict__ row, int h, float (&f)[32],
                                            float mul) {
    const f32x4* p = reinterpret_cast<const f32x4*>(row + 32 * h);
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const f32x4 x = p[i];
        f[4 * i + 0] = x[0] * mul;
        f[4 * i + 1] = x[1] * mul;
        f[4 * i + 2] = x[2] * mul;
        f[4 * i + 3] = x[3] * mul;
    }
}

// one 64x64 block (rows row0.. of a head) into registers: 4 float4 per thread
__device__ __forceinline__ void fetch_block(const float* __restrict__ base, int64_t D, int64_t row0,
                                            f32x4 (&v)[4]) {
#pragma unroll
    for(int i = 0; i < 4; ++i) {
        const int idx = threadIdx.x + 256 * i;
        const int r = idx >> 4, c4 = idx & 15;
        v[i] = *reinterpret_cast<const f32x4*>(base + (row0 + r) * D + 4 * c4);
    }
}

__device__ __forceinline__ void store_block(float* lds, const f32x4 (&v)[4]) {
#pragma unroll
    for(int i = 0; i < 4; ++i) {
        const int idx = threadIdx.x + 256 * i;
        const int r = idx >> 4, c4 = idx & 15;
        *reinterpret_cast<f32x4*>(lds + r * LDT + 4 * c4) = v[i];
    }
}

// acc (+)= A.B over the 64 head dims: A row = lds row (sub*32 + lane%32),
// B = the lane's register fragment
__device__ __forceinline__ f32x16 dot_rows(const float* lds, int sub, int lq, int lh,
                                           const float (&bf)[32], f32x16 acc) {
    const f32x4* a4 = reinterpret_cast<const f32x4*>(lds + (sub * 32 + lq) * LDT + 32 * lh);
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const f32x4 a = a4[i];
        acc = mfma(a[0], bf[4 * i + 0], acc);
        acc = mfma(a[1], bf[4 * i + 1], acc);
        acc = mfma(a[2], bf[4 * i + 2], acc);
        acc = mfma(a[3], bf[4 * i + 3], acc);
    }
    return acc;
}

// acc (+)= X^T . W over the 32 rows of sub-block `sub`: A[d][row] read from the
// row-major lds tile (column cb*32 + lane%32), B = the lane's 16 registers w,
// rows taken in acc_row order
__device__ __forceinline__ f32x16 dot_cols(const float* lds, int sub, int cb, int lq, int lh,
                                           const f32x16& w, f32x16 acc) {
#pragma unroll
    for(int s = 0; s < 16; ++s) {
        const float a = lds[(sub * 32 + acc_row(s, lh)) * LDT + cb * 32 + lq];
        acc = mfma(a, w[s], acc);
    }
    return acc;
}

// store a transposed accumulator pair (d rows, one row of the output per lane)
// as out[row][d] * mul (+ out if accumulate), 4 consecutive d per float4
__device__ __forceinline__ void store_rowT(float* __restrict__ dst, const f32x16 (&acc)[2], int lh,
                                           float mul, bool accumulate) {
#pragma unroll
    for(int cb = 0; cb < 2; ++cb)
#pragma unroll
        for(int g = 0; g < 4; ++g) {
            f32x4 v;
#pragma unroll
            for(int e = 0; e < 4; ++e) v[e] = acc[cb][4 * g + e] * mul;
            f32x4* p = reinterpret_cast<f32x4*>(dst + cb * 32 + 8 * g + 4 * lh);
            if(accumulate) v += *p;
            *p = v;
        }
}

// ======================================================================= forward
// Workgroup: 128 queries of one (b, h), 4 waves of 32.  Heaviest query blocks
// (the ones that see the most keys) are dispatched first.
__global__ __launch_bounds__(256, 2) void flash_fwd(FlashParams p) {
    __shared__ __attribute__((aligned(16))) float sK[2][TILE];
    __shared__ __attribute__((aligned(16))) float sV[2][TILE];
    const int64_t BH = p.B * p.H, nqb = p.T / ROWS;
    const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base;
    const int w = threadIdx.x / 64, l = threadIdx.x % 64, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;

    float qf[32];
    load_frag32(Q + qi * p.D, lh, qf, p.scale * kLog2e);
    f32x16 o[2] = {zero16(), zero16()};
    float m = -INFINITY, lsum = 0.0f;

    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    f32x4 rk[4], rv[4];
    fetch_block(K, p.D, 0, rk);
    fetch_block(V, p.D, 0, rv);
    store_block(sK[0], rk);
    store_block(sV[0], rv);
    for(int j = 0; j < nkv; ++j) {
        const int st = j & 1;
        __syncthreads();
        const bool more = j + 1 < nkv;
        if(more) {
            fetch_block(K, p.D, (int64_t)(j + 1) * BLK, rk);
            fetch_block(V, p.D, (int64_t)(j + 1) * BLK, rv);
        }
        const int64_t kv0 = (int64_t)j * BLK;
        if(kv0 <= q0 + 31) {  // some key of this block is visible to this wave
            f32x16 s0 = dot_rows(sK[st], 0, lq, lh, qf, zero16());
            f32x16 s1 = dot_rows(sK[st], 1, lq, lh, qf, zero16());
            if(kv0 + BLK - 1 > q0) {  // the block crosses this wave's diagonal
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    if(kv0 + acc_row(r, lh) > qi) s0[r] = -INFINITY;
                    if(kv0 + 32 + acc_row(r, lh) > qi) s1[r] = -INFINITY;
                }
            }
            float mx = -INFINITY;
#pragma unroll
            for(int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m, mx);
            const float alpha = exp2f(m - mn);  // m = -inf on the first block: 0
            float ls = 0.0f;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                s0[r] = exp2f(s0[r] - mn);
                s1[r] = exp2f(s1[r] - mn);
                ls += s0[r] + s1[r];
            }
            ls += __shfl_xor(ls, 32, 64);
            lsum = lsum * alpha + ls;
            m = mn;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                o[0][r] *= alpha;
                o[1][r] *= alpha;
            }
            // O^T[d][q] += sum_kv V[kv][d] P^T[kv][q]
#pragma unroll
            for(int cb = 0; cb < 2; ++cb) {
                o[cb] = dot_cols(sV[st], 0, cb, lq, lh, s0, o[cb]);
                o[cb] = dot_cols(sV[st], 1, cb, lq, lh, s1, o[cb]);
            }
        }
        if(more) {
            store_block(sK[st ^ 1], rk);
            store_block(sV[st ^ 1], rv);
        }
    }
    store_rowT(p.out + base + qi * p.D, o, lh, 1.0f / lsum, false);
    if(lh == 0 && p.lse_out) p.lse_out[bh * p.T + qi] = (m + log2f(lsum)) * kLn2;
}

// ============================================================ backward: D = rowsum(dO*O)
__global__ void flash_dsum(FlashParams p) {
    const int64_t BH = p.B * p.H, n = BH * p.T;
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t bh = i / p.T, t = i % p.T, b = bh / p.H, h = bh % p.H;
        const int64_t off = (b * p.T + t) * p.D + h * HD;
        const f32x4* x = reinterpret_cast<const f32x4*>(p.dout + off);
        const f32x4* y = reinterpret_cast<const f32x4*>(p.o + off);
        float s = 0.0f;
#pragma unroll
        for(int c = 0; c < HD / 4; ++c) {
            const f32x4 a = x[c], o = y[c];
            s += a[0] * o[0] + a[1] * o[1] + a[2] * o[2] + a[3] * o[3];
        }
        p.dsum_out[i] = s;
    }
}

// ================================================================ backward: dK, dV
// Workgroup: 128 keys of one (b, h), one key per lane; query blocks of 64 with
// q >= key are streamed through LDS (Q and dO rows, their lse and D).
//   S = Q.K^T (per lane: its key's column)        P = exp2(S' - lse2)
//   dV^T += dO^T.P         dP = dO.V^T           dS = P*(dP - D)
//   dK^T += Q^T.dS  (x scale at the end)
__global__ __launch_bounds__(256, 2) void flash_bwd_dkdv(FlashParams p) {
    __shared__ __attribute__((aligned(16))) float sQ[2][TILE];
    __shared__ __attribute__((aligned(16))) float sO[2][TILE];  // dO rows
    __shared__ float sL[2][BLK], sDs[2][BLK];
    const int64_t BH = p.B * p.H, nkb = p.T / ROWS;
    const int64_t kb = (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base, *dO = p.dout + base;
    const float* lse = p.lse + bh * p.T;
    const float* dsum = p.dsum + bh * p.T;
    const int w = threadIdx.x / 64, l = threadIdx.x % 64, lq = l & 31, lh = l >> 5;
    const int64_t k0 = kb * ROWS + w * 32, ki = k0 + lq;
    (void)nkb;

    float kf[32], vf[32];
    load_frag32(K + ki * p.D, lh, kf, p.scale * kLog2e);
    load_frag32(V + ki * p.D, lh, vf, 1.0f);
    f32x16 dv[2] = {zero16(), zero16()}, dk[2] = {zero16(), zero16()};

    const int j0 = (int)(kb * ROWS / BLK), nq = (int)(p.T / BLK);
    f32x4 rq[4], ro[4];
    float rl = 0.0f, rd = 0.0f;
    auto fetch = [&](int j) {
        fetch_block(Q, p.D, (int64_t)j * BLK, rq);
        fetch_block(dO, p.D, (int64_t)j * BLK, ro);
        if(threadIdx.x < BLK) {
            rl = lse[(int64_t)j * BLK + threadIdx.x] * kLog2e;
            rd = dsum[(int64_t)j * BLK + threadIdx.x];
        }
    };
    auto put = [&](int st) {
        store_block(sQ[st], rq);
        store_block(sO[st], ro);
        if(threadIdx.x < BLK) {
            sL[st][threadIdx.x] = rl;
            sDs[st][threadIdx.x] = rd;
        }
    };
    fetch(j0);
    put(0);
    for(int j = j0; j < nq; ++j) {
        const int st = (j - j0) & 1;
        __syncthreads();
        const bool more = j + 1 < nq;
        if(more) fetch(j + 1);
        const int64_t qs = (int64_t)j * BLK;
        if(qs + BLK - 1 >= k0) {  // some query of this block sees this wave's keys
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                f32x16 s = dot_rows(sQ[st], sub, lq, lh, kf, zero16());
                f32x16 dp = dot_rows(sO[st], sub, lq, lh, vf, zero16());
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const int qr = sub * 32 + acc_row(r, lh);
                    const bool vis = qs + qr >= ki;
                    const float pr = vis ? exp2f(s[r] - sL[st][qr]) : 0.0f;
                    s[r] = pr;
                    dp[r] = pr * (dp[r] - sDs[st][qr]);
                }
#pragma unroll
                for(int cb = 0; cb < 2; ++cb) {
                    dv[cb] = dot_cols(sO[st], sub, cb, lq, lh, s, dv[cb]);
                    dk[cb] = dot_cols(sQ[st], sub, cb, lq, lh, dp, dk[cb]);
                }
            }
        }
        if(more) put(st ^ 1);
    }
    store_rowT(p.dv + base + ki * p.D, dv, lh, 1.0f, (p.flags & PK_ACCUM3) != 0);
    store_rowT(p.dk + base + ki * p.D, dk, lh, p.scale, (p.flags & PK_ACCUM2) != 0);
}

// =================================================================== backward: dQ
// Workgroup: 128 queries of one (b, h), one query per lane; key blocks of 64
// with key <= query streamed through LDS (K and V rows).
//   S^T = K.Q^T   P^T = exp2(S'^T - lse2)   dP^T = V.dO^T   dS^T = P^T*(dP^T - D)
//   dQ^T += K^T.dS^T  (x scale at the end)
__global__ __launch_bounds__(256, 2) void flash_bwd_dq(FlashParams p) {
    __shared__ __attribute__((aligned(16))) float sK[2][TILE];
    __shared__ __attribute__((aligned(16))) float sV[2][TILE];
    const int64_t BH = p.B * p.H, nqb = p.T / ROWS;
    const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base, *dO = p.dout + base;
    const int w = threadIdx.x / 64, l = threadIdx.x % 64, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;

    float qf[32], of[32];
    load_frag32(Q + qi * p.D, lh, qf, p.scale * kLog2e);
    load_frag32(dO + qi * p.D, lh, of, 1.0f);
    const float l2 = p.lse[bh * p.T + qi] * kLog2e;
    const float dd = p.dsum[bh * p.T + qi];
    f32x16 dq[2] = {zero16(), zero16()};

    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    f32x4 rk[4], rv[4];
    fetch_block(K, p.D, 0, rk);
    fetch_block(V, p.D, 0, rv);
    store_block(sK[0], rk);
    store_block(sV[0], rv);
    for(int j = 0; j < nkv; ++j) {
        const int st = j & 1;
        __syncthreads();
        const bool more = j + 1 < nkv;
        if(more) {
            fetch_block(K, p.D, (int64_t)(j + 1) * BLK, rk);
            fetch_block(V, p.D, (int64_t)(j + 1) * BLK, rv);
        }
        const int64_t kv0 = (int64_t)j * BLK;
        if(kv0 <= q0 + 31) {
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                f32x16 s = dot_rows(sK[st], sub, lq, lh, qf, zero16());
                f32x16 dp = dot_rows(sV[st], sub, lq, lh, of, zero16());
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const bool vis = kv0 + sub * 32 + acc_row(r, lh) <= qi;
                    const float pr = vis ? exp2f(s[r] - l2) : 0.0f;
                    dp[r] = pr * (dp[r] - dd);
                }
#pragma unroll
                for(int cb = 0; cb < 2; ++cb) dq[cb] = dot_cols(sK[st], sub, cb, lq, lh, dp, dq[cb]);
            }
        }
        if(more) {
            store_block(sK[st ^ 1], rk);
            store_block(sV[st ^ 1], rv);
        }
    }
    store_rowT(p.dq + base + qi * p.D, dq, lh, p.scale, (p.flags & PK_ACCUM) != 0);
}

int flash_check(const char* who, int64_t B, int64_t H, int64_t T, int64_t hd, const void* a,
                const void* b, const void* c) {
    if(B < 0 || H < 1 || T < 0) return pk::fail("%s: bad sizes", who);
    if(hd != HD) return pk::fail("%s: head size %lld (this kernel handles 64)", who, (long long)hd);
    if(T % ROWS) return pk::fail("%s: T=%lld must be a multiple of %d", who, (long long)T, ROWS);
    if(!pk::aligned16(a) || !pk::aligned16(b) || !pk::aligned16(c))
        return pk::fail("%s: q, k, v must be 16-byte aligned", who);
    if(B * H * (T / ROWS) > 0x7fffffff) return pk::fail("%s: problem too large", who);
    return PK_OK;
}

}  // namespace

extern "C" int pk_flash_attn_supported(int64_t T, int64_t hd) {
    return hd == HD && T > 0 && T % ROWS == 0;
}

extern "C" int pk_flash_attn_fwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, float scale,
                                     const float* q, const float* k, const float* v, float* o,
                                     float* lse, pk_stream_t stream) {
    int rc = flash_check("pk_flash_attn_fwd_f32", B, H, T, hd, q, k, v);
    if(rc) return rc;
    if(B == 0 || T == 0) return PK_OK;
    if(!o || !pk::aligned16(o)) return pk::fail("pk_flash_attn_fwd_f32: o NULL or unaligned");
    FlashParams p = {};
    p.q = q;
    p.k = k;
    p.v = v;
    p.out = o;
    p.lse_out = lse;
    p.B = B;
    p.H = H;
    p.T = T;
    p.D = H * HD;
    p.scale = scale;
    const unsigned grid = (unsigned)(B * H * (T / ROWS));
    flash_fwd<<<grid, 256, 0, pk::as_stream(stream)>>>(p);
    return pk::launch_status("pk_flash_attn_fwd_f32");
}

extern "C" size_t pk_flash_attn_bwd_workspace(int64_t B, int64_t H, int64_t T) {
    return B > 0 && H > 0 && T > 0 ? (size_t)(B * H * T) * sizeof(float) : 0;
}

extern "C" int pk_flash_attn_bwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, float scale,
                                     const float* q, const float* k, const float* v,
                                     const float* o, const float* lse, const float* dout,
                                     float* dq, float* dk, float* dv, void* workspace,
                                     size_t workspace_bytes, int flags, pk_stream_t stream) {
    int rc = flash_check("pk_flash_attn_bwd_f32", B, H, T, hd, q, k, v);
    if(rc) return rc;
    if(B == 0 || T == 0) return PK_OK;
    if(!o || !lse || !dout || !dq || !dk || !dv)
        return pk::fail("pk_flash_attn_bwd_f32: NULL pointer");
    if(!pk::aligned16(o) || !pk::aligned16(dout) || !pk::aligned16(dq) || !pk::aligned16(dk) ||
       !pk::aligned16(dv))
        return pk::fail("pk_flash_attn_bwd_f32: o, dout, dq, dk, dv must be 16-byte aligned");
    if(!workspace || workspace_bytes < pk_flash_attn_bwd_workspace(B, H, T))
        return pk::fail("pk_flash_attn_bwd_f32: workspace needs %zu bytes",
                        pk_flash_attn_bwd_workspace(B, H, T));
    FlashParams p = {};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.lse = lse;
    p.dout = dout;
    p.dq = dq;
    p.dk = dk;
    p.dv = dv;
    p.dsum = static_cast<const float*>(workspace);
    p.dsum_out = static_cast<float*>(workspace);
    p.B = B;
    p.H = H;
    p.T = T;
    p.D = H * HD;
    p.scale = scale;
    p.flags = flags;
    hipStream_t st = pk::as_stream(stream);
    flash_dsum<<<pk::grid_for(B * H * T, 256), 256, 0, st>>>(p);
    if((rc = pk::launch_status("pk_flash_attn_bwd_f32 (rowsum)"))) return rc;
    const unsigned grid = (unsigned)(B * H * (T / ROWS));
    flash_bwd_dkdv<<<grid, 256, 0, st>>>(p);
    if((rc = pk::launch_status("pk_flash_attn_bwd_f32 (dK, dV)"))) return rc;
    flash_bwd_dq<<<grid, 256, 0, st>>>(p);
    return pk::launch_status("pk_flash_attn_bwd_f32 (dQ)");
}
