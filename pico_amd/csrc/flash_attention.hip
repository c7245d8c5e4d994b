// pico_amd/csrc/flash_attention.hip -- fused causal attention for head size 64
// on gfx950 fp32 matrix cores (no reference counterpart: pico has no attention;
// the softmax Jacobian it would need is the comment at src/autograd.h:38-40).
//
// q, k, v, o are token-major [B*T, H*64]; head h of sequence b is the column
// block h*64.. of rows b*T..; lse is [B*H, T] (natural log).  q, k, v (and
// their gradients) may have a row stride ld > H*64 -- column blocks of one
// fused [B*T, 3*H*64] projection; o and dout are contiguous.  The score matrix
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

#include <algorithm>
#include <queue>
#include <utility>
#include <vector>

#include "pk_common.h"

namespace {

constexpr int HD = 64;        // head size handled here
constexpr int ROWS = 128;     // query (or key) rows per workgroup: 4 waves x 32
constexpr int BLK = 64;       // rows of the streamed operand per LDS stage
constexpr int LDT = HD + 4;   // padded LDS row stride (floats)
constexpr int TILE = BLK * LDT;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int64_t kCUs = 256;  // MI355X

struct FlashParams {
    const float *q, *k, *v, *o, *dout, *lse, *dsum;
    float *out, *lse_out, *dq, *dk, *dv, *dsum_out;
    float* ds;  // dS tiles: written by the dK/dV kernel, read by the dQ kernel
    int64_t B, H, T, D;  // D = H*64: row stride of o, dout (and the output)
    int64_t Tp;          // T rounded up to 128: the grid and workspace layout
    int64_t ld;          // row stride of q, k, v and dq, dk, dv (>= D)
    float scale;         // softmax scale (normally 1/8)
    int flags;
    const float* amax;   // fp8 kernels: max|q|, max|k|, max|v|, max|dO|
};

// Which block (a forward or dQ query block) each of a launch's first
// slots*kCUs workgroups takes.  `slots` workgroups of a kernel
// share a CU, and the dispatcher places workgroup b on CU b % 256 as slot
// b / 256 (measured: b, b+256, b+512 run on one CU, all from the start), so
// this table decides each CU's work.  The host fills it longest-first, each
// block to the CU with the least work so far; config 5's forward CUs then hold
// 26-28 key blocks each (the plain heaviest-first order left 24-30, and the
// launch waited on the 30s).  Later workgroups take the remaining blocks
// heaviest first as slots free.  The table only moves work between CUs:
// every block is computed the same way wherever it runs.  The dK/dV kernel
// (two slots per CU, so a third of its workgroups start as slots free) keeps
// the plain heaviest-first order: the table measured slower there (backward
// 330.1 against 323.3 us at config 5).
constexpr int kMaxSlots = 4;
struct FlashPlan {
    uint16_t rank[kMaxSlots * kCUs];  // workgroup b < n takes rank[b]; others rank b
    int n;
};
// ranks run heaviest first: rank r is block (nblk-1-r/BH) of the forward and
// dQ (a query block seeing the most keys first), block r/BH of dK/dV (a key
// block seen by the most queries first; its rank is its workgroup index), of
// head r%BH
__device__ __forceinline__ int64_t plan_rank(const FlashPlan& plan) {
    return (int)blockIdx.x < plan.n ? (int64_t)plan.rank[blockIdx.x] : (int64_t)blockIdx.x;
}

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
                                            float mul, bool ok = true) {
    if(!ok) {  // a row past the sequence's end (T not a multiple of 128): zeros
#pragma unroll
        for(int i = 0; i < 32; ++i) f[i] = 0.0f;
        return;
    }
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

// The same product for both 32-row sub-blocks of the tile at once, the two
// accumulator chains alternating: consecutive MFMAs are then independent, so
// neither waits for the previous one's result.  The 128-bit operand reads run
// two k-groups (16 products) ahead of their use; scheduling barriers keep
// that order.  Every chain still accumulates k in increasing order, as
// dot_rows does.
__device__ __forceinline__ void dot_rows2(const float* lds, int lq, int lh, const float (&bf)[32],
                                          f32x16& acc0, f32x16& acc1) {
    const f32x4* a0 = reinterpret_cast<const f32x4*>(lds + lq * LDT + 32 * lh);
    const f32x4* a1 = reinterpret_cast<const f32x4*>(lds + (32 + lq) * LDT + 32 * lh);
    f32x4 x[8], y[8];
    x[0] = a0[0];
    y[0] = a1[0];
    x[1] = a0[1];
    y[1] = a1[1];
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        if(i + 2 < 8) {
            x[i + 2] = a0[i + 2];
            y[i + 2] = a1[i + 2];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            acc0 = mfma(x[i][e], bf[4 * i + e], acc0);
            acc1 = mfma(y[i][e], bf[4 * i + e], acc1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
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

// acc0 (+)= X^T.W over columns lq and acc1 over columns 32 + lq of the tile's
// 64 rows, the rows taken as dot_cols takes them (sub-block 0, then 1, each in
// acc_row order), so each chain accumulates in dot_cols's order.  The two
// chains alternate, and the operand reads (one 2-float read per pair of
// products) run two groups of 8 products ahead, fenced by scheduling barriers
// so that only three groups' operands are live.
__device__ __forceinline__ void dot_cols2(const float* lds, int lq, int lh, const f32x16 (&w)[2],
                                          f32x16& acc0, f32x16& acc1) {
    const float* base = lds + 4 * lh * LDT + lq;
    float a0[32], a1[32];
    auto rd = [&](int t) {
        const int sub = t >> 4, s = t & 15;
        const float* q = base + (sub * 32 + 8 * (s >> 2) + (s & 3)) * LDT;
        a0[t] = q[0];
        a1[t] = q[32];
    };
#pragma unroll
    for(int t = 0; t < 8; ++t) rd(t);
#pragma unroll
    for(int g = 0; g < 8; ++g) {
        if(g + 2 < 8) {
#pragma unroll
            for(int t = 4 * (g + 2); t < 4 * (g + 3); ++t) rd(t);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for(int t = 4 * g; t < 4 * g + 4; ++t) {
            acc0 = mfma(a0[t], w[t >> 4][t & 15], acc0);
            acc1 = mfma(a1[t], w[t >> 4][t & 15], acc1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
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

// ------------------------------------------------- direct-to-LDS block loads
// buffer_load_dwordx4 ... lds writes lane l's 16 bytes to LDS at (wave-uniform
// base) + 16*l, so one instruction fills 1 KB of a tile straight from global
// memory, without passing through registers.  A padded 64-row tile (stride
// LDT = 68 floats) is 17 KB: instruction n (0..16) covers floats 256n ..
// 256n+255, and lane l lands at float f = 256n + 4l, i.e. row f / 68, column
// f % 68.  Column 64 is the padding: that lane fetches the row's first chunk
// again, which lands in the pad and is never read.  Wave w issues
// instructions w, w+4, w+8, w+12, and wave 0 also instruction 16.
//
// Each block load builds a buffer resource that starts at the block's first
// row and ends at the head's last element (row T-1, column 63), and puts the
// whole per-lane offset in the bounds-checked vector offset (the scalar offset
// of a buffer access is not bounds checked).  Rows at or past T -- the padding
// rows of a last block when T is not a multiple of 128 -- therefore load as
// zeros without reading memory: not the next sequence's rows, and nothing past
// the end of the tensor.
constexpr int LOADS = TILE * 4 / 1024;  // 17
static_assert(TILE * 4 == LOADS * 1024, "a tile is a whole number of 1 KB loads");
typedef __attribute__((address_space(3))) void lds_ptr_t;

// rows row0.. of a head (row stride D) that holds T rows; empty when row0 >= T
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const float* head, int64_t T,
                                                             int64_t D, int64_t row0) {
    const int64_t bytes = T > row0 ? ((T - 1 - row0) * D + HD) * 4 : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(head + row0 * D), (short)0,
                                             (int)bytes, 0x00020000);
}

// this lane's byte offsets (relative to the block's first row) for its wave's
// instructions; slot 4 is used by wave 0 only
struct BlockLoad {
    unsigned off[5];
    __device__ __forceinline__ BlockLoad(int64_t D, int w, int l) {
#pragma unroll
        for(int i = 0; i < 5; ++i) {
            const int n = i < 4 ? w + 4 * i : LOADS - 1;
            const int f = 256 * n + 4 * l, r = f / LDT, c = f % LDT;
            off[i] = (unsigned)((r * D + (c < HD ? c : 0)) * 4);
        }
    }
    // issue the loads of rows row0..row0+63 of a head of T rows into tile
    __device__ __forceinline__ void issue(const float* head, int64_t T, int64_t D, int64_t row0,
                                          float* tile, int w) const {
        const __amdgpu_buffer_rsrc_t rs = block_rsrc(head, T, D, row0);
#pragma unroll
        for(int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t*)(tile + 256 * (w + 4 * i)), 16,
                                                     off[i], 0, 0, 0);
        if(w == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t*)(tile + 256 * (LOADS - 1)), 16,
                                                     off[4], 0, 0, 0);
    }
};

// wait for this wave's outstanding global loads (the direct-to-LDS ones
// included); a barrier after it publishes every wave's loads
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// The loop bodies take the block being read and the buffer being loaded as
// __restrict__ pointers: that tells the compiler the two never overlap, so
// the direct-to-LDS loads can run under the reads.  (Without it the compiler
// has to assume they may overlap and waits for every direct-to-LDS load
// before the next LDS read, which serialises the double buffering.)

// ======================================================================= forward
// Workgroup: 128 queries of one (b, h), 4 waves of 32; which query block a
// workgroup takes comes from the dispatch plan (FlashPlan).
//
// Three workgroups share a CU (at most 168 VGPRs and 51 KB of LDS each), so
// config 5's 768 workgroups (B 8, H 12, T 1024) are all resident from the
// start: no second dispatch round, whose light query blocks would otherwise
// start late on CUs still busy with heavy ones.  Per key block j:
//   wait for K(j), V(j); barrier; load V(j+1) into the other V buffer;
//   S = Q.K(j)^T; barrier; load K(j+1) into the one K buffer;
//   softmax; O += P.V(j)
// so K(j+1) lands under the softmax and P.V, V(j+1) under a whole block.
//
// VALU and MFMA work of the waves sharing a SIMD do not run concurrently on
// gfx950, so every VALU instruction of the softmax adds to the kernel's time.
// The softmax therefore keeps a stale running max m: m is exact after the
// first key block and is raised only when a block's scores exceed it by more
// than kTau (a wave-wide decision, rare after the first blocks), so the output
// and the row sum are rescaled only then.  The score products start from -m
// instead of 0, so the scores come out already relative to m and exp2 needs no
// subtraction.  A block's scores are exponentiated against an m at most kTau
// below the true running max (values <= 2^kTau) and never against one above
// it, so nothing underflows that the exact online softmax would keep, and O
// and l (the row sum) are the same sums in exact arithmetic.
constexpr float kTau = 8.0f;

constexpr int kFwdSlots = 3;
__global__ __launch_bounds__(256, kFwdSlots) void flash_fwd(FlashParams p, FlashPlan plan) {
    __shared__ __attribute__((aligned(16))) float sK[TILE];
    __shared__ __attribute__((aligned(16))) float sV[2][TILE];
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS;
    const int64_t rank = plan_rank(plan);
    const int64_t qb = nqb - 1 - rank / BH, bh = rank % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;
    const int nkv = (int)((qb * ROWS + ROWS) / BLK);  // blocks the workgroup streams
    const int nw = (int)((q0 + 31) / BLK) + 1;          // blocks this wave sees

    const BlockLoad blk(p.ld, w, l);
    blk.issue(K, p.T, p.ld, 0, sK, w);
    blk.issue(V, p.T, p.ld, 0, sV[0], w);
    float qf[32];
    load_frag32(Q + qi * p.ld, lh, qf, p.scale * kLog2e, qi < p.T);
    f32x16 o[2] = {zero16(), zero16()};
    // m: the offset the scores are taken against (log2 units); ls: this lane's
    // share of the row sum (its 32 keys of each block; the two halves of the
    // wave hold the other keys of the same queries and are added at the end)
    float m = 0.0f, ls = 0.0f;

    // A wave's last block j = nw-1 is the one that crosses its diagonal: key
    // kv0 + sub*32 + acc_row(r, lh) is hidden from query qi when it exceeds
    // qi; lim folds the lane's offsets into one compare per element
    auto mask = [&](int j, f32x16 (&s)[2]) {
        const int lim = (int)(qi - (int64_t)j * BLK) - 4 * lh;
#pragma unroll
        for(int sub = 0; sub < 2; ++sub)
#pragma unroll
            for(int r = 0; r < 16; ++r)
                if(sub * 32 + 8 * (r >> 2) + (r & 3) > lim) s[sub][r] = -INFINITY;
    };
    auto lane_max = [&](const f32x16 (&s)[2]) {
        float mx = -INFINITY;
#pragma unroll
        for(int sub = 0; sub < 2; ++sub)
#pragma unroll
            for(int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sub][r]);
        return mx;
    };
    auto exp_sum = [&](f32x16 (&s)[2]) {
        float l0 = 0.0f, l1 = 0.0f;
#pragma unroll
        for(int r = 0; r < 16; ++r) {
            s[0][r] = __builtin_amdgcn_exp2f(s[0][r]);
            l0 += s[0][r];
            s[1][r] = __builtin_amdgcn_exp2f(s[1][r]);
            l1 += s[1][r];
        }
        ls += l0 + l1;
    };
    // -m in all 16 registers: the start of the next block's score products
    auto start_scores = [&]() {
        f32x16 z;
#pragma unroll
        for(int r = 0; r < 16; ++r) z[r] = -m;
        return z;
    };
    // block 0: m is its exact row max (finite: key 0 is visible to every query)
    auto softmax_first = [&](f32x16 (&s)[2]) {
        float mx = lane_max(s);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
#pragma unroll
        for(int sub = 0; sub < 2; ++sub)
#pragma unroll
            for(int r = 0; r < 16; ++r) s[sub][r] -= mx;
        m = mx;
        exp_sum(s);
    };
    auto softmax = [&](f32x16 (&s)[2]) {
        float mx = lane_max(s);
        if(__builtin_amdgcn_ballot_w64(mx > kTau)) {  // raise m to the block's row max
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float d = fmaxf(mx, 0.0f);
            const float alpha = __builtin_amdgcn_exp2f(-d);
#pragma unroll
            for(int sub = 0; sub < 2; ++sub)
#pragma unroll
                for(int r = 0; r < 16; ++r) s[sub][r] -= d;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                o[0][r] *= alpha;
                o[1][r] *= alpha;
            }
            ls *= alpha;
            m += d;
        }
        exp_sum(s);
    };
    // o += V(j)^T . P^T
    auto pv = [&](const float* tv, const f32x16 (&s)[2]) { dot_cols2(tv, lq, lh, s, o[0], o[1]); };
    // every block j of the workgroup: wait for K(j), V(j); barrier; load
    // V(j+1); S; barrier; load K(j+1); softmax and P.V.  The waves whose last
    // query precedes the workgroup's last key block skip the products there.
    auto begin_block = [&](int j) {
        wait_loads();
        __syncthreads();  // K(j), V(j) are in; V(j-1)'s buffer is free
        if(j + 1 < nkv) blk.issue(V, p.T, p.ld, (int64_t)(j + 1) * BLK, sV[(j + 1) & 1], w);
    };
    auto mid_block = [&](int j) {
        __syncthreads();  // every wave has read K(j)
        if(j + 1 < nkv) blk.issue(K, p.T, p.ld, (int64_t)(j + 1) * BLK, sK, w);
    };
    const bool half = (q0 & (BLK - 1)) == 0;
    {  // block 0: the exact max; masked when it is also the wave's last
        begin_block(0);
        f32x16 s[2] = {zero16(), zero16()};
        if(nw == 1 && half) s[0] = dot_rows(sK, 0, lq, lh, qf, s[0]);
        else dot_rows2(sK, lq, lh, qf, s[0], s[1]);
        mid_block(0);
        if(nw == 1) mask(0, s);
        softmax_first(s);
        if(nw == 1 && half) {
            o[0] = dot_cols(sV[0], 0, 0, lq, lh, s[0], o[0]);
            o[1] = dot_cols(sV[0], 0, 1, lq, lh, s[0], o[1]);
        } else {
            pv(sV[0], s);
        }
    }
    int j = 1;
    for(; j < nw - 1; ++j) {  // blocks wholly below the diagonal
        begin_block(j);
        f32x16 s[2];
        s[0] = s[1] = start_scores();
        dot_rows2(sK, lq, lh, qf, s[0], s[1]);
        mid_block(j);
        softmax(s);
        pv(sV[j & 1], s);
    }
    if(j == nw - 1) {  // the wave's last block (when it is not block 0)
        begin_block(j);
        f32x16 s[2];
        s[0] = s[1] = start_scores();
        // a wave whose 32 queries end before the block's second key group
        // (q0 a multiple of 64) computes the first group only: the second is
        // wholly masked, its probabilities exactly 0
        if(half) s[0] = dot_rows(sK, 0, lq, lh, qf, s[0]);
        else dot_rows2(sK, lq, lh, qf, s[0], s[1]);
        mid_block(j);
        mask(j, s);
        softmax(s);
        if(half) {
            o[0] = dot_cols(sV[j & 1], 0, 0, lq, lh, s[0], o[0]);
            o[1] = dot_cols(sV[j & 1], 0, 1, lq, lh, s[0], o[1]);
        } else {
            pv(sV[j & 1], s);
        }
        ++j;
    }
    for(; j < nkv; ++j) {  // the workgroup's blocks past this wave's last
        begin_block(j);
        mid_block(j);
    }
    if(qi >= p.T) return;  // a padding row of the last block
    const float lsum = ls + __shfl_xor(ls, 32, 64);
    store_rowT(p.out + obase + qi * p.D, o, lh, 1.0f / lsum, false);
    if(lh == 0 && p.lse_out) p.lse_out[bh * p.T + qi] = (m + log2f(lsum)) * kLn2;
}

// ============================================== backward: per-query constants
// For each 64-query block the workspace holds 64 values of L2 = lse*log2(e)
// followed by 64 values of D = rowsum(dO*O): [B*H][T/64][2][64].  One 512-byte
// load per block brings both into LDS.
// Sixteen lanes per query row, one float4 of dO and O each, so a wave reads
// four rows as four contiguous 256-byte runs.
// Rows T..Tp-1 (T not a multiple of 128) get L2 = +inf and D = 0, so their
// probabilities, and with them their share of dS, dK and dV, are exactly 0.
__global__ void flash_dsum(FlashParams p) {
    const int64_t BH = p.B * p.H, n = BH * p.Tp;
    const int c = threadIdx.x & 15;
    for(int64_t i = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 4; i < n;
        i += ((int64_t)gridDim.x * blockDim.x) >> 4) {
        const int64_t bh = i / p.Tp, t = i % p.Tp, b = bh / p.H, h = bh % p.H;
        float* blk = p.dsum_out + bh * 2 * p.Tp + (t / BLK) * 2 * BLK + t % BLK;
        if(t >= p.T) {  // the whole 16-lane group: one row
            if(c == 0) {
                blk[0] = INFINITY;
                blk[BLK] = 0.0f;
            }
            continue;
        }
        const int64_t off = (b * p.T + t) * p.D + h * HD;
        const f32x4 a = reinterpret_cast<const f32x4*>(p.dout + off)[c];
        const f32x4 o = reinterpret_cast<const f32x4*>(p.o + off)[c];
        float s = a[0] * o[0] + a[1] * o[1] + a[2] * o[2] + a[3] * o[3];
        s += __shfl_xor(s, 8, 16);
        s += __shfl_xor(s, 4, 16);
        s += __shfl_xor(s, 2, 16);
        s += __shfl_xor(s, 1, 16);
        if(c == 0) {
            blk[0] = p.lse[bh * p.T + t] * kLog2e;
            blk[BLK] = s;
        }
    }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t consts_rsrc(const float* ws, int64_t bh,
                                                              int64_t T) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ws + bh * 2 * T), (short)0,
                                             (int)(2 * T * 4), 0x00020000);
}

// dS of one (b, h) is kept as 32x32 tiles, one per (query group qg, key group
// kg) with kg <= qg, packed by rows of that triangle: tile qg*(qg+1)/2 + kg.
// Inside a tile the 16 values that the dQ kernel's lane (q, h) multiplies --
// keys 8(s/4) + 4h + s%4 for s = 0..15, the accumulator-row order -- are the
// consecutive floats (2q + h)*16 + s, so the dQ kernel reads a tile as one
// contiguous 4 KB stream; the dK/dV kernel writes it 128 bytes per row.
__host__ __device__ __forceinline__ int64_t ds_tiles(int64_t T) {
    return (T / 32) * (T / 32 + 1) / 2;
}
__device__ __forceinline__ int64_t ds_tile(int64_t bh, int64_t T, int64_t qg, int64_t kg) {
    return (bh * ds_tiles(T) + qg * (qg + 1) / 2 + kg) * 1024;
}

// ================================================================ backward: dK, dV
// Workgroup: 128 keys of one (b, h), one key per lane; query blocks of 64 with
// q >= key stream through LDS (Q and dO rows, their L2 and D), loaded
// straight into LDS one block ahead.
//   S = Q.K^T (per lane: its key's column)        P = exp2(S' - L2)
//   dV^T += dO^T.P         dP = dO.V^T           dS = P*(dP - D)
//   dK^T += Q^T.dS  (x scale at the end)
// The two 32-query halves of a block run one after the other (two waves per
// SIMD overlap one's exponentials with the other's products).  dS goes to the
// tile store for the dQ kernel.
__global__ __launch_bounds__(256, 2) void flash_bwd_dkdv(FlashParams p) {
    __shared__ __attribute__((aligned(16))) float sQ[2][TILE];
    __shared__ __attribute__((aligned(16))) float sO[2][TILE];      // dO rows
    __shared__ __attribute__((aligned(16))) float sLD[2][2 * BLK];  // L2, then D
    const int64_t BH = p.B * p.H;
    const int64_t kb = (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *K = p.k + base, *V = p.v + base;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t k0 = kb * ROWS + w * 32, ki = k0 + lq;

    const BlockLoad blq(p.ld, w, l), blo(p.D, w, l);
    const float *Qh = p.q + base, *Oh = p.dout + obase;
    const __amdgpu_buffer_rsrc_t rc = consts_rsrc(p.dsum, bh, p.Tp);
    auto issue = [&](int j, float* __restrict__ tq, float* __restrict__ to,
                     float* __restrict__ tl) {
        blq.issue(Qh, p.T, p.ld, (int64_t)j * BLK, tq, w);
        blo.issue(Oh, p.T, p.D, (int64_t)j * BLK, to, w);
        if(w == 1 && l < 32)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_ptr_t*)tl, 16, 16 * l,
                                                     (unsigned)(j * 2 * BLK * 4), 0, 0);
    };
    const int j0 = (int)(kb * ROWS / BLK), nq = (int)(p.Tp / BLK);
    issue(j0, sQ[0], sO[0], sLD[0]);
    float kf[32], vf[32];
    load_frag32(K + ki * p.ld, lh, kf, p.scale * kLog2e, ki < p.T);
    load_frag32(V + ki * p.ld, lh, vf, 1.0f, ki < p.T);
    f32x16 dv[2] = {zero16(), zero16()}, dk[2] = {zero16(), zero16()};
    // this lane's column of every dS tile of key group kg (rows 32 floats apart)
    const int64_t kg = k0 / 32;
    float* dsk = p.ds ? p.ds + ds_tile(bh, p.Tp, 0, 0) + ((lq >> 2) & 1) * 16 + 4 * (lq >> 3) + (lq & 3)
                      : nullptr;

    // iteration j reads buffer set st = (j - j0) & 1 and loads block j+1 into
    // the other one
    auto iter = [&](int j, const float* __restrict__ tq, const float* __restrict__ to,
                    const float* __restrict__ tl, float* __restrict__ nq_, float* __restrict__ no_,
                    float* __restrict__ nl_) {
        wait_loads();
        __syncthreads();  // block j is in; the other set (block j-1) is free
        if(j + 1 < nq) issue(j + 1, nq_, no_, nl_);
        const int64_t qs = (int64_t)j * BLK;
        if(qs + BLK - 1 >= k0) {  // some query of this block sees this wave's keys
            // query qs + sub*32 + acc_row(r, lh) sees key ki when it is >= ki
            const int lim = (int)(ki - qs) - 4 * lh;
            const bool diag = qs < k0 + 32;  // some query of the block precedes a key
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                // every query of this half precedes the wave's first key: its
                // P and dS would be all zeros (and no dS tile holds them)
                if(qs + sub * 32 + 31 < k0) continue;
                f32x16 sc = dot_rows(tq, sub, lq, lh, kf, zero16());
                f32x16 dp = dot_rows(to, sub, lq, lh, vf, zero16());
                // one 128-bit operand read per 4 products, so the reads are
                // not all hoisted into registers at once
#pragma unroll
                for(int i = 0; i < 16; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                }
                // read and exponentiate unconditionally, then select: the
                // masked lanes' values are discarded.  Only a block that
                // crosses this wave's diagonal has masked lanes.
                if(diag) {
#pragma unroll
                    for(int r = 0; r < 16; ++r) {
                        const int qr = sub * 32 + acc_row(r, lh);
                        const float e = __builtin_amdgcn_exp2f(sc[r] - tl[qr]);
                        const float pr = sub * 32 + 8 * (r >> 2) + (r & 3) >= lim ? e : 0.0f;
                        sc[r] = pr;
                        dp[r] = pr * (dp[r] - tl[BLK + qr]);
                    }
                } else {
#pragma unroll
                    for(int r = 0; r < 16; ++r) {
                        const int qr = sub * 32 + acc_row(r, lh);
                        const float pr = __builtin_amdgcn_exp2f(sc[r] - tl[qr]);
                        sc[r] = pr;
                        dp[r] = pr * (dp[r] - tl[BLK + qr]);
                    }
                }
                const int64_t qg = 2 * j + sub;
                if(qg >= kg && dsk) {  // no tile store: the dQ kernel recomputes dS
                    float* t = dsk + (qg * (qg + 1) / 2 + kg) * 1024;
#pragma unroll
                    for(int r = 0; r < 16; ++r) t[acc_row(r, lh) * 32] = dp[r];
                }
                // keep the dV/dK operand reads of this half below its softmax
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for(int cb = 0; cb < 2; ++cb) {
                    dv[cb] = dot_cols(to, sub, cb, lq, lh, sc, dv[cb]);
                    dk[cb] = dot_cols(tq, sub, cb, lq, lh, dp, dk[cb]);
                }
#pragma unroll
                for(int i = 0; i < 32; ++i) {  // two 32-bit reads per 2 products
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    for(int j = j0; j < nq; ++j) {
        const int st = (j - j0) & 1;
        iter(j, sQ[st], sO[st], sLD[st], sQ[st ^ 1], sO[st ^ 1], sLD[st ^ 1]);
    }
    if(ki >= p.T) return;  // a padding row of the last block
    store_rowT(p.dv + base + ki * p.ld, dv, lh, 1.0f, (p.flags & PK_ACCUM3) != 0);
    store_rowT(p.dk + base + ki * p.ld, dk, lh, p.scale, (p.flags & PK_ACCUM2) != 0);
}

// =================================================================== backward: dQ
// Workgroup: 128 queries of one (b, h), one query per lane.  dQ^T += K^T.dS^T
// (x scale at the end) over the key blocks of 64 with key <= query: K blocks
// stream through LDS one block ahead, the dS tiles the dK/dV kernel stored
// are read straight into registers one block ahead.
// Four workgroups share a CU (112 VGPRs, 34 KB of LDS), so config 5's 768
// are resident at once, placed by the dispatch plan.
constexpr int kDqSlots = 4;
__global__ __launch_bounds__(256, kDqSlots) void flash_bwd_dq(FlashParams p, FlashPlan plan) {
    __shared__ __attribute__((aligned(16))) float sK[2][TILE];
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS, rank = plan_rank(plan);
    const int64_t qb = nqb - 1 - rank / BH, bh = rank % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq, qg = q0 / 32;

    const BlockLoad blk(p.ld, w, l);
    const float* Kh = p.k + base;
    blk.issue(Kh, p.T, p.ld, 0, sK[0], w);
    // tile (qg, kg) is at ds + kg*1024; this lane's 16 values at (2*lq + lh)*16
    const float* ds = p.ds + ds_tile(bh, p.Tp, qg, 0) + (2 * lq + lh) * 16;
    auto fetch = [&](int j, f32x16 (&x)[2]) {
#pragma unroll
        for(int sub = 0; sub < 2; ++sub) {
            const int64_t kg = 2 * j + sub;
            if(kg <= qg) {
                const f32x4* src = reinterpret_cast<const f32x4*>(ds + kg * 1024);
#pragma unroll
                for(int i = 0; i < 4; ++i) {
                    const f32x4 v = src[i];
#pragma unroll
                    for(int e = 0; e < 4; ++e) x[sub][4 * i + e] = v[e];
                }
            }
        }
    };
    f32x16 dq[2] = {zero16(), zero16()};
    f32x16 cur[2] = {zero16(), zero16()}, nxt[2] = {zero16(), zero16()};
    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    const int nw = (int)((q0 + 31) / BLK) + 1;  // key blocks this wave sees
    fetch(0, cur);
    auto iter = [&](int j, const float* __restrict__ tk, float* __restrict__ kd) {
        wait_loads();
        __syncthreads();
        if(j + 1 < nkv) blk.issue(Kh, p.T, p.ld, (int64_t)(j + 1) * BLK, kd, w);
        if(j + 1 < nw) fetch(j + 1, nxt);
        if(j < nw) {
            const int lim = (int)(qi - (int64_t)j * BLK) - 4 * lh;  // key offset <= lim visible
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                if(2 * j + sub > qg) continue;  // the whole key group is in this wave's future
                if((int64_t)j * BLK + BLK - 1 > q0) {  // the block crosses the diagonal
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) > lim) cur[sub][r] = 0.0f;
                }
            }
            // the two column chains alternate, each accumulating the keys in
            // the order dot_cols takes them
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                if(2 * j + sub > qg) continue;
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const float* a = tk + (sub * 32 + acc_row(r, lh)) * LDT + lq;
                    dq[0] = mfma(a[0], cur[sub][r], dq[0]);
                    dq[1] = mfma(a[32], cur[sub][r], dq[1]);
                }
            }
            cur[0] = nxt[0];
            cur[1] = nxt[1];
        }
    };
    for(int j = 0; j < nkv; ++j) iter(j, sK[j & 1], sK[(j + 1) & 1]);
    if(qi >= p.T) return;  // a padding row of the last block
    store_rowT(p.dq + base + qi * p.ld, dq, lh, p.scale, (p.flags & PK_ACCUM) != 0);
}

// ====================================================== backward: dQ, recomputed
// The dQ kernel for callers whose workspace cannot hold the dS tiles (they take
// about 2*B*H*T^2 bytes): each workgroup recomputes its queries' scores and
// dP block by block instead of reading dS.  Workgroup: 128 queries of one
// (b, h), one query per lane; K and V blocks of 64 stream through LDS one
// block ahead.  Per block: S^T = K'.Q^T (K' = K * scale*log2(e), rounded as
// the dK/dV kernel rounds its K fragment), dP^T = V.dO^T, dS = P*(dP - D),
// dQ^T += K^T.dS^T.  Every product multiplies the same fp32 values in the same
// order as the dK/dV kernel (whose lanes hold keys) and the stored-dS dQ
// kernel, so dS and dQ come out bit for bit the same; it costs three products
// per block where the stored path costs one.
__device__ __forceinline__ f32x16 dot_rows_scaled(const float* lds, int sub, int lq, int lh,
                                                  const float (&bf)[32], float mul) {
    const f32x4* a4 = reinterpret_cast<const f32x4*>(lds + (sub * 32 + lq) * LDT + 32 * lh);
    f32x16 acc = zero16();
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const f32x4 a = a4[i];
        acc = mfma(a[0] * mul, bf[4 * i + 0], acc);
        acc = mfma(a[1] * mul, bf[4 * i + 1], acc);
        acc = mfma(a[2] * mul, bf[4 * i + 2], acc);
        acc = mfma(a[3] * mul, bf[4 * i + 3], acc);
    }
    return acc;
}

__global__ __launch_bounds__(256, 2) void flash_bwd_dq_recompute(FlashParams p) {
    __shared__ __attribute__((aligned(16))) float sK[2][TILE];
    __shared__ __attribute__((aligned(16))) float sV[2][TILE];
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS;
    // heaviest query blocks first, alternate passes of one workgroup per CU reversed
    const int64_t nwg = BH * nqb, pass = blockIdx.x / kCUs;
    const int64_t lo = pass * kCUs, hi = min(lo + kCUs, nwg);
    const int64_t rank = (pass & 1) ? lo + hi - 1 - blockIdx.x : blockIdx.x;
    const int64_t qb = nqb - 1 - rank / BH, bh = rank % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq, qg = q0 / 32;

    const BlockLoad blk(p.ld, w, l);
    const float *Kh = p.k + base, *Vh = p.v + base;
    blk.issue(Kh, p.T, p.ld, 0, sK[0], w);
    blk.issue(Vh, p.T, p.ld, 0, sV[0], w);
    float qf[32], of[32];
    load_frag32(p.q + base + qi * p.ld, lh, qf, 1.0f, qi < p.T);
    load_frag32(p.dout + obase + qi * p.D, lh, of, 1.0f, qi < p.T);
    // this query's L2 = lse*log2(e) and D = rowsum(dO*O) ([B*H][Tp/64][2][64])
    const float* rc = p.dsum + bh * 2 * p.Tp + (qi / BLK) * 2 * BLK + qi % BLK;
    const float L2 = rc[0], Dq = rc[BLK];
    const float mul = p.scale * kLog2e;
    f32x16 dq[2] = {zero16(), zero16()};
    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    const int nw = (int)((q0 + 31) / BLK) + 1;  // key blocks this wave sees
    for(int j = 0; j < nkv; ++j) {
        const float* __restrict__ tk = sK[j & 1];
        const float* __restrict__ tv = sV[j & 1];
        wait_loads();
        __syncthreads();  // block j is in; the other buffers (block j-1) are free
        if(j + 1 < nkv) {
            blk.issue(Kh, p.T, p.ld, (int64_t)(j + 1) * BLK, sK[(j + 1) & 1], w);
            blk.issue(Vh, p.T, p.ld, (int64_t)(j + 1) * BLK, sV[(j + 1) & 1], w);
        }
        if(j >= nw) continue;
        const int lim = (int)(qi - (int64_t)j * BLK) - 4 * lh;  // key offset <= lim visible
        const bool diag = (int64_t)j * BLK + BLK - 1 > q0;       // the block crosses the diagonal
#pragma unroll
        for(int sub = 0; sub < 2; ++sub) {
            if(2 * j + sub > qg) continue;  // the whole key group is in this wave's future
            const f32x16 sc = dot_rows_scaled(tk, sub, lq, lh, qf, mul);
            const f32x16 dp = dot_rows(tv, sub, lq, lh, of, zero16());
            f32x16 ds;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                const float pr = __builtin_amdgcn_exp2f(sc[r] - L2);
                ds[r] = pr * (dp[r] - Dq);
                if(diag && sub * 32 + 8 * (r >> 2) + (r & 3) > lim) ds[r] = 0.0f;
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for(int cb = 0; cb < 2; ++cb) dq[cb] = dot_cols(tk, sub, cb, lq, lh, ds, dq[cb]);
        }
    }
    if(qi >= p.T) return;  // a padding row of the last block
    store_rowT(p.dq + base + qi * p.ld, dq, lh, p.scale, (p.flags & PK_ACCUM) != 0);
}

// ================================================================ bf16 products
// The same three kernels with bf16 multiplies (v_mfma_f32_32x32x16_bf16,
// fp32 accumulation): Q (pre-scaled), K, V, dO and the probabilities P and
// dS are rounded to bf16 (nearest even) where they enter a product; the
// softmax statistics, exponentials and accumulators stay fp32.
//
// An MFMA contracts 16 values of k, lane l supplying slots 8*(l/32)..+7.  A
// contraction over the head dims takes d = 16t + 8h + j (h = l/32).  A
// contraction over the rows of an accumulator (keys in the forward, queries
// in the backward) uses the rows the lane already holds: group g of a 32-row
// sub-block pairs slot (h, j) with row 16g + 8(j/4) + 4h + j%4, which is
// acc_row(8g + j, h) -- registers 8g..8g+7 of the accumulator.  The other
// operand reads the same rows: two runs of 4 from a transposed tile.
//
// Blocks are staged from global memory through registers (rounded on the way
// into LDS), as 4x4 sub-blocks per thread so that a tile can be written
// row-major, transposed or both.  bf16 tiles have rows of LDB = 72 elements
// (144 bytes): 16-byte aligned for the b128 reads and conflict-free for them.
constexpr int LDB = HD + 8;
constexpr int TILEB = BLK * LDB;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma16(const bf16x8& a, const bf16x8& b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// thread t holds rows 4*(t/16)..+3, columns 4*(t%16)..+3 of a 64x64 block;
// rows at or past T read as zeros
__device__ __forceinline__ void fetch_quad(const float* __restrict__ base, int64_t D, int64_t row0,
                                           f32x4 (&x)[4], int64_t T) {
    const int rq = threadIdx.x >> 4, c4 = threadIdx.x & 15;
#pragma unroll
    for(int i = 0; i < 4; ++i) {
        const int64_t r = row0 + 4 * rq + i;
        x[i] = r < T ? *reinterpret_cast<const f32x4*>(base + r * D + 4 * c4)
                     : f32x4{0.f, 0.f, 0.f, 0.f};
    }
}

// the lo part of a split value: x - hi rounded, hi = bf16(x) (x - hi is exact
// in fp32, so hi + lo is x to 2^-17)
__device__ __forceinline__ __bf16 lo_part(float x, __bf16 hi) { return (__bf16)(x - (float)hi); }

// SPLIT: a tile is followed (at + TILEB) by the lo parts of its values
template <bool SPLIT = false>
__device__ __forceinline__ void put_rows(__bf16* t, const f32x4 (&x)[4]) {
    const int rq = threadIdx.x >> 4, c4 = threadIdx.x & 15;
#pragma unroll
    for(int i = 0; i < 4; ++i) {
        const bf16x4 h = {(__bf16)x[i][0], (__bf16)x[i][1], (__bf16)x[i][2], (__bf16)x[i][3]};
        *reinterpret_cast<bf16x4*>(t + (4 * rq + i) * LDB + 4 * c4) = h;
        if constexpr(SPLIT)
            *reinterpret_cast<bf16x4*>(t + TILEB + (4 * rq + i) * LDB + 4 * c4) =
                bf16x4{lo_part(x[i][0], h[0]), lo_part(x[i][1], h[1]), lo_part(x[i][2], h[2]),
                       lo_part(x[i][3], h[3])};
    }
}

template <bool SPLIT = false>
__device__ __forceinline__ void put_cols(__bf16* t, const f32x4 (&x)[4]) {
    const int rq = threadIdx.x >> 4, c4 = threadIdx.x & 15;
#pragma unroll
    for(int c = 0; c < 4; ++c) {
        const bf16x4 h = {(__bf16)x[0][c], (__bf16)x[1][c], (__bf16)x[2][c], (__bf16)x[3][c]};
        *reinterpret_cast<bf16x4*>(t + (4 * c4 + c) * LDB + 4 * rq) = h;
        if constexpr(SPLIT)
            *reinterpret_cast<bf16x4*>(t + TILEB + (4 * c4 + c) * LDB + 4 * rq) =
                bf16x4{lo_part(x[0][c], h[0]), lo_part(x[1][c], h[1]), lo_part(x[2][c], h[2]),
                       lo_part(x[3][c], h[3])};
    }
}

// a lane's 32 head dims of one row, rounded, in the 4 MFMA steps' slots
__device__ __forceinline__ void load_frag_bf16(const float* __restrict__ row, int h, bf16x8 (&f)[4],
                                               float mul, bool ok = true) {
    if(!ok) {
        const __bf16 z = (__bf16)0.0f;
#pragma unroll
        for(int t = 0; t < 4; ++t) f[t] = bf16x8{z, z, z, z, z, z, z, z};
        return;
    }
#pragma unroll
    for(int t = 0; t < 4; ++t) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(row + 16 * t + 8 * h);
        const f32x4 b = *reinterpret_cast<const f32x4*>(row + 16 * t + 8 * h + 4);
        f[t] = bf16x8{(__bf16)(a[0] * mul), (__bf16)(a[1] * mul), (__bf16)(a[2] * mul),
                      (__bf16)(a[3] * mul), (__bf16)(b[0] * mul), (__bf16)(b[1] * mul),
                      (__bf16)(b[2] * mul), (__bf16)(b[3] * mul)};
    }
}

// the same fragments with their lo parts (fl) for the split products
__device__ __forceinline__ void load_frag_split(const float* __restrict__ row, int h, bf16x8 (&f)[4],
                                                bf16x8 (&fl)[4], float mul, bool ok) {
    load_frag_bf16(row, h, f, mul, ok);
#pragma unroll
    for(int t = 0; t < 4; ++t) {
        if(!ok) {
            fl[t] = f[t];  // zeros
            continue;
        }
        const f32x4 a = *reinterpret_cast<const f32x4*>(row + 16 * t + 8 * h);
        const f32x4 b = *reinterpret_cast<const f32x4*>(row + 16 * t + 8 * h + 4);
        fl[t] = bf16x8{lo_part(a[0] * mul, f[t][0]), lo_part(a[1] * mul, f[t][1]),
                       lo_part(a[2] * mul, f[t][2]), lo_part(a[3] * mul, f[t][3]),
                       lo_part(b[0] * mul, f[t][4]), lo_part(b[1] * mul, f[t][5]),
                       lo_part(b[2] * mul, f[t][6]), lo_part(b[3] * mul, f[t][7])};
    }
}

// acc (+)= A.B over the head dims: A = row (sub*32 + lane%32) of a row-major
// tile, B = the lane's fragments.  SPLIT: hi.hi + hi.lo + lo.hi per step (bl:
// the fragments' lo parts; the tile's at + TILEB)
template <bool SPLIT = false>
__device__ __forceinline__ f32x16 dot_rows16(const __bf16* t, int sub, int lq, int lh,
                                             const bf16x8 (&bf)[4], const bf16x8 (&bl)[SPLIT ? 4 : 1],
                                             f32x16 acc) {
    const __bf16* row = t + (sub * 32 + lq) * LDB + 8 * lh;
#pragma unroll
    for(int s = 0; s < 4; ++s) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(row + 16 * s);
        acc = mfma16(a, bf[s], acc);
        if constexpr(SPLIT) {
            acc = mfma16(a, bl[s], acc);
            acc = mfma16(*reinterpret_cast<const bf16x8*>(row + TILEB + 16 * s), bf[s], acc);
        }
    }
    return acc;
}
__device__ __forceinline__ f32x16 dot_rows16(const __bf16* t, int sub, int lq, int lh,
                                             const bf16x8 (&bf)[4], f32x16 acc) {
    const bf16x8 none[1] = {};
    return dot_rows16<false>(t, sub, lq, lh, bf, none, acc);
}

// the accumulator rows of group g as a B operand (slot (h, j) <- register 8g + j)
__device__ __forceinline__ bf16x8 pack_group(const f32x16& x, int g) {
    return bf16x8{(__bf16)x[8 * g + 0], (__bf16)x[8 * g + 1], (__bf16)x[8 * g + 2],
                  (__bf16)x[8 * g + 3], (__bf16)x[8 * g + 4], (__bf16)x[8 * g + 5],
                  (__bf16)x[8 * g + 6], (__bf16)x[8 * g + 7]};
}

// acc (+)= X^T . W over the 32 accumulator rows of sub-block `sub`: A[i][row]
// read from the transposed tile (row cb*32 + lane%32, the group's rows), B = w.
// SPLIT: w is split as it is packed, hi.hi + hi.lo + lo.hi per group
template <bool SPLIT = false>
__device__ __forceinline__ f32x16 dot_cols16(const __bf16* t, int sub, int cb, int lq, int lh,
                                             const f32x16& w, f32x16 acc) {
    const __bf16* row = t + (cb * 32 + lq) * LDB + sub * 32 + 4 * lh;
#pragma unroll
    for(int g = 0; g < 2; ++g) {
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row + 16 * g);
        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(row + 16 * g + 8);
        const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        const bf16x8 wh = pack_group(w, g);
        acc = mfma16(a, wh, acc);
        if constexpr(SPLIT) {
            bf16x8 wl;
#pragma unroll
            for(int j = 0; j < 8; ++j) wl[j] = lo_part(w[8 * g + j], wh[j]);
            acc = mfma16(a, wl, acc);
            const bf16x4 lo2 = *reinterpret_cast<const bf16x4*>(row + TILEB + 16 * g);
            const bf16x4 hi2 = *reinterpret_cast<const bf16x4*>(row + TILEB + 16 * g + 8);
            const bf16x8 al = {lo2[0], lo2[1], lo2[2], lo2[3], hi2[0], hi2[1], hi2[2], hi2[3]};
            acc = mfma16(al, wh, acc);
        }
    }
    return acc;
}

// ------------------------------------------------------------- bf16 forward
// SPLIT (the split-bf16 products): every operand as hi and lo bf16 parts
// (tiles of lo parts after the hi tiles, fragments ql), each product as
// hi.hi + hi.lo + lo.hi
template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void flash_fwd_bf16(FlashParams p) {
    constexpr int NS = SPLIT ? 2 : 1;
    __shared__ __attribute__((aligned(16))) __bf16 sK[2][NS * TILEB];   // [key][d]
    __shared__ __attribute__((aligned(16))) __bf16 sVt[2][NS * TILEB];  // [d][key]
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS;
    const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;

    bf16x8 qf[4], ql[SPLIT ? 4 : 1];
    if constexpr(SPLIT) load_frag_split(Q + qi * p.ld, lh, qf, ql, p.scale * kLog2e, qi < p.T);
    else load_frag_bf16(Q + qi * p.ld, lh, qf, p.scale * kLog2e, qi < p.T);
    f32x16 o[2] = {zero16(), zero16()};
    float m = -INFINITY, lsum = 0.0f;
    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    f32x4 rk[4], rv[4];
    fetch_quad(K, p.ld, 0, rk, p.T);
    fetch_quad(V, p.ld, 0, rv, p.T);
    put_rows<SPLIT>(sK[0], rk);
    put_cols<SPLIT>(sVt[0], rv);
    for(int j = 0; j < nkv; ++j) {
        const int st = j & 1;
        __syncthreads();
        const bool more = j + 1 < nkv;
        if(more) {
            fetch_quad(K, p.ld, (int64_t)(j + 1) * BLK, rk, p.T);
            fetch_quad(V, p.ld, (int64_t)(j + 1) * BLK, rv, p.T);
        }
        const int64_t kv0 = (int64_t)j * BLK;
        if(kv0 <= q0 + 31) {
            f32x16 s[2] = {dot_rows16<SPLIT>(sK[st], 0, lq, lh, qf, ql, zero16()),
                           dot_rows16<SPLIT>(sK[st], 1, lq, lh, qf, ql, zero16())};
            if(kv0 + BLK - 1 > q0) {  // the block crosses this wave's diagonal
                const int lim = (int)(qi - kv0) - 4 * lh;
#pragma unroll
                for(int sub = 0; sub < 2; ++sub)
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) > lim) s[sub][r] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for(int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[0][r], s[1][r]));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            float ls = 0.0f;
#pragma unroll
            for(int sub = 0; sub < 2; ++sub)
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    s[sub][r] = __builtin_amdgcn_exp2f(s[sub][r] - mn);
                    ls += s[sub][r];
                }
            ls += __shfl_xor(ls, 32, 64);
            lsum = lsum * alpha + ls;
            m = mn;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                o[0][r] *= alpha;
                o[1][r] *= alpha;
            }
#pragma unroll
            for(int cb = 0; cb < 2; ++cb) {
                o[cb] = dot_cols16<SPLIT>(sVt[st], 0, cb, lq, lh, s[0], o[cb]);
                o[cb] = dot_cols16<SPLIT>(sVt[st], 1, cb, lq, lh, s[1], o[cb]);
            }
        }
        if(more) {
            put_rows<SPLIT>(sK[st ^ 1], rk);
            put_cols<SPLIT>(sVt[st ^ 1], rv);
        }
    }
    if(qi >= p.T) return;  // a padding row of the last block
    store_rowT(p.out + obase + qi * p.D, o, lh, 1.0f / lsum, false);
    if(lh == 0 && p.lse_out) p.lse_out[bh * p.T + qi] = (m + log2f(lsum)) * kLn2;
}

// ------------------------------------------------------- bf16 backward: dK, dV
// SPLIT: as in the forward; the tiles then take one workgroup a CU
template <bool SPLIT>
__global__ __launch_bounds__(256, SPLIT ? 1 : 2) void flash_bwd_dkdv_bf16(FlashParams p) {
    constexpr int NS = SPLIT ? 2 : 1;
    __shared__ __attribute__((aligned(16))) __bf16 sQ[2][NS * TILEB];   // [q][d]
    __shared__ __attribute__((aligned(16))) __bf16 sQt[2][NS * TILEB];  // [d][q]
    __shared__ __attribute__((aligned(16))) __bf16 sO[2][NS * TILEB];   // dO [q][d]
    __shared__ __attribute__((aligned(16))) __bf16 sOt[2][NS * TILEB];  // dO [d][q]
    __shared__ float sLD[2][2 * BLK];                              // L2, then D
    const int64_t BH = p.B * p.H;
    const int64_t kb = (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base, *dO = p.dout + obase;
    const float* cst = p.dsum + bh * 2 * p.Tp;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t k0 = kb * ROWS + w * 32, ki = k0 + lq;

    bf16x8 kf[4], vf[4], kl[SPLIT ? 4 : 1], vl[SPLIT ? 4 : 1];
    if constexpr(SPLIT) {
        load_frag_split(K + ki * p.ld, lh, kf, kl, p.scale * kLog2e, ki < p.T);
        load_frag_split(V + ki * p.ld, lh, vf, vl, 1.0f, ki < p.T);
    } else {
        load_frag_bf16(K + ki * p.ld, lh, kf, p.scale * kLog2e, ki < p.T);
        load_frag_bf16(V + ki * p.ld, lh, vf, 1.0f, ki < p.T);
    }
    f32x16 dv[2] = {zero16(), zero16()}, dk[2] = {zero16(), zero16()};

    const int j0 = (int)(kb * ROWS / BLK), nq = (int)(p.Tp / BLK);
    f32x4 rq[4], ro[4];
    float rc = 0.0f;
    auto fetch = [&](int j) {
        fetch_quad(Q, p.ld, (int64_t)j * BLK, rq, p.T);
        fetch_quad(dO, p.D, (int64_t)j * BLK, ro, p.T);
        if(threadIdx.x < 2 * BLK) rc = cst[(int64_t)j * 2 * BLK + threadIdx.x];
    };
    auto put = [&](int st) {
        put_rows<SPLIT>(sQ[st], rq);
        put_cols<SPLIT>(sQt[st], rq);
        put_rows<SPLIT>(sO[st], ro);
        put_cols<SPLIT>(sOt[st], ro);
        if(threadIdx.x < 2 * BLK) sLD[st][threadIdx.x] = rc;
    };
    fetch(j0);
    put(0);
    for(int j = j0; j < nq; ++j) {
        const int st = (j - j0) & 1;
        __syncthreads();
        const bool more = j + 1 < nq;
        if(more) fetch(j + 1);
        const int64_t qs = (int64_t)j * BLK;
        if(qs + BLK - 1 >= k0) {
            const float* tl = sLD[st];
            const int lim = (int)(ki - qs) - 4 * lh;  // query row qr sees key ki when qr >= lim
            const bool diag = qs < k0 + 32;           // some query of the block precedes a key
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                if(qs + sub * 32 + 31 < k0) continue;  // all of P would be zeros
                f32x16 sc = dot_rows16<SPLIT>(sQ[st], sub, lq, lh, kf, kl, zero16());
                f32x16 dp = dot_rows16<SPLIT>(sO[st], sub, lq, lh, vf, vl, zero16());
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const int qr = sub * 32 + acc_row(r, lh);
                    sc[r] = __builtin_amdgcn_exp2f(sc[r] - tl[qr]);
                }
                if(diag) {
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) < lim) sc[r] = 0.0f;
                }
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const int qr = sub * 32 + acc_row(r, lh);
                    dp[r] = sc[r] * (dp[r] - tl[BLK + qr]);
                }
#pragma unroll
                for(int cb = 0; cb < 2; ++cb) {
                    dv[cb] = dot_cols16<SPLIT>(sOt[st], sub, cb, lq, lh, sc, dv[cb]);
                    dk[cb] = dot_cols16<SPLIT>(sQt[st], sub, cb, lq, lh, dp, dk[cb]);
                }
            }
        }
        if(more) put(st ^ 1);
    }
    if(ki >= p.T) return;  // a padding row of the last block
    store_rowT(p.dv + base + ki * p.ld, dv, lh, 1.0f, (p.flags & PK_ACCUM3) != 0);
    store_rowT(p.dk + base + ki * p.ld, dk, lh, p.scale, (p.flags & PK_ACCUM2) != 0);
}

// ----------------------------------------------------------- bf16 backward: dQ
template <bool SPLIT>
__global__ __launch_bounds__(256, SPLIT ? 1 : 2) void flash_bwd_dq_bf16(FlashParams p) {
    constexpr int NS = SPLIT ? 2 : 1;
    __shared__ __attribute__((aligned(16))) __bf16 sK[2][NS * TILEB];   // [key][d]
    __shared__ __attribute__((aligned(16))) __bf16 sKt[2][NS * TILEB];  // [d][key]
    __shared__ __attribute__((aligned(16))) __bf16 sV[2][NS * TILEB];   // [key][d]
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS;
    const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base, *dO = p.dout + obase;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;

    bf16x8 qf[4], of[4], ql[SPLIT ? 4 : 1], ol[SPLIT ? 4 : 1];
    if constexpr(SPLIT) {
        load_frag_split(Q + qi * p.ld, lh, qf, ql, p.scale * kLog2e, qi < p.T);
        load_frag_split(dO + qi * p.D, lh, of, ol, 1.0f, qi < p.T);
    } else {
        load_frag_bf16(Q + qi * p.ld, lh, qf, p.scale * kLog2e, qi < p.T);
        load_frag_bf16(dO + qi * p.D, lh, of, 1.0f, qi < p.T);
    }
    const float* cst = p.dsum + bh * 2 * p.Tp + (qi / BLK) * 2 * BLK + qi % BLK;
    const float l2 = cst[0], dd = cst[BLK];
    f32x16 dq[2] = {zero16(), zero16()};

    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    f32x4 rk[4], rv[4];
    fetch_quad(K, p.ld, 0, rk, p.T);
    fetch_quad(V, p.ld, 0, rv, p.T);
    put_rows<SPLIT>(sK[0], rk);
    put_cols<SPLIT>(sKt[0], rk);
    put_rows<SPLIT>(sV[0], rv);
    for(int j = 0; j < nkv; ++j) {
        const int st = j & 1;
        __syncthreads();
        const bool more = j + 1 < nkv;
        if(more) {
            fetch_quad(K, p.ld, (int64_t)(j + 1) * BLK, rk, p.T);
            fetch_quad(V, p.ld, (int64_t)(j + 1) * BLK, rv, p.T);
        }
        const int64_t kv0 = (int64_t)j * BLK;
        if(kv0 <= q0 + 31) {
            const int lim = (int)(qi - kv0) - 4 * lh;
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                f32x16 sc = dot_rows16<SPLIT>(sK[st], sub, lq, lh, qf, ql, zero16());
                f32x16 dp = dot_rows16<SPLIT>(sV[st], sub, lq, lh, of, ol, zero16());
#pragma unroll
                for(int r = 0; r < 16; ++r) sc[r] = __builtin_amdgcn_exp2f(sc[r] - l2);
                if(kv0 + BLK - 1 > q0) {  // the block crosses this wave's diagonal
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) > lim) sc[r] = 0.0f;
                }
#pragma unroll
                for(int r = 0; r < 16; ++r) dp[r] = sc[r] * (dp[r] - dd);
#pragma unroll
                for(int cb = 0; cb < 2; ++cb) dq[cb] = dot_cols16<SPLIT>(sKt[st], sub, cb, lq, lh, dp, dq[cb]);
            }
        }
        if(more) {
            put_rows<SPLIT>(sK[st ^ 1], rk);
            put_cols<SPLIT>(sKt[st ^ 1], rk);
            put_rows<SPLIT>(sV[st ^ 1], rv);
        }
    }
    if(qi >= p.T) return;  // a padding row of the last block
    store_rowT(p.dq + base + qi * p.ld, dq, lh, p.scale, (p.flags & PK_ACCUM) != 0);
}

// ================================================================= fp8 products
// The same three kernels with e4m3 multiplies on v_mfma_scale_f32_32x32x64_f8f6f4
// (fp32 accumulation), which contracts 64 values of k per instruction: one
// MFMA is a whole 64-dim head product (S = Q.K^T, dP = dO.V^T) or a whole
// 64-row block of a contraction over keys or queries (O += P.V, dV += P^T.dO,
// dK += dS^T.Q, dQ += dS.K) -- 2 or 4 instructions where the bf16 kernels
// issue 8 or 16.
//
// Scaling.  q, k, v and dO enter with per-tensor powers of two: amax[] holds
// max|q|, max|k|, max|v|, max|dO| (attn_amax_kernel); a tensor x is stored as
// e4m3(x * 2^-e) with e the smallest exponent putting its largest (scaled)
// value within 448, and the MFMA's E8M0 operand scale 127 + e undoes the
// division exactly, for free.  P (in [0, 1]) enters as e4m3(256 P) with
// scale 2^-8, keeping probabilities down to 2^-17 instead of flushing those
// below e4m3's 2^-9.  dS has no range known in advance: each 32-row half of
// a 64-row block gets its own power of two (OCP MX style), from the largest
// magnitude the two lanes that hold it find between them.  The softmax
// statistics, exponentials and accumulators stay fp32.
//
// Operand layout.  Lane l supplies 32 bytes; the MFMA takes bytes 0-15 of
// every lane as k-block 0 and bytes 16-31 as k-block 1, each block scaled by
// the E8M0 scale of lane l%32 (block 0) or l%32 + 32 (block 1).  A head-dim
// contraction (row tiles, fragments) puts dims 16h..16h+15 in bytes 0-15 and
// 32+16h.. in bytes 16-31 of lane half h: the same for both operands, so each
// product pairs equal dims.  A contraction over the 64 rows of an
// accumulator pair (s[0], s[1]: rows sub*32 + acc_row(r, h)) packs s[0] into
// bytes 0-15 and s[1] into bytes 16-31, so k-block b is sub-block b; the
// other operand is a transposed tile whose columns are permuted to match:
// row position 32h + 16 sub + 4 (r / 4) + r % 4 holds row sub*32 +
// acc_row(r, h), and lane half h reads its 32 bytes from position 32h.
// Tiles have rows of LD8 = 80 bytes (16 of padding): the 8 lanes a 128-bit
// read serves per cycle hit 8 disjoint sets of 4 banks.
constexpr int LD8 = HD + 16;
constexpr int TILE8 = BLK * LD8;  // bytes
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma64(const i32x8& a, const i32x8& b, f32x16 c, int sa, int sb) {
    // formats 0, 0: both operands OCP e4m3
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

// the smallest e with amax * 2^-e <= 448, held to [-126, 126]; 0 for 0 (and NaN)
__device__ __forceinline__ int fp8_exp(float amax) {
    if(!(amax > 0.0f)) return 0;
    if(!(amax <= 3.4028235e38f)) return 126;
    int E;
    const float m = frexpf(amax, &E);
    return min(max(E - 9 + (m > 0.875f ? 1 : 0), -126), 126);
}

// four e4m3 bytes, nearest even.  No clamp: every operand here is scaled
// into e4m3's range by a power of two taken from its exact largest magnitude
// (or is 256 P <= 256), so nothing exceeds 448.
__device__ __forceinline__ int pack4_fp8(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return __builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// e4m3 of (x[0..15] * mul) as 4 dwords
__device__ __forceinline__ i32x4 pack16_fp8(const float* x, float mul) {
    i32x4 r;
#pragma unroll
    for(int q = 0; q < 4; ++q) r[q] = pack4_fp8(x[4 * q] * mul, x[4 * q + 1] * mul, x[4 * q + 2] * mul,
                                                x[4 * q + 3] * mul);
    return r;
}

// a lane's head-dim fragment of one row (see the layout note), times mul
__device__ __forceinline__ i32x8 load_frag_fp8(const float* __restrict__ row, int h, float mul, bool ok) {
    i32x8 f;
    if(!ok) {
#pragma unroll
        for(int q = 0; q < 8; ++q) f[q] = 0;
        return f;
    }
    float x[32];
#pragma unroll
    for(int c = 0; c < 4; ++c) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(row + 16 * h + 4 * c);
        const f32x4 b = *reinterpret_cast<const f32x4*>(row + 32 + 16 * h + 4 * c);
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            x[4 * c + e] = a[e];
            x[16 + 4 * c + e] = b[e];
        }
    }
    f.lo = pack16_fp8(x, mul);
    f.hi = pack16_fp8(x + 16, mul);
    return f;
}

// row-major tile: thread t's quad (rows 4*(t/16)+i, dims 4*(t%16)..+3) times mul
__device__ __forceinline__ void put_rows8(uint8_t* t, const f32x4 (&x)[4], float mul) {
    const int rq = threadIdx.x >> 4, c4 = threadIdx.x & 15;
#pragma unroll
    for(int i = 0; i < 4; ++i)
        *reinterpret_cast<int*>(t + (4 * rq + i) * LD8 + 4 * c4) =
            pack4_fp8(x[i][0] * mul, x[i][1] * mul, x[i][2] * mul, x[i][3] * mul);
}

// transposed tile with the row permutation of the layout note: dim-major,
// rows 4*(t/16)..+3 (one acc_row run of 4) at 4 consecutive positions
__device__ __forceinline__ void put_cols8(uint8_t* t, const f32x4 (&x)[4], float mul) {
    const int rq = threadIdx.x >> 4, c4 = threadIdx.x & 15;
    const int row = 4 * rq;  // sub = row/32, g = (row/8)%4, h = (row/4)%2
    const int pos = 32 * ((row >> 2) & 1) + 16 * (row >> 5) + 4 * ((row >> 3) & 3);
#pragma unroll
    for(int c = 0; c < 4; ++c)
        *reinterpret_cast<int*>(t + (4 * c4 + c) * LD8 + pos) =
            pack4_fp8(x[0][c] * mul, x[1][c] * mul, x[2][c] * mul, x[3][c] * mul);
}

// a row tile's head-dim fragment (row r) / a transposed tile's 64-row fragment
__device__ __forceinline__ i32x8 tile_frag_dims(const uint8_t* t, int r, int h) {
    i32x8 f;
    f.lo = *reinterpret_cast<const i32x4*>(t + r * LD8 + 16 * h);
    f.hi = *reinterpret_cast<const i32x4*>(t + r * LD8 + 32 + 16 * h);
    return f;
}
__device__ __forceinline__ i32x8 tile_frag_rows(const uint8_t* t, int r, int h) {
    i32x8 f;
    f.lo = *reinterpret_cast<const i32x4*>(t + r * LD8 + 32 * h);
    f.hi = *reinterpret_cast<const i32x4*>(t + r * LD8 + 32 * h + 16);
    return f;
}

// an accumulator pair (rows of two 32-row sub-blocks) as a B operand, times mul
__device__ __forceinline__ i32x8 pack_pair(const f32x16 (&x)[2], float mul) {
    float a[16], b[16];
#pragma unroll
    for(int r = 0; r < 16; ++r) {
        a[r] = x[0][r];
        b[r] = x[1][r];
    }
    i32x8 f;
    f.lo = pack16_fp8(a, mul);
    f.hi = pack16_fp8(b, mul);
    return f;
}

// the same with a power of two per sub-block (k-block): the largest magnitude
// of each sub-block over this lane and its partner (l ^ 32), which hold its
// 32 rows between them; returns this lane's E8M0 scale (its half's block)
__device__ __forceinline__ i32x8 pack_pair_mx(const f32x16 (&x)[2], int h, int& scale) {
    float am[2];
#pragma unroll
    for(int sb = 0; sb < 2; ++sb) {
        float a = 0.0f;
#pragma unroll
        for(int r = 0; r < 16; ++r) a = fmaxf(a, fabsf(x[sb][r]));
        am[sb] = fmaxf(a, __shfl_xor(a, 32, 64));
    }
    const int e0 = fp8_exp(am[0]), e1 = fp8_exp(am[1]);
    scale = 127 + (h ? e1 : e0);
    float a[16], b[16];
#pragma unroll
    for(int r = 0; r < 16; ++r) {
        a[r] = x[0][r];
        b[r] = x[1][r];
    }
    i32x8 f;
    f.lo = pack16_fp8(a, ldexpf(1.0f, -e0));
    f.hi = pack16_fp8(b, ldexpf(1.0f, -e1));
    return f;
}

// the tensors' exponents from amax[] (q times qmul, k times kmul)
struct Fp8Exps {
    int q, k, v, o;
};
__device__ __forceinline__ Fp8Exps fp8_exps(const float* amax, float qmul, float kmul) {
    return Fp8Exps{fp8_exp(amax[0] * qmul), fp8_exp(amax[1] * kmul), fp8_exp(amax[2]), fp8_exp(amax[3])};
}
constexpr int kPScale = 8;  // P enters as 2^8 P

// ------------------------------------------------------------- fp8 forward
__global__ __launch_bounds__(256, 2) void flash_fwd_fp8(FlashParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t sK[2][TILE8];   // [key][d]
    __shared__ __attribute__((aligned(16))) uint8_t sVt[2][TILE8];  // [d][key position]
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS;
    const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;
    const float qmul = p.scale * kLog2e;
    const Fp8Exps ex = fp8_exps(p.amax, qmul, 1.0f);
    const float kmul = ldexpf(1.0f, -ex.k), vmul = ldexpf(1.0f, -ex.v);

    const i32x8 qf = load_frag_fp8(Q + qi * p.ld, lh, qmul * ldexpf(1.0f, -ex.q), qi < p.T);
    f32x16 o[2] = {zero16(), zero16()};
    float m = -INFINITY, lsum = 0.0f;
    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    f32x4 rk[4], rv[4];
    fetch_quad(K, p.ld, 0, rk, p.T);
    fetch_quad(V, p.ld, 0, rv, p.T);
    put_rows8(sK[0], rk, kmul);
    put_cols8(sVt[0], rv, vmul);
    for(int j = 0; j < nkv; ++j) {
        const int st = j & 1;
        __syncthreads();
        const bool more = j + 1 < nkv;
        if(more) {
            fetch_quad(K, p.ld, (int64_t)(j + 1) * BLK, rk, p.T);
            fetch_quad(V, p.ld, (int64_t)(j + 1) * BLK, rv, p.T);
        }
        const int64_t kv0 = (int64_t)j * BLK;
        if(kv0 <= q0 + 31) {
            f32x16 s[2];
#pragma unroll
            for(int sub = 0; sub < 2; ++sub)
                s[sub] = mfma64(tile_frag_dims(sK[st], sub * 32 + lq, lh), qf, zero16(), 127 + ex.k,
                                127 + ex.q);
            if(kv0 + BLK - 1 > q0) {  // the block crosses this wave's diagonal
                const int lim = (int)(qi - kv0) - 4 * lh;
#pragma unroll
                for(int sub = 0; sub < 2; ++sub)
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) > lim) s[sub][r] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for(int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[0][r], s[1][r]));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            float ls = 0.0f;
#pragma unroll
            for(int sub = 0; sub < 2; ++sub)
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    s[sub][r] = __builtin_amdgcn_exp2f(s[sub][r] - mn);
                    ls += s[sub][r];
                }
            ls += __shfl_xor(ls, 32, 64);
            lsum = lsum * alpha + ls;
            m = mn;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                o[0][r] *= alpha;
                o[1][r] *= alpha;
            }
            const i32x8 pf = pack_pair(s, (float)(1 << kPScale));
#pragma unroll
            for(int cb = 0; cb < 2; ++cb)
                o[cb] = mfma64(tile_frag_rows(sVt[st], cb * 32 + lq, lh), pf, o[cb], 127 + ex.v, 127 - kPScale);
        }
        if(more) {
            put_rows8(sK[st ^ 1], rk, kmul);
            put_cols8(sVt[st ^ 1], rv, vmul);
        }
    }
    if(qi >= p.T) return;  // a padding row of the last block
    store_rowT(p.out + obase + qi * p.D, o, lh, 1.0f / lsum, false);
    if(lh == 0 && p.lse_out) p.lse_out[bh * p.T + qi] = (m + log2f(lsum)) * kLn2;
}

// -------------------------------------------------------- fp8 backward: dK, dV
__global__ __launch_bounds__(256, 2) void flash_bwd_dkdv_fp8(FlashParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t sQ[2][TILE8];   // [q][d]
    __shared__ __attribute__((aligned(16))) uint8_t sQt[2][TILE8];  // [d][q position]
    __shared__ __attribute__((aligned(16))) uint8_t sO[2][TILE8];   // dO [q][d]
    __shared__ __attribute__((aligned(16))) uint8_t sOt[2][TILE8];  // dO [d][q position]
    __shared__ float sLD[2][2 * BLK];                               // L2, then D
    const int64_t BH = p.B * p.H;
    const int64_t kb = (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base, *dO = p.dout + obase;
    const float* cst = p.dsum + bh * 2 * p.Tp;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t k0 = kb * ROWS + w * 32, ki = k0 + lq;
    const float kscale = p.scale * kLog2e;
    const Fp8Exps ex = fp8_exps(p.amax, 1.0f, kscale);
    const float qmul = ldexpf(1.0f, -ex.q), omul = ldexpf(1.0f, -ex.o);

    const i32x8 kf = load_frag_fp8(K + ki * p.ld, lh, kscale * ldexpf(1.0f, -ex.k), ki < p.T);
    const i32x8 vf = load_frag_fp8(V + ki * p.ld, lh, ldexpf(1.0f, -ex.v), ki < p.T);
    f32x16 dv[2] = {zero16(), zero16()}, dk[2] = {zero16(), zero16()};

    const int j0 = (int)(kb * ROWS / BLK), nq = (int)(p.Tp / BLK);
    f32x4 rq[4], ro[4];
    float rc = 0.0f;
    auto fetch = [&](int j) {
        fetch_quad(Q, p.ld, (int64_t)j * BLK, rq, p.T);
        fetch_quad(dO, p.D, (int64_t)j * BLK, ro, p.T);
        if(threadIdx.x < 2 * BLK) rc = cst[(int64_t)j * 2 * BLK + threadIdx.x];
    };
    auto put = [&](int st) {
        put_rows8(sQ[st], rq, qmul);
        put_cols8(sQt[st], rq, qmul);
        put_rows8(sO[st], ro, omul);
        put_cols8(sOt[st], ro, omul);
        if(threadIdx.x < 2 * BLK) sLD[st][threadIdx.x] = rc;
    };
    fetch(j0);
    put(0);
    for(int j = j0; j < nq; ++j) {
        const int st = (j - j0) & 1;
        __syncthreads();
        const bool more = j + 1 < nq;
        if(more) fetch(j + 1);
        const int64_t qs = (int64_t)j * BLK;
        if(qs + BLK - 1 >= k0) {
            const float* tl = sLD[st];
            const int lim = (int)(ki - qs) - 4 * lh;  // query row qr sees key ki when qr >= lim
            const bool diag = qs < k0 + 32;           // some query of the block precedes a key
            f32x16 sc[2], dp[2];
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                sc[sub] = mfma64(tile_frag_dims(sQ[st], sub * 32 + lq, lh), kf, zero16(), 127 + ex.q,
                                 127 + ex.k);
                dp[sub] = mfma64(tile_frag_dims(sO[st], sub * 32 + lq, lh), vf, zero16(), 127 + ex.o,
                                 127 + ex.v);
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const int qr = sub * 32 + acc_row(r, lh);
                    sc[sub][r] = __builtin_amdgcn_exp2f(sc[sub][r] - tl[qr]);
                }
                if(diag) {
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) < lim) sc[sub][r] = 0.0f;
                }
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const int qr = sub * 32 + acc_row(r, lh);
                    dp[sub][r] = sc[sub][r] * (dp[sub][r] - tl[BLK + qr]);
                }
            }
            const i32x8 pf = pack_pair(sc, (float)(1 << kPScale));
            int dss;
            const i32x8 df = pack_pair_mx(dp, lh, dss);
#pragma unroll
            for(int cb = 0; cb < 2; ++cb) {
                dv[cb] = mfma64(tile_frag_rows(sOt[st], cb * 32 + lq, lh), pf, dv[cb], 127 + ex.o,
                                127 - kPScale);
                dk[cb] = mfma64(tile_frag_rows(sQt[st], cb * 32 + lq, lh), df, dk[cb], 127 + ex.q, dss);
            }
        }
        if(more) put(st ^ 1);
    }
    if(ki >= p.T) return;  // a padding row of the last block
    store_rowT(p.dv + base + ki * p.ld, dv, lh, 1.0f, (p.flags & PK_ACCUM3) != 0);
    store_rowT(p.dk + base + ki * p.ld, dk, lh, p.scale, (p.flags & PK_ACCUM2) != 0);
}

// ------------------------------------------------------------- fp8 backward: dQ
__global__ __launch_bounds__(256, 2) void flash_bwd_dq_fp8(FlashParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t sK[2][TILE8];   // [key][d]
    __shared__ __attribute__((aligned(16))) uint8_t sKt[2][TILE8];  // [d][key position]
    __shared__ __attribute__((aligned(16))) uint8_t sV[2][TILE8];   // [key][d]
    const int64_t BH = p.B * p.H, nqb = p.Tp / ROWS;
    const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / BH, bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t base = b * p.T * p.ld + h * HD, obase = b * p.T * p.D + h * HD;
    const float *Q = p.q + base, *K = p.k + base, *V = p.v + base, *dO = p.dout + obase;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lq = l & 31, lh = l >> 5;
    const int64_t q0 = qb * ROWS + w * 32, qi = q0 + lq;
    const float qmul = p.scale * kLog2e;
    const Fp8Exps ex = fp8_exps(p.amax, qmul, 1.0f);
    const float kmul = ldexpf(1.0f, -ex.k), vmul = ldexpf(1.0f, -ex.v);

    const i32x8 qf = load_frag_fp8(Q + qi * p.ld, lh, qmul * ldexpf(1.0f, -ex.q), qi < p.T);
    const i32x8 of = load_frag_fp8(dO + qi * p.D, lh, ldexpf(1.0f, -ex.o), qi < p.T);
    const float* cst = p.dsum + bh * 2 * p.Tp + (qi / BLK) * 2 * BLK + qi % BLK;
    const float l2 = cst[0], dd = cst[BLK];
    f32x16 dq[2] = {zero16(), zero16()};

    const int nkv = (int)((qb * ROWS + ROWS) / BLK);
    f32x4 rk[4], rv[4];
    fetch_quad(K, p.ld, 0, rk, p.T);
    fetch_quad(V, p.ld, 0, rv, p.T);
    put_rows8(sK[0], rk, kmul);
    put_cols8(sKt[0], rk, kmul);
    put_rows8(sV[0], rv, vmul);
    for(int j = 0; j < nkv; ++j) {
        const int st = j & 1;
        __syncthreads();
        const bool more = j + 1 < nkv;
        if(more) {
            fetch_quad(K, p.ld, (int64_t)(j + 1) * BLK, rk, p.T);
            fetch_quad(V, p.ld, (int64_t)(j + 1) * BLK, rv, p.T);
        }
        const int64_t kv0 = (int64_t)j * BLK;
        if(kv0 <= q0 + 31) {
            const int lim = (int)(qi - kv0) - 4 * lh;
            f32x16 sc[2], dp[2];
#pragma unroll
            for(int sub = 0; sub < 2; ++sub) {
                sc[sub] = mfma64(tile_frag_dims(sK[st], sub * 32 + lq, lh), qf, zero16(), 127 + ex.k,
                                 127 + ex.q);
                dp[sub] = mfma64(tile_frag_dims(sV[st], sub * 32 + lq, lh), of, zero16(), 127 + ex.v,
                                 127 + ex.o);
#pragma unroll
                for(int r = 0; r < 16; ++r) sc[sub][r] = __builtin_amdgcn_exp2f(sc[sub][r] - l2);
                if(kv0 + BLK - 1 > q0) {  // the block crosses this wave's diagonal
#pragma unroll
                    for(int r = 0; r < 16; ++r)
                        if(sub * 32 + 8 * (r >> 2) + (r & 3) > lim) sc[sub][r] = 0.0f;
                }
#pragma unroll
                for(int r = 0; r < 16; ++r) dp[sub][r] = sc[sub][r] * (dp[sub][r] - dd);
            }
            int dss;
            const i32x8 df = pack_pair_mx(dp, lh, dss);
#pragma unroll
            for(int cb = 0; cb < 2; ++cb)
                dq[cb] = mfma64(tile_frag_rows(sKt[st], cb * 32 + lq, lh), df, dq[cb], 127 + ex.k, dss);
        }
        if(more) {
            put_rows8(sK[st ^ 1], rk, kmul);
            put_cols8(sKt[st ^ 1], rk, kmul);
            put_rows8(sV[st ^ 1], rv, vmul);
        }
    }
    if(qi >= p.T) return;  // a padding row of the last block
    store_rowT(p.dq + base + qi * p.ld, dq, lh, p.scale, (p.flags & PK_ACCUM) != 0);
}

// amax[0..3] = max|q|, max|k|, max|v| over the heads' columns of rows
// [0, rows) (row stride ld), max|dO| (row stride D), each taken when its
// pointer is given; amax must be zero beforehand (attn_amax_zero).  Positive
// floats order as their bit patterns, so an integer atomic max combines them.
__global__ void attn_amax_zero(float* amax, int first, int n) {
    if((int)threadIdx.x < n) amax[first + threadIdx.x] = 0.0f;
}
// blockIdx.y picks the tensor; a workgroup takes 32 rows, its lanes walking
// their float4s (lane e = l + 256 j of the 32 * D/4) with all of a lane's
// loads independent, so they are in flight together
__global__ __launch_bounds__(256) void attn_amax_kernel(const float* q, const float* k, const float* v,
                                                        const float* dout, int64_t rows, int64_t D, int64_t ld,
                                                        float* amax) {
    const int t = blockIdx.y;
    const float* src = t == 0 ? q : t == 1 ? k : t == 2 ? v : dout;
    if(!src) return;
    const int64_t stride = t == 3 ? D : ld;
    const int c4n = (int)(D / 4);
    const int64_t r0 = (int64_t)blockIdx.x * 32;
    const int n = (int)(std::min<int64_t>(32, rows - r0)) * c4n;
    int row = (int)threadIdx.x / c4n, col = (int)threadIdx.x - row * c4n;
    const int drow = 256 / c4n, dcol = 256 - drow * c4n;
    float a = 0.0f;
    for(int e0 = 0; e0 < n; e0 += 16 * 256) {
        // up to 16 loads a lane, all issued before the first is used
        f32x4 x[16];
#pragma unroll
        for(int j = 0; j < 16; ++j) {
            x[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if(e0 + (int)threadIdx.x + 256 * j < n)
                x[j] = *reinterpret_cast<const f32x4*>(src + (r0 + row) * stride + 4 * col);
            row += drow;
            col += dcol;
            if(col >= c4n) {
                col -= c4n;
                ++row;
            }
        }
#pragma unroll
        for(int j = 0; j < 16; ++j)
            a = fmaxf(a, fmaxf(fmaxf(fabsf(x[j][0]), fabsf(x[j][1])), fmaxf(fabsf(x[j][2]), fabsf(x[j][3]))));
    }
    // one atomic per workgroup: thousands on one address queue up at the cache
    __shared__ float wmax[4];
    a = pk::wave_max(a);
    if((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = a;
    __syncthreads();
    a = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    if(threadIdx.x == 0 && a > 0.0f) atomicMax(reinterpret_cast<unsigned*>(amax + t), __float_as_uint(a));
}

int flash_check(const char* who, int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                const void* a, const void* b, const void* c) {
    if(B < 0 || H < 1 || T < 0) return pk::fail("%s: bad sizes", who);
    if(hd != HD) return pk::fail("%s: head size %lld (this kernel handles 64)", who, (long long)hd);
    if(ld < H * HD || ld % 4)
        return pk::fail("%s: row stride %lld of q, k, v must be >= %lld and a multiple of 4", who,
                        (long long)ld, (long long)(H * HD));
    if(!pk::aligned16(a) || !pk::aligned16(b) || !pk::aligned16(c))
        return pk::fail("%s: q, k, v must be 16-byte aligned", who);
    const int64_t Tp = (T + ROWS - 1) / ROWS * ROWS;
    if(B * H * (Tp / ROWS) > 0x7fffffff || Tp * ld * 4 > 0x7fffffff)
        return pk::fail("%s: problem too large", who);
    return PK_OK;
}

}  // namespace

extern "C" int pk_flash_attn_supported(int64_t T, int64_t hd) { return hd == HD && T > 0; }

namespace {

// The dispatch table of a launch over BH heads of nqb 128-row blocks with
// `slots` workgroups per CU (cached per shape, per host thread).  Rank r
// (heaviest first) streams 2*(nqb - r/BH) 64-row blocks of the other operand.  Slot k of CU c is workgroup c + kCUs*k and
// exists when that is below the table's length.
const FlashPlan& flash_plan(int64_t BH, int64_t nqb, int slots) {
    // one cached plan per slot count (each kernel has its own)
    thread_local int64_t cached_bh[kMaxSlots + 1] = {-1, -1, -1, -1, -1},
                         cached_nqb[kMaxSlots + 1] = {-1, -1, -1, -1, -1};
    thread_local FlashPlan plans[kMaxSlots + 1];
    FlashPlan& plan = plans[slots];
    if(cached_bh[slots] == BH && cached_nqb[slots] == nqb) return plan;
    const int n = (int)std::min<int64_t>(BH * nqb, slots * kCUs);
    std::vector<int> used(kCUs, 0);
    // (work so far, cu) of the CUs with a free slot, least work first
    std::priority_queue<std::pair<int64_t, int>, std::vector<std::pair<int64_t, int>>,
                        std::greater<std::pair<int64_t, int>>>
        free_cus;
    for(int c = 0; c < kCUs && c < n; ++c) free_cus.push({0, c});
    for(int r = 0; r < n; ++r) {
        const std::pair<int64_t, int> top = free_cus.top();
        free_cus.pop();
        const int c = top.second, b = c + kCUs * used[c]++;
        plan.rank[b] = (uint16_t)r;
        if(c + kCUs * used[c] < n) free_cus.push({top.first + 2 * (nqb - r / BH), c});
    }
    plan.n = n;
    cached_bh[slots] = BH;
    cached_nqb[slots] = nqb;
    return plan;
}

// products of a launch: fp32, bf16, fp8 (e4m3) or split bf16 (three bf16
// products per fp32 one)
enum FlashPrec { kF32 = 0, kBF16 = 1, kFP8 = 2, kBF16X3 = 3 };

// fp8: max|.| of q, k, v (first = 0, the forward) or of dout (first = 3, the
// backward) into amax[first..]
void attn_amax(int first, int64_t rows, int64_t D, int64_t ld, const float* q, const float* k,
               const float* v, const float* dout, float* amax, hipStream_t st) {
    attn_amax_zero<<<1, 64, 0, st>>>(amax, first, first == 0 ? 3 : 1);
    attn_amax_kernel<<<dim3((unsigned)((rows + 31) / 32), 4), 256, 0, st>>>(q, k, v, dout, rows, D, ld,
                                                                           amax);
}

int flash_fwd_launch(const char* who, int prec, int64_t B, int64_t H, int64_t T, int64_t hd,
                     int64_t ld, float scale, const float* q, const float* k, const float* v,
                     float* o, float* lse, float* amax, pk_stream_t stream) {
    int rc = flash_check(who, B, H, T, hd, ld, q, k, v);
    if(rc) return rc;
    if(B == 0 || T == 0) return PK_OK;
    if(!o || !pk::aligned16(o)) return pk::fail("%s: o NULL or unaligned", who);
    if(prec == kFP8 && !amax) return pk::fail("%s: NULL amax", who);
    FlashParams p = {};
    p.q = q;
    p.k = k;
    p.v = v;
    p.out = o;
    p.lse_out = lse;
    p.B = B;
    p.H = H;
    p.T = T;
    p.Tp = (T + ROWS - 1) / ROWS * ROWS;
    p.D = H * HD;
    p.ld = ld;
    p.scale = scale;
    const unsigned grid = (unsigned)(B * H * (p.Tp / ROWS));
    hipStream_t st = pk::as_stream(stream);
    if(prec == kFP8) {
        attn_amax(0, B * T, p.D, ld, q, k, v, nullptr, amax, st);
        if((rc = pk::launch_status(who))) return rc;
        p.amax = amax;
        flash_fwd_fp8<<<grid, 256, 0, st>>>(p);
    } else if(prec == kBF16) {
        flash_fwd_bf16<false><<<grid, 256, 0, st>>>(p);
    } else if(prec == kBF16X3) {
        flash_fwd_bf16<true><<<grid, 256, 0, st>>>(p);
    } else {
        flash_fwd<<<grid, 256, 0, st>>>(p, flash_plan(B * H, p.Tp / ROWS, kFwdSlots));
    }
    return pk::launch_status(who);
}

}  // namespace

extern "C" int pk_flash_attn_fwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                     float scale, const float* q, const float* k, const float* v,
                                     float* o, float* lse, pk_stream_t stream) {
    return flash_fwd_launch("pk_flash_attn_fwd_f32", kF32, B, H, T, hd, ld, scale, q, k, v, o,
                            lse, nullptr, stream);
}

extern "C" int pk_flash_attn_fwd_bf16_f32(int64_t B, int64_t H, int64_t T, int64_t hd,
                                          int64_t ld, float scale, const float* q, const float* k,
                                          const float* v, float* o, float* lse,
                                          pk_stream_t stream) {
    return flash_fwd_launch("pk_flash_attn_fwd_bf16_f32", kBF16, B, H, T, hd, ld, scale, q, k, v,
                            o, lse, nullptr, stream);
}

extern "C" int pk_flash_attn_fwd_bf16x3_f32(int64_t B, int64_t H, int64_t T, int64_t hd,
                                            int64_t ld, float scale, const float* q, const float* k,
                                            const float* v, float* o, float* lse,
                                            pk_stream_t stream) {
    return flash_fwd_launch("pk_flash_attn_fwd_bf16x3_f32", kBF16X3, B, H, T, hd, ld, scale, q, k, v,
                            o, lse, nullptr, stream);
}

extern "C" int pk_flash_attn_fwd_fp8_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                         float scale, const float* q, const float* k,
                                         const float* v, float* o, float* lse, float* amax,
                                         pk_stream_t stream) {
    return flash_fwd_launch("pk_flash_attn_fwd_fp8_f32", kFP8, B, H, T, hd, ld, scale, q, k, v, o,
                            lse, amax, stream);
}

// row constants (2*B*H*Tp floats, Tp = T rounded up to 128), then the dS tiles
extern "C" size_t pk_flash_attn_bwd_workspace(int64_t B, int64_t H, int64_t T) {
    if(B <= 0 || H <= 0 || T <= 0) return 0;
    const int64_t Tp = (T + ROWS - 1) / ROWS * ROWS;
    return (size_t)(2 * B * H * Tp + B * H * ds_tiles(Tp) * 1024) * sizeof(float);
}

// the row constants only (PK_FLASH_RECOMPUTE)
extern "C" size_t pk_flash_attn_bwd_workspace_recompute(int64_t B, int64_t H, int64_t T) {
    if(B <= 0 || H <= 0 || T <= 0) return 0;
    const int64_t Tp = (T + ROWS - 1) / ROWS * ROWS;
    return (size_t)(2 * B * H * Tp) * sizeof(float);
}

namespace {

int flash_bwd_launch(const char* who, int prec, int64_t B, int64_t H, int64_t T, int64_t hd,
                     int64_t ld, float scale, const float* q, const float* k, const float* v,
                     const float* o, const float* lse, const float* dout, float* dq, float* dk,
                     float* dv, float* amax, void* workspace, size_t workspace_bytes, int flags,
                     pk_stream_t stream) {
    int rc = flash_check(who, B, H, T, hd, ld, q, k, v);
    if(rc) return rc;
    if(B == 0 || T == 0) return PK_OK;
    if(!o || !lse || !dout || !dq || !dk || !dv) return pk::fail("%s: NULL pointer", who);
    if(!pk::aligned16(o) || !pk::aligned16(dout) || !pk::aligned16(dq) || !pk::aligned16(dk) ||
       !pk::aligned16(dv))
        return pk::fail("%s: o, dout, dq, dk, dv must be 16-byte aligned", who);
    const bool recompute = (flags & PK_FLASH_RECOMPUTE) != 0;
    if(recompute && prec != kF32)
        return pk::fail("%s: PK_FLASH_RECOMPUTE is built for the fp32 products only", who);
    if(prec == kFP8 && !amax) return pk::fail("%s: NULL amax", who);
    const size_t need = recompute ? pk_flash_attn_bwd_workspace_recompute(B, H, T)
                                  : pk_flash_attn_bwd_workspace(B, H, T);
    if(!workspace || workspace_bytes < need)
        return pk::fail("%s: workspace needs %zu bytes", who, need);
    if(!pk::aligned16(workspace)) return pk::fail("%s: workspace must be 16-byte aligned", who);
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
    const int64_t Tp = (T + ROWS - 1) / ROWS * ROWS;
    p.ds = recompute ? nullptr : static_cast<float*>(workspace) + 2 * B * H * Tp;
    p.B = B;
    p.H = H;
    p.T = T;
    p.Tp = (T + ROWS - 1) / ROWS * ROWS;
    p.D = H * HD;
    p.ld = ld;
    p.scale = scale;
    p.flags = flags & (PK_ACCUM | PK_ACCUM2 | PK_ACCUM3);
    hipStream_t st = pk::as_stream(stream);
    if(prec == kFP8) {
        attn_amax(3, B * T, p.D, ld, nullptr, nullptr, nullptr, dout, amax, st);
        if((rc = pk::launch_status(who))) return rc;
        p.amax = amax;
    }
    flash_dsum<<<pk::grid_for(B * H * p.Tp * 16, 256), 256, 0, st>>>(p);
    if((rc = pk::launch_status(who))) return rc;
    const unsigned grid = (unsigned)(B * H * (p.Tp / ROWS));
    if(prec == kFP8)
        flash_bwd_dkdv_fp8<<<grid, 256, 0, st>>>(p);
    else if(prec == kBF16)
        flash_bwd_dkdv_bf16<false><<<grid, 256, 0, st>>>(p);
    else if(prec == kBF16X3)
        flash_bwd_dkdv_bf16<true><<<grid, 256, 0, st>>>(p);
    else
        flash_bwd_dkdv<<<grid, 256, 0, st>>>(p);
    if((rc = pk::launch_status(who))) return rc;
    if(prec == kFP8)
        flash_bwd_dq_fp8<<<grid, 256, 0, st>>>(p);
    else if(prec == kBF16)
        flash_bwd_dq_bf16<false><<<grid, 256, 0, st>>>(p);
    else if(prec == kBF16X3)
        flash_bwd_dq_bf16<true><<<grid, 256, 0, st>>>(p);
    else if(recompute)
        flash_bwd_dq_recompute<<<grid, 256, 0, st>>>(p);
    else
        flash_bwd_dq<<<grid, 256, 0, st>>>(p, flash_plan(B * H, p.Tp / ROWS, kDqSlots));
    return pk::launch_status(who);
}

}  // namespace

extern "C" int pk_flash_attn_bwd_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                     float scale, const float* q, const float* k, const float* v,
                                     const float* o, const float* lse, const float* dout,
                                     float* dq, float* dk, float* dv, void* workspace,
                                     size_t workspace_bytes, int flags, pk_stream_t stream) {
    return flash_bwd_launch("pk_flash_attn_bwd_f32", kF32, B, H, T, hd, ld, scale, q, k, v, o,
                            lse, dout, dq, dk, dv, nullptr, workspace, workspace_bytes, flags, stream);
}

extern "C" int pk_flash_attn_bwd_bf16_f32(int64_t B, int64_t H, int64_t T, int64_t hd,
                                          int64_t ld, float scale, const float* q, const float* k,
                                          const float* v, const float* o, const float* lse,
                                          const float* dout, float* dq, float* dk, float* dv,
                                          void* workspace, size_t workspace_bytes, int flags,
                                          pk_stream_t stream) {
    return flash_bwd_launch("pk_flash_attn_bwd_bf16_f32", kBF16, B, H, T, hd, ld, scale, q, k, v,
                            o, lse, dout, dq, dk, dv, nullptr, workspace, workspace_bytes, flags,
                            stream);
}

extern "C" int pk_flash_attn_bwd_bf16x3_f32(int64_t B, int64_t H, int64_t T, int64_t hd,
                                            int64_t ld, float scale, const float* q, const float* k,
                                            const float* v, const float* o, const float* lse,
                                            const float* dout, float* dq, float* dk, float* dv,
                                            void* workspace, size_t workspace_bytes, int flags,
                                            pk_stream_t stream) {
    return flash_bwd_launch("pk_flash_attn_bwd_bf16x3_f32", kBF16X3, B, H, T, hd, ld, scale, q, k, v,
                            o, lse, dout, dq, dk, dv, nullptr, workspace, workspace_bytes, flags,
                            stream);
}

extern "C" int pk_flash_attn_bwd_fp8_f32(int64_t B, int64_t H, int64_t T, int64_t hd, int64_t ld,
                                         float scale, const float* q, const float* k,
                                         const float* v, const float* o, const float* lse,
                                         const float* dout, float* dq, float* dk, float* dv,
                                         float* amax, void* workspace, size_t workspace_bytes,
                                         int flags, pk_stream_t stream) {
    return flash_bwd_launch("pk_flash_attn_bwd_fp8_f32", kFP8, B, H, T, hd, ld, scale, q, k, v, o,
                            lse, dout, dq, dk, dv, amax, workspace, workspace_bytes, flags, stream);
}
