// pico_amd/csrc/gemm_fp8q.hip -- fp8 products from fp8 operands held in HBM
// (opt-in, outside the fp32 parity contract; no reference counterpart: pico
// is fp32 only, src/tensor.h:14-15).
//
// pk_gemm_fp8_f32 rounds fp32 operands to e4m3 on their way into LDS, so it
// moves 4 bytes per operand element and multiplies with
// v_mfma_f32_32x32x16_fp8_fp8 (the bf16 rate).  Here the operands are
// quantized once (pk_fp8_quantize_f32: e4m3 of scale * x, K-contiguous rows,
// zero padding to whole tiles) and the product reads 1 byte per element and
// multiplies with v_mfma_scale_f32_32x32x64_f8f6f4, twice the flops per
// cycle of the 32x32x16 form:
//   C = alpha / (sA * sB) * A.B^T (+ beta * C),  A [M, K], B [N, K] e4m3.
//
// Design (one 256-thread workgroup = 4 waves per 256x256 C tile; each wave
// 128x128 as 4x4 blocks of 32x32, 256 fp32 accumulators per lane):
//  * K advances 64 bytes a slice through a QSTAGES-deep LDS ring (32 KB a
//    stage): the loads of slice s+QSTAGES are issued while slice s is
//    multiplied, straight from global memory into LDS (buffer_load_dwordx4
//    ... lds: one instruction fills 1 KB, lane l's 16 bytes at +16*l), so no
//    staging registers and no VALU work.
//  * An LDS row is one 64-byte slice row, its four 16-byte chunks XOR-
//    swizzled: chunk c of row r sits in slot c ^ ((r >> 1) & 3).  The 8 lanes
//    a 128-bit read serves per cycle read rows r..r+7 at one chunk; their
//    (row parity, slot) pairs are all different, so they hit 8 disjoint sets
//    of 4 banks.  A load lane picks the global chunk that belongs in its slot.
//  * An MFMA takes 32 bytes of row l%32 of A (column l%32 of B) from lane l:
//    its first 16 belong to the instruction's k-block 0 (k 0-31, lanes 0-31
//    holding k 0-15, lanes 32-63 k 16-31), its last 16 to k-block 1, and the
//    E8M0 scale of lane l serves k-block l/32 of its row (measured: a scale
//    of 2 on lanes 32-63 doubles exactly the products of bytes 16-31 of every
//    lane).  So lane l reads 16-byte chunks l/32 and l/32 + 2 of the slice
//    row -- two 128-bit LDS reads per operand block -- and k-block b of the
//    instruction is bytes 32b..32b+31 of the slice, the 32 values a scale of
//    the quantizer covers.
//  * The fragments of slice s+1 are read into a second register set while the
//    16 MFMAs of slice s run, so each wave's matrix core waits on LDS only in
//    the prologue.
//  * Tile order as the fp32 kernel's: XCD-contiguous runs, GROUP_M tile-rows.
#include <stdint.h>

#include "pk_common.h"

namespace {

constexpr int NT = 256;
constexpr int QB = 64;                        // k bytes per slice = bytes of an LDS row
constexpr int QKPAD = 2 * QB;                 // K padding: an even number of slices
constexpr int QT = 256;                       // rows of an operand tile (and C tile side)
constexpr int QSTAGE = QT * QB;               // bytes of one operand's tile in one stage
constexpr int QSTAGES = 4;
constexpr int QLW = QSTAGE / 1024 / 4;        // 1 KB load instructions per wave per operand: 4
constexpr int QGROUP_M = 8;
constexpr int64_t kTileQ = 256;

typedef __attribute__((address_space(3))) void lds_ptr_t;
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

struct Fp8qParams {
    const uint8_t *A, *B;
    const uint8_t *SA, *SB;  // MX: E8M0 block scales, [slice][rows][2]
    int64_t sstride_a, sstride_b;  // MX: bytes of one slice's scales (2 * padded rows)
    float* C;
    const float* X;       // C = alpha * product (+ beta * X); X == C accumulates
    const float* scales;  // per-tensor mode: device sA, sB (NULL: 1, 1)
    int64_t M, N, lda, ldb, ldc, ldx;
    int nslices;
    float alpha, beta;
    int tiles_m, tiles_n;
};

__device__ __forceinline__ int slot_of(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

// the load instructions of one operand tile: lane l of instruction n fills
// LDS slot l % 4 of row 16n + l / 4 (n = w + 4i), from the chunk that belongs there
struct QLoad {
    int voff[QLW];
    __device__ __forceinline__ QLoad(int64_t ld, int w, int l) {
#pragma unroll
        for(int i = 0; i < QLW; ++i) {
            const int r = 16 * (w + 4 * i) + l / 4;
            voff[i] = r * (int)ld + 16 * slot_of(r, l % 4);  // slot_of is its own inverse
        }
    }
    __device__ __forceinline__ void issue_one(int i, __amdgpu_buffer_rsrc_t rs, int soff, uint8_t* tile,
                                              int w) const {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t*)(tile + 1024 * (w + 4 * i)), 16, voff[i],
                                                 soff, 0, 0);
    }
    __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, int soff, uint8_t* tile,
                                          int w) const {
#pragma unroll
        for(int i = 0; i < QLW; ++i) issue_one(i, rs, soff, tile, w);
    }
};

// 16-byte chunk lh + 2h of row `row` of a stage's operand tile: half h of
// this lane's MFMA operand (see the layout note at the top)
__device__ __forceinline__ i32x4 frag_half(const uint8_t* __restrict__ tile, int row, int lh, int h) {
    return *reinterpret_cast<const i32x4*>(tile + row * QB + 16 * slot_of(row, lh + 2 * h));
}
__device__ __forceinline__ i32x8 frag(const uint8_t* __restrict__ tile, int row, int lh) {
    i32x8 f;
    f.lo = frag_half(tile, row, lh, 0);
    f.hi = frag_half(tile, row, lh, 1);
    return f;
}

// e4m3 x e4m3 -> fp32 on the 32x32x64 matrix core; sa, sb: this lane's E8M0
// block scales (byte 0; 127 = 2^0)
__device__ __forceinline__ f32x16 mfma_fp8(const i32x8& a, const i32x8& b, const f32x16& c, int sa,
                                           int sb) {
    // formats 0, 0: both operands OCP e4m3
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

// wait until at most n of this wave's vector-memory loads are outstanding and
// its LDS reads are done
template <int n>
__device__ __forceinline__ void wait_vm_lds() {
    static_assert(n >= 0 && n < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(((n >> 4) << 14) | 0x0070 | (n & 15));
}

// workgroup barrier that leaves later loads in flight: __syncthreads' fence
// would wait for every outstanding load, the next slices' included.  The LDS
// writes it orders are the direct-to-LDS loads, each wave having waited for
// its own, and the LDS reads of the stage refilled after it, each wave
// having waited for those too (wait_vm_lds).
__device__ __forceinline__ void barrier_keep_loads() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// MX: operands carry E8M0 scales per 32 k (one per lane's 32 bytes of an
// MFMA operand), streamed into LDS beside the bytes and handed to the MFMA;
// otherwise the scales are 2^0 and the tensor scales divide in the epilogue.
template <bool MX>
__global__ __launch_bounds__(NT, 1) void gemm_fp8q_kernel(Fp8qParams p) {
    // a stage: each operand's 256 rows of 64 bytes, then (MX) its scales,
    // [row][2 halves of the slice's k]
    constexpr int OPB = QSTAGE + (MX ? QT * 2 : 0);
    __shared__ __attribute__((aligned(16))) uint8_t lds[QSTAGES][2][OPB];
    const int ntiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
    const int group_span = QGROUP_M * p.tiles_n;
    const int first_m = (bid / group_span) * QGROUP_M;
    const int gm = min(p.tiles_m - first_m, QGROUP_M);
    const int local = bid % group_span;
    const int64_t row0 = (int64_t)(first_m + local % gm) * QT, col0 = (int64_t)(local / gm) * QT;

    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lr = l & 31, lh = l >> 5;
    const int wm = w >> 1, wn = w & 1;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.A), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.B), (short)0, 0x7fffffff, 0x00020000);
    const QLoad la(p.lda, w, l), lb(p.ldb, w, l);
    const int sa = (int)(row0 * p.lda), sb = (int)(col0 * p.ldb);
    // MX scales: wave w fetches 128 rows' (w & 1) of operand w >> 1, 256 bytes
    // (4 per lane); the operand and half are wave-uniform
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(wm ? p.SB : p.SA), (short)0, 0x7fffffff, 0x00020000);
    const int sc0 = (int)((wm ? col0 : row0) * 2 + (w & 1) * 256);
    const int sc_stride = (int)(wm ? p.sstride_b : p.sstride_a);
    const int ns = p.nslices;
    auto issue_scales = [&](int s, int st) {
        if constexpr(MX)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t*)(&lds[st][wm][QSTAGE + (w & 1) * 256]), 4, 4 * l,
                                                     sc0 + min(s, ns - 1) * sc_stride, 0, 0);
    };
    // slice s into stage s % QSTAGES; past the last slice the last one is
    // fetched again (into a stage nobody reads), which keeps every iteration's
    // count of outstanding loads the same
    auto issue = [&](int s) {
        const int st = s % QSTAGES, k = min(s, ns - 1) * QB;
        la.issue(ra, sa + k, lds[st][0], w);
        lb.issue(rb, sb + k, lds[st][1], w);
        issue_scales(s, st);
    };

    f32x16 acc[4][4];
#pragma unroll
    for(int i = 0; i < 4; ++i)
#pragma unroll
        for(int j = 0; j < 4; ++j)
#pragma unroll
            for(int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // this lane's scale of block i of an operand in stage st
    auto scale_of = [&](int st, int op, int i) -> int {
        if constexpr(MX)
            return lds[st][op][QSTAGE + ((op ? wn : wm) * 128 + 32 * i + lr) * 2 + lh];
        else
            return 127;
    };
    auto read = [&](int s, i32x8 (&fa)[4], i32x8 (&fb)[4], int (&ca)[4], int (&cb)[4]) {
        const int st = s % QSTAGES;
#pragma unroll
        for(int i = 0; i < 4; ++i) {
            fa[i] = frag(lds[st][0], wm * 128 + 32 * i + lr, lh);
            ca[i] = scale_of(st, 0, i);
        }
#pragma unroll
        for(int j = 0; j < 4; ++j) {
            fb[j] = frag(lds[st][1], wn * 128 + 32 * j + lr, lh);
            cb[j] = scale_of(st, 1, j);
        }
    };
    constexpr int PER = 2 * QLW + (MX ? 1 : 0);  // loads of one slice, per wave
    // slice s with its fragments in (fa, fb) and scales in (ca, cb): wait for
    // slice s+1's loads and every wave's reads of slice s, then 16 groups,
    // each one MFMA of slice s, one 128-bit LDS read of slice s+1's fragments
    // into (ga, gb) (in the order the next slice's MFMAs use them: A0,
    // B0..B3, A1..A3), in the first 8 one load refilling slice s's stage with
    // slice s+QSTAGES, in the 9th its scales' load, and in the last 8 one read
    // of slice s+1's scales.  The scheduling barriers keep that order: left
    // alone, the compiler moves the next slice's wait above the last MFMAs.
    auto step = [&](int s, i32x8 (&fa)[4], i32x8 (&fb)[4], int (&ca)[4], int (&cb)[4], i32x8 (&ga)[4],
                    i32x8 (&gb)[4], int (&da)[4], int (&db)[4]) {
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_lds<(QSTAGES - 2) * PER>();
        barrier_keep_loads();
        const int nx = (s + 1) % QSTAGES, fill = s % QSTAGES;
        const int k = min(s + QSTAGES, ns - 1) * QB;
#pragma unroll
        for(int g = 0; g < 16; ++g) {
            const int i = g >> 2, j = g & 3;
            acc[i][j] = mfma_fp8(fa[i], fb[j], acc[i][j], ca[i], cb[j]);
            constexpr int order[8] = {0, 4, 5, 6, 7, 1, 2, 3};
            const int f = order[g >> 1], h = g & 1;
            if(f < 4) {
                const i32x4 v = frag_half(lds[nx][0], wm * 128 + 32 * f + lr, lh, h);
                if(h) ga[f].hi = v; else ga[f].lo = v;
            } else {
                const i32x4 v = frag_half(lds[nx][1], wn * 128 + 32 * (f - 4) + lr, lh, h);
                if(h) gb[f - 4].hi = v; else gb[f - 4].lo = v;
            }
            if(g < QLW)
                la.issue_one(g, ra, sa + k, lds[fill][0], w);
            else if(g < 2 * QLW)
                lb.issue_one(g - QLW, rb, sb + k, lds[fill][1], w);
            else if(g == 2 * QLW)
                issue_scales(s + QSTAGES, fill);
            if(g >= 8) {
                const int q = g - 8;
                if(q < 4) da[q] = scale_of(nx, 0, q); else db[q - 4] = scale_of(nx, 1, q - 4);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if(ns > 0) {
#pragma unroll
        for(int s = 0; s < QSTAGES; ++s) issue(s);
        i32x8 a0[4], b0[4], a1[4], b1[4];
        int ca0[4], cb0[4], ca1[4], cb1[4];
        wait_vm_lds<(QSTAGES - 1) * PER>();
        barrier_keep_loads();
        read(0, a0, b0, ca0, cb0);
        for(int s = 0; s < ns; s += 2) {  // ns is even: K is padded to 128 bytes
            step(s, a0, b0, ca0, cb0, a1, b1, ca1, cb1);
            step(s + 1, a1, b1, ca1, cb1, a0, b0, ca0, cb0);
        }
        wait_vm_lds<0>();  // no load may land in LDS after the workgroup ends
    }

    const float scale = MX || !p.scales ? p.alpha : p.alpha / (p.scales[0] * p.scales[1]);
    const bool full = row0 + QT <= p.M && col0 + QT <= p.N;
    if(full && !p.X) {
#pragma unroll
        for(int i = 0; i < 4; ++i)
#pragma unroll
            for(int j = 0; j < 4; ++j) {
                float* c = p.C + (row0 + wm * 128 + 32 * i + 4 * lh) * p.ldc + col0 + wn * 128 + 32 * j + lr;
#pragma unroll
                for(int r = 0; r < 16; ++r) c[(8 * (r >> 2) + (r & 3)) * p.ldc] = scale * acc[i][j][r];
            }
        return;
    }
#pragma unroll
    for(int i = 0; i < 4; ++i)
#pragma unroll
        for(int j = 0; j < 4; ++j) {
            const int64_t col = col0 + wn * 128 + 32 * j + lr;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * 128 + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                if(row >= p.M || col >= p.N) continue;
                float v = scale * acc[i][j][r];
                if(p.X) v += p.beta * p.X[row * p.ldx + col];
                p.C[row * p.ldc + col] = v;
            }
        }
}

// ---- quantization: Q[r][k] = e4m3(scale * op(X)[r][k]), zero padding -------
__device__ __forceinline__ float e4m3_clamp(float x) {
    return x != x ? x : fminf(fmaxf(x, -448.0f), 448.0f);
}

// MX block exponent: the smallest e with amax * 2^-e <= 448 (e4m3's largest
// finite value), held to E8M0's [-127, 127]; 0 for an all-zero block.  With
// amax = m * 2^E, m in [0.5, 1): amax * 2^-e <= 0.875 * 2^9 iff
// e >= E - 9 (m <= 0.875) or E - 8 (m > 0.875).
__device__ __forceinline__ int mx_exponent(float amax) {
    if(!(amax > 0.0f)) return 0;
    if(!(amax <= 3.4028235e38f)) return 127;
    int E;
    const float m = frexpf(amax, &E);
    return min(max(E - 9 + (m > 0.875f ? 1 : 0), -127), 127);
}

// one 64 x 64 block of op(X) through LDS: read along X's contiguous dimension,
// written as 16 e4m3 bytes per thread along k.  MX: each 32-value half row
// (threads t, t ^ 1) takes its own scale 2^-e; its E8M0 byte e + 127 goes to
// S[slice][row][half] (slice = the block's 64 k, rows padded to Rp).
template <bool MX>
__global__ __launch_bounds__(NT) void fp8_quantize_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                          int64_t ldx, int trans, const float* scale_p,
                                                          uint8_t* __restrict__ Q, int64_t ldq,
                                                          uint8_t* __restrict__ S, int64_t Rp) {
    __shared__ float tile[64][65];
    const int64_t r0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
    const int t = threadIdx.x;
#pragma unroll
    for(int i = 0; i < 16; ++i) {
        const int idx = t + NT * i;
        const int a = idx / 64, b = idx % 64;  // a: slow, b: fast (contiguous in X)
        const int rr = trans ? b : a, kk = trans ? a : b;
        const int64_t r = r0 + rr, k = k0 + kk;
        float v = 0.0f;
        if(r < R && k < K) v = trans ? X[k * ldx + r] : X[r * ldx + k];
        tile[rr][kk] = v;
    }
    __syncthreads();
    const int rr = t / 4, kq = (t % 4) * 16;
    float v[16];
#pragma unroll
    for(int q = 0; q < 16; ++q) v[q] = tile[rr][kq + q];
    int e = 0;
    if constexpr(MX) {
        float amax = 0.0f;
#pragma unroll
        for(int q = 0; q < 16; ++q) amax = fmaxf(amax, fabsf(v[q]));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        e = mx_exponent(amax);
#pragma unroll
        for(int q = 0; q < 16; ++q) v[q] = ldexpf(v[q], -e);
        if((t & 1) == 0) S[(int64_t)blockIdx.x * Rp * 2 + (r0 + rr) * 2 + ((t >> 1) & 1)] = (uint8_t)(e + 127);
    } else {
        const float scale = *scale_p;
#pragma unroll
        for(int q = 0; q < 16; ++q) v[q] *= scale;
    }
    i32x4 out;
#pragma unroll
    for(int q = 0; q < 4; ++q) {
        int x = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(v[4 * q]), e4m3_clamp(v[4 * q + 1]), 0, false);
        x = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(v[4 * q + 2]), e4m3_clamp(v[4 * q + 3]), x, true);
        out[q] = x;
    }
    *reinterpret_cast<i32x4*>(Q + (r0 + rr) * ldq + k0 + kq) = out;
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

}  // namespace

extern "C" size_t pk_fp8_quantized_bytes(int64_t R, int64_t K, int64_t* ld) {
    if(R <= 0 || K <= 0) {
        if(ld) *ld = 0;
        return 0;
    }
    const int64_t l = round_up(K, QKPAD);
    if(ld) *ld = l;
    return (size_t)(round_up(R, kTileQ) * l);
}

extern "C" int pk_fp8_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans,
                                   const float* scale, uint8_t* Q, int64_t ldq, pk_stream_t stream) {
    if(R < 0 || K < 0) return pk::fail("pk_fp8_quantize_f32: negative size");
    if(R == 0 || K == 0) return PK_OK;
    if(!X || !scale || !Q) return pk::fail("pk_fp8_quantize_f32: NULL pointer");
    if(ldx < (trans ? R : K)) return pk::fail("pk_fp8_quantize_f32: ldx below the row length");
    if(ldq < round_up(K, QKPAD) || ldq % 16 || !pk::aligned16(Q))
        return pk::fail("pk_fp8_quantize_f32: ldq must be >= K rounded up to 128, a multiple of 16, "
                        "Q 16-byte aligned");
    const int64_t Rp = round_up(R, kTileQ), Kp = round_up(K, QKPAD);
    if(Rp / 64 > 65535 || Kp / 64 > INT32_MAX) return pk::fail("pk_fp8_quantize_f32: too large");
    fp8_quantize_kernel<false><<<dim3((unsigned)(Kp / 64), (unsigned)(Rp / 64)), NT, 0, pk::as_stream(stream)>>>(
        R, K, X, ldx, trans, scale, Q, ldq, nullptr, Rp);
    return pk::launch_status("pk_fp8_quantize_f32");
}

namespace {

// launch checks shared by both products; fills the shapes of p
int fp8q_shapes(const char* name, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, const void* A,
                const void* B, float* C, int64_t ldc, Fp8qParams& p) {
    if(M < 0 || N < 0 || K < 0) return pk::fail("%s: negative size", name);
    if(!C || (K > 0 && (!A || !B))) return pk::fail("%s: NULL pointer", name);
    if(ldc < N) return pk::fail("%s: ldc < N", name);
    const int64_t Kp = round_up(K > 0 ? K : 1, QKPAD), Mp = round_up(M, kTileQ), Np = round_up(N, kTileQ);
    if(K > 0 && (lda < Kp || ldb < Kp || lda % 16 || ldb % 16 || !pk::aligned16(A) || !pk::aligned16(B)))
        return pk::fail("%s: operands as the quantizer writes them: row strides >= K rounded up to 128, "
                        "multiples of 16, 16-byte aligned", name);
    if(Mp * lda > INT32_MAX || Np * ldb > INT32_MAX)
        return pk::fail("%s: an operand spans 2^31 bytes or more", name);
    if((Mp / kTileQ) * (Np / kTileQ) > INT32_MAX) return pk::fail("%s: too many tiles", name);
    p = Fp8qParams{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = C;
    p.M = M;
    p.N = N;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.nslices = K > 0 ? (int)(Kp / QB) : 0;
    p.tiles_m = (int)(Mp / kTileQ);
    p.tiles_n = (int)(Np / kTileQ);
    return PK_OK;
}

}  // namespace

extern "C" int pk_gemm_fp8q_f32(int64_t M, int64_t N, int64_t K, float alpha, const uint8_t* A,
                                int64_t lda, const uint8_t* B, int64_t ldb, const float* scales,
                                float beta, float* C, int64_t ldc, pk_stream_t stream) {
    if(M > 0 && N > 0 && !scales) return pk::fail("pk_gemm_fp8q_f32: NULL scales");
    Fp8qParams p;
    if(int st = fp8q_shapes("pk_gemm_fp8q_f32", M, N, K, lda, ldb, A, B, C, ldc, p)) return st;
    if(M == 0 || N == 0) return PK_OK;
    p.scales = scales;
    p.alpha = alpha;
    p.beta = beta;
    p.X = beta != 0.0f ? C : nullptr;
    p.ldx = ldc;
    gemm_fp8q_kernel<false><<<(unsigned)(p.tiles_m * p.tiles_n), NT, 0, pk::as_stream(stream)>>>(p);
    return pk::launch_status("pk_gemm_fp8q_f32");
}

// ---- MX: e4m3 values with an E8M0 scale per 32 k (OCP Microscaling MXFP8) -----
// An MX8 matrix of R rows and K values per row: Rp = R rounded up to 256,
// Kp = K rounded up to 128; Rp * Kp e4m3 bytes (row stride Kp), then the
// scales, Kp / 64 slices of Rp rows of 2 bytes.
extern "C" size_t pk_mx8_bytes(int64_t R, int64_t K) {
    if(R <= 0 || K <= 0) return 0;
    const int64_t Rp = round_up(R, kTileQ), Kp = round_up(K, QKPAD);
    return (size_t)(Rp * Kp + Rp * (Kp / 32));
}

extern "C" int pk_mx8_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, void* Q,
                                   pk_stream_t stream) {
    if(R < 0 || K < 0) return pk::fail("pk_mx8_quantize_f32: negative size");
    if(R == 0 || K == 0) return PK_OK;
    if(!X || !Q) return pk::fail("pk_mx8_quantize_f32: NULL pointer");
    if(ldx < (trans ? R : K)) return pk::fail("pk_mx8_quantize_f32: ldx below the row length");
    if(!pk::aligned16(Q)) return pk::fail("pk_mx8_quantize_f32: Q must be 16-byte aligned");
    const int64_t Rp = round_up(R, kTileQ), Kp = round_up(K, QKPAD);
    if(Rp / 64 > 65535 || Kp / 64 > INT32_MAX) return pk::fail("pk_mx8_quantize_f32: too large");
    uint8_t* q = static_cast<uint8_t*>(Q);
    fp8_quantize_kernel<true><<<dim3((unsigned)(Kp / 64), (unsigned)(Rp / 64)), NT, 0, pk::as_stream(stream)>>>(
        R, K, X, ldx, trans, nullptr, q, Kp, q + Rp * Kp, Rp);
    return pk::launch_status("pk_mx8_quantize_f32");
}

extern "C" int pk_gemm_mx8_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                               float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                               pk_stream_t stream) {
    const int64_t Kp = round_up(K > 0 ? K : 1, QKPAD), Mp = round_up(M, kTileQ), Np = round_up(N, kTileQ);
    Fp8qParams p;
    if(int st = fp8q_shapes("pk_gemm_mx8_f32", M, N, K, Kp, Kp, A, B, C, ldc, p)) return st;
    if(M == 0 || N == 0) return PK_OK;
    if(beta != 0.0f && !X) return pk::fail("pk_gemm_mx8_f32: beta != 0 needs X");
    if(beta != 0.0f && ldx != 0 && ldx < N) return pk::fail("pk_gemm_mx8_f32: ldx < N");
    if(Mp * Kp / 32 > INT32_MAX || Np * Kp / 32 > INT32_MAX)
        return pk::fail("pk_gemm_mx8_f32: scales span 2^31 bytes or more");
    p.SA = static_cast<const uint8_t*>(A) + Mp * Kp;
    p.SB = static_cast<const uint8_t*>(B) + Np * Kp;
    p.sstride_a = 2 * Mp;
    p.sstride_b = 2 * Np;
    p.alpha = alpha;
    p.beta = beta;
    p.X = beta != 0.0f ? X : nullptr;
    p.ldx = ldx;
    gemm_fp8q_kernel<true><<<(unsigned)(p.tiles_m * p.tiles_n), NT, 0, pk::as_stream(stream)>>>(p);
    return pk::launch_status("pk_gemm_mx8_f32");
}
