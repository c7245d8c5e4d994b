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

#include <algorithm>

#include "pk_common.h"

namespace {

constexpr int NT = 256;
constexpr int QB = 64;                        // k bytes per slice = bytes of an LDS row
constexpr int QKPAD = 2 * QB;                 // K padding: an even number of slices
constexpr int QSTAGES = 4;
constexpr int QGROUP_M = 8;
constexpr int64_t kTileQ = 256;               // row padding of the quantized operands
constexpr int kMaxSplits = 16;

typedef __attribute__((address_space(3))) void lds_ptr_t;
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// operand formats of the product kernel: e4m3 with per-tensor scales, MX8
// (e4m3 with an E8M0 scale per 32 values), bf16 (2 bytes a value, no scales),
// split bf16 (a value as hi = bf16(x) and lo = bf16(x - hi): 4 bytes a value)
enum QKind { kQE4M3 = 0, kQMX8 = 1, kQBF16 = 2, kQBF16X3 = 3 };

struct Fp8qParams {
    const uint8_t *A, *B;
    const uint8_t *SA, *SB;  // MX: E8M0 block scales, [slice][rows][2]
    int64_t sstride_a, sstride_b;  // MX: bytes of one slice's scales (2 * padded rows)
    float* C;
    const float* X;       // C = alpha * product (+ beta * X); X == C accumulates
    const float* scales;  // per-tensor mode: device sA, sB (NULL: 1, 1)
    float* P;             // K split: partial planes [splits][M][N], summed by fp8q_reduce_kernel
    int64_t M, N, lda, ldb, ldc, ldx;
    int nslices;          // slices of one split (even); the last split takes what remains
    int total_slices;     // slices of the whole K (even)
    int splits;
    float alpha, beta;
    int tiles_m, tiles_n;
};

__host__ __device__ inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

__device__ __forceinline__ int slot_of(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

// the load instructions of an operand tile of ROWS rows: lane l of
// instruction n fills LDS slot l % 4 of row 16n + l / 4 (n = w + 4i), from
// the chunk that belongs there
template <int ROWS>
struct QLoad {
    static constexpr int N = ROWS / 64;  // per wave
    int voff[N];
    __device__ __forceinline__ QLoad(int64_t ld, int w, int l) {
#pragma unroll
        for(int i = 0; i < N; ++i) {
            const int r = 16 * (w + 4 * i) + l / 4;
            voff[i] = r * (int)ld + 16 * slot_of(r, l % 4);  // slot_of is its own inverse
        }
    }
    __device__ __forceinline__ void issue_one(int i, __amdgpu_buffer_rsrc_t rs, int soff, uint8_t* tile,
                                              int w) const {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t*)(tile + 1024 * (w + 4 * i)), 16, voff[i],
                                                 soff, 0, 0);
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

// one 64-byte slice of a lane's operand rows (a, b: its 32 bytes, chunks
// lane/32 and lane/32 + 2 of the slice) into c.  fp8: one 32x32x64 MFMA.
// bf16: the slice holds 32 values; chunk lane/32 is values 8(lane/32)..+7,
// the lane's share of k 0-15 on the 32x32x16 bf16 MFMA, and chunk lane/32 + 2
// its share of k 16-31 -- two MFMAs, k 0-15 first, each taking as many
// cycles as half the fp8 one.  Split bf16: the slice holds 16 values, their
// hi parts in chunks 0-1 and lo parts in chunks 2-3, so chunk lane/32 is the
// lane's hi share of k 0-15 and chunk lane/32 + 2 its lo share -- three
// MFMAs, hi.hi + hi.lo + lo.hi (lo.lo is below 2^-16 of the product), the
// order pk_gemm_bf16x3_f32 takes them in.
template <int KIND>
__device__ __forceinline__ f32x16 slice_mma(const i32x8& a, const i32x8& b, const f32x16& c, int sa, int sb) {
    if constexpr(KIND == kQBF16X3) {
        const i32x4 ah = __builtin_shufflevector(a, a, 0, 1, 2, 3), al = __builtin_shufflevector(a, a, 4, 5, 6, 7);
        const i32x4 bh = __builtin_shufflevector(b, b, 0, 1, 2, 3), bl = __builtin_shufflevector(b, b, 4, 5, 6, 7);
        f32x16 r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah),
                                                          __builtin_bit_cast(bf16x8, bh), c, 0, 0, 0);
        r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah), __builtin_bit_cast(bf16x8, bl),
                                                    r, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, al),
                                                      __builtin_bit_cast(bf16x8, bh), r, 0, 0, 0);
    } else if constexpr(KIND == kQBF16) {
        // the halves by shufflevector: bit-casting the .hi swizzle of an
        // 8-int vector compiled to its .lo here (both MFMAs read k 0-15)
        const i32x4 al = __builtin_shufflevector(a, a, 0, 1, 2, 3), ah = __builtin_shufflevector(a, a, 4, 5, 6, 7);
        const i32x4 bl = __builtin_shufflevector(b, b, 0, 1, 2, 3), bh = __builtin_shufflevector(b, b, 4, 5, 6, 7);
        const f32x16 r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, al),
                                                                __builtin_bit_cast(bf16x8, bl), c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah),
                                                      __builtin_bit_cast(bf16x8, bh), r, 0, 0, 0);
    } else {
        return mfma_fp8(a, b, c, sa, sb);
    }
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

// C tile TM x TN = (64 WM) x (64 WN): 2 x 2 waves of WM x WN blocks of 32 x 32.
// MX: operands carry E8M0 scales per 32 k (one per lane's 32 bytes of an
// MFMA operand), streamed into LDS beside the bytes and handed to the MFMA;
// otherwise the scales are 2^0 and the tensor scales divide in the epilogue.
// With splits > 1, workgroup b runs split b / tiles (nslices slices from
// slice split * nslices) and writes its raw sums to plane `split` of P.
template <int KIND, int WM, int WN>
__global__ __launch_bounds__(NT, WM * WN <= 4 ? 2 : 1) void gemm_fp8q_kernel(Fp8qParams p) {
    constexpr bool MX = KIND == kQMX8;
    constexpr int TM = 64 * WM, TN = 64 * WN;
    static_assert(TM % 128 == 0 && TN % 128 == 0, "scale loads cover 128 rows each");
    constexpr int SCB = MX ? (TM + TN) * 2 : 0;  // scale bytes of a stage: [A rows | B rows][2]
    constexpr int NSC = SCB / 256;                // scale load instructions of a stage (4 bytes a lane)
    constexpr int STAGE = (TM + TN) * QB + SCB;
    constexpr int OB = TM * QB, OS = (TM + TN) * QB;  // B's bytes and the scales in a stage
    __shared__ __attribute__((aligned(16))) uint8_t lds[QSTAGES][STAGE];

    const int ntiles = p.tiles_m * p.tiles_n, total = ntiles * p.splits;
    int bid = blockIdx.x;
    if((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    const int split = bid / ntiles;
    bid -= split * ntiles;
    const int group_span = QGROUP_M * p.tiles_n;
    const int first_m = (bid / group_span) * QGROUP_M;
    const int gm = min(p.tiles_m - first_m, QGROUP_M);
    const int local = bid % group_span;
    const int64_t row0 = (int64_t)(first_m + local % gm) * TM, col0 = (int64_t)(local / gm) * TN;

    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lr = l & 31, lh = l >> 5;
    const int wm = w >> 1, wn = w & 1;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.A), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.B), (short)0, 0x7fffffff, 0x00020000);
    const QLoad<TM> la(p.lda, w, l);
    const QLoad<TN> lb(p.ldb, w, l);
    const int sa = (int)(row0 * p.lda), sb = (int)(col0 * p.ldb);
    // this split's slices: nslices, or what remains for the last split (even,
    // at least 2: the plan never leaves an empty split)
    const int s0 = split * p.nslices, ns = min(p.nslices, p.total_slices - s0);
    // MX scales: wave w fetches 128 rows (256 bytes, 4 a lane) of the stage's
    // [A | B] scale rows: block min(w, NSC - 1), a repeat where there are fewer
    // blocks than waves (the same bytes to the same place)
    const int scb = min(w, (NSC > 0 ? NSC : 1) - 1);
    const bool sc_b = scb * 128 >= TM;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(sc_b ? p.SB : p.SA), (short)0, 0x7fffffff, 0x00020000);
    const int sc0 = (int)((sc_b ? col0 + scb * 128 - TM : row0 + scb * 128) * 2);
    const int sc_stride = (int)(sc_b ? p.sstride_b : p.sstride_a);
    auto issue_scales = [&](int s, int st) {
        if constexpr(MX)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t*)(&lds[st][OS + scb * 256]), 4, 4 * l,
                                                     sc0 + (s0 + min(s, ns - 1)) * sc_stride, 0, 0);
    };
    // slice s of the split into stage s % QSTAGES; past its last slice the
    // last one is fetched again (into a stage nobody reads), which keeps every
    // iteration's count of outstanding loads the same
    auto issue = [&](int s) {
        const int st = s % QSTAGES, k = (s0 + min(s, ns - 1)) * QB;
#pragma unroll
        for(int i = 0; i < WM; ++i) la.issue_one(i, ra, sa + k, &lds[st][0], w);
#pragma unroll
        for(int i = 0; i < WN; ++i) lb.issue_one(i, rb, sb + k, &lds[st][OB], w);
        issue_scales(s, st);
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for(int i = 0; i < WM; ++i)
#pragma unroll
        for(int j = 0; j < WN; ++j)
#pragma unroll
            for(int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // LDS rows of this lane's operand blocks within a stage
    auto a_row = [&](int i) { return wm * (TM / 2) + 32 * i + lr; };
    auto b_row = [&](int j) { return wn * (TN / 2) + 32 * j + lr; };
    // this lane's scale of A block i / B block j in stage st
    auto scale_a = [&](int st, int i) -> int {
        if constexpr(MX) return lds[st][OS + a_row(i) * 2 + lh];
        else return 127;
    };
    auto scale_b = [&](int st, int j) -> int {
        if constexpr(MX) return lds[st][OS + (TM + b_row(j)) * 2 + lh];
        else return 127;
    };
    auto read = [&](int s, i32x8 (&fa)[WM], i32x8 (&fb)[WN], int (&ca)[WM], int (&cb)[WN]) {
        const int st = s % QSTAGES;
#pragma unroll
        for(int i = 0; i < WM; ++i) {
            fa[i] = frag(&lds[st][0], a_row(i), lh);
            ca[i] = scale_a(st, i);
        }
#pragma unroll
        for(int j = 0; j < WN; ++j) {
            fb[j] = frag(&lds[st][OB], b_row(j), lh);
            cb[j] = scale_b(st, j);
        }
    };
    constexpr int NG = WM * WN;                 // MFMAs of a slice, per wave
    constexpr int NR = 2 * (WM + WN);           // 128-bit fragment reads of a slice
    constexpr int NS = MX ? WM + WN : 0;        // scale reads of a slice
    constexpr int PER = WM + WN + (MX ? 1 : 0); // loads of a slice, per wave
    // slice s with its fragments in (fa, fb) and scales in (ca, cb): wait for
    // slice s+1's loads and every wave's reads of slice s, then NG groups, each
    // one MFMA of slice s and an even share of: the 128-bit LDS reads of slice
    // s+1's fragments into (ga, gb) (in the order the next slice's MFMAs use
    // them: A0, B0.., A1..), the loads refilling slice s's stage with slice
    // s+QSTAGES, and the reads of slice s+1's scales.  The scheduling barriers
    // keep that order: left alone, the compiler moves the next slice's wait
    // above the last MFMAs.
    auto step = [&](int s, i32x8 (&fa)[WM], i32x8 (&fb)[WN], int (&ca)[WM], int (&cb)[WN], i32x8 (&ga)[WM],
                    i32x8 (&gb)[WN], int (&da)[WM], int (&db)[WN]) {
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_lds<(QSTAGES - 2) * PER>();
        barrier_keep_loads();
        const int nx = (s + 1) % QSTAGES, fill = s % QSTAGES;
        const int k = (s0 + min(s + QSTAGES, ns - 1)) * QB;
#pragma unroll
        for(int g = 0; g < NG; ++g) {
            const int i = g / WN, j = g % WN;
            acc[i][j] = slice_mma<KIND>(fa[i], fb[j], acc[i][j], ca[i], cb[j]);
#pragma unroll
            for(int r = g * NR / NG; r < (g + 1) * NR / NG; ++r) {
                // fragment r / 2 in the order A0, B0..B(WN-1), A1..A(WM-1); half r % 2
                const int f = r >> 1, h = r & 1;
                const bool is_a = f == 0 || f > WN;
                const int idx = f == 0 ? 0 : (f <= WN ? f - 1 : f - WN);
                if(is_a) {
                    const i32x4 v = frag_half(&lds[nx][0], a_row(idx), lh, h);
                    if(h) ga[idx].hi = v; else ga[idx].lo = v;
                } else {
                    const i32x4 v = frag_half(&lds[nx][OB], b_row(idx), lh, h);
                    if(h) gb[idx].hi = v; else gb[idx].lo = v;
                }
            }
#pragma unroll
            for(int q = g * PER / NG; q < (g + 1) * PER / NG; ++q) {
                if(q < WM)
                    la.issue_one(q, ra, sa + k, &lds[fill][0], w);
                else if(q < WM + WN)
                    lb.issue_one(q - WM, rb, sb + k, &lds[fill][OB], w);
                else
                    issue_scales(s + QSTAGES, fill);
            }
#pragma unroll
            for(int q = g * NS / NG; q < (g + 1) * NS / NG; ++q) {
                if(q < WM) da[q] = scale_a(nx, q); else db[q - WM] = scale_b(nx, q - WM);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if(ns > 0) {
#pragma unroll
        for(int s = 0; s < QSTAGES; ++s) issue(s);
        i32x8 a0[WM], b0[WN], a1[WM], b1[WN];
        // scales: MX reads them with every slice; otherwise they stay 2^0
        int ca0[WM], cb0[WN], ca1[WM], cb1[WN];
#pragma unroll
        for(int i = 0; i < WM; ++i) ca0[i] = ca1[i] = 127;
#pragma unroll
        for(int j = 0; j < WN; ++j) cb0[j] = cb1[j] = 127;
        wait_vm_lds<(QSTAGES - 1) * PER>();
        barrier_keep_loads();
        read(0, a0, b0, ca0, cb0);
        for(int s = 0; s < ns; s += 2) {  // ns is even: K is padded to 128 bytes, splits take pairs
            step(s, a0, b0, ca0, cb0, a1, b1, ca1, cb1);
            step(s + 1, a1, b1, ca1, cb1, a0, b0, ca0, cb0);
        }
        wait_vm_lds<0>();  // no load may land in LDS after the workgroup ends
    }

    const int64_t rw = row0 + wm * (TM / 2) + 4 * lh, cw = col0 + wn * (TN / 2) + lr;
    if(p.splits > 1) {  // raw sums into this split's plane of P (row stride N)
        float* P = p.P + (int64_t)split * p.M * p.N;
#pragma unroll
        for(int i = 0; i < WM; ++i)
#pragma unroll
            for(int j = 0; j < WN; ++j) {
                const int64_t col = cw + 32 * j;
#pragma unroll
                for(int r = 0; r < 16; ++r) {
                    const int64_t row = rw + 32 * i + 8 * (r >> 2) + (r & 3);
                    if(row < p.M && col < p.N) P[row * p.N + col] = acc[i][j][r];
                }
            }
        return;
    }
    const float scale = MX || !p.scales ? p.alpha : p.alpha / (p.scales[0] * p.scales[1]);
    const bool full = row0 + TM <= p.M && col0 + TN <= p.N;
    if(full && !p.X) {
#pragma unroll
        for(int i = 0; i < WM; ++i)
#pragma unroll
            for(int j = 0; j < WN; ++j) {
                float* c = p.C + (rw + 32 * i) * p.ldc + cw + 32 * j;
#pragma unroll
                for(int r = 0; r < 16; ++r) c[(8 * (r >> 2) + (r & 3)) * p.ldc] = scale * acc[i][j][r];
            }
        return;
    }
#pragma unroll
    for(int i = 0; i < WM; ++i)
#pragma unroll
        for(int j = 0; j < WN; ++j) {
            const int64_t col = cw + 32 * j;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                const int64_t row = rw + 32 * i + 8 * (r >> 2) + (r & 3);
                if(row >= p.M || col >= p.N) continue;
                float v = scale * acc[i][j][r];
                if(p.X) v += p.beta * p.X[row * p.ldx + col];
                p.C[row * p.ldc + col] = v;
            }
        }
}

// every launch shape, instantiated here so that each gets its host stub
#define PK_FP8Q_SHAPES(KIND)                                              \
    template __global__ void gemm_fp8q_kernel<KIND, 4, 4>(Fp8qParams); \
    template __global__ void gemm_fp8q_kernel<KIND, 4, 2>(Fp8qParams); \
    template __global__ void gemm_fp8q_kernel<KIND, 2, 4>(Fp8qParams); \
    template __global__ void gemm_fp8q_kernel<KIND, 2, 2>(Fp8qParams);
PK_FP8Q_SHAPES(kQE4M3)
PK_FP8Q_SHAPES(kQMX8)
PK_FP8Q_SHAPES(kQBF16)
PK_FP8Q_SHAPES(kQBF16X3)
#undef PK_FP8Q_SHAPES

// C = alpha * (P[0] + P[1] + ... in plane order) + beta * X: a split product's
// planes summed in a fixed order, so the result does not depend on timing
__global__ __launch_bounds__(NT) void fp8q_reduce_kernel(int64_t M, int64_t N, int splits, const float* __restrict__ P,
                                                         float alpha, float beta, const float* X, int64_t ldx,
                                                         float* C, int64_t ldc) {
    const int64_t plane = M * N;
    for(int64_t e = (int64_t)blockIdx.x * NT + threadIdx.x; e < plane; e += (int64_t)gridDim.x * NT) {
        const int64_t row = e / N, col = e - row * N;
        float v = P[e];
        for(int s = 1; s < splits; ++s) v += P[s * plane + e];
        v *= alpha;
        if(X) v += beta * X[row * ldx + col];
        C[row * ldc + col] = v;
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

// four e4m3 bytes of four values (clamped to +-448, nearest even)
__device__ __forceinline__ int e4m3x4(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(a), e4m3_clamp(b), 0, false);
    return __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(c), e4m3_clamp(d), lo, true);
}

// four consecutive values of row `row` of a row-major [rows, cols] matrix
// from column c; zero outside it.  vec: row starts 16-byte aligned.
__device__ __forceinline__ f32x4 load4(const float* __restrict__ X, int64_t ld, int64_t rows, int64_t cols,
                                      int64_t row, int64_t c, bool vec) {
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if(row >= rows || c >= cols) return v;
    const float* p = X + row * ld + c;
    if(vec && c + 4 <= cols) return *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for(int q = 0; q < 4; ++q)
        if(c + q < cols) v[q] = p[q];
    return v;
}

// the scale byte of MX block b (32 values from k = 32b) of row r, for the
// [slice][row][2] layout
__device__ __forceinline__ uint8_t* scale_slot(uint8_t* S, int64_t Rp, int64_t r, int64_t b) {
    return S + (b >> 1) * Rp * 2 + r * 2 + (b & 1);
}

// op(X) = X (rows contiguous): a wave covers 256 values of a row, 4 per
// lane (one 1 KB load), 8 lanes per MX block (the block's largest magnitude
// by 3 exchanges), 4 rows per wave in flight; a block of 4 waves covers 16
// rows.  Writes every byte of [Rp, Kp] and every scale.
template <bool MX>
__global__ __launch_bounds__(NT) void quantize_rows_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                           int64_t ldx, bool vec, const float* scale_p,
                                                           uint8_t* __restrict__ Q, int64_t ldq, int64_t Kp,
                                                           uint8_t* __restrict__ S, int64_t Rp) {
    constexpr int RW = 4;  // rows per wave
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int64_t k = (int64_t)blockIdx.x * 256 + 4 * l;
    const int64_t r0 = ((int64_t)blockIdx.y * 4 + w) * RW;
    f32x4 v[RW];
#pragma unroll
    for(int i = 0; i < RW; ++i) v[i] = load4(X, ldx, R, K, r0 + i, k, vec);
    const float tscale = MX ? 1.0f : *scale_p;
#pragma unroll
    for(int i = 0; i < RW; ++i) {
        const int64_t r = r0 + i;
        int e = 0;
        if constexpr(MX) {
            float amax = fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3])));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
            e = mx_exponent(amax);
        }
        if(r >= Rp || k >= Kp) continue;
        int q;
        if constexpr(MX)
            q = e4m3x4(ldexpf(v[i][0], -e), ldexpf(v[i][1], -e), ldexpf(v[i][2], -e), ldexpf(v[i][3], -e));
        else
            q = e4m3x4(v[i][0] * tscale, v[i][1] * tscale, v[i][2] * tscale, v[i][3] * tscale);
        *reinterpret_cast<int*>(Q + r * ldq + k) = q;
        if constexpr(MX)
            if((l & 7) == 0) *scale_slot(S, Rp, r, k >> 5) = (uint8_t)(e + 127);
    }
}

// op(X) = X^T (X [K, R], rows of op(X) are X's columns): a block stages a
// 64 (k) x 128 (r) tile through LDS -- read as 16-byte pieces along X's
// rows, written transposed -- and then each thread takes one MX block: 32
// consecutive k of one r (tile row), 32 output bytes and its scale.
template <bool MX>
__global__ __launch_bounds__(NT) void quantize_cols_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                           int64_t ldx, bool vec, const float* scale_p,
                                                           uint8_t* __restrict__ Q, int64_t ldq,
                                                           uint8_t* __restrict__ S, int64_t Rp) {
    __shared__ float tile[128][65];
    const int t = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 128;
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const int idx = t + NT * i;
        const int kk = idx >> 5, rq = (idx & 31) * 4;
        const f32x4 v = load4(X, ldx, K, R, k0 + kk, r0 + rq, vec);
#pragma unroll
        for(int c = 0; c < 4; ++c) tile[rq + c][kk] = v[c];
    }
    __syncthreads();
    const int rr = t >> 1, half = t & 1;
    const int64_t r = r0 + rr;
    if(r >= Rp) return;
    float v[32];
#pragma unroll
    for(int q = 0; q < 32; ++q) v[q] = tile[rr][32 * half + q];
    int e = 0;
    float sc = 1.0f;
    if constexpr(MX) {
        float amax = 0.0f;
#pragma unroll
        for(int q = 0; q < 32; ++q) amax = fmaxf(amax, fabsf(v[q]));
        e = mx_exponent(amax);
        *scale_slot(S, Rp, r, (k0 >> 5) + half) = (uint8_t)(e + 127);
    } else {
        sc = *scale_p;
    }
    i32x4 o[2];
#pragma unroll
    for(int q = 0; q < 8; ++q) {
        const float* p = &v[4 * q];
        o[q >> 2][q & 3] = MX ? e4m3x4(ldexpf(p[0], -e), ldexpf(p[1], -e), ldexpf(p[2], -e), ldexpf(p[3], -e))
                              : e4m3x4(p[0] * sc, p[1] * sc, p[2] * sc, p[3] * sc);
    }
    i32x4* dst = reinterpret_cast<i32x4*>(Q + r * ldq + k0 + 32 * half);
    dst[0] = o[0];
    dst[1] = o[1];
}

// Both MX8 casts of one row-major matrix X [M, N] from one read of it: QR =
// X as [M, N] (blocks along N) and QT = X^T as [N, M] (blocks along M), equal
// byte for byte to two calls of pk_mx8_quantize_f32.  A block stages a 64 (M)
// x 128 (N) tile through LDS as quantize_cols_kernel does; each thread then
// takes one MX block of QT (32 rows of X at one column) and one of QR (32
// columns of one row of X), the latter read across the LDS tile.  The grid
// covers the larger padded extents; a tile writes only the parts of QR and QT
// inside their own padded shapes.
__global__ __launch_bounds__(NT) void quantize_dual_kernel(int64_t M, int64_t N, const float* __restrict__ X,
                                                           int64_t ldx, bool vec, uint8_t* __restrict__ QR,
                                                           uint8_t* __restrict__ QT) {
    __shared__ float tile[128][65];
    const int t = threadIdx.x;
    const int64_t m0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 128;
    const int64_t MpR = round_up(M, kTileQ), NpR = round_up(N, QKPAD);  // QR [MpR, NpR]
    const int64_t NpT = round_up(N, kTileQ), MpT = round_up(M, QKPAD);  // QT [NpT, MpT]
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const int idx = t + NT * i;
        const int mm = idx >> 5, nq = (idx & 31) * 4;
        const f32x4 v = load4(X, ldx, M, N, m0 + mm, n0 + nq, vec);
#pragma unroll
        for(int c = 0; c < 4; ++c) tile[nq + c][mm] = v[c];
    }
    __syncthreads();
    // QT: row n0 + t/2 of X^T, k = m0 + 32*(t%2) .. +31
    {
        const int rr = t >> 1, half = t & 1;
        const int64_t r = n0 + rr;
        if(r < NpT && m0 < MpT) {
            float v[32];
#pragma unroll
            for(int q = 0; q < 32; ++q) v[q] = tile[rr][32 * half + q];
            float amax = 0.0f;
#pragma unroll
            for(int q = 0; q < 32; ++q) amax = fmaxf(amax, fabsf(v[q]));
            const int e = mx_exponent(amax);
            *scale_slot(QT + NpT * MpT, NpT, r, (m0 >> 5) + half) = (uint8_t)(e + 127);
            i32x4 o[2];
#pragma unroll
            for(int q = 0; q < 8; ++q) {
                const float* p = &v[4 * q];
                o[q >> 2][q & 3] = e4m3x4(ldexpf(p[0], -e), ldexpf(p[1], -e), ldexpf(p[2], -e), ldexpf(p[3], -e));
            }
            i32x4* dst = reinterpret_cast<i32x4*>(QT + r * MpT + m0 + 32 * half);
            dst[0] = o[0];
            dst[1] = o[1];
        }
    }
    // QR: row m0 + t/4 of X, k = n0 + 32*(t%4) .. +31
    {
        const int rr = t >> 2, blk = t & 3;
        const int64_t r = m0 + rr, k0 = n0 + 32 * blk;
        if(r < MpR && k0 < NpR) {
            float v[32];
#pragma unroll
            for(int q = 0; q < 32; ++q) v[q] = tile[32 * blk + q][rr];
            float amax = 0.0f;
#pragma unroll
            for(int q = 0; q < 32; ++q) amax = fmaxf(amax, fabsf(v[q]));
            const int e = mx_exponent(amax);
            *scale_slot(QR + MpR * NpR, MpR, r, k0 >> 5) = (uint8_t)(e + 127);
            i32x4 o[2];
#pragma unroll
            for(int q = 0; q < 8; ++q) {
                const float* p = &v[4 * q];
                o[q >> 2][q & 3] = e4m3x4(ldexpf(p[0], -e), ldexpf(p[1], -e), ldexpf(p[2], -e), ldexpf(p[3], -e));
            }
            i32x4* dst = reinterpret_cast<i32x4*>(QR + r * NpR + k0);
            dst[0] = o[0];
            dst[1] = o[1];
        }
    }
}

// ---- bf16 operands: fp32 rounded to nearest even, 2 bytes a value ----------
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}
__device__ __forceinline__ uint2 bf16_quad(f32x4 v) {
    return make_uint2(bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3]));
}
// 32 consecutive values as 64 bytes (four 16-byte stores)
__device__ __forceinline__ void bf16_store32(uint8_t* __restrict__ dst, const float (&v)[32]) {
#pragma unroll
    for(int q = 0; q < 4; ++q) {
        i32x4 o;
#pragma unroll
        for(int e = 0; e < 4; ++e) o[e] = (int)bf16_pair(v[8 * q + 2 * e], v[8 * q + 2 * e + 1]);
        reinterpret_cast<i32x4*>(dst)[q] = o;
    }
}

// op(X) = X: as quantize_rows_kernel, 4 values (8 bytes) a lane, 4 rows a
// wave; writes every value of [Rp, Kv] (Kv: K padded to 64 values)
__global__ __launch_bounds__(NT) void bf16_rows_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                       int64_t ldx, bool vec, uint8_t* __restrict__ Q,
                                                       int64_t ldq, int64_t Kv, int64_t Rp) {
    constexpr int RW = 4;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int64_t k = (int64_t)blockIdx.x * 256 + 4 * l;
    const int64_t r0 = ((int64_t)blockIdx.y * 4 + w) * RW;
    f32x4 v[RW];
#pragma unroll
    for(int i = 0; i < RW; ++i) v[i] = load4(X, ldx, R, K, r0 + i, k, vec);
#pragma unroll
    for(int i = 0; i < RW; ++i) {
        const int64_t r = r0 + i;
        if(r >= Rp || k >= Kv) continue;
        *reinterpret_cast<uint2*>(Q + r * ldq + 2 * k) = bf16_quad(v[i]);
    }
}

// op(X) = X^T (X [K, R]): a 64 (k) x 128 (r) tile through LDS as in
// quantize_cols_kernel, then 32 consecutive k of one r per thread
__global__ __launch_bounds__(NT) void bf16_cols_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                       int64_t ldx, bool vec, uint8_t* __restrict__ Q,
                                                       int64_t ldq, int64_t Rp) {
    __shared__ float tile[128][65];
    const int t = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 128;
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const int idx = t + NT * i;
        const int kk = idx >> 5, rq = (idx & 31) * 4;
        const f32x4 v = load4(X, ldx, K, R, k0 + kk, r0 + rq, vec);
#pragma unroll
        for(int c = 0; c < 4; ++c) tile[rq + c][kk] = v[c];
    }
    __syncthreads();
    const int rr = t >> 1, half = t & 1;
    const int64_t r = r0 + rr;
    if(r >= Rp) return;
    float v[32];
#pragma unroll
    for(int q = 0; q < 32; ++q) v[q] = tile[rr][32 * half + q];
    bf16_store32(Q + r * ldq + 2 * (k0 + 32 * half), v);
}

// Both bf16 casts of one row-major X [M, N] from one read, as
// quantize_dual_kernel: QR = X [MpR, NvR], QT = X^T [NpT, MvT]
__global__ __launch_bounds__(NT) void bf16_dual_kernel(int64_t M, int64_t N, const float* __restrict__ X,
                                                       int64_t ldx, bool vec, uint8_t* __restrict__ QR,
                                                       uint8_t* __restrict__ QT) {
    __shared__ float tile[128][65];
    const int t = threadIdx.x;
    const int64_t m0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 128;
    const int64_t MpR = round_up(M, kTileQ), NvR = round_up(N, QB);  // QR rows, values a row
    const int64_t NpT = round_up(N, kTileQ), MvT = round_up(M, QB);  // QT rows, values a row
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const int idx = t + NT * i;
        const int mm = idx >> 5, nq = (idx & 31) * 4;
        const f32x4 v = load4(X, ldx, M, N, m0 + mm, n0 + nq, vec);
#pragma unroll
        for(int c = 0; c < 4; ++c) tile[nq + c][mm] = v[c];
    }
    __syncthreads();
    {  // QT: row n0 + t/2, values m0 + 32*(t%2) .. +31
        const int rr = t >> 1, half = t & 1;
        const int64_t r = n0 + rr;
        if(r < NpT && m0 < MvT) {
            float v[32];
#pragma unroll
            for(int q = 0; q < 32; ++q) v[q] = tile[rr][32 * half + q];
            bf16_store32(QT + r * 2 * MvT + 2 * (m0 + 32 * half), v);
        }
    }
    {  // QR: row m0 + t/4, values n0 + 32*(t%4) .. +31
        const int rr = t >> 2, blk = t & 3;
        const int64_t r = m0 + rr, k0 = n0 + 32 * blk;
        if(r < MpR && k0 < NvR) {
            float v[32];
#pragma unroll
            for(int q = 0; q < 32; ++q) v[q] = tile[32 * blk + q][rr];
            bf16_store32(QR + r * 2 * NvR + 2 * k0, v);
        }
    }
}

// ---- split-bf16 operands: hi = bf16(x), lo = bf16(x - hi), nearest even ----
// A row holds its values in groups of 16: the group's 16 hi parts (32 bytes),
// then its 16 lo parts, so a 64-byte slice row is one group
__device__ __forceinline__ uint32_t split_pair(float a, float b, uint32_t& lo) {
    const __bf16 ha = (__bf16)a, hb = (__bf16)b;
    lo = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(a - (float)ha)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(b - (float)hb)) << 16);
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}
// one group (16 consecutive values) as its 64 bytes
__device__ __forceinline__ void split_store16(uint8_t* __restrict__ dst, const float* v) {
    i32x4 h[2], l[2];
#pragma unroll
    for(int q = 0; q < 8; ++q) {
        uint32_t lo;
        h[q >> 2][q & 3] = (int)split_pair(v[2 * q], v[2 * q + 1], lo);
        l[q >> 2][q & 3] = (int)lo;
    }
    i32x4* d = reinterpret_cast<i32x4*>(dst);
    d[0] = h[0];
    d[1] = h[1];
    d[2] = l[0];
    d[3] = l[1];
}

// op(X) = X: as bf16_rows_kernel, 4 values a lane (8 bytes of hi and 8 of
// lo in their group), 4 rows a wave; writes every value of [Rp, Kv]
__global__ __launch_bounds__(NT) void split_rows_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                        int64_t ldx, bool vec, uint8_t* __restrict__ Q,
                                                        int64_t ldq, int64_t Kv, int64_t Rp) {
    constexpr int RW = 4;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int64_t k = (int64_t)blockIdx.x * 256 + 4 * l;
    const int64_t r0 = ((int64_t)blockIdx.y * 4 + w) * RW;
    f32x4 v[RW];
#pragma unroll
    for(int i = 0; i < RW; ++i) v[i] = load4(X, ldx, R, K, r0 + i, k, vec);
    const int64_t at = 64 * (k >> 4) + 2 * (k & 15);
#pragma unroll
    for(int i = 0; i < RW; ++i) {
        const int64_t r = r0 + i;
        if(r >= Rp || k >= Kv) continue;
        uint32_t l0, l1;
        const uint2 hi = make_uint2(split_pair(v[i][0], v[i][1], l0), split_pair(v[i][2], v[i][3], l1));
        uint8_t* row = Q + r * ldq;
        *reinterpret_cast<uint2*>(row + at) = hi;
        *reinterpret_cast<uint2*>(row + at + 32) = make_uint2(l0, l1);
    }
}

// op(X) = X^T (X [K, R]): a 64 (k) x 128 (r) tile through LDS as in
// bf16_cols_kernel, then two groups (32 consecutive k) of one r per thread
__global__ __launch_bounds__(NT) void split_cols_kernel(int64_t R, int64_t K, const float* __restrict__ X,
                                                        int64_t ldx, bool vec, uint8_t* __restrict__ Q,
                                                        int64_t ldq, int64_t Kv, int64_t Rp) {
    __shared__ float tile[128][65];
    const int t = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 128;
#pragma unroll
    for(int i = 0; i < 8; ++i) {
        const int idx = t + NT * i;
        const int kk = idx >> 5, rq = (idx & 31) * 4;
        const f32x4 v = load4(X, ldx, K, R, k0 + kk, r0 + rq, vec);
#pragma unroll
        for(int c = 0; c < 4; ++c) tile[rq + c][kk] = v[c];
    }
    __syncthreads();
    const int rr = t >> 1, half = t & 1;
    const int64_t r = r0 + rr, kh = k0 + 32 * half;
    if(r >= Rp || kh >= Kv) return;  // Kv is a multiple of 32: a half is all in or all out
    float v[32];
#pragma unroll
    for(int q = 0; q < 32; ++q) v[q] = tile[rr][32 * half + q];
    uint8_t* dst = Q + r * ldq + 4 * kh;
    split_store16(dst, v);
    split_store16(dst + 64, v + 16);
}

// launch: every byte of [Rp, Kp] (row stride ldq) and, MX, every scale
template <bool MX>
void launch_quantize(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, const float* scale,
                     uint8_t* Q, int64_t ldq, uint8_t* S, hipStream_t st) {
    const int64_t Rp = round_up(R, kTileQ), Kp = round_up(K, QKPAD);
    const bool vec = ldx % 4 == 0 && pk::aligned16(X);
    if(trans)
        quantize_cols_kernel<MX><<<dim3((unsigned)(Kp / 64), (unsigned)(Rp / 128)), NT, 0, st>>>(
            R, K, X, ldx, vec, scale, Q, ldq, S, Rp);
    else
        quantize_rows_kernel<MX><<<dim3((unsigned)((Kp + 255) / 256), (unsigned)(Rp / 16)), NT, 0, st>>>(
            R, K, X, ldx, vec, scale, Q, ldq, Kp, S, Rp);
}

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
    (void)Kp;
    launch_quantize<false>(R, K, X, ldx, trans, scale, Q, ldq, nullptr, pk::as_stream(stream));
    return pk::launch_status("pk_fp8_quantize_f32");
}

namespace {

// A launch plan: the tile (WM x WN blocks a wave) and the K split, from a
// timing model fitted (least squares in log time) to graph-replayed launches
// of every tile and split on MI355X over the products of a transformer step
// and square products: each CU runs its share of the workgroups' slices at
// the tile's cost per slice (two 128 x 128 workgroups share a CU at 0.8 of
// the cost each), plus a fixed cost per round of workgroups, plus C's bytes
// to HBM; a split adds its partial planes and the reduction launch.  On those
// products the plan's pick ran within 13 % of the best tile and split.
struct MxPlan {
    int wm, wn, splits, per;  // per: slices of one split
};

constexpr int64_t kCUs = 256;  // MI355X

MxPlan mx8_plan(int64_t M, int64_t N, int64_t K, bool allow_split) {
    const int64_t ns = round_up(K > 0 ? K : 1, QKPAD) / QB;
    struct Cand {
        int wm, wn, slots;  // slots: workgroups a CU holds
        double slice_us;    // per slice of one workgroup
    };
    const Cand cands[] = {{4, 4, 1, 0.80}, {4, 2, 1, 0.45}, {2, 4, 1, 0.45}, {2, 2, 2, 0.35}};
    const double hbm = 6.0e12, round_us = 1.0, launch_us = 6.0, shared = 0.8;
    MxPlan best{4, 4, 1, (int)ns};
    double best_t = 1e30;
    for(const Cand& c : cands) {
        const int64_t tiles = ((M + 64 * c.wm - 1) / (64 * c.wm)) * ((N + 64 * c.wn - 1) / (64 * c.wn));
        for(int S = 1; S <= (allow_split ? kMaxSplits : 1); ++S) {
            const int64_t per = round_up((ns + S - 1) / S, 2);
            const int64_t splits = (ns + per - 1) / per;
            if(splits != S || (S > 1 && per < 4)) continue;
            const int64_t wgs = tiles * splits;
            const int64_t per_cu = (wgs + kCUs - 1) / kCUs;
            const int64_t rounds = (wgs + kCUs * c.slots - 1) / (kCUs * c.slots);
            double t = per_cu * per * c.slice_us * (c.slots > 1 && wgs > kCUs ? shared : 1.0) +
                       rounds * round_us + (double)M * N * 4 / hbm * 1e6;
            // fewer workgroups than CUs: charged half again.  The fitted costs
            // come from launches alone on the GPU, where idle CUs cost nothing;
            // in a training step the other stream's work runs beside every
            // product, and tiles that give each CU a workgroup measured faster
            // there ([8192, 768] outputs on 128x128 rather than 256x128 tiles,
            // the weight gradients on smaller tiles: config-5 fp8 step 14.76 ->
            // 14.23-14.26 ms, same box, alternating)
            if(wgs < kCUs) t *= 1.5;
            if(splits > 1) t += (splits + 1.0) * M * N * 4 / hbm * 1e6 + launch_us;
            if(t < best_t) {
                best_t = t;
                best = MxPlan{c.wm, c.wn, (int)splits, (int)per};
            }
        }
    }
    return best;
}

// launch checks shared by both products; fills the shapes of p for a plan
int fp8q_shapes(const char* name, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, const void* A,
                const void* B, float* C, int64_t ldc, const MxPlan& plan, Fp8qParams& p) {
    if(M < 0 || N < 0 || K < 0) return pk::fail("%s: negative size", name);
    if(!C || (K > 0 && (!A || !B))) return pk::fail("%s: NULL pointer", name);
    if(ldc < N) return pk::fail("%s: ldc < N", name);
    const int64_t Kp = round_up(K > 0 ? K : 1, QKPAD), Mp = round_up(M, kTileQ), Np = round_up(N, kTileQ);
    if(K > 0 && (lda < Kp || ldb < Kp || lda % 16 || ldb % 16 || !pk::aligned16(A) || !pk::aligned16(B)))
        return pk::fail("%s: operands as the quantizer writes them: row strides >= K rounded up to 128, "
                        "multiples of 16, 16-byte aligned", name);
    if(Mp * lda > INT32_MAX || Np * ldb > INT32_MAX)
        return pk::fail("%s: an operand spans 2^31 bytes or more", name);
    const int64_t tm = (M + 64 * plan.wm - 1) / (64 * plan.wm), tn = (N + 64 * plan.wn - 1) / (64 * plan.wn);
    if(tm * tn * plan.splits > INT32_MAX) return pk::fail("%s: too many tiles", name);
    p = Fp8qParams{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = C;
    p.M = M;
    p.N = N;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.nslices = K > 0 ? plan.per : 0;
    p.total_slices = K > 0 ? (int)(Kp / QB) : 0;
    p.splits = K > 0 ? plan.splits : 1;
    // every split in range and none empty: (splits - 1) * per < total <= splits * per
    if(K > 0 && (plan.per % 2 || (int64_t)(plan.splits - 1) * plan.per >= p.total_slices ||
                 (int64_t)plan.splits * plan.per < p.total_slices))
        return pk::fail("%s: inconsistent K split (%d x %d slices for %d)", name, plan.splits, plan.per,
                        p.total_slices);
    p.tiles_m = (int)tm;
    p.tiles_n = (int)tn;
    return PK_OK;
}

template <int KIND>
void launch_fp8q_kind(int shape, unsigned grid, const Fp8qParams& p, hipStream_t st) {
    switch(shape) {
        case 0: gemm_fp8q_kernel<KIND, 4, 4><<<grid, NT, 0, st>>>(p); break;
        case 1: gemm_fp8q_kernel<KIND, 4, 2><<<grid, NT, 0, st>>>(p); break;
        case 2: gemm_fp8q_kernel<KIND, 2, 4><<<grid, NT, 0, st>>>(p); break;
        default: gemm_fp8q_kernel<KIND, 2, 2><<<grid, NT, 0, st>>>(p); break;
    }
}

void launch_fp8q(int kind, const MxPlan& plan, const Fp8qParams& p, hipStream_t st) {
    const unsigned grid = (unsigned)(p.tiles_m * p.tiles_n * p.splits);
    const int shape = plan.wm == 4 ? (plan.wn == 4 ? 0 : 1) : (plan.wn == 4 ? 2 : 3);
    if(kind == kQMX8) launch_fp8q_kind<kQMX8>(shape, grid, p, st);
    else if(kind == kQBF16) launch_fp8q_kind<kQBF16>(shape, grid, p, st);
    else if(kind == kQBF16X3) launch_fp8q_kind<kQBF16X3>(shape, grid, p, st);
    else launch_fp8q_kind<kQE4M3>(shape, grid, p, st);
}

}  // namespace

extern "C" int pk_gemm_fp8q_f32(int64_t M, int64_t N, int64_t K, float alpha, const uint8_t* A,
                                int64_t lda, const uint8_t* B, int64_t ldb, const float* scales,
                                float beta, float* C, int64_t ldc, pk_stream_t stream) {
    if(M > 0 && N > 0 && !scales) return pk::fail("pk_gemm_fp8q_f32: NULL scales");
    const MxPlan plan = mx8_plan(M, N, K, false);
    Fp8qParams p;
    if(int st = fp8q_shapes("pk_gemm_fp8q_f32", M, N, K, lda, ldb, A, B, C, ldc, plan, p)) return st;
    if(M == 0 || N == 0) return PK_OK;
    p.scales = scales;
    p.alpha = alpha;
    p.beta = beta;
    p.X = beta != 0.0f ? C : nullptr;
    p.ldx = ldc;
    launch_fp8q(kQE4M3, plan, p, pk::as_stream(stream));
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
    launch_quantize<true>(R, K, X, ldx, trans, nullptr, q, Kp, q + Rp * Kp, pk::as_stream(stream));
    return pk::launch_status("pk_mx8_quantize_f32");
}

extern "C" int pk_gemm_mx8_plan(int64_t M, int64_t N, int64_t K, int* tile_m, int* tile_n, int* splits) {
    if(M < 0 || N < 0 || K < 0) return pk::fail("pk_gemm_mx8_plan: negative size");
    const MxPlan plan = mx8_plan(M, N, K, true);
    if(tile_m) *tile_m = 64 * plan.wm;
    if(tile_n) *tile_n = 64 * plan.wn;
    if(splits) *splits = K > 0 ? plan.splits : 1;
    return PK_OK;
}

extern "C" size_t pk_gemm_mx8_workspace(int64_t M, int64_t N, int64_t K) {
    if(M <= 0 || N <= 0 || K <= 0) return 0;
    const MxPlan plan = mx8_plan(M, N, K, true);
    return plan.splits > 1 ? (size_t)plan.splits * M * N * sizeof(float) : 0;
}

extern "C" int pk_mx8_quantize2_f32(int64_t M, int64_t N, const float* X, int64_t ldx, void* QR, void* QT,
                                    pk_stream_t stream) {
    if(M < 0 || N < 0) return pk::fail("pk_mx8_quantize2_f32: negative size");
    if(M == 0 || N == 0) return PK_OK;
    if(!X || !QR || !QT) return pk::fail("pk_mx8_quantize2_f32: NULL pointer");
    if(ldx < N) return pk::fail("pk_mx8_quantize2_f32: ldx below the row length");
    if(!pk::aligned16(QR) || !pk::aligned16(QT)) return pk::fail("pk_mx8_quantize2_f32: Q must be 16-byte aligned");
    const int64_t Mg = round_up(M, kTileQ), Ng = round_up(N, kTileQ);
    if(Mg / 64 > INT32_MAX || Ng / 128 > 65535) return pk::fail("pk_mx8_quantize2_f32: too large");
    const bool vec = ldx % 4 == 0 && pk::aligned16(X);
    quantize_dual_kernel<<<dim3((unsigned)(Mg / 64), (unsigned)(Ng / 128)), NT, 0, pk::as_stream(stream)>>>(
        M, N, X, ldx, vec, static_cast<uint8_t*>(QR), static_cast<uint8_t*>(QT));
    return pk::launch_status("pk_mx8_quantize2_f32");
}

namespace {

// An MX8 or bf16 product of operands as the casts write them: Kb bytes a row
// (Kb = K for MX8, 2K for bf16), both padded to 128 bytes; MX8 scales follow
// the values.
int narrow_product(int kind, const char* name, int64_t M, int64_t N, int64_t Kb, float alpha, const void* A,
                   const void* B, float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                   void* workspace, size_t workspace_bytes, pk_stream_t stream) {
    const int64_t Kp = round_up(Kb > 0 ? Kb : 1, QKPAD), Mp = round_up(M, kTileQ), Np = round_up(N, kTileQ);
    MxPlan plan = mx8_plan(M, N, Kb, true);
    if(plan.splits > 1 && (!workspace || workspace_bytes < (size_t)plan.splits * M * N * sizeof(float)))
        plan = mx8_plan(M, N, Kb, false);
    Fp8qParams p;
    if(int st = fp8q_shapes(name, M, N, Kb, Kp, Kp, A, B, C, ldc, plan, p)) return st;
    if(M == 0 || N == 0) return PK_OK;
    if(beta != 0.0f && !X) return pk::fail("%s: beta != 0 needs X", name);
    if(beta != 0.0f && ldx != 0 && ldx < N) return pk::fail("%s: ldx < N", name);
    if(kind == kQMX8) {
        if(Mp * Kp / 32 > INT32_MAX || Np * Kp / 32 > INT32_MAX)
            return pk::fail("%s: scales span 2^31 bytes or more", name);
        p.SA = static_cast<const uint8_t*>(A) + Mp * Kp;
        p.SB = static_cast<const uint8_t*>(B) + Np * Kp;
        p.sstride_a = 2 * Mp;
        p.sstride_b = 2 * Np;
    }
    p.alpha = alpha;
    p.beta = beta;
    p.X = beta != 0.0f ? X : nullptr;
    p.ldx = ldx;
    hipStream_t st = pk::as_stream(stream);
    if(p.splits > 1) {
        p.P = static_cast<float*>(workspace);
        launch_fp8q(kind, plan, p, st);
        if(int e = pk::launch_status(name)) return e;
        const int64_t plane = M * N;
        const unsigned blocks = (unsigned)std::min<int64_t>((plane + NT - 1) / NT, 4 * kCUs * 8);
        fp8q_reduce_kernel<<<blocks, NT, 0, st>>>(M, N, p.splits, p.P, alpha, beta, p.X, ldx, C, ldc);
        return pk::launch_status(name);
    }
    launch_fp8q(kind, plan, p, st);
    return pk::launch_status(name);
}

}  // namespace

extern "C" int pk_gemm_mx8_ex_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                                  float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                                  void* workspace, size_t workspace_bytes, pk_stream_t stream) {
    return narrow_product(kQMX8, "pk_gemm_mx8_f32", M, N, K, alpha, A, B, beta, X, ldx, C, ldc, workspace,
                          workspace_bytes, stream);
}

extern "C" int pk_gemm_mx8_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                               float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                               pk_stream_t stream) {
    return pk_gemm_mx8_ex_f32(M, N, K, alpha, A, B, beta, X, ldx, C, ldc, nullptr, 0, stream);
}

// ---- bf16 operands ---------------------------------------------------------
// A bf16 matrix of R rows and K values per row: Rp = R rounded up to 256,
// Kv = K rounded up to 64; Rp * Kv values of 2 bytes (row stride 2 Kv bytes),
// each fp32 value rounded to nearest even, zero padding.
extern "C" size_t pk_bf16q_bytes(int64_t R, int64_t K) {
    if(R <= 0 || K <= 0) return 0;
    return (size_t)(round_up(R, kTileQ) * round_up(2 * K, QKPAD));
}

extern "C" int pk_bf16q_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, void* Q,
                                     pk_stream_t stream) {
    if(R < 0 || K < 0) return pk::fail("pk_bf16q_quantize_f32: negative size");
    if(R == 0 || K == 0) return PK_OK;
    if(!X || !Q) return pk::fail("pk_bf16q_quantize_f32: NULL pointer");
    if(ldx < (trans ? R : K)) return pk::fail("pk_bf16q_quantize_f32: ldx below the row length");
    if(!pk::aligned16(Q)) return pk::fail("pk_bf16q_quantize_f32: Q must be 16-byte aligned");
    const int64_t Rp = round_up(R, kTileQ), Kv = round_up(K, QB);
    if(Rp / 16 > 65535 || Kv / 64 > INT32_MAX) return pk::fail("pk_bf16q_quantize_f32: too large");
    const bool vec = ldx % 4 == 0 && pk::aligned16(X);
    uint8_t* q = static_cast<uint8_t*>(Q);
    hipStream_t st = pk::as_stream(stream);
    if(trans)
        bf16_cols_kernel<<<dim3((unsigned)(Kv / 64), (unsigned)(Rp / 128)), NT, 0, st>>>(R, K, X, ldx, vec, q,
                                                                                         2 * Kv, Rp);
    else
        bf16_rows_kernel<<<dim3((unsigned)((Kv + 255) / 256), (unsigned)(Rp / 16)), NT, 0, st>>>(
            R, K, X, ldx, vec, q, 2 * Kv, Kv, Rp);
    return pk::launch_status("pk_bf16q_quantize_f32");
}

extern "C" int pk_bf16q_quantize2_f32(int64_t M, int64_t N, const float* X, int64_t ldx, void* QR, void* QT,
                                      pk_stream_t stream) {
    if(M < 0 || N < 0) return pk::fail("pk_bf16q_quantize2_f32: negative size");
    if(M == 0 || N == 0) return PK_OK;
    if(!X || !QR || !QT) return pk::fail("pk_bf16q_quantize2_f32: NULL pointer");
    if(ldx < N) return pk::fail("pk_bf16q_quantize2_f32: ldx below the row length");
    if(!pk::aligned16(QR) || !pk::aligned16(QT))
        return pk::fail("pk_bf16q_quantize2_f32: Q must be 16-byte aligned");
    const int64_t Mg = round_up(M, kTileQ), Ng = round_up(N, kTileQ);
    if(Mg / 64 > INT32_MAX || Ng / 128 > 65535) return pk::fail("pk_bf16q_quantize2_f32: too large");
    const bool vec = ldx % 4 == 0 && pk::aligned16(X);
    bf16_dual_kernel<<<dim3((unsigned)(Mg / 64), (unsigned)(Ng / 128)), NT, 0, pk::as_stream(stream)>>>(
        M, N, X, ldx, vec, static_cast<uint8_t*>(QR), static_cast<uint8_t*>(QT));
    return pk::launch_status("pk_bf16q_quantize2_f32");
}

extern "C" size_t pk_gemm_bf16q_workspace(int64_t M, int64_t N, int64_t K) {
    if(M <= 0 || N <= 0 || K <= 0) return 0;
    const MxPlan plan = mx8_plan(M, N, 2 * K, true);
    return plan.splits > 1 ? (size_t)plan.splits * M * N * sizeof(float) : 0;
}

extern "C" int pk_gemm_bf16q_ex_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                                    float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                                    void* workspace, size_t workspace_bytes, pk_stream_t stream) {
    if(K < 0) return pk::fail("pk_gemm_bf16q_f32: negative size");
    return narrow_product(kQBF16, "pk_gemm_bf16q_f32", M, N, 2 * K, alpha, A, B, beta, X, ldx, C, ldc,
                          workspace, workspace_bytes, stream);
}

extern "C" int pk_gemm_bf16q_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                                 float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                                 pk_stream_t stream) {
    return pk_gemm_bf16q_ex_f32(M, N, K, alpha, A, B, beta, X, ldx, C, ldc, nullptr, 0, stream);
}

// ---- split-bf16 operands (three bf16 products per fp32 one) -----------------
// A split matrix of R rows and K values per row: Rp = R rounded up to 256,
// Kv = K rounded up to 32; each row is Kv / 16 groups of 64 bytes (16 hi parts,
// then their 16 lo parts), row stride 4 Kv bytes, zero padding.
extern "C" size_t pk_bf16x3q_bytes(int64_t R, int64_t K) {
    if(R <= 0 || K <= 0) return 0;
    return (size_t)(round_up(R, kTileQ) * round_up(4 * K, QKPAD));
}

extern "C" int pk_bf16x3q_quantize_f32(int64_t R, int64_t K, const float* X, int64_t ldx, int trans, void* Q,
                                       pk_stream_t stream) {
    if(R < 0 || K < 0) return pk::fail("pk_bf16x3q_quantize_f32: negative size");
    if(R == 0 || K == 0) return PK_OK;
    if(!X || !Q) return pk::fail("pk_bf16x3q_quantize_f32: NULL pointer");
    if(ldx < (trans ? R : K)) return pk::fail("pk_bf16x3q_quantize_f32: ldx below the row length");
    if(!pk::aligned16(Q)) return pk::fail("pk_bf16x3q_quantize_f32: Q must be 16-byte aligned");
    const int64_t Rp = round_up(R, kTileQ), Kv = round_up(K, 32);
    if(Rp / 16 > 65535 || Kv / 64 > INT32_MAX) return pk::fail("pk_bf16x3q_quantize_f32: too large");
    const bool vec = ldx % 4 == 0 && pk::aligned16(X);
    uint8_t* q = static_cast<uint8_t*>(Q);
    hipStream_t st = pk::as_stream(stream);
    if(trans)
        split_cols_kernel<<<dim3((unsigned)((Kv + 63) / 64), (unsigned)(Rp / 128)), NT, 0, st>>>(R, K, X, ldx, vec,
                                                                                                 q, 4 * Kv, Kv, Rp);
    else
        split_rows_kernel<<<dim3((unsigned)((Kv + 255) / 256), (unsigned)(Rp / 16)), NT, 0, st>>>(
            R, K, X, ldx, vec, q, 4 * Kv, Kv, Rp);
    return pk::launch_status("pk_bf16x3q_quantize_f32");
}

extern "C" size_t pk_gemm_bf16x3q_workspace(int64_t M, int64_t N, int64_t K) {
    if(M <= 0 || N <= 0 || K <= 0) return 0;
    const MxPlan plan = mx8_plan(M, N, 4 * K, true);
    return plan.splits > 1 ? (size_t)plan.splits * M * N * sizeof(float) : 0;
}

extern "C" int pk_gemm_bf16x3q_ex_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A,
                                      const void* B, float beta, const float* X, int64_t ldx, float* C,
                                      int64_t ldc, void* workspace, size_t workspace_bytes,
                                      pk_stream_t stream) {
    if(K < 0) return pk::fail("pk_gemm_bf16x3q_f32: negative size");
    return narrow_product(kQBF16X3, "pk_gemm_bf16x3q_f32", M, N, 4 * K, alpha, A, B, beta, X, ldx, C, ldc,
                          workspace, workspace_bytes, stream);
}

extern "C" int pk_gemm_bf16x3q_f32(int64_t M, int64_t N, int64_t K, float alpha, const void* A, const void* B,
                                   float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                                   pk_stream_t stream) {
    return pk_gemm_bf16x3q_ex_f32(M, N, K, alpha, A, B, beta, X, ldx, C, ldc, nullptr, 0, stream);
}
