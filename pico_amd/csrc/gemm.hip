// pico_amd/csrc/gemm.hip -- fp32 GEMM on gfx950 matrix cores.
//
// C = alpha * op(A) . op(B) + beta * C, row-major, the three layouts pico's
// matmul and its backward need (A.B, A.B^T, A^T.B; src/ops.c:144-190 and
// src/autograd.h:96-130), plus a two-level batch and the causal tile/k-range
// restrictions attention uses.
//
// Design (one 256-thread workgroup = 4 waves per C tile):
//  * Five tile shapes built from v_mfma_f32_32x32x2f32 blocks (4096 FLOP per
//    instruction, 16 fp32 accumulators per lane per block), chosen per call by
//    how evenly they spread over the 256 CUs:
//      256x256  2x2 waves of 128x128 (4x4 blocks, 256 accumulators held in
//               AGPRs), one workgroup per CU -- large products;
//      256x96   4x1 waves of 64x96, one per CU -- N a multiple of 96 (an
//               [8192, 768] output, d_model 768, is 256 of them);
//      128x128  2x2 waves of 64x64, two workgroups per CU;
//      128x96   4x1 waves of 32x96, two per CU -- N a multiple of 96;
//      64x64    2x2 waves of 32x32, four per CU -- small products.
//  * Tiles on the edge of C are handled in the same kernel: with M, N, K and
//    the strides multiples of 4 each 128-bit load is predicated as a whole;
//    otherwise loads fall back to 32-bit elements.
//  * K advances 32 at a time through a double-buffered LDS ring.  A 32-wide
//    slice is consumed as four k-groups of 4; the fragments of group q+1 are
//    read from LDS while the MFMAs of group q run (two register sets).  The
//    next slice is staged into the other LDS buffer, and the slice after it
//    fetched into registers with 128-bit global loads, spread over groups 0-2.
//    Unsplit products of the tiles up to 128x128 and of 256x96, which have at
//    most two workgroups per CU to hide a load, hold two slices in registers
//    and fetch three ahead.  Every memory instruction is interleaved with the MFMAs through
//    sched_group_barrier, so the wave never issues a long run of loads or
//    stores while the matrix pipe drains (measured: a block of 16 back-to-back
//    stores + 16 loads per slice cost 13 % of the MFMA rate).  One barrier per
//    slice sits before group 3, so group 0 of the next slice is read under
//    group 3's MFMAs.
//  * LDS holds every operand k-contiguous, [rows][32 + 4 pad]: an operand that
//    is row-contiguous in memory is fetched one row and four consecutive k per
//    thread (four 32-bit loads, each a contiguous run of 64 rows per wave), so
//    its values arrive k-contiguous in registers and go to LDS as one 128-bit
//    store, with no transposing moves (VALU work, which on gfx950 does not
//    overlap the matrix products).  Within a 32-wide k slice, lanes 0-31 take
//    k 0..15 and lanes 32-63 take k 16..31, so every fragment read is a 128-bit
//    LDS load, for all four layouts (measured: paired 32-bit reads of a
//    row-contiguous tile held NN and TN 5 % below NT).
//  * Tile order is XCD-aware: the hardware deals consecutive workgroups to
//    the 8 XCDs round-robin, so the launch index is remapped to give each XCD
//    a contiguous run of tiles, walked in groups of 8 tile-rows so concurrently
//    running tiles share A rows and B columns in that XCD's L2.
//  * Each output element accumulates k in the same order (k, then k+16 within
//    each pair of a slice) for every tile shape, so the shape choice never
//    changes a result bit.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <type_traits>

#include "pk_common.h"

namespace {

constexpr int BK = 32, NT = 256;
constexpr int KF = BK + 4;  // row stride of a k-contiguous LDS tile [rows][36]
constexpr int GROUP_M = 8;
constexpr int64_t kCUs = 256;  // MI355X

// One operand's R x BK slice, staged into a k-contiguous LDS tile [R][KF].
// Each staging item is 4 consecutive k of one row, held as one float4 and
// stored to LDS as one 128-bit write; R/32 items per thread.
//  * k-contiguous in memory (KFAST: op(A) when A is not transposed, op(B)^T
//    when B is): the item is one 128-bit load.
//  * row-contiguous in memory: the item is four 32-bit loads, one per k, and
//    consecutive threads take consecutive rows, so each load instruction of a
//    wave reads one k-row's 64 consecutive floats.  (An earlier staging of
//    4 x 4 blocks -- 128-bit loads along the rows, transposed in registers --
//    spent 15-30 VALU moves per slice, and its loads touched 8 k-rows 64 KB
//    apart per instruction, which shared vector-L1 sets.)
template <bool KFAST, int R>
struct Operand {
    static constexpr int ITEMS = R * BK / 4 / NT;
    static constexpr int F4 = ITEMS;            // float4 registers per thread
    static constexpr int OPS = KFAST ? 2 : 5;   // memory instructions per item (loads + store)
    static constexpr int FLOATS = R * KF;       // LDS floats of one stage
};

// A tile shape: WGM x (4 / WGM) waves, each TM x TN blocks of 32 x 32.
template <int BM_, int BN_, int WGM_, int TM_, int TN_, int OCC_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = 4 / WGM_, TM = TM_, TN = TN_;
    static constexpr int OCC = OCC_;  // resident workgroups per CU
    static_assert(WGM * TM * 32 == BM && WGN * TN * 32 == BN, "tile does not tile");
};
using Tile256 = Tile<256, 256, 2, 4, 4, 1>;
using Tile128 = Tile<128, 128, 2, 2, 2, 2>;
using Tile96 = Tile<128, 96, 4, 1, 3, 2>;
using Tile64 = Tile<64, 64, 2, 1, 1, 4>;
using Tile256x96 = Tile<256, 96, 4, 2, 3, 1>;

struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    int64_t M, N, K, lda, ldb, ldc;
    int64_t sAo, sAi, sBo, sBi, sCo, sCi, inner;
    float alpha, beta;
    int causal;
    int tiles_m, tiles_n;
    int splits;      // > 1: blockIdx.y is a K slice of kchunk, partials go to ws
    int64_t kchunk;
    float* ws;
    // the beta term's source: C itself, or another matrix (batch 1 only)
    const float* Cin;
    int64_t ldcin;
    // SwiGLU-backward epilogue (sg_a non-null, batch 1, no K split): the
    // product is the upstream gradient dh of h = silu(a) * u and is not
    // stored; the tile writes da (+)= dh*u*s*(1 + a*(1-s)) and du (+)= dh*a*s
    // (s = sigmoid(a)), accumulating per sg_flags bit 0 (da) and bit 1 (du)
    const float *sg_a, *sg_u;
    float *sg_da, *sg_du;
    int64_t sg_lda, sg_ldu, sg_ldd;
    int sg_flags;
    // the staged epilogue may use float4 accesses: every matrix it touches is
    // 16-byte aligned with a row stride that is a multiple of 4
    int epi_vec;
    // fp8 products: the device address of the two operand scales (NULL: 1, 1)
    const float* fp8_scale;
    // SwiGLU-forward epilogue (pair_F > 0, 'N','N', batch 1, no K split): C is
    // [gate | up], N = 2 pair_F columns.  A tile takes BN/2 gate columns and
    // the BN/2 up columns pair_F to their right, so it holds matching pairs;
    // it writes both to C and h = silu(gate) * up to sf_h
    int64_t pair_F;
    float* sf_h;
    int64_t sf_ldh;
};

// Bounds handling of a tile's loads and stores: none (whole tiles), per float4
// (M, N, K, the leading dimensions and batch strides multiples of 4, 16-byte
// aligned operands: a float4 is wholly inside or wholly outside), or per element.
constexpr int kEdgeNone = 0, kEdgeVec = 1, kEdgeScalar = 2;

// The float4 at logical (row r, k) of an operand: 4 consecutive k when
// KFAST (element (r,k) at base[r*ld + k]), else 4 consecutive rows (element
// (r,k) at base[k*ld + r]).  Edge modes zero-fill outside [Rlim) x [K).
template <bool KFAST, int EDGE>
__device__ __forceinline__ f32x4 load_f4(const float* __restrict__ base, int64_t ld, int64_t r,
                                         int64_t k, int64_t Rlim, int64_t K) {
    if(EDGE == kEdgeNone) {
        const float* p = KFAST ? base + r * ld + k : base + k * ld + r;
        return *reinterpret_cast<const f32x4*>(p);
    }
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if(EDGE == kEdgeVec) {
        // load from element (0, 0) when outside and select zero: no branch
        // splits the main loop (the launcher guarantees M, N, K > 0 here)
        const bool in = r < Rlim && k < K;
        const int64_t rs = in ? r : 0, ks = in ? k : 0;
        const f32x4 y =
            *reinterpret_cast<const f32x4*>(KFAST ? base + rs * ld + ks : base + ks * ld + rs);
        return in ? y : x;
    }
    if(KFAST) {
        if(r < Rlim) {
            const float* p = base + r * ld;
#pragma unroll
            for(int e = 0; e < 4; ++e)
                if(k + e < K) x[e] = p[k + e];
        }
    } else {
        if(k < K) {
            const float* p = base + k * ld;
#pragma unroll
            for(int e = 0; e < 4; ++e)
                if(r + e < Rlim) x[e] = p[r + e];
        }
    }
    return x;
}

// The 4 consecutive k (k..k+3) of row r of a row-contiguous operand
// (element (r, k) at base[k*ld + r]): four 32-bit loads.  Edge modes
// zero-fill outside [Rlim) x [K); with kEdgeVec K is a multiple of 4, so the
// four are in or out together.
template <int EDGE>
__device__ __forceinline__ f32x4 load_k4(const float* __restrict__ base, int64_t ld, int64_t r,
                                         int64_t k, int64_t Rlim, int64_t K) {
    f32x4 x;
    if(EDGE == kEdgeNone) {
        const float* p = base + k * ld + r;
#pragma unroll
        for(int t = 0; t < 4; ++t) x[t] = p[t * ld];
        return x;
    }
    if(EDGE == kEdgeVec) {
        // load from element (0, 0) when outside and select zero: no branch
        // splits the main loop (the launcher guarantees M, N, K > 0 here)
        const bool in = r < Rlim && k < K;
        const int64_t off = in ? k * ld + r : 0, step = in ? ld : 0;
#pragma unroll
        for(int t = 0; t < 4; ++t) {
            const float y = base[off + t * step];
            x[t] = in ? y : 0.0f;
        }
        return x;
    }
#pragma unroll
    for(int t = 0; t < 4; ++t) x[t] = r < Rlim && k + t < K ? base[(k + t) * ld + r] : 0.0f;
    return x;
}

// staging item `item` of this thread: the (row, k) origin of its 4 k
template <bool KFAST, int R>
__device__ __forceinline__ void item_origin(int item, int& rr, int& kk) {
    const int u = threadIdx.x + item * NT;
    if(KFAST) {
        // 8 consecutive threads read one row's 32 k (128 contiguous bytes)
        rr = u >> 3;
        kk = (u & 7) * 4;
    } else {
        // consecutive threads take consecutive rows at the same 4 k; their
        // 128-bit LDS stores (rows 36 floats apart) fall in distinct banks
        rr = u % R;
        kk = (u / R) * 4;
    }
}

// PAIR: rows R/2.. of the slice come from `shift` rows further on (the up
// columns of a paired SwiGLU product).
// Whole tiles (kEdgeNone) load through a buffer resource over the operand:
// the byte offset splits into a per-lane part (the item's place in the
// slice), which stays the same from slice to slice, and a uniform part (the
// tile's first row, the slice's first k, the k row of each of a row-contiguous
// item's four loads) that goes to the instruction's scalar offset, so no
// per-lane address arithmetic is repeated per slice.  The launcher takes this
// path only when every operand's extent is below 2^31 bytes.
template <bool KFAST, int EDGE, int R, bool PAIR = false>
__device__ __forceinline__ void load_item(const float* __restrict__ base, int64_t ld, int64_t r0,
                                          int64_t k0, int64_t Rlim, int64_t K, int item,
                                          f32x4* v, int64_t shift = 0) {
    int rr, kk;
    item_origin<KFAST, R>(item, rr, kk);
    if constexpr(EDGE == kEdgeNone) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(base), (short)0, 0x7fffffff, 0x00020000);
        const int lshift = PAIR && rr >= R / 2 ? (int)shift : 0;
        if(KFAST) {
            const int voff = ((rr + lshift) * (int)ld + kk) * 4;
            const int soff = (int)((r0 * ld + k0) * 4);
            v[0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
        } else {
            const int voff = (kk * (int)ld + rr + lshift) * 4;
            const int soff = (int)((k0 * ld + r0) * 4), step = (int)(ld * 4);
#pragma unroll
            for(int t = 0; t < 4; ++t)
                v[0][t] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff + t * step, 0));
        }
        return;
    }
    const int64_t r = r0 + rr + (PAIR && rr >= R / 2 ? shift : 0);
    if(KFAST) {
        v[0] = load_f4<true, EDGE>(base, ld, r, k0 + kk, Rlim, K);
    } else {
        v[0] = load_k4<EDGE>(base, ld, r, k0 + kk, Rlim, K);
    }
}

// Row stride (elements) of a k-contiguous LDS tile: fp32 [rows][36]; bf16
// [rows][40] (80 bytes: the 16-lane passes of 128-bit reads down a column of
// rows touch 16 distinct 4-bank groups).
constexpr int KFB = BK + 8;
// An e4m3 element of an fp8 tile (OCP FP8 E4M3: bias 7, 3 mantissa bits,
// largest finite 448), one byte.  fp8 tiles have rows of KF8 = 48 bytes:
// the 64-bit fragment reads of 16 consecutive rows then start 12 banks apart
// and never share a bank.
template <int OP>  // OP 0: an element of op(A)'s tile, 1: of op(B)'s
struct Fp8T {
    unsigned char v;
};
using Fp8A = Fp8T<0>;
using Fp8B = Fp8T<1>;
constexpr int KF8 = BK + 16;

// The fp8 kernel's operand scales (powers of two, so scaling is exact): op(A)
// and op(B) are multiplied by them before rounding, and the accumulated
// product is divided by both.  Set by each workgroup at its start.
__shared__ float g_fp8_scale[2];

template <class E>
constexpr int lds_stride() {
    return sizeof(E) == 4 ? KF : sizeof(E) == 1 ? KF8 : KFB;
}

// x rounded to e4m3 (nearest even) after clamping to the finite range, so
// the conversion's overflow handling never matters; NaN stays NaN
__device__ __forceinline__ float fp8_clamp(float x) {
    return x != x ? x : fminf(fmaxf(x, -448.0f), 448.0f);
}
// two e4m3 values into bytes 0-1 (HI false) or 2-3 (HI true) of old
template <bool HI>
__device__ __forceinline__ int fp8_pack2(float a, float b, int old) {
    return __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(a), fp8_clamp(b), old, HI);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// An element of a split-bf16 tile: x is stored as hi = bf16(x) and
// lo = bf16(x - hi), in two tiles LO elements apart (x - hi is exact in fp32,
// so hi + lo is x to 2^-17 relative).
template <int LO>
struct SplitBf16 {
    __bf16 hi;
};

template <int LO>
__device__ __forceinline__ void put_split(__bf16* t, int off, const float* w, int n) {
#pragma unroll
    for(int e = 0; e < 4; ++e) {
        if(e >= n) break;
        const __bf16 h = (__bf16)w[e];
        t[off + e] = h;
        t[off + LO + e] = (__bf16)(w[e] - (float)h);
    }
}

// store 4 consecutive k of one row; a bf16 tile gets them rounded to nearest
// even, a split tile their hi and lo parts
template <int LO>
__device__ __forceinline__ void put4(SplitBf16<LO>* lds, int off, f32x4 w) {
    __bf16* t = reinterpret_cast<__bf16*>(lds);
    bf16x4 h, l;
#pragma unroll
    for(int e = 0; e < 4; ++e) {
        h[e] = (__bf16)w[e];
        l[e] = (__bf16)(w[e] - (float)h[e]);
    }
    *reinterpret_cast<bf16x4*>(t + off) = h;
    *reinterpret_cast<bf16x4*>(t + off + LO) = l;
}

template <int OP>
__device__ __forceinline__ void put4(Fp8T<OP>* lds, int off, f32x4 w) {
    const float sc = g_fp8_scale[OP];
    const int v = fp8_pack2<true>(w[2] * sc, w[3] * sc, fp8_pack2<false>(w[0] * sc, w[1] * sc, 0));
    *reinterpret_cast<int*>(reinterpret_cast<unsigned char*>(lds) + off) = v;
}

template <class E>
__device__ __forceinline__ void put4(E* lds, int off, f32x4 w) {
    if constexpr(sizeof(E) == 4) {
        *reinterpret_cast<f32x4*>(lds + off) = w;
    } else {
        const bf16x4 b = {(__bf16)w[0], (__bf16)w[1], (__bf16)w[2], (__bf16)w[3]};
        *reinterpret_cast<bf16x4*>(lds + off) = b;
    }
}

template <bool KFAST, int R, class E>
__device__ __forceinline__ void store_item(E* lds, int item, const f32x4* v) {
    constexpr int LS = lds_stride<E>();
    int rr, kk;
    item_origin<KFAST, R>(item, rr, kk);
    put4(lds, rr * LS + kk, v[0]);
}

// k-group q (k = 4q..4q+3 for lanes 0-31, 16+4q.. for lanes 32-63) of the
// fragments of NB blocks starting at LDS row r0 (one row per lane)
template <int NB>
__device__ __forceinline__ void read_group(const float* lds, int r0, int lr, int lh, int q,
                                           float (&f)[NB][4]) {
#pragma unroll
    for(int b = 0; b < NB; ++b) {
        const f32x4 x =
            *reinterpret_cast<const f32x4*>(lds + (r0 + b * 32 + lr) * KF + lh * 16 + 4 * q);
        f[b][0] = x[0];
        f[b][1] = x[1];
        f[b][2] = x[2];
        f[b][3] = x[3];
    }
}

template <int TM, int TN>
__device__ __forceinline__ void mfma_group(f32x16 (&acc)[TM][TN], const float (&fa)[TM][4],
                                           const float (&fb)[TN][4]) {
#pragma unroll
    for(int t = 0; t < 4; ++t)
#pragma unroll
        for(int i = 0; i < TM; ++i)
#pragma unroll
            for(int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][t], fb[j][t], acc[i][j], 0,
                                                                 0, 0);
}

// Scheduling hints for one k-group: NMEM memory instructions (LDS or global)
// spread evenly after the group's NMFMA matrix instructions.
constexpr int kMaskMfma = 0x008, kMaskMem = 0x090;  // MFMA; all VMEM | all DS

template <int NMFMA, int NMEM, int I = 0>
__device__ __forceinline__ void interleave() {
    if constexpr(I < NMFMA) {
        constexpr int m = (I + 1) * NMEM / NMFMA - I * NMEM / NMFMA;
        __builtin_amdgcn_sched_group_barrier(kMaskMfma, 1, 0);
        if constexpr(m > 0) __builtin_amdgcn_sched_group_barrier(kMaskMem, m, 0);
        interleave<NMFMA, NMEM, I + 1>();
    }
}

// Staging of the next operand slice, spread over k-groups 0..2: the items
// of A then B, split where the memory instructions (a store and a load per
// float4) divide most evenly in three.  Each item is stored from registers to
// LDS, then refetched from k slice kn.
template <bool AK, bool BKF, class T>
struct Staging {
    using OA = Operand<AK, T::BM>;
    using OB = Operand<BKF, T::BN>;
    static constexpr int ITEMS = OA::ITEMS + OB::ITEMS;
    static constexpr int ops(int item) { return item < OA::ITEMS ? OA::OPS : OB::OPS; }
    static constexpr int ops_before(int item) {
        int n = 0;
        for(int i = 0; i < item; ++i) n += ops(i);
        return n;
    }
    // first item of group g: the first whose preceding ops reach g/3 of the total
    static constexpr int lo(int g) {
        if(g >= 3) return ITEMS;
        int i = 0;
        while(i < ITEMS && 3 * ops_before(i) < g * ops_before(ITEMS)) ++i;
        return i;
    }
    static constexpr int group_ops(int g) { return ops_before(lo(g + 1)) - ops_before(lo(g)); }
};

template <bool AK, bool BKF, int EDGE, class T, int G, bool PAIR = false, int NA, int NB, class EA,
          class EB>
__device__ __forceinline__ void stage(f32x4 (&ra)[NA], f32x4 (&rb)[NB], EA* sa, EB* sb,
                                      const float* __restrict__ A, const float* __restrict__ B,
                                      const GemmParams& p, int64_t row0, int64_t col0, int64_t kn,
                                      int64_t kend) {
    using S = Staging<AK, BKF, T>;
    constexpr int IA = S::OA::ITEMS, FA = 1, FB = 1;
    constexpr int lo = S::lo(G), hi = S::lo(G + 1);
#pragma unroll
    for(int e = lo; e < hi; ++e) {
        if(e < IA)
            store_item<AK, T::BM>(sa, e, &ra[e * FA]);
        else
            store_item<BKF, T::BN>(sb, e - IA, &rb[(e - IA) * FB]);
    }
#pragma unroll
    for(int e = lo; e < hi; ++e) {
        if(e < IA)
            load_item<AK, EDGE, T::BM>(A, p.lda, row0, kn, p.M, kend, e, &ra[e * FA]);
        else
            load_item<BKF, EDGE, T::BN, PAIR>(B, p.ldb, col0, kn, p.N, kend, e - IA,
                                              &rb[(e - IA) * FB], p.pair_F - T::BN / 2);
    }
}

// One workgroup's job: its tile, operand bases, output, K range.
struct TileJob {
    const float* A;
    const float* B;
    float* C;
    const float* Cin;
    int64_t ldc, ldcin, row0, col0, kbeg, kend;
    float alpha, beta;
    int nslices;
    bool skip;
};

template <class T>
__device__ __forceinline__ TileJob tile_job(const GemmParams& p) {
    TileJob j;
    // tile selection: XCD-contiguous runs, grouped by GROUP_M tile-rows
    const int ntiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
    const int group_span = GROUP_M * p.tiles_n;
    const int first_m = (bid / group_span) * GROUP_M;
    const int gm = min(p.tiles_m - first_m, GROUP_M);
    const int local = bid % group_span;
    const int tm = first_m + local % gm;
    const int tn = local / gm;

    // blockIdx.y is the batch index, or the K slice of a split product
    const int64_t z = p.splits > 1 ? 0 : blockIdx.y;
    const int64_t zo = z / p.inner, zi = z % p.inner;
    j.A = p.A + zo * p.sAo + zi * p.sAi;
    j.B = p.B + zo * p.sBo + zi * p.sBi;
    j.C = p.C + zo * p.sCo + zi * p.sCi;
    j.ldc = p.ldc;
    j.Cin = p.Cin ? p.Cin : j.C;
    j.ldcin = p.Cin ? p.ldcin : p.ldc;
    j.alpha = p.alpha;
    j.beta = p.beta;

    j.row0 = (int64_t)tm * T::BM;
    j.col0 = (int64_t)tn * (p.pair_F ? T::BN / 2 : T::BN);
    j.kbeg = 0;
    j.kend = p.K;
    j.skip = p.causal == 1 && j.col0 > j.row0 + T::BM - 1;  // wholly above the diagonal
    if(p.causal == 2) j.kend = min(p.K, j.row0 + T::BM);
    if(p.causal == 3) j.kbeg = min(p.K, (j.row0 / BK) * BK);
    if(p.splits > 1) {
        // slice s of K; its partial product goes to workspace plane s
        j.kbeg = (int64_t)blockIdx.y * p.kchunk;
        j.kend = min(p.K, j.kbeg + p.kchunk);
        j.C = p.ws + (int64_t)blockIdx.y * p.M * p.N;
        j.ldc = p.N;
        j.Cin = j.C;
        j.ldcin = p.N;
        j.alpha = 1.0f;
        j.beta = 0.0f;
    }
    j.nslices = (int)((j.kend - j.kbeg + BK - 1) / BK);
    return j;
}

// C tile = alpha * acc (+ beta * C).  32x32 block accumulator r of lane l is
// row 8*(r/4) + 4*(l/32) + r%4, column l%32: each half-wave writes 128
// contiguous bytes per register.
template <int EDGE, int TM, int TN>
__device__ __forceinline__ void store_tile(const GemmParams& p, const TileJob& j,
                                           const f32x16 (&acc)[TM][TN], int ar0, int br0, int lr,
                                           int lh) {
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int jj = 0; jj < TN; ++jj) {
            const int64_t col = j.col0 + br0 + jj * 32 + lr;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                const int64_t row = j.row0 + ar0 + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                if(EDGE != kEdgeNone && (row >= p.M || col >= p.N)) continue;
                float v = j.alpha * acc[i][jj][r];
                float* c = j.C + row * j.ldc + col;
                if(j.beta != 0.0f) v += j.beta * *c;
                // 64x64 tiles (products of about 1024^2 outputs, where the
                // launch's end is a large share of its time) store C
                // non-temporally: 1024^3 1.1-1.6 % and 768^3 0.6-1.1 % faster,
                // config-4 and config-5 steps unchanged (same box, alternating);
                // for every tile they cost a config-5 step 0.05 ms
                if constexpr(TM * TN == 1) __builtin_nontemporal_store(v, c);
                else *c = v;
            }
        }
}

// Epilogues that read other matrices: the tile goes through LDS (free once
// the main loop is done) in passes of RP rows, and all 256 threads then walk
// the staged rows in float4 runs, so every global access is a coalesced
// 128-bit one and no per-element loads wait inside the accumulator loops
// (which, in the 256x256 tile, also pushed the accumulators out of
// registers).
//   kEpiAdd:    C = alpha * acc + beta * Cin
//   kEpiSwiglu: dh = alpha * acc; da (+)= dh*u*s*(1 + a*(1-s)), du (+)= dh*a*s
//   kEpiSwigluFwd: the tile's two column halves are matching gate and up
//               columns: C gets g = alpha * acc and u alike (as the plain
//               store writes them), sf_h gets silu(g) * u
constexpr int kEpiPlain = 0, kEpiAdd = 1, kEpiSwiglu = 2, kEpiSwigluFwd = 3;

template <int EPI>
__device__ __forceinline__ void epi_one(const GemmParams& p, const TileJob& j, int64_t row,
                                        int64_t col, float x) {
    if constexpr(EPI == kEpiAdd) {
        float v = j.alpha * x;
        if(j.beta != 0.0f) v += j.beta * j.Cin[row * j.ldcin + col];
        j.C[row * j.ldc + col] = v;
    } else {
        float ga, gu;
        pk::swiglu_bwd1(p.sg_a[row * p.sg_lda + col], p.sg_u[row * p.sg_ldu + col], j.alpha * x,
                        ga, gu);
        float* da = p.sg_da + row * p.sg_ldd + col;
        float* du = p.sg_du + row * p.sg_ldd + col;
        if(p.sg_flags & PK_ACCUM) ga = pk::add_nc(*da, ga);
        if(p.sg_flags & PK_ACCUM2) gu = pk::add_nc(*du, gu);
        *da = ga;
        *du = gu;
    }
}

template <int EPI>
__device__ __forceinline__ void epi_four(const GemmParams& p, const TileJob& j, int64_t row,
                                         int64_t col, f32x4 x) {
    if constexpr(EPI == kEpiAdd) {
        f32x4 v;
#pragma unroll
        for(int e = 0; e < 4; ++e) v[e] = j.alpha * x[e];
        if(j.beta != 0.0f) {
            const f32x4 c = *reinterpret_cast<const f32x4*>(j.Cin + row * j.ldcin + col);
#pragma unroll
            for(int e = 0; e < 4; ++e) v[e] += j.beta * c[e];
        }
        *reinterpret_cast<f32x4*>(j.C + row * j.ldc + col) = v;
    } else {
        const f32x4 a = *reinterpret_cast<const f32x4*>(p.sg_a + row * p.sg_lda + col);
        const f32x4 u = *reinterpret_cast<const f32x4*>(p.sg_u + row * p.sg_ldu + col);
        f32x4* dap = reinterpret_cast<f32x4*>(p.sg_da + row * p.sg_ldd + col);
        f32x4* dup = reinterpret_cast<f32x4*>(p.sg_du + row * p.sg_ldd + col);
        f32x4 pa = {0.f, 0.f, 0.f, 0.f}, pu = {0.f, 0.f, 0.f, 0.f};
        if(p.sg_flags & PK_ACCUM) pa = *dap;
        if(p.sg_flags & PK_ACCUM2) pu = *dup;
        f32x4 ga, gu;
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            float y, z;
            pk::swiglu_bwd1(a[e], u[e], j.alpha * x[e], y, z);
            ga[e] = (p.sg_flags & PK_ACCUM) ? pk::add_nc(pa[e], y) : y;
            gu[e] = (p.sg_flags & PK_ACCUM2) ? pk::add_nc(pu[e], z) : z;
        }
        *dap = ga;
        *dup = gu;
    }
}

template <int EPI, class T, int LDS_FLOATS>
__device__ __forceinline__ void staged_epilogue(const GemmParams& p, const TileJob& j,
                                                const f32x16 (&acc)[T::TM][T::TN], float* lds,
                                                int ar0, int br0, int lr, int lh) {
    constexpr int BN = T::BN, LDE = BN + 4, TM = T::TM, TN = T::TN;
    // rows per pass: whole 32-row blocks that fit in the operand buffers
    constexpr int rp = (LDS_FLOATS / LDE) / 32 * 32 < T::BM ? (LDS_FLOATS / LDE) / 32 * 32 : T::BM;
    static_assert(rp >= 32, "the staging buffer must hold at least one 32-row block");
    __syncthreads();  // every wave is done reading the operand tiles
    for(int lo = 0; lo < T::BM; lo += rp) {
#pragma unroll
        for(int i = 0; i < TM; ++i) {
            const int rb = ar0 + i * 32;
            if(rb < lo || rb >= lo + rp) continue;
#pragma unroll
            for(int jj = 0; jj < TN; ++jj)
#pragma unroll
                for(int r = 0; r < 16; ++r)
                    lds[(rb - lo + (r >> 2) * 8 + lh * 4 + (r & 3)) * LDE + br0 + jj * 32 + lr] =
                        acc[i][jj][r];
        }
        __syncthreads();
        const int rows = rp < T::BM - lo ? rp : T::BM - lo;
        if constexpr(EPI == kEpiSwigluFwd) {
            // column c of the gate half pairs with column BN/2 + c; the host
            // guarantees whole column halves (pair_F a multiple of BN/2)
            constexpr int HB = BN / 2;
            for(int idx = threadIdx.x; idx < rows * (HB / 4); idx += NT) {
                const int rr = idx / (HB / 4), c = (idx % (HB / 4)) * 4;
                const int64_t row = j.row0 + lo + rr, col = j.col0 + c;
                if(row >= p.M) continue;
                const f32x4 g = *reinterpret_cast<const f32x4*>(lds + rr * LDE + c);
                const f32x4 u = *reinterpret_cast<const f32x4*>(lds + rr * LDE + HB + c);
                f32x4 gv, uv, hv;
#pragma unroll
                for(int e = 0; e < 4; ++e) {
                    gv[e] = j.alpha * g[e];
                    uv[e] = j.alpha * u[e];
                    hv[e] = pk::swiglu_fwd1(gv[e], uv[e]);
                }
                float* cg = j.C + row * j.ldc + col;
                float* hp = p.sf_h + row * p.sf_ldh + col;
                if(p.epi_vec) {
                    *reinterpret_cast<f32x4*>(cg) = gv;
                    *reinterpret_cast<f32x4*>(cg + p.pair_F) = uv;
                    *reinterpret_cast<f32x4*>(hp) = hv;
                } else {
#pragma unroll
                    for(int e = 0; e < 4; ++e) {
                        cg[e] = gv[e];
                        cg[p.pair_F + e] = uv[e];
                        hp[e] = hv[e];
                    }
                }
            }
        } else {
            for(int idx = threadIdx.x; idx < rows * (BN / 4); idx += NT) {
                const int rr = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
                const int64_t row = j.row0 + lo + rr, col = j.col0 + c;
                const f32x4 x = *reinterpret_cast<const f32x4*>(lds + rr * LDE + c);
                if(row >= p.M) continue;
                if(p.epi_vec && col + 3 < p.N) {
                    epi_four<EPI>(p, j, row, col, x);
                } else {
#pragma unroll
                    for(int e = 0; e < 4; ++e)
                        if(col + e < p.N) epi_one<EPI>(p, j, row, col + e, x[e]);
                }
            }
        }
        __syncthreads();
    }
}

// prologue shared by both kernels: slice 0 into LDS buffer 0, slice 1 into
// the staging registers
template <bool AK, bool BKF, int EDGE, class T, bool PAIR = false, int NA, int NB, class EA,
          class EB>
__device__ __forceinline__ void prologue(const GemmParams& p, const TileJob& j, f32x4 (&ra)[NA],
                                         f32x4 (&rb)[NB], EA* sa, EB* sb) {
    using OA = Operand<AK, T::BM>;
    using OB = Operand<BKF, T::BN>;
#pragma unroll
    for(int e = 0; e < OA::ITEMS; ++e)
        load_item<AK, EDGE, T::BM>(j.A, p.lda, j.row0, j.kbeg, p.M, j.kend, e, &ra[e]);
#pragma unroll
    for(int e = 0; e < OB::ITEMS; ++e)
        load_item<BKF, EDGE, T::BN, PAIR>(j.B, p.ldb, j.col0, j.kbeg, p.N, j.kend, e,
                                          &rb[e], p.pair_F - T::BN / 2);
#pragma unroll
    for(int e = 0; e < OA::ITEMS; ++e) store_item<AK, T::BM>(sa, e, &ra[e]);
#pragma unroll
    for(int e = 0; e < OB::ITEMS; ++e) store_item<BKF, T::BN>(sb, e, &rb[e]);
    const int64_t k1 = j.kbeg + (j.nslices > 1 ? BK : 0);
#pragma unroll
    for(int e = 0; e < OA::ITEMS; ++e)
        load_item<AK, EDGE, T::BM>(j.A, p.lda, j.row0, k1, p.M, j.kend, e, &ra[e]);
#pragma unroll
    for(int e = 0; e < OB::ITEMS; ++e)
        load_item<BKF, EDGE, T::BN, PAIR>(j.B, p.ldb, j.col0, k1, p.N, j.kend, e,
                                          &rb[e], p.pair_F - T::BN / 2);
}

// the tiles that can hold a second slice in their staging registers
template <class T>
constexpr bool deep_staging() {
    return T::BM * T::BN <= 128 * 128 || (T::BM == 256 && T::BN == 96);
}

template <bool TA, bool TB, int EDGE, class T, int EPI, bool DEEP = false>
__global__ __launch_bounds__(NT, T::OCC) void gemm_f32_kernel(GemmParams p) {
    constexpr int BM = T::BM, BN = T::BN, TM = T::TM, TN = T::TN, WGN = T::WGN;
    // op(A) rows are k-contiguous when A is not transposed; op(B)^T rows
    // (indexed by n) are k-contiguous when B is transposed.
    constexpr bool AK = !TA, BKF = TB;
    using OA = Operand<AK, BM>;
    using OB = Operand<BKF, BN>;
    using S = Staging<AK, BKF, T>;
    __shared__ __attribute__((aligned(16))) float ldsA[2][OA::FLOATS];
    __shared__ __attribute__((aligned(16))) float ldsB[2][OB::FLOATS];

    const TileJob job = tile_job<T>(p);
    if(job.skip) return;
    const float* __restrict__ A = job.A;
    const float* __restrict__ B = job.B;
    const int64_t row0 = job.row0, col0 = job.col0, kbeg = job.kbeg, kend = job.kend;
    const int nslices = job.nslices;

    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    const int wm = w / WGN, wn = w % WGN;
    const int lr = l & 31, lh = l >> 5;
    const int ar0 = wm * TM * 32, br0 = wn * TN * 32;

    f32x16 acc[TM][TN];
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int j = 0; j < TN; ++j)
#pragma unroll
            for(int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    constexpr int RD = TM + TN;  // 128-bit LDS reads per k-group
    constexpr int NMFMA = TM * TN * 4;

    if(nslices > 0) {
        constexpr bool PAIR = EPI == kEpiSwigluFwd;
        // DEEP (tiles of at most 128x128, whose slices are short: 0.4-1.7 us,
        // and 256x96, one workgroup per CU): two slices in the staging
        // registers, fetched three slices ahead, so a load has two slices'
        // time to arrive rather than one.  It costs 15-60 VGPRs, which the
        // launcher spends only on unsplit products; 256x256 has none to spare
        constexpr bool PF2 = DEEP && deep_staging<T>();
        constexpr int AHEAD = PF2 ? 3 : 2;
        f32x4 ra[OA::F4], rb[OB::F4];
        prologue<AK, BKF, EDGE, T, PAIR>(p, job, ra, rb, ldsA[0], ldsB[0]);
        f32x4 ra2[PF2 ? OA::F4 : 1], rb2[PF2 ? OB::F4 : 1];
        if constexpr(PF2) {
            const int64_t k2 = kbeg + (int64_t)min(2, nslices - 1) * BK;
#pragma unroll
            for(int e = 0; e < OA::ITEMS; ++e)
                load_item<AK, EDGE, BM>(A, p.lda, row0, k2, p.M, kend, e, &ra2[e]);
#pragma unroll
            for(int e = 0; e < OB::ITEMS; ++e)
                load_item<BKF, EDGE, BN, PAIR>(B, p.ldb, col0, k2, p.N, kend, e, &rb2[e],
                                               p.pair_F - BN / 2);
        }
        __syncthreads();
        float fa0[TM][4], fb0[TN][4], fa1[TM][4], fb1[TN][4];
        read_group<TM>(ldsA[0], ar0, lr, lh, 0, fa0);
        read_group<TN>(ldsB[0], br0, lr, lh, 0, fb0);
        // slice s: stage (xa, xb) -- slice s+1 -- into the other LDS buffer and
        // refill them with slice s+AHEAD; past the end the refill re-fetches the
        // last slice, which keeps the loop free of branches
        auto slice = [&](int s, f32x4 (&xa)[OA::F4], f32x4 (&xb)[OB::F4]) {
            const int cur = s & 1;
            const float* la = ldsA[cur];
            const float* lb = ldsB[cur];
            float* sa = ldsA[cur ^ 1];
            float* sb = ldsB[cur ^ 1];
            const int64_t kn = kbeg + (int64_t)min(s + AHEAD, nslices - 1) * BK;

            // group 0: read group 1, stage part 0
            read_group<TM>(la, ar0, lr, lh, 1, fa1);
            read_group<TN>(lb, br0, lr, lh, 1, fb1);
            stage<AK, BKF, EDGE, T, 0, PAIR>(xa, xb, sa, sb, A, B, p, row0, col0, kn, kend);
            mfma_group<TM, TN>(acc, fa0, fb0);
            interleave<NMFMA, RD + S::group_ops(0)>();
            __builtin_amdgcn_sched_barrier(0);
            // group 1: read group 2, stage part 1
            read_group<TM>(la, ar0, lr, lh, 2, fa0);
            read_group<TN>(lb, br0, lr, lh, 2, fb0);
            stage<AK, BKF, EDGE, T, 1, PAIR>(xa, xb, sa, sb, A, B, p, row0, col0, kn, kend);
            mfma_group<TM, TN>(acc, fa1, fb1);
            interleave<NMFMA, RD + S::group_ops(1)>();
            __builtin_amdgcn_sched_barrier(0);
            // group 2: read group 3, stage part 2
            read_group<TM>(la, ar0, lr, lh, 3, fa1);
            read_group<TN>(lb, br0, lr, lh, 3, fb1);
            stage<AK, BKF, EDGE, T, 2, PAIR>(xa, xb, sa, sb, A, B, p, row0, col0, kn, kend);
            mfma_group<TM, TN>(acc, fa0, fb0);
            interleave<NMFMA, RD + S::group_ops(2)>();
            __builtin_amdgcn_sched_barrier(0);
            // every wave has staged slice s+1 and finished reading slice s
            __syncthreads();
            // group 3, with group 0 of slice s+1 read underneath (on the last
            // slice this reads the re-staged data and is discarded)
            read_group<TM>(sa, ar0, lr, lh, 0, fa0);
            read_group<TN>(sb, br0, lr, lh, 0, fb0);
            mfma_group<TM, TN>(acc, fa1, fb1);
            interleave<NMFMA, RD>();
            __builtin_amdgcn_sched_barrier(0);
        };
        if constexpr(PF2) {
            // even slices stage ra/rb, odd ones ra2/rb2
            int s = 0;
            for(; s + 1 < nslices; s += 2) {
                slice(s, ra, rb);
                slice(s + 1, ra2, rb2);
            }
            if(s < nslices) slice(s, ra, rb);
        } else {
            for(int s = 0; s < nslices; ++s) slice(s, ra, rb);
        }
    }
    if constexpr(EPI == kEpiPlain)
        store_tile<EDGE, TM, TN>(p, job, acc, ar0, br0, lr, lh);
    else if constexpr(sizeof(ldsA) >= sizeof(ldsB))
        staged_epilogue<EPI, T, sizeof(ldsA) / sizeof(float)>(p, job, acc, &ldsA[0][0], ar0, br0,
                                                             lr, lh);
    else
        staged_epilogue<EPI, T, sizeof(ldsB) / sizeof(float)>(p, job, acc, &ldsB[0][0], ar0, br0,
                                                             lr, lh);
}

// The same product with bf16 multiplies: op(A) and op(B) are rounded to bf16
// (nearest even) on their way to LDS and multiplied by
// v_mfma_f32_32x32x16_bf16 (32768 FLOP per instruction, eight times the fp32
// rate), accumulating in fp32.  Global traffic, staging, tiles and split-K
// are the fp32 kernel's; a 32-wide k slice is two MFMA steps of k 16, the
// second step's fragments read under the first step's MFMAs and the next
// slice's first fragments under the second.  A lane's 8 k of a step are k
// 16t + 8*(lane/32) .. +7, the same for both operands.
template <int NB>
__device__ __forceinline__ void read_step(const __bf16* lds, int r0, int lr, int lh, int t,
                                          bf16x8 (&f)[NB]) {
#pragma unroll
    for(int b = 0; b < NB; ++b)
        f[b] = *reinterpret_cast<const bf16x8*>(lds + (r0 + b * 32 + lr) * KFB + 16 * t + 8 * lh);
}

template <int TM, int TN>
__device__ __forceinline__ void mfma_step(f32x16 (&acc)[TM][TN], const bf16x8 (&fa)[TM],
                                          const bf16x8 (&fb)[TN]) {
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
}

template <bool TA, bool TB, int EDGE, class T, bool SPLIT, int EPI>
__global__ __launch_bounds__(NT, T::OCC) void gemm_bf16_kernel(GemmParams p) {
    constexpr int BM = T::BM, BN = T::BN, TM = T::TM, TN = T::TN, WGN = T::WGN;
    constexpr bool AK = !TA, BKF = TB;
    using OA = Operand<AK, BM>;
    using OB = Operand<BKF, BN>;
    using S = Staging<AK, BKF, T>;
    // SPLIT: each operand tile is followed by its lo tile (split-bf16)
    constexpr int LA = BM * KFB, LB = BN * KFB, NS = SPLIT ? 2 : 1;
    using EA = typename std::conditional<SPLIT, SplitBf16<LA>, __bf16>::type;
    using EB = typename std::conditional<SPLIT, SplitBf16<LB>, __bf16>::type;
    __shared__ __attribute__((aligned(16))) __bf16 ldsA[2][NS * LA];
    __shared__ __attribute__((aligned(16))) __bf16 ldsB[2][NS * LB];

    const TileJob job = tile_job<T>(p);
    if(job.skip) return;
    const int nslices = job.nslices;
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    const int wm = w / WGN, wn = w % WGN;
    const int lr = l & 31, lh = l >> 5;
    const int ar0 = wm * TM * 32, br0 = wn * TN * 32;

    f32x16 acc[TM][TN];
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int j = 0; j < TN; ++j)
#pragma unroll
            for(int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    constexpr int RD = NS * (TM + TN);
    constexpr int NMFMA = (SPLIT ? 3 : 1) * TM * TN;
    constexpr int STAGE_OPS = S::group_ops(0) + S::group_ops(1) + S::group_ops(2);

    if(nslices > 0) {
        f32x4 ra[OA::F4], rb[OB::F4];
        prologue<AK, BKF, EDGE, T, EPI == kEpiSwigluFwd>(p, job, ra, rb, reinterpret_cast<EA*>(ldsA[0]),
                                   reinterpret_cast<EB*>(ldsB[0]));
        __syncthreads();
        // fragments of step 0 / step 1 (and their lo parts when SPLIT)
        bf16x8 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
        bf16x8 la0[SPLIT ? TM : 1], lb0[SPLIT ? TN : 1], la1[SPLIT ? TM : 1], lb1[SPLIT ? TN : 1];
        auto read = [&](const __bf16* ta, const __bf16* tb, int t, bf16x8 (&fa)[TM],
                        bf16x8 (&fb)[TN], bf16x8 (&la)[SPLIT ? TM : 1],
                        bf16x8 (&lb)[SPLIT ? TN : 1]) {
            read_step<TM>(ta, ar0, lr, lh, t, fa);
            read_step<TN>(tb, br0, lr, lh, t, fb);
            if constexpr(SPLIT) {
                read_step<TM>(ta + LA, ar0, lr, lh, t, la);
                read_step<TN>(tb + LB, br0, lr, lh, t, lb);
            }
        };
        // a.b ~ ahi.bhi + ahi.blo + alo.bhi (alo.blo is below 2^-16 of a.b)
        auto mma = [&](const bf16x8 (&fa)[TM], const bf16x8 (&fb)[TN],
                       const bf16x8 (&la)[SPLIT ? TM : 1], const bf16x8 (&lb)[SPLIT ? TN : 1]) {
            mfma_step<TM, TN>(acc, fa, fb);
            if constexpr(SPLIT) {
                mfma_step<TM, TN>(acc, fa, lb);
                mfma_step<TM, TN>(acc, la, fb);
            }
        };
        read(ldsA[0], ldsB[0], 0, fa0, fb0, la0, lb0);
        for(int s = 0; s < nslices; ++s) {
            const int cur = s & 1;
            __bf16* sa = ldsA[cur ^ 1];
            __bf16* sb = ldsB[cur ^ 1];
            const int64_t kn = job.kbeg + (int64_t)min(s + 2, nslices - 1) * BK;
            // step 0: read step 1, stage slice s+1 and fetch s+2
            read(ldsA[cur], ldsB[cur], 1, fa1, fb1, la1, lb1);
            stage<AK, BKF, EDGE, T, 0, EPI == kEpiSwigluFwd>(ra, rb, reinterpret_cast<EA*>(sa), reinterpret_cast<EB*>(sb),
                                       job.A, job.B, p, job.row0, job.col0, kn, job.kend);
            stage<AK, BKF, EDGE, T, 1, EPI == kEpiSwigluFwd>(ra, rb, reinterpret_cast<EA*>(sa), reinterpret_cast<EB*>(sb),
                                       job.A, job.B, p, job.row0, job.col0, kn, job.kend);
            stage<AK, BKF, EDGE, T, 2, EPI == kEpiSwigluFwd>(ra, rb, reinterpret_cast<EA*>(sa), reinterpret_cast<EB*>(sb),
                                       job.A, job.B, p, job.row0, job.col0, kn, job.kend);
            mma(fa0, fb0, la0, lb0);
            interleave<NMFMA, RD + STAGE_OPS>();
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            // step 1, with step 0 of slice s+1 read underneath
            read(sa, sb, 0, fa0, fb0, la0, lb0);
            mma(fa1, fb1, la1, lb1);
            interleave<NMFMA, RD>();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if constexpr(EPI == kEpiPlain)
        store_tile<EDGE, TM, TN>(p, job, acc, ar0, br0, lr, lh);
    else if constexpr(sizeof(ldsA) >= sizeof(ldsB))
        staged_epilogue<EPI, T, sizeof(ldsA) / sizeof(float)>(
            p, job, acc, reinterpret_cast<float*>(&ldsA[0][0]), ar0, br0, lr, lh);
    else
        staged_epilogue<EPI, T, sizeof(ldsB) / sizeof(float)>(
            p, job, acc, reinterpret_cast<float*>(&ldsB[0][0]), ar0, br0, lr, lh);
}

// The same product with fp8 multiplies: op(A) and op(B) are rounded to e4m3
// (after clamping to +-448) on their way to LDS and multiplied by
// v_mfma_f32_32x32x16_fp8_fp8, accumulating in fp32.  Staging, tiles,
// split-K and epilogues are the bf16 kernel's; a lane's 8 k of an MFMA step
// are k 16t + 8*(lane/32) .. +7, read as one 64-bit LDS load.
template <int NB>
__device__ __forceinline__ void read_step8(const unsigned char* lds, int r0, int lr, int lh, int t,
                                           long (&f)[NB]) {
#pragma unroll
    for(int b = 0; b < NB; ++b)
        f[b] = *reinterpret_cast<const long*>(lds + (r0 + b * 32 + lr) * KF8 + 16 * t + 8 * lh);
}

template <bool TA, bool TB, int EDGE, class T, int EPI>
__global__ __launch_bounds__(NT, T::OCC) void gemm_fp8_kernel(GemmParams p) {
    constexpr int BM = T::BM, BN = T::BN, TM = T::TM, TN = T::TN, WGN = T::WGN;
    constexpr bool AK = !TA, BKF = TB;
    using OA = Operand<AK, BM>;
    using OB = Operand<BKF, BN>;
    using S = Staging<AK, BKF, T>;
    constexpr int LA = BM * KF8, LB = BN * KF8;
    // ldsA also stages the epilogue: at least one 32-row block of floats
    constexpr int EPI_BYTES = EPI == kEpiPlain ? 0 : 32 * (BN + 4) * 4;
    constexpr int A_BYTES = 2 * LA > EPI_BYTES ? 2 * LA : EPI_BYTES;
    __shared__ __attribute__((aligned(16))) unsigned char ldsA_buf[A_BYTES];
    __shared__ __attribute__((aligned(16))) unsigned char ldsB[2][LB];
    unsigned char* const ldsA0 = ldsA_buf;
    unsigned char* const ldsA1 = ldsA_buf + LA;

    TileJob job = tile_job<T>(p);
    if(job.skip) return;
    if(threadIdx.x < 2) g_fp8_scale[threadIdx.x] = p.fp8_scale ? p.fp8_scale[threadIdx.x] : 1.0f;
    __syncthreads();
    job.alpha *= 1.0f / (g_fp8_scale[0] * g_fp8_scale[1]);  // powers of two: exact
    const int nslices = job.nslices;
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    const int wm = w / WGN, wn = w % WGN;
    const int lr = l & 31, lh = l >> 5;
    const int ar0 = wm * TM * 32, br0 = wn * TN * 32;

    f32x16 acc[TM][TN];
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int j = 0; j < TN; ++j)
#pragma unroll
            for(int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    constexpr int RD = TM + TN;
    constexpr int NMFMA = TM * TN;
    constexpr int STAGE_OPS = S::group_ops(0) + S::group_ops(1) + S::group_ops(2);

    if(nslices > 0) {
        f32x4 ra[OA::F4], rb[OB::F4];
        prologue<AK, BKF, EDGE, T, EPI == kEpiSwigluFwd>(p, job, ra, rb, reinterpret_cast<Fp8A*>(ldsA0),
                                   reinterpret_cast<Fp8B*>(ldsB[0]));
        __syncthreads();
        long fa0[TM], fb0[TN], fa1[TM], fb1[TN];
        auto mma = [&](const long (&fa)[TM], const long (&fb)[TN]) {
#pragma unroll
            for(int i = 0; i < TM; ++i)
#pragma unroll
                for(int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(fa[i], fb[j], acc[i][j],
                                                                          0, 0, 0);
        };
        read_step8<TM>(ldsA0, ar0, lr, lh, 0, fa0);
        read_step8<TN>(ldsB[0], br0, lr, lh, 0, fb0);
        for(int s = 0; s < nslices; ++s) {
            const int cur = s & 1;
            unsigned char* const la = cur ? ldsA1 : ldsA0;
            unsigned char* const na = cur ? ldsA0 : ldsA1;
            Fp8A* sa = reinterpret_cast<Fp8A*>(na);
            Fp8B* sb = reinterpret_cast<Fp8B*>(ldsB[cur ^ 1]);
            const int64_t kn = job.kbeg + (int64_t)min(s + 2, nslices - 1) * BK;
            // step 0: read step 1, stage slice s+1 and fetch s+2
            read_step8<TM>(la, ar0, lr, lh, 1, fa1);
            read_step8<TN>(ldsB[cur], br0, lr, lh, 1, fb1);
            stage<AK, BKF, EDGE, T, 0, EPI == kEpiSwigluFwd>(ra, rb, sa, sb, job.A, job.B, p, job.row0, job.col0, kn,
                                       job.kend);
            stage<AK, BKF, EDGE, T, 1, EPI == kEpiSwigluFwd>(ra, rb, sa, sb, job.A, job.B, p, job.row0, job.col0, kn,
                                       job.kend);
            stage<AK, BKF, EDGE, T, 2, EPI == kEpiSwigluFwd>(ra, rb, sa, sb, job.A, job.B, p, job.row0, job.col0, kn,
                                       job.kend);
            mma(fa0, fb0);
            interleave<NMFMA, RD + STAGE_OPS>();
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            // step 1, with step 0 of slice s+1 read underneath
            read_step8<TM>(na, ar0, lr, lh, 0, fa0);
            read_step8<TN>(ldsB[cur ^ 1], br0, lr, lh, 0, fb0);
            mma(fa1, fb1);
            interleave<NMFMA, RD>();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if constexpr(EPI == kEpiPlain)
        store_tile<EDGE, TM, TN>(p, job, acc, ar0, br0, lr, lh);
    else
        staged_epilogue<EPI, T, A_BYTES / sizeof(float)>(
            p, job, acc, reinterpret_cast<float*>(ldsA_buf), ar0, br0, lr, lh);
}

// ---- small products ---------------------------------------------------------
// A product whose output is too small to give every CU a tile of the shapes
// above (512^3: 64 tiles of 64x64 for 256 CUs) runs on 32x32 tiles, one per
// workgroup of W waves, with K split between the waves: wave w multiplies the
// tile's 32 rows and 32 columns over its own K range of `kq` (k slices of 32),
// taking its MFMA operands straight from global memory into registers (no LDS
// staging, no barrier in the main loop), D slices in flight.  A lane holds 16
// consecutive k of one row of op(A) and of one column of op(B) per slice --
// the same fragment assignment as the tiled kernel: lanes 0-31 take k 0..15 of
// the slice, lanes 32-63 k 16..31 -- loaded as four 128-bit loads when the
// operand is k-contiguous in memory, else as 16 32-bit loads, each a
// contiguous 128-byte row run across the lanes.  The W partial tiles then meet
// in LDS and are added in wave order (ascending K), so the result is
// deterministic.  Whole tiles only: M, N multiples of 32, K a multiple of
// 32*W*D, operands 16-byte aligned with leading dimensions multiples of 4.
struct SmallParams {
    const float *A, *B, *Cin;
    float* C;
    int64_t lda, ldb, ldc, ldcin;
    int64_t kq;  // K per wave
    float alpha, beta;
    int tiles_m, tiles_n;
};

// One operand's fragment of a slice through a buffer resource over the
// operand: the per-lane byte offset `voff` stays fixed, the slice moves the
// uniform `soff`.  k-contiguous (element (r, k) at base[r*ld + k]): 16
// consecutive floats, four 128-bit loads; row-contiguous (element (r, k) at
// base[k*ld + r]): one float per k row, `step` = ld*4 bytes apart.
template <bool KFAST>
__device__ __forceinline__ void small_frag(__amdgpu_buffer_rsrc_t rs, int voff, int soff, int step,
                                           float (&f)[16]) {
    if(KFAST) {
#pragma unroll
        for(int i = 0; i < 4; ++i) {
            const f32x4 x =
                __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 * i, soff, 0));
            f[4 * i + 0] = x[0];
            f[4 * i + 1] = x[1];
            f[4 * i + 2] = x[2];
            f[4 * i + 3] = x[3];
        }
    } else {
#pragma unroll
        for(int i = 0; i < 16; ++i)
            f[i] = __builtin_bit_cast(float,
                                      __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff + i * step, 0));
    }
}

template <bool TA, bool TB, int W, int D>
__global__ __launch_bounds__(64 * W) void gemm_small_kernel(SmallParams p) {
    __shared__ __attribute__((aligned(16))) float part[W][32 * 32];
    // XCD-contiguous runs of tiles (the dispatcher deals workgroups to the 8
    // XCDs in turn), walked down GROUP_M tile-rows at a time
    const int ntiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
    const int group_span = GROUP_M * p.tiles_n;
    const int first_m = (bid / group_span) * GROUP_M;
    const int gm = min(p.tiles_m - first_m, GROUP_M);
    const int local = bid % group_span;
    const int row0 = (first_m + local % gm) * 32, col0 = (local / gm) * 32;

    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lr = l & 31, lh = l >> 5;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    const int kw = w * (int)p.kq;   // this wave's first k
    const int ns = (int)(p.kq / BK);  // a multiple of D
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.A), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.B), (short)0, 0x7fffffff, 0x00020000);
    // op(A) is k-contiguous unless TA, op(B) unless !TB
    const int va = !TA ? (lr * lda + 16 * lh) * 4 : (16 * lh * lda + lr) * 4;
    const int vb = TB ? (lr * ldb + 16 * lh) * 4 : (16 * lh * ldb + lr) * 4;
    auto fetch = [&](int s, float (&fa)[16], float (&fb)[16]) {
        const int k = kw + s * BK;
        small_frag<!TA>(ra, va, !TA ? (row0 * lda + k) * 4 : (k * lda + row0) * 4, lda * 4, fa);
        small_frag<TB>(rb, vb, TB ? (col0 * ldb + k) * 4 : (k * ldb + col0) * 4, ldb * 4, fb);
    };
    float a[D][16], b[D][16];
#pragma unroll
    for(int d = 0; d < D; ++d) {
        fetch(d, a[d], b[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
    f32x16 acc;
#pragma unroll
    for(int r = 0; r < 16; ++r) acc[r] = 0.0f;
    auto mul = [&](const float (&fa)[16], const float (&fb)[16]) {
#pragma unroll
        for(int i = 0; i < 16; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[i], acc, 0, 0, 0);
    };
    // every slice's buffer is refilled right after its products, D slices
    // ahead, with no condition inside the loop, and the scheduling barriers
    // keep the slices' loads in slice order: the wait-count analysis then
    // knows at the loop head and after it which loads a slice's products
    // wait for (with a conditional refill, or loads of different slices
    // interleaved, it lost that, and every slice waited for all loads in
    // flight); the last D slices refill nothing
    __builtin_amdgcn_sched_barrier(0);
    int s0 = 0;
    for(; s0 + D < ns; s0 += D) {
#pragma unroll
        for(int d = 0; d < D; ++d) {
            mul(a[d], b[d]);
            fetch(s0 + d + D, a[d], b[d]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for(int d = 0; d < D; ++d) mul(a[d], b[d]);
    // partial tile of wave w: C[row][col] with col = lane%32 and row =
    // 8(r/4) + 4(lane/32) + r%4 for accumulator register r
#pragma unroll
    for(int r = 0; r < 16; ++r) part[w][(8 * (r >> 2) + 4 * lh + (r & 3)) * 32 + lr] = acc[r];
    __syncthreads();
    constexpr int PER = 32 * 32 / (64 * W);  // outputs per thread: 4 (W 4) or 2 (W 8)
    const int e0 = threadIdx.x * PER, row = e0 / 32, col = e0 % 32;
    float v[PER];
#pragma unroll
    for(int e = 0; e < PER; ++e) v[e] = part[0][e0 + e];
#pragma unroll
    for(int q = 1; q < W; ++q)
#pragma unroll
        for(int e = 0; e < PER; ++e) v[e] += part[q][e0 + e];
    typedef float vec_t __attribute__((ext_vector_type(PER)));
    vec_t* c = reinterpret_cast<vec_t*>(p.C + (row0 + row) * p.ldc + col0 + col);
    vec_t x;
#pragma unroll
    for(int e = 0; e < PER; ++e) x[e] = p.alpha * v[e];
    if(p.beta != 0.0f) {
        const vec_t y = *reinterpret_cast<const vec_t*>(p.Cin + (row0 + row) * p.ldcin + col0 + col);
#pragma unroll
        for(int e = 0; e < PER; ++e) x[e] += p.beta * y[e];
    }
    *c = x;
}

// The same product for any M, N, K (partial tiles, K not a multiple of the
// slice, unaligned operands): every operand element is one 32-bit load of an
// in-range address, selected to zero outside [0, rows) x [0, K), and wave w
// takes slices w, w + W, w + 2W, ... (one in flight), so every wave has
// ceil or floor of ns/W slices; stores are predicated.  For tiny products (a
// training step of a small MLP: [64, 784] . [784, 128] and smaller), where a
// launch is a few workgroups' latency chain.
template <bool KFAST, bool VEC>
__device__ __forceinline__ void small_frag_edge(__amdgpu_buffer_rsrc_t rs, int ld, int r, int rlim,
                                                int k, int K, float (&f)[16]) {
    const int rr = r < rlim ? r : rlim - 1;  // a valid row; its products are never stored
    if constexpr(KFAST && VEC) {
        // 16-byte aligned rows and K a multiple of 4: four 128-bit loads, each
        // float4 wholly inside or outside [0, K)
#pragma unroll
        for(int i = 0; i < 4; ++i) {
            const bool in = k + 4 * i < K;
            const int off = (rr * ld + (in ? k + 4 * i : 0)) * 4;
            const f32x4 x =
                __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
#pragma unroll
            for(int e = 0; e < 4; ++e) f[4 * i + e] = in ? x[e] : 0.0f;
        }
        return;
    }
#pragma unroll
    for(int i = 0; i < 16; ++i) {
        const bool in = k + i < K;
        const int kk = in ? k + i : 0;
        const int off = KFAST ? (rr * ld + kk) * 4 : (kk * ld + rr) * 4;
        const float x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
        f[i] = in ? x : 0.0f;
    }
}

struct SmallEdgeParams {
    const float *A, *B, *Cin;
    float* C;
    int M, N, K, lda, ldb;
    int64_t ldc, ldcin;
    float alpha, beta;
    int tiles_m, tiles_n;
};

template <bool TA, bool TB, int W, bool VEC>
__global__ __launch_bounds__(64 * W) void gemm_small_edge_kernel(SmallEdgeParams p) {
    __shared__ __attribute__((aligned(16))) float part[W][32 * 32];
    const int tm = blockIdx.x % p.tiles_m, tn = blockIdx.x / p.tiles_m;
    const int row0 = tm * 32, col0 = tn * 32;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, lr = l & 31, lh = l >> 5;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.A), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.B), (short)0, 0x7fffffff, 0x00020000);
    const int ns = (p.K + BK - 1) / BK;
    f32x16 acc;
#pragma unroll
    for(int r = 0; r < 16; ++r) acc[r] = 0.0f;
    for(int s = w; s < ns; s += W) {
        float a[16], b[16];
        const int k = s * BK + 16 * lh;
        small_frag_edge<!TA, VEC>(ra, p.lda, row0 + lr, p.M, k, p.K, a);
        small_frag_edge<TB, VEC>(rb, p.ldb, col0 + lr, p.N, k, p.K, b);
#pragma unroll
        for(int i = 0; i < 16; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[i], acc, 0, 0, 0);
    }
#pragma unroll
    for(int r = 0; r < 16; ++r) part[w][(8 * (r >> 2) + 4 * lh + (r & 3)) * 32 + lr] = acc[r];
    __syncthreads();
    for(int e = threadIdx.x; e < 32 * 32; e += 64 * W) {
        const int row = row0 + e / 32, col = col0 + e % 32;
        if(row >= p.M || col >= p.N) continue;
        float v = part[0][e];
#pragma unroll
        for(int q = 1; q < W; ++q) v += part[q][e];
        float x = p.alpha * v;
        if(p.beta != 0.0f) x += p.beta * p.Cin[row * p.ldcin + col];
        p.C[row * p.ldc + col] = x;
    }
}

// W = 0 when the small-product kernel does not apply
struct SmallChoice {
    int W, D;
};

// Whether a product goes to the small-product kernels: the tiled kernels'
// choice leaves CUs without a tile, at most one round of 32x32 tiles covers
// the output, and each operand spans under 2^31 bytes (32-bit offsets).
bool small_product(int64_t M, int64_t N, int64_t K, bool TA, bool TB, int64_t lda, int64_t ldb);

template <bool TA, bool TB, bool VEC>
void launch_small_edge_v(const SmallEdgeParams& ep, hipStream_t st) {
    const unsigned grid = (unsigned)(ep.tiles_m * ep.tiles_n);
    // sixteen waves when there are twelve or more slices of 32 k (one or two
    // slices each), else four
    if((ep.K + BK - 1) / BK >= 12)
        gemm_small_edge_kernel<TA, TB, 16, VEC><<<grid, 1024, 0, st>>>(ep);
    else
        gemm_small_edge_kernel<TA, TB, 4, VEC><<<grid, 256, 0, st>>>(ep);
}

// vec: a k-contiguous operand is 16-byte aligned with a row stride and K that
// are multiples of 4, so it loads 128 bits at a time
template <bool TA, bool TB>
void launch_small_edge(const SmallEdgeParams& ep, bool vec, hipStream_t st) {
    if(vec) launch_small_edge_v<TA, TB, true>(ep, st);
    else launch_small_edge_v<TA, TB, false>(ep, st);
}

// The whole-tile kernel's shape (W = 0: the edge kernel instead).  Small
// products are limited to one round of tiles (at most one per CU): with more,
// the 64x64 tiles' LDS staging, which reads each operand once per 64 rows
// instead of once per 32, wins (measured 768^3: 576 small tiles 48-62 TFLOP/s
// against 59-64 tiled; 1024^3: 69-82 against 107-117).  Eight waves split K
// when it divides (512^3: 51-53 TFLOP/s against 40-47 with four, 24-25
// tiled); D = the most slices in flight (4, 2 or 1) that divides a wave's
// slice count.  At K = 1024 sixteen waves of two slices each (512^2 x 1024:
// 70-74 TFLOP/s NN and TN against 60-65 with eight; at K = 512 sixteen waves
// of one slice measured 2-5 % slower than eight).
SmallChoice small_choice(int64_t M, int64_t N, int64_t K) {
    if(M % 32 || N % 32 || K <= 0) return {0, 0};
    if(K == BK * 16 * 2) return {16, 2};
    const int W = K % (BK * 8) == 0 ? 8 : K % (BK * 4) == 0 ? 4 : 0;
    if(!W) return {0, 0};
    const int64_t ns = K / (BK * W);  // odd when W is 4
    return {W, ns % 4 == 0 ? 4 : ns % 2 == 0 ? 2 : 1};
}

template <bool TA, bool TB>
void launch_small(const SmallParams& sp, SmallChoice sc, hipStream_t st) {
    const unsigned grid = (unsigned)(sp.tiles_m * sp.tiles_n);
    if(sc.W == 16) {
        gemm_small_kernel<TA, TB, 16, 2><<<grid, 1024, 0, st>>>(sp);
    } else if(sc.W == 8) {
        if(sc.D == 4) gemm_small_kernel<TA, TB, 8, 4><<<grid, 512, 0, st>>>(sp);
        else if(sc.D == 2) gemm_small_kernel<TA, TB, 8, 2><<<grid, 512, 0, st>>>(sp);
        else gemm_small_kernel<TA, TB, 8, 1><<<grid, 512, 0, st>>>(sp);
    } else {  // four waves: K/128 is odd, one slice in flight
        gemm_small_kernel<TA, TB, 4, 1><<<grid, 256, 0, st>>>(sp);
    }
}

// C = alpha * sum_s ws[s] + beta * Cin, planes summed in order s = 0, 1, ...
__global__ void splitk_reduce(int64_t M, int64_t N, int S, const float* __restrict__ ws,
                              float alpha, float beta, const float* Cin, int64_t ldcin, float* C,
                              int64_t ldc) {
    const int64_t plane = M * N;
    if((N & 3) == 0 && (ldc & 3) == 0 && (ldcin & 3) == 0 &&
       (reinterpret_cast<uintptr_t>(C) & 15) == 0 && (reinterpret_cast<uintptr_t>(Cin) & 15) == 0) {
        const int64_t n4 = plane / 4, N4 = N / 4;
        for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
            i += (int64_t)gridDim.x * blockDim.x) {
            f32x4 acc = reinterpret_cast<const f32x4*>(ws)[i];
            for(int s = 1; s < S; ++s) acc += reinterpret_cast<const f32x4*>(ws + s * plane)[i];
            f32x4 v = alpha * acc;
            if(beta != 0.0f) v += beta * reinterpret_cast<const f32x4*>(Cin + (i / N4) * ldcin)[i % N4];
            reinterpret_cast<f32x4*>(C + (i / N4) * ldc)[i % N4] = v;
        }
        return;
    }
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < plane;
        i += (int64_t)gridDim.x * blockDim.x) {
        float acc = ws[i];
        for(int s = 1; s < S; ++s) acc += ws[s * plane + i];
        float v = alpha * acc;
        if(beta != 0.0f) v += beta * Cin[(i / N) * ldcin + (i % N)];
        C[(i / N) * ldc + (i % N)] = v;
    }
}

// Tile shape: the estimated time of a shape is the work of the busiest CU --
// its share of the tiles, ceil(tiles / 256 CUs), times the work of one tile in
// units of a 128x128 tile (256x256: 4, 256x96: 1.5, 128x96: 0.75, 64x64:
// 0.25).  Workgroups resident on one CU share its matrix pipes, and a CU with
// no tile adds nothing.  The one-per-CU shapes (256x256, 256x96) run their
// MFMAs about 5 % more efficiently (measured 1-5 % for 256x96 against 128x96
// at [8192, 768] and [8192, 2304], K 768-4096); 64x64 tiles move twice the
// operand bytes per FLOP of 128x128 ones and are charged 20 % for it.
// Examples: 4096^2 -> 256 tiles of 256x256; an [8192, 768] output (every
// projection of a d_model-768 transformer) -> 256 of 256x96; 2048^2 -> 256
// of 128x128; 1024^2 -> 256 of 64x64 rather than 64 of 128x128.
enum TileKind { kTile128, kTile96, kTile256, kTile64, kTile256x96 };

struct TileChoice {
    TileKind kind;
    int bm, bn;
};

// pair_F > 0 (the SwiGLU-forward product): only shapes whose half width
// divides pair_F, so every tile holds whole gate/up column pairs; bm = 0 when
// none does.
TileChoice pick_tile(int64_t M, int64_t N, int64_t batch, bool allow_all, int64_t pair_F = 0) {
    auto cost = [&](int bm, int bn, double units) {
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch;
        return units * (double)((tiles + kCUs - 1) / kCUs);
    };
    auto fits = [&](int bn) { return pair_F == 0 || pair_F % (bn / 2) == 0; };
    TileChoice best = {kTile128, 128, 128};
    double c = fits(128) ? cost(128, 128, 1.0) : 1e300;
    if(!fits(128)) best.bm = 0;
    auto consider = [&](TileKind k, int bm, int bn, double ck) {
        if(ck < c) {
            c = ck;
            best = {k, bm, bn};
        }
    };
    if(N % 96 == 0 && fits(96)) consider(kTile96, 128, 96, cost(128, 96, 0.75));
    if(allow_all) {
        if(fits(64)) consider(kTile64, 64, 64, cost(64, 64, 0.25) * 1.2);
        if(N % 96 == 0 && fits(96) && cost(256, 96, 1.5) / 1.05 <= c) {
            c = cost(256, 96, 1.5) / 1.05;
            best = {kTile256x96, 256, 96};
        }
        if(fits(256) && cost(256, 256, 4.0) / 1.05 <= c) best = {kTile256, 256, 256};
    }
    return best;
}

bool small_product(int64_t M, int64_t N, int64_t K, bool TA, bool TB, int64_t lda, int64_t ldb) {
    if(((M + 31) / 32) * ((N + 31) / 32) > kCUs) return false;
    const TileChoice t = pick_tile(M, N, 1, true);
    if(((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) >= kCUs) return false;
    auto extent = [K](bool kfast, int64_t rows, int64_t ld) {
        return 4 * (kfast ? (rows - 1) * ld + K : (K - 1) * ld + rows);
    };
    return lda < INT32_MAX && ldb < INT32_MAX && extent(!TA, M, lda) < INT32_MAX &&
           extent(TB, N, ldb) < INT32_MAX;
}

// K split for a product whose output has too few tiles to fill the chip: 2
// resident workgroups per CU x 256 CUs want >= 512 workgroups.
//  * K >= 1024 (weight gradients: M, N ~ d_model, K = tokens): slices of at
//    least 256 (8 LDS stages).  The split count minimises the estimated time
//    in units of one 32-deep stage over a full round of 512 workgroups of
//    128x128 tiles (~3.9 us):
//        rounds x (stages per split + 2.5 for a workgroup's prologue and
//        epilogue) + (s + 1) planes of M*N floats for the reduction (~19.5 MB
//        of HBM traffic per unit).
//    A second round of workgroups can beat one round that leaves slots idle:
//    a [768, 4096] gradient with K = 8192 (192 tiles) takes 8 splits (three
//    rounds of 32 stages) rather than 2 (one round of 128 stages, 384 of 512
//    slots busy).  [768, 768] takes 14 and [768, 2048] 5.
//  * 512 <= K < 1024: only when even 64x64 tiles would leave three quarters
//    of the CUs idle (the MLP's [64, 784] . [784, 128]: 2 tiles); slices of
//    at least 128, which turns one latency-bound workgroup chain into six.
//    Wider outputs take the 64x64 tiles instead.
//  * K < 512: never.
//  * K < 4096 and the unsplit tile choice already gives every CU a tile
//    (2048^2: 256 tiles of 128x128; 1024^2: 256 of 64x64): never.  The split
//    adds a second workgroup per CU but not its throughput, and pays for the
//    reduction (measured best of three: 2048^3 130 TF/s unsplit against 122
//    with 2 splits; 1024^3 82 against 72 with 4).  Longer K keeps splitting:
//    [768, 2304] with K = 8192 (432 tiles of 64x64) runs at 97 TF/s unsplit
//    and 109-115 split.
//  * K >= 4096, op(A) not transposed (NN, NT: a training step's forward and
//    input-gradient products, on its critical stream), fp32 and at least two
//    64x64 tiles per CU: never.  Those run unsplit with the two-slice staging and
//    no reduction pass (config 4's LM-head input gradient [4096, 512] with
//    K 8192: step 1.78-1.80 against 1.82-1.84 ms).  A^T.B products (weight
//    gradients, which a training step runs beside other work) keep splitting:
//    their shorter split workgroups share the CUs better ([768, 4096] unsplit
//    cost a config-5 step 1 ms).
constexpr int64_t kSplitTarget = 512, kMinSplitK = 512;

int choose_splits(int64_t M, int64_t N, int64_t K, bool ta, bool fp32, int64_t* kchunk) {
    const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
    *kchunk = K;
    if(tiles <= 0 || tiles * 2 > kSplitTarget || K < kMinSplitK) return 1;
    if(K < 1024 && ((M + 63) / 64) * ((N + 63) / 64) * 4 >= 256) return 1;
    if(K < 4096) {
        const TileChoice t = pick_tile(M, N, 1, true);
        if(((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) >= kCUs) return 1;
    } else if(!ta && fp32 && ((M + 63) / 64) * ((N + 63) / 64) >= 2 * kCUs) {
        return 1;
    }
    const int64_t min_slice = K >= 1024 ? 256 : 128;
    int64_t s_max = K / min_slice;
    if(s_max > 64) s_max = 64;
    int64_t best_s = 1;
    double best = -1.0;
    const double plane = (double)M * (double)N * 4.0 / 19.5e6;
    for(int64_t s = 1; s <= s_max; ++s) {
        const int64_t chunk = ((K + s - 1) / s + BK - 1) / BK * BK;
        const int64_t splits = (K + chunk - 1) / chunk;
        const int64_t rounds = (tiles * splits + kSplitTarget - 1) / kSplitTarget;
        const double cost = (double)rounds * ((double)(chunk / BK) + 2.5) +
                            (splits > 1 ? (double)(splits + 1) * plane : 0.0);
        if(best < 0.0 || cost < best) {
            best = cost;
            best_s = s;
        }
    }
    if(best_s < 2) return 1;
    const int64_t chunk = ((K + best_s - 1) / best_s + BK - 1) / BK * BK;
    *kchunk = chunk;
    return (int)((K + chunk - 1) / chunk);
}

enum Precision { kFp32 = 0, kBf16 = 1, kBf16x3 = 2, kFp8 = 3 };

template <bool TA, bool TB, class T, int EDGE, int EPI>
void launch_epi(const GemmParams& gp, dim3 grid, int prec, hipStream_t st) {
    if(prec == kFp8)
        gemm_fp8_kernel<TA, TB, EDGE, T, EPI><<<grid, NT, 0, st>>>(gp);
    else if(prec == kBf16)
        gemm_bf16_kernel<TA, TB, EDGE, T, false, EPI><<<grid, NT, 0, st>>>(gp);
    else if(prec == kBf16x3)
        gemm_bf16_kernel<TA, TB, EDGE, T, true, EPI><<<grid, NT, 0, st>>>(gp);
    else if constexpr(deep_staging<T>()) {
        // unsplit products of the small tiles stage two slices ahead; a split
        // product (weight gradients, concurrent with other work) keeps the
        // smaller register footprint, which lets more of that work share its
        // CUs (a config-5 step measured 0.5 ms slower with both deep)
        if(gp.splits == 1)
            gemm_f32_kernel<TA, TB, EDGE, T, EPI, true><<<grid, NT, 0, st>>>(gp);
        else
            gemm_f32_kernel<TA, TB, EDGE, T, EPI><<<grid, NT, 0, st>>>(gp);
    } else {
        gemm_f32_kernel<TA, TB, EDGE, T, EPI><<<grid, NT, 0, st>>>(gp);
    }
}

// The staged epilogues are instantiated only where they are used: the
// residual add and the SwiGLU forward for 'N','N' (x + a.W, x.[W1 | W3]), the
// SwiGLU backward for 'N','T' (dY . W2^T); gemm_impl refuses other
// combinations.
template <bool TA, bool TB, class T, int EDGE>
void launch_kernel(const GemmParams& gp, dim3 grid, int prec, hipStream_t st) {
    if constexpr(!TA && TB) {
        if(gp.sg_a) return launch_epi<TA, TB, T, EDGE, kEpiSwiglu>(gp, grid, prec, st);
    }
    if constexpr(!TA && !TB) {
        if(gp.sf_h) return launch_epi<TA, TB, T, EDGE, kEpiSwigluFwd>(gp, grid, prec, st);
        if(gp.Cin) return launch_epi<TA, TB, T, EDGE, kEpiAdd>(gp, grid, prec, st);
    }
    launch_epi<TA, TB, T, EDGE, kEpiPlain>(gp, grid, prec, st);
}

template <bool TA, bool TB, class T>
int launch_tile(const GemmParams& gp, int64_t batch, int edge, int prec, hipStream_t st) {
    dim3 grid((unsigned)(gp.tiles_m * gp.tiles_n), (unsigned)(gp.splits > 1 ? gp.splits : batch));
    if(edge == kEdgeNone)
        launch_kernel<TA, TB, T, kEdgeNone>(gp, grid, prec, st);
    else if(edge == kEdgeVec)
        launch_kernel<TA, TB, T, kEdgeVec>(gp, grid, prec, st);
    else
        launch_kernel<TA, TB, T, kEdgeScalar>(gp, grid, prec, st);
    return pk::launch_status(prec == kBf16     ? "pk_gemm_bf16_f32"
                             : prec == kBf16x3 ? "pk_gemm_bf16x3_f32"
                             : prec == kFp8    ? "pk_gemm_fp8_f32"
                                               : "pk_gemm_f32");
}

template <bool TA, bool TB>
int launch(const GemmParams& gp, int64_t batch, int edge, TileKind kind, int prec,
           hipStream_t st) {
    switch(kind) {
    case kTile256: return launch_tile<TA, TB, Tile256>(gp, batch, edge, prec, st);
    case kTile256x96: return launch_tile<TA, TB, Tile256x96>(gp, batch, edge, prec, st);
    case kTile96: return launch_tile<TA, TB, Tile96>(gp, batch, edge, prec, st);
    case kTile64: return launch_tile<TA, TB, Tile64>(gp, batch, edge, prec, st);
    default: return launch_tile<TA, TB, Tile128>(gp, batch, edge, prec, st);
    }
}

// what a product's tiles write besides alpha * op(A) . op(B): the beta term's
// source when it is not C, or the SwiGLU-backward epilogue
struct Epilogue {
    const float* fp8_scale = nullptr;
    const float* Cin = nullptr;
    int64_t ldcin = 0;
    const float *sg_a = nullptr, *sg_u = nullptr;
    float *sg_da = nullptr, *sg_du = nullptr;
    int64_t sg_lda = 0, sg_ldu = 0, sg_ldd = 0;
    int sg_flags = 0;
    float* sf_h = nullptr;  // SwiGLU forward: h [M, N/2]
    int64_t sf_ldh = 0;
};

int gemm_impl(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
              int64_t lda, int64_t sA_outer, int64_t sA_inner, const float* B, int64_t ldb,
              int64_t sB_outer, int64_t sB_inner, float beta, float* C, int64_t ldc,
              int64_t sC_outer, int64_t sC_inner, int64_t batch, int64_t inner_count, int causal,
              float* ws, size_t ws_bytes, int prec, pk_stream_t stream,
              const Epilogue& epi = Epilogue()) {
    const bool TA = ta == 'T' || ta == 't', TB = tb == 'T' || tb == 't';
    if(!(TA || ta == 'N' || ta == 'n') || !(TB || tb == 'N' || tb == 'n'))
        return pk::fail("pk_gemm_f32: transpose flags must be 'N' or 'T' (got '%c','%c')", ta, tb);
    if(M < 0 || N < 0 || K < 0 || batch < 0)
        return pk::fail("pk_gemm_f32: negative size M=%lld N=%lld K=%lld batch=%lld",
                        (long long)M, (long long)N, (long long)K, (long long)batch);
    if(causal < 0 || causal > 3) return pk::fail("pk_gemm_f32: causal mode %d not in 0..3", causal);
    if(inner_count < 1) return pk::fail("pk_gemm_f32: inner_count must be >= 1");
    if(M == 0 || N == 0 || batch == 0) return PK_OK;
    const bool swiglu = epi.sg_a != nullptr, sfwd = epi.sf_h != nullptr;
    if(!C && !swiglu) return pk::fail("pk_gemm_f32: C is NULL");
    if(K > 0 && (!A || !B)) return pk::fail("pk_gemm_f32: A or B is NULL");
    const int64_t a_cols = TA ? M : K, b_cols = TB ? K : N;
    if(K > 0 && (lda < a_cols || ldb < b_cols))
        return pk::fail("pk_gemm_f32: leading dimension too small (lda=%lld needs >= %lld, "
                        "ldb=%lld needs >= %lld)",
                        (long long)lda, (long long)a_cols, (long long)ldb, (long long)b_cols);
    if(!swiglu && ldc < N)
        return pk::fail("pk_gemm_f32: ldc=%lld < N=%lld", (long long)ldc, (long long)N);
    if(batch > 65535) return pk::fail("pk_gemm_f32: problem too large for one launch");

    GemmParams gp;
    gp.A = A;
    gp.B = B;
    gp.C = C;
    gp.M = M;
    gp.N = N;
    gp.K = K;
    gp.lda = lda;
    gp.ldb = ldb;
    gp.ldc = ldc;
    gp.sAo = sA_outer;
    gp.sAi = sA_inner;
    gp.sBo = sB_outer;
    gp.sBi = sB_inner;
    gp.sCo = sC_outer;
    gp.sCi = sC_inner;
    gp.inner = inner_count;
    gp.alpha = alpha;
    gp.beta = beta;
    gp.causal = causal;
    // a beta source that is C itself is the plain accumulate
    const bool own_c = epi.Cin == nullptr || (epi.Cin == C && epi.ldcin == ldc) || beta == 0.0f;
    if(!own_c && (TA || TB))
        return pk::fail("pk_gemm_add_f32: a separate X is built for the ('N','N') layout only");
    if(swiglu && (TA || !TB))
        return pk::fail("pk_gemm_swiglu_bwd_f32: only the ('N','T') layout (dY . W^T) is built");
    gp.Cin = own_c ? nullptr : epi.Cin;
    gp.ldcin = own_c ? 0 : epi.ldcin;
    gp.sg_a = epi.sg_a;
    gp.sg_u = epi.sg_u;
    gp.sg_da = epi.sg_da;
    gp.sg_du = epi.sg_du;
    gp.sg_lda = epi.sg_lda;
    gp.sg_ldu = epi.sg_ldu;
    gp.sg_ldd = epi.sg_ldd;
    gp.sg_flags = epi.sg_flags;
    gp.fp8_scale = prec == kFp8 ? epi.fp8_scale : nullptr;
    gp.pair_F = 0;
    gp.sf_h = nullptr;
    gp.sf_ldh = 0;
    if(sfwd) {
        if(TA || TB || batch != 1 || causal != 0 || beta != 0.0f || !own_c)
            return pk::fail("pk_gemm_swiglu_fwd_f32: only the plain ('N','N') product is built");
        if(N % 8 != 0)
            return pk::fail("pk_gemm_swiglu_fwd_f32: N=%lld must be 2F with F a multiple of 4",
                            (long long)N);
        if(epi.sf_ldh < N / 2)
            return pk::fail("pk_gemm_swiglu_fwd_f32: ldh=%lld < F=%lld", (long long)epi.sf_ldh,
                            (long long)(N / 2));
        gp.pair_F = N / 2;
        gp.sf_h = epi.sf_h;
        gp.sf_ldh = epi.sf_ldh;
    }
    hipStream_t st = pk::as_stream(stream);
    // an output that the tiled kernels leave short of one tile per CU, with
    // K <= 1024: the small-product kernels, before any K split is considered
    // (a split of such a product is a few workgroups' latency chain plus a
    // reduction pass; longer K, such as a weight gradient over a batch of
    // tokens, keeps the tiled kernels and their split)
    if(prec == kFp32 && batch == 1 && causal == 0 && !swiglu && !sfwd && K > 0 && K <= 1024 &&
       small_product(M, N, K, TA, TB, lda, ldb)) {
        const bool vec = pk::aligned16(A) && pk::aligned16(B) && lda % 4 == 0 && ldb % 4 == 0 &&
                         pk::aligned16(C) && ldc % 4 == 0 &&
                         (gp.Cin == nullptr || (pk::aligned16(gp.Cin) && gp.ldcin % 4 == 0));
        const SmallChoice sc = vec ? small_choice(M, N, K) : SmallChoice{0, 0};
        if(sc.W) {
            SmallParams sp;
            sp.A = A;
            sp.B = B;
            sp.C = C;
            sp.Cin = gp.Cin ? gp.Cin : C;
            sp.lda = lda;
            sp.ldb = ldb;
            sp.ldc = ldc;
            sp.ldcin = gp.Cin ? gp.ldcin : ldc;
            sp.kq = K / sc.W;
            sp.alpha = alpha;
            sp.beta = beta;
            sp.tiles_m = (int)(M / 32);
            sp.tiles_n = (int)(N / 32);
            if(!TA && !TB) launch_small<false, false>(sp, sc, st);
            else if(!TA && TB) launch_small<false, true>(sp, sc, st);
            else if(TA && !TB) launch_small<true, false>(sp, sc, st);
            else launch_small<true, true>(sp, sc, st);
        } else {
            SmallEdgeParams ep;
            ep.A = A;
            ep.B = B;
            ep.C = C;
            ep.Cin = gp.Cin ? gp.Cin : C;
            ep.M = (int)M;
            ep.N = (int)N;
            ep.K = (int)K;
            ep.lda = (int)lda;
            ep.ldb = (int)ldb;
            ep.ldc = ldc;
            ep.ldcin = gp.Cin ? gp.ldcin : ldc;
            ep.alpha = alpha;
            ep.beta = beta;
            ep.tiles_m = (int)((M + 31) / 32);
            ep.tiles_n = (int)((N + 31) / 32);
            // the k-contiguous operands (op(A) unless TA, op(B) if TB) may load
            // 128 bits at a time
            const bool kvec = K % 4 == 0 && (TA || (pk::aligned16(A) && lda % 4 == 0)) &&
                              (!TB || (pk::aligned16(B) && ldb % 4 == 0));
            if(!TA && !TB) launch_small_edge<false, false>(ep, kvec, st);
            else if(!TA && TB) launch_small_edge<false, true>(ep, kvec, st);
            else if(TA && !TB) launch_small_edge<true, false>(ep, kvec, st);
            else launch_small_edge<true, true>(ep, kvec, st);
        }
        return pk::launch_status("pk_gemm_f32 (small product)");
    }
    gp.splits = 1;
    gp.kchunk = K;
    gp.ws = nullptr;
    if(batch == 1 && causal == 0 && ws && K > 0 && !swiglu && !sfwd) {
        int64_t kchunk;
        const int S = choose_splits(M, N, K, TA, prec == kFp32, &kchunk);
        if(S > 1 && ws_bytes >= (size_t)S * (size_t)M * (size_t)N * sizeof(float)) {
            gp.splits = S;
            gp.kchunk = kchunk;
            gp.ws = ws;
        }
    }
    auto v4 = [](const void* q, int64_t ld) {
        return q == nullptr || (pk::aligned16(q) && ld % 4 == 0);
    };
    gp.epi_vec = v4(C, ldc) && v4(gp.Cin, gp.ldcin) && v4(gp.sg_a, gp.sg_lda) &&
                 v4(gp.sg_u, gp.sg_ldu) && v4(gp.sg_da, gp.sg_ldd) && v4(gp.sg_du, gp.sg_ldd) &&
                 v4(gp.sf_h, gp.sf_ldh) && (gp.splits == 1 || v4(gp.ws, N));
    // split products keep 128x128 tiles (the split count is sized for them);
    // causal products keep 128-row tiles (the attention chain's diagonal logic
    // is exercised at that size)
    TileChoice tc = gp.splits > 1 ? TileChoice{kTile128, 128, 128}
                                  : pick_tile(M, N, batch, causal == 0, gp.pair_F);
    // a short K over two or more rounds of 256x256 tiles (fp32, unsplit):
    // 128x128 tiles with the two-slice staging, two per CU, where one tile's
    // C stores and first loads overlap the other's products.  Measured in the
    // config-5 forward (the SwiGLU-forward [8192, 4096] and LM-head [8192,
    // 32000] products, K 768) and config 4's LM head ([4096, 8192], K 512):
    // config-5 step 46.36-46.44 -> 46.16-46.23 ms on one box, 47.48-47.56 ->
    // 47.40-47.46 on another.  One round (4096^2) and long K (8192^3) keep
    // 256x256.
    if(prec == kFp32 && gp.splits == 1 && tc.kind == kTile256 && K <= 1024 &&
       ((M + 255) / 256) * ((N + 255) / 256) * batch > kCUs &&
       (gp.pair_F == 0 || gp.pair_F % 64 == 0))
        tc = TileChoice{kTile128, 128, 128};
    // A.B products on 256x96 tiles (one per CU) take 128x96 (two per CU,
    // two-slice staging), so one tile's start and C writes overlap the other's
    // products.  In a training step the A.B products are the forward's, which
    // run alone: config 5's Q/K/V projection 213 -> 207 us, the residual-add
    // products 81 -> 76 us (K 768) and 184 -> 180 us (K 2048), step 46.63-46.67
    // -> 46.36-46.39 ms.  A.B^T and A^T.B keep 256x96: the backward runs them
    // beside the weight-gradient stream, where 128x96 cost the step 0.75 ms.
    if(prec == kFp32 && gp.splits == 1 && tc.kind == kTile256x96 && !TA && !TB)
        tc = TileChoice{kTile96, 128, 96};
    if(tc.bm == 0)
        return pk::fail("pk_gemm_swiglu_fwd_f32: F=%lld is not a multiple of 32 (no tile holds "
                        "whole gate/up column pairs)", (long long)gp.pair_F);
    const int64_t tiles_m = (M + tc.bm - 1) / tc.bm, tiles_n = (N + tc.bn - 1) / tc.bn;
    if(tiles_m * tiles_n > (int64_t)1 << 30)
        return pk::fail("pk_gemm_f32: problem too large for one launch");
    gp.tiles_m = (int)tiles_m;
    gp.tiles_n = (int)tiles_n;
    // float4 loads need 16-byte aligned operands and leading dimensions and
    // batch strides that are multiples of 4; the unchecked path also needs
    // whole tiles
    const bool vec = (lda % 4) == 0 && (ldb % 4) == 0 && (sA_outer % 4) == 0 &&
                     (sA_inner % 4) == 0 && (sB_outer % 4) == 0 && (sB_inner % 4) == 0 &&
                     pk::aligned16(A) && pk::aligned16(B);
    const bool whole = (M % tc.bm) == 0 && (N % tc.bn) == 0 && (K % BK) == 0;
    // whole tiles load through buffer resources with 32-bit offsets from each
    // operand's start: op(A) and op(B) must each span less than 2^31 bytes
    auto extent = [K](bool kfast, int64_t rows, int64_t ld) {
        return 4 * (kfast ? (rows - 1) * ld + K : (K - 1) * ld + rows);
    };
    const bool small = extent(!TA, M, lda) < INT32_MAX && extent(TB, N, ldb) < INT32_MAX;
    const int edge = vec && whole && small ? kEdgeNone
                     : vec && (M % 4) == 0 && (N % 4) == 0 && (K % 4) == 0 ? kEdgeVec
                                                                           : kEdgeScalar;
    const TileKind kind = tc.kind;
    int rc;
    if(!TA && !TB)
        rc = launch<false, false>(gp, batch, edge, kind, prec, st);
    else if(!TA && TB)
        rc = launch<false, true>(gp, batch, edge, kind, prec, st);
    else if(TA && !TB)
        rc = launch<true, false>(gp, batch, edge, kind, prec, st);
    else
        rc = launch<true, true>(gp, batch, edge, kind, prec, st);
    if(rc || gp.splits == 1) return rc;
    splitk_reduce<<<pk::grid_for(M * N / 4 + 1, NT), NT, 0, st>>>(
        M, N, gp.splits, gp.ws, alpha, beta, gp.Cin ? gp.Cin : C, gp.Cin ? gp.ldcin : ldc, C, ldc);
    return pk::launch_status("pk_gemm_ex_f32 (split-K reduction)");
}

}  // namespace

extern "C" int pk_gemm_small_product_f32(int64_t M, int64_t N, int64_t K) {
    return M > 0 && N > 0 && K > 0 && K <= 1024 && small_product(M, N, K, false, false, K, N);
}

extern "C" int pk_gemm_batched_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                                   const float* A, int64_t lda, int64_t sA_outer, int64_t sA_inner,
                                   const float* B, int64_t ldb, int64_t sB_outer, int64_t sB_inner,
                                   float beta, float* C, int64_t ldc, int64_t sC_outer,
                                   int64_t sC_inner, int64_t batch, int64_t inner_count,
                                   int causal, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, sA_outer, sA_inner, B, ldb, sB_outer,
                     sB_inner, beta, C, ldc, sC_outer, sC_inner, batch, inner_count, causal,
                     nullptr, 0, kFp32, stream);
}

extern "C" int pk_gemm_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                           const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                           float* C, int64_t ldc, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, nullptr, 0, kFp32, stream);
}

// the split-K partials of op(A) . op(B) for one layout of A
static size_t gemm_workspace(int64_t M, int64_t N, int64_t K, bool ta) {
    if(M <= 0 || N <= 0 || K <= 0) return 0;
    int64_t kchunk;
    const int S = choose_splits(M, N, K, ta, true, &kchunk);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// any layout: A^T.B splits whenever another layout of the shape does
extern "C" size_t pk_gemm_workspace_f32(int64_t M, int64_t N, int64_t K) {
    return gemm_workspace(M, N, K, true);
}

extern "C" int pk_gemm_ex_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                              const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                              float* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                              pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, static_cast<float*>(workspace), workspace_bytes, kFp32, stream);
}

extern "C" int pk_gemm_bf16_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                                const float* A, int64_t lda, const float* B, int64_t ldb,
                                float beta, float* C, int64_t ldc, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, nullptr, 0, kBf16, stream);
}

extern "C" int pk_gemm_ex_bf16_f32(char ta, char tb, int64_t M, int64_t N, int64_t K,
                                   float alpha, const float* A, int64_t lda, const float* B,
                                   int64_t ldb, float beta, float* C, int64_t ldc,
                                   void* workspace, size_t workspace_bytes, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, static_cast<float*>(workspace), workspace_bytes, kBf16, stream);
}

extern "C" int pk_gemm_bf16x3_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                                  const float* A, int64_t lda, const float* B, int64_t ldb,
                                  float beta, float* C, int64_t ldc, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, nullptr, 0, kBf16x3, stream);
}

extern "C" int pk_gemm_ex_bf16x3_f32(char ta, char tb, int64_t M, int64_t N, int64_t K,
                                     float alpha, const float* A, int64_t lda, const float* B,
                                     int64_t ldb, float beta, float* C, int64_t ldc,
                                     void* workspace, size_t workspace_bytes, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, static_cast<float*>(workspace), workspace_bytes, kBf16x3, stream);
}

extern "C" int pk_gemm_fp8_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                               const float* A, int64_t lda, const float* B, int64_t ldb,
                               float beta, float* C, int64_t ldc, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, nullptr, 0, kFp8, stream);
}

extern "C" int pk_gemm_ex_fp8_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                                  const float* A, int64_t lda, const float* B, int64_t ldb,
                                  float beta, float* C, int64_t ldc, void* workspace,
                                  size_t workspace_bytes, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, static_cast<float*>(workspace), workspace_bytes, kFp8, stream);
}

// ---- fp8 operand scales -------------------------------------------------------
namespace {
__global__ void fp8_scale_zero(unsigned* bits) {
    if(threadIdx.x < 2) bits[threadIdx.x] = 0u;
}

// max |x| over matrix blockIdx.y (0: A, 1: B), as the bits of a non-negative
// float (their unsigned order is the float order); NaNs are ignored
__global__ void fp8_scale_amax(int64_t ra, int64_t ca, const float* __restrict__ A, int64_t lda,
                               int64_t rb, int64_t cb, const float* __restrict__ B, int64_t ldb,
                               unsigned* bits) {
    __shared__ float red[NT / 64];
    const bool isb = blockIdx.y == 1;
    const int64_t rows = isb ? rb : ra, cols = isb ? cb : ca, ld = isb ? ldb : lda;
    const float* x = isb ? B : A;
    float m = 0.0f;
    for(int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < rows * cols;
        i += (int64_t)gridDim.x * NT)
        m = fmaxf(m, fabsf(x[(i / cols) * ld + i % cols]));
    m = pk::block_max<NT / 64>(m, red);
    if(threadIdx.x == 0 && m > 0.0f) atomicMax(bits + blockIdx.y, __float_as_uint(m));
}

// scale = 2^floor(log2(448 / amax)): the largest power of two that keeps
// amax * scale within e4m3's finite range; 1 for an all-zero or non-finite
// amax.  The exponent is held to [-kFp8ScaleExp, kFp8ScaleExp], so each scale,
// the product of two and its reciprocal (the kernel's alpha / (sA * sB)) stay
// finite normals: below amax ~ 5e-17 (448 * 2^-63) the operand is scaled by
// 2^63 only, above ~ 4e21 by 2^-63 only (and saturates at +-448).
constexpr float kFp8ScaleExp = 63.0f;
__global__ void fp8_scale_finish(unsigned* bits) {
    if(threadIdx.x >= 2) return;
    const float a = __uint_as_float(bits[threadIdx.x]);
    float sc = 1.0f;
    if(a > 0.0f && a <= 3.0e38f) {
        // a = m * 2^E with m in [0.5, 1) (subnormal a included) and 448 =
        // 0.875 * 2^9, so a * 2^s <= 448 for s = 9 - E when m <= 0.875 and
        // 8 - E otherwise, and not for s + 1: exact, no logarithm or 448 / a
        int E;
        const float m = frexpf(a, &E);
        const float s = (float)((m <= 0.875f ? 9 : 8) - E);
        sc = ldexpf(1.0f, (int)fminf(fmaxf(s, -kFp8ScaleExp), kFp8ScaleExp));
    }
    reinterpret_cast<float*>(bits)[threadIdx.x] = sc;
}
}  // namespace

extern "C" int pk_fp8_scales_f32(int64_t ra, int64_t ca, const float* A, int64_t lda, int64_t rb,
                                 int64_t cb, const float* B, int64_t ldb, float* scales,
                                 pk_stream_t stream) {
    if(ra < 0 || ca < 0 || rb < 0 || cb < 0)
        return pk::fail("pk_fp8_scales_f32: negative size");
    if(!scales) return pk::fail("pk_fp8_scales_f32: scales is NULL");
    if((ra * ca > 0 && (!A || lda < ca)) || (rb * cb > 0 && (!B || ldb < cb)))
        return pk::fail("pk_fp8_scales_f32: NULL matrix or row stride below its columns");
    hipStream_t st = pk::as_stream(stream);
    unsigned* bits = reinterpret_cast<unsigned*>(scales);
    fp8_scale_zero<<<1, 64, 0, st>>>(bits);
    const int64_t most = ra * ca > rb * cb ? ra * ca : rb * cb;
    if(most > 0)
        fp8_scale_amax<<<dim3(pk::grid_for(most, NT, 1024), 2), NT, 0, st>>>(ra, ca, A, lda, rb, cb,
                                                                           B, ldb, bits);
    fp8_scale_finish<<<1, 64, 0, st>>>(bits);
    return pk::launch_status("pk_fp8_scales_f32");
}

// ---- fused epilogues -------------------------------------------------------
namespace {
int prec_of(int precision, const char* who) {
    if(precision < kFp32 || precision > kFp8)
        return pk::fail("%s: precision %d is not 0 (fp32), 1 (bf16), 2 (bf16x3) or 3 (fp8)", who,
                        precision);
    return precision;
}
}  // namespace

extern "C" int pk_gemm_add_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                               const float* A, int64_t lda, const float* B, int64_t ldb,
                               float beta, const float* X, int64_t ldx, float* C, int64_t ldc,
                               int precision, const float* fp8_scales, void* workspace,
                               size_t workspace_bytes, pk_stream_t stream) {
    const int prec = prec_of(precision, "pk_gemm_add_f32");
    if(prec < 0) return PK_EINVAL;
    Epilogue e;
    e.fp8_scale = fp8_scales;
    if(beta != 0.0f && M > 0 && N > 0) {
        if(!X) return pk::fail("pk_gemm_add_f32: X is NULL");
        // ldx 0: one row of X for every row of C (a bias)
        if(ldx != 0 && ldx < N)
            return pk::fail("pk_gemm_add_f32: ldx=%lld < N=%lld (and not 0)", (long long)ldx,
                            (long long)N);
        e.Cin = X;
        e.ldcin = ldx;
    }
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, static_cast<float*>(workspace), workspace_bytes, prec, stream, e);
}

extern "C" int pk_gemm_swiglu_bwd_f32(char ta, char tb, int64_t M, int64_t N, int64_t K,
                                      float alpha, const float* A, int64_t lda, const float* B,
                                      int64_t ldb, const float* gate, int64_t ldg, const float* up,
                                      int64_t ldu, float* dgate, float* dup, int64_t ldd, int flags,
                                      int precision, const float* fp8_scales, pk_stream_t stream) {
    const int prec = prec_of(precision, "pk_gemm_swiglu_bwd_f32");
    if(prec < 0) return PK_EINVAL;
    if(M > 0 && N > 0) {
        if(!gate || !up || !dgate || !dup)
            return pk::fail("pk_gemm_swiglu_bwd_f32: NULL gate, up or gradient pointer");
        if(ldg < N || ldu < N || ldd < N)
            return pk::fail("pk_gemm_swiglu_bwd_f32: a row stride is below N=%lld", (long long)N);
        if(dgate == dup) return pk::fail("pk_gemm_swiglu_bwd_f32: dgate and dup must differ");
    }
    const bool nt = (ta == 'N' || ta == 'n') && (tb == 'T' || tb == 't');
    if(!nt) return pk::fail("pk_gemm_swiglu_bwd_f32: only the ('N','T') layout (dY . W^T) is built");
    Epilogue e;
    e.fp8_scale = fp8_scales;
    e.sg_a = gate;
    e.sg_u = up;
    e.sg_da = dgate;
    e.sg_du = dup;
    e.sg_lda = ldg;
    e.sg_ldu = ldu;
    e.sg_ldd = ldd;
    e.sg_flags = flags & (PK_ACCUM | PK_ACCUM2);
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, 0.0f, nullptr, N, 0, 0, 1,
                     1, 0, nullptr, 0, prec, stream, e);
}

extern "C" int pk_gemm_swiglu_fwd_f32(char ta, char tb, int64_t M, int64_t N, int64_t K,
                                      float alpha, const float* A, int64_t lda, const float* B,
                                      int64_t ldb, float* C, int64_t ldc, float* h, int64_t ldh,
                                      int precision, const float* fp8_scales, pk_stream_t stream) {
    const int prec = prec_of(precision, "pk_gemm_swiglu_fwd_f32");
    if(prec < 0) return PK_EINVAL;
    if(M > 0 && N > 0 && (!C || !h)) return pk::fail("pk_gemm_swiglu_fwd_f32: NULL C or h");
    Epilogue e;
    e.fp8_scale = fp8_scales;
    e.sf_h = h;
    e.sf_ldh = ldh;
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, 0.0f, C, ldc, 0, 0, 1, 1,
                     0, nullptr, 0, prec, stream, e);
}

// ---- pk_gemm_noalloc_f32: the split-K GEMM without a caller workspace ------
// For callers that cannot allocate (code under graph capture, tight serving
// loops): the split-K partial planes go to `scratch`, a file-scope device
// array of kNoAllocScratchBytes that every GPU holds from the code object's
// load until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory, so the kernels get the array's device address,
// looked up once per device with hipGetSymbolAddress (each GPU holds its own
// copy at its own address).  Calls that overlap on one GPU (two streams, two
// threads) share that GPU's array and race.
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
float* g_scratch_dev[kMaxDevices];  // the array's device address, per device
std::mutex g_scratch_lock;

// the current device's address of `scratch` (nullptr + message on failure)
float* scratch_on_current_device() {
    int dev = -1;
    if(hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        pk::fail("pk_gemm_noalloc_f32: no current HIP device (or device id above %d)",
                 kMaxDevices - 1);
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if(!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if(e != hipSuccess || !p) {
            pk::fail("pk_gemm_noalloc_f32: hipGetSymbolAddress(scratch) failed on device %d: %s",
                     dev, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_dev[dev] = static_cast<float*>(p);
    }
    return g_scratch_dev[dev];
}
}  // namespace

extern "C" size_t pk_gemm_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int pk_gemm_noalloc_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                                   const float* A, int64_t lda, const float* B, int64_t ldb,
                                   float beta, float* C, int64_t ldc, pk_stream_t stream) {
    const size_t need = gemm_workspace(M, N, K, ta == 'T' || ta == 't');
    if(need > kNoAllocScratchBytes)
        return pk::fail("pk_gemm_noalloc_f32: this product's split-K partials need %zu bytes, "
                        "above the %zu-byte static scratch (use pk_gemm_ex_f32 with a workspace)",
                        need, kNoAllocScratchBytes);
    float* ws = nullptr;
    if(need > 0 && !(ws = scratch_on_current_device())) return PK_EINVAL;
    // every partial-plane element the reduction reads is written by its split
    // in the same call, so nothing in the scratch has to start at zero
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, ws, ws ? kNoAllocScratchBytes : 0, kFp32, stream);
}
