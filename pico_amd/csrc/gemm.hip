// pico_amd/csrc/gemm.hip -- fp32 GEMM on gfx950 matrix cores.
//
// C = alpha * op(A) . op(B) + beta * C, row-major, the three layouts pico's
// matmul and its backward need (A.B, A.B^T, A^T.B; src/ops.c:144-190 and
// src/autograd.h:96-130), plus a two-level batch and the causal tile/k-range
// restrictions attention uses.
//
// Design (one 256-thread workgroup per 128x128 C tile):
//  * 4 waves in a 2x2 grid, each wave owns a 64x64 sub-tile = 2x2 blocks of
//    v_mfma_f32_32x32x2f32 (4096 FLOP per instruction, 16 fp32 accumulators
//    per lane per block).
//  * K advances 32 at a time through LDS, double-buffered: the next slice is
//    fetched into registers with 128-bit global loads while the current slice
//    feeds the MFMAs, then written to the other LDS buffer; one barrier per slice.
//  * LDS keeps each operand in its global orientation (no transposes on the
//    store).  Within a 32-wide k slice, lanes 0-31 take k 0..15 and lanes 32-63
//    take k 16..31, so a k-contiguous tile is read with 128-bit LDS loads and a
//    row-contiguous tile with conflict-free 32-bit loads.  Row strides are
//    padded by 4 floats.
//  * Tile order is XCD-aware: the hardware deals consecutive workgroups to
//    the 8 XCDs round-robin, so the launch index is remapped to give each XCD
//    a contiguous run of tiles, walked in groups of 8 tile-rows so concurrently
//    running tiles share A rows and B columns in that XCD's L2.
#include <stdarg.h>
#include <stdio.h>

#include "pk_common.h"

namespace {

constexpr int BM = 128, BK = 32, NT = 256;
constexpr int KF = BK + 4;  // row stride of a k-contiguous LDS tile [rows][36]
constexpr int GROUP_M = 8;

// An R x BK operand slice (R = 128 or 96 rows): float4 per thread, the row
// stride of its row-contiguous LDS form [BK][R+4], and the LDS floats it needs.
template <int R>
struct Slice {
    static constexpr int V = R * BK / 4 / NT;
    static constexpr int Q4 = R / 4;  // float4 per k-row of the row-contiguous form
    static constexpr int RF = R + 4;
    static constexpr int FLOATS = R * KF > BK * RF ? R * KF : BK * RF;
};

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
};

// One R x 32 operand slice -> Slice<R>::V float4 per thread.  KFAST: element
// (r,k) at base[r*ld + k]; otherwise at base[k*ld + r].  EDGE zero-fills
// outside [Rlim) x [K).
template <bool KFAST, bool EDGE, int R>
__device__ __forceinline__ void load_slice(const float* __restrict__ base, int64_t ld, int64_t r0,
                                           int64_t k0, int64_t Rlim, int64_t K,
                                           f32x4 (&v)[Slice<R>::V]) {
#pragma unroll
    for(int i = 0; i < Slice<R>::V; ++i) {
        const int idx = threadIdx.x + i * NT;
        int rr, kk;
        if(KFAST) {
            rr = idx >> 3;
            kk = (idx & 7) * 4;
        } else {
            kk = idx / Slice<R>::Q4;
            rr = (idx % Slice<R>::Q4) * 4;
        }
        const int64_t r = r0 + rr, k = k0 + kk;
        if(!EDGE) {
            const float* p = KFAST ? base + r * ld + k : base + k * ld + r;
            v[i] = *reinterpret_cast<const f32x4*>(p);
        } else {
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
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
            v[i] = x;
        }
    }
}

template <bool KFAST, int R>
__device__ __forceinline__ void store_slice(float* lds, const f32x4 (&v)[Slice<R>::V]) {
#pragma unroll
    for(int i = 0; i < Slice<R>::V; ++i) {
        const int idx = threadIdx.x + i * NT;
        if(KFAST)
            *reinterpret_cast<f32x4*>(lds + (idx >> 3) * KF + (idx & 7) * 4) = v[i];
        else
            *reinterpret_cast<f32x4*>(lds + (idx / Slice<R>::Q4) * Slice<R>::RF +
                                      (idx % Slice<R>::Q4) * 4) = v[i];
    }
}

// 16 k-values of LDS row r for this lane's k half
template <bool KFAST, int R>
__device__ __forceinline__ void read_frag(const float* lds, int r, int h, float (&f)[16]) {
    if(KFAST) {
        const f32x4* p = reinterpret_cast<const f32x4*>(lds + r * KF + h * 16);
#pragma unroll
        for(int q = 0; q < 4; ++q) {
            f32x4 x = p[q];
            f[4 * q + 0] = x[0];
            f[4 * q + 1] = x[1];
            f[4 * q + 2] = x[2];
            f[4 * q + 3] = x[3];
        }
    } else {
#pragma unroll
        for(int s = 0; s < 16; ++s) f[s] = lds[(h * 16 + s) * Slice<R>::RF + r];
    }
}

// Wave layout of a BM x BN tile: BN = 128 -> 2 x 2 waves, each 64 x 64 = 2 x 2
// blocks of 32 x 32; BN = 96 -> 4 x 1 waves, each 32 x 96 = 1 x 3 blocks.
template <int BN>
struct WaveGrid {
    static constexpr int TN = BN == 128 ? 2 : 3;  // 32x32 blocks per wave along N
    static constexpr int TM = BN == 128 ? 2 : 1;  // along M
    static constexpr int WN = BN / (32 * TN);     // waves along N
};

template <bool TA, bool TB, bool EDGE, int BN>
__global__ __launch_bounds__(NT, 2) void gemm_f32_kernel(GemmParams p) {
    constexpr int TM = WaveGrid<BN>::TM, TN = WaveGrid<BN>::TN, WN = WaveGrid<BN>::WN;
    __shared__ __attribute__((aligned(16))) float ldsA[2][Slice<BM>::FLOATS];
    __shared__ __attribute__((aligned(16))) float ldsB[2][Slice<BN>::FLOATS];

    // ---- tile selection: XCD-contiguous runs, grouped by GROUP_M tile-rows
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
    const float* __restrict__ A = p.A + zo * p.sAo + zi * p.sAi;
    const float* __restrict__ B = p.B + zo * p.sBo + zi * p.sBi;
    float* __restrict__ C = p.C + zo * p.sCo + zi * p.sCi;
    int64_t ldc = p.ldc;
    float alpha = p.alpha, beta = p.beta;

    const int64_t row0 = (int64_t)tm * BM, col0 = (int64_t)tn * BN;
    int64_t kbeg = 0, kend = p.K;
    if(p.causal == 1 && col0 > row0 + BM - 1) return;  // wholly above the diagonal
    if(p.causal == 2) kend = min(p.K, row0 + BM);
    if(p.causal == 3) kbeg = min(p.K, (row0 / BK) * BK);
    if(p.splits > 1) {
        // slice s of K; its partial product goes to workspace plane s
        kbeg = (int64_t)blockIdx.y * p.kchunk;
        kend = min(p.K, kbeg + p.kchunk);
        C = p.ws + (int64_t)blockIdx.y * p.M * p.N;
        ldc = p.N;
        alpha = 1.0f;
        beta = 0.0f;
    }
    const int nslices = (int)((kend - kbeg + BK - 1) / BK);

    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    const int wm = w / WN, wn = w % WN;
    const int lr = l & 31, lh = l >> 5;

    f32x16 acc[TM][TN];
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int j = 0; j < TN; ++j)
#pragma unroll
            for(int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // op(A) rows are k-contiguous when A is not transposed; op(B)^T rows
    // (indexed by n) are k-contiguous when B is transposed.
    constexpr bool AK = !TA, BKF = TB;
    f32x4 ra[Slice<BM>::V], rb[Slice<BN>::V];
    if(nslices > 0) {
        load_slice<AK, EDGE, BM>(A, p.lda, row0, kbeg, p.M, kend, ra);
        load_slice<BKF, EDGE, BN>(B, p.ldb, col0, kbeg, p.N, kend, rb);
        store_slice<AK, BM>(ldsA[0], ra);
        store_slice<BKF, BN>(ldsB[0], rb);
    }
    __syncthreads();

    for(int s = 0; s < nslices; ++s) {
        const int cur = s & 1;
        const bool more = s + 1 < nslices;
        if(more) {
            const int64_t k0 = kbeg + (int64_t)(s + 1) * BK;
            load_slice<AK, EDGE, BM>(A, p.lda, row0, k0, p.M, kend, ra);
            load_slice<BKF, EDGE, BN>(B, p.ldb, col0, k0, p.N, kend, rb);
        }
        float fa[TM][16], fb[TN][16];
#pragma unroll
        for(int i = 0; i < TM; ++i)
            read_frag<AK, BM>(ldsA[cur], wm * TM * 32 + i * 32 + lr, lh, fa[i]);
#pragma unroll
        for(int j = 0; j < TN; ++j)
            read_frag<BKF, BN>(ldsB[cur], wn * TN * 32 + j * 32 + lr, lh, fb[j]);
#pragma unroll
        for(int kk = 0; kk < 16; ++kk)
#pragma unroll
            for(int i = 0; i < TM; ++i)
#pragma unroll
                for(int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][kk], fb[j][kk],
                                                                     acc[i][j], 0, 0, 0);
        if(more) {
            store_slice<AK, BM>(ldsA[cur ^ 1], ra);
            store_slice<BKF, BN>(ldsB[cur ^ 1], rb);
        }
        __syncthreads();
    }

    // ---- epilogue: 32x32 block accumulator r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
    // column l%32
#pragma unroll
    for(int i = 0; i < TM; ++i)
#pragma unroll
        for(int j = 0; j < TN; ++j) {
            const int64_t col = col0 + wn * TN * 32 + j * 32 + lr;
#pragma unroll
            for(int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wm * TM * 32 + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                if(EDGE && (row >= p.M || col >= p.N)) continue;
                float v = alpha * acc[i][j][r];
                float* c = C + row * ldc + col;
                if(beta != 0.0f) v += beta * *c;
                *c = v;
            }
        }
}

// C = alpha * sum_s ws[s] + beta * C, planes summed in order s = 0, 1, ...
__global__ void splitk_reduce(int64_t M, int64_t N, int S, const float* __restrict__ ws,
                              float alpha, float beta, float* __restrict__ C, int64_t ldc) {
    const int64_t plane = M * N;
    if((N & 3) == 0 && (ldc & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0) {
        const int64_t n4 = plane / 4, N4 = N / 4;
        for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
            i += (int64_t)gridDim.x * blockDim.x) {
            f32x4 acc = reinterpret_cast<const f32x4*>(ws)[i];
            for(int s = 1; s < S; ++s) acc += reinterpret_cast<const f32x4*>(ws + s * plane)[i];
            f32x4* c = reinterpret_cast<f32x4*>(C + (i / N4) * ldc) + (i % N4);
            f32x4 v = alpha * acc;
            if(beta != 0.0f) v += beta * *c;
            *c = v;
        }
        return;
    }
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < plane;
        i += (int64_t)gridDim.x * blockDim.x) {
        float acc = ws[i];
        for(int s = 1; s < S; ++s) acc += ws[s * plane + i];
        float* c = C + (i / N) * ldc + (i % N);
        float v = alpha * acc;
        if(beta != 0.0f) v += beta * *c;
        *c = v;
    }
}

// K split for a product whose output has too few tiles to fill the chip: 2
// resident workgroups per CU x 256 CUs want >= 512 workgroups; each slice keeps
// at least 256 of K (8 LDS stages) so the pipeline stays long.
constexpr int64_t kSplitTarget = 512, kMinSliceK = 256;

int choose_splits(int64_t M, int64_t N, int64_t K, int64_t* kchunk) {
    const int64_t tiles = ((M + BM - 1) / BM) * ((N + 127) / 128);
    *kchunk = K;
    if(tiles <= 0 || tiles * 2 > kSplitTarget || K < 4 * kMinSliceK) return 1;
    int64_t s = kSplitTarget / tiles;
    if(s > K / kMinSliceK) s = K / kMinSliceK;
    if(s < 2) return 1;
    const int64_t chunk = ((K + s - 1) / s + BK - 1) / BK * BK;
    *kchunk = chunk;
    return (int)((K + chunk - 1) / chunk);
}

// Tile width: 96-wide tiles when N is a multiple of 96 and they fill the 512
// resident workgroup slots (2 per CU) clearly better than 128-wide ones.  An
// [8192, 768] output, every projection of a d_model-768 transformer, makes 384
// 128-wide tiles (75 % of the slots busy) but 512 96-wide ones.
constexpr int64_t kSlots = 512;

double slot_fill(int64_t tiles) {
    const int64_t rounds = (tiles + kSlots - 1) / kSlots;
    return rounds ? (double)tiles / (double)(rounds * kSlots) : 0.0;
}

int pick_bn(int64_t M, int64_t N, int64_t batch) {
    if(N % 96) return 128;
    const int64_t tm = (M + BM - 1) / BM;
    const int64_t t128 = tm * ((N + 127) / 128) * batch, t96 = tm * (N / 96) * batch;
    return slot_fill(t96) > slot_fill(t128) + 0.1 ? 96 : 128;
}

template <bool TA, bool TB, int BN>
int launch_bn(const GemmParams& gp, int64_t batch, bool edge, hipStream_t st) {
    dim3 grid((unsigned)(gp.tiles_m * gp.tiles_n), (unsigned)(gp.splits > 1 ? gp.splits : batch));
    if(edge)
        gemm_f32_kernel<TA, TB, true, BN><<<grid, NT, 0, st>>>(gp);
    else
        gemm_f32_kernel<TA, TB, false, BN><<<grid, NT, 0, st>>>(gp);
    return pk::launch_status("pk_gemm_f32");
}

template <bool TA, bool TB>
int launch(const GemmParams& gp, int64_t batch, bool edge, int bn, hipStream_t st) {
    return bn == 96 ? launch_bn<TA, TB, 96>(gp, batch, edge, st)
                    : launch_bn<TA, TB, 128>(gp, batch, edge, st);
}

int gemm_impl(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
              int64_t lda, int64_t sA_outer, int64_t sA_inner, const float* B, int64_t ldb,
              int64_t sB_outer, int64_t sB_inner, float beta, float* C, int64_t ldc,
              int64_t sC_outer, int64_t sC_inner, int64_t batch, int64_t inner_count, int causal,
              float* ws, size_t ws_bytes, pk_stream_t stream) {
    const bool TA = ta == 'T' || ta == 't', TB = tb == 'T' || tb == 't';
    if(!(TA || ta == 'N' || ta == 'n') || !(TB || tb == 'N' || tb == 'n'))
        return pk::fail("pk_gemm_f32: transpose flags must be 'N' or 'T' (got '%c','%c')", ta, tb);
    if(M < 0 || N < 0 || K < 0 || batch < 0)
        return pk::fail("pk_gemm_f32: negative size M=%lld N=%lld K=%lld batch=%lld",
                        (long long)M, (long long)N, (long long)K, (long long)batch);
    if(causal < 0 || causal > 3) return pk::fail("pk_gemm_f32: causal mode %d not in 0..3", causal);
    if(inner_count < 1) return pk::fail("pk_gemm_f32: inner_count must be >= 1");
    if(M == 0 || N == 0 || batch == 0) return PK_OK;
    if(!C) return pk::fail("pk_gemm_f32: C is NULL");
    if(K > 0 && (!A || !B)) return pk::fail("pk_gemm_f32: A or B is NULL");
    const int64_t a_cols = TA ? M : K, b_cols = TB ? K : N;
    if(K > 0 && (lda < a_cols || ldb < b_cols))
        return pk::fail("pk_gemm_f32: leading dimension too small (lda=%lld needs >= %lld, "
                        "ldb=%lld needs >= %lld)",
                        (long long)lda, (long long)a_cols, (long long)ldb, (long long)b_cols);
    if(ldc < N) return pk::fail("pk_gemm_f32: ldc=%lld < N=%lld", (long long)ldc, (long long)N);
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
    hipStream_t st = pk::as_stream(stream);
    gp.splits = 1;
    gp.kchunk = K;
    gp.ws = nullptr;
    if(batch == 1 && causal == 0 && ws && K > 0) {
        int64_t kchunk;
        const int S = choose_splits(M, N, K, &kchunk);
        if(S > 1 && ws_bytes >= (size_t)S * (size_t)M * (size_t)N * sizeof(float)) {
            gp.splits = S;
            gp.kchunk = kchunk;
            gp.ws = ws;
        }
    }
    const int bn = gp.splits > 1 ? 128 : pick_bn(M, N, batch);
    const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + bn - 1) / bn;
    if(tiles_m * tiles_n > (int64_t)1 << 30)
        return pk::fail("pk_gemm_f32: problem too large for one launch");
    gp.tiles_m = (int)tiles_m;
    gp.tiles_n = (int)tiles_n;
    // the unchecked path needs whole tiles and 16-byte aligned float4 loads
    const bool edge = (M % BM) || (N % bn) || (K % BK) || (lda % 4) || (ldb % 4) ||
                      (sA_outer % 4) || (sA_inner % 4) || (sB_outer % 4) || (sB_inner % 4) ||
                      !pk::aligned16(A) || !pk::aligned16(B);
    int rc;
    if(!TA && !TB)
        rc = launch<false, false>(gp, batch, edge, bn, st);
    else if(!TA && TB)
        rc = launch<false, true>(gp, batch, edge, bn, st);
    else if(TA && !TB)
        rc = launch<true, false>(gp, batch, edge, bn, st);
    else
        rc = launch<true, true>(gp, batch, edge, bn, st);
    if(rc || gp.splits == 1) return rc;
    splitk_reduce<<<pk::grid_for(M * N / 4 + 1, NT), NT, 0, st>>>(M, N, gp.splits, gp.ws, alpha,
                                                                  beta, C, ldc);
    return pk::launch_status("pk_gemm_ex_f32 (split-K reduction)");
}

}  // namespace

extern "C" int pk_gemm_batched_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                                   const float* A, int64_t lda, int64_t sA_outer, int64_t sA_inner,
                                   const float* B, int64_t ldb, int64_t sB_outer, int64_t sB_inner,
                                   float beta, float* C, int64_t ldc, int64_t sC_outer,
                                   int64_t sC_inner, int64_t batch, int64_t inner_count,
                                   int causal, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, sA_outer, sA_inner, B, ldb, sB_outer,
                     sB_inner, beta, C, ldc, sC_outer, sC_inner, batch, inner_count, causal,
                     nullptr, 0, stream);
}

extern "C" int pk_gemm_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                           const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                           float* C, int64_t ldc, pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, nullptr, 0, stream);
}

extern "C" size_t pk_gemm_workspace_f32(int64_t M, int64_t N, int64_t K) {
    if(M <= 0 || N <= 0 || K <= 0) return 0;
    int64_t kchunk;
    const int S = choose_splits(M, N, K, &kchunk);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

extern "C" int pk_gemm_ex_f32(char ta, char tb, int64_t M, int64_t N, int64_t K, float alpha,
                              const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                              float* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                              pk_stream_t stream) {
    return gemm_impl(ta, tb, M, N, K, alpha, A, lda, 0, 0, B, ldb, 0, 0, beta, C, ldc, 0, 0, 1, 1,
                     0, static_cast<float*>(workspace), workspace_bytes, stream);
}
