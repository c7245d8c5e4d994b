// pico_amd/csrc/elementwise.hip -- broadcast binary ops and their gradients,
// unary math, relu, fill, axpy, sum, SGD, AdamW, embedding gather/scatter.
//
// Everything here is HBM-bound streaming: contiguous operands go through
// 128-bit loads and stores, grid-stride loops sized to a few waves per CU.
// Floating-point contraction is off in this file so each a*b+c rounds twice,
// as pico's C11 build does (src/kernels/cpu/cpu_scalar.h, src/optim/SGD.c);
// add/sub/mul, their gradients, relu and SGD are then bit-identical to the
// reference's CPU results.
#include <math.h>

#include "pk_common.h"

#pragma clang fp contract(off)

namespace {

constexpr int kMaxDims = 8;
constexpr int NT = 256;

struct Strides {
    int ndim;
    int64_t shape[kMaxDims];
    int64_t sa[kMaxDims];  // first operand's strides over the output dims
    int64_t sb[kMaxDims];  // second operand's strides over the output dims
};

__device__ __forceinline__ float bin_apply(int op, float x, float y) {
    return op == 0 ? x + y : op == 1 ? x - y : x * y;
}

// out[i] = a[ia] op b[ib], the broadcast index map of pico's map_index
__global__ void binary_general(int op, Strides s, int64_t n, const float* __restrict__ a,
                               const float* __restrict__ b, float* __restrict__ out) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        int64_t rem = i, ia = 0, ib = 0;
        for(int d = s.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % s.shape[d];
            rem /= s.shape[d];
            ia += c * s.sa[d];
            ib += c * s.sb[d];
        }
        out[i] = bin_apply(op, a[ia], b[ib]);
    }
}

__global__ void binary_same4(int op, int64_t n4, const f32x4* __restrict__ a,
                             const f32x4* __restrict__ b, f32x4* __restrict__ out) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
        i += (int64_t)gridDim.x * blockDim.x) {
        const f32x4 x = a[i], y = b[i];
        f32x4 r;
        r[0] = bin_apply(op, x[0], y[0]);
        r[1] = bin_apply(op, x[1], y[1]);
        r[2] = bin_apply(op, x[2], y[2]);
        r[3] = bin_apply(op, x[3], y[3]);
        out[i] = r;
    }
}

// Gradient of one operand x.  The output dims split into "kept" dims (x has
// them) and "reduced" dims (x is broadcast there).  Thread j owns the j-th
// element of x in row-major order (stored at sum c_k * kx[k], x's own strides,
// so a transposed view's grad lands where pico's map_index puts it) and
// walks the reduced dims in increasing flat order, adding one term at a time
// to the running value -- the same order and rounding as the reference's
// single pass (src/autograd.h:53-94).
struct BwdDesc {
    int nk, nr;
    int64_t kshape[kMaxDims], kout[kMaxDims], koth[kMaxDims], kx[kMaxDims];
    int64_t rshape[kMaxDims], rout[kMaxDims], roth[kMaxDims];
    int64_t red_numel;
};

__device__ __forceinline__ float grad_term(int op, int which, float g, float other) {
    if(op == 2) return g * other;
    return (op == 1 && which == 1) ? -g : g;
}

__global__ void binary_bwd_reduce(int op, int which, BwdDesc d, int64_t xn,
                                  const float* __restrict__ gout, const float* __restrict__ other,
                                  float* __restrict__ gx, int accum) {
    for(int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < xn;
        j += (int64_t)gridDim.x * blockDim.x) {
        int64_t rem = j, bo = 0, bt = 0, bx = 0;
        for(int k = d.nk - 1; k >= 0; --k) {
            const int64_t c = rem % d.kshape[k];
            rem /= d.kshape[k];
            bo += c * d.kout[k];
            bt += c * d.koth[k];
            bx += c * d.kx[k];
        }
        float acc = accum ? gx[bx] : 0.0f;
        for(int64_t r = 0; r < d.red_numel; ++r) {
            int64_t rr = r, oo = bo, ot = bt;
            for(int k = d.nr - 1; k >= 0; --k) {
                const int64_t c = rr % d.rshape[k];
                rr /= d.rshape[k];
                oo += c * d.rout[k];
                ot += c * d.roth[k];
            }
            // sub's second operand: grad -= g, the reference's form
            if(op == 1 && which == 1)
                acc -= gout[oo];
            else
                acc += grad_term(op, which, gout[oo], op == 2 ? other[ot] : 0.0f);
        }
        gx[bx] = acc;
    }
}

// Fast paths of the same gradient, with the same order and rounding:
//  * x has the output's shape and layout (a residual add): one float4 per thread;
//  * x is broadcast over leading rows only (a bias): out viewed as [R, C], one
//    thread per column j adds the R rows in increasing order.
__device__ __forceinline__ float grad_add(int op, int which, float acc, float g, float other) {
    // sub's second operand: grad -= g, the reference's form
    if(op == 1 && which == 1) return acc - g;
    return acc + grad_term(op, which, g, other);
}

__global__ void binary_bwd_same4(int op, int which, int64_t n4, const f32x4* __restrict__ gout,
                                 const f32x4* __restrict__ other, f32x4* __restrict__ gx,
                                 int accum) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
        i += (int64_t)gridDim.x * blockDim.x) {
        const f32x4 g = pk::ld_stream(gout + i);
        const f32x4 o = op == 2 ? pk::ld_stream(other + i) : f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 acc = accum ? gx[i] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for(int e = 0; e < 4; ++e) acc[e] = grad_add(op, which, acc[e], g[e], o[e]);
        pk::st_stream(gx + i, acc);
    }
}

__global__ void binary_bwd_rows(int op, int which, int64_t R, int64_t C,
                                const float* __restrict__ gout, const float* __restrict__ other,
                                float* __restrict__ gx, int accum) {
    for(int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < C;
        j += (int64_t)gridDim.x * blockDim.x) {
        float acc = accum ? gx[j] : 0.0f;
        // the adds stay in row order; unrolling lets the loads run ahead of them
#pragma unroll 8
        for(int64_t r = 0; r < R; ++r)
            acc = grad_add(op, which, acc, gout[r * C + j], op == 2 ? other[r * C + j] : 0.0f);
        gx[j] = acc;
    }
}

// ---------------------------------------------------------------- unary
__device__ __forceinline__ float un_apply(int op, float x) {
    switch(op) {
        case 0: return sqrtf(x);
        case 1: return (float)sin((double)x);
        case 2: return (float)cos((double)x);
        case 3: return (float)tan((double)x);
        case 4: return (float)tanh((double)x);
        default: return logf(x);
    }
}

__device__ __forceinline__ float un_bwd(int op, float gx, float x, float y, float g) {
    switch(op) {
        case 0: return gx + g * (1.0f / (2.0f * y));
        case 1: return (float)((double)gx + (double)g * cos((double)x));
        case 2: return (float)((double)gx - (double)g * sin((double)x));
        case 3: {
            const float sec = (float)(1.0 / cos((double)x));
            return gx + g * (sec * sec);
        }
        case 4: return gx + (g * 1.0f - y * y);
        default: return gx + g * 1.0f / x;
    }
}

__global__ void unary_kernel(int op, int64_t n, const float* __restrict__ x, float* __restrict__ y) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x)
        y[i] = un_apply(op, x[i]);
}

__global__ void unary_bwd_kernel(int op, int64_t n, const float* __restrict__ x,
                                 const float* __restrict__ y, const float* __restrict__ gy,
                                 float* __restrict__ gx, int accum) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x)
        gx[i] = un_bwd(op, accum ? gx[i] : 0.0f, x[i], y[i], gy[i]);
}

// ------------------------------------------------------------------ relu
__device__ __forceinline__ float relu1(float x) { return x > 0.0f ? x : 0.0f; }

__global__ void relu_kernel(int64_t n, const float* __restrict__ x, float* __restrict__ y) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x)
        y[i] = relu1(x[i]);
}

__global__ void relu_bwd_kernel(int64_t n, const float* __restrict__ y,
                                const float* __restrict__ gy, float* __restrict__ gx, int accum) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const float gate = (float)(y[i] > 0.0f);
        const float t = gy[i] * gate;
        gx[i] = accum ? gx[i] + t : t;
    }
}

// ------------------------------------------------------- fill, axpy, sum
__global__ void fill_kernel(int64_t n, float v, float* __restrict__ x) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x)
        x[i] = v;
}

// a [rows, cols] block with row stride ld (grid-stride over rows x cols)
__global__ void fill2d_kernel(int64_t rows, int64_t cols, float v, float* __restrict__ x,
                              int64_t ld) {
    const int64_t n = rows * cols;
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x)
        x[(i / cols) * ld + i % cols] = v;
}

// splitmix64 finaliser: a bijective 64-bit mix (Steele, Lea & Flood 2014)
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(int64_t n, uint64_t seed, float mean, float std,
                                   float* __restrict__ x) {
    const uint64_t key = mix64(seed ^ 0x9e3779b97f4a7c15ull);
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t r = mix64(key + (uint64_t)i * 0x9e3779b97f4a7c15ull);
        // two 24-bit uniforms: u1 in (0, 1], u2 in [0, 1)
        const float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);
        const float u2 = (float)(uint32_t)((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958648f * u2);
        x[i] = mean + std * z;
    }
}

__global__ void axpy_kernel(int64_t n, float alpha, const float* __restrict__ alpha_dev,
                            const float* __restrict__ x, float* __restrict__ y, int accum) {
    const float a = alpha_dev ? alpha * *alpha_dev : alpha;
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const float t = a * x[i];
        y[i] = accum ? y[i] + t : t;
    }
}

// one 1024-thread block: fixed partition and tree, so the result is deterministic
__global__ __launch_bounds__(1024) void sum_kernel(int64_t n, const float* __restrict__ x,
                                                   float scale, float* __restrict__ out, int accum) {
    __shared__ float red[16];
    double s = 0.0;
    for(int64_t i = threadIdx.x; i < n; i += 1024) s += (double)x[i];
    float v = pk::block_sum<16>((float)s, red);
    if(threadIdx.x == 0) {
        const float t = scale * v;
        out[0] = accum ? out[0] + t : t;
    }
}

// ------------------------------------------------------------ optimizers
__global__ void sgd_kernel(int64_t n, float lr, float* __restrict__ p, const float* __restrict__ g) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const float step = lr * g[i];
        p[i] = p[i] - step;
    }
}

// SGD over up to kSgdMax tensors in one launch: blockIdx.y picks the tensor,
// each element updated as sgd_kernel updates it
constexpr int kSgdMax = 32;
struct SgdBatch {
    float* p[kSgdMax];
    const float* g[kSgdMax];
    int64_t n[kSgdMax];
};

__global__ void sgd_multi_kernel(SgdBatch b, float lr) {
    const int t = blockIdx.y;
    float* __restrict__ p = b.p[t];
    const float* __restrict__ g = b.g[t];
    const int64_t n = b.n[t];
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const float step = lr * g[i];
        p[i] = p[i] - step;
    }
}

// decoupled decay, then the bias-corrected Adam update of one element
__device__ __forceinline__ float adamw_elem(float& p, float gi, float& m, float& v, float b1,
                                            float b2, float eps, float decay, float step_size,
                                            float bc2_sqrt) {
    const float pj = p * decay;
    const float mj = b1 * m + (1.0f - b1) * gi;
    const float vj = b2 * v + (1.0f - b2) * gi * gi;
    const float denom = sqrtf(vj) / bc2_sqrt + eps;
    p = pj - step_size * (mj / denom);
    m = mj;
    v = vj;
    return p;
}

__global__ void adamw_kernel(int64_t n, float b1, float b2, float eps, float decay,
                             float step_size, float bc2_sqrt, float* __restrict__ p,
                             const float* __restrict__ g, float* __restrict__ m,
                             float* __restrict__ v) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const float gi = g ? g[i] : 0.0f;
        adamw_elem(p[i], gi, m[i], v[i], b1, b2, eps, decay, step_size, bc2_sqrt);
    }
}

// One multi-tensor AdamW step: the step counter and the two bias corrections
// live in device memory, so the launch parameters never change between steps.
__global__ void adamw_prep_kernel(int32_t* step, float lr, float b1, float b2, float* coef) {
    if(threadIdx.x != 0 || blockIdx.x != 0) return;
    const int32_t t = *step + 1;
    *step = t;
    const double bc1 = 1.0 - pow((double)b1, (double)t);
    const double bc2 = 1.0 - pow((double)b2, (double)t);
    coef[0] = (float)((double)lr / bc1);
    coef[1] = (float)sqrt(bc2);
}

// kAdamwSplit workgroups per chunk (<= PK_ADAMW_CHUNK elements of one tensor),
// interleaved by float4, two float4 of each array per lane in flight.  Short
// workgroups keep the memory pipes evenly loaded to the end of the pass:
// 134 M parameters measured 719 us with 4 per chunk, 650 with 16 (5.8 TB/s),
// 657-685 with 32-128, 643 with 16 and two in flight per lane.
constexpr int kAdamwSplit = 16;
__global__ __launch_bounds__(256) void adamw_multi_kernel(const PkAdamwChunk* __restrict__ chunks,
                                                          float b1, float b2, float eps,
                                                          float decay,
                                                          const float* __restrict__ coef) {
    const PkAdamwChunk c = chunks[blockIdx.x / kAdamwSplit];
    const float step_size = coef[0], bc2_sqrt = coef[1];
    const uintptr_t align = reinterpret_cast<uintptr_t>(c.p) | reinterpret_cast<uintptr_t>(c.g) |
                            reinterpret_cast<uintptr_t>(c.m) | reinterpret_cast<uintptr_t>(c.v);
    const int64_t n4 = (align & 15) ? 0 : c.n / 4;
    // four distinct tensors, each element read and written once: streaming
    // (nontemporal) accesses, two float4 of each per lane in flight
    f32x4* __restrict__ p4 = reinterpret_cast<f32x4*>(c.p);
    f32x4* __restrict__ m4 = reinterpret_cast<f32x4*>(c.m);
    f32x4* __restrict__ v4 = reinterpret_cast<f32x4*>(c.v);
    const f32x4* __restrict__ g4 = reinterpret_cast<const f32x4*>(c.g);
    auto update = [&](f32x4& p, const f32x4& g, f32x4& m, f32x4& v) {
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            float pe = p[e], me = m[e], ve = v[e];
            adamw_elem(pe, g[e], me, ve, b1, b2, eps, decay, step_size, bc2_sqrt);
            p[e] = pe;
            m[e] = me;
            v[e] = ve;
        }
    };
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const int64_t stride = (int64_t)blockDim.x * kAdamwSplit;
    int64_t i = threadIdx.x + (int64_t)(blockIdx.x % kAdamwSplit) * blockDim.x;
    for(; i + stride < n4; i += 2 * stride) {
        const int64_t j = i + stride;
        f32x4 pa = pk::ld_stream(p4 + i), ma = pk::ld_stream(m4 + i), va = pk::ld_stream(v4 + i);
        f32x4 pb = pk::ld_stream(p4 + j), mb = pk::ld_stream(m4 + j), vb = pk::ld_stream(v4 + j);
        const f32x4 ga = c.g ? pk::ld_stream(g4 + i) : zero;
        const f32x4 gb = c.g ? pk::ld_stream(g4 + j) : zero;
        update(pa, ga, ma, va);
        update(pb, gb, mb, vb);
        pk::st_stream(p4 + i, pa);
        pk::st_stream(m4 + i, ma);
        pk::st_stream(v4 + i, va);
        pk::st_stream(p4 + j, pb);
        pk::st_stream(m4 + j, mb);
        pk::st_stream(v4 + j, vb);
    }
    for(; i < n4; i += stride) {
        f32x4 p = pk::ld_stream(p4 + i), m = pk::ld_stream(m4 + i), v = pk::ld_stream(v4 + i);
        const f32x4 g = c.g ? pk::ld_stream(g4 + i) : zero;
        update(p, g, m, v);
        pk::st_stream(p4 + i, p);
        pk::st_stream(m4 + i, m);
        pk::st_stream(v4 + i, v);
    }
    if(blockIdx.x % kAdamwSplit) return;  // the scalar tail: the chunk's first workgroup
    for(int64_t i = n4 * 4 + threadIdx.x; i < c.n; i += blockDim.x) {
        const float gi = c.g ? c.g[i] : 0.0f;
        adamw_elem(c.p[i], gi, c.m[i], c.v[i], b1, b2, eps, decay, step_size, bc2_sqrt);
    }
}

// ------------------------------------------------------------- embedding
__global__ void embed_fwd_kernel(int64_t n, int64_t d, int64_t vocab, const int32_t* __restrict__ ids,
                                 const float* __restrict__ table, float* __restrict__ out) {
    const int64_t total = n * d;
    for(int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
        t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = t / d, e = t % d;
        const int32_t id = ids[i];
        out[t] = (id >= 0 && id < vocab) ? table[(int64_t)id * d + e] : 0.0f;
    }
}

__global__ void embed_fwd4_kernel(int64_t n, int64_t d4, int64_t vocab,
                                  const int32_t* __restrict__ ids, const f32x4* __restrict__ table,
                                  f32x4* __restrict__ out) {
    const int64_t total = n * d4;
    for(int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
        t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = t / d4, e = t % d4;
        const int32_t id = ids[i];
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        out[t] = (id >= 0 && id < vocab) ? table[(int64_t)id * d4 + e] : z;
    }
}

// ---- deterministic embedding backward -------------------------------------
// dtable[r,:] += dout[i,:] for every i with ids[i] == r, the adds of one row
// made in increasing i -- the order of the sequential loop, so the result is
// the same bits on every run and replay.
//   sort:  the positions are sorted by id with a stable LSD radix sort of 8-bit
//          digits (an id outside [0, vocab) takes the key vocab and sorts
//          last), ceil(bits(vocab)/8) passes of O(n) work.  A pass is a
//          histogram of each 2048-key block, one exclusive scan over (digit,
//          block), and a scatter that keeps a block's keys of one digit in
//          position order (ranks within a wave from ballots, across waves and
//          chunks from counts in LDS), so equal ids stay in increasing i.
//   sum:   one workgroup per run of equal ids adds its rows in that order.
constexpr int kSortThreads = 256, kSortItems = 8, kSortTile = kSortThreads * kSortItems;
constexpr int kDigits = 256, kScanThreads = 1024, kScanPer = 8;

__device__ __forceinline__ int32_t embed_key(const int32_t* __restrict__ ids, int64_t i,
                                             int64_t vocab) {
    const int32_t id = ids[i];
    return (id >= 0 && id < vocab) ? id : (int32_t)vocab;
}

// hist[digit * blocks + block]: the block's keys with that digit (keys NULL:
// the first pass, keys made from ids)
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(
    int64_t n, int64_t vocab, const int32_t* __restrict__ ids, const int32_t* __restrict__ keys,
    int shift, int32_t* __restrict__ hist) {
    __shared__ int32_t h[kDigits];
    for(int t = threadIdx.x; t < kDigits; t += kSortThreads) h[t] = 0;
    __syncthreads();
    const int64_t b0 = (int64_t)blockIdx.x * kSortTile;
#pragma unroll
    for(int e = 0; e < kSortItems; ++e) {
        const int64_t i = b0 + e * kSortThreads + threadIdx.x;
        if(i < n) {
            const int32_t k = keys ? keys[i] : embed_key(ids, i, vocab);
            atomicAdd(&h[(k >> shift) & (kDigits - 1)], 1);  // integer counts: any order
        }
    }
    __syncthreads();
    for(int t = threadIdx.x; t < kDigits; t += kSortThreads)
        hist[(int64_t)t * gridDim.x + blockIdx.x] = h[t];
}

// exclusive prefix sums of a[0..m), in place, one workgroup
__global__ __launch_bounds__(kScanThreads) void radix_scan_kernel(int64_t m,
                                                                  int32_t* __restrict__ a) {
    __shared__ int32_t sums[kScanThreads];
    __shared__ int32_t carry;
    if(threadIdx.x == 0) carry = 0;
    for(int64_t base = 0; base < m; base += (int64_t)kScanThreads * kScanPer) {
        const int64_t b = base + (int64_t)threadIdx.x * kScanPer;
        int32_t v[kScanPer];
        int32_t local = 0;
#pragma unroll
        for(int e = 0; e < kScanPer; ++e) {
            v[e] = b + e < m ? a[b + e] : 0;
            local += v[e];
        }
        __syncthreads();
        sums[threadIdx.x] = local;
        __syncthreads();
        for(int o = 1; o < kScanThreads; o <<= 1) {
            const int32_t add = threadIdx.x >= o ? sums[threadIdx.x - o] : 0;
            __syncthreads();
            sums[threadIdx.x] += add;
            __syncthreads();
        }
        int32_t run = carry + (threadIdx.x ? sums[threadIdx.x - 1] : 0);
#pragma unroll
        for(int e = 0; e < kScanPer; ++e) {
            if(b + e < m) a[b + e] = run;
            run += v[e];
        }
        __syncthreads();
        if(threadIdx.x == kScanThreads - 1) carry = run;
    }
}

// stable scatter of one pass: key i of the block goes to offs[digit, block] +
// (keys of that digit earlier in the block).  keys_in NULL: the first pass
// (keys from ids, values the positions).
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    int64_t n, int64_t vocab, const int32_t* __restrict__ ids, const int32_t* __restrict__ keys_in,
    const int32_t* __restrict__ vals_in, int shift, const int32_t* __restrict__ offs,
    int32_t* __restrict__ keys_out, int32_t* __restrict__ vals_out) {
    constexpr int W = kSortThreads / 64;
    __shared__ int32_t run[kDigits];     // where this block's next key of each digit goes
    __shared__ int32_t wcnt[W][kDigits];  // keys of each digit per wave, this chunk
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for(int t = threadIdx.x; t < kDigits; t += kSortThreads) {
        run[t] = offs[(int64_t)t * gridDim.x + blockIdx.x];
#pragma unroll
        for(int ww = 0; ww < W; ++ww) wcnt[ww][t] = 0;
    }
    __syncthreads();
    const uint64_t below_mask = (1ull << lane) - 1;
    const int64_t b0 = (int64_t)blockIdx.x * kSortTile;
    for(int e = 0; e < kSortItems; ++e) {
        const int64_t i = b0 + e * kSortThreads + threadIdx.x;
        const bool ok = i < n;
        int32_t k = 0, v = 0, dg = 0;
        if(ok) {
            k = keys_in ? keys_in[i] : embed_key(ids, i, vocab);
            v = vals_in ? vals_in[i] : (int32_t)i;
            dg = (k >> shift) & (kDigits - 1);
        }
        // the lanes of this wave holding the same digit
        uint64_t same = __ballot(ok);
#pragma unroll
        for(int bit = 0; bit < 8; ++bit) {
            const bool set = (dg >> bit) & 1;
            const uint64_t bb = __ballot(set);
            same &= set ? bb : ~bb;
        }
        const int below = __popcll(same & below_mask);
        if(ok && below == 0) wcnt[w][dg] = __popcll(same);  // the digit's lowest lane
        __syncthreads();
        if(ok) {
            int32_t pos = run[dg] + below;
            for(int ww = 0; ww < w; ++ww) pos += wcnt[ww][dg];
            keys_out[pos] = k;
            vals_out[pos] = v;
        }
        __syncthreads();
        for(int t = threadIdx.x; t < kDigits; t += kSortThreads) {
            int32_t c = 0;
#pragma unroll
            for(int ww = 0; ww < W; ++ww) {
                c += wcnt[ww][t];
                wcnt[ww][t] = 0;
            }
            run[t] += c;
        }
        __syncthreads();
    }
}

// one workgroup per sorted position; the first of each run of equal valid
// keys adds the run's rows, in order, into its table row
__global__ __launch_bounds__(256) void embed_sum_kernel(int64_t n, int64_t d, int64_t vocab,
                                                        const int32_t* __restrict__ keys,
                                                        const int32_t* __restrict__ pos,
                                                        const float* __restrict__ dout,
                                                        float* __restrict__ dtable) {
    const int64_t s = blockIdx.x;
    const int32_t id = keys[s];
    if(id >= vocab || (s > 0 && keys[s - 1] == id)) return;
    int64_t c = 1;
    while(s + c < n && keys[s + c] == id) ++c;
    float* row = dtable + (int64_t)id * d;
    if((d & 3) == 0 && pk::aligned16(dout) && pk::aligned16(dtable)) {
        const int64_t d4 = d / 4;
        for(int64_t col = threadIdx.x; col < d4; col += blockDim.x) {
            f32x4 acc = reinterpret_cast<f32x4*>(row)[col];
            for(int64_t k = 0; k < c; ++k)
                acc += reinterpret_cast<const f32x4*>(dout + (int64_t)pos[s + k] * d)[col];
            reinterpret_cast<f32x4*>(row)[col] = acc;
        }
        return;
    }
    for(int64_t col = threadIdx.x; col < d; col += blockDim.x) {
        float acc = row[col];
        for(int64_t k = 0; k < c; ++k) acc += dout[(int64_t)pos[s + k] * d + col];
        row[col] = acc;
    }
}

bool valid_op(int op, int hi) { return op >= 0 && op <= hi; }

}  // namespace

// ======================================================================= C-ABI

extern "C" int pk_binary_f32(int op, int ndim, const int64_t* out_shape, const int64_t* a_strides,
                             const int64_t* b_strides, const float* a, const float* b, float* out,
                             pk_stream_t stream) {
    if(!valid_op(op, 2)) return pk::fail("pk_binary_f32: op %d not in 0..2", op);
    if(ndim < 1 || ndim > kMaxDims) return pk::fail("pk_binary_f32: ndim %d not in 1..8", ndim);
    if(!out_shape || !a_strides || !b_strides) return pk::fail("pk_binary_f32: NULL descriptor");
    Strides s;
    s.ndim = ndim;
    int64_t n = 1;
    bool same = true;
    int64_t cs = 1;
    for(int d = ndim - 1; d >= 0; --d) {
        if(out_shape[d] < 0) return pk::fail("pk_binary_f32: negative dim");
        s.shape[d] = out_shape[d];
        s.sa[d] = a_strides[d];
        s.sb[d] = b_strides[d];
        if(out_shape[d] > 1 && (a_strides[d] != cs || b_strides[d] != cs)) same = false;
        cs *= out_shape[d];
        n *= out_shape[d];
    }
    if(n == 0) return PK_OK;
    if(!a || !b || !out) return pk::fail("pk_binary_f32: NULL data pointer");
    hipStream_t st = pk::as_stream(stream);
    if(same && n % 4 == 0 && pk::aligned16(a) && pk::aligned16(b) && pk::aligned16(out))
        binary_same4<<<pk::grid_for(n / 4, NT), NT, 0, st>>>(
            op, n / 4, (const f32x4*)a, (const f32x4*)b, (f32x4*)out);
    else
        binary_general<<<pk::grid_for(n, NT), NT, 0, st>>>(op, s, n, a, b, out);
    return pk::launch_status("pk_binary_f32");
}

extern "C" int pk_binary_bwd_f32(int op, int which, int ndim, const int64_t* out_shape,
                                 const int64_t* x_strides, const int64_t* other_strides,
                                 int64_t x_numel, const float* gout, const float* other, float* gx,
                                 int flags, pk_stream_t stream) {
    if(!valid_op(op, 2) || (which != 0 && which != 1))
        return pk::fail("pk_binary_bwd_f32: op %d / operand %d invalid", op, which);
    if(ndim < 1 || ndim > kMaxDims) return pk::fail("pk_binary_bwd_f32: ndim %d not in 1..8", ndim);
    if(!out_shape || !x_strides || !other_strides)
        return pk::fail("pk_binary_bwd_f32: NULL descriptor");
    BwdDesc d;
    d.nk = d.nr = 0;
    d.red_numel = 1;
    int64_t cs = 1, kept_numel = 1, out_n = 1;
    int64_t out_stride[kMaxDims];
    for(int k = ndim - 1; k >= 0; --k) {
        out_stride[k] = cs;
        cs *= out_shape[k];
        out_n *= out_shape[k];
    }
    for(int k = 0; k < ndim; ++k) {
        if(out_shape[k] == 1) continue;
        if(x_strides[k] != 0) {
            d.kshape[d.nk] = out_shape[k];
            d.kout[d.nk] = out_stride[k];
            d.koth[d.nk] = other_strides[k];
            d.kx[d.nk] = x_strides[k];
            d.nk++;
            kept_numel *= out_shape[k];
        } else {
            d.rshape[d.nr] = out_shape[k];
            d.rout[d.nr] = out_stride[k];
            d.roth[d.nr] = other_strides[k];
            d.nr++;
            d.red_numel *= out_shape[k];
        }
    }
    if(x_numel != kept_numel)
        return pk::fail("pk_binary_bwd_f32: x_numel %lld does not match its broadcast (%lld)",
                        (long long)x_numel, (long long)kept_numel);
    if(out_n == 0 || x_numel == 0) return PK_OK;
    if(!gout || !gx || (op == 2 && !other)) return pk::fail("pk_binary_bwd_f32: NULL data pointer");
    hipStream_t st = pk::as_stream(stream);
    const int accum = flags & PK_ACCUM;
    // x and (for mul) the other operand laid out exactly like the output
    // over the kept dims, and every reduced dim ahead of every kept dim
    bool kept_like_out = true, reduced_first = true;
    for(int k = 0; k < d.nk; ++k)
        if(d.kx[k] != d.kout[k] || (op == 2 && d.koth[k] != d.kout[k])) kept_like_out = false;
    for(int k = 0; k < d.nr; ++k)
        if(op == 2 && d.roth[k] != d.rout[k]) kept_like_out = false;
    if(d.nk > 0 && d.nr > 0 && d.rout[d.nr - 1] < d.kout[0]) reduced_first = false;
    if(kept_like_out && reduced_first && d.nr == 0 && x_numel % 4 == 0 && pk::aligned16(gout) &&
       pk::aligned16(gx) && (op != 2 || pk::aligned16(other))) {
        binary_bwd_same4<<<pk::grid_stream(x_numel / 4, NT), NT, 0, st>>>(
            op, which, x_numel / 4, (const f32x4*)gout, (const f32x4*)other, (f32x4*)gx, accum);
        return pk::launch_status("pk_binary_bwd_f32");
    }
    if(kept_like_out && reduced_first) {  // R = 1 when nothing is reduced
        binary_bwd_rows<<<pk::grid_for(x_numel, NT), NT, 0, st>>>(op, which, d.red_numel, x_numel,
                                                                  gout, other, gx, accum);
        return pk::launch_status("pk_binary_bwd_f32");
    }
    binary_bwd_reduce<<<pk::grid_for(x_numel, NT), NT, 0, st>>>(op, which, d, x_numel, gout,
                                                                  other, gx, accum);
    return pk::launch_status("pk_binary_bwd_f32");
}

extern "C" int pk_unary_f32(int op, int64_t n, const float* x, float* y, pk_stream_t stream) {
    if(!valid_op(op, 5)) return pk::fail("pk_unary_f32: op %d not in 0..5", op);
    if(n <= 0) return n < 0 ? pk::fail("pk_unary_f32: negative n") : PK_OK;
    if(!x || !y) return pk::fail("pk_unary_f32: NULL pointer");
    unary_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(op, n, x, y);
    return pk::launch_status("pk_unary_f32");
}

extern "C" int pk_unary_bwd_f32(int op, int64_t n, const float* x, const float* y, const float* gy,
                                float* gx, int flags, pk_stream_t stream) {
    if(!valid_op(op, 5)) return pk::fail("pk_unary_bwd_f32: op %d not in 0..5", op);
    if(n <= 0) return n < 0 ? pk::fail("pk_unary_bwd_f32: negative n") : PK_OK;
    if(!x || !y || !gy || !gx) return pk::fail("pk_unary_bwd_f32: NULL pointer");
    unary_bwd_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(op, n, x, y, gy, gx,
                                                                           flags & PK_ACCUM);
    return pk::launch_status("pk_unary_bwd_f32");
}

extern "C" int pk_relu_f32(int64_t n, const float* x, float* y, pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_relu_f32: negative n") : PK_OK;
    if(!x || !y) return pk::fail("pk_relu_f32: NULL pointer");
    relu_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(n, x, y);
    return pk::launch_status("pk_relu_f32");
}

extern "C" int pk_relu_bwd_f32(int64_t n, const float* y, const float* gy, float* gx, int flags,
                               pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_relu_bwd_f32: negative n") : PK_OK;
    if(!y || !gy || !gx) return pk::fail("pk_relu_bwd_f32: NULL pointer");
    relu_bwd_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(n, y, gy, gx,
                                                                          flags & PK_ACCUM);
    return pk::launch_status("pk_relu_bwd_f32");
}

extern "C" int pk_fill_f32(int64_t n, float value, float* x, pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_fill_f32: negative n") : PK_OK;
    if(!x) return pk::fail("pk_fill_f32: NULL pointer");
    fill_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(n, value, x);
    return pk::launch_status("pk_fill_f32");
}

extern "C" int pk_fill2d_f32(int64_t rows, int64_t cols, float value, float* x, int64_t ld,
                             pk_stream_t stream) {
    if(rows < 0 || cols < 0 || (rows > 1 && ld < cols)) return pk::fail("pk_fill2d_f32: bad sizes");
    if(rows == 0 || cols == 0) return PK_OK;
    if(!x) return pk::fail("pk_fill2d_f32: NULL pointer");
    fill2d_kernel<<<pk::grid_for(rows * cols, NT), NT, 0, pk::as_stream(stream)>>>(rows, cols,
                                                                                 value, x, ld);
    return pk::launch_status("pk_fill2d_f32");
}

extern "C" int pk_fill_normal_f32(int64_t n, uint64_t seed, float mean, float std, float* x,
                                  pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_fill_normal_f32: negative n") : PK_OK;
    if(!x) return pk::fail("pk_fill_normal_f32: NULL pointer");
    fill_normal_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(n, seed, mean, std,
                                                                             x);
    return pk::launch_status("pk_fill_normal_f32");
}

extern "C" int pk_axpy_f32(int64_t n, float alpha, const float* alpha_dev, const float* x, float* y,
                           int flags, pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_axpy_f32: negative n") : PK_OK;
    if(!x || !y) return pk::fail("pk_axpy_f32: NULL pointer");
    axpy_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(n, alpha, alpha_dev, x, y,
                                                                       flags & PK_ACCUM);
    return pk::launch_status("pk_axpy_f32");
}

extern "C" int pk_reduce_sum_f32(int64_t n, const float* x, float scale, float* out, int flags,
                                 pk_stream_t stream) {
    if(n < 0) return pk::fail("pk_reduce_sum_f32: negative n");
    if(!out || (n > 0 && !x)) return pk::fail("pk_reduce_sum_f32: NULL pointer");
    sum_kernel<<<1, 1024, 0, pk::as_stream(stream)>>>(n, x, scale, out, flags & PK_ACCUM);
    return pk::launch_status("pk_reduce_sum_f32");
}

extern "C" int pk_sgd_f32(int64_t n, float lr, float* p, const float* g, pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_sgd_f32: negative n") : PK_OK;
    if(!p || !g) return pk::fail("pk_sgd_f32: NULL pointer");
    sgd_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(n, lr, p, g);
    return pk::launch_status("pk_sgd_f32");
}

extern "C" int pk_sgd_multi_f32(int count, float* const* p, const float* const* g,
                                const int64_t* n, float lr, pk_stream_t stream) {
    if(count < 0) return pk::fail("pk_sgd_multi_f32: negative count");
    if(count > 0 && (!p || !g || !n)) return pk::fail("pk_sgd_multi_f32: NULL array");
    for(int base = 0; base < count; base += kSgdMax) {
        SgdBatch b = {};
        int k = 0;
        int64_t most = 0;
        for(int i = base; i < count && i < base + kSgdMax; ++i) {
            if(n[i] < 0) return pk::fail("pk_sgd_multi_f32: tensor %d has a negative size", i);
            if(n[i] == 0) continue;
            if(!p[i] || !g[i]) return pk::fail("pk_sgd_multi_f32: tensor %d has a NULL pointer", i);
            b.p[k] = p[i];
            b.g[k] = g[i];
            b.n[k] = n[i];
            most = n[i] > most ? n[i] : most;
            ++k;
        }
        if(k == 0) continue;
        sgd_multi_kernel<<<dim3(pk::grid_for(most, NT), k), NT, 0, pk::as_stream(stream)>>>(b, lr);
        const int rc = pk::launch_status("pk_sgd_multi_f32");
        if(rc) return rc;
    }
    return PK_OK;
}

extern "C" int pk_adamw_f32(int64_t n, float lr, float beta1, float beta2, float eps,
                            float weight_decay, int step, float* p, const float* g, float* m,
                            float* v, pk_stream_t stream) {
    if(n <= 0) return n < 0 ? pk::fail("pk_adamw_f32: negative n") : PK_OK;
    if(step < 1) return pk::fail("pk_adamw_f32: step %d must be >= 1", step);
    if(!p || !m || !v) return pk::fail("pk_adamw_f32: NULL pointer");
    const double bc1 = 1.0 - pow((double)beta1, (double)step);
    const double bc2 = 1.0 - pow((double)beta2, (double)step);
    const float step_size = (float)((double)lr / bc1);
    const float bc2_sqrt = (float)sqrt(bc2);
    const float decay = 1.0f - lr * weight_decay;
    adamw_kernel<<<pk::grid_for(n, NT), NT, 0, pk::as_stream(stream)>>>(
        n, beta1, beta2, eps, decay, step_size, bc2_sqrt, p, g, m, v);
    return pk::launch_status("pk_adamw_f32");
}

extern "C" int pk_adamw_prep_f32(int32_t* step, float lr, float beta1, float beta2,
                                 float* coef, pk_stream_t stream) {
    if(!step || !coef) return pk::fail("pk_adamw_prep_f32: NULL pointer");
    adamw_prep_kernel<<<1, 64, 0, pk::as_stream(stream)>>>(step, lr, beta1, beta2, coef);
    return pk::launch_status("pk_adamw_prep_f32");
}

extern "C" int pk_adamw_multi_f32(int64_t nchunks, const PkAdamwChunk* chunks, float lr,
                                  float beta1, float beta2, float eps, float weight_decay,
                                  const float* coef, pk_stream_t stream) {
    if(nchunks < 0) return pk::fail("pk_adamw_multi_f32: negative chunk count");
    if(nchunks == 0) return PK_OK;
    if(!chunks || !coef) return pk::fail("pk_adamw_multi_f32: NULL pointer");
    if(nchunks > 0x7fffffff) return pk::fail("pk_adamw_multi_f32: too many chunks");
    const float decay = 1.0f - lr * weight_decay;
    if(nchunks > 0x7fffffff / kAdamwSplit) return pk::fail("pk_adamw_multi_f32: too many chunks");
    adamw_multi_kernel<<<(unsigned)(nchunks * kAdamwSplit), 256, 0, pk::as_stream(stream)>>>(
        chunks, beta1, beta2, eps, decay, coef);
    return pk::launch_status("pk_adamw_multi_f32");
}

extern "C" int pk_embed_fwd_f32(int64_t n, int64_t d, int64_t vocab, const int32_t* ids,
                                const float* table, float* out, pk_stream_t stream) {
    if(n < 0 || d < 0 || vocab < 0) return pk::fail("pk_embed_fwd_f32: negative size");
    if(n == 0 || d == 0) return PK_OK;
    if(!ids || !table || !out) return pk::fail("pk_embed_fwd_f32: NULL pointer");
    hipStream_t st = pk::as_stream(stream);
    if(d % 4 == 0 && pk::aligned16(table) && pk::aligned16(out))
        embed_fwd4_kernel<<<pk::grid_for(n * d / 4, NT), NT, 0, st>>>(
            n, d / 4, vocab, ids, (const f32x4*)table, (f32x4*)out);
    else
        embed_fwd_kernel<<<pk::grid_for(n * d, NT), NT, 0, st>>>(n, d, vocab, ids, table, out);
    return pk::launch_status("pk_embed_fwd_f32");
}

// keys and positions, twice (the passes ping-pong), then the histogram
extern "C" size_t pk_embed_bwd_workspace(int64_t n) {
    if(n <= 0) return 0;
    const int64_t blocks = (n + kSortTile - 1) / kSortTile;
    return (size_t)(4 * n + kDigits * blocks) * sizeof(int32_t) + 256;
}
extern "C" int pk_embed_bwd_f32(int64_t n, int64_t d, int64_t vocab, const int32_t* ids,
                                const float* dout, float* dtable, void* workspace,
                                size_t workspace_bytes, pk_stream_t stream) {
    if(n < 0 || d < 0 || vocab < 0) return pk::fail("pk_embed_bwd_f32: negative size");
    if(n == 0 || d == 0) return PK_OK;
    if(!ids || !dout || !dtable) return pk::fail("pk_embed_bwd_f32: NULL pointer");
    if(n > 0x7fffffff) return pk::fail("pk_embed_bwd_f32: more than 2^31 - 1 ids");
    if(vocab > 0x7fffffff) return pk::fail("pk_embed_bwd_f32: vocab above 2^31 - 1");
    if(!workspace || workspace_bytes < pk_embed_bwd_workspace(n))
        return pk::fail("pk_embed_bwd_f32: workspace of %zu bytes, %zu needed", workspace_bytes,
                        pk_embed_bwd_workspace(n));
    const int64_t blocks = (n + kSortTile - 1) / kSortTile;
    int32_t* base = static_cast<int32_t*>(workspace);
    int32_t *ka = base, *va = base + n, *kb = base + 2 * n, *vb = base + 3 * n;
    int32_t* hist = base + 4 * n;
    int bits = 1;  // keys run 0..vocab
    while(bits < 31 && ((int64_t)1 << bits) <= vocab) ++bits;
    hipStream_t st = pk::as_stream(stream);
    const int32_t *kin = nullptr, *vin = nullptr;  // the first pass reads ids
    int32_t *kout = ka, *vout = va;
    for(int shift = 0; shift < bits; shift += 8) {
        radix_hist_kernel<<<(unsigned)blocks, kSortThreads, 0, st>>>(n, vocab, ids, kin, shift,
                                                                    hist);
        radix_scan_kernel<<<1, kScanThreads, 0, st>>>(kDigits * blocks, hist);
        radix_scatter_kernel<<<(unsigned)blocks, kSortThreads, 0, st>>>(
            n, vocab, ids, kin, vin, shift, hist, kout, vout);
        kin = kout;
        vin = vout;
        kout = kout == ka ? kb : ka;
        vout = vout == va ? vb : va;
    }
    embed_sum_kernel<<<(unsigned)n, 256, 0, st>>>(n, d, vocab, kin, vin, dout, dtable);
    return pk::launch_status("pk_embed_bwd_f32");
}
