// pico_amd/csrc/rows.hip -- fused row kernels: softmax cross-entropy, argmax,
// RMSNorm fwd/bwd, SwiGLU fwd/bwd, and the causal softmax of attention.
//
// All of these are HBM-bound.  Each row is loaded once with 128-bit loads into
// registers (one 64-lane wave per row for rows up to 8192 floats, one
// workgroup per row for the 32000-wide logits), reduced with cross-lane
// shuffles, and written once.  Rows whose width is not a multiple of 4, or
// whose base is not 16-byte aligned, or that do not fit the register cache,
// take a scalar two-pass path that re-reads the row.
#include <math.h>

#include "pk_common.h"

namespace {

constexpr float kNegInf = -INFINITY;

// ============================================================ cross-entropy
// One workgroup of NT threads per row, each thread caching NV float4 of the row
// in registers: max, one exponential per element (kept for the gradient), sum,
// gradient, store.  Measured on MI355X at 8192 x 32000, the row in registers
// beat 1024 threads walking rows with a prefetch (70 % vs 61 % of HBM peak):
// more independent workgroups per CU, cheaper reductions.  Rows of 16 K-32 K
// floats take 512 threads of 16 float4 rather than 256 of 32 (72.4 % vs
// 71.0 %: half the registers per lane, so more rows in flight per CU).
template <int NT, int NV>
__global__ __launch_bounds__(NT) void xent_reg_kernel(int64_t V, const float* __restrict__ logits,
                                                      int64_t ldz, const int32_t* __restrict__ labels,
                                                      float* __restrict__ loss_rows,
                                                      float* __restrict__ dlogits, int64_t ldd,
                                                      float scale_in,
                                                      const float* __restrict__ scale_dev,
                                                      int accum) {
    __shared__ float red[2][NT / 64];
    const float scale = scale_dev ? scale_in * *scale_dev : scale_in;
    const int64_t r = blockIdx.x, V4 = V / 4;
    const f32x4* z4 = reinterpret_cast<const f32x4*>(logits + r * ldz);
    f32x4 z[NV];
#pragma unroll
    for(int i = 0; i < NV; ++i) {
        const int64_t c = threadIdx.x + (int64_t)i * NT;
        z[i] = c < V4 ? pk::ld_stream(z4 + c) : f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    }
    float m = kNegInf;
#pragma unroll
    for(int v = 0; v < NV; ++v)
        m = fmaxf(m, fmaxf(fmaxf(z[v][0], z[v][1]), fmaxf(z[v][2], z[v][3])));
    m = pk::block_max<NT / 64>(m, red[0]);
    float s = 0.0f;
#pragma unroll
    for(int v = 0; v < NV; ++v)
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            z[v][e] = __expf(z[v][e] - m);
            s += z[v][e];
        }
    s = pk::block_sum<NT / 64>(s, red[1]);
    const float lse = m + logf(s);
    const int32_t y = labels[r];
    const bool ok = y >= 0 && y < V;
    if(loss_rows && threadIdx.x == 0) loss_rows[r] = ok ? lse - logits[r * ldz + y] : NAN;
    if(!dlogits) return;
    f32x4* d4 = reinterpret_cast<f32x4*>(dlogits + r * ldd);
    const float ps = scale / s;
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = threadIdx.x + (int64_t)v * NT;
        if(c >= V4) continue;
        f32x4 g;
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            const int64_t col = c * 4 + e;
            g[e] = ok ? z[v][e] * ps - (col == y ? scale : 0.0f) : 0.0f;
        }
        if(accum) g = g + d4[c];
        pk::st_stream(d4 + c, g);
    }
}

// any width: online max/sum pass, then a second pass writes the gradient
template <int NT>
__global__ __launch_bounds__(NT) void xent_any_kernel(int64_t V, const float* __restrict__ logits,
                                                      int64_t ldz, const int32_t* __restrict__ labels,
                                                      float* __restrict__ loss_rows,
                                                      float* __restrict__ dlogits, int64_t ldd,
                                                      float scale_in,
                                                      const float* __restrict__ scale_dev,
                                                      int accum) {
    __shared__ float red[NT / 64];
    const float scale = scale_dev ? scale_in * *scale_dev : scale_in;
    const int64_t r = blockIdx.x;
    const float* z = logits + r * ldz;
    float m = kNegInf, s = 0.0f;
    for(int64_t c = threadIdx.x; c < V; c += NT) {
        const float x = z[c];
        if(x > m) {
            s = s * expf(m - x) + 1.0f;
            m = x;
        } else {
            s += expf(x - m);
        }
    }
    const float bm = pk::block_max<NT / 64>(m, red);
    s = (m == kNegInf) ? 0.0f : s * expf(m - bm);
    s = pk::block_sum<NT / 64>(s, red);
    const float lse = bm + logf(s);
    const int32_t y = labels[r];
    const bool ok = y >= 0 && y < V;
    if(loss_rows && threadIdx.x == 0) loss_rows[r] = ok ? lse - z[y] : NAN;
    if(!dlogits) return;
    float* d = dlogits + r * ldd;
    for(int64_t c = threadIdx.x; c < V; c += NT) {
        const float p = expf(z[c] - lse);
        float g = ok ? scale * (p - (c == y ? 1.0f : 0.0f)) : 0.0f;
        d[c] = accum ? d[c] + g : g;
    }
}

// Tiny problems (V <= 64, R <= 1024: a classifier head): every row in one
// workgroup, a wave per row with one class per lane, and the rows' mean in
// the same launch, summed as pk_reduce_sum_f32 sums.  The per-row arithmetic
// is xent_any_kernel's (its block reductions over one wave's values and
// zeros), so rows and gradients are the same bits.
constexpr int kTinyRows = 1024, kTinyV = 64;
__global__ __launch_bounds__(1024) void xent_tiny_kernel(int64_t R, int64_t V, const float* __restrict__ logits,
                                                         int64_t ldz, const int32_t* __restrict__ labels,
                                                         float* __restrict__ loss_rows,
                                                         float* __restrict__ dlogits, int64_t ldd,
                                                         float scale_in, const float* __restrict__ scale_dev,
                                                         int accum, float mean_scale, float* __restrict__ out,
                                                         int out_accum) {
    __shared__ float rows[kTinyRows];
    __shared__ float red[16];
    const float scale = scale_dev ? scale_in * *scale_dev : scale_in;
    const int w = threadIdx.x >> 6, c = threadIdx.x & 63;
    for(int64_t r = w; r < R; r += 16) {
        const float* z = logits + r * ldz;
        const float x = c < V ? z[c] : kNegInf;
        const float m = pk::wave_max(x);
        // a -inf logit adds nothing (an all -inf row: lse = -inf, as xent_any_kernel)
        const float s = pk::wave_sum(c < V && x != kNegInf ? expf(x - m) : 0.0f);
        const float lse = m + logf(s);
        const int32_t y = labels[r];
        const bool ok = y >= 0 && y < V;
        if(c == 0) {
            const float loss = ok ? lse - z[y] : NAN;
            rows[r] = loss;
            if(loss_rows) loss_rows[r] = loss;
        }
        if(dlogits && c < V) {
            const float p = expf(x - lse);
            const float g = ok ? scale * (p - (c == y ? 1.0f : 0.0f)) : 0.0f;
            float* d = dlogits + r * ldd + c;
            *d = accum ? *d + g : g;
        }
    }
    __syncthreads();
    const double sd = threadIdx.x < R ? (double)rows[threadIdx.x] : 0.0;
    const float v = pk::block_sum<16>((float)sd, red);
    if(threadIdx.x == 0) {
        const float t = mean_scale * v;
        out[0] = out_accum ? out[0] + t : t;
    }
}

// ================================================================== argmax
struct ArgBest {
    float v;
    int32_t i;
};
// a NaN is greater than every number; ties go to the smaller index
__device__ __forceinline__ bool better(float av, int32_t ai, float bv, int32_t bi) {
    const bool an = isnan(av), bn = isnan(bv);
    if(an || bn) return an && (!bn || ai < bi);
    if(av != bv) return av > bv;
    return ai < bi;
}

template <int NT>
__global__ __launch_bounds__(NT) void argmax_kernel(int64_t V, const float* __restrict__ x,
                                                    int64_t ldx, int32_t* __restrict__ idx) {
    __shared__ float rv[NT / 64];
    __shared__ int32_t ri[NT / 64];
    const float* z = x + blockIdx.x * ldx;
    float bv = 0.0f;
    int32_t bi = INT32_MAX;
    for(int64_t c = threadIdx.x; c < V; c += NT) {
        const float v = z[c];
        if(bi == INT32_MAX || better(v, (int32_t)c, bv, bi)) {
            bv = v;
            bi = (int32_t)c;
        }
    }
#pragma unroll
    for(int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int32_t oi = __shfl_xor(bi, o, 64);
        if(oi != INT32_MAX && (bi == INT32_MAX || better(ov, oi, bv, bi))) {
            bv = ov;
            bi = oi;
        }
    }
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    if(l == 0) {
        rv[w] = bv;
        ri[w] = bi;
    }
    __syncthreads();
    if(threadIdx.x == 0) {
        float fv = rv[0];
        int32_t fi = ri[0];
        for(int k = 1; k < NT / 64; ++k)
            if(ri[k] != INT32_MAX && (fi == INT32_MAX || better(rv[k], ri[k], fv, fi))) {
                fv = rv[k];
                fi = ri[k];
            }
        idx[blockIdx.x] = fi;
    }
}

// ================================================================= RMSNorm
// One wave per row, NV float4 per lane (row width C <= 256*NV, C % 4 == 0).
// Each wave walks rows gridDim.x*4 apart and loads its next row while it
// reduces and stores the current one, so loads and stores overlap.
template <int NV>
__device__ __forceinline__ void load_row4(const float* __restrict__ base, int64_t C4, int lane,
                                          f32x4 (&v)[NV]) {
    const f32x4* r = reinterpret_cast<const f32x4*>(base);
#pragma unroll
    for(int i = 0; i < NV; ++i) {
        const int64_t c = lane + i * 64;
        v[i] = c < C4 ? pk::ld_stream(r + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
}

template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_fwd_reg(int64_t R, int64_t C, float eps,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ y,
                                                       float* __restrict__ rstd) {
    const int lane = threadIdx.x % 64;
    const int64_t step = (int64_t)gridDim.x * 4;
    int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    if(row >= R) return;
    const int64_t C4 = C / 4;
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    f32x4 cur[NV], nxt[NV];
    load_row4<NV>(x + row * C, C4, lane, cur);
    for(; row < R; row += step) {
        const bool more = row + step < R;
        if(more) load_row4<NV>(x + (row + step) * C, C4, lane, nxt);
        float ss = 0.0f;
#pragma unroll
        for(int v = 0; v < NV; ++v)
            ss += cur[v][0] * cur[v][0] + cur[v][1] * cur[v][1] + cur[v][2] * cur[v][2] +
                  cur[v][3] * cur[v][3];
        ss = pk::wave_sum(ss);
        const float rs = 1.0f / sqrtf(ss / (float)C + eps);
        if(lane == 0 && rstd) rstd[row] = rs;
        f32x4* yr = reinterpret_cast<f32x4*>(y + row * C);
#pragma unroll
        for(int v = 0; v < NV; ++v) {
            const int64_t c = lane + v * 64;
            if(c < C4) pk::st_stream(yr + c, cur[v] * rs * g4[c]);
        }
        if(more) {
#pragma unroll
            for(int v = 0; v < NV; ++v) cur[v] = nxt[v];
        }
    }
}

// Wide rows (C4 = C/4 >= 512): the 4 waves of a workgroup share each row (wave
// w owns float4 columns [w*Q, (w+1)*Q), Q = ceil(C4/4)), combine the sum of
// squares through LDS (one barrier per row, double-buffered), and walk rows
// gridDim.x apart with the next row prefetched.  Measured at 8192 x 4096: 76 %
// of HBM peak, against 67-71 % for one wave per row.
template <int NQ, bool EXACT>
__global__ __launch_bounds__(256) void rmsnorm_fwd_cols(int64_t R, int64_t C, float eps,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ g,
                                                        float* __restrict__ y,
                                                        float* __restrict__ rstd) {
    __shared__ float red[2][4];
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t C4 = C / 4, Q = (C4 + 3) / 4, c0 = w * Q;
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g) + c0;
    // EXACT: C is a multiple of 1024, so every lane owns NQ whole float4s and
    // the loads and stores need no predicates
    bool on[NQ];
#pragma unroll
    for(int v = 0; v < NQ; ++v) {
        const int64_t q = lane + v * 64;
        on[v] = EXACT || (q < Q && c0 + q < C4);
    }
    f32x4 xv[NQ], xn[NQ];
    auto load = [&](int64_t r, f32x4 (&a)[NQ]) {
        const f32x4* xr = reinterpret_cast<const f32x4*>(x + r * C) + c0;
#pragma unroll
        for(int v = 0; v < NQ; ++v)
            a[v] = on[v] ? pk::ld_stream(xr + lane + v * 64) : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    int64_t row = blockIdx.x;
    if(row < R) load(row, xv);
    for(int it = 0; row < R; row += gridDim.x, ++it) {
        const bool more = row + gridDim.x < R;
        if(more) load(row + gridDim.x, xn);
        float ss = 0.0f;
#pragma unroll
        for(int v = 0; v < NQ; ++v)
            ss += xv[v][0] * xv[v][0] + xv[v][1] * xv[v][1] + xv[v][2] * xv[v][2] +
                  xv[v][3] * xv[v][3];
        ss = pk::wave_sum(ss);
        if(lane == 0) red[it & 1][w] = ss;
        __syncthreads();
        ss = ((red[it & 1][0] + red[it & 1][1]) + red[it & 1][2]) + red[it & 1][3];
        const float rs = 1.0f / sqrtf(ss / (float)C + eps);
        if(threadIdx.x == 0 && rstd) rstd[row] = rs;
        f32x4* yr = reinterpret_cast<f32x4*>(y + row * C) + c0;
#pragma unroll
        for(int v = 0; v < NQ; ++v)
            if(on[v]) pk::st_stream(yr + lane + v * 64, xv[v] * rs * g4[lane + v * 64]);
        if(more) {
#pragma unroll
            for(int v = 0; v < NQ; ++v) xv[v] = xn[v];
        }
    }
}

__global__ __launch_bounds__(256) void rmsnorm_fwd_any(int64_t R, int64_t C, float eps,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ y,
                                                       float* __restrict__ rstd) {
    const int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if(row >= R) return;
    const float* xr = x + row * C;
    float ss = 0.0f;
    for(int64_t c = lane; c < C; c += 64) ss += xr[c] * xr[c];
    ss = pk::wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / (float)C + eps);
    if(lane == 0 && rstd) rstd[row] = rs;
    for(int64_t c = lane; c < C; c += 64) y[row * C + c] = xr[c] * rs * g[c];
}

// The backward runs on the training step's critical stream while the weight
// gradients' matrix products run beside it on the same CUs.  On gfx950 a
// wave's VALU instructions do not issue while another wave's MFMAs hold the
// SIMD's matrix pipe, so at the default priority these rows got a few percent
// of the issue cycles (about 200 us per call in a config-5 step against 20
// alone).  Its waves take the top issue priority: 118 us per call in the step,
// which measured 0.1 ms faster.  Alone it changes nothing.
__device__ __forceinline__ void rows_beside_products() { __builtin_amdgcn_s_setprio(3); }

// backward, stage 1: dx for each row, and this workgroup's partial of dg
// (over the rows it walked) into ws[block][C].  Internal flags: 4 = write dx,
// 8 = produce dg partials, bit 0 = accumulate dx.
//
// Narrow rows (C <= 256*NV): one wave per row, rows gridDim.x*4 apart, the
// next row's x and dy prefetched while the current one is finished; the 4
// waves' dg partials are combined in LDS in a fixed order.
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_reg(int64_t R, int64_t C,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       const float* __restrict__ rstd,
                                                       const float* __restrict__ dy,
                                                       const float* dxin, float* dx,
                                                       float* __restrict__ ws, int flags) {
    rows_beside_products();
    extern __shared__ float part[];  // C floats
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t C4 = C / 4;
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    f32x4 gv[NV], dg[NV];
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        gv[v] = c < C4 ? g4[c] : f32x4{0.f, 0.f, 0.f, 0.f};
        dg[v] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float invC = 1.0f / (float)C;
    const int64_t step = (int64_t)gridDim.x * 4;
    int64_t row = (int64_t)blockIdx.x * 4 + w;
    f32x4 xv[NV], dv[NV], xn[NV], dn[NV];
    if(row < R) {
        load_row4<NV>(x + row * C, C4, lane, xv);
        load_row4<NV>(dy + row * C, C4, lane, dv);
    }
    for(; row < R; row += step) {
        const bool more = row + step < R;
        if(more) {
            load_row4<NV>(x + (row + step) * C, C4, lane, xn);
            load_row4<NV>(dy + (row + step) * C, C4, lane, dn);
        }
        float dot = 0.0f;
#pragma unroll
        for(int v = 0; v < NV; ++v) {
            const f32x4 t = gv[v] * dv[v] * xv[v];
            dot += t[0] + t[1] + t[2] + t[3];
        }
        dot = pk::wave_sum(dot);
        const float rs = rstd[row];
        const float k = rs * rs * rs * dot * invC;
        f32x4* dxr = reinterpret_cast<f32x4*>(dx + row * C);
        const f32x4* dxi = reinterpret_cast<const f32x4*>(dxin + row * C);
#pragma unroll
        for(int v = 0; v < NV; ++v) {
            const int64_t c = lane + v * 64;
            if(c < C4) {
                if(flags & 4) {
                    f32x4 o = rs * gv[v] * dv[v] - xv[v] * k;
                    if(flags & PK_ACCUM) o = o + dxi[c];
                    pk::st_stream(dxr + c, o);
                }
                dg[v] = dg[v] + dv[v] * xv[v] * rs;
            }
        }
        if(more) {
#pragma unroll
            for(int v = 0; v < NV; ++v) {
                xv[v] = xn[v];
                dv[v] = dn[v];
            }
        }
    }
    if(!(flags & 8)) return;  // dg not requested
    // combine the 4 waves' partials in LDS, one wave at a time
    for(int ww = 0; ww < 4; ++ww) {
        if(w == ww) {
#pragma unroll
            for(int v = 0; v < NV; ++v) {
                const int64_t c = lane + v * 64;
                if(c < C4) {
                    f32x4* p = reinterpret_cast<f32x4*>(part) + c;
                    *p = ww == 0 ? dg[v] : *p + dg[v];
                }
            }
        }
        __syncthreads();
    }
    f32x4* out = reinterpret_cast<f32x4*>(ws + (int64_t)blockIdx.x * C);
    for(int64_t c = threadIdx.x; c < C4; c += 256) out[c] = reinterpret_cast<f32x4*>(part)[c];
}

// Wide rows (C4 = C/4 >= 512): the 4 waves of a workgroup share each row, wave w
// owning the float4 columns [w*Q, (w+1)*Q), Q = ceil(C4/4), NQ float4 per lane.
// The row's dot product is combined across waves through LDS (one barrier per
// row, double-buffered); each wave keeps dg for its own columns, so the
// workgroup's partial needs no combine.  The next row is prefetched.
template <int NQ, bool EXACT>
__global__ __launch_bounds__(256) void rmsnorm_bwd_cols(int64_t R, int64_t C,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ g,
                                                        const float* __restrict__ rstd,
                                                        const float* __restrict__ dy,
                                                        const float* dxin, float* dx,
                                                        float* __restrict__ ws, int flags) {
    rows_beside_products();
    __shared__ float red[2][4];
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t C4 = C / 4, Q = (C4 + 3) / 4;
    const int64_t c0 = w * Q;
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    f32x4 gv[NQ], dg[NQ];
    bool on[NQ];
#pragma unroll
    for(int v = 0; v < NQ; ++v) {
        const int64_t q = lane + v * 64, c = c0 + q;
        on[v] = EXACT || (q < Q && c < C4);
        gv[v] = on[v] ? g4[c] : f32x4{0.f, 0.f, 0.f, 0.f};
        dg[v] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float invC = 1.0f / (float)C;
    f32x4 xv[NQ], dv[NQ], xn[NQ], dn[NQ];
    auto load = [&](int64_t r, f32x4 (&a)[NQ], f32x4 (&b)[NQ]) {
        const f32x4* xr = reinterpret_cast<const f32x4*>(x + r * C) + c0;
        const f32x4* dr = reinterpret_cast<const f32x4*>(dy + r * C) + c0;
#pragma unroll
        for(int v = 0; v < NQ; ++v) {
            const int64_t q = lane + v * 64;
            a[v] = on[v] ? pk::ld_stream(xr + q) : f32x4{0.f, 0.f, 0.f, 0.f};
            b[v] = on[v] ? pk::ld_stream(dr + q) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    int64_t row = blockIdx.x;
    if(row < R) load(row, xv, dv);
    for(int it = 0; row < R; row += gridDim.x, ++it) {
        const bool more = row + gridDim.x < R;
        if(more) load(row + gridDim.x, xn, dn);
        float dot = 0.0f;
#pragma unroll
        for(int v = 0; v < NQ; ++v) {
            const f32x4 t = gv[v] * dv[v] * xv[v];
            dot += t[0] + t[1] + t[2] + t[3];
        }
        dot = pk::wave_sum(dot);
        if(lane == 0) red[it & 1][w] = dot;
        __syncthreads();
        dot = ((red[it & 1][0] + red[it & 1][1]) + red[it & 1][2]) + red[it & 1][3];
        const float rs = rstd[row];
        const float k = rs * rs * rs * dot * invC;
        f32x4* dxr = reinterpret_cast<f32x4*>(dx + row * C) + c0;
        const f32x4* dxi = reinterpret_cast<const f32x4*>(dxin + row * C) + c0;
#pragma unroll
        for(int v = 0; v < NQ; ++v) {
            if(!on[v]) continue;
            const int64_t q = lane + v * 64;
            if(flags & 4) {
                f32x4 o = rs * gv[v] * dv[v] - xv[v] * k;
                if(flags & PK_ACCUM) o = o + dxi[q];
                pk::st_stream(dxr + q, o);
            }
            dg[v] = dg[v] + dv[v] * xv[v] * rs;
        }
        if(more) {
#pragma unroll
            for(int v = 0; v < NQ; ++v) {
                xv[v] = xn[v];
                dv[v] = dn[v];
            }
        }
    }
    if(!(flags & 8)) return;
    f32x4* out = reinterpret_cast<f32x4*>(ws + (int64_t)blockIdx.x * C) + c0;
#pragma unroll
    for(int v = 0; v < NQ; ++v)
        if(on[v]) out[lane + v * 64] = dg[v];
}

__global__ __launch_bounds__(256) void rmsnorm_bwd_any(int64_t R, int64_t C,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       const float* __restrict__ rstd,
                                                       const float* __restrict__ dy,
                                                       const float* dxin, float* dx,
                                                       float* __restrict__ ws, int flags) {
    rows_beside_products();
    // one wave per row for dx; dg partials accumulated per block column-wise
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const float invC = 1.0f / (float)C;
    for(int64_t row = (int64_t)blockIdx.x * 4 + w; row < R; row += (int64_t)gridDim.x * 4) {
        const float* xr = x + row * C;
        const float* dyr = dy + row * C;
        float dot = 0.0f;
        for(int64_t c = lane; c < C; c += 64) dot += g[c] * dyr[c] * xr[c];
        dot = pk::wave_sum(dot);
        const float rs = rstd[row];
        const float k = rs * rs * rs * dot * invC;
        if(flags & 4)
            for(int64_t c = lane; c < C; c += 64) {
                float o = rs * g[c] * dyr[c] - xr[c] * k;
                dx[row * C + c] = (flags & PK_ACCUM) ? dxin[row * C + c] + o : o;
            }
    }
    if(!(flags & 8)) return;
    // partial dg of this block's rows: thread per column, rows of this block in order
    for(int64_t c = threadIdx.x; c < C; c += 256) {
        float acc = 0.0f;
        for(int64_t row = (int64_t)blockIdx.x * 4; row < R; row += (int64_t)gridDim.x * 4)
            for(int ww = 0; ww < 4 && row + ww < R; ++ww)
                acc += dy[(row + ww) * C + c] * x[(row + ww) * C + c] * rstd[row + ww];
        ws[(int64_t)blockIdx.x * C + c] = acc;
    }
}

// backward, stage 2: dg (+)= sum over the partial rows.  64 columns per
// block; its 16 waves each sum every 16th partial row (independent loads, so
// they are in flight together), then the 16 sums are combined in a fixed order.
constexpr int kColsumWaves = 16;
__global__ __launch_bounds__(64 * kColsumWaves) void colsum_kernel(int64_t P, int64_t C,
                                                                 const float* __restrict__ ws,
                                                                 float* __restrict__ dg,
                                                                 int accum) {
    __shared__ float part[kColsumWaves][64];
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if(c < C) {
#pragma unroll 8
        for(int64_t p = w; p < P; p += kColsumWaves) acc += ws[p * C + c];
    }
    part[w][lane] = acc;
    __syncthreads();
    if(w == 0 && c < C) {
        float s = part[0][lane];
#pragma unroll
        for(int i = 1; i < kColsumWaves; ++i) s += part[i][lane];
        dg[c] = accum ? dg[c] + s : s;
    }
}

int64_t rms_parts(int64_t R) {
    const int64_t blocks = (R + 3) / 4;
    return blocks < 512 ? blocks : 512;
}

// ================================================================== SwiGLU

__global__ void swiglu_fwd4(int64_t n4, const f32x4* __restrict__ a, const f32x4* __restrict__ u,
                            f32x4* __restrict__ h) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
        i += (int64_t)gridDim.x * blockDim.x) {
        const f32x4 av = pk::ld_stream(a + i), uv = pk::ld_stream(u + i);
        f32x4 o;
#pragma unroll
        for(int e = 0; e < 4; ++e) o[e] = pk::swiglu_fwd1(av[e], uv[e]);
        pk::st_stream(h + i, o);
    }
}

__global__ void swiglu_fwd_any(int64_t R, int64_t F, const float* __restrict__ a, int64_t lda,
                               const float* __restrict__ u, int64_t ldu, float* __restrict__ h,
                               int64_t ldh) {
    const int64_t n = R * F;
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / F, c = i % F;
        const float av = a[r * lda + c];
        h[r * ldh + c] = pk::swiglu_fwd1(av, u[r * ldu + c]);
    }
}

__global__ void swiglu_bwd4(int64_t n4, const f32x4* __restrict__ a, const f32x4* __restrict__ u,
                            const f32x4* __restrict__ dh, f32x4* __restrict__ da,
                            f32x4* __restrict__ du, int flags) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
        i += (int64_t)gridDim.x * blockDim.x) {
        const f32x4 av = pk::ld_stream(a + i), uv = pk::ld_stream(u + i), g = pk::ld_stream(dh + i);
        f32x4 ga, gu;
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            float x, y;
            pk::swiglu_bwd1(av[e], uv[e], g[e], x, y);
            ga[e] = x;
            gu[e] = y;
        }
        if(flags & (PK_ACCUM | PK_ACCUM2)) {
            const f32x4 pa = (flags & PK_ACCUM) ? da[i] : f32x4{0.f, 0.f, 0.f, 0.f};
            const f32x4 pu = (flags & PK_ACCUM2) ? du[i] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for(int e = 0; e < 4; ++e) {
                if(flags & PK_ACCUM) ga[e] = pk::add_nc(pa[e], ga[e]);
                if(flags & PK_ACCUM2) gu[e] = pk::add_nc(pu[e], gu[e]);
            }
        }
        if(flags & 4) pk::st_stream(da + i, ga);
        if(flags & 8) pk::st_stream(du + i, gu);
    }
}

// Row-strided operands (the two halves of a fused [R, 2F] projection), F and
// every row stride a multiple of 4 and every base 16-byte aligned: block
// (x, y) covers float4 columns 256x.. of rows y, y + gridDim.y, ...
__global__ void swiglu_fwd_rows4(int64_t R, int64_t F4, const float* __restrict__ a, int64_t lda,
                                 const float* __restrict__ u, int64_t ldu, float* __restrict__ h,
                                 int64_t ldh) {
    const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if(c >= F4) return;
    for(int64_t r = blockIdx.y; r < R; r += gridDim.y) {
        const f32x4 av = pk::ld_stream(reinterpret_cast<const f32x4*>(a + r * lda) + c);
        const f32x4 uv = pk::ld_stream(reinterpret_cast<const f32x4*>(u + r * ldu) + c);
        f32x4 o;
#pragma unroll
        for(int e = 0; e < 4; ++e) o[e] = pk::swiglu_fwd1(av[e], uv[e]);
        pk::st_stream(reinterpret_cast<f32x4*>(h + r * ldh) + c, o);
    }
}

__global__ void swiglu_bwd_rows4(int64_t R, int64_t F4, const float* __restrict__ a, int64_t lda,
                                 const float* __restrict__ u, int64_t ldu,
                                 const float* __restrict__ dh, int64_t ldh, float* __restrict__ da,
                                 float* __restrict__ du, int64_t ldd, int flags) {
    const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if(c >= F4) return;
    for(int64_t r = blockIdx.y; r < R; r += gridDim.y) {
        const f32x4 av = pk::ld_stream(reinterpret_cast<const f32x4*>(a + r * lda) + c);
        const f32x4 uv = pk::ld_stream(reinterpret_cast<const f32x4*>(u + r * ldu) + c);
        const f32x4 g = pk::ld_stream(reinterpret_cast<const f32x4*>(dh + r * ldh) + c);
        f32x4 ga, gu;
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            float x, y;
            pk::swiglu_bwd1(av[e], uv[e], g[e], x, y);
            ga[e] = x;
            gu[e] = y;
        }
        if(flags & 4) {
            f32x4* p = reinterpret_cast<f32x4*>(da + r * ldd) + c;
            if(flags & PK_ACCUM) {
                const f32x4 old = *p;
#pragma unroll
                for(int e = 0; e < 4; ++e) ga[e] = pk::add_nc(old[e], ga[e]);
            }
            pk::st_stream(p, ga);
        }
        if(flags & 8) {
            f32x4* p = reinterpret_cast<f32x4*>(du + r * ldd) + c;
            if(flags & PK_ACCUM2) {
                const f32x4 old = *p;
#pragma unroll
                for(int e = 0; e < 4; ++e) gu[e] = pk::add_nc(old[e], gu[e]);
            }
            pk::st_stream(p, gu);
        }
    }
}

dim3 rows4_grid(int64_t R, int64_t F4) {
    const int64_t gy = R < 8192 ? R : 8192;
    return dim3((unsigned)((F4 + 255) / 256), (unsigned)gy);
}

__global__ void swiglu_bwd_any(int64_t R, int64_t F, const float* __restrict__ a, int64_t lda,
                               const float* __restrict__ u, int64_t ldu,
                               const float* __restrict__ dh, int64_t ldh, float* __restrict__ da,
                               float* __restrict__ du, int64_t ldd, int flags) {
    const int64_t n = R * F;
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
        i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / F, c = i % F;
        const float av = a[r * lda + c], uv = u[r * ldu + c], g = dh[r * ldh + c];
        float ga, gu;
        pk::swiglu_bwd1(av, uv, g, ga, gu);
        const int64_t o = r * ldd + c;
        if(flags & 4) da[o] = (flags & PK_ACCUM) ? pk::add_nc(da[o], ga) : ga;
        if(flags & 8) du[o] = (flags & PK_ACCUM2) ? pk::add_nc(du[o], gu) : gu;
    }
}

// ========================================================= causal softmax
// rows of a [BH, T, T] score tensor; row i keeps columns j <= i.
// one wave per row, NV float4 per lane (T <= 256*NV, T % 4 == 0)
template <int NV>
__global__ __launch_bounds__(256) void csoftmax_fwd_reg(int64_t rows, int64_t T, float scale,
                                                        const float* __restrict__ S,
                                                        float* __restrict__ P,
                                                        float* __restrict__ lse) {
    const int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if(row >= rows) return;
    const int64_t i = row % T, T4 = T / 4;
    const f32x4* sr = reinterpret_cast<const f32x4*>(S + row * T);
    f32x4 s[NV];
    float m = kNegInf;
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        f32x4 t = {kNegInf, kNegInf, kNegInf, kNegInf};
        if(c < T4 && c * 4 <= i) {
            const f32x4 x = sr[c];
#pragma unroll
            for(int e = 0; e < 4; ++e)
                if(c * 4 + e <= i) t[e] = x[e] * scale;
        }
        s[v] = t;
        m = fmaxf(m, fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3])));
    }
    m = pk::wave_max(m);
    float sum = 0.0f;
#pragma unroll
    for(int v = 0; v < NV; ++v)
#pragma unroll
        for(int e = 0; e < 4; ++e) sum += expf(s[v][e] - m);
    sum = pk::wave_sum(sum);
    const float l = m + logf(sum);
    if(lane == 0 && lse) lse[row] = l;
    f32x4* pr = reinterpret_cast<f32x4*>(P + row * T);
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        if(c >= T4) continue;
        f32x4 o;
#pragma unroll
        for(int e = 0; e < 4; ++e) o[e] = expf(s[v][e] - l);  // exp(-inf) = 0 above the diagonal
        pr[c] = o;
    }
}

__global__ __launch_bounds__(256) void csoftmax_fwd_any(int64_t rows, int64_t T, float scale,
                                                        const float* __restrict__ S,
                                                        float* __restrict__ P,
                                                        float* __restrict__ lse) {
    const int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if(row >= rows) return;
    const int64_t i = row % T;
    const float* sr = S + row * T;
    float m = kNegInf;
    for(int64_t j = lane; j <= i; j += 64) m = fmaxf(m, sr[j] * scale);
    m = pk::wave_max(m);
    float sum = 0.0f;
    for(int64_t j = lane; j <= i; j += 64) sum += expf(sr[j] * scale - m);
    sum = pk::wave_sum(sum);
    const float l = m + logf(sum);
    if(lane == 0 && lse) lse[row] = l;
    // S may alias P: every lane reads its own columns before writing them
    for(int64_t j = lane; j < T; j += 64) P[row * T + j] = j <= i ? expf(sr[j] * scale - l) : 0.0f;
}

template <int NV>
__global__ __launch_bounds__(256) void csoftmax_bwd_reg(int64_t rows, int64_t T,
                                                        const float* __restrict__ P,
                                                        const float* dP, float* dS) {
    const int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if(row >= rows) return;
    const int64_t i = row % T, T4 = T / 4;
    const f32x4* pr = reinterpret_cast<const f32x4*>(P + row * T);
    const f32x4* dpr = reinterpret_cast<const f32x4*>(dP + row * T);
    f32x4 p[NV], d[NV];
    float D = 0.0f;
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        p[v] = f32x4{0.f, 0.f, 0.f, 0.f};
        d[v] = f32x4{0.f, 0.f, 0.f, 0.f};
        if(c < T4 && c * 4 <= i) {
            const f32x4 pv = pr[c], dv = dpr[c];
#pragma unroll
            for(int e = 0; e < 4; ++e)
                if(c * 4 + e <= i) {
                    p[v][e] = pv[e];
                    d[v][e] = dv[e];
                }
            const f32x4 t = p[v] * d[v];
            D += t[0] + t[1] + t[2] + t[3];
        }
    }
    D = pk::wave_sum(D);
    f32x4* out = reinterpret_cast<f32x4*>(dS + row * T);
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        if(c < T4) out[c] = p[v] * (d[v] - D);  // p is 0 above the diagonal
    }
}

__global__ __launch_bounds__(256) void csoftmax_bwd_any(int64_t rows, int64_t T,
                                                        const float* __restrict__ P,
                                                        const float* dP, float* dS) {
    const int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if(row >= rows) return;
    const int64_t i = row % T;
    float D = 0.0f;
    for(int64_t j = lane; j <= i; j += 64) D += P[row * T + j] * dP[row * T + j];
    D = pk::wave_sum(D);
    for(int64_t j = lane; j < T; j += 64) {
        const float v = j <= i ? P[row * T + j] * (dP[row * T + j] - D) : 0.0f;
        dS[row * T + j] = v;
    }
}

// pick the register-cache width: smallest NV in {1,2,4,8,16,32} with C <= 256*NV
int pick_nv(int64_t C) {
    for(int nv = 1; nv <= 32; nv *= 2)
        if(C <= 256 * nv) return nv;
    return 0;
}

}  // namespace

// =================================================================== C-ABI

extern "C" int pk_xent_fwd_bwd_f32(int64_t R, int64_t V, const float* logits, int64_t ldz,
                                   const int32_t* labels, float* loss_rows, float* dlogits,
                                   int64_t ldd, float scale, const float* scale_dev, int flags,
                                   pk_stream_t stream) {
    if(R < 0 || V < 1) return pk::fail("pk_xent_fwd_bwd_f32: need R >= 0 and V >= 1");
    if(R == 0) return PK_OK;
    if(R > 0x7fffffff) return pk::fail("pk_xent_fwd_bwd_f32: too many rows");
    if(!logits || !labels) return pk::fail("pk_xent_fwd_bwd_f32: NULL logits or labels");
    if(ldz < V || (dlogits && ldd < V)) return pk::fail("pk_xent_fwd_bwd_f32: row stride < V");
    hipStream_t st = pk::as_stream(stream);
    const int accum = flags & PK_ACCUM;
    const bool vec = V % 4 == 0 && ldz % 4 == 0 && pk::aligned16(logits) &&
                     (!dlogits || (ldd % 4 == 0 && pk::aligned16(dlogits)));
    const int64_t V4 = V / 4;
    dim3 grid((unsigned)R);
#define PK_XENT(NT_, NV_)                                                                       \
    xent_reg_kernel<NT_, NV_><<<grid, NT_, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, \
                                                    ldd, scale, scale_dev, accum)
    if(vec && V4 <= 256 * 1)
        PK_XENT(256, 1);
    else if(vec && V4 <= 256 * 2)
        PK_XENT(256, 2);
    else if(vec && V4 <= 256 * 4)
        PK_XENT(256, 4);
    else if(vec && V4 <= 256 * 8)
        PK_XENT(256, 8);
    else if(vec && V4 <= 256 * 16)
        PK_XENT(256, 16);
    else if(vec && V4 <= 512 * 16)
        PK_XENT(512, 16);
    else if(vec && V4 <= 1024 * 16)
        PK_XENT(1024, 16);
    else
        xent_any_kernel<1024><<<grid, 1024, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd,
                                                     scale, scale_dev, accum);
#undef PK_XENT
    return pk::launch_status("pk_xent_fwd_bwd_f32");
}

extern "C" int pk_xent_mean_f32(int64_t R, int64_t V, const float* logits, int64_t ldz,
                                const int32_t* labels, float* loss_rows, float* dlogits, int64_t ldd,
                                float scale, int flags, float mean_scale, float* out,
                                pk_stream_t stream) {
    if(R < 0 || V < 1) return pk::fail("pk_xent_mean_f32: need R >= 0 and V >= 1");
    if(!out) return pk::fail("pk_xent_mean_f32: NULL out");
    if(R > 0 && R <= kTinyRows && V <= kTinyV) {
        if(!logits || !labels) return pk::fail("pk_xent_mean_f32: NULL logits or labels");
        if(ldz < V || (dlogits && ldd < V)) return pk::fail("pk_xent_mean_f32: row stride < V");
        xent_tiny_kernel<<<1, 1024, 0, pk::as_stream(stream)>>>(R, V, logits, ldz, labels, loss_rows, dlogits,
                                                                ldd, scale, nullptr, flags & PK_ACCUM,
                                                                mean_scale, out, (flags & PK_ACCUM2) != 0);
        return pk::launch_status("pk_xent_mean_f32");
    }
    if(R > 0 && !loss_rows) return pk::fail("pk_xent_mean_f32: NULL loss_rows (needed above the tiny sizes)");
    if(int st = pk_xent_fwd_bwd_f32(R, V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, nullptr,
                                    flags & PK_ACCUM, stream))
        return st;
    return pk_reduce_sum_f32(R, loss_rows, mean_scale, out, (flags & PK_ACCUM2) ? PK_ACCUM : 0, stream);
}

extern "C" int pk_argmax_f32(int64_t R, int64_t V, const float* x, int64_t ldx, int32_t* idx,
                             pk_stream_t stream) {
    if(R < 0 || V < 1 || V > 0x7fffffff) return pk::fail("pk_argmax_f32: need R >= 0, 1 <= V < 2^31");
    if(R == 0) return PK_OK;
    if(!x || !idx || ldx < V) return pk::fail("pk_argmax_f32: NULL pointer or row stride < V");
    argmax_kernel<256><<<(unsigned)R, 256, 0, pk::as_stream(stream)>>>(V, x, ldx, idx);
    return pk::launch_status("pk_argmax_f32");
}

extern "C" int pk_rmsnorm_fwd_f32(int64_t R, int64_t C, float eps, const float* x, const float* g,
                                  float* y, float* rstd, pk_stream_t stream) {
    if(R < 0 || C < 1) return pk::fail("pk_rmsnorm_fwd_f32: need R >= 0 and C >= 1");
    if(R == 0) return PK_OK;
    if(!x || !g || !y) return pk::fail("pk_rmsnorm_fwd_f32: NULL pointer");
    hipStream_t st = pk::as_stream(stream);
    const bool vec = C % 4 == 0 && pk::aligned16(x) && pk::aligned16(g) && pk::aligned16(y);
    const int nv = vec ? pick_nv(C) : 0;
    const int64_t blocks = (R + 3) / 4;
    const unsigned grid = (unsigned)blocks;  // one row per wave
    if(vec && C / 4 >= 512 && C <= 16384) {
        const int64_t Q = (C / 4 + 3) / 4;
        const unsigned cgrid = (unsigned)(R < 512 ? R : 512);
#define PK_RMSF(NQ_)                                                                        \
    if(C % 1024 == 0 && Q == NQ_ * 64)                                                       \
        rmsnorm_fwd_cols<NQ_, true><<<cgrid, 256, 0, st>>>(R, C, eps, x, g, y, rstd);       \
    else                                                                                     \
        rmsnorm_fwd_cols<NQ_, false><<<cgrid, 256, 0, st>>>(R, C, eps, x, g, y, rstd)
        if(Q <= 128) {
            PK_RMSF(2);
        } else if(Q <= 256) {
            PK_RMSF(4);
        } else if(Q <= 512) {
            PK_RMSF(8);
        } else {
            PK_RMSF(16);
        }
#undef PK_RMSF
        return pk::launch_status("pk_rmsnorm_fwd_f32");
    }
    switch(nv) {
        case 1: rmsnorm_fwd_reg<1><<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd); break;
        case 2: rmsnorm_fwd_reg<2><<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd); break;
        case 4: rmsnorm_fwd_reg<4><<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd); break;
        case 8: rmsnorm_fwd_reg<8><<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd); break;
        case 16: rmsnorm_fwd_reg<16><<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd); break;
        case 32: rmsnorm_fwd_reg<32><<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd); break;
        default: rmsnorm_fwd_any<<<grid, 256, 0, st>>>(R, C, eps, x, g, y, rstd);
    }
    return pk::launch_status("pk_rmsnorm_fwd_f32");
}

extern "C" size_t pk_rmsnorm_bwd_workspace(int64_t R, int64_t C) {
    if(R <= 0 || C <= 0) return 0;
    return (size_t)rms_parts(R) * (size_t)C * sizeof(float);
}

extern "C" int pk_rmsnorm_bwd_f32(int64_t R, int64_t C, const float* x, const float* g,
                                  const float* rstd, const float* dy, float* dx, float* dg,
                                  int flags, void* workspace, size_t workspace_bytes,
                                  pk_stream_t stream) {
    return pk_rmsnorm_bwd_into_f32(R, C, x, g, rstd, dy, (flags & PK_ACCUM) ? dx : nullptr, dx,
                                   dg, flags & PK_ACCUM2, workspace, workspace_bytes, stream);
}

extern "C" int pk_rmsnorm_bwd_into_f32(int64_t R, int64_t C, const float* x, const float* g,
                                       const float* rstd, const float* dy, const float* dx_in,
                                       float* dx, float* dg, int flags, void* workspace,
                                       size_t workspace_bytes, pk_stream_t stream) {
    if(R < 0 || C < 1) return pk::fail("pk_rmsnorm_bwd_f32: need R >= 0 and C >= 1");
    if(R == 0) return PK_OK;
    if(!x || !g || !rstd || !dy) return pk::fail("pk_rmsnorm_bwd_f32: NULL input pointer");
    const bool parts = dg || (flags & PK_RMS_KEEP_PARTIALS);
    if(!dx && !parts) return PK_OK;
    const int64_t P = rms_parts(R);
    if(parts && (!workspace || workspace_bytes < pk_rmsnorm_bwd_workspace(R, C)))
        return pk::fail("pk_rmsnorm_bwd_f32: workspace needs %zu bytes",
                        pk_rmsnorm_bwd_workspace(R, C));
    hipStream_t st = pk::as_stream(stream);
    float* ws = (float*)workspace;
    // internal flags: 4 = write dx, 8 = produce dg partials; bit 0 = add dx_in
    const float* dxin = dx ? dx_in : nullptr;
    const int kf = (dxin ? PK_ACCUM : 0) | (dx ? 4 : 0) | (parts ? 8 : 0);
    const bool vec = C % 4 == 0 && pk::aligned16(x) && pk::aligned16(g) && pk::aligned16(dy) &&
                     (!dx || pk::aligned16(dx)) && (!dxin || pk::aligned16(dxin)) &&
                     (!ws || pk::aligned16(ws));
    const int nv = vec && C <= 8192 ? pick_nv(C) : 0;
    const size_t lds = (size_t)C * sizeof(float);
    if(vec && C / 4 >= 512 && C <= 16384) {
        const int64_t Q = (C / 4 + 3) / 4;
        const unsigned grid = (unsigned)P;
#define PK_RMSB(NQ_)                                                                           \
    if(C % 1024 == 0 && Q == NQ_ * 64)                                                          \
        rmsnorm_bwd_cols<NQ_, true><<<grid, 256, 0, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf);   \
    else                                                                                        \
        rmsnorm_bwd_cols<NQ_, false><<<grid, 256, 0, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf)
        if(Q <= 128) {
            PK_RMSB(2);
        } else if(Q <= 256) {
            PK_RMSB(4);
        } else if(Q <= 512) {
            PK_RMSB(8);
        } else {
            PK_RMSB(16);
        }
#undef PK_RMSB
    } else switch(nv) {
        case 1: rmsnorm_bwd_reg<1><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf); break;
        case 2: rmsnorm_bwd_reg<2><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf); break;
        case 4: rmsnorm_bwd_reg<4><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf); break;
        case 8: rmsnorm_bwd_reg<8><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf); break;
        case 16: rmsnorm_bwd_reg<16><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf); break;
        case 32: rmsnorm_bwd_reg<32><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf); break;
        default: rmsnorm_bwd_any<<<(unsigned)P, 256, 0, st>>>(R, C, x, g, rstd, dy, dxin, dx, ws, kf);
    }
    int rc = pk::launch_status("pk_rmsnorm_bwd_f32");
    if(rc || !dg) return rc;
    colsum_kernel<<<(unsigned)((C + 63) / 64), 64 * kColsumWaves, 0, st>>>(
        P, C, ws, dg, (flags & PK_ACCUM2) ? 1 : 0);
    return pk::launch_status("pk_rmsnorm_bwd_f32");
}

extern "C" int pk_rmsnorm_dg_reduce_f32(int64_t R, int64_t C, const void* workspace,
                                        size_t workspace_bytes, float* dg, int flags,
                                        pk_stream_t stream) {
    if(R < 0 || C < 1) return pk::fail("pk_rmsnorm_dg_reduce_f32: need R >= 0 and C >= 1");
    if(R == 0) return PK_OK;
    if(!dg) return pk::fail("pk_rmsnorm_dg_reduce_f32: NULL dg");
    if(!workspace || workspace_bytes < pk_rmsnorm_bwd_workspace(R, C))
        return pk::fail("pk_rmsnorm_dg_reduce_f32: workspace needs %zu bytes",
                        pk_rmsnorm_bwd_workspace(R, C));
    colsum_kernel<<<(unsigned)((C + 63) / 64), 64 * kColsumWaves, 0, pk::as_stream(stream)>>>(
        rms_parts(R), C, static_cast<const float*>(workspace), dg, (flags & PK_ACCUM) ? 1 : 0);
    return pk::launch_status("pk_rmsnorm_dg_reduce_f32");
}

extern "C" int pk_swiglu_fwd_f32(int64_t R, int64_t F, const float* a, int64_t lda, const float* u,
                                 int64_t ldu, float* h, int64_t ldh, pk_stream_t stream) {
    if(R < 0 || F < 0) return pk::fail("pk_swiglu_fwd_f32: negative size");
    if(R == 0 || F == 0) return PK_OK;
    if(!a || !u || !h) return pk::fail("pk_swiglu_fwd_f32: NULL pointer");
    if(lda < F || ldu < F || ldh < F) return pk::fail("pk_swiglu_fwd_f32: row stride < F");
    hipStream_t st = pk::as_stream(stream);
    const int64_t n = R * F;
    const bool al = pk::aligned16(a) && pk::aligned16(u) && pk::aligned16(h);
    if(lda == F && ldu == F && ldh == F && n % 4 == 0 && al)
        swiglu_fwd4<<<pk::grid_stream(n / 4, 256), 256, 0, st>>>(n / 4, (const f32x4*)a,
                                                                       (const f32x4*)u, (f32x4*)h);
    else if(F % 4 == 0 && lda % 4 == 0 && ldu % 4 == 0 && ldh % 4 == 0 && al)
        swiglu_fwd_rows4<<<rows4_grid(R, F / 4), 256, 0, st>>>(R, F / 4, a, lda, u, ldu, h, ldh);
    else
        swiglu_fwd_any<<<pk::grid_for(n, 256, 256 * 8), 256, 0, st>>>(R, F, a, lda, u, ldu, h, ldh);
    return pk::launch_status("pk_swiglu_fwd_f32");
}

extern "C" int pk_swiglu_bwd_f32(int64_t R, int64_t F, const float* a, int64_t lda, const float* u,
                                 int64_t ldu, const float* dh, int64_t ldh, float* da, float* du,
                                 int64_t ldd, int flags, pk_stream_t stream) {
    if(R < 0 || F < 0) return pk::fail("pk_swiglu_bwd_f32: negative size");
    if(R == 0 || F == 0 || (!da && !du)) return PK_OK;
    if(!a || !u || !dh) return pk::fail("pk_swiglu_bwd_f32: NULL input pointer");
    if(lda < F || ldu < F || ldh < F || ldd < F) return pk::fail("pk_swiglu_bwd_f32: row stride < F");
    hipStream_t st = pk::as_stream(stream);
    const int kf = (flags & (PK_ACCUM | PK_ACCUM2)) | (da ? 4 : 0) | (du ? 8 : 0);
    const int64_t n = R * F;
    const bool al = pk::aligned16(a) && pk::aligned16(u) && pk::aligned16(dh) &&
                    (!da || pk::aligned16(da)) && (!du || pk::aligned16(du));
    if(lda == F && ldu == F && ldh == F && ldd == F && n % 4 == 0 && al)
        swiglu_bwd4<<<pk::grid_stream(n / 4, 256), 256, 0, st>>>(
            n / 4, (const f32x4*)a, (const f32x4*)u, (const f32x4*)dh, (f32x4*)da, (f32x4*)du, kf);
    else if(F % 4 == 0 && lda % 4 == 0 && ldu % 4 == 0 && ldh % 4 == 0 && ldd % 4 == 0 && al)
        swiglu_bwd_rows4<<<rows4_grid(R, F / 4), 256, 0, st>>>(R, F / 4, a, lda, u, ldu, dh, ldh, da,
                                                              du, ldd, kf);
    else
        swiglu_bwd_any<<<pk::grid_for(n, 256, 256 * 8), 256, 0, st>>>(R, F, a, lda, u, ldu, dh, ldh,
                                                                     da, du, ldd, kf);
    return pk::launch_status("pk_swiglu_bwd_f32");
}

extern "C" int pk_causal_softmax_fwd_f32(int64_t BH, int64_t T, float scale, const float* S,
                                         float* P, float* lse, pk_stream_t stream) {
    if(BH < 0 || T < 0) return pk::fail("pk_causal_softmax_fwd_f32: negative size");
    if(BH == 0 || T == 0) return PK_OK;
    if(!S || !P) return pk::fail("pk_causal_softmax_fwd_f32: NULL pointer");
    const int64_t rows = BH * T;
    const unsigned grid = (unsigned)((rows + 3) / 4);
    hipStream_t st = pk::as_stream(stream);
    const bool vec = T % 4 == 0 && pk::aligned16(S) && pk::aligned16(P);
    const int nv = vec ? pick_nv(T) : 0;
    switch(nv) {
        case 1: csoftmax_fwd_reg<1><<<grid, 256, 0, st>>>(rows, T, scale, S, P, lse); break;
        case 2: csoftmax_fwd_reg<2><<<grid, 256, 0, st>>>(rows, T, scale, S, P, lse); break;
        case 4: csoftmax_fwd_reg<4><<<grid, 256, 0, st>>>(rows, T, scale, S, P, lse); break;
        case 8: csoftmax_fwd_reg<8><<<grid, 256, 0, st>>>(rows, T, scale, S, P, lse); break;
        default: csoftmax_fwd_any<<<grid, 256, 0, st>>>(rows, T, scale, S, P, lse);
    }
    return pk::launch_status("pk_causal_softmax_fwd_f32");
}

extern "C" int pk_causal_softmax_bwd_f32(int64_t BH, int64_t T, const float* P, const float* dP,
                                         float* dS, pk_stream_t stream) {
    if(BH < 0 || T < 0) return pk::fail("pk_causal_softmax_bwd_f32: negative size");
    if(BH == 0 || T == 0) return PK_OK;
    if(!P || !dP || !dS) return pk::fail("pk_causal_softmax_bwd_f32: NULL pointer");
    const int64_t rows = BH * T;
    const unsigned grid = (unsigned)((rows + 3) / 4);
    hipStream_t st = pk::as_stream(stream);
    const bool vec = T % 4 == 0 && pk::aligned16(P) && pk::aligned16(dP) && pk::aligned16(dS);
    const int nv = vec ? pick_nv(T) : 0;
    switch(nv) {
        case 1: csoftmax_bwd_reg<1><<<grid, 256, 0, st>>>(rows, T, P, dP, dS); break;
        case 2: csoftmax_bwd_reg<2><<<grid, 256, 0, st>>>(rows, T, P, dP, dS); break;
        case 4: csoftmax_bwd_reg<4><<<grid, 256, 0, st>>>(rows, T, P, dP, dS); break;
        case 8: csoftmax_bwd_reg<8><<<grid, 256, 0, st>>>(rows, T, P, dP, dS); break;
        default: csoftmax_bwd_any<<<grid, 256, 0, st>>>(rows, T, P, dP, dS);
    }
    return pk::launch_status("pk_causal_softmax_bwd_f32");
}
