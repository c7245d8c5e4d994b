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
// one workgroup of NT threads per row; each thread caches NV float4 of the row
template <int NT, int NV>
__global__ __launch_bounds__(NT) void xent_reg_kernel(int64_t V, const float* __restrict__ logits,
                                                      int64_t ldz, const int32_t* __restrict__ labels,
                                                      float* __restrict__ loss_rows,
                                                      float* __restrict__ dlogits, int64_t ldd,
                                                      float scale_in,
                                                      const float* __restrict__ scale_dev,
                                                      int accum) {
    __shared__ float red[NT / 64];
    const float scale = scale_dev ? scale_in * *scale_dev : scale_in;
    const int64_t r = blockIdx.x;
    const f32x4* z4 = reinterpret_cast<const f32x4*>(logits + r * ldz);
    const int64_t V4 = V / 4;
    f32x4 z[NV];
    float m = kNegInf;
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = threadIdx.x + (int64_t)v * NT;
        if(c < V4) {
            z[v] = z4[c];
            m = fmaxf(m, fmaxf(fmaxf(z[v][0], z[v][1]), fmaxf(z[v][2], z[v][3])));
        } else {
            z[v] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
        }
    }
    m = pk::block_max<NT / 64>(m, red);
    float s = 0.0f;
#pragma unroll
    for(int v = 0; v < NV; ++v)
#pragma unroll
        for(int e = 0; e < 4; ++e) s += expf(z[v][e] - m);
    s = pk::block_sum<NT / 64>(s, red);
    const float lse = m + logf(s);
    const int32_t y = labels[r];
    const bool ok = y >= 0 && y < V;
    if(loss_rows && threadIdx.x == 0) loss_rows[r] = ok ? lse - logits[r * ldz + y] : NAN;
    if(!dlogits) return;
    f32x4* d4 = reinterpret_cast<f32x4*>(dlogits + r * ldd);
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = threadIdx.x + (int64_t)v * NT;
        if(c >= V4) continue;
        f32x4 g;
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            const int64_t col = c * 4 + e;
            const float p = expf(z[v][e] - lse);
            g[e] = ok ? scale * (p - (col == y ? 1.0f : 0.0f)) : 0.0f;
        }
        if(accum) {
            const f32x4 o = d4[c];
            g = g + o;
        }
        d4[c] = g;
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
// one wave per row, NV float4 per lane (row width C <= 256*NV, C % 4 == 0)
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_fwd_reg(int64_t R, int64_t C, float eps,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ y,
                                                       float* __restrict__ rstd) {
    const int64_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if(row >= R) return;
    const int64_t C4 = C / 4;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * C);
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    f32x4 xv[NV];
    float ss = 0.0f;
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        if(c < C4) {
            xv[v] = xr[c];
            ss += xv[v][0] * xv[v][0] + xv[v][1] * xv[v][1] + xv[v][2] * xv[v][2] +
                  xv[v][3] * xv[v][3];
        }
    }
    ss = pk::wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / (float)C + eps);
    if(lane == 0 && rstd) rstd[row] = rs;
    f32x4* yr = reinterpret_cast<f32x4*>(y + row * C);
#pragma unroll
    for(int v = 0; v < NV; ++v) {
        const int64_t c = lane + v * 64;
        if(c < C4) yr[c] = xv[v] * rs * g4[c];
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

// backward, stage 1: dx for each row; per-workgroup partial of dg into ws[block][C]
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_reg(int64_t R, int64_t C,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       const float* __restrict__ rstd,
                                                       const float* __restrict__ dy,
                                                       float* __restrict__ dx,
                                                       float* __restrict__ ws, int flags) {
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
    for(int64_t row = (int64_t)blockIdx.x * 4 + w; row < R; row += (int64_t)gridDim.x * 4) {
        const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * C);
        const f32x4* dyr = reinterpret_cast<const f32x4*>(dy + row * C);
        f32x4 xv[NV], dv[NV];
        float dot = 0.0f;
#pragma unroll
        for(int v = 0; v < NV; ++v) {
            const int64_t c = lane + v * 64;
            if(c < C4) {
                xv[v] = xr[c];
                dv[v] = dyr[c];
                const f32x4 t = gv[v] * dv[v] * xv[v];
                dot += t[0] + t[1] + t[2] + t[3];
            }
        }
        dot = pk::wave_sum(dot);
        const float rs = rstd[row];
        const float k = rs * rs * rs * dot * invC;
        f32x4* dxr = reinterpret_cast<f32x4*>(dx + row * C);
#pragma unroll
        for(int v = 0; v < NV; ++v) {
            const int64_t c = lane + v * 64;
            if(c < C4) {
                if(flags & 4) {  // dx requested
                    f32x4 o = rs * gv[v] * dv[v] - xv[v] * k;
                    if(flags & PK_ACCUM) o = o + dxr[c];
                    dxr[c] = o;
                }
                dg[v] = dg[v] + dv[v] * xv[v] * rs;
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

__global__ __launch_bounds__(256) void rmsnorm_bwd_any(int64_t R, int64_t C,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ g,
                                                       const float* __restrict__ rstd,
                                                       const float* __restrict__ dy,
                                                       float* __restrict__ dx,
                                                       float* __restrict__ ws, int flags) {
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
                dx[row * C + c] = (flags & PK_ACCUM) ? dx[row * C + c] + o : o;
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

// backward, stage 2: dg (+)= sum over the partial rows; 64 columns per block,
// 4 waves split the partial rows, combined in a fixed order
__global__ __launch_bounds__(256) void colsum_kernel(int64_t P, int64_t C, const float* __restrict__ ws,
                                                     float* __restrict__ dg, int accum) {
    __shared__ float part[4][64];
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if(c < C)
        for(int64_t p = w; p < P; p += 4) acc += ws[p * C + c];
    part[w][lane] = acc;
    __syncthreads();
    if(w == 0 && c < C) {
        const float s = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
        dg[c] = accum ? dg[c] + s : s;
    }
}

int64_t rms_parts(int64_t R) {
    const int64_t blocks = (R + 3) / 4;
    return blocks < 512 ? blocks : 512;
}

// ================================================================== SwiGLU
__device__ __forceinline__ float sigmoidf_(float a) { return 1.0f / (1.0f + expf(-a)); }

__global__ void swiglu_fwd4(int64_t n4, const f32x4* __restrict__ a, const f32x4* __restrict__ u,
                            f32x4* __restrict__ h) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
        i += (int64_t)gridDim.x * blockDim.x) {
        const f32x4 av = a[i], uv = u[i];
        f32x4 o;
#pragma unroll
        for(int e = 0; e < 4; ++e) o[e] = av[e] * sigmoidf_(av[e]) * uv[e];
        h[i] = o;
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
        h[r * ldh + c] = av * sigmoidf_(av) * u[r * ldu + c];
    }
}

__global__ void swiglu_bwd4(int64_t n4, const f32x4* __restrict__ a, const f32x4* __restrict__ u,
                            const f32x4* __restrict__ dh, f32x4* __restrict__ da,
                            f32x4* __restrict__ du, int flags) {
    for(int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
        i += (int64_t)gridDim.x * blockDim.x) {
        const f32x4 av = a[i], uv = u[i], g = dh[i];
        f32x4 ga, gu;
#pragma unroll
        for(int e = 0; e < 4; ++e) {
            const float s = sigmoidf_(av[e]);
            ga[e] = g[e] * uv[e] * s * (1.0f + av[e] * (1.0f - s));
            gu[e] = g[e] * av[e] * s;
        }
        if(flags & 4) da[i] = (flags & PK_ACCUM) ? da[i] + ga : ga;
        if(flags & 8) du[i] = (flags & PK_ACCUM2) ? du[i] + gu : gu;
    }
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
        const float s = sigmoidf_(av);
        const float ga = g * uv * s * (1.0f + av * (1.0f - s));
        const float gu = g * av * s;
        const int64_t o = r * ldd + c;
        if(flags & 4) da[o] = (flags & PK_ACCUM) ? da[o] + ga : ga;
        if(flags & 8) du[o] = (flags & PK_ACCUM2) ? du[o] + gu : gu;
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
    if(vec && V4 <= 256 * 1)
        xent_reg_kernel<256, 1><<<grid, 256, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, scale_dev, accum);
    else if(vec && V4 <= 256 * 2)
        xent_reg_kernel<256, 2><<<grid, 256, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, scale_dev, accum);
    else if(vec && V4 <= 256 * 4)
        xent_reg_kernel<256, 4><<<grid, 256, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, scale_dev, accum);
    else if(vec && V4 <= 256 * 8)
        xent_reg_kernel<256, 8><<<grid, 256, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, scale_dev, accum);
    else if(vec && V4 <= 1024 * 8)
        xent_reg_kernel<1024, 8><<<grid, 1024, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, scale_dev, accum);
    else
        xent_any_kernel<1024><<<grid, 1024, 0, st>>>(V, logits, ldz, labels, loss_rows, dlogits, ldd, scale, scale_dev, accum);
    return pk::launch_status("pk_xent_fwd_bwd_f32");
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
    const unsigned grid = (unsigned)((R + 3) / 4);
    const bool vec = C % 4 == 0 && pk::aligned16(x) && pk::aligned16(g) && pk::aligned16(y);
    const int nv = vec ? pick_nv(C) : 0;
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
    if(R < 0 || C < 1) return pk::fail("pk_rmsnorm_bwd_f32: need R >= 0 and C >= 1");
    if(R == 0) return PK_OK;
    if(!x || !g || !rstd || !dy) return pk::fail("pk_rmsnorm_bwd_f32: NULL input pointer");
    if(!dx && !dg) return PK_OK;
    const int64_t P = rms_parts(R);
    if(dg && (!workspace || workspace_bytes < pk_rmsnorm_bwd_workspace(R, C)))
        return pk::fail("pk_rmsnorm_bwd_f32: workspace needs %zu bytes",
                        pk_rmsnorm_bwd_workspace(R, C));
    hipStream_t st = pk::as_stream(stream);
    float* ws = (float*)workspace;
    // internal flags: 4 = write dx, 8 = produce dg partials; bit 0 = accumulate dx
    const int kf = (flags & PK_ACCUM) | (dx ? 4 : 0) | (dg ? 8 : 0);
    const bool vec = C % 4 == 0 && pk::aligned16(x) && pk::aligned16(g) && pk::aligned16(dy) &&
                     (!dx || pk::aligned16(dx)) && (!ws || pk::aligned16(ws));
    const int nv = vec && C <= 8192 ? pick_nv(C) : 0;
    const size_t lds = (size_t)C * sizeof(float);
    switch(nv) {
        case 1: rmsnorm_bwd_reg<1><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dx, ws, kf); break;
        case 2: rmsnorm_bwd_reg<2><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dx, ws, kf); break;
        case 4: rmsnorm_bwd_reg<4><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dx, ws, kf); break;
        case 8: rmsnorm_bwd_reg<8><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dx, ws, kf); break;
        case 16: rmsnorm_bwd_reg<16><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dx, ws, kf); break;
        case 32: rmsnorm_bwd_reg<32><<<(unsigned)P, 256, lds, st>>>(R, C, x, g, rstd, dy, dx, ws, kf); break;
        default: rmsnorm_bwd_any<<<(unsigned)P, 256, 0, st>>>(R, C, x, g, rstd, dy, dx, ws, kf);
    }
    int rc = pk::launch_status("pk_rmsnorm_bwd_f32");
    if(rc || !dg) return rc;
    colsum_kernel<<<(unsigned)((C + 63) / 64), 256, 0, st>>>(P, C, ws, dg, (flags & PK_ACCUM2) ? 1 : 0);
    return pk::launch_status("pk_rmsnorm_bwd_f32");
}

extern "C" int pk_swiglu_fwd_f32(int64_t R, int64_t F, const float* a, int64_t lda, const float* u,
                                 int64_t ldu, float* h, int64_t ldh, pk_stream_t stream) {
    if(R < 0 || F < 0) return pk::fail("pk_swiglu_fwd_f32: negative size");
    if(R == 0 || F == 0) return PK_OK;
    if(!a || !u || !h) return pk::fail("pk_swiglu_fwd_f32: NULL pointer");
    if(lda < F || ldu < F || ldh < F) return pk::fail("pk_swiglu_fwd_f32: row stride < F");
    hipStream_t st = pk::as_stream(stream);
    const int64_t n = R * F;
    if(lda == F && ldu == F && ldh == F && n % 4 == 0 && pk::aligned16(a) && pk::aligned16(u) &&
       pk::aligned16(h))
        swiglu_fwd4<<<pk::grid_for(n / 4, 256, 256 * 8), 256, 0, st>>>(n / 4, (const f32x4*)a,
                                                                       (const f32x4*)u, (f32x4*)h);
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
    if(lda == F && ldu == F && ldh == F && ldd == F && n % 4 == 0 && pk::aligned16(a) &&
       pk::aligned16(u) && pk::aligned16(dh) && (!da || pk::aligned16(da)) &&
       (!du || pk::aligned16(du)))
        swiglu_bwd4<<<pk::grid_for(n / 4, 256, 256 * 8), 256, 0, st>>>(
            n / 4, (const f32x4*)a, (const f32x4*)u, (const f32x4*)dh, (f32x4*)da, (f32x4*)du, kf);
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
