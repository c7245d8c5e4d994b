// pico_amd/csrc/pk_common.h -- shared pieces of the gfx950 kernels: status
// reporting, vector types, 64-lane wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pico_hip.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace pk {

constexpr int kWave = 64;  // CDNA wavefront width

// Records a refusal message (thread-local) and returns PK_EINVAL.
int fail(const char* fmt, ...);
// Maps the last launch's error to a status.
int launch_status(const char* what);

inline hipStream_t as_stream(pk_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- wavefront reductions over all 64 lanes (DPP/permute via shfl_xor) ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for(int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for(int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for(int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Block-wide sum/max for blocks of NW waves; `red` is NW floats of LDS.
// Every thread receives the result.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    if(NW == 1) return v;
    __syncthreads();
    if(l == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for(int i = 0; i < NW; i++) t += red[i];
    return t;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    if(NW == 1) return v;
    __syncthreads();
    if(l == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for(int i = 1; i < NW; i++) t = fmaxf(t, red[i]);
    return t;
}

// Streaming accesses for data touched once per kernel: the nontemporal hint
// keeps a pass over a large tensor from evicting reusable lines (measured on
// MI355X: a float4 copy reaches ~6.0 TB/s with these, ~5.4 TB/s without).
template <class T>
__device__ __forceinline__ T ld_stream(const T* p) {
    return __builtin_nontemporal_load(p);
}
template <class T>
__device__ __forceinline__ void st_stream(T* p, T v) {
    __builtin_nontemporal_store(v, p);
}

// SwiGLU h = silu(a) * u = a * s * u with s = sigmoid(a), and its gradients
// for an upstream g: dh/da = u * s * (1 + a * (1 - s)), dh/du = a * s.  One
// definition for the row kernels and the GEMM epilogue that fuses the
// backward, so both round alike: contraction is off here (and in add_nc, the
// accumulation of a gradient), so no multiply is fused with an add of the
// surrounding code, whose shape differs between the two callers.
__device__ __forceinline__ float swiglu_sigmoid(float a) {
#pragma clang fp contract(off)
    return 1.0f / (1.0f + expf(-a));
}
__device__ __forceinline__ float swiglu_fwd1(float a, float u) {
#pragma clang fp contract(off)
    return a * swiglu_sigmoid(a) * u;
}
__device__ __forceinline__ void swiglu_bwd1(float a, float u, float g, float& ga, float& gu) {
#pragma clang fp contract(off)
    const float s = swiglu_sigmoid(a);
    ga = g * u * s * (1.0f + a * (1.0f - s));
    gu = g * a * s;
}
__device__ __forceinline__ float add_nc(float x, float y) {
#pragma clang fp contract(off)
    return x + y;
}

// grid for a streaming kernel that gives each thread one element per pass
inline unsigned grid_stream(int64_t work_items, int threads) {
    int64_t g = (work_items + threads - 1) / threads;
    if(g < 1) g = 1;
    if(g > (int64_t)1 << 20) g = (int64_t)1 << 20;
    return (unsigned)g;
}

// grid size for a grid-stride elementwise kernel
inline unsigned grid_for(int64_t work_items, int threads, int64_t cap = 256 * 16) {
    int64_t g = (work_items + threads - 1) / threads;
    if(g < 1) g = 1;
    if(g > cap) g = cap;
    return (unsigned)g;
}

}  // namespace pk
