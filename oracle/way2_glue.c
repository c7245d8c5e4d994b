/*
 * oracle/way2_glue.c -- test infrastructure: the few helpers the "Way 2"
 * binding (pico's own GPU op seams calling libpico_amd.so) needs in pico's own
 * sources (linked with a copy of
 * them patched by way2_patch.py into oracle/_ref/libpico_way2.so), plus entry
 * points a test uses to make GPU tensors the way pico would and to move their
 * values.  Not part of the product.
 *
 * A GPU tensor here is pico's own 64-byte PicoTensor whose data and grad are
 * device memory: op outputs get theirs from the op's arena through
 * libpico_amd.so's arena_alloc_device (the device side table keyed by pico's
 * 16-byte arena), params from hipMalloc.  pico zero-fills both
 * (src/tensor.c:114-117); here pk_fill_f32 does, on the library's stream.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "arena.h"
#include "tensor.h"

void* arena_alloc_device(struct Arena* arena, size_t bytes);
void* pico_gpu_stream(void);
int pico_gpu_synchronize(void);
int pk_fill_f32(int64_t n, float value, float* x, void* stream);
int pk_sgd_f32(int64_t n, float lr, float* p, const float* g, void* stream);

static int zero_both(struct PicoTensor* t) {
    void* st = pico_gpu_stream();
    return pk_fill_f32(t->numel, 0.0f, t->data, st) || pk_fill_f32(t->numel, 0.0f, t->grad, st);
}

/* an op's GPU output: device data and grad from the op's arena, zeroed */
int pico_way2_adopt(struct Arena* arena, struct PicoTensor* t) {
    const size_t bytes = sizeof(float) * (size_t)(t->numel > 0 ? t->numel : 1);
    float* d = (float*)arena_alloc_device(arena, bytes);
    float* g = (float*)arena_alloc_device(arena, bytes);
    if(!d || !g) return -1;
    t->data = d;
    t->grad = g;
    return zero_both(t);
}

/* pico_backward's seed (src/tensor.c:27-30) on the device */
void pico_way2_seed(struct PicoTensor* t) { pk_fill_f32(t->numel, 1.0f, t->grad, pico_gpu_stream()); }

/* SGD's step and zero_grad (src/optim/SGD.c:29-47) on the device */
void pico_way2_sgd(struct PicoTensor* t, float lr) {
    pk_sgd_f32(t->numel, lr, t->data, t->grad, pico_gpu_stream());
}
void pico_way2_zero_grad(struct PicoTensor* t) {
    pk_fill_f32(t->numel, 0.0f, t->grad, pico_gpu_stream());
}

/* ---- for tests: pico_param with device data and grad, and copies ---- */
struct PicoTensor* way2_param_device(int64_t* shape, uint8_t ndim) {
    struct PicoTensor* t = pico_param(shape, ndim);
    if(!t) return NULL;
    free(t->data);
    free(t->grad);
    t->data = t->grad = NULL;
    const size_t bytes = sizeof(float) * (size_t)(t->numel > 0 ? t->numel : 1);
    if(hipMalloc((void**)&t->data, bytes) != hipSuccess ||
       hipMalloc((void**)&t->grad, bytes) != hipSuccess || zero_both(t)) {
        hipFree(t->data);
        hipFree(t->grad);
        free(t->shape);
        free(t->strides);
        free(t);
        return NULL;
    }
    t->backend = GPU;
    return t;
}

void way2_free_device(struct PicoTensor* t) {
    if(!t) return;
    pico_gpu_synchronize();
    hipFree(t->data);
    hipFree(t->grad);
    free(t->shape);
    free(t->strides);
    free(t);
}

/* which: 0 data, 1 grad; returns 0 on success */
int way2_copy(struct PicoTensor* t, int which, float* host, int to_device) {
    float* dev = which ? t->grad : t->data;
    const size_t bytes = sizeof(float) * (size_t)t->numel;
    if(pico_gpu_synchronize()) return -1;
    hipError_t e = to_device ? hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice)
                             : hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? 0 : -1;
}
