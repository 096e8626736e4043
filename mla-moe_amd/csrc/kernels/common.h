/* common.h -- device helpers shared by the gfx950 kernels. */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kernel_params.h"

#define MM_WAVE 64

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

/* bf16 held in the low / high half of a 32-bit word -> fp32 (a shift or a
 * mask, include/tensor.h:9-14). */
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

/* 8 bf16 weights (one 128-bit load) dotted with 8 fp32 activations read as
 * two 128-bit loads (x must be 16-byte aligned). */
__device__ __forceinline__ float dot8_bf16(u32x4 w, const float *x, float acc) {
    const f32x4 a = *(const f32x4 *)x, b = *(const f32x4 *)(x + 4);
    acc = __builtin_fmaf(bf16_lo(w.x), a.x, acc);
    acc = __builtin_fmaf(bf16_hi(w.x), a.y, acc);
    acc = __builtin_fmaf(bf16_lo(w.y), a.z, acc);
    acc = __builtin_fmaf(bf16_hi(w.y), a.w, acc);
    acc = __builtin_fmaf(bf16_lo(w.z), b.x, acc);
    acc = __builtin_fmaf(bf16_hi(w.z), b.y, acc);
    acc = __builtin_fmaf(bf16_lo(w.w), b.z, acc);
    acc = __builtin_fmaf(bf16_hi(w.w), b.w, acc);
    return acc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, MM_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, MM_WAVE));
    return v;
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, MM_WAVE));
    return v;
}

/* SwiGLU activation for the GEMM/GEMV epilogues: silu(g) * u with
 * silu(x) = x / (1 + e^-x) (src/run.c:39). */
__device__ __forceinline__ float swiglu_f(float g, float u) {
    return g / (1.0f + __expf(-g)) * u;
}

/* Correctly rounded e^x in fp32 (evaluated in fp64, then one rounding).  Used
 * where the result feeds a selection that must match the CPU reference
 * (router softmax/sigmoid), so that only an input whose exact e^x lies within
 * ~2^-29 relative of a rounding boundary can differ from a correctly rounded
 * libm expf. */
__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }
