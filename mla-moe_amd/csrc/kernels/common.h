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
/* fp32 -> bf16, round to nearest even (the hi part of the hi/lo splits of
 * fp32 activations; lo = rne16(x - bf16_f32(hi))) */
__device__ __forceinline__ uint16_t rne16(float x) {
    uint32_t u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* 8 bf16 weights (one 128-bit load) dotted with 8 fp32 activations read as
 * two 128-bit loads (x must be 16-byte aligned). */
/* as dot8_bf16 with x in LDS */
__device__ __forceinline__ float dot8_bf16_lds(u32x4 w, const __attribute__((address_space(3))) float *x, float acc) {
    const f32x4 a = *(const __attribute__((address_space(3))) f32x4 *)x;
    const f32x4 b = *(const __attribute__((address_space(3))) f32x4 *)(x + 4);
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

/* ---- direct-to-LDS loads and LDS reads the compiler does not track ---- */

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

/* 16 bytes per lane from `src` into LDS at `dst` + 16 * lane (direct
 * global -> LDS load, no VGPR staging). */
__device__ __forceinline__ void lds_dma16(const void *src, void *dst) {
    __builtin_amdgcn_global_load_lds((glb_void_t *)src, (lds_void_t *)dst, 16, 0, 0);
}

/* Buffer resource of a raw byte range (four scalar registers):
 * base, no stride, num_records bytes, the raw 32-bit format word. */
typedef uint32_t rsrc_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ rsrc_t raw_rsrc(const void *base, uint32_t num_records) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    rsrc_t r;
    r.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
    r.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu;
    r.z = num_records;
    r.w = 0x00020000u;
    return r;
}

/* 16 bytes per lane at byte offset `voff` of buffer `r` into LDS at byte
 * address `dst` (wave-uniform) + 16 * lane, as inline assembly.  An offset
 * past num_records reads no memory and stages zeros.  The compiler does not
 * see this LDS write, so it adds no wait for the load before later LDS
 * accesses (for a direct-to-LDS load it knows of, it waits for every load
 * and store in flight before any LDS read it cannot tell apart from the
 * destination); the caller orders every access to the destination itself,
 * with vmcnt waits and barriers. */
__device__ __forceinline__ void lds_dma16_buf(uint32_t voff, rsrc_t r, uint32_t dst) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 : : "v"(voff), "s"(r), "{m0}"(__builtin_amdgcn_readfirstlane(dst)) : "memory");
}

/* LDS byte address of a __shared__ location. */
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const lds_void_t *)p;
}

/* ds_read_b128 issued as inline assembly: the compiler's conservative
 * "wait for every outstanding direct-to-LDS load before any LDS read" would
 * otherwise drain the whole load ring every K step.  The caller orders the
 * reads with explicit vmcnt waits and a barrier, and must follow them with
 * lds_wait_regs() before using the results. */
__device__ __forceinline__ i32x4 ds_read16(uint32_t addr) {
    i32x4 r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
    return r;
}
/* As ds_read16 at addr + off, with off (a constant after unrolling,
 * < 65536) in the instruction's offset field. */
__device__ __forceinline__ i32x4 ds_read16(uint32_t addr, int off) {
    i32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off));
    return r;
}



/* s_waitcnt vmcnt(n) only (expcnt and lgkmcnt left at their maxima). */
#define VMCNT_WAIT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))
