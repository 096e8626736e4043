/* i8_tile.h -- helpers shared by the int8 MoE GEMM kernels (decode-shaped
 * and big-tile): the SwiGLU epilogues. */
#pragma once
#include "common.h"

/* silu(g) * u with silu(x) = x / (1 + e^-x) (src/run.c:39, 85-93). */
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

/* The same with the hardware exponential and reciprocal (v_exp_f32 of
 * -g log2(e), v_rcp_f32): a few ulp instead of a correctly rounded e^x and
 * an IEEE division, at a quarter of the VALU work -- the prefill GEMM's
 * gate/up epilogue evaluates it for every element of its output tile.
 * g -> -inf gives e^-g = inf and 0; g -> +inf gives 1 / 1. */
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

