/* i8_tile.h -- helpers shared by the int8 MoE GEMM kernels (decode-shaped
 * and big-tile): the SwiGLU epilogue and the LDS swizzle of staged A rows. */
#pragma once
#include "common.h"

/* silu(g) * u with silu(x) = x / (1 + e^-x) (src/run.c:39, 85-93). */
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

