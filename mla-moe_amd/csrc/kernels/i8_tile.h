/* i8_tile.h -- helpers shared by the int8 MoE GEMM kernels (decode-shaped,
 * tiled and big-tile): the SwiGLU epilogue, the LDS swizzle of staged A rows
 * and the row-group -> expert map of the grouped GEMMs. */
#pragma once
#include "common.h"

/* silu(g) * u with silu(x) = x / (1 + e^-x) (src/run.c:39, 85-93). */
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

/* position of 16 B chunk q of tile row R within the row's 128 B in LDS */
__device__ __forceinline__ int t_swz(int R) { return (R >> 1) & 7; }

/* Expert, first row and row count of row-group `tile` (a group is up to
 * a.mgroup consecutive 128-row tiles of one expert); all threads of the
 * block get the same answer; false when the group is past the last expert. */
__device__ __forceinline__ bool tile_owner(const mm_i8_tiled_args &a, int tile, int *e_out,
                                           int *m0_out, int *M_out) {
    __shared__ int s_e, s_m0, s_M;
    if (threadIdx.x < MM_WAVE) {
        const int lane = threadIdx.x;
        int found = -1, m0 = 0, Mf = 0;
        const int GR = MM_I8T_BM * a.mgroup;   /* rows per group */
        if (!a.cnt) {
            if (tile * GR < a.T) { found = 0; m0 = tile * GR; Mf = a.T; }
        } else {
            int base = 0;   /* tiles before this group of 64 experts */
            for (int e0 = 0; e0 < a.E && found < 0; e0 += MM_WAVE) {
                const int e = e0 + lane;
                const int M = e < a.E ? min(a.cnt[e], a.T) : 0;
                const int nt = (M + GR - 1) / GR;
                int incl = nt;   /* inclusive wave prefix sum */
#pragma unroll
                for (int off = 1; off < MM_WAVE; off <<= 1) {
                    int v = __shfl_up(incl, off, MM_WAVE);
                    if (lane >= off) incl += v;
                }
                const int excl = base + incl - nt;
                const bool mine = tile >= excl && tile < excl + nt;
                const unsigned long long bal = __ballot(mine);
                if (bal) {
                    const int src = __ffsll((long long)bal) - 1;
                    found = e0 + src;
                    m0 = (tile - __shfl(excl, src, MM_WAVE)) * GR;
                    Mf = __shfl(M, src, MM_WAVE);
                }
                base += __shfl(incl, MM_WAVE - 1, MM_WAVE);
            }
        }
        if (lane == 0) { s_e = found; s_m0 = m0; s_M = Mf; }
    }
    __syncthreads();
    *e_out = s_e;
    *m0_out = s_m0;
    *M_out = s_M;
    return s_e >= 0;
}
