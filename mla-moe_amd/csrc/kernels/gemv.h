/* gemv.h -- the register-resident GEMV core shared by the LM head and the
 * decode projections: y[t, r] = sum_i x'[t, i] * W[r, i] for up to NB tokens,
 * W bf16 row-major (nn.Linear layout), every weight row read once.
 *
 * Lane l owns the 16-byte weight pieces p = l + 64 j (8 inputs each) of every
 * row it touches, so each wave holds the NB tokens' activations x' for those
 * pieces in registers (at most GV_HMAX inputs).  x' is x itself, x truncated
 * to bf16, or rmsnorm(x) (src/run.c:22-27: the wave's own sum of squares,
 * then (x * inv) * w).  A wave takes GV_RPW rows per turn, issuing all
 * GV_RPW * GV_PPL 16-byte loads before the first is used, and walks rows
 * wave0, wave0 + nwaves, ... of the row space.
 */
#pragma once
#include "common.h"

#define GV_HMAX MM_LM_HMAX
#define GV_PPL (GV_HMAX / 8 / MM_WAVE)   /* pieces per lane at the maximum H */
#define GV_RPW MM_GEMV_RPW               /* rows per wave per turn */

/* Load NB tokens' activation rows x [B, H] (16-byte aligned, H % 8 == 0) as
 * pieces; tokens >= B and pieces past H read as zero.  norm != NULL applies
 * rmsnorm with weight `norm` [H] and `eps`; else x_bf16 truncates to bf16. */
template <int NB>
__device__ __forceinline__ void gemv_load_x(f32x4 (&xv)[NB][GV_PPL][2], const float *x, int B,
                                            int H, const uint16_t *norm, float eps, bool x_bf16) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int np = H / 8;
    const int ppl = (np + MM_WAVE - 1) / MM_WAVE;
    float ss[NB];
#pragma unroll
    for (int t = 0; t < NB; t++) {
        ss[t] = 0.0f;
        /* loads at clamped addresses, unconditionally, zeroed after: a load
         * under a condition becomes a branch around it, each then waited
         * for on its own */
#pragma unroll
        for (int j = 0; j < GV_PPL; j++) {
            const int p = min(lane + MM_WAVE * j, np - 1);
            const float *src = x + (size_t)min(t, B - 1) * H + 8 * p;
            xv[t][j][0] = *(const f32x4 *)src;
            xv[t][j][1] = *(const f32x4 *)(src + 4);
        }
#pragma unroll
        for (int j = 0; j < GV_PPL; j++) {
            const int p = lane + MM_WAVE * j;
            if (!(j < ppl && p < np && t < B))
                xv[t][j][0] = xv[t][j][1] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int u = 0; u < 4; u++) ss[t] += xv[t][j][h][u] * xv[t][j][h][u];
        }
    }
    if (norm) {
#pragma unroll
        for (int j = 0; j < GV_PPL; j++) {
            const int p = lane + MM_WAVE * j;
            const bool ok = j < ppl && p < np;
            const u32x4 nl = *(const u32x4 *)(norm + 8 * min(p, np - 1));
            const u32x4 nw = ok ? nl : (u32x4){0u, 0u, 0u, 0u};
            const float wn[8] = {bf16_lo(nw.x), bf16_hi(nw.x), bf16_lo(nw.y), bf16_hi(nw.y),
                                 bf16_lo(nw.z), bf16_hi(nw.z), bf16_lo(nw.w), bf16_hi(nw.w)};
#pragma unroll
            for (int t = 0; t < NB; t++) {
                if (j == 0) ss[t] = 1.0f / sqrtf(wave_sum(ss[t]) / (float)H + eps);
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        xv[t][j][h][u] = xv[t][j][h][u] * ss[t] * wn[4 * h + u];
            }
        }
    } else if (x_bf16) {
#pragma unroll
        for (int t = 0; t < NB; t++)
#pragma unroll
            for (int j = 0; j < GV_PPL; j++)
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        xv[t][j][h][u] = __uint_as_float(__float_as_uint(xv[t][j][h][u]) & 0xffff0000u);
    }
}

/* Rows [0, nrows) of the row space: rowptr(r) gives row r's weights (H
 * bf16), sink(r, t, v) receives y[t, r] (the same value in every lane) for
 * every token t < NB.  The wave sums are taken in the same order for every
 * row, so a row's result does not depend on which wave computed it. */
template <int NB, class RowPtr, class Sink>
__device__ __forceinline__ void gemv_rows(const f32x4 (&xv)[NB][GV_PPL][2], int H, int nrows,
                                          RowPtr rowptr, Sink &sink) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int np = H / 8;
    const int ppl = (np + MM_WAVE - 1) / MM_WAVE;
    const int nwaves = gridDim.x * (blockDim.x / MM_WAVE);
    const int wave0 = blockIdx.x * (blockDim.x / MM_WAVE) + threadIdx.x / MM_WAVE;
    for (int r0 = wave0 * GV_RPW; r0 < nrows; r0 += nwaves * GV_RPW) {
        u32x4 wv[GV_RPW][GV_PPL];
#pragma unroll
        for (int r = 0; r < GV_RPW; r++) {
            const uint16_t *wr = rowptr(min(r0 + r, nrows - 1));
#pragma unroll
            for (int j = 0; j < GV_PPL; j++)
                wv[r][j] = __builtin_nontemporal_load((const u32x4 *)wr + min(lane + MM_WAVE * j, np - 1));
        }
#pragma unroll
        for (int r = 0; r < GV_RPW; r++)
#pragma unroll
            for (int j = 0; j < GV_PPL; j++)
                if (!(j < ppl && lane + MM_WAVE * j < np)) wv[r][j] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < GV_RPW; r++) {
            float acc[NB];
#pragma unroll
            for (int t = 0; t < NB; t++) acc[t] = 0.0f;
#pragma unroll
            for (int j = 0; j < GV_PPL; j++) {
                const u32x4 w = wv[r][j];
#pragma unroll
                for (int t = 0; t < NB; t++) {
                    const f32x4 x0 = xv[t][j][0], x1 = xv[t][j][1];
                    float s = acc[t];
                    s = __builtin_fmaf(bf16_lo(w.x), x0.x, s);
                    s = __builtin_fmaf(bf16_hi(w.x), x0.y, s);
                    s = __builtin_fmaf(bf16_lo(w.y), x0.z, s);
                    s = __builtin_fmaf(bf16_hi(w.y), x0.w, s);
                    s = __builtin_fmaf(bf16_lo(w.z), x1.x, s);
                    s = __builtin_fmaf(bf16_hi(w.z), x1.y, s);
                    s = __builtin_fmaf(bf16_lo(w.w), x1.z, s);
                    s = __builtin_fmaf(bf16_hi(w.w), x1.w, s);
                    acc[t] = s;
                }
            }
            const int row = r0 + r;
#pragma unroll
            for (int t = 0; t < NB; t++) {
                const float v = wave_sum(acc[t]);
                if (row < nrows) sink(row, t, v);
            }
        }
    }
}
