/* lm_head.hip -- the decode step's LM head on gfx950: final RMSNorm, logits
 * over the vocabulary, greedy argmax.
 *
 * Reference semantics (src/run.c):
 *   rmsnorm  run.c:22-27   y = (x * inv) * w, inv = 1 / sqrtf(ss / n + eps),
 *                          ss the sum of squares
 *   logits   run.c:493-494 matmul(logits, xb, lm_head, vocab, hidden)
 *   sample   run.c:503-508 first index of the maximum under a strict '>'
 *                          scan from index 0
 * The sum of squares and the logit dot products are reduced in parallel
 * (fp32, a different association than the reference's sequential loops):
 * results agree to ~1e-6 relative, which the tests bound.
 *
 * Kernels:
 *   mm_lm_gemv   for up to MM_LM_NB tokens: rmsnorm, logits (every weight
 *                row read once: HBM-bound, 2 bytes per weight) and per-wave
 *                argmax partials in one pass; each wave holds the tokens'
 *                activations in registers and walks many rows with LM_RPW
 *                rows' loads in flight
 *   mm_rmsnorm   one block per token (the GEMM path for more tokens)
 *   mm_argmax_part / mm_argmax_final   segments of every row in parallel
 *                (the GEMV path writes its partials itself), then one block
 *                per row over the partials
 */
#include "common.h"

/* ---- RMSNorm ---------------------------------------------------------------- */

extern "C" __global__ __launch_bounds__(256) void mm_rmsnorm(mm_rmsnorm_args a) {
    __shared__ float red[256 / MM_WAVE];
    const int t = blockIdx.x;
    const float *x = a.x + (size_t)t * a.n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < a.n; i += 256) ss += x[i] * x[i];
    ss = wave_sum(ss);
    const int lane = threadIdx.x & (MM_WAVE - 1), wave = threadIdx.x / MM_WAVE;
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < 256 / MM_WAVE; w++) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)a.n + a.eps);
    float *y = a.y + (size_t)t * a.n;
    for (int i = threadIdx.x; i < a.n; i += 256) y[i] = x[i] * inv * bf16_f32(a.w[i]);
}

/* ---- greedy argmax ---------------------------------------------------------- */

/* (v, i) beats (bv, bi) when v is a number and bv is not, or v > bv, or
 * v == bv at a lower index: the first maximum of the sequential strict-'>'
 * scan, NaNs never winning.  A NaN at index 0 is the scan's start value and
 * is never beaten (handled by the caller). */
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
    if (v != v) return false;
    if (bv != bv) return true;
    return v > bv || (v == bv && i < bi);
}

/* ---- logits GEMV -------------------------------------------------------------- */

/* Lane l owns the 16-byte pieces p = l + 64 j (8 hidden indices each) of
 * every row it touches, so each wave holds the NB tokens' whole activation
 * rows in registers.  It normalises them itself (rmsnorm, run.c:22-27: the
 * wave's sum of squares, then (x * inv) * w), so no separate norm pass
 * runs.  A wave takes rows wave0, wave0 + nwaves, ..., LM_RPW at a time:
 * LM_RPW * PPL 16-byte weight loads per lane are issued before the first is
 * used.  Each wave keeps its best (logit, row) per token; the block's best
 * goes to part_v / part_i [t][block]: the argmax then only reduces those
 * partials. */
#define LM_RPW 4
template <int NB>
__device__ __forceinline__ void lm_gemv(const mm_lm_gemv_args &a) {
    constexpr int PPL = MM_LM_HMAX / 8 / MM_WAVE;     /* pieces per lane at the maximum H */
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int np = a.H / 8;                            /* pieces per row */
    const int ppl = (np + MM_WAVE - 1) / MM_WAVE;      /* used pieces per lane (<= PPL) */
    const int nwaves = gridDim.x * (blockDim.x / MM_WAVE);
    const int wave0 = blockIdx.x * (blockDim.x / MM_WAVE) + threadIdx.x / MM_WAVE;

    f32x4 xv[NB][PPL][2];
    float ss[NB];
#pragma unroll
    for (int t = 0; t < NB; t++) {
        ss[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < PPL; j++) {
            const int p = lane + MM_WAVE * j;
            const bool ok = j < ppl && p < np && t < a.B;
            const float *src = a.x + (size_t)min(t, a.B - 1) * a.H + 8 * (ok ? p : 0);
            xv[t][j][0] = ok ? *(const f32x4 *)src : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            xv[t][j][1] = ok ? *(const f32x4 *)(src + 4) : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int u = 0; u < 4; u++) ss[t] += xv[t][j][h][u] * xv[t][j][h][u];
        }
    }
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int p = lane + MM_WAVE * j;
        const bool ok = j < ppl && p < np;
        const u32x4 nw = ok ? *(const u32x4 *)(a.norm + 8 * p) : (u32x4){0u, 0u, 0u, 0u};
        const float wn[8] = {bf16_lo(nw.x), bf16_hi(nw.x), bf16_lo(nw.y), bf16_hi(nw.y),
                             bf16_lo(nw.z), bf16_hi(nw.z), bf16_lo(nw.w), bf16_hi(nw.w)};
#pragma unroll
        for (int t = 0; t < NB; t++) {
            if (j == 0) ss[t] = 1.0f / sqrtf(wave_sum(ss[t]) / (float)a.H + a.eps);
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int u = 0; u < 4; u++) xv[t][j][h][u] = xv[t][j][h][u] * ss[t] * wn[4 * h + u];
        }
    }

    float bv[NB];
    int bi[NB];
#pragma unroll
    for (int t = 0; t < NB; t++) { bv[t] = __builtin_nanf(""); bi[t] = 0x7fffffff; }
    for (int r0 = wave0 * LM_RPW; r0 < a.V; r0 += nwaves * LM_RPW) {
        u32x4 wv[LM_RPW][PPL];
#pragma unroll
        for (int r = 0; r < LM_RPW; r++)
#pragma unroll
            for (int j = 0; j < PPL; j++) {
                const int p = lane + MM_WAVE * j;
                const int row = min(r0 + r, a.V - 1);
                wv[r][j] = (j < ppl && p < np)
                               ? __builtin_nontemporal_load((const u32x4 *)(a.w + (size_t)row * a.H) + p)
                               : (u32x4){0u, 0u, 0u, 0u};
            }
#pragma unroll
        for (int r = 0; r < LM_RPW; r++) {
            float acc[NB];
#pragma unroll
            for (int t = 0; t < NB; t++) acc[t] = 0.0f;
#pragma unroll
            for (int j = 0; j < PPL; j++) {
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
                const float v = wave_sum(acc[t]);   /* every lane holds the sum */
                if (row < a.V) {
                    if (lane == 0 && t < a.B) a.y[(size_t)t * a.V + row] = v;
                    if (am_better(v, row, bv[t], bi[t])) { bv[t] = v; bi[t] = row; }
                }
            }
        }
    }
    /* the block's best per token: one partial per block */
    __shared__ float sv[NB][256 / MM_WAVE];
    __shared__ int si[NB][256 / MM_WAVE];
    const int wave = threadIdx.x / MM_WAVE;
    if (lane == 0)
#pragma unroll
        for (int t = 0; t < NB; t++) { sv[t][wave] = bv[t]; si[t][wave] = bi[t]; }
    __syncthreads();
    if (threadIdx.x < NB && (int)threadIdx.x < a.B) {
        const int t = threadIdx.x;
        float v = sv[t][0];
        int i = si[t][0];
        for (int w = 1; w < 256 / MM_WAVE; w++)
            if (am_better(sv[t][w], si[t][w], v, i)) { v = sv[t][w]; i = si[t][w]; }
        a.part_v[(size_t)t * gridDim.x + blockIdx.x] = v;
        a.part_i[(size_t)t * gridDim.x + blockIdx.x] = i;
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_lm_gemv(mm_lm_gemv_args a) {
    if (a.B <= 1)
        lm_gemv<1>(a);
    else if (a.B <= 2)
        lm_gemv<2>(a);
    else
        lm_gemv<MM_LM_NB>(a);
}

/* Pass 1: block (seg, t) scans its contiguous segment of row t and writes
 * the segment's best (value, index) to part[t][seg]. */
extern "C" __global__ __launch_bounds__(256) void mm_argmax_part(mm_argmax_args a) {
    __shared__ float sv[256 / MM_WAVE];
    __shared__ int si[256 / MM_WAVE];
    const int t = blockIdx.y, seg = blockIdx.x;
    const float *lg = a.logits + (size_t)t * a.n;
    const int len = (a.n + a.nseg - 1) / a.nseg;
    const int i0 = seg * len, i1 = min(a.n, i0 + len);
    float bv = __builtin_nanf("");
    int bi = 0x7fffffff;
    for (int i = i0 + threadIdx.x; i < i1; i += 256) {
        const float v = lg[i];
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, MM_WAVE);
        const int oi = __shfl_xor(bi, off, MM_WAVE);
        if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & (MM_WAVE - 1), wave = threadIdx.x / MM_WAVE;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 256 / MM_WAVE; w++)
            if (am_better(sv[w], si[w], sv[0], si[0])) { sv[0] = sv[w]; si[0] = si[w]; }
        a.part_v[(size_t)t * a.nseg + seg] = sv[0];
        a.part_i[(size_t)t * a.nseg + seg] = si[0];
    }
}

/* Pass 2: one block per row reduces the partials (8 loads per thread in
 * flight) in the same order-independent rule, then applies the scan's
 * start at index 0. */
extern "C" __global__ __launch_bounds__(256) void mm_argmax_final(mm_argmax_args a) {
    __shared__ float sv[256 / MM_WAVE];
    __shared__ int si[256 / MM_WAVE];
    const int t = blockIdx.x;
    const float *pv = a.part_v + (size_t)t * a.nseg;
    const int32_t *pi = a.part_i + (size_t)t * a.nseg;
    float bv = __builtin_nanf("");
    int bi = 0x7fffffff;
    for (int s0 = 0; s0 < a.nseg; s0 += 8 * 256) {
        float v[8];
        int i[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int s = s0 + k * 256 + threadIdx.x;
            v[k] = s < a.nseg ? pv[s] : __builtin_nanf("");
            i[k] = s < a.nseg ? pi[s] : 0x7fffffff;
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (am_better(v[k], i[k], bv, bi)) { bv = v[k]; bi = i[k]; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, MM_WAVE);
        const int oi = __shfl_xor(bi, off, MM_WAVE);
        if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & (MM_WAVE - 1), wave = threadIdx.x / MM_WAVE;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 256 / MM_WAVE; w++)
            if (am_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
        const float v0 = a.logits[(size_t)t * a.n];
        /* run.c:504-508 starts its scan at logits[0]: a NaN there is never
         * replaced; no number at all (every entry NaN) also leaves 0 */
        a.tokens[t] = (v0 != v0 || bi == 0x7fffffff) ? 0 : bi;
    }
}
