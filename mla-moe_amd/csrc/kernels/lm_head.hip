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
 *                argmax partials in one pass (the GEMV core of gemv.h)
 *   mm_rmsnorm   one block per token (the GEMM path for more tokens)
 *   mm_argmax_part / mm_argmax_final   segments of every row in parallel
 *                (the GEMV path writes its partials itself), then one block
 *                per row over the partials
 */
#include "gemv.h"

/* ---- RMSNorm ---------------------------------------------------------------- */

/* 1 / sqrt(sum / n + eps) over the block's NT threads, ss = this thread's
 * sum of squares (every thread calls it). */
template <int NT>
__device__ __forceinline__ float rms_inv_block(float ss, int n, float eps) {
    __shared__ float red[NT / MM_WAVE];
    ss = wave_sum(ss);
    const int lane = threadIdx.x & (MM_WAVE - 1), wave = threadIdx.x / MM_WAVE;
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / MM_WAVE; w++) tot += red[w];
    return 1.0f / sqrtf(tot / (float)n + eps);
}

extern "C" __global__ __launch_bounds__(256) void mm_rmsnorm(mm_rmsnorm_args a) {
    const int t = blockIdx.x;
    const float *x = a.x + (size_t)t * a.n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < a.n; i += 256) ss += x[i] * x[i];
    const float inv = rms_inv_block<256>(ss, a.n, a.eps);
    float *y = a.y + (size_t)t * a.n;
    for (int i = threadIdx.x; i < a.n; i += 256) y[i] = x[i] * inv * bf16_f32(a.w[i]);
}

/* mm_reduce_rmsnorm_args: one block of RRN_T threads per row, each thread
 * RRN_PT elements (n <= RRN_T * RRN_PT) kept in registers between the sum
 * and the norm.  The partial loads of up to RRN_SU splits are issued
 * together: a row block is one latency-bound pass, so the loads must not
 * wait for each other. */
#define RRN_T MM_RRN_THREADS
#define RRN_PT MM_RRN_PT
#define RRN_SU 8
extern "C" __global__ __launch_bounds__(RRN_T) void mm_reduce_rmsnorm(mm_reduce_rmsnorm_args a) {
    const int t = blockIdx.x, n = a.n;
    const size_t plane = (size_t)a.T * n;
    float *x = a.x + (size_t)t * n;
    const float *p0 = a.part + (size_t)t * n;
    float v[RRN_PT];
#pragma unroll
    for (int k = 0; k < RRN_PT; k++) v[k] = 0.0f;
    for (int s0 = 0; s0 < a.nsplit; s0 += RRN_SU) {
        float pv[RRN_SU][RRN_PT];
#pragma unroll
        for (int u = 0; u < RRN_SU; u++)
#pragma unroll
            for (int k = 0; k < RRN_PT; k++) {
                const int i = threadIdx.x + RRN_T * k;
                pv[u][k] = (s0 + u < a.nsplit && i < n) ? p0[(size_t)(s0 + u) * plane + i] : 0.0f;
            }
#pragma unroll
        for (int u = 0; u < RRN_SU; u++)
#pragma unroll
            for (int k = 0; k < RRN_PT; k++)
                if (s0 + u < a.nsplit) v[k] = (s0 + u == 0) ? pv[u][k] : v[k] + pv[u][k];
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < RRN_PT; k++) {
        const int i = threadIdx.x + RRN_T * k;
        if (i < n) {
            const float xv = x[i] + v[k];
            x[i] = xv;
            v[k] = xv;
            ss += xv * xv;
        }
    }
    const float inv = rms_inv_block<RRN_T>(ss, n, a.eps);
    float *xn = a.xn + (size_t)t * n;
#pragma unroll
    for (int k = 0; k < RRN_PT; k++) {
        const int i = threadIdx.x + RRN_T * k;
        if (i < n) xn[i] = v[k] * inv * bf16_f32(a.w[i]);
    }
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

/* The register-resident GEMV core (gemv.h) over the vocabulary with the
 * final norm applied to the activations in registers, so no separate norm
 * pass runs.  Each wave keeps its best (logit, row) per token; the block's
 * best goes to part_v / part_i [t][block]: the argmax then only reduces
 * those partials. */
template <int NB>
struct lm_sink {
    float *y;
    int V, B;
    float bv[NB];
    int bi[NB];
    __device__ __forceinline__ void operator()(int row, int t, float v) {
        if ((threadIdx.x & (MM_WAVE - 1)) == 0 && t < B) y[(size_t)t * V + row] = v;
        if (am_better(v, row, bv[t], bi[t])) { bv[t] = v; bi[t] = row; }
    }
};

template <int NB>
__device__ __forceinline__ void lm_gemv(const mm_lm_gemv_args &a) {
    f32x4 xv[NB][GV_PPL][2];
    gemv_load_x<NB>(xv, a.x, a.B, a.H, a.norm, a.eps, false);
    lm_sink<NB> sk;
    sk.y = a.y;
    sk.V = a.V;
    sk.B = a.B;
#pragma unroll
    for (int t = 0; t < NB; t++) { sk.bv[t] = __builtin_nanf(""); sk.bi[t] = 0x7fffffff; }
    const uint16_t *w = a.w;
    const int H = a.H;
    gemv_rows<NB>(xv, H, a.V, [=](int r) { return w + (size_t)r * H; }, sk);
    /* the block's best per token: one partial per block */
    __shared__ float sv[NB][256 / MM_WAVE];
    __shared__ int si[NB][256 / MM_WAVE];
    const int lane = threadIdx.x & (MM_WAVE - 1), wave = threadIdx.x / MM_WAVE;
    if (lane == 0)
#pragma unroll
        for (int t = 0; t < NB; t++) { sv[t][wave] = sk.bv[t]; si[t][wave] = sk.bi[t]; }
    __syncthreads();
    if (threadIdx.x < NB && (int)threadIdx.x < a.B) {
        const int t = threadIdx.x;
        float v = sv[t][0];
        int i = si[t][0];
        for (int w2 = 1; w2 < 256 / MM_WAVE; w2++)
            if (am_better(sv[t][w2], si[t][w2], v, i)) { v = sv[t][w2]; i = si[t][w2]; }
        a.part_v[(size_t)t * gridDim.x + blockIdx.x] = v;
        a.part_i[(size_t)t * gridDim.x + blockIdx.x] = i;
    }
}

/* one entry point per token count (register allocation per instance) */
extern "C" __global__ __launch_bounds__(256) void mm_lm_gemv_1(mm_lm_gemv_args a) { lm_gemv<1>(a); }
extern "C" __global__ __launch_bounds__(256) void mm_lm_gemv_2(mm_lm_gemv_args a) { lm_gemv<2>(a); }
extern "C" __global__ __launch_bounds__(256) void mm_lm_gemv_4(mm_lm_gemv_args a) { lm_gemv<4>(a); }

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
