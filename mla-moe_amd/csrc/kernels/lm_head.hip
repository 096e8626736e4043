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

/* As mm_rmsnorm (the same arithmetic), the normalised row written as bf16
 * hi/lo planes: hi = rne16(y), lo = rne16(y - hi), the split the bf16 GEMMs
 * apply to fp32 activations.  grid (T). */
extern "C" __global__ __launch_bounds__(256) void mm_rmsnorm_hl(mm_rmsnorm_hl_args a) {
    const int t = blockIdx.x;
    const float *x = a.x + (size_t)t * a.n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < a.n; i += 256) ss += x[i] * x[i];
    const float inv = rms_inv_block<256>(ss, a.n, a.eps);
    uint16_t *hi = a.yhl + (size_t)t * a.n, *lo = hi + (size_t)gridDim.x * a.n;
    /* 8 consecutive values per thread (n is a multiple of 8): 16-byte
     * stores of each plane */
    typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
    for (int i = 8 * threadIdx.x; i < a.n; i += 8 * 256) {
        const f32x4 x0 = *(const f32x4 *)(x + i), x1 = *(const f32x4 *)(x + i + 4);
        const u16x8_t w8 = *(const u16x8_t *)(a.w + i);
        u16x8_t h8, l8;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            /* no contraction: lo splits the rounded fp32 y, as the GEMMs
             * that split a stored row do (y - hi fused with y's last
             * product would split the unrounded product) */
#pragma clang fp contract(off)
            const float v = (k < 4 ? x0[k & 3] : x1[k & 3]) * inv * bf16_f32(w8[k]);
            h8[k] = rne16(v);
            l8[k] = rne16(v - bf16_f32(h8[k]));
        }
        *(u16x8_t *)(hi + i) = h8;
        *(u16x8_t *)(lo + i) = l8;
    }
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

/* ---- logits GEMM for 5..64 rows ----------------------------------------------
 *
 * y[T, N] = x . W^T for the LM head's batch rows: MM_LMG_BN = 256 vocabulary
 * rows (output columns) per block, one block per CU (4 waves, wave w owns
 * columns 64 w .. + 63 for all 64 token rows: 4 x 4 tiles of
 * v_mfma_f32_16x16x32_bf16, x as the A operand and W as B, each fp32 x a
 * bf16 hi/lo pair as in mm_gemm_skinny, the same MFMA sequence per output:
 * per 32-wide K step the hi product, then the lo product).
 *
 * Both operands go global -> LDS by direct loads into a ring of
 * MM_LMG_NS stages of one 64-wide K chunk (W: 256 rows x 128 B; x: the hi
 * and lo planes, 64 rows x 128 B each), two chunks ahead of their use.  The
 * skinny GEMM staged x through registers, so each wait for x -- an L2 hit
 * -- also waited for the weight loads issued before it (vector memory
 * counts complete in order) and the weight stream ran ~2 chunks deep:
 * 0.35 of HBM peak at the LM head.  Here every load in the loop belongs to
 * the ring, whose stages complete in the order they are consumed.
 * Measured against streaming W into registers four chunks deep with x alone
 * in the ring (one wave per SIMD): 114 against 161 us at 64 x 102400 x 2048.
 *
 * LDS rows are 128 B (8 pieces of 16 B); piece p of row r sits in slot
 * p ^ swz(r), so the 16 lanes of an MFMA operand read (16 consecutive rows,
 * one piece) hit 16 distinct 16-byte bank groups. */
#define LMG_WB (MM_LMG_BN * 128)     /* W bytes per stage */
#define LMG_LPW 12                   /* direct loads per wave per stage: 8 of W, 4 of x */
typedef __bf16 lmg_bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int lmg_swz(int r) { return (r >> 1) & 7; }

extern "C" __global__ __launch_bounds__(256) void mm_lm_gemm(mm_lm_gemm_args a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * MM_LMG_BN;
    const int K = a.K, T = a.T, N = a.N, nch = K / 64;
    const int q = lane & 7;

    /* direct loads of a chunk: W instruction 8 wave + u covers tile rows
     * (columns) 8 (8 wave + u) .. + 7, x instruction 4 wave + u plane
     * (4 wave + u) / 8, token rows 8 ((4 wave + u) % 8) .. + 7; lane l loads
     * row + l / 8, slot q = l % 8, i.e. piece q ^ swz(row).  Rows past N or
     * T load the last one (not stored). */
    const uint16_t *wp[8], *xp[4];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int c = 8 * (8 * wave + u) + (lane >> 3);
        wp[u] = a.w + (size_t)min(n0 + c, N - 1) * K + 8 * (q ^ lmg_swz(c));
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int i = 4 * wave + u, r = 8 * (i & 7) + (lane >> 3);
        xp[u] = a.xhl + (size_t)(i >> 3) * T * K + (size_t)min(r, T - 1) * K + 8 * (q ^ lmg_swz(r));
    }
    auto issue = [&](int c, int st) {
        uint8_t *sb = lds + st * MM_LMG_STAGE;
#pragma unroll
        for (int u = 0; u < 8; u++) lds_dma16(wp[u] + 64 * c, sb + (8 * wave + u) * 1024);
#pragma unroll
        for (int u = 0; u < 4; u++) lds_dma16(xp[u] + 64 * c, sb + LMG_WB + (4 * wave + u) * 1024);
    };

    /* operand reads (bytes within a stage), K half s: A rows 16 g + l % 16,
     * B rows (columns) 64 wave + 16 j + l % 16, piece 4 s + l / 16 */
    uint32_t ao[2][4], bo[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int p = 4 * s + (lane >> 4);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int r = 16 * g + (lane & 15);
            ao[s][g] = LMG_WB + r * 128 + 16 * (p ^ lmg_swz(r));
            const int c = 64 * wave + 16 * g + (lane & 15);
            bo[s][g] = c * 128 + 16 * (p ^ lmg_swz(c));
        }
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) acc[j][g] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t l0 = lds_addr(lds);
    issue(0, 0);
    if (nch > 1) issue(1, 1);
    for (int c = 0; c < nch; c++) {
        /* chunk c landed: the loads of chunk c + 1 (issued after) may stay
         * out; the barrier makes every wave's loads of chunk c visible and
         * frees the stage of chunk c - 1 for chunk c + 2 */
        if (c + 1 < nch) VMCNT_WAIT(LMG_LPW);
        else VMCNT_WAIT(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (c + 2 < nch) issue(c + 2, (c + 2) % MM_LMG_NS);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t sb = l0 + (uint32_t)((c % MM_LMG_NS) * MM_LMG_STAGE);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            i32x4 xa[4][2], wb[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                xa[g][0] = ds_read16(sb + ao[s][g]);
                xa[g][1] = ds_read16(sb + ao[s][g] + 64 * 128);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) wb[j] = ds_read16(sb + bo[s][j]);
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(xa[0][0]), "+v"(xa[0][1]), "+v"(xa[1][0]), "+v"(xa[1][1]),
                           "+v"(xa[2][0]), "+v"(xa[2][1]), "+v"(xa[3][0]), "+v"(xa[3][1]),
                           "+v"(wb[0]), "+v"(wb[1]), "+v"(wb[2]), "+v"(wb[3]));
            /* every output takes its hi product, then its lo product; the
             * 16 hi MFMAs go first so that no MFMA waits on the one just
             * issued */
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(lmg_bf16x8, xa[g][h]),
                            __builtin_bit_cast(lmg_bf16x8, wb[j]), acc[j][g], 0, 0, 0);
        }
    }
    /* C[token 16 g + 4 (l / 16) + i][column n0 + 64 wave + 16 j + l % 16] */
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + 64 * wave + 16 * j + (lane & 15);
        if (n >= N) continue;
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * g + 4 * (lane >> 4) + i;
                if (t < T) a.y[(size_t)t * N + n] = acc[j][g][i];
            }
    }
}
