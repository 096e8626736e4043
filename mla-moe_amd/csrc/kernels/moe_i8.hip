/* moe_i8.hip -- MoE expert FFN with int8 weights and int8 activations on
 * v_mfma_i32_16x16x64_i8 (int32 accumulation).
 *
 * Semantics follow ffn_compute (src/run.c:116-162) with each expert matmul
 * replaced by: per-token int8 activations (s = max|x|/127, q = rint(x/s)),
 * per-output-channel int8 weights (same rule), exact int32 dot products,
 * dequantisation ((float)acc * s_a) * s_w, SwiGLU in fp32, per-route int8
 * quantisation of the hidden row, int8 down projection, and the combine of
 * run.c:151-160 in slot order with the shared expert last.
 *
 * Kernels, in launch order:
 *   mm_i8_route    router (router.h), per-expert row lists built with one
 *                  atomic slot per route, per-token quantisation of x
 *   mm_i8_gu       grouped gate/up GEMM + SwiGLU epilogue -> h (fp32),
 *                  routed and shared experts in one launch (decode sizes)
 *   mm_i8_quant_h  per-row quantisation of h -> qh, sh
 *   mm_i8_down     grouped down GEMM -> y per route (fp32)
 *   mm_i8_gemm_tiled  block-tiled variant of both GEMMs for prefill sizes
 *   mm_i8_combine  out[t] = sum_r w_r * y[t, r] + y_shared[t]
 *
 * The order of rows inside an expert's list depends on atomic timing, but
 * every row is computed independently and written to its own route slot,
 * so results do not depend on it.
 *
 * MFMA operand layout (16x16x64 i8): lane l supplies row (l % 16) of the
 * A operand and column (l % 16) of the B operand, bytes 16*(l/16) .. +15 of
 * the 64-wide K step, for both; the int32 result element i of lane l is
 * D[4*(l/16) + i][l % 16].  Weights are pre-packed so that a wave's B
 * operand for one K step is one contiguous 1 KB block (kernel_params.h).
 */
#include "router.h"

typedef int32_t v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i ldg16(const int8_t *p) {
    return __builtin_nontemporal_load((const v4i *)p);
}

/* ---- routing + activation quantisation ----------------------------------- */

/* s = max|x| / 127; q = clamp(rint(x / s), -127, 127), IEEE division and
 * round-half-even, identical to the CPU quantiser.  One wave, n % 4 == 0. */
__device__ __forceinline__ void quant_row_wave(const float *x, int n, int8_t *q, float *s) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    float amax = 0.0f;
    for (int i = lane * 4; i < n; i += MM_WAVE * 4) {
        f32x4 v = *(const f32x4 *)(x + i);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    amax = wave_max(amax);
    const float sc = amax / 127.0f;
    if (lane == 0) *s = sc;
    for (int i = lane * 4; i < n; i += MM_WAVE * 4) {
        f32x4 v = *(const f32x4 *)(x + i);
        int b[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float r = sc == 0.0f ? 0.0f : fminf(fmaxf(rintf(v[j] / sc), -127.0f), 127.0f);
            b[j] = (int)r & 0xff;
        }
        *(uint32_t *)(q + i) = (uint32_t)(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24));
    }
}

extern "C" __global__ __launch_bounds__(MM_ROUTER_THREADS) void mm_i8_route(mm_i8_route_args a) {
    __shared__ float lds[MM_ROUTER_LDS_FLOATS];
    const int lane = threadIdx.x & (MM_WAVE - 1);
    router_block(a.r, blockIdx.x, lds, [&](int tok, const int *idx, const float *) {
        int e = 0;
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++)
            if (lane == r) e = idx[r];
        if (lane < a.r.K) {
            int pos = atomicAdd(&a.cnt[e], 1);
            if (pos < a.r.T) a.rows[(size_t)e * a.r.T + pos] = tok * a.r.K + lane;
        }
        quant_row_wave(a.x + (size_t)tok * a.r.H, a.r.H, a.qx + (size_t)tok * a.r.H,
                       a.sx + tok);
    });
}

/* ---- streaming grouped GEMM (decode) ------------------------------------------- */

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

/* One work unit = one wave = NF weight fragment columns (16 output columns
 * each; for gate/up the gate and the up fragment of one column block) of one
 * expert over the whole K, against MT 16-row tiles of that expert's rows.
 *
 * Weights stream once from HBM with non-temporal loads through a D-deep
 * register ring: the loads of K step kb + D are issued as soon as step kb's
 * MFMAs have been issued, so every wave keeps D steps of fragments in flight
 * and never drains its queue inside the K loop.  The A rows (a few KB, read
 * by every unit of the expert) come through the caches.
 *
 * Rows are independent in D = A * B, so lanes whose row is past M read any
 * valid row and their results are discarded by the epilogue.
 *   bp[f]  : lane's 16-byte slice of fragment column f at K step 0
 *   ap[mi] : lane's 16-byte slice of A row tile mi at K step 0
 * On return acc[mi][f] holds D[4*(lane/16) + i][lane % 16] of tile mi,
 * fragment column f. */
template <int NF, int MT, int D>
__device__ __forceinline__ void stream_k(const int8_t *const (&bp)[NF], const int8_t *const (&ap)[MT],
                                         int KB, v4i (&acc)[MT][NF]) {
    v4i bq[D][NF], aq[D][MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int f = 0; f < NF; f++) acc[mi][f] = (v4i){0, 0, 0, 0};
    /* The scheduling barriers keep the loads in slot order, which is what
     * lets the inserted waits stay partial (vmcnt counts in issue order). */
    auto load = [&](int slot, int kb) {
#pragma unroll
        for (int f = 0; f < NF; f++) bq[slot][f] = ldg16(bp[f] + (size_t)kb * 1024);
#pragma unroll
        for (int mi = 0; mi < MT; mi++) aq[slot][mi] = *(const v4i *)(ap[mi] + kb * 64);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto consume = [&](int slot) {
#pragma unroll
        for (int mi = 0; mi < MT; mi++)
#pragma unroll
            for (int f = 0; f < NF; f++) acc[mi][f] = mfma_i8(aq[slot][mi], bq[slot][f], acc[mi][f]);
        __builtin_amdgcn_sched_barrier(0);
    };
    /* unconditional (clamped) so that the loop is entered with a known
     * number of loads in flight and the waits inside it stay partial */
#pragma unroll
    for (int d = 0; d < D; d++) load(d, min(d, KB - 1));
    int kb0 = 0;
    /* steady state: every slot is refilled D steps ahead, unconditionally */
    for (; kb0 + 2 * D <= KB; kb0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            consume(d);
            load(d, kb0 + d + D);
        }
    }
    /* last D .. 2D-1 steps */
#pragma unroll
    for (int d = 0; d < D; d++) {
        if (kb0 + d < KB) consume(d);
        if (kb0 + d + D < KB) load(d, kb0 + d + D);
    }
#pragma unroll
    for (int d = 0; d < D; d++)
        if (kb0 + D + d < KB) consume(d);
}

/* Row ids of a 16-row tile for the epilogue: lane l's results are rows
 * 4*(l/16) + i; the A-side row id of tile row r sits in lane r. */
__device__ __forceinline__ int tile_row_id(int a_side_id, int i) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    return __shfl(a_side_id, 4 * (lane >> 4) + i, MM_WAVE);
}

/* Gate/up + SwiGLU for one unit: rows m0 .. min(M, m0 + 16*MT) - 1 of an
 * expert (or of the shared expert), column blocks nb0 .. nb0 + NBW - 1.
 * rid_of(m): route id of row m (the row of h written); tok_of(rid): row of qx. */
template <int NBW, int MT, int D, class RidOf, class TokOf>
__device__ __forceinline__ void gu_unit(const mm_i8_gemm_args &a, const int8_t *bbase, int KB,
                                        int nb0, int m0, int M, const float *sg, const float *su,
                                        float *hout, int ncols, int32_t *dbg, RidOf rid_of,
                                        TokOf tok_of) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int8_t *bp[2 * NBW];
#pragma unroll
    for (int j = 0; j < NBW; j++) {
        bp[2 * j] = bbase + (size_t)(nb0 + j) * 2 * KB * 1024 + lane * 16;
        bp[2 * j + 1] = bp[2 * j] + (size_t)KB * 1024;
    }
    int rid_a[MT];
    float sx_a[MT];
    const int8_t *ap[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const int m = min(m0 + mi * 16 + (lane & 15), M - 1);
        rid_a[mi] = rid_of(m);
        const int t = tok_of(rid_a[mi]);
        sx_a[mi] = a.sa[t];
        ap[mi] = a.a + (size_t)t * a.H + 16 * (lane >> 4);
    }
    float cg[NBW], cu[NBW];
#pragma unroll
    for (int j = 0; j < NBW; j++) {
        const int col = (nb0 + j) * 16 + (lane & 15);
        cg[j] = sg[col];
        cu[j] = su[col];
    }
    v4i acc[MT][2 * NBW];
    stream_k<2 * NBW, MT, D>(bp, ap, KB, acc);
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + mi * 16 + 4 * (lane >> 4) + i;
            const int rid = tile_row_id(rid_a[mi], i);
            const float sx = __shfl(sx_a[mi], 4 * (lane >> 4) + i, MM_WAVE);
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < NBW; j++) {
                const int col = (nb0 + j) * 16 + (lane & 15);
                const int32_t ag = acc[mi][2 * j][i], au = acc[mi][2 * j + 1][i];
                const float g = ((float)ag * sx) * cg[j];
                const float u = ((float)au * sx) * cu[j];
                hout[(size_t)rid * ncols + col] = silu_mul(g, u);
                if (dbg) {
                    dbg[((size_t)rid * 2) * ncols + col] = ag;
                    dbg[((size_t)rid * 2 + 1) * ncols + col] = au;
                }
            }
        }
}

/* Down projection for one unit; y[rid] = dequantised A row rid times W_d. */
template <int NBW, int MT, int D, class RidOf>
__device__ __forceinline__ void down_unit(const int8_t *abase, const float *sa, int Kd,
                                          const int8_t *bbase, int nb0, int m0, int M,
                                          const float *sd, float *yout, int ncols, int32_t *dbg,
                                          RidOf rid_of) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int KB = Kd / 64;
    const int8_t *bp[NBW];
#pragma unroll
    for (int j = 0; j < NBW; j++) bp[j] = bbase + (size_t)(nb0 + j) * KB * 1024 + lane * 16;
    int rid_a[MT];
    float sa_a[MT];
    const int8_t *ap[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const int m = min(m0 + mi * 16 + (lane & 15), M - 1);
        rid_a[mi] = rid_of(m);
        sa_a[mi] = sa[rid_a[mi]];
        ap[mi] = abase + (size_t)rid_a[mi] * Kd + 16 * (lane >> 4);
    }
    float cd[NBW];
#pragma unroll
    for (int j = 0; j < NBW; j++) cd[j] = sd[(nb0 + j) * 16 + (lane & 15)];
    v4i acc[MT][NBW];
    stream_k<NBW, MT, D>(bp, ap, KB, acc);
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + mi * 16 + 4 * (lane >> 4) + i;
            const int rid = tile_row_id(rid_a[mi], i);
            const float s = __shfl(sa_a[mi], 4 * (lane >> 4) + i, MM_WAVE);
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < NBW; j++) {
                const int col = (nb0 + j) * 16 + (lane & 15);
                const int32_t ac = acc[mi][j][i];
                yout[(size_t)rid * ncols + col] = ((float)ac * s) * cd[j];
                if (dbg) dbg[(size_t)rid * ncols + col] = ac;
            }
        }
}

#define GU_NBW MM_I8S_NBW_GU
#define DN_NBW MM_I8S_NBW_DOWN
#define S_WAVES MM_I8S_WAVES

/* Decode-shaped gate/up.  Block = S_WAVES waves.  Blocks [0, S/16/GU_NBW)
 * serve the shared expert: one column unit per block, wave w taking the
 * 16-row tiles w, w + S_WAVES, ... of the T rows, so the block's waves
 * stream the same weight fragments at the same time and all but the first
 * read of each is a cache hit.  The remaining blocks serve the routed
 * experts: S_WAVES consecutive column units of one expert per block, every
 * wave all of the expert's rows (16 at a time).  Shared blocks come first so
 * their longer work starts early; a routed block of an expert with no rows
 * exits at once. */
extern "C" __global__ __launch_bounds__(MM_I8S_WAVES * MM_WAVE) void mm_i8_gu(mm_i8_gemm_args a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int KB = a.H / 64;
    const int n_sh = a.S / (16 * GU_NBW);
    const int b = blockIdx.x;
    /* one call site for both kinds of block (a single copy of the unit) */
    const int8_t *bbase;
    const float *sg, *su;
    const int32_t *rows;
    float *hout;
    int32_t *dbg;
    int nb0, M, m0, mstep, ncols, kdiv;
    if (b < n_sh) {
        bbase = a.w.sgu;
        sg = a.w.ss_g;
        su = a.w.ss_u;
        rows = nullptr;
        hout = a.hs;
        dbg = nullptr;
        nb0 = b * GU_NBW;
        M = a.T;
        m0 = wave * 16;
        mstep = 16 * S_WAVES;
        ncols = a.S;
        kdiv = 1;
    } else {
        const int nbl = a.I / 16;
        const int per_e = (nbl + S_WAVES * GU_NBW - 1) / (S_WAVES * GU_NBW);
        const int v = b - n_sh, e = v / per_e;
        nb0 = ((v % per_e) * S_WAVES + wave) * GU_NBW;
        M = min(a.cnt[e], a.T);
        if (M == 0 || nb0 >= nbl) return;
        bbase = a.w.gu + (size_t)e * nbl * 2 * KB * 1024;
        sg = a.w.s_g + (size_t)e * a.I;
        su = a.w.s_u + (size_t)e * a.I;
        rows = a.rows + (size_t)e * a.T;
        hout = a.h;
        dbg = a.dbg_acc;
        m0 = 0;
        mstep = 16;
        ncols = a.I;
        kdiv = a.K;
    }
    for (; m0 < M; m0 += mstep)
        gu_unit<GU_NBW, 1, 4>(a, bbase, KB, nb0, m0, M, sg, su, hout, ncols, dbg,
                              [&](int m) { return rows ? rows[m] : m; },
                              [&](int r) { return r / kdiv; });
}

/* Decode-shaped down projection, same block layout: H/16/DN_NBW shared
 * blocks (when there is a shared expert), then the routed experts'. */
extern "C" __global__ __launch_bounds__(MM_I8S_WAVES * MM_WAVE) void mm_i8_down(mm_i8_gemm_args a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int nbl = a.H / 16;
    const int n_sh = a.S ? nbl / DN_NBW : 0;
    const int b = blockIdx.x;
    const int8_t *abase, *bbase;
    const float *sa, *sd;
    const int32_t *rows;
    float *yout;
    int32_t *dbg;
    int nb0, M, m0, mstep, Kd;
    if (b < n_sh) {
        abase = a.a_sh;
        sa = a.sa_sh;
        Kd = a.S;
        bbase = a.w.sdn;
        sd = a.w.ss_d;
        rows = nullptr;
        yout = a.ys;
        dbg = nullptr;
        nb0 = b * DN_NBW;
        M = a.T;
        m0 = wave * 16;
        mstep = 16 * S_WAVES;
    } else {
        const int per_e = (nbl + S_WAVES * DN_NBW - 1) / (S_WAVES * DN_NBW);
        const int v = b - n_sh, e = v / per_e;
        nb0 = ((v % per_e) * S_WAVES + wave) * DN_NBW;
        M = min(a.cnt[e], a.T);
        if (M == 0 || nb0 >= nbl) return;
        abase = a.a;
        sa = a.sa;
        Kd = a.I;
        bbase = a.w.d + (size_t)e * nbl * (a.I / 64) * 1024;
        sd = a.w.s_d + (size_t)e * a.H;
        rows = a.rows + (size_t)e * a.T;
        yout = a.y;
        dbg = a.dbg_acc;
        m0 = 0;
        mstep = 16;
    }
    for (; m0 < M; m0 += mstep)
        down_unit<DN_NBW, 1, 4>(abase, sa, Kd, bbase, nb0, m0, M, sd, yout, a.H, dbg,
                                [&](int m) { return rows ? rows[m] : m; });
}

/* ---- hidden-row quantisation and combine ------------------------------------- */

extern "C" __global__ __launch_bounds__(256) void mm_i8_quant_h(mm_i8_quant_rows_args a) {
    const int row = blockIdx.x * (blockDim.x / MM_WAVE) + threadIdx.x / MM_WAVE;
    if (row < a.rows)
        quant_row_wave(a.h + (size_t)row * a.n, a.n, a.q + (size_t)row * a.n, a.s + row);
    else if (row - a.rows < a.rows2) {
        const int r = row - a.rows;
        quant_row_wave(a.h2 + (size_t)r * a.n2, a.n2, a.q2 + (size_t)r * a.n2, a.s2 + r);
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_i8_combine(mm_i8_combine_args a) {
    const int t = blockIdx.x;
    const float *w = a.topk_w + (size_t)t * a.K;
    for (int n = threadIdx.x * 4; n < a.H; n += blockDim.x * 4) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int r = 0; r < a.K; r++) {
            const f32x4 y = *(const f32x4 *)(a.y + ((size_t)t * a.K + r) * a.H + n);
            acc += w[r] * y;
        }
        if (a.has_shared) acc += *(const f32x4 *)(a.ys + (size_t)t * a.H + n);
        f32x4 *o = (f32x4 *)(a.out + (size_t)t * a.H + n);
        *o = a.accumulate ? *o + acc : acc;
    }
    if (t == 0)
        for (int e = threadIdx.x; e < a.E; e += blockDim.x) a.cnt[e] = 0;
}

/* ---- weight packing ----------------------------------------------------------- */

/* One thread per 16-byte lane slice of a fragment. */
extern "C" __global__ __launch_bounds__(256) void mm_pack_i8(mm_pack_i8_args a) {
    const int KB = a.K / 64, NB = a.N / 16, NS = a.src1 ? 2 : 1;
    const size_t total = (size_t)NB * NS * KB * 64;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i & 63);
        const size_t f = i >> 6;
        const int kb = (int)(f % KB);
        const int which = (int)((f / KB) % NS);
        const int nb = (int)(f / ((size_t)KB * NS));
        const int8_t *src = which ? a.src1 : a.src0;
        const size_t row = (size_t)nb * 16 + (lane & 15);
        const size_t col = (size_t)kb * 64 + 16 * (lane >> 4);
        *(v4i *)(a.dst + i * 16) = *(const v4i *)(src + row * a.K + col);
    }
}

/* ---- tiled grouped GEMM (prefill) ------------------------------------------- */

/* Block tile: MM_I8T_BM rows x 8 B fragments (gate/up: 4 column blocks of
 * 16 with their gate and up fragments = 64 output columns; plain: 8 column
 * blocks = 128 output columns), K step 64.  Four waves in a 2 x 2 grid, each
 * a 64-row x 4-fragment tile: 16 v_mfma_i32_16x16x64_i8 per K step.
 * A (gathered rows) and B (packed fragments) are staged through two LDS
 * buffers of 16 KB in MFMA operand order; the next K step's global loads are
 * issued before the current step's MFMAs.  grid.x = column tile, grid.y =
 * row tile over all experts (prefix of ceil(rows_e / 128)). */
#define T_FRAGS 8

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

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

/* 16 bytes per lane from `src` into LDS at `dst` + 16 * lane (direct
 * global -> LDS load, no VGPR staging). */
__device__ __forceinline__ void lds_dma16(const void *src, void *dst) {
    __builtin_amdgcn_global_load_lds((glb_void_t *)src, (lds_void_t *)dst, 16, 0, 0);
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
__device__ __forceinline__ v4i ds_read16(uint32_t addr) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
    return r;
}

/* s_waitcnt vmcnt(n) only (expcnt and lgkmcnt left at their maxima). */
#define VMCNT_WAIT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))

#define T_STAGES 4
#define T_STAGE_BYTES (2 * T_FRAGS * 1024)

/* One 128-row x 8-fragment tile starting at row m0 of expert e (M rows). */
__device__ __forceinline__ void tiled_tile(const mm_i8_tiled_args &a, int8_t (*lds)[T_STAGE_BYTES],
                                           int e, int m0, int M) {
    const int tid = threadIdx.x, lane = tid & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / MM_WAVE);
    const int wm = wave >> 1, wn = wave & 1;
    const int KB = a.Kd / 64;
    const int nfr_total = (a.gu ? 2 : 1) * (a.N / 16);
    const int fr0 = blockIdx.x * T_FRAGS;
    const int32_t *rows = a.rows ? a.rows + (size_t)e * a.T : nullptr;
    const int8_t *bexp = a.b + (size_t)e * a.b_expert_stride;

    /* Wave w loads A fragments 2w, 2w+1 (rows 32w .. 32w+31 of the tile) and
     * B fragments 2w, 2w+1 of every K step.  Lane L of an A fragment carries
     * row (L % 16), bytes 16 * (L / 16) of the 64-byte K step. */
    const int8_t *asrc[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int m = m0 + (2 * wave + h) * 16 + (lane & 15);
        int arow = 0;
        if (m < M) {
            const int rid = rows ? rows[m] : m;
            arow = (a.a_by_route || !rows) ? rid : rid / a.K;
        } else {
            const int rid = rows ? rows[m0] : m0;   /* any valid row; result discarded */
            arow = (a.a_by_route || !rows) ? rid : rid / a.K;
        }
        asrc[h] = a.a + (size_t)arow * a.Kd + (lane >> 4) * 16;
    }
    const int8_t *bsrc[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
        bsrc[h] = bexp + (size_t)min(fr0 + 2 * wave + h, nfr_total - 1) * KB * 1024 + lane * 16;
    auto issue = [&](int kb) {
        int8_t *st = lds[kb % T_STAGES];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            lds_dma16(asrc[h] + kb * 64, st + (2 * wave + h) * 1024);
            lds_dma16(bsrc[h] + (size_t)kb * 1024, st + T_FRAGS * 1024 + (2 * wave + h) * 1024);
        }
    };

    v4i acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int f = 0; f < 4; f++) acc[mi][f] = (v4i){0, 0, 0, 0};

#pragma unroll
    for (int s = 0; s < T_STAGES - 1; s++)
        if (s < KB) issue(s);
    for (int kb = 0; kb < KB; kb++) {
        /* this wave's loads for step kb are done once at most 4 * (number of
         * later steps already issued) of its loads are outstanding */
        const int later = min(T_STAGES - 2, KB - 1 - kb);
        if (later >= 2) VMCNT_WAIT(8);
        else if (later == 1) VMCNT_WAIT(4);
        else VMCNT_WAIT(0);
        __builtin_amdgcn_s_barrier();   /* every wave's part of stage kb has landed,
                                           and stage kb-1 is no longer being read */
        if (kb + T_STAGES - 1 < KB) issue(kb + T_STAGES - 1);
        const uint32_t st = lds_addr(lds[kb % T_STAGES]) + lane * 16;
        v4i av[4], bv[4];
#pragma unroll
        for (int mi = 0; mi < 4; mi++) av[mi] = ds_read16(st + (wm * 4 + mi) * 1024);
#pragma unroll
        for (int f = 0; f < 4; f++) bv[f] = ds_read16(st + T_FRAGS * 1024 + (wn * 4 + f) * 1024);
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]), "+v"(bv[0]),
                       "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]));
#pragma unroll
        for (int mi = 0; mi < 4; mi++)
#pragma unroll
            for (int f = 0; f < 4; f++) acc[mi][f] = mfma_i8(av[mi], bv[f], acc[mi][f]);
    }

    /* epilogue */
    const float *sb0 = a.sb0 + (size_t)e * a.sb_expert_stride;
    const float *sb1 = a.sb1 ? a.sb1 + (size_t)e * a.sb_expert_stride : nullptr;
#pragma unroll
    for (int mi = 0; mi < 4; mi++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + wm * 64 + mi * 16 + 4 * (lane >> 4) + i;
            if (m >= M) continue;
            const int rid = rows ? rows[m] : m;
            const int arow = (a.a_by_route || !rows) ? rid : rid / a.K;
            const float sa = a.sa[arow];
            if (a.gu) {
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int nb = (fr0 >> 1) + wn * 2 + k;
                    if (nb * 16 >= a.N) continue;
                    const int col = nb * 16 + (lane & 15);
                    const int32_t ag = acc[mi][2 * k][i], au = acc[mi][2 * k + 1][i];
                    const float g = ((float)ag * sa) * sb0[col];
                    const float u = ((float)au * sa) * sb1[col];
                    a.out[(size_t)rid * a.N + col] = silu_mul(g, u);
                    if (a.dbg_acc) {
                        a.dbg_acc[((size_t)rid * 2) * a.N + col] = ag;
                        a.dbg_acc[((size_t)rid * 2 + 1) * a.N + col] = au;
                    }
                }
            } else {
#pragma unroll
                for (int f = 0; f < 4; f++) {
                    const int nb = fr0 + wn * 4 + f;
                    if (nb * 16 >= a.N) continue;
                    const int col = nb * 16 + (lane & 15);
                    const int32_t ac = acc[mi][f][i];
                    a.out[(size_t)rid * a.N + col] = ((float)ac * sa) * sb0[col];
                    if (a.dbg_acc) a.dbg_acc[(size_t)rid * a.N + col] = ac;
                }
            }
        }
    }
}

/* grid.x = 8-fragment column slab, grid.y = row group.  A block walks the
 * group's 128-row tiles in order, so the slab's weights (K x 128 bytes) come
 * from HBM once and from this CU's L2 for the group's later tiles. */
extern "C" __global__ __launch_bounds__(256) void mm_i8_gemm_tiled(mm_i8_tiled_args a) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[T_STAGES][T_STAGE_BYTES];
    int e, g0, M;
    if (!tile_owner(a, blockIdx.y, &e, &g0, &M)) return;
    const int nfr_total = (a.gu ? 2 : 1) * (a.N / 16);
    if ((int)blockIdx.x * T_FRAGS >= nfr_total) return;   /* uniform per block */
    const int g1 = min(M, g0 + a.mgroup * MM_I8T_BM);
    for (int m0 = g0; m0 < g1; m0 += MM_I8T_BM) {
        tiled_tile(a, lds, e, m0, M);
        __builtin_amdgcn_s_barrier();   /* the LDS ring is refilled by the next tile */
    }
}
