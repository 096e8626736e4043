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
 *   mm_i8_gu       grouped gate/up GEMM + SwiGLU epilogue -> h (fp32)
 *   mm_i8_quant_h  per-row quantisation of h -> qh, sh
 *   mm_i8_down     grouped down GEMM -> y per route (fp32)
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

#define I8_WAVES MM_I8_WAVES
#define I8_NBW MM_I8_NBW
#define I8_MT 4        /* 16-row tiles per pass (64 rows) */

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

/* ---- grouped GEMM ---------------------------------------------------------- */

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

/* One pass of up to MT*16 rows against this wave's I8_NBW column blocks.
 * GU: gate/up pair per column block (B fragments interleaved), SwiGLU
 * epilogue; otherwise a plain GEMM with a dequantising epilogue.  The K loop
 * is unrolled UNR deep so that UNR * I8_NBW * (GU ? 2 : 1) weight fragments
 * are in flight per wave.
 *   arow(m) -> pointer to row m of A (int8, K bytes), only called for m < M
 *   epi(m, col, acc0, acc1) consumes the int32 results of row m, column col */
template <bool GU, int MT, int UNR, class ARow, class Epi>
__device__ __forceinline__ void gemm_pass(const int8_t *bbase, int nb0, int nbl, int KB, int m0,
                                          int M, ARow arow, Epi epi) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int NB_STRIDE = (GU ? 2 : 1) * KB * 1024;
    const int nmt = min(MT, (M - m0 + 15) >> 4);
    const int8_t *ap[MT];
    bool av[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const int m = m0 + mi * 16 + (lane & 15);
        av[mi] = mi < nmt && m < M;
        ap[mi] = (av[mi] ? arow(m) : arow(m0)) + 16 * (lane >> 4);
    }
    const int8_t *bp[I8_NBW];
#pragma unroll
    for (int j = 0; j < I8_NBW; j++)
        bp[j] = bbase + (size_t)min(nb0 + j, nbl - 1) * NB_STRIDE + lane * 16;

    v4i acc0[MT][I8_NBW], acc1[MT][I8_NBW];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int j = 0; j < I8_NBW; j++) {
            acc0[mi][j] = (v4i){0, 0, 0, 0};
            acc1[mi][j] = (v4i){0, 0, 0, 0};
        }

    auto step = [&](int kb, const v4i *b0, const v4i *b1) {
        v4i a_[MT];
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            if (mi < nmt) {
                a_[mi] = *(const v4i *)(ap[mi] + kb * 64);
                if (!av[mi]) a_[mi] = (v4i){0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
            if (mi < nmt) {
#pragma unroll
                for (int j = 0; j < I8_NBW; j++) {
                    acc0[mi][j] = mfma_i8(a_[mi], b0[j], acc0[mi][j]);
                    if (GU) acc1[mi][j] = mfma_i8(a_[mi], b1[j], acc1[mi][j]);
                }
            }
        }
    };
    int kb = 0;
    for (; kb + UNR <= KB; kb += UNR) {
        v4i b0[UNR][I8_NBW], b1[UNR][I8_NBW];
#pragma unroll
        for (int u = 0; u < UNR; u++)
#pragma unroll
            for (int j = 0; j < I8_NBW; j++) {
                b0[u][j] = ldg16(bp[j] + (kb + u) * 1024);
                if (GU) b1[u][j] = ldg16(bp[j] + (KB + kb + u) * 1024);
            }
#pragma unroll
        for (int u = 0; u < UNR; u++) step(kb + u, b0[u], b1[u]);
    }
    for (; kb < KB; kb++) {
        v4i b0[I8_NBW], b1[I8_NBW];
#pragma unroll
        for (int j = 0; j < I8_NBW; j++) {
            b0[j] = ldg16(bp[j] + kb * 1024);
            if (GU) b1[j] = ldg16(bp[j] + (KB + kb) * 1024);
        }
        step(kb, b0, b1);
    }
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        if (mi < nmt) {
#pragma unroll
            for (int j = 0; j < I8_NBW; j++) {
                if (nb0 + j < nbl) {
                    const int col = (nb0 + j) * 16 + (lane & 15);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int m = m0 + mi * 16 + 4 * (lane >> 4) + i;
                        if (m < M) epi(m, col, acc0[mi][j][i], acc1[mi][j][i]);
                    }
                }
            }
        }
    }
}

/* Decode-shaped grouped GEMMs: one block per (expert, 128-column slab), every
 * row of the expert against the slab, weights streamed once.  SMALL = true
 * serves the routed experts with at most 16 rows (one 16-row tile, deep K
 * unroll, low register use); SMALL = false serves the rest and the shared
 * expert (four 16-row tiles per pass).  Both are launched; each block exits
 * when its expert belongs to the other variant. */
template <bool SMALL>
__device__ __forceinline__ void i8_gu_decode(const mm_i8_gemm_args &a) {
    constexpr int MT = SMALL ? 1 : I8_MT, UNR = SMALL ? 4 : 2;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int KB = a.H / 64;
    const int routed_blocks = a.E * a.wg_per_expert;
    const int b = blockIdx.x;
    if (b < routed_blocks) {
        const int e = b / a.wg_per_expert, wgi = b % a.wg_per_expert;
        const int M = min(a.cnt[e], a.T);
        const int nbl = a.I / 16;
        const int nb0 = (wgi * I8_WAVES + wave) * I8_NBW;
        if (M == 0 || nb0 >= nbl || (SMALL != (M <= 16))) return;
        const int32_t *rows = a.rows + (size_t)e * a.T;
        const int8_t *bbase = a.w.gu + (size_t)e * nbl * 2 * KB * 1024;
        const float *sg = a.w.s_g + (size_t)e * a.I, *su = a.w.s_u + (size_t)e * a.I;
        for (int m0 = 0; m0 < M; m0 += MT * 16) {
            gemm_pass<true, MT, UNR>(
                bbase, nb0, nbl, KB, m0, M,
                [&](int m) { return a.a + (size_t)(rows[m] / a.K) * a.H; },
                [&](int m, int col, int32_t ag, int32_t au) {
                    const int rid = rows[m];
                    const float sx = a.sa[rid / a.K];
                    const float g = ((float)ag * sx) * sg[col];
                    const float u = ((float)au * sx) * su[col];
                    a.h[(size_t)rid * a.I + col] = silu_mul(g, u);
                    if (a.dbg_acc) {
                        a.dbg_acc[((size_t)rid * 2) * a.I + col] = ag;
                        a.dbg_acc[((size_t)rid * 2 + 1) * a.I + col] = au;
                    }
                });
        }
    } else if (!SMALL) {
        const int sb = b - routed_blocks;
        const int nbl = a.S / 16;
        const int nb0 = (sb * I8_WAVES + wave) * I8_NBW;
        if (nb0 >= nbl) return;
        for (int m0 = 0; m0 < a.T; m0 += MT * 16) {
            gemm_pass<true, MT, UNR>(
                a.w.sgu, nb0, nbl, KB, m0, a.T,
                [&](int m) { return a.a + (size_t)m * a.H; },
                [&](int m, int col, int32_t ag, int32_t au) {
                    const float sx = a.sa[m];
                    const float g = ((float)ag * sx) * a.w.ss_g[col];
                    const float u = ((float)au * sx) * a.w.ss_u[col];
                    a.hs[(size_t)m * a.S + col] = silu_mul(g, u);
                });
        }
    }
}

template <bool SMALL>
__device__ __forceinline__ void i8_down_decode(const mm_i8_gemm_args &a) {
    constexpr int MT = SMALL ? 1 : I8_MT, UNR = SMALL ? 4 : 2;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int routed_blocks = a.E * a.wg_per_expert;
    const int nbl = a.H / 16;
    const int b = blockIdx.x;
    if (b < routed_blocks) {
        const int e = b / a.wg_per_expert, wgi = b % a.wg_per_expert;
        const int M = min(a.cnt[e], a.T);
        const int nb0 = (wgi * I8_WAVES + wave) * I8_NBW;
        if (M == 0 || nb0 >= nbl || (SMALL != (M <= 16))) return;
        const int KB = a.I / 64;
        const int32_t *rows = a.rows + (size_t)e * a.T;
        const int8_t *bbase = a.w.d + (size_t)e * nbl * KB * 1024;
        const float *sd = a.w.s_d + (size_t)e * a.H;
        for (int m0 = 0; m0 < M; m0 += MT * 16) {
            gemm_pass<false, MT, UNR>(
                bbase, nb0, nbl, KB, m0, M,
                [&](int m) { return a.a + (size_t)rows[m] * a.I; },
                [&](int m, int col, int32_t acc, int32_t) {
                    const int rid = rows[m];
                    a.y[(size_t)rid * a.H + col] = ((float)acc * a.sa[rid]) * sd[col];
                    if (a.dbg_acc) a.dbg_acc[(size_t)rid * a.H + col] = acc;
                });
        }
    } else if (!SMALL) {
        const int sb = b - routed_blocks;
        const int nb0 = (sb * I8_WAVES + wave) * I8_NBW;
        if (nb0 >= nbl) return;
        const int KB = a.S / 64;
        for (int m0 = 0; m0 < a.T; m0 += MT * 16) {
            gemm_pass<false, MT, UNR>(
                a.w.sdn, nb0, nbl, KB, m0, a.T,
                [&](int m) { return a.a_sh + (size_t)m * a.S; },
                [&](int m, int col, int32_t acc, int32_t) {
                    a.ys[(size_t)m * a.H + col] = ((float)acc * a.sa_sh[m]) * a.w.ss_d[col];
                });
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_i8_gu_s(mm_i8_gemm_args a) {
    i8_gu_decode<true>(a);
}
extern "C" __global__ __launch_bounds__(256) void mm_i8_gu(mm_i8_gemm_args a) {
    i8_gu_decode<false>(a);
}
extern "C" __global__ __launch_bounds__(256) void mm_i8_down_s(mm_i8_gemm_args a) {
    i8_down_decode<true>(a);
}
extern "C" __global__ __launch_bounds__(256) void mm_i8_down(mm_i8_gemm_args a) {
    i8_down_decode<false>(a);
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
