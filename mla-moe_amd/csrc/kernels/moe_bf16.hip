/* moe_bf16.hip -- MoE expert FFN with bf16 weights and fp32 activations for
 * small token counts (T=1 decode), as three GEMV stages.
 *
 * Reference semantics: ffn_compute (src/run.c:116-162).  Weights are
 * row-major [rows, K] bf16 exactly as the reference stores them; every GEMV
 * reads a weight row once with 128-bit loads, 64 lanes covering 1 KB
 * contiguous per instruction, and accumulates in fp32.
 *
 *   stage 1  blocks [0, n_router_blocks): router (router.h)
 *            other blocks: shared-expert gate/up rows for all T tokens,
 *            SwiGLU, written to hcat[t, K*I + j]
 *   stage 2  routed gate/up for every (token, slot) route, SwiGLU scaled by
 *            the route weight, written to hcat[t, r*I + j]
 *   stage 3  out[t, d] = sum over the K routed segments and the shared
 *            segment of down_seg[d, :] . hcat[t, seg]
 *
 * The router and the shared expert do not depend on each other, so they run
 * in one launch: the router's dependent add chains overlap the shared
 * expert's weight stream.  The route weight is folded into the hidden row
 * (w_r * silu(g) * u) so the combine of run.c:151-160 becomes a single dot
 * product over the concatenated hidden rows.
 */
#include "router.h"

#define GU_THREADS 256
#define GU_WAVES (GU_THREADS / MM_WAVE)
#define NT_MAX 8

/* Gate/up rows [row0, row0+nrows) against T tokens xs [T, H] (global memory;
 * every wave of a block reads the same activations, so they stay in L1/L2).
 * Writes h[t*hstride + hoff + j] = wt[t] * silu(g) * u. */
__device__ __forceinline__ void gu_rows(const uint16_t *__restrict__ gate, const uint16_t *__restrict__ up,
                        const float *xs, int T, int H, int row0, int nrows,
                        float *__restrict__ h, size_t hstride, int hoff, const float *wt) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = threadIdx.x / MM_WAVE;
    const int nch = H >> 3;
    for (int rr = wave; rr < nrows; rr += GU_WAVES) {
        const int row = row0 + rr;
        const u32x4 *gp = (const u32x4 *)(gate + (size_t)row * H);
        const u32x4 *up_ = (const u32x4 *)(up + (size_t)row * H);
        float ag[NT_MAX], au[NT_MAX];
#pragma unroll
        for (int t = 0; t < NT_MAX; t++) { ag[t] = 0.0f; au[t] = 0.0f; }
#pragma unroll 4
        for (int c = lane; c < nch; c += MM_WAVE) {
            u32x4 gv = __builtin_nontemporal_load(gp + c);
            u32x4 uv = __builtin_nontemporal_load(up_ + c);
#pragma unroll
            for (int t = 0; t < NT_MAX; t++) {
                if (t < T) {
                    const float *xv = xs + (size_t)t * H + 8 * c;
                    ag[t] = dot8_bf16(gv, xv, ag[t]);
                    au[t] = dot8_bf16(uv, xv, au[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT_MAX; t++) {
            if (t < T) {
                float g = wave_sum(ag[t]);
                float u = wave_sum(au[t]);
                if (lane == 0) h[(size_t)t * hstride + hoff + row] = wt[t] * swiglu_f(g, u);
            }
        }
    }
}

/* gu_rows for stage 2, one token: each wave keeps the token's x chunks in
 * registers (loaded with its first weights) and takes its rows GU_RPW at a
 * time with all of their gate and up loads in flight together (gu_rows
 * reads x from global memory again for every row). */
#define GU_RPW 2
#define GU_MAXC 4
template <bool STAGE = false>
__device__ __forceinline__ void gu_rows_x1(const uint16_t *__restrict__ gate,
                                           const uint16_t *__restrict__ up, const float *x, int H,
                                           int row0, int nrows, float *__restrict__ h, int hoff,
                                           float wt) {
    extern __shared__ __attribute__((aligned(16))) float xl[];
    const __attribute__((address_space(3))) float *xl3 = (const __attribute__((address_space(3))) float *)xl;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int nch = H >> 3;
    if (STAGE) {
        /* x staged once per block (1 KB pieces over the waves, before the
         * weights; assembly, waited for by hand below): read per wave it
         * was a third of each wave's bytes.  Bytes past x read as zeros. */
        const rsrc_t xr = raw_rsrc(x, (uint32_t)H * 4u);
        const int np = (H * 4 + 1023) / 1024;
        for (int j = wave; j < np; j += GU_WAVES)
            lds_dma16_buf((uint32_t)(1024 * j + 16 * lane), xr, lds_addr(xl) + 1024u * (uint32_t)j);
    }
    for (int rb = wave * GU_RPW; rb < nrows; rb += GU_WAVES * GU_RPW) {
        float ag[GU_RPW], au[GU_RPW];
#pragma unroll
        for (int q = 0; q < GU_RPW; q++) ag[q] = au[q] = 0.0f;
        /* groups of 64 * GU_MAXC chunks of the row (one for H <= 2048) */
        for (int c0 = 0; c0 < nch; c0 += MM_WAVE * GU_MAXC) {
            u32x4 gv[GU_RPW][GU_MAXC], uv[GU_RPW][GU_MAXC];
            f32x4 xa[GU_MAXC], xb[GU_MAXC];
#pragma unroll
            for (int q = 0; q < GU_RPW; q++) {
                const int row = row0 + min(rb + q, nrows - 1);
                const u32x4 *gp = (const u32x4 *)(gate + (size_t)row * H);
                const u32x4 *upp = (const u32x4 *)(up + (size_t)row * H);
#pragma unroll
                for (int k = 0; k < GU_MAXC; k++) {
                    const int c = c0 + lane + MM_WAVE * k;
                    if (STAGE) {   /* every load issued (clamped), for the count below */
                        gv[q][k] = __builtin_nontemporal_load(gp + min(c, nch - 1));
                        uv[q][k] = __builtin_nontemporal_load(upp + min(c, nch - 1));
                    } else if (c < nch) {
                        gv[q][k] = __builtin_nontemporal_load(gp + c);
                        uv[q][k] = __builtin_nontemporal_load(upp + c);
                    }
                }
            }
            if (STAGE && c0 == 0) {
                /* this wave's pieces have landed once at most the group's
                 * weight loads are outstanding; the barrier waits for the
                 * other waves' (every wave takes exactly one row group) */
                static_assert(2 * GU_RPW * GU_MAXC == 16, "wait count");
                asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
                __syncthreads();
            }
#pragma unroll
            for (int k = 0; k < GU_MAXC; k++) {
                const int c = c0 + lane + MM_WAVE * k;
                if (STAGE) {
                    const int cc = min(c, nch - 1);
                    xa[k] = *(const __attribute__((address_space(3))) f32x4 *)(xl3 + 8 * cc);
                    xb[k] = *(const __attribute__((address_space(3))) f32x4 *)(xl3 + 8 * cc + 4);
                } else if (c < nch) {
                    xa[k] = *(const f32x4 *)(x + 8 * c);
                    xb[k] = *(const f32x4 *)(x + 8 * c + 4);
                }
            }
#pragma unroll
            for (int k = 0; k < GU_MAXC; k++) {
                const int c = c0 + lane + MM_WAVE * k;
                if (c >= nch) continue;
                float xv[8] = {xa[k].x, xa[k].y, xa[k].z, xa[k].w, xb[k].x, xb[k].y, xb[k].z, xb[k].w};
#pragma unroll
                for (int q = 0; q < GU_RPW; q++) {
                    ag[q] = dot8_bf16(gv[q][k], xv, ag[q]);
                    au[q] = dot8_bf16(uv[q][k], xv, au[q]);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < GU_RPW; q++) {
            if (rb + q >= nrows) break;
            const float g = wave_sum(ag[q]);
            const float u = wave_sum(au[q]);
            if (lane == 0) h[hoff + row0 + rb + q] = wt * swiglu_f(g, u);
        }
    }
}

extern "C" __global__ __launch_bounds__(MM_ROUTER_WAVES_LOGITS * MM_WAVE) void mm_router(mm_router_args a) {
    __shared__ float lds[MM_ROUTER_LDS_FLOATS_NW(MM_ROUTER_WAVES_LOGITS)];
    router_block<MM_ROUTER_WAVES_LOGITS>(a, blockIdx.x, lds);
}

/* Router logits for any E (the wide path, E > MM_EMAX_FAST): block (token
 * group tb, expert group eb) of 4 x 64 threads, thread (t, e) owning the
 * logit of token 4 tb + t, expert 64 eb + e: the sum over ascending hidden
 * index of the separately rounded products x[i] * W[e, i] (run.c:29-37),
 * chunks of 64 hidden indices of W (widened to fp32) and of x staged in LDS
 * (W rows padded to 65 floats: the 64 threads of a token read 64 rows at one
 * column conflict-free).  Indices past H contribute +0 (exact). */
#pragma clang fp contract(off)
extern "C" __global__ __launch_bounds__(256) void mm_router_wide(mm_router_args a) {
    __shared__ float wsh[64][65];
    __shared__ float xsh[4][64];
    const int tt = threadIdx.x >> 6, el = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + tt, e = blockIdx.y * 64 + el;
    const int H = a.H;
    float acc = 0.0f;
    for (int i0 = 0; i0 < H; i0 += 64) {
        __syncthreads();
        for (int k = threadIdx.x; k < 64 * 64; k += 256) {
            const int rr = k >> 6, c = k & 63, ee = blockIdx.y * 64 + rr, ii = i0 + c;
            wsh[rr][c] = (ee < a.E && ii < H) ? bf16_f32(a.wg[(size_t)ee * H + ii]) : 0.0f;
        }
        xsh[tt][el] = (t < a.T && i0 + el < H) ? a.x[(size_t)t * H + i0 + el] : 0.0f;
        __syncthreads();
#pragma unroll 8
        for (int c = 0; c < 64; c++) {
            const float pr = xsh[tt][c] * wsh[el][c];
            acc = acc + pr;
        }
    }
    if (t < a.T && e < a.E)
        a.logits_out[(size_t)t * a.E + e] = a.logit_bias ? acc + a.logit_bias[e] : acc;
}
#pragma clang fp contract(on)

/* Router logits, one token per block (E <= 64; router_logits_pc). */
extern "C" __global__ __launch_bounds__(4 * MM_WAVE) void mm_router_pc(mm_router_args a) {
    __shared__ __attribute__((aligned(16))) float lds[RPC_LDS_FLOATS];
    router_block_pc<RPC_HC>(a, lds);
}

/* Router logits only, RPC_EB_SPLIT experts per block: grid (T, ceil(E /
 * RPC_EB_SPLIT)); each logit is the same sequential sum as in mm_router_pc. */
extern "C" __global__ __launch_bounds__(4 * MM_WAVE) void mm_router_pc_split(mm_router_args a) {
    __shared__ __attribute__((aligned(16))) float lds[rpc_shape<RPC_HC, RPC_EB_SPLIT>::LDS_FLOATS];
    const float acc = router_logits_pc<RPC_HC, RPC_EB_SPLIT>(a, lds);
    const int e = (int)blockIdx.y * RPC_EB_SPLIT + (int)threadIdx.x;
    if (threadIdx.x < RPC_EB_SPLIT && e < a.E)
        a.logits_out[(size_t)blockIdx.x * a.E + e] = a.logit_bias ? acc + a.logit_bias[e] : acc;
}

/* Router logits of MM_RSH_EB experts of token tok (expert group eg of
 * ngr), then the token's selection by the block whose logits complete it:
 * every block stores its logits to a.lg and arrives on a.cnt[tok] (a
 * workgroup barrier, then one thread's agent-scope release fence before the
 * atomic); the last one (agent-scope acquire) reads the token's E logits
 * back, clears the counter and selects.  No block waits on another. */
__device__ __forceinline__ void router_split_block(const mm_gu_bf16_args &a, int tok, int eg, int ngr,
                                                   float *lds) {
    __shared__ int s_last;
    const mm_router_args &r = a.r;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const float acc = router_logits_pc<RPC_HC, MM_RSH_EB>(r, lds, tok, eg);
    const int e = eg * MM_RSH_EB + lane;
    if (threadIdx.x < MM_RSH_EB && e < r.E)
        a.lg[(size_t)tok * r.E + e] = r.logit_bias ? acc + r.logit_bias[e] : acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const int last = atomicAdd(a.cnt + tok, 1) == ngr - 1;
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            a.cnt[tok] = 0;   /* every block of the token has arrived */
        }
        s_last = last;
    }
    __syncthreads();
    if (!s_last || threadIdx.x >= MM_WAVE) return;
    /* the other waves have left: their LDS is this wave's scratch */
    const float v = lane < r.E ? a.lg[(size_t)tok * r.E + lane] : 0.0f;
    router_select_one(r, tok, v, lds, router_no_post());
}

/* Small T: the router and the shared expert's gate/up (stage 2's shared
 * parts: row block x, then (token, part) v = t nsh_parts + j) in one launch
 * -- the shared weight stream runs on the CUs the router's add chains leave
 * idle.  Router blocks [0, T ngr): with computed logits ngr = E / MM_RSH_EB
 * blocks per token (router_split_block: a quarter of the 64-expert block's
 * LDS product traffic per block, and LDS for five blocks per CU, so the
 * shared stream is not held to one block per CU); with given logits one
 * block per token selects. */
extern "C" __global__ __launch_bounds__(4 * MM_WAVE) void mm_moe_bf16_router_sh(mm_gu_bf16_args a) {
    __shared__ __attribute__((aligned(16))) float lds[rpc_shape<RPC_HC, MM_RSH_EB>::LDS_FLOATS];
    const int ngr = a.r.logits_in ? 1 : (a.r.E + MM_RSH_EB - 1) / MM_RSH_EB;
    if ((int)blockIdx.x < a.T * ngr) {
        if (!a.r.logits_in) {
            router_split_block(a, (int)blockIdx.x / ngr, (int)blockIdx.x % ngr, ngr, lds);
        } else if (threadIdx.x < MM_WAVE) {   /* given logits: the selection only */
            const int tok = blockIdx.x, lane = threadIdx.x;
            const float v = lane < a.r.E ? a.r.logits_in[(size_t)tok * a.r.E + lane] : 0.0f;
            router_select_one(a.r, tok, v, lds, router_no_post());
        }
        return;
    }
    const int b = blockIdx.x - a.T * ngr;
    const int row0 = (b % a.n_blocks_per_token) * a.rows_per_block;
    const int nrows = min(a.rows_per_block, a.I - row0);
    const int v = b / a.n_blocks_per_token, t = v / a.nsh_parts, j = v % a.nsh_parts;
    const size_t off = (size_t)j * a.I * a.H;
    gu_rows_x1(a.sgate + off, a.sup + off, a.x + (size_t)t * a.H, a.H, row0, nrows,
               a.hcat + (size_t)t * ((size_t)a.K * a.I + a.S), (a.K + j) * a.I, 1.0f);
}

extern "C" __global__ __launch_bounds__(GU_THREADS) void mm_moe_bf16_stage1(mm_gu_bf16_args a) {
    __shared__ float lds[MM_ROUTER_LDS_FLOATS];
    if ((int)blockIdx.x < a.r.n_router_blocks) {
        router_block(a.r, blockIdx.x, lds);
        return;
    }
    const int b = blockIdx.x - a.r.n_router_blocks;
    const int row0 = b * a.rows_per_block;
    const int nrows = min(a.rows_per_block, a.S - row0);
    if (nrows <= 0) return;
    float one[NT_MAX];
#pragma unroll
    for (int t = 0; t < NT_MAX; t++) one[t] = 1.0f;
    gu_rows(a.gate, a.up, a.x, a.T, a.H, row0, nrows, a.hcat, (size_t)a.K * a.I + a.S,
            a.K * a.I, one);
}

/* STAGE: x staged once per block in LDS (dynamic, H * 4 bytes rounded up
 * to 1 KB); needs every wave to take exactly one row group
 * (rows_per_block == GU_WAVES * GU_RPW, a divisor of I). */
template <bool STAGE>
__device__ __forceinline__ void stage2_body(const mm_gu_bf16_args &a) {
    const int route = blockIdx.y;               /* t*K + r */
    const int row0 = blockIdx.x * a.rows_per_block;
    const int nrows = min(a.rows_per_block, a.I - row0);
    if (nrows <= 0) return;
    if (route >= a.T * a.K) {
        /* shared expert of token t as nsh_parts blocks of I rows: part j is
         * rows j I .. j I + I - 1 of the shared gate/up, hidden columns
         * K I + j I .. of hcat (weight 1) */
        const int v = route - a.T * a.K, t = v / a.nsh_parts, j = v % a.nsh_parts;
        const size_t off = (size_t)j * a.I * a.H;
        gu_rows_x1<STAGE>(a.sgate + off, a.sup + off, a.x + (size_t)t * a.H, a.H, row0, nrows,
                          a.hcat + (size_t)t * ((size_t)a.K * a.I + a.S), (a.K + j) * a.I, 1.0f);
        return;
    }
    const int t = route / a.K, r = route % a.K;
    const int e = min(max(a.r.topk_idx[route], 0), a.r.E - 1);
    const float wr = a.r.topk_w[route];
    const size_t off = (size_t)e * a.I * a.H;
    gu_rows_x1<STAGE>(a.gate + off, a.up + off, a.x + (size_t)t * a.H, a.H, row0, nrows,
                      a.hcat + (size_t)t * ((size_t)a.K * a.I + a.S), r * a.I, wr);
}

extern "C" __global__ __launch_bounds__(GU_THREADS) void mm_moe_bf16_stage2(mm_gu_bf16_args a) {
    stage2_body<false>(a);
}
extern "C" __global__ __launch_bounds__(GU_THREADS) void mm_moe_bf16_stage2_lds(mm_gu_bf16_args a) {
    stage2_body<true>(a);
}

/* Down rows: a wave's row d takes, per lane, chunks c = lane, lane + 64, ...
 * of each routed segment in slot order, then of the shared segment -- the
 * accumulation order of the sequential loops.  The loads of up to DN_BATCH
 * chunks are issued before any is used (chunks past a segment's end load
 * chunk 0 of it and are skipped), so a row costs ceil(chunks / DN_BATCH)
 * round trips instead of one per segment. */
#define DN_BATCH 24
/* STAGE: the token's concatenated hidden row is staged once per block into
 * LDS (dynamic: 1 KB pieces by direct loads spread over the waves, issued
 * before the weights; the first batch's weight loads stay in flight across
 * the barrier) and read from there: read per wave from
 * global memory it cost every wave the whole row (45 KB at DeepSeek-V2-Lite
 * shape) from L2, twice the bytes of the wave's weights.  One output row
 * per wave (rows_per_block == GU_WAVES). */
template <bool STAGE>
__device__ __forceinline__ void stage3_body(const mm_down_bf16_args &a) {
    extern __shared__ __attribute__((aligned(16))) float hl[];
    const __attribute__((address_space(3))) float *hl3 = (const __attribute__((address_space(3))) float *)hl;
    const int t = blockIdx.y;
    const size_t hw = (size_t)a.K * a.I + a.S;
    const float *hs = a.hcat + (size_t)t * hw;

    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int d0 = blockIdx.x * a.rows_per_block;
    const int nrows = min(a.rows_per_block, a.H - d0);
    const int nci = a.I >> 3, ncs = a.S >> 3;
    const int cpl = (nci + MM_WAVE - 1) / MM_WAVE;        /* chunk slots per routed segment */
    const int cps = (ncs + MM_WAVE - 1) / MM_WAVE;        /* ... of the shared segment */
    const int nf = a.K * cpl + (a.S > 0 ? cps : 0);
    /* the routed segments' experts, read once (uniform) */
    int er[MM_KMAX];
#pragma unroll
    for (int r = 0; r < MM_KMAX; r++)
        er[r] = r < a.K ? min(max(a.topk_idx[(size_t)t * a.K + r], 0), a.E - 1) : 0;
    if (STAGE) {
        /* assembly loads: the compiler would wait for every load in flight
         * at the first use of a weight register after a direct-to-LDS load
         * it knows of; these are waited for by hand below.  Bytes past the
         * row read as zeros (past the buffer's range: no memory read). */
        const rsrc_t hr = raw_rsrc(hs, (uint32_t)(hw * 4));
        const int np = (int)((hw * 4 + 1023) / 1024);
        for (int j = __builtin_amdgcn_readfirstlane(wave); j < np; j += GU_WAVES)
            lds_dma16_buf((uint32_t)(1024 * j + 16 * lane), hr, lds_addr(hl) + 1024u * (uint32_t)j);
    }
    for (int rr = wave; rr < (STAGE ? GU_WAVES : nrows); rr += GU_WAVES) {
        const int d = d0 + min(rr, nrows - 1);   /* STAGE: a wave past the rows loads row nrows - 1 */
        float acc = 0.0f;
        for (int f0 = 0; f0 < nf; f0 += DN_BATCH) {
            u32x4 wv[DN_BATCH];
            int ho[DN_BATCH];
            bool ok[DN_BATCH];
#pragma unroll
            for (int b = 0; b < DN_BATCH; b++) {
                const int f = min(f0 + b, nf - 1);
                const u32x4 *p;
                int c;
                if (f < a.K * cpl) {
                    const int r = f / cpl;
                    c = lane + MM_WAVE * (f % cpl);
                    ok[b] = f0 + b < nf && c < nci;
                    int e = er[0];
#pragma unroll
                    for (int q = 1; q < MM_KMAX; q++) e = r == q ? er[q] : e;
                    p = (const u32x4 *)(a.down + ((size_t)e * a.H + d) * a.I);
                    ho[b] = r * a.I;
                } else {
                    c = lane + MM_WAVE * (f - a.K * cpl);
                    ok[b] = f0 + b < nf && c < ncs;
                    p = (const u32x4 *)(a.sdown + (size_t)d * a.S);
                    ho[b] = a.K * a.I;
                }
                if (!ok[b]) c = 0;
                wv[b] = __builtin_nontemporal_load(p + c);
                ho[b] += 8 * c;
            }
            if (STAGE && f0 == 0) {
                /* this wave's pieces have landed once at most the batch's
                 * weight loads are outstanding; the barrier waits for the
                 * other waves' pieces */
                static_assert(DN_BATCH == 24, "wait count");
                asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
                __syncthreads();
            }
#pragma unroll
            for (int b = 0; b < DN_BATCH; b++)
                if (ok[b]) acc = STAGE ? dot8_bf16_lds(wv[b], hl3 + ho[b], acc) : dot8_bf16(wv[b], hs + ho[b], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0 && rr < nrows) {
            float *o = a.out + (size_t)t * a.H + d;
            *o = a.accumulate ? *o + acc : acc;
        }
    }
}

extern "C" __global__ __launch_bounds__(GU_THREADS) void mm_moe_bf16_stage3(mm_down_bf16_args a) {
    stage3_body<false>(a);
}
extern "C" __global__ __launch_bounds__(GU_THREADS) void mm_moe_bf16_stage3_lds(mm_down_bf16_args a) {
    stage3_body<true>(a);
}
