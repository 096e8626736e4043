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
 *   (prefill sizes use the big-tile GEMM of gemm_i8.hip instead of gu/down)
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
#include "i8_tile.h"

typedef i32x4 v4i;

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i ldg16(const int8_t *p) {
    return __builtin_nontemporal_load((const v4i *)p);
}

/* ---- routing + activation quantisation ----------------------------------- */

/* s = max|x| / 127; q = clamp(rint(x / s), -127, 127), IEEE division and
 * round-half-even, identical to the CPU quantiser.  One wave, n % 4 == 0.
 * Loads are issued QC float4 per lane at a time (one round trip per 256*QC
 * floats); rows of at most 256*QC floats stay in registers between the max
 * and the quantisation. */
#define QC 8
__device__ __forceinline__ void quant_row_load(const float *x, int n, int base, f32x4 (&v)[QC]) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
#pragma unroll
    for (int c = 0; c < QC; c++) {
        const int i = base + (c * MM_WAVE + lane) * 4;
        v[c] = i < n ? *(const f32x4 *)(x + i) : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
}

/* v: the row's first chunk, already loaded by quant_row_load(x, n, 0, v). */
__device__ __forceinline__ void quant_row_wave_pre(const float *x, int n, int8_t *q, float *s,
                                                   f32x4 (&v)[QC]) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    auto load = [&](int base) { quant_row_load(x, n, base, v); };
    float amax = 0.0f;
    for (int base = 0; base < n; base += QC * MM_WAVE * 4) {
        if (base) load(base);
#pragma unroll
        for (int c = 0; c < QC; c++)
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[c].x), fabsf(v[c].y)),
                                     fmaxf(fabsf(v[c].z), fabsf(v[c].w))));
    }
    amax = wave_max(amax);
    const float sc = amax / 127.0f;
    if (lane == 0) *s = sc;
    for (int base = 0; base < n; base += QC * MM_WAVE * 4) {
        if (n > QC * MM_WAVE * 4) load(base);
#pragma unroll
        for (int c = 0; c < QC; c++) {
            const int i = base + (c * MM_WAVE + lane) * 4;
            if (i >= n) continue;
            int b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float r = sc == 0.0f ? 0.0f : fminf(fmaxf(rintf(v[c][j] / sc), -127.0f), 127.0f);
                b[j] = (int)r & 0xff;
            }
            *(uint32_t *)(q + i) = (uint32_t)(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24));
        }
    }
}

__device__ __forceinline__ void quant_row_wave(const float *x, int n, int8_t *q, float *s) {
    f32x4 v[QC];
    quant_row_load(x, n, 0, v);
    quant_row_wave_pre(x, n, q, s, v);
}

/* ---- routing ------------------------------------------------------------------- */

#define RT_TPW 1                             /* tokens per wave */
#define RT_TOKENS (RT_TPW * MM_I8_RT_WAVES)  /* tokens per block */
static_assert(RT_TOKENS == MM_I8_RT_TOKENS, "route block size");

/* Scores, top-k and weights of one token from its logits (lane holds experts
 * lane + 64 j), following run.c:124-149 exactly:
 *   softmax: max, e^(x - max) (-inf -> 0), sum in ascending expert order,
 *   divide; or sigmoid 1 / (1 + e^-x);
 *   top-k: the expert picked in pass r of the CPU's strict '>' scan is the
 *   one with exactly r others ahead of it in the order (score + bias
 *   descending, index ascending), so every lane computes its expert's rank
 *   against all scores (broadcast LDS reads) and ranks < K are the slots;
 *   weight = raw score, optional normalisation seeded with 1e-20 summed in
 *   slot order, times routed_scaling.
 * On return lanes r < K hold slot r's expert (*e_out) and weight (*w_out).
 * `ws` is this wave's LDS scratch of 2 * MM_EMAX_FAST + 2 * MM_KMAX words. */
template <int EJ>
__device__ __forceinline__ void route_token(const mm_router_args &a, int tok, const float (&lg)[EJ],
                                            float *ws, int *e_out, float *w_out) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int E = a.E, K = a.K;
    float *sp = ws, *ss = ws + MM_EMAX_FAST;
    int *slot_e = (int *)(ws + 2 * MM_EMAX_FAST);
    float *slot_w = ws + 2 * MM_EMAX_FAST + MM_KMAX;
    float p[EJ];
    if (a.sigmoid) {
#pragma unroll
        for (int j = 0; j < EJ; j++) p[j] = 1.0f / (1.0f + exp_cr(-lg[j]));
    } else {
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < EJ; j++)
            if (lane + MM_WAVE * j < E) mx = fmaxf(mx, lg[j]);
        mx = wave_max(mx);
#pragma unroll
        for (int j = 0; j < EJ; j++) {
            const int e = lane + MM_WAVE * j;
            p[j] = (e < E && lg[j] != -INFINITY) ? exp_cr(lg[j] - mx) : 0.0f;
            if (e < E) sp[e] = p[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        float sum = 0.0f;   /* ascending expert order, as the CPU sums */
        for (int e = 0; e < E; e += 4) {
            const f32x4 v = *(const f32x4 *)(sp + e);
            sum += v.x;
            if (e + 1 < E) sum += v.y;
            if (e + 2 < E) sum += v.z;
            if (e + 3 < E) sum += v.w;
        }
#pragma unroll
        for (int j = 0; j < EJ; j++) p[j] = p[j] / sum;
    }
    if (a.probs) {
#pragma unroll
        for (int j = 0; j < EJ; j++) {
            const int e = lane + MM_WAVE * j;
            if (e < E) a.probs[(size_t)tok * E + e] = p[j];
        }
    }
    float sel[EJ];
    int rank[EJ];
#pragma unroll
    for (int j = 0; j < EJ; j++) {
        const int e = lane + MM_WAVE * j;
        sel[j] = p[j] + (a.bias && e < E ? a.bias[e] : 0.0f);
        /* NaN: after every number (ties by index), so the ranks stay a
         * permutation and every slot below K gets exactly one expert */
        if (sel[j] != sel[j]) sel[j] = -INFINITY;
        rank[j] = 0;
        if (e < E) ss[e] = sel[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    for (int e0 = 0; e0 < E; e0 += 4) {
        const f32x4 v = *(const f32x4 *)(ss + e0);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int eo = e0 + k;
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                const int e = lane + MM_WAVE * j;
                rank[j] += (eo < E && (v[k] > sel[j] || (v[k] == sel[j] && eo < e))) ? 1 : 0;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < EJ; j++) {
        const int e = lane + MM_WAVE * j;
        if (e < E && rank[j] < K) {
            slot_e[rank[j]] = e;
            slot_w[rank[j]] = p[j];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float norm = 1.0f;
    if (a.norm_topk) {
        float sw = 1e-20f;
        for (int r = 0; r < K; r++) sw += slot_w[r];
        norm = sw;
    }
    const int r = min(lane, K - 1);
    float w = slot_w[r];
    if (a.norm_topk) w /= norm;
    *w_out = w * a.scale;
    *e_out = slot_e[r];
}

/* Routing, per-expert row lists and per-token quantisation of x.  Block =
 * 2 * MM_I8_RT_WAVES waves over RT_TOKENS tokens: wave w < MM_I8_RT_WAVES
 * routes token t0 + w while wave MM_I8_RT_WAVES + w quantises the same
 * token's x row, so the two chains run side by side.  Row-list slots are
 * claimed per block: LDS counters give each route its place among the
 * block's routes to the same expert, then one global atomic per (block,
 * expert) reserves the block's range of the expert's list.  Logits come
 * from logits_in. */
template <int EJ>
__device__ __forceinline__ void i8_route(const mm_i8_route_args &a) {
    static_assert(RT_TPW == 1, "one token per routing wave");
    __shared__ int lcnt[MM_EMAX_FAST];
    __shared__ float wsc[MM_I8_RT_WAVES][2 * MM_EMAX_FAST + 2 * MM_KMAX];
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const bool router = wave < MM_I8_RT_WAVES;
    const mm_router_args &r = a.r;
    const int T = r.T, E = r.E, K = r.K;
    for (int e = threadIdx.x; e < E; e += blockDim.x) lcnt[e] = 0;
    const int tok = blockIdx.x * RT_TOKENS + (router ? wave : wave - MM_I8_RT_WAVES);
    if (!router) {
        /* quantising wave: its x row in one round trip, nothing shared */
        if (tok < T) quant_row_wave(a.x + (size_t)tok * r.H, r.H, a.qx + (size_t)tok * r.H, a.sx + tok);
        if (a.rows) {   /* the block's barriers of the row-list pass */
            __syncthreads();
            __syncthreads();
            __syncthreads();
        }
        return;
    }
    float lg[EJ];
#pragma unroll
    for (int j = 0; j < EJ; j++) {
        const int e = lane + MM_WAVE * j, tt = min(tok, T - 1);
        lg[j] = e < E ? r.logits_in[(size_t)tt * E + e] : -INFINITY;
    }
    int my_e = -1, my_pos = 0;
    if (tok < T) {
        int e;
        float w;
        route_token<EJ>(r, tok, lg, wsc[wave], &e, &w);
        if (lane < K) {
            r.topk_idx[(size_t)tok * K + lane] = e;
            r.topk_w[(size_t)tok * K + lane] = w;
            my_e = e;
        }
    }
    if (a.rows) {   /* per-expert row lists (block-uniform) */
        __syncthreads();   /* lcnt cleared */
        if (my_e >= 0) my_pos = atomicAdd(&lcnt[my_e], 1);
        __syncthreads();
        for (int e = threadIdx.x; e < E; e += MM_I8_RT_WAVES * MM_WAVE) {
            const int n = lcnt[e];
            lcnt[e] = n ? atomicAdd(&a.cnt[e * MM_CNT_STRIDE], n) : 0;   /* now the block's base */
        }
        __syncthreads();
        if (my_e >= 0) {
            const int pos = lcnt[my_e] + my_pos;
            if (pos < T) a.rows[(size_t)my_e * T + pos] = tok * K + lane;
        }
    }
}

extern "C" __global__ __launch_bounds__(2 * MM_I8_RT_WAVES * MM_WAVE) void mm_i8_route(mm_i8_route_args a) {
    if (a.r.E <= 64)
        i8_route<1>(a);
    else if (a.r.E <= 128)
        i8_route<2>(a);
    else
        i8_route<4>(a);
}

/* ---- routing for more than MM_EMAX_FAST experts ------------------------------- */

/* One wave per token, lane l holding experts l + 64 j (j < MM_RW_EJ), for
 * E up to MM_EMAX (run.c:133-134's limit).  Scores as route_token: softmax
 * (max, e^(x - max) with -inf -> 0, the sum in ascending expert order,
 * divide) or sigmoid.  Top-k by K passes of a wave-wide argmax over the
 * unused experts in the order (score + bias descending, index ascending),
 * NaN ranked as -inf: the experts the CPU's strict '>' scan picks
 * (run.c:132-143), pass for pass, and the same permutation as the rank form
 * of the narrower routers.  Weight = raw score, optional normalisation
 * seeded with 1e-20 summed in slot order, times routed_scaling
 * (run.c:144-149).  Then, optionally, the token's int8 quantisation and its
 * places in the per-expert row lists (one atomic per route). */
extern "C" __global__ __launch_bounds__(4 * MM_WAVE) void mm_route_wide(mm_route_wide_args a) {
    __shared__ __attribute__((aligned(16))) float sp[4][MM_EMAX];
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const mm_router_args &r = a.r;
    const int T = r.T, E = r.E, K = r.K;
    const int tok = blockIdx.x * 4 + wave;
    if (tok >= T) return;
    float p[MM_RW_EJ];
#pragma unroll
    for (int j = 0; j < MM_RW_EJ; j++) {
        const int e = lane + MM_WAVE * j;
        p[j] = e < E ? r.logits_in[(size_t)tok * E + e] : -INFINITY;
    }
    if (r.sigmoid) {
#pragma unroll
        for (int j = 0; j < MM_RW_EJ; j++) p[j] = 1.0f / (1.0f + exp_cr(-p[j]));
    } else {
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < MM_RW_EJ; j++)
            if (lane + MM_WAVE * j < E) mx = fmaxf(mx, p[j]);
        mx = wave_max(mx);
        float *ws = sp[wave];
#pragma unroll
        for (int j = 0; j < MM_RW_EJ; j++) {
            const int e = lane + MM_WAVE * j;
            p[j] = (e < E && p[j] != -INFINITY) ? exp_cr(p[j] - mx) : 0.0f;
            if (e < E) ws[e] = p[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        float sum = 0.0f;   /* ascending expert order, as the CPU sums */
        for (int e = 0; e < E; e += 4) {
            const f32x4 v = *(const f32x4 *)(ws + e);
            sum += v.x;
            if (e + 1 < E) sum += v.y;
            if (e + 2 < E) sum += v.z;
            if (e + 3 < E) sum += v.w;
        }
#pragma unroll
        for (int j = 0; j < MM_RW_EJ; j++) p[j] = p[j] / sum;
    }
    if (r.probs) {
#pragma unroll
        for (int j = 0; j < MM_RW_EJ; j++) {
            const int e = lane + MM_WAVE * j;
            if (e < E) r.probs[(size_t)tok * E + e] = p[j];
        }
    }
    float sel[MM_RW_EJ];
#pragma unroll
    for (int j = 0; j < MM_RW_EJ; j++) {
        const int e = lane + MM_WAVE * j;
        sel[j] = e < E ? p[j] + (r.bias ? r.bias[e] : 0.0f) : -INFINITY;
        if (sel[j] != sel[j]) sel[j] = -INFINITY;
    }
    unsigned used = 0;                      /* bit j: expert lane + 64 j taken */
    int my_e = -1;
    float my_w = 0.0f;
    for (int k = 0; k < K; k++) {
        /* this lane's best unused expert (ascending j: the lowest index
         * wins a tie), then the wave's */
        float bv = -INFINITY;
        int be = 0x7fffffff;
        float bp = 0.0f;
#pragma unroll
        for (int j = 0; j < MM_RW_EJ; j++) {
            const int e = lane + MM_WAVE * j;
            if (e < E && !(used & (1u << j)) && (sel[j] > bv || be == 0x7fffffff)) {
                bv = sel[j];
                be = e;
                bp = p[j];
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, MM_WAVE);
            const int oe = __shfl_xor(be, off, MM_WAVE);
            const float op = __shfl_xor(bp, off, MM_WAVE);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
                bp = op;
            }
        }
        if ((be & (MM_WAVE - 1)) == lane) used |= 1u << (be / MM_WAVE);
        if (lane == k) {
            my_e = be;
            my_w = bp;
        }
    }
    /* weights in slot order */
    if (r.norm_topk) {
        float s = 1e-20f;
        for (int k = 0; k < K; k++) s += __shfl(my_w, k, MM_WAVE);
        my_w /= s;
    }
    my_w *= r.scale;
    if (lane < K) {
        r.topk_idx[(size_t)tok * K + lane] = my_e;
        r.topk_w[(size_t)tok * K + lane] = my_w;
        if (a.rows) {
            const int pos = atomicAdd(&a.cnt[my_e * MM_CNT_STRIDE], 1);
            if (pos < T) a.rows[(size_t)my_e * T + pos] = tok * K + lane;
        }
    }
    if (a.qx) quant_row_wave(a.x + (size_t)tok * r.H, r.H, a.qx + (size_t)tok * r.H, a.sx + tok);
}

/* ---- streaming grouped GEMM (decode) ------------------------------------------- */



/* Decode-shaped grouped GEMMs.
 *
 * A block of MM_I8S_W waves serves one 16-row tile of one expert (or of the
 * shared expert).  The tile's A rows (16 x K int8) are staged once into LDS
 * in MFMA operand order, [K step][lane][16 B], and every wave reads them
 * from there.  Each wave streams its own MM_I8S_SEG consecutive 16-column
 * blocks of the expert's weights -- one contiguous run of fragments
 * (gate/up: [gate|up] 2 KB per K step, down: 1 KB per K step) -- and the
 * waves of a block take column units G apart (G = blocks per expert), so
 * that no two waves of a block stream neighbouring memory.
 *
 * Weights stream from HBM with non-temporal loads through a D-deep register
 * ring: the loads of step s + D go out right after step s's MFMAs, across
 * column-block boundaries, so each wave keeps D steps in flight from its
 * first load to its last.  The first D steps' loads are issued before the
 * A tile is staged (they only depend on the block index).  At the end of
 * each column block the epilogue runs on that block's accumulators while
 * the next block's fragments are arriving.
 *
 * Rows past M are staged as zeros; their results are never stored. */
template <bool GU, int D, class Epi>
__device__ __forceinline__ void stream_lds(const int8_t *bp, int KB, int nseg, uint32_t lds_a,
                                           bool prologue_issued, v4i (&bq)[D][GU ? 2 : 1], Epi epi) {
    constexpr int NF = GU ? 2 : 1;
    constexpr int BSTEP = NF * 1024;
    const int total = KB * nseg;
    auto load_b = [&](int slot, int st) {
#pragma unroll
        for (int f = 0; f < NF; f++)
            bq[slot][f] = ldg16(bp + (size_t)min(st, total - 1) * BSTEP + f * 1024);
    };
    if (!prologue_issued) {
#pragma unroll
        for (int d = 0; d < D; d++) load_b(d, d);
    }
    v4i acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    int ck = 0, seg = 0;   /* K step and column block of the next consume */
    auto step = [&](int slot, int st) {
        v4i av = ds_read16(lds_a + ck * 1024);
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(av));
        acc0 = mfma_i8(av, bq[slot][0], acc0);
        if (GU) acc1 = mfma_i8(av, bq[slot][NF - 1], acc1);
        __builtin_amdgcn_sched_barrier(0);
        load_b(slot, st + D);
        __builtin_amdgcn_sched_barrier(0);
        if (++ck == KB) {
            epi(seg, acc0, acc1);
            acc0 = (v4i){0, 0, 0, 0};
            acc1 = (v4i){0, 0, 0, 0};
            ck = 0;
            ++seg;
        }
    };
    /* full ring turns (unconditional body), then the last partial turn */
    int s0 = 0;
    for (; s0 + D <= total; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) step(d, s0 + d);
    }
#pragma unroll
    for (int d = 0; d < D; d++)
        if (s0 + d < total) step(d, s0 + d);
}

/* Stage the 16-row A tile into LDS ([K step][lane][16 B], 1 KB per step):
 * thread t copies the 16-byte pieces of tile row (t % 16) it is responsible
 * for.  arow: that row's K bytes, or nullptr for rows past M (zeros). */
#define STAGE_BATCH 4
__device__ __forceinline__ void stage_a(int8_t *lds, const int8_t *arow, int KB, const int8_t *any) {
    constexpr int NTHR = MM_I8S_W * MM_WAVE;
    const int tid = threadIdx.x;
    const int part = (tid & (MM_WAVE - 1)) >> 4;   /* 16-byte column of the 64-byte step */
    const int n = KB * MM_WAVE;                    /* 16-byte pieces */
    const int8_t *src = arow ? arow : any;         /* rows past M: any valid row, zeroed */
    for (int i0 = 0; i0 < n; i0 += STAGE_BATCH * NTHR) {
        /* all of a batch's loads are issued (unconditionally) before its stores */
        v4i v[STAGE_BATCH];
#pragma unroll
        for (int j = 0; j < STAGE_BATCH; j++) {
            const int i = min(i0 + j * NTHR + tid, n - 1);
            v[j] = *(const v4i *)(src + (i / MM_WAVE) * 64 + part * 16);
        }
#pragma unroll
        for (int j = 0; j < STAGE_BATCH; j++) {
            const int i = i0 + j * NTHR + tid;
            if (i < n) *(v4i *)(lds + (size_t)i * 16) = arow ? v[j] : (v4i){0, 0, 0, 0};
        }
    }
}

__device__ __forceinline__ int tile_row_i(int a_side, int i) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    return __shfl(a_side, 4 * (lane >> 4) + i, MM_WAVE);
}
__device__ __forceinline__ float tile_row_f(float a_side, int i) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    return __shfl(a_side, 4 * (lane >> 4) + i, MM_WAVE);
}

/* Row list of routed expert e, built by the whole block from the routing
 * (topk [R] expert ids): the route ids with topk[rid] == e in ascending
 * order, into LDS `list` (at most cap = T entries: a token picks an expert
 * at most once; hits past cap are dropped, so a malformed routing cannot
 * write past the list).  Returns the count (block-uniform).  No atomics:
 * each wave ballots its hits and places them after the hits of the waves
 * before it. */
__device__ __forceinline__ int expert_rows(const int32_t *topk, int R, int e, int *list, int cap) {
    __shared__ int wsum[MM_I8S_W];
    constexpr int NTHR = MM_I8S_W * MM_WAVE;
    const int tid = threadIdx.x, lane = tid & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / MM_WAVE);
    int total = 0;
    for (int base = 0; base < R; base += NTHR) {
        const int i = base + tid;
        const bool hit = i < R && topk[i] == e;
        const unsigned long long bal = __ballot(hit);
        if (lane == 0) wsum[wave] = __popcll(bal);
        __syncthreads();
        int off = total, all = 0;
#pragma unroll
        for (int w = 0; w < MM_I8S_W; w++) {
            const int c = wsum[w];
            off += w < wave ? c : 0;
            all += c;
        }
        const int pos = off + __popcll(bal & ((1ull << lane) - 1ull));
        if (hit && pos < cap) list[pos] = i;
        __syncthreads();
        total += all;
    }
    return min(total, cap);
}

/* Shared-expert block b of a decode GEMM: column group and row tile, with
 * the MM_I8S_RT blocks of a column group 8 block ids apart (one XCD, so
 * their identical weight reads meet in that XCD's L2). */
__device__ __forceinline__ void shared_block(int b, int *group, int *rt) {
    constexpr int G = MM_I8S_XCD * MM_I8S_RT;
    *group = (b / G) * MM_I8S_XCD + b % MM_I8S_XCD;
    *rt = (b / MM_I8S_XCD) % MM_I8S_RT;
}

/* Column groups (blocks per expert) of a decode GEMM over nbl 16-column
 * blocks: MM_I8S_W * MM_I8S_SEG column blocks per group, or one when the
 * waves split K (ksplit). */
__device__ __forceinline__ int units_per_wave_group(int nbl, int ksplit) {
    const int upg = ksplit ? 1 : MM_I8S_W * MM_I8S_SEG;
    return (nbl + upg - 1) / upg;
}

/* K split (few rows, hence few active experts: too few blocks to stream the
 * weights at full rate otherwise): the block's waves share one column block,
 * wave w taking K steps [w KB / W, (w + 1) KB / W); their int32 partials
 * meet in LDS (exact, so the sum equals the one-wave accumulation) and wave
 * 0 runs the epilogue.  ks_range gives a wave's first step and count. */
__device__ __forceinline__ void ks_range(int KB, int wave, int *k0, int *n) {
    *k0 = wave * KB / MM_I8S_W;
    *n = (wave + 1) * KB / MM_I8S_W - *k0;
}
static_assert(MM_I8S_SEG == 1, "the K split serves one column block per block");

/* Expert of routed block row u: expert u, or with the K split (grid over
 * route slots, T * K of them) the expert of slot u unless an earlier slot
 * names it too (-1: that block has nothing to do). */
template <bool KS>
__device__ __forceinline__ int routed_expert(const mm_i8_gemm_args &a, int u) {
    if (!KS) return u;
    const int e = a.topk[u];
    for (int j = 0; j < u; j++)
        if (a.topk[j] == e) return -1;
    return e;
}

/* Decode-shaped gate/up + SwiGLU.  Blocks [0, n_sh): the shared expert
 * (column group g, row tile rt + MM_I8S_RT * k); the rest: routed expert e,
 * column group g, all of e's rows 16 at a time.  Shared blocks come first so
 * that their work starts early; a routed block of an expert with no rows
 * exits at once.  Dynamic LDS: 16 * H bytes (the A tile), then T ints (the
 * expert's row list). */
template <bool KS>
__device__ __forceinline__ void i8_gu(const mm_i8_gemm_args &a) {
    extern __shared__ __attribute__((aligned(1024))) int8_t lds_a[];
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int KB = a.H / 64;
    const int gs = units_per_wave_group(a.S / 16, KS);
    const int n_sh = a.S ? (gs + MM_I8S_XCD - 1) / MM_I8S_XCD * MM_I8S_XCD * MM_I8S_RT : 0;
    const int b = blockIdx.x;
    const int8_t *bbase;
    const float *sg, *su;
    const int *rows;
    float *hout;
    int32_t *dbg;
    int nbl, G, g, M, m0, mstep, kdiv;
    if (b < n_sh) {
        int rt;
        shared_block(b, &g, &rt);
        if (g >= gs) return;
        nbl = a.S / 16;
        G = gs;
        bbase = a.w.sgu;
        sg = a.w.ss_g;
        su = a.w.ss_u;
        rows = nullptr;
        hout = a.hs;
        dbg = nullptr;
        M = a.T;
        m0 = rt * 16;
        mstep = 16 * MM_I8S_RT;
        kdiv = 1;
    } else {
        nbl = a.I / 16;
        G = units_per_wave_group(nbl, KS);
        const int v = b - n_sh, e = routed_expert<KS>(a, v / G);
        if (e < 0) return;
        g = v % G;
        int *list = (int *)(lds_a + 16 * a.H);
        M = expert_rows(a.topk, a.T * a.K, e, list, a.T);
        if (M == 0) return;
        bbase = a.w.gu + (size_t)e * nbl * 2 * KB * 1024;
        sg = a.w.s_g + (size_t)e * a.I;
        su = a.w.s_u + (size_t)e * a.I;
        rows = list;
        hout = a.h;
        dbg = a.dbg_acc;
        m0 = 0;
        mstep = 16;
        kdiv = a.K;
    }
    if (m0 >= M) return;   /* whole block: a shared row tile past T */
    const int ncols = nbl * 16;
    /* this wave's first column block (K split: the block's one) */
    const int nb0 = KS ? g : (g + G * wave) * MM_I8S_SEG;
    const int nseg = max(0, min(MM_I8S_SEG, nbl - nb0));
    /* per-column scales: lane l holds column l % 16 of block nb0 + l / 16 */
    const int scol = (min(nb0 + min(lane >> 4, MM_I8S_SEG - 1), nbl - 1)) * 16 + (lane & 15);
    const float cg_all = sg[scol], cu_all = su[scol];
    int kw0 = 0, nkw = KB;                          /* this wave's K steps */
    if (KS) ks_range(KB, wave, &kw0, &nkw);
    const int8_t *bp = bbase + (size_t)min(nb0, nbl - 1) * 2 * KB * 1024 + (size_t)kw0 * 2048 + lane * 16;
    v4i *red = (v4i *)(lds_a + 16 * a.H + ((4 * a.T + 15) & ~15));   /* K split: [W][2][64] */
    v4i bq[MM_I8S_DEPTH_GU][2];
    for (; m0 < M; m0 += mstep) {
        /* row of this thread's A piece (tile row lane % 16) */
        /* row lookup first, then the first ring turn (it does not depend on
         * the rows), then the A tile; all unconditional so that the waits
         * stay partial */
        const int m = m0 + (lane & 15);
        const int rl = rows ? rows[min(m, M - 1)] : min(m, M - 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < MM_I8S_DEPTH_GU; d++)
#pragma unroll
            for (int f = 0; f < 2; f++)
                bq[d][f] = ldg16(bp + (size_t)min(d, nkw * max(nseg, 1) - 1) * 2048 + f * 1024);
        __builtin_amdgcn_sched_barrier(0);
        const int rid_a = m < M ? rl : -1;
        const int t = rid_a >= 0 ? rid_a / kdiv : 0;
        const float sx_a = rid_a >= 0 ? a.sa[t] : 0.0f;
        __syncthreads();   /* the previous tile's LDS reads are done */
        stage_a(lds_a, rid_a >= 0 ? a.a + (size_t)t * a.H : nullptr, KB, a.a);
        __syncthreads();
        if (nseg == 0) continue;
        auto finish = [&](int seg, v4i ag, v4i au) {
                const int col = (nb0 + seg) * 16 + (lane & 15);
                const float cg = __shfl(cg_all, seg * 16 + (lane & 15), MM_WAVE);
                const float cu = __shfl(cu_all, seg * 16 + (lane & 15), MM_WAVE);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int rid = tile_row_i(rid_a, i);
                    const float sx = tile_row_f(sx_a, i);
                    const float gv = ((float)ag[i] * sx) * cg;
                    const float uv = ((float)au[i] * sx) * cu;
                    if (rid < 0) continue;
                    hout[(size_t)rid * ncols + col] = silu_mul(gv, uv);
                    if (dbg) {
                        dbg[((size_t)rid * 2) * ncols + col] = ag[i];
                        dbg[((size_t)rid * 2 + 1) * ncols + col] = au[i];
                    }
                }
        };
        if (!KS) {
            stream_lds<true, MM_I8S_DEPTH_GU>(bp, KB, nseg, lds_addr(lds_a) + lane * 16, true, bq,
                                              finish);
            continue;
        }
        stream_lds<true, MM_I8S_DEPTH_GU>(bp, nkw, 1, lds_addr(lds_a) + kw0 * 1024 + lane * 16,
                                          true, bq, [&](int, v4i ag, v4i au) {
                                              red[(2 * wave) * MM_WAVE + lane] = ag;
                                              red[(2 * wave + 1) * MM_WAVE + lane] = au;
                                          });
        __syncthreads();
        if (wave == 0) {
            v4i ag = red[lane], au = red[MM_WAVE + lane];
            for (int w = 1; w < MM_I8S_W; w++) {
                ag += red[(2 * w) * MM_WAVE + lane];
                au += red[(2 * w + 1) * MM_WAVE + lane];
            }
            finish(0, ag, au);
        }
    }
}

/* The gate/up GEMM in two kernels: column groups, and the K split (few
 * tokens): the K split's partial-sum code and registers would otherwise
 * hold every launch to fewer resident blocks (94 against 72 VGPRs: two
 * six-wave blocks per CU instead of three). */
extern "C" __global__ __launch_bounds__(MM_I8S_W * MM_WAVE) void mm_i8_gu(mm_i8_gemm_args a) {
    i8_gu<false>(a);
}
extern "C" __global__ __launch_bounds__(MM_I8S_W * MM_WAVE) void mm_i8_gu_ks(mm_i8_gemm_args a) {
    i8_gu<true>(a);
}

/* Decode-shaped down projection, same block layout (shared blocks over the
 * H/16 column blocks, then the routed experts').  Dynamic LDS:
 * 16 * max(I, S) bytes, then T ints. */
extern "C" __global__ __launch_bounds__(MM_I8S_W * MM_WAVE) void mm_i8_down(mm_i8_gemm_args a) {
    extern __shared__ __attribute__((aligned(1024))) int8_t lds_a[];
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int nbl = a.H / 16;
    const int G = units_per_wave_group(nbl, 0);
    const int n_sh = a.S ? (G + MM_I8S_XCD - 1) / MM_I8S_XCD * MM_I8S_XCD * MM_I8S_RT : 0;
    const int b = blockIdx.x;
    const int8_t *abase, *bbase;
    const float *sa, *sd;
    const int *rows;
    float *yout;
    int32_t *dbg;
    int g, M, m0, mstep, Kd;
    if (b < n_sh) {
        int rt;
        shared_block(b, &g, &rt);
        if (g >= G) return;
        abase = a.a_sh;
        sa = a.sa_sh;
        Kd = a.S;
        bbase = a.w.sdn;
        sd = a.w.ss_d;
        rows = nullptr;
        yout = a.ys;
        dbg = nullptr;
        M = a.T;
        m0 = rt * 16;
        mstep = 16 * MM_I8S_RT;
    } else {
        const int v = b - n_sh, e = v / G;
        g = v % G;
        int *list = (int *)(lds_a + 16 * (a.S > a.I ? a.S : a.I));
        M = expert_rows(a.topk, a.T * a.K, e, list, a.T);
        if (M == 0) return;
        abase = a.a;
        sa = a.sa;
        Kd = a.I;
        bbase = a.w.d + (size_t)e * nbl * (a.I / 64) * 1024;
        sd = a.w.s_d + (size_t)e * a.H;
        rows = list;
        yout = a.y;
        dbg = a.dbg_acc;
        m0 = 0;
        mstep = 16;
    }
    if (m0 >= M) return;
    const int KB = Kd / 64;
    const int nb0 = (g + G * wave) * MM_I8S_SEG;
    const int nseg = max(0, min(MM_I8S_SEG, nbl - nb0));
    const float cd_all = sd[(min(nb0 + min(lane >> 4, MM_I8S_SEG - 1), nbl - 1)) * 16 + (lane & 15)];
    const int8_t *bp = bbase + (size_t)min(nb0, nbl - 1) * KB * 1024 + lane * 16;
    v4i bq[MM_I8S_DEPTH_DOWN][1];
    for (; m0 < M; m0 += mstep) {
        const int m = m0 + (lane & 15);
        const int rl = rows ? rows[min(m, M - 1)] : min(m, M - 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < MM_I8S_DEPTH_DOWN; d++)
            bq[d][0] = ldg16(bp + (size_t)min(d, KB * max(nseg, 1) - 1) * 1024);
        __builtin_amdgcn_sched_barrier(0);
        const int rid_a = m < M ? rl : -1;
        const float sa_a = rid_a >= 0 ? sa[rid_a] : 0.0f;
        __syncthreads();
        stage_a(lds_a, rid_a >= 0 ? abase + (size_t)rid_a * Kd : nullptr, KB, abase);
        __syncthreads();
        if (nseg == 0) continue;
        stream_lds<false, MM_I8S_DEPTH_DOWN>(
            bp, KB, nseg, lds_addr(lds_a) + lane * 16, true, bq,
            [&](int seg, v4i ac, v4i) {
                const int col = (nb0 + seg) * 16 + (lane & 15);
                const float cd = __shfl(cd_all, seg * 16 + (lane & 15), MM_WAVE);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int rid = tile_row_i(rid_a, i);
                    const float sv = tile_row_f(sa_a, i);
                    if (rid < 0) continue;
                    yout[(size_t)rid * a.H + col] = ((float)ac[i] * sv) * cd;
                    if (dbg) dbg[(size_t)rid * a.H + col] = ac[i];
                }
            });
    }
}

/* ---- hidden-row quantisation and combine ------------------------------------- */

/* One wave per row.  Rows of up to QH_MAXF4 * 256 values are held in
 * registers whole (every load issued before the max: one round trip);
 * longer rows take the chunked quantiser.  Same formula either way. */
#define QH_MAXF4 12
__device__ __forceinline__ void quant_row_regs(const float *x, int n, int8_t *q, float *s) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    if ((n / 4 + MM_WAVE - 1) / MM_WAVE > QH_MAXF4) {
        quant_row_wave(x, n, q, s);
        return;
    }
    f32x4 v[QH_MAXF4];
#pragma unroll
    for (int c = 0; c < QH_MAXF4; c++) v[c] = *(const f32x4 *)(x + min((c * MM_WAVE + lane) * 4, n - 4));
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < QH_MAXF4; c++)
        if ((c * MM_WAVE + lane) * 4 < n)
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[c].x), fabsf(v[c].y)), fmaxf(fabsf(v[c].z), fabsf(v[c].w))));
    amax = wave_max(amax);
    const float sc = amax / 127.0f;
    if (lane == 0) *s = sc;
#pragma unroll
    for (int c = 0; c < QH_MAXF4; c++) {
        const int i = (c * MM_WAVE + lane) * 4;
        if (i >= n) continue;
        int b[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float r = sc == 0.0f ? 0.0f : fminf(fmaxf(rintf(v[c][j] / sc), -127.0f), 127.0f);
            b[j] = (int)r & 0xff;
        }
        *(uint32_t *)(q + i) = (uint32_t)(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24));
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_i8_quant_h(mm_i8_quant_rows_args a) {
    const int row = blockIdx.x * (blockDim.x / MM_WAVE) + threadIdx.x / MM_WAVE;
    if (row < a.rows)
        quant_row_regs(a.h + (size_t)row * a.n, a.n, a.q + (size_t)row * a.n, a.s + row);
    else if (row - a.rows < a.rows2) {
        const int r = row - a.rows;
        quant_row_regs(a.h2 + (size_t)r * a.n2, a.n2, a.q2 + (size_t)r * a.n2, a.s2 + r);
    }
}

/* out[t] (=|+=) sum_r w_r * y[t*K + r] (slot order) + ys[t].  grid (T,
 * column parts): block (t, p) takes every gridDim.y-th group of 4 columns
 * from 4 * p; all of a thread's loads are issued before the sums (one round
 * trip per group). */
extern "C" __global__ __launch_bounds__(256) void mm_i8_combine(mm_i8_combine_args a) {
    const int t = blockIdx.x;
    const float *w = a.topk_w + (size_t)t * a.K;
    for (int n = (blockIdx.y * blockDim.x + threadIdx.x) * 4; n < a.H;
         n += gridDim.y * blockDim.x * 4) {
        f32x4 y[MM_KMAX], ys = {0.0f, 0.0f, 0.0f, 0.0f}, o = {0.0f, 0.0f, 0.0f, 0.0f};
        float wr[MM_KMAX];
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++)
            if (r < a.K) {
                y[r] = *(const f32x4 *)(a.y + ((size_t)t * a.K + r) * a.H + n);
                wr[r] = w[r];
            }
        if (a.has_shared) ys = *(const f32x4 *)(a.ys + (size_t)t * a.H + n);
        f32x4 *op = (f32x4 *)(a.out + (size_t)t * a.H + n);
        if (a.accumulate) o = *op;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++)
            if (r < a.K) acc += wr[r] * y[r];
        if (a.has_shared) acc += ys;
        *op = a.accumulate ? o + acc : acc;
    }
    if (a.cnt && t == 0 && blockIdx.y == 0)
        for (int e = threadIdx.x; e < a.E; e += blockDim.x) a.cnt[e * MM_CNT_STRIDE] = 0;
}

/* ---- weight packing ----------------------------------------------------------- */

/* One thread per 16-byte lane slice of a fragment. */
/* mm_i8_combine for one token per block, then the RMSNorm of the combined
 * row (src/run.c:22-27: (x * inv) * w, inv = 1 / sqrt(sum x^2 / n + eps))
 * into xn: the next layer's input norm in the same pass.  The row's values
 * stay in registers; the sum of squares is reduced over the block. */
extern "C" __global__ __launch_bounds__(MM_I8_CN_THREADS) void mm_i8_combine_norm(mm_i8_combine_args a) {
    constexpr int NI = MM_I8_CN_MAXH / (4 * MM_I8_CN_THREADS);
    __shared__ float red[MM_I8_CN_THREADS / MM_WAVE];
    const int t = blockIdx.x;
    const float *w = a.topk_w + (size_t)t * a.K;
    f32x4 res[NI];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int n = (threadIdx.x + MM_I8_CN_THREADS * k) * 4;
        if (n >= a.H) continue;
        f32x4 y[MM_KMAX], ys = {0.0f, 0.0f, 0.0f, 0.0f}, o = {0.0f, 0.0f, 0.0f, 0.0f};
        float wr[MM_KMAX];
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++)
            if (r < a.K) {
                y[r] = *(const f32x4 *)(a.y + ((size_t)t * a.K + r) * a.H + n);
                wr[r] = w[r];
            }
        if (a.has_shared) ys = *(const f32x4 *)(a.ys + (size_t)t * a.H + n);
        f32x4 *op = (f32x4 *)(a.out + (size_t)t * a.H + n);
        if (a.accumulate) o = *op;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++)
            if (r < a.K) acc += wr[r] * y[r];
        if (a.has_shared) acc += ys;
        res[k] = a.accumulate ? o + acc : acc;
        *op = res[k];
#pragma unroll
        for (int u = 0; u < 4; u++) ss += res[k][u] * res[k][u];
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & (MM_WAVE - 1)) == 0) red[threadIdx.x / MM_WAVE] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int v = 0; v < MM_I8_CN_THREADS / MM_WAVE; v++) tot += red[v];
    const float inv = 1.0f / sqrtf(tot / (float)a.H + a.eps);
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int n = (threadIdx.x + MM_I8_CN_THREADS * k) * 4;
        if (n >= a.H) continue;
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 nw = *(const u32x2 *)(a.norm_w + n);   /* 4 bf16 weights */
        f32x4 o;
        o.x = res[k].x * inv * bf16_lo(nw.x);
        o.y = res[k].y * inv * bf16_hi(nw.x);
        o.z = res[k].z * inv * bf16_lo(nw.y);
        o.w = res[k].w * inv * bf16_hi(nw.y);
        *(f32x4 *)(a.xn + (size_t)t * a.H + n) = o;
        if (a.xn_hl) {   /* the split of the stored fp32 values (no contraction) */
            typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
            u16x4 hi, lo;
#pragma unroll
            for (int u = 0; u < 4; u++) {
#pragma clang fp contract(off)
                hi[u] = rne16(o[u]);
                lo[u] = rne16(o[u] - bf16_f32(hi[u]));
            }
            *(u16x4 *)(a.xn_hl + (size_t)t * a.H + n) = hi;
            *(u16x4 *)(a.xn_hl + ((size_t)a.T + t) * a.H + n) = lo;
        }
    }
    if (a.cnt && t == 0)
        for (int e = threadIdx.x; e < a.E; e += blockDim.x) a.cnt[e * MM_CNT_STRIDE] = 0;
}

extern "C" __global__ __launch_bounds__(256) void mm_pack_i8(mm_pack_i8_args a) {
    const int KB = a.K / 64, NB = a.N / 16, NS = a.src1 ? 2 : 1;
    const size_t total = (size_t)NB * NS * KB * 64;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i & 63);
        const size_t f = i >> 6;
        const int which = (int)(f % NS);
        const int kb = (int)((f / NS) % KB);
        const int nb = (int)(f / ((size_t)KB * NS));
        const int8_t *src = which ? a.src1 : a.src0;
        const size_t row = (size_t)nb * 16 + (lane & 15);
        const size_t col = (size_t)kb * 64 + 16 * (lane >> 4);
        *(v4i *)(a.dst + i * 16) = *(const v4i *)(src + row * a.K + col);
    }
}
