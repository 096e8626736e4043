/* router.h -- MoE router on gfx950: logits, scores, greedy top-k.
 *
 * Follows src/run.c:124-150 (ffn_compute's router) so that the selected
 * experts are identical to the CPU reference:
 *   - logits: y[e] = sum_i x[i] * W[e, i] accumulated in fp32 in ascending i
 *     with a separate multiply and add (run.c:29-37).  One lane owns one
 *     (token, expert) dependent add chain.  The router weight is kept
 *     transposed ([H, E], fp32); the block streams it through LDS in
 *     double-buffered chunks that all its waves share, and each wave reads
 *     its tokens' x through scalar loads, so the add chains never wait on
 *     HBM.
 *   - softmax (run.c:95-105): max, e^(x - max) (-inf -> 0), sum in ascending
 *     expert order, divide; or sigmoid 1 / (1 + e^-x) (run.c:125-127).
 *   - top-k (run.c:132-143): K passes; each picks the unused expert with the
 *     largest score + bias, lowest index on a tie (the CPU's strict '>'),
 *     computed as each expert's rank in that order.
 *   - weight = raw score; optional normalisation seeded with 1e-20; times
 *     routed_scaling (run.c:144-149).
 * A wave routes TPW tokens; lane l holds experts l, l+64, ... (EJ of them).
 */
#pragma once
#include "common.h"

#define MM_KMAX 16
#define MM_ROUTER_TPW 2
#define MM_ROUTER_WAVES 4
#define MM_ROUTER_THREADS (MM_ROUTER_WAVES * MM_WAVE)
#define MM_ROUTER_CHUNK_FLOATS 8192   /* router-weight chunk: HC rows x E experts */
#define MM_ROUTER_TOKENS (MM_ROUTER_WAVES * MM_ROUTER_TPW)
#define MM_ROUTER_XCHUNK_FLOATS (MM_ROUTER_TOKENS * (MM_ROUTER_CHUNK_FLOATS / MM_WAVE))
#define MM_ROUTER_BUF_FLOATS (MM_ROUTER_CHUNK_FLOATS + MM_ROUTER_XCHUNK_FLOATS)
#define MM_ROUTER_LDS_FLOATS (2 * MM_ROUTER_BUF_FLOATS)

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

struct router_no_post {
    __device__ void operator()(int, const int *, const float *) const {}
};

/* Block-cooperative logits for the block's MM_ROUTER_TOKENS tokens.  Every
 * thread of the block must call this (it synchronises).  Each LDS buffer
 * holds a chunk of HC router-weight rows ([HC][E]) and the same HC columns
 * of the block's token rows ([tokens][HC]); the next chunk is fetched into
 * registers while the current one is consumed.  Inside a chunk the lanes'
 * add chains run on operands already in LDS, read one group of 8 ahead.
 * On return lg[t][j] is the logit of token t0 + t, expert lane + 64 j. */
template <int EJ, int TPW>
__device__ __forceinline__ void router_logits_block(const mm_router_args &a, int tb0, int t0,
                                                    float (&lg)[TPW][EJ], float *lds) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int E = a.E, H = a.H, T = a.T;
    constexpr int HC = MM_ROUTER_CHUNK_FLOATS / (MM_WAVE * EJ);   /* rows per chunk */
    const int CH = HC * E;
    const bool active = t0 < T;
    const int tw = t0 - tb0;                                       /* wave's first row in x chunk */
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int j = 0; j < EJ; j++) lg[t][j] = 0.0f;

    constexpr int PER = MM_ROUTER_CHUNK_FLOATS / 4 / MM_ROUTER_THREADS;
    constexpr int XPER = (MM_ROUTER_TOKENS * HC / 4 + MM_ROUTER_THREADS - 1) / MM_ROUTER_THREADS;
    f32x4 stage[PER], xstage[XPER];
    auto fetch = [&](int c0) {
        const f32x4 *src = (const f32x4 *)(a.wgT + (size_t)c0 * E);
        const int n4 = (min(HC, H - c0) * E) >> 2;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = threadIdx.x + k * MM_ROUTER_THREADS;
            stage[k] = i < n4 ? src[i] : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int k = 0; k < XPER; k++) {
            const int i = threadIdx.x + k * MM_ROUTER_THREADS;   /* float4 index in [tokens][HC] */
            const int row = i / (HC / 4), col = (i % (HC / 4)) * 4;
            const int tok = min(tb0 + row, T - 1);
            xstage[k] = (row < MM_ROUTER_TOKENS && c0 + col < H)
                            ? *(const f32x4 *)(a.x + (size_t)tok * H + c0 + col)
                            : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    auto store = [&](float *buf) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = threadIdx.x + k * MM_ROUTER_THREADS;
            if (i * 4 < CH) *(f32x4 *)(buf + i * 4) = stage[k];
        }
#pragma unroll
        for (int k = 0; k < XPER; k++) {
            const int i = threadIdx.x + k * MM_ROUTER_THREADS;
            if (i < MM_ROUTER_TOKENS * HC / 4)
                *(f32x4 *)(buf + MM_ROUTER_CHUNK_FLOATS + i * 4) = xstage[k];
        }
    };
    fetch(0);
    store(lds);
    __syncthreads();
    int cur = 0;
    for (int c0 = 0; c0 < H; c0 += HC) {
        const bool more = c0 + HC < H;
        if (more) fetch(c0 + HC);
        if (active) {
#pragma clang fp contract(off)
            /* Rows of the chunk past H were fetched as zeros: x*w = +0 and
             * acc + (+0) = acc exactly (acc starts at +0 and never becomes -0
             * under round-to-nearest), so the whole chunk is consumed with a
             * constant trip count and the result is bit-identical. */
            const float *wb = lds + cur * MM_ROUTER_BUF_FLOATS + lane;
            const float *xb = lds + cur * MM_ROUTER_BUF_FLOATS + MM_ROUTER_CHUNK_FLOATS + tw * HC;
            float w[2][8][EJ], xv[2][TPW][8];
            auto load = [&](int s, int i0) {
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int j = 0; j < EJ; j++) w[s][u][j] = wb[(i0 + u) * E + MM_WAVE * j];
#pragma unroll
                for (int t = 0; t < TPW; t++) {
                    const f32x4 lo = *(const f32x4 *)(xb + t * HC + i0);
                    const f32x4 hi = *(const f32x4 *)(xb + t * HC + i0 + 4);
                    xv[s][t][0] = lo.x; xv[s][t][1] = lo.y; xv[s][t][2] = lo.z; xv[s][t][3] = lo.w;
                    xv[s][t][4] = hi.x; xv[s][t][5] = hi.y; xv[s][t][6] = hi.z; xv[s][t][7] = hi.w;
                }
            };
            /* products first (independent), then the ordered adds, so the
             * only serial dependency left is each accumulator's add chain */
            auto compute = [&](int s) {
                float prod[8][TPW][EJ];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int t = 0; t < TPW; t++)
#pragma unroll
                        for (int j = 0; j < EJ; j++) prod[u][t][j] = xv[s][t][u] * w[s][u][j];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int t = 0; t < TPW; t++)
#pragma unroll
                        for (int j = 0; j < EJ; j++) lg[t][j] = lg[t][j] + prod[u][t][j];
            };
            /* two register stages, statically indexed: one group of 8 ahead */
            load(0, 0);
#pragma unroll
            for (int g = 0; g < HC / 8; g++) {
                if (g + 1 < HC / 8) load((g + 1) & 1, (g + 1) * 8);
                compute(g & 1);
            }
        }
        if (more) {
            store(lds + (cur ^ 1) * MM_ROUTER_BUF_FLOATS);
            __syncthreads();
            cur ^= 1;
        }
    }
#pragma unroll
    for (int j = 0; j < EJ; j++)
        if (lane + MM_WAVE * j >= E)
#pragma unroll
            for (int t = 0; t < TPW; t++) lg[t][j] = 0.0f;
}

/* Scores and top-k of one wave's tokens from their logits; calls
 * post(token, idx, w) with the wave-uniform selection of each token. */
template <int EJ, int TPW, class Post>
__device__ __forceinline__ void router_select_wave(const mm_router_args &a, int t0,
                                                   float (&lg)[TPW][EJ], Post post) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int E = a.E, K = a.K, T = a.T;
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int tok = t0 + t;
        if (tok >= T) continue;
        float p[EJ];
        if (a.sigmoid) {
#pragma unroll
            for (int j = 0; j < EJ; j++) p[j] = 1.0f / (1.0f + exp_cr(-lg[t][j]));
        } else {
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < EJ; j++)
                if (lane + MM_WAVE * j < E) mx = fmaxf(mx, lg[t][j]);
            mx = wave_max(mx);
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                float v = lg[t][j];
                p[j] = (lane + MM_WAVE * j < E && v != -INFINITY) ? exp_cr(v - mx) : 0.0f;
            }
            float sum = 0.0f;   /* ascending expert order, as the CPU sums */
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                int n = min(MM_WAVE, E - MM_WAVE * j);
                for (int l = 0; l < n; l++) sum += readlane_f(p[j], l);
            }
#pragma unroll
            for (int j = 0; j < EJ; j++) p[j] = p[j] / sum;
        }
        if (a.probs) {
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                int e = lane + MM_WAVE * j;
                if (e < E) a.probs[(size_t)tok * E + e] = p[j];
            }
        }

        /* Greedy top-k of run.c:132-143 as ranks: the expert chosen in pass
         * r is the one with exactly r others ahead of it in the order
         * (score + bias descending, index ascending), which is the order the
         * CPU's strict '>' scan picks them in.  One readlane sweep computes
         * every expert's rank; no cross-lane shuffles. */
        float sel[EJ];
        int rank[EJ];
#pragma unroll
        for (int j = 0; j < EJ; j++) {
            const int e = lane + MM_WAVE * j;
            sel[j] = p[j] + (a.bias && e < E ? a.bias[e] : 0.0f);
            rank[j] = 0;
        }
#pragma unroll
        for (int jo = 0; jo < EJ; jo++) {
            const int n = min(MM_WAVE, E - MM_WAVE * jo);
            for (int l = 0; l < n; l++) {
                const float so = readlane_f(sel[jo], l);
                const int eo = l + MM_WAVE * jo;
#pragma unroll
                for (int j = 0; j < EJ; j++) {
                    const int e = lane + MM_WAVE * j;
                    rank[j] += (so > sel[j] || (so == sel[j] && eo < e)) ? 1 : 0;
                }
            }
        }
        int idx[MM_KMAX];
        float w[MM_KMAX];
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++) {
            idx[r] = 0;
            w[r] = 0.0f;
            if (r >= K) continue;
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                const unsigned long long m =
                    __ballot(lane + MM_WAVE * j < E && rank[j] == r);
                if (m) {
                    const int l = __ffsll((long long)m) - 1;
                    idx[r] = l + MM_WAVE * j;
                    w[r] = readlane_f(p[j], l);
                }
            }
        }
        if (a.norm_topk) {
            float s = 1e-20f;
#pragma unroll
            for (int r = 0; r < MM_KMAX; r++)
                if (r < K) s += w[r];
#pragma unroll
            for (int r = 0; r < MM_KMAX; r++)
                if (r < K) w[r] /= s;
        }
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++)
            if (r < K) w[r] *= a.scale;
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < MM_KMAX; r++)
                if (r < K) {
                    a.topk_idx[(size_t)tok * K + r] = idx[r];
                    a.topk_w[(size_t)tok * K + r] = w[r];
                }
        }
        post(tok, idx, w);
    }
}

template <int EJ, class Post>
__device__ __forceinline__ void router_block_t(const mm_router_args &a, int block, float *lds,
                                               Post post) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int t0 = (block * MM_ROUTER_WAVES + wave) * MM_ROUTER_TPW;
    float lg[MM_ROUTER_TPW][EJ];
    if (a.logits_in) {
#pragma unroll
        for (int t = 0; t < MM_ROUTER_TPW; t++)
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                const int e = lane + MM_WAVE * j, tt = min(t0 + t, a.T - 1);
                lg[t][j] = e < a.E ? a.logits_in[(size_t)tt * a.E + e] : 0.0f;
            }
    } else {
        router_logits_block<EJ, MM_ROUTER_TPW>(a, block * MM_ROUTER_TOKENS, t0, lg, lds);
        if (a.logit_bias) {
#pragma unroll
            for (int t = 0; t < MM_ROUTER_TPW; t++)
#pragma unroll
                for (int j = 0; j < EJ; j++) {
                    const int e = lane + MM_WAVE * j;
                    if (e < a.E) lg[t][j] += a.logit_bias[e];
                }
        }
    }
    if (a.logits_out) {
#pragma unroll
        for (int t = 0; t < MM_ROUTER_TPW; t++)
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                const int e = lane + MM_WAVE * j;
                if (t0 + t < a.T && e < a.E) a.logits_out[(size_t)(t0 + t) * a.E + e] = lg[t][j];
            }
        return;
    }
    router_select_wave<EJ, MM_ROUTER_TPW>(a, t0, lg, post);
}

/* One block of MM_ROUTER_WAVES waves routes MM_ROUTER_TOKENS tokens.  All
 * threads of the block must call it; `lds` holds MM_ROUTER_LDS_FLOATS. */
template <class Post = router_no_post>
__device__ __forceinline__ void router_block(const mm_router_args &a, int block, float *lds,
                                             Post post = Post()) {
    if (a.E <= 64)
        router_block_t<1>(a, block, lds, post);
    else if (a.E <= 128)
        router_block_t<2>(a, block, lds, post);
    else
        router_block_t<4>(a, block, lds, post);
}
