/* router.h -- MoE router on gfx950: logits, scores, greedy top-k.
 *
 * Follows src/run.c:124-150 (ffn_compute's router) so that the selected
 * experts are identical to the CPU reference:
 *   - logits: y[e] = sum_i x[i] * W[e, i] accumulated in fp32 in ascending i
 *     with a separate multiply and add (run.c:29-37).  One lane owns one
 *     (token, expert) dependent add chain.  The block streams the bf16
 *     router weight ([E, H], its checkpoint layout) and the tokens' x
 *     through LDS in chunks that all its waves share, prefetched several
 *     chunks ahead, so the add chains rarely wait on memory.
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
#include <type_traits>
#include "common.h"

#define MM_KMAX 16
#define MM_ROUTER_WAVES 4             /* waves per router block of the bf16 stage 1 */
#define MM_ROUTER_CHUNK_FLOATS 8192   /* router-weight chunk: HC rows x E experts */
/* LDS of a router block of nw waves: two buffers, each the weight chunk
 * widened to fp32 with 4 pad floats per expert row (at most 256 rows), then
 * the token columns */
#define MM_ROUTER_LDS_FLOATS_NW(nw) \
    (2 * (MM_ROUTER_CHUNK_FLOATS + 4 * 256 + (nw) * MM_ROUTER_TPW * (MM_ROUTER_CHUNK_FLOATS / MM_WAVE)))
#define MM_ROUTER_LDS_FLOATS MM_ROUTER_LDS_FLOATS_NW(MM_ROUTER_WAVES)

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

struct router_no_post {
    __device__ void operator()(int, const int *, const float *) const {}
};

/* Block-cooperative logits for the block's NW * TPW tokens (NW waves).
 * Every thread of the block must call this (it synchronises).
 *
 * The router weight is used in its checkpoint layout, W [E][H] bf16 (its
 * fp32 values are exact).  It is consumed in chunks of HC hidden indices:
 * the chunk's [E][HC] block of W (16 KB of bf16) goes to LDS widened to
 * fp32, expert-major with rows padded by 16 bytes, so that a lane reads the
 * next 4 weights of its expert with one conflict-free 16-byte read; the same
 * HC columns of the block's token rows ([tokens][HC] fp32) go beside it.  Chunks are loaded into
 * registers RL_PF chunks ahead of their use and written to one of two LDS
 * buffers when their turn comes, so the serial add chains (one add per
 * hidden index, in the reference's ascending order) rarely wait for memory.
 * On return lg[t][j] is the logit of token t0 + t, expert lane + 64 j. */
#define RL_PF 3                                    /* chunks in flight in registers */
#define RL_WBYTES (MM_ROUTER_CHUNK_FLOATS * 2)      /* bf16 weight bytes per chunk */
template <int EJ, int TPW, int NW = MM_ROUTER_WAVES>
__device__ __forceinline__ void router_logits_block(const mm_router_args &a, int tb0, int t0,
                                                    float (&lg)[TPW][EJ], float *lds) {
    constexpr int NTHR = NW * MM_WAVE, NTOK = NW * TPW;
    static_assert(TPW <= 2, "tail handling assumes at most two tokens per wave");
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int E = a.E, H = a.H, T = a.T;
    constexpr int HC = MM_ROUTER_CHUNK_FLOATS / (MM_WAVE * EJ);   /* hidden indices per chunk */
    constexpr int RS = HC + 4;                                    /* padded LDS row, fp32 */
    constexpr int WLDS = MM_WAVE * EJ * RS * 4;                   /* weight bytes in LDS */
    constexpr int XB = NTOK * HC * 4;                 /* x bytes per chunk */
    constexpr int BUF = WLDS + XB;                                /* LDS bytes per buffer */
    static_assert(2 * BUF <= MM_ROUTER_LDS_FLOATS_NW(NW) * 4, "router LDS");
    constexpr int PPE = HC / 8;                                   /* 16-byte pieces per expert row */
    constexpr int WP = RL_WBYTES / 16 / NTHR;        /* weight pieces per thread */
    constexpr int XP = (XB / 16 + NTHR - 1) / NTHR;
    const int nch = (H + HC - 1) / HC;
    const bool active = t0 < T;
    const int tw = t0 - tb0;                                       /* wave's first row in x chunk */
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int j = 0; j < EJ; j++) lg[t][j] = 0.0f;

    /* register slots for chunks c+1 .. c+PF (statically indexed: the chunk
     * loop below is unrolled by PF) */
    u32x4 wr[RL_PF][WP], xr[RL_PF][XP];
    auto fetch = [&](int slot, int c) {
        const int c0 = c * HC;
        /* every load is unconditional (addresses clamped into range, the
         * value zeroed afterwards) so that the waits for a chunk stay
         * partial */
#pragma unroll
        for (int k = 0; k < WP; k++) {
            const int i = threadIdx.x + k * NTHR;   /* piece: expert i / PPE */
            const int e = i / PPE, o = (i % PPE) * 8;
            const bool ok = c < nch && e < E && c0 + o < H;
            const u32x4 v = *(const u32x4 *)(a.wg + (size_t)min(e, E - 1) * H + min(c0 + o, H - 8));
            wr[slot][k] = ok ? v : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < XP; k++) {
            const int i = threadIdx.x + k * NTHR;   /* float4 index in [tokens][HC] */
            const int row = i / (HC / 4), col = (i % (HC / 4)) * 4;
            const int tok = min(tb0 + row, T - 1);
            const bool ok = c < nch && row < NTOK && c0 + col < H;
            const u32x4 v = *(const u32x4 *)(a.x + (size_t)tok * H + min(c0 + col, H - 4));
            xr[slot][k] = ok ? v : (u32x4){0u, 0u, 0u, 0u};
        }
    };
    auto store = [&](int slot, uint8_t *buf) {
#pragma unroll
        for (int k = 0; k < WP; k++) {
            /* the bf16 weights widened to fp32 once here (exact), so the
             * serial compute below spends no instruction on unpacking */
            const int i = threadIdx.x + k * NTHR;
            const int e = i / PPE, o = (i % PPE) * 8;
            const u32x4 d = wr[slot][k];
            const f32x4 lo = {__uint_as_float(d.x << 16), __uint_as_float(d.x & 0xffff0000u),
                              __uint_as_float(d.y << 16), __uint_as_float(d.y & 0xffff0000u)};
            const f32x4 hi = {__uint_as_float(d.z << 16), __uint_as_float(d.z & 0xffff0000u),
                              __uint_as_float(d.w << 16), __uint_as_float(d.w & 0xffff0000u)};
            *(f32x4 *)(buf + ((size_t)e * RS + o) * 4) = lo;
            *(f32x4 *)(buf + ((size_t)e * RS + o + 4) * 4) = hi;
        }
#pragma unroll
        for (int k = 0; k < XP; k++) {
            const int i = threadIdx.x + k * NTHR;
            if (i < XB / 16) *(u32x4 *)(buf + WLDS + (size_t)i * 16) = xr[slot][k];
        }
    };
    auto compute = [&](const uint8_t *buf) {
#pragma clang fp contract(off)
        if (!active) return;
        /* Indices of the chunk past H were fetched as zeros: x*w = +0 and
         * acc + (+0) = acc exactly (acc starts at +0 and never becomes -0
         * under round-to-nearest), so the whole chunk is consumed with a
         * constant trip count and the result is bit-identical. */
        const float *wb = (const float *)buf + (size_t)lane * RS;
        const float *xb = (const float *)(buf + WLDS) + tw * HC;
        f32x4 wq[3][EJ][2];
        float xv[3][TPW][8];
        auto load = [&](int s, int i0) {
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                wq[s][j][0] = *(const f32x4 *)(wb + (size_t)j * MM_WAVE * RS + i0);
                wq[s][j][1] = *(const f32x4 *)(wb + (size_t)j * MM_WAVE * RS + i0 + 4);
            }
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const f32x4 lo = *(const f32x4 *)(xb + t * HC + i0);
                const f32x4 hi = *(const f32x4 *)(xb + t * HC + i0 + 4);
                xv[s][t][0] = lo.x; xv[s][t][1] = lo.y; xv[s][t][2] = lo.z; xv[s][t][3] = lo.w;
                xv[s][t][4] = hi.x; xv[s][t][5] = hi.y; xv[s][t][6] = hi.z; xv[s][t][7] = hi.w;
            }
        };
        /* products first (independent), then the ordered adds, so the only
         * serial dependency left is each accumulator's add chain; NT token
         * chains (the wave's tokens inside T) */
        auto comp = [&](int s, auto nt) {
            constexpr int NT = decltype(nt)::value;
            float prod[8][NT][EJ];
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int j = 0; j < EJ; j++) {
                    const float w = wq[s][j][u >> 2][u & 3];
#pragma unroll
                    for (int t = 0; t < NT; t++) prod[u][t][j] = xv[s][t][u] * w;
                }
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int j = 0; j < EJ; j++) lg[t][j] = lg[t][j] + prod[u][t][j];
        };
        /* LDS reads run two groups of 8 ahead of the adds (an LDS round trip
         * is longer than one group's 8 dependent adds) */
        auto run = [&](auto nt) {
            load(0, 0);
            load(1, 8);
#pragma unroll
            for (int g = 0; g < HC / 8; g++) {
                if (g + 2 < HC / 8) load((g + 2) % 3, (g + 2) * 8);
                comp(g % 3, nt);
            }
        };
        if (TPW == 1 || t0 + TPW <= T)
            run(std::integral_constant<int, TPW>());
        else
            run(std::integral_constant<int, 1>());   /* TPW = 2 at the tail: one chain */
    };
    uint8_t *lbuf = (uint8_t *)lds;
#pragma unroll
    for (int k = 0; k < RL_PF; k++) fetch(k, k);
    /* chunk c: slot c % PF -> LDS buffer c % 2, barrier, refill the slot with
     * chunk c + PF, consume the buffer.  One barrier per chunk suffices: the
     * buffer written for chunk c was last read for chunk c - 2, which every
     * wave finished before the barrier of chunk c - 1. */
    for (int c0 = 0; c0 < nch; c0 += RL_PF) {
#pragma unroll
        for (int k = 0; k < RL_PF; k++) {
            const int c = c0 + k;
            if (c < nch) {   /* block-uniform */
                uint8_t *buf = lbuf + (c & 1) * BUF;
                store(k, buf);
                __syncthreads();
                fetch(k, c + RL_PF);
                compute(buf);
            }
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
            /* a NaN score is never picked by the CPU's strict '>' scan; as
             * -inf it ranks after every number (ties by index), so the
             * ranks stay a permutation and no expert is picked twice */
            if (sel[j] != sel[j]) sel[j] = -INFINITY;
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

template <int EJ, int NW, class Post>
__device__ __forceinline__ void router_block_t(const mm_router_args &a, int block, float *lds,
                                               Post post) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int t0 = (block * NW + wave) * MM_ROUTER_TPW;
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
        router_logits_block<EJ, MM_ROUTER_TPW, NW>(a, block * NW * MM_ROUTER_TPW, t0, lg, lds);
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

/* One block of NW waves routes NW * MM_ROUTER_TPW tokens.  All threads of
 * the block must call it; `lds` holds MM_ROUTER_LDS_FLOATS_NW(NW). */
template <int NW = MM_ROUTER_WAVES, class Post = router_no_post>
__device__ __forceinline__ void router_block(const mm_router_args &a, int block, float *lds,
                                             Post post = Post()) {
    if (a.E <= 64)
        router_block_t<1, NW>(a, block, lds, post);
    else if (a.E <= 128)
        router_block_t<2, NW>(a, block, lds, post);
    else
        router_block_t<4, NW>(a, block, lds, post);
}

/* ---- logits of one token per block, products and sums on separate waves ----
 *
 * For small T the sequential add chains above leave most of the machine idle
 * and each chain's wave spends more than half of its instructions on loads
 * and multiplies.  Here a block of 4 waves serves one token (blockIdx.x)
 * with E <= 64: wave 0 (the chain wave, lane e = expert e) only adds, in
 * ascending hidden order, the products x[i] * W[e, i] that waves 1..3
 * compute (each rounded to fp32 on its own, as the reference's separate
 * multiply and add round them) and leave in LDS.  Chunks of HC hidden
 * indices: in phase k the product waves fill chunks 3 k .. 3 k + 2 while the
 * chain wave consumes those of phase k - 1 (two sets of three buffers, one
 * barrier per phase), the W loads of a product wave RPC_PF phases ahead of
 * its products.  A chunk's [64 experts][HC] block of W is read as
 * whole rows: load j of lane l is expert (64 / LPR) j + l / LPR, hidden
 * offsets 8 (l % LPR) .. + 7, LPR = HC / 8 lanes per row.  Indices past H
 * contribute +0 (exact, as in router_logits_block).  Returns the logit of
 * expert `lane` in wave 0 (0 elsewhere).
 *
 * EB < 64: the block serves experts EB eg .. + EB - 1 of its token (eg:
 * blockIdx.y unless given) only (lane e of the chain wave: expert EB eg + e, lanes >= EB
 * idle), so a token's products -- written to LDS and read back, 2 x 4 B
 * per product -- spread over 64 / EB CUs: with all 64 experts in one block
 * that LDS traffic (1 MB per token), not the add chains, set the pace. */
#define RPC_NPROD 3
#ifndef RPC_PF
#define RPC_PF 2            /* phases of W loads in flight ahead of the one computed */
#endif
template <int HC, int EB = MM_WAVE>
struct rpc_shape {
    static constexpr int RS = HC + 4;                   /* padded product row (floats) */
    static constexpr int BUF = EB * RS;                 /* floats per chunk buffer */
    static constexpr int LDS_FLOATS = 2 * RPC_NPROD * (BUF + HC);
    static constexpr int LPR = HC / 8;                  /* lanes per W row */
    static constexpr int NLD = EB / (MM_WAVE / LPR);    /* W loads per lane per chunk */
};
#define RPC_HC 64                                       /* chunk of the standalone kernel */
#define RPC_LDS_FLOATS (rpc_shape<RPC_HC>::LDS_FLOATS)
#define RPC_EB_SPLIT MM_ROUTER_PC_EB                    /* experts per block, logits only */

template <int HC, int EB = MM_WAVE>
__device__ __forceinline__ float router_logits_pc(const mm_router_args &a, float *lds,
                                                  int tok = blockIdx.x, int eg = blockIdx.y) {
    using S = rpc_shape<HC, EB>;
    static_assert(HC % 8 == 0 && MM_WAVE % S::LPR == 0, "chunk rows of whole 16-byte pieces");
    static_assert(EB <= MM_WAVE && EB % (MM_WAVE / S::LPR) == 0, "whole loads of expert rows");
    const int e0 = EB < MM_WAVE ? eg * EB : 0;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int H = a.H, E = a.E;
    const int nch = (H + HC - 1) / HC;
    const int nph = (nch + RPC_NPROD - 1) / RPC_NPROD;
    float *prod = lds;                                   /* [6][EB][RS] */
    float *xs = lds + 2 * RPC_NPROD * S::BUF;            /* [6][HC] */
    const float *xrow = a.x + (size_t)tok * H;
    float acc = 0.0f;
    if (wave > 0) {
        /* product wave p fills chunk 3 k + p of every phase k; the loads of
         * the chunks of the next RPC_PF phases are in flight meanwhile */
        constexpr int RPL = MM_WAVE / S::LPR;            /* rows per load */
        constexpr int NSL = RPC_PF + 1;                  /* register slots */
        const int p = wave - 1;
        const int o = 8 * (lane % S::LPR);
        u32x4 wr[NSL][S::NLD];
        float xv[NSL];
        /* loads unconditional (addresses clamped into the matrix; chunks
         * past the end re-read the last), the values past H or past the
         * last chunk zeroed where they are used: a load under a condition
         * becomes a branch, and the compiler then drains every outstanding
         * load before the next use instead of waiting for the one it needs */
        auto fetch = [&](int slot, int c) {
            const int cc = min(c, nch - 1);
            const int i = min(cc * HC + o, H - 8);
#pragma unroll
            for (int j = 0; j < S::NLD; j++) {
                const int e = min(e0 + RPL * j + lane / S::LPR, E - 1);
                wr[slot][j] = *(const u32x4 *)(a.wg + (size_t)e * H + i);
            }
            xv[slot] = xrow[min(cc * HC + min(lane, HC - 1), H - 1)];
        };
#pragma unroll
        for (int d = 0; d < RPC_PF; d++) fetch(d, RPC_NPROD * d + p);
        /* phase k uses slot k % NSL and refills slot (k + RPC_PF) % NSL;
         * whole turns of NSL phases first, then the last partial turn */
        auto phase = [&](int d, int k) {
#pragma clang fp contract(off)
            const int b = (k & 1) * RPC_NPROD + p;
            const int c = RPC_NPROD * k + p;             /* this phase's chunk */
            float *xb = xs + b * HC;
            /* this chunk's x to LDS (read back by this wave only: its LDS
             * accesses complete in order); zeros past H or past the last
             * chunk, and their weights zeroed too */
            if (lane < HC) xb[lane] = (c < nch && c * HC + lane < H) ? xv[d] : 0.0f;
            const bool wok = c < nch && c * HC + o < H;
            fetch((d + RPC_PF) % NSL, RPC_NPROD * (k + RPC_PF) + p);
            const f32x4 x0 = *(const f32x4 *)(xb + o);
            const f32x4 x1 = *(const f32x4 *)(xb + o + 4);
            float *pb = prod + b * S::BUF + o;
#pragma unroll
            for (int j = 0; j < S::NLD; j++) {
                const u32x4 w = wok ? wr[d][j] : (u32x4){0u, 0u, 0u, 0u};
                f32x4 lo, hi;
                lo.x = x0.x * __uint_as_float(w.x << 16);
                lo.y = x0.y * __uint_as_float(w.x & 0xffff0000u);
                lo.z = x0.z * __uint_as_float(w.y << 16);
                lo.w = x0.w * __uint_as_float(w.y & 0xffff0000u);
                hi.x = x1.x * __uint_as_float(w.z << 16);
                hi.y = x1.y * __uint_as_float(w.z & 0xffff0000u);
                hi.z = x1.z * __uint_as_float(w.w << 16);
                hi.w = x1.w * __uint_as_float(w.w & 0xffff0000u);
                float *row = pb + (size_t)(RPL * j + lane / S::LPR) * S::RS;
                *(f32x4 *)row = lo;
                *(f32x4 *)(row + 4) = hi;
            }
        };
        int k0 = 0;
        for (; k0 + NSL <= nph; k0 += NSL) {
#pragma unroll
            for (int d = 0; d < NSL; d++) {
                phase(d, k0 + d);
                __syncthreads();
            }
        }
        /* phases k0 .. nph: the last product phases, then the barrier of
         * the chain wave's final consumption (nph + 1 barriers in all) */
#pragma unroll
        for (int d = 0; d < NSL; d++) {
            const int k = k0 + d;
            if (k > nph) break;
            if (k < nph) phase(d, k);
            __syncthreads();
        }
    } else {
        for (int k = 0; k <= nph; k++) {
            if (k > 0) {
#pragma clang fp contract(off)
                const int kp = k - 1;
#pragma unroll
                for (int j = 0; j < RPC_NPROD; j++) {
                    if (RPC_NPROD * kp + j >= nch) break;
                    const float *pb =
                        prod + ((kp & 1) * RPC_NPROD + j) * S::BUF + (size_t)min(lane, EB - 1) * S::RS;
                    f32x4 v[HC / 4];
#pragma unroll
                    for (int q = 0; q < HC / 4; q++) v[q] = *(const f32x4 *)(pb + 4 * q);
#pragma unroll
                    for (int q = 0; q < HC / 4; q++) {
                        acc = acc + v[q].x;
                        acc = acc + v[q].y;
                        acc = acc + v[q].z;
                        acc = acc + v[q].w;
                    }
                }
            }
            __syncthreads();
        }
    }
    return acc;
}

/* Scores and top-k of one token (E <= 64, lane e = expert e), the result
 * of router_select_wave<1, 1> computed with LDS broadcasts instead of 64
 * readlane rounds: the softmax sum in ascending expert order and each
 * expert's rank read the 64 values from `ws` (this wave's LDS scratch of
 * 64 floats; nothing else may use it meanwhile).  Calls post(tok, idx, w). */
template <class Post>
__device__ __forceinline__ void router_select_one(const mm_router_args &a, int tok, float v,
                                                  float *ws, Post post) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int E = a.E, K = a.K;
    const bool ok = lane < E;
    /* the sequential sum of ws[0 .. E - 1] (every lane) */
    auto seq_sum = [&]() {
        float sum = 0.0f;
        for (int l0 = 0; l0 < E; l0 += 4) {
            const f32x4 q = *(const f32x4 *)(ws + l0);
            sum += q.x;
            if (l0 + 1 < E) sum += q.y;
            if (l0 + 2 < E) sum += q.z;
            if (l0 + 3 < E) sum += q.w;
        }
        return sum;
    };
    float p;
    if (a.sigmoid) {
        p = 1.0f / (1.0f + exp_cr(-v));
    } else {
        const float mx = wave_max(ok ? v : -INFINITY);
        p = (ok && v != -INFINITY) ? exp_cr(v - mx) : 0.0f;
        ws[lane] = p;
        p = p / seq_sum();
    }
    if (a.probs && ok) a.probs[(size_t)tok * E + lane] = p;
    /* rank of this expert in the order (score + bias descending, index
     * ascending): the pass of the CPU's strict '>' scan that picks it */
    float sel = p + (a.bias && ok ? a.bias[lane] : 0.0f);
    if (sel != sel) sel = -INFINITY;   /* NaN: after every number, ranks stay a permutation */
    ws[lane] = sel;
    int rank = 0;
    for (int l0 = 0; l0 < E; l0 += 4) {
        const f32x4 q = *(const f32x4 *)(ws + l0);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int l = l0 + u;
            const float so = q[u];
            rank += (l < E && (so > sel || (so == sel && l < lane))) ? 1 : 0;
        }
    }
    int idx[MM_KMAX];
    float w[MM_KMAX];
#pragma unroll
    for (int r = 0; r < MM_KMAX; r++) {
        idx[r] = 0;
        w[r] = 0.0f;
        if (r >= K) continue;
        const unsigned long long m = __ballot(ok && rank == r);
        if (m) {
            const int l = __ffsll((long long)m) - 1;
            idx[r] = l;
            w[r] = readlane_f(p, l);
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

/* Router of one token per block with the logits of router_logits_pc (the
 * selection by the chain wave, as router_block_t does it for its tokens).
 * Every thread of the block must call it; lds holds
 * rpc_shape<HC>::LDS_FLOATS floats. */
template <int HC, class Post = router_no_post>
__device__ __forceinline__ void router_block_pc(const mm_router_args &a, float *lds,
                                                Post post = Post()) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    float lg[1][1];
    if (a.logits_in) {       /* given logits: the selection only */
        if (threadIdx.x >= MM_WAVE) return;
        lg[0][0] = lane < a.E ? a.logits_in[(size_t)blockIdx.x * a.E + lane] : 0.0f;
        router_select_one(a, (int)blockIdx.x, lg[0][0], lds, post);
        return;
    }
    const float acc = router_logits_pc<HC>(a, lds);
    if (threadIdx.x >= MM_WAVE) return;
    lg[0][0] = lane < a.E ? acc : 0.0f;
    if (a.logit_bias && lane < a.E) lg[0][0] += a.logit_bias[lane];
    if (a.logits_out) {
        if (lane < a.E) a.logits_out[(size_t)blockIdx.x * a.E + lane] = lg[0][0];
        return;
    }
    /* the other waves have left after the last barrier of the logits:
     * their LDS is this wave's scratch */
    router_select_one(a, (int)blockIdx.x, lg[0][0], lds, post);
}

