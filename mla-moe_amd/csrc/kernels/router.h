/* router.h -- MoE router on gfx950: logits, scores, greedy top-k.
 *
 * Follows src/run.c:124-150 (ffn_compute's router) so that the selected
 * experts are identical to the CPU reference:
 *   - logits: y[e] = sum_i x[i] * W[e, i] accumulated in fp32 in ascending i
 *     with a separate multiply and add (run.c:29-37).  One lane owns one
 *     expert's dependent add chain; the router weight is stored transposed
 *     ([H, E], fp32) so a wave's 64 experts load as one coalesced row.
 *   - softmax (run.c:95-105): max, e^(x - max) (-inf -> 0), sum in ascending
 *     expert order, divide; or sigmoid 1 / (1 + e^-x) (run.c:125-127).
 *   - top-k (run.c:132-143): K passes; each picks the unused expert with the
 *     largest score + bias, lowest index on a tie (the CPU's strict '>').
 *   - weight = raw score; optional normalisation seeded with 1e-20; times
 *     routed_scaling (run.c:144-149).
 * A wave routes TPW tokens; lane l holds experts l, l+64, ... (EJ of them).
 */
#pragma once
#include "common.h"

#define MM_KMAX 16

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

struct router_no_post {
    __device__ void operator()(int, const int *, const float *) const {}
};

/* Routes tokens [wave_id*TPW, wave_id*TPW + TPW) and then calls
 * post(token, idx, w) with the wave-uniform selection of each token. */
template <int EJ, int TPW, class Post = router_no_post>
__device__ __forceinline__ void router_wave(const mm_router_args &a, int wave_id,
                                            Post post = Post()) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int t0 = wave_id * TPW;
    if (t0 >= a.T) return;
    const int E = a.E, H = a.H, K = a.K, T = a.T;

    float lg[TPW][EJ];
    if (a.logits_in) {
#pragma unroll
        for (int t = 0; t < TPW; t++)
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                int e = lane + MM_WAVE * j, tt = min(t0 + t, T - 1);
                lg[t][j] = e < E ? a.logits_in[(size_t)tt * E + e] : 0.0f;
            }
    } else {
#pragma clang fp contract(off)
        const float *xr[TPW];
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            xr[t] = a.x + (size_t)min(t0 + t, T - 1) * H;
#pragma unroll
            for (int j = 0; j < EJ; j++) lg[t][j] = 0.0f;
        }
        const float *wp = a.wgT + lane;
        for (int i0 = 0; i0 < H; i0 += 8) {
            float w[8][EJ];
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int j = 0; j < EJ; j++) {
                    int e = lane + MM_WAVE * j;
                    w[u][j] = (e < E && i0 + u < H) ? wp[(size_t)(i0 + u) * E + MM_WAVE * j] : 0.0f;
                }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (i0 + u < H) {
#pragma unroll
                    for (int t = 0; t < TPW; t++) {
                        float xv = xr[t][i0 + u];
#pragma unroll
                        for (int j = 0; j < EJ; j++) {
                            float prod = xv * w[u][j];
                            lg[t][j] = lg[t][j] + prod;
                        }
                    }
                }
            }
        }
    }

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

        bool used[EJ];
        float sel[EJ];
#pragma unroll
        for (int j = 0; j < EJ; j++) {
            int e = lane + MM_WAVE * j;
            used[j] = e >= E;
            sel[j] = p[j] + (a.bias && e < E ? a.bias[e] : 0.0f);
        }
        int idx[MM_KMAX];
        float w[MM_KMAX];
#pragma unroll
        for (int r = 0; r < MM_KMAX; r++) {
            idx[r] = 0;
            w[r] = 0.0f;
            if (r >= K) continue;
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < EJ; j++)
                if (!used[j] && (bi == 0x7fffffff || sel[j] > bv)) {
                    bv = sel[j];
                    bi = lane + MM_WAVE * j;
                }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                float ov = __shfl_xor(bv, off, MM_WAVE);
                int oi = __shfl_xor(bi, off, MM_WAVE);
                if (oi != 0x7fffffff &&
                    (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
            bi = __builtin_amdgcn_readfirstlane(bi);
            const int owner = bi & (MM_WAVE - 1), jj = bi / MM_WAVE;
            float pw = 0.0f;
#pragma unroll
            for (int j = 0; j < EJ; j++)
                if (j == jj) {
                    pw = readlane_f(p[j], owner);
                    if (lane == owner) used[j] = true;
                }
            idx[r] = bi;
            w[r] = pw;
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

#define MM_ROUTER_TPW 2
#define MM_ROUTER_WAVES 4

/* One block of MM_ROUTER_WAVES waves routes MM_ROUTER_WAVES * TPW tokens. */
template <class Post = router_no_post>
__device__ __forceinline__ void router_block(const mm_router_args &a, int block,
                                             Post post = Post()) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int wid = block * MM_ROUTER_WAVES + wave;
    if (a.E <= 64)
        router_wave<1, MM_ROUTER_TPW>(a, wid, post);
    else if (a.E <= 128)
        router_wave<2, MM_ROUTER_TPW>(a, wid, post);
    else
        router_wave<4, MM_ROUTER_TPW>(a, wid, post);
}
