/* kernel_params.h -- argument blocks shared by the C11 host code and the HIP
 * kernels.  Each kernel takes exactly one of these structs by value, so the
 * host launches it with hipModuleLaunchKernel(kernelParams = {&params}).
 * Only plain C types appear here so that both compilers agree on the layout. */
#ifndef MLAMOE_KERNEL_PARAMS_H
#define MLAMOE_KERNEL_PARAMS_H

#include <stdint.h>

/* Router: logits (sequential fp32 dot products in the reference's order, or
 * caller-supplied), softmax/sigmoid, greedy top-k with the lowest-index tie
 * rule, optional normalisation and scaling. */
typedef struct {
    const float *x;          /* [T, H] activations (unused when logits_in != 0) */
    const float *wgT;        /* [H, E] router weight, fp32, transposed */
    const float *logits_in;  /* [T, E] or 0 */
    const float *bias;       /* [E] or 0 */
    float *probs;            /* [T, E] scores out, or 0 */
    int32_t *topk_idx;       /* [T, K] */
    float *topk_w;           /* [T, K] */
    int T, H, E, K;
    int sigmoid, norm_topk;
    float scale;
    int n_router_blocks;     /* blocks [0, n_router_blocks) run the router */
} mm_router_args;

/* bf16 GEMV MoE, stage 1 = router + shared-expert gate/up (+SwiGLU).
 * Stage 2 = routed gate/up.  Both write hidden rows pre-multiplied by the
 * route weight (1 for shared) into hcat [T, K*I + S]. */
typedef struct {
    mm_router_args r;
    const float *x;          /* [T, H] */
    const uint16_t *gate;    /* stage 1: shared gate [S, H]; stage 2: routed [E, I, H] */
    const uint16_t *up;
    float *hcat;             /* [T, K*I + S] */
    int T, H, I, S, K;
    int rows_per_block;      /* gate/up row pairs per block */
    int n_blocks_per_token;  /* stage 2: row blocks per route */
} mm_gu_bf16_args;

/* bf16 GEMV MoE, stage 3: out[t] (=|+=) sum over routed slots and the shared
 * expert of down_seg[d, :] . hcat[t, seg] */
typedef struct {
    const float *hcat;       /* [T, K*I + S] */
    const uint16_t *down;    /* routed [E, H, I] */
    const uint16_t *sdown;   /* shared [H, S] */
    const int32_t *topk_idx; /* [T, K] */
    float *out;              /* [T, H] */
    int T, H, I, S, K, E;
    int accumulate;
    int rows_per_block;
} mm_down_bf16_args;

/* Synthetic data and format conversion utilities. */
typedef struct {
    void *dst;
    uint64_t n;
    uint64_t seed;
    float std;
    int kind;                /* 0: bf16 normal, 1: fp32 normal, 2: fp32 uniform [0,1) */
} mm_fill_args;

typedef struct {
    const uint16_t *w;       /* [rows, K] bf16 */
    int8_t *q;               /* [rows, K] */
    float *s;                /* [rows] */
    int rows, K;
} mm_quant_w_args;

typedef struct {
    const uint16_t *src;     /* [E, H] bf16 */
    float *dst;              /* [H, E] fp32 */
    int E, H;
} mm_transpose_gate_args;

#endif
