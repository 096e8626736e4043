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
#ifndef MM_ROUTER_TPW
#define MM_ROUTER_TPW 1           /* router: tokens per wave */
#endif
/* waves (tokens) per block of mm_router, the logits of larger T: every block
 * streams the whole gate weight through LDS, so 8 tokens per block take half
 * the weight traffic of 4 at the same two waves per SIMD (measured at config
 * 3: 33 against 39 us; 16 per block leave half the CUs idle, 50 us) */
#define MM_ROUTER_WAVES_LOGITS 8

/* Logits-only router with one token per block (mm_router_pc): used for
 * E <= 64, H % 8 == 0 and T up to this many tokens. */
#define MM_ROUTER_PC_TMAX 256
#ifndef MM_ROUTER_PC_EB
#define MM_ROUTER_PC_EB 16        /* experts per block of the logits-only product/chain router */
#endif

typedef struct {
    const float *x;          /* [T, H] activations (unused when logits_in != 0) */
    const uint16_t *wg;      /* [E, H] router weight, bf16 (checkpoint layout) */
    const float *logits_in;  /* [T, E] or 0 */
    const float *bias;       /* [E] selection bias (GLM e_score correction) or 0 */
    const float *logit_bias; /* [E] added to computed logits (logits-only mode) or 0 */
    float *logits_out;       /* [T, E]: write the logits and stop, or 0 */
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
    /* stage 2 may also take the shared expert (then no stage 1 gate/up):
     * grid rows T*K .. T*K + T*nsh_parts - 1, S = nsh_parts * I */
    const uint16_t *sgate, *sup;
    int nsh_parts;
    /* mm_moe_bf16_router_sh with computed logits: MM_RSH_EB experts per
     * router block, the logits through lg [T, E]; the block that completes
     * a token's count in cnt [T] (zero on entry, cleared by that block)
     * selects its experts */
    float *lg;
    int32_t *cnt;
} mm_gu_bf16_args;
#define MM_RSH_EB 16

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

/* dst[i] = 0 for i < n 32-bit words. */
typedef struct {
    uint32_t *dst;
    uint64_t n;
} mm_zero32_args;

/* Embedding rows of B tokens: x[b, :] = embed[tokens[b], :] in fp32. */
typedef struct {
    const uint16_t *embed;   /* [vocab, H] bf16 */
    const int32_t *tokens;   /* [B] */
    float *x;                /* [B, H] */
    int H, vocab;
} mm_embed_args;

/* dst[j, :] = src[idx[j], :] for n rows of H floats. */
typedef struct {
    const float *src;
    const int32_t *idx;
    float *dst;
    int n, H;
} mm_gather_rows_args;

/* h = silu(g) * u elementwise over n values (the dense SwiGLU MLP). */
typedef struct {
    const float *g, *u;
    float *h;
    size_t n;
} mm_swiglu_args;

/* y = bf16(x), round to nearest even, over n values (the host-pointer
 * absorbed-decode entry point's fp32 cache rows). */
typedef struct {
    const float *x;
    uint16_t *y;
    uint64_t n;
} mm_f32_bf16_args;

/* ---- int8 MoE path ------------------------------------------------------ */

/* Per-layer int8 weights in MFMA fragment order.  A "fragment" is the
 * 16-row x 64-column int8 block one v_mfma_i32_16x16x64_i8 consumes as its
 * B operand: 1 KB, lane l holding row (l % 16), columns 16*(l/16) .. +15.
 *   gu   [E][I/16][H/64][2] fragments: for each 16-row block and K step, the
 *        gate fragment then the up fragment (the SwiGLU pair), so that one
 *        column block's whole K range is one contiguous 2*H*16-byte stream
 *   d    [E][H/16][I/64] fragments of the down projection
 *   sgu  [S/16][H/64][2], sdn [H/16][S/64] for the shared expert */
typedef struct {
    const int8_t *gu, *d, *sgu, *sdn;
    const float *s_g, *s_u, *s_d;       /* [E, I], [E, I], [E, H] */
    const float *ss_g, *ss_u, *ss_d;    /* [S], [S], [H] */
} mm_i8_weights;

/* Routing + per-token activation quantisation (logits given). */
#define MM_I8_RT_WAVES 4
#define MM_I8_RT_TOKENS 4        /* tokens per block: one per wave */
#define MM_EMAX_FAST 256         /* experts served by the routers below (E / 64 per lane) */
/* The per-expert row counters of the tiled path sit one per 128-byte line
 * (counter e at cnt[e * MM_CNT_STRIDE]): every routing block adds to the
 * counters of the experts it routes to, and counters sharing a line
 * serialise those atomics. */
#define MM_CNT_STRIDE 32
#define MM_EMAX 1024             /* experts served at all (run.c:133-134's limit): above
                                    MM_EMAX_FAST by the wide routers (mm_router_wide,
                                    mm_route_wide) */
typedef struct {
    mm_router_args r;
    int32_t *cnt;            /* [E * MM_CNT_STRIDE] rows per expert (zero on entry), or 0 */
    int32_t *rows;           /* [E, T] route ids (t*K + r) per expert, or 0 (no lists) */
    const float *x;          /* [T, H] */
    int8_t *qx;              /* [T, H] */
    float *sx;               /* [T] */
} mm_i8_route_args;

/* Grouped int8 GEMM over experts 0..E-1 (routed) and the shared expert. */
typedef struct {
    mm_i8_weights w;
    const int32_t *cnt;      /* [E * MM_CNT_STRIDE] (tiled path) */
    const int32_t *rows;     /* [E, T] (tiled path) */
    const int32_t *topk;     /* [T, K] expert ids (decode path builds its row lists) */
    const int8_t *a;         /* gate/up: qx [T, H];  down: qh [T*K, I] */
    const float *sa;         /* gate/up: sx [T];     down: sh [T*K] */
    const int8_t *a_sh;      /* down: shared qhs [T, S] */
    const float *sa_sh;      /* down: shared shs [T] */
    float *h;                /* gate/up out: routed [T*K, I] */
    float *hs;               /* gate/up out: shared [T, S] */
    float *y;                /* down out: routed [T*K, H] */
    float *ys;               /* down out: shared [T, H] */
    int32_t *dbg_acc;        /* debug: raw accumulators, gate/up [T*K, 2, I], down [T*K, H], or 0 */
    int T, H, I, S, E, K;
    int ksplit;              /* gate/up: 1 = a block's waves split K for one column block (few rows) */
} mm_i8_gemm_args;
/* The decode gate/up GEMM splits K over a block's waves up to this many tokens. */
#define MM_I8_KSPLIT_TMAX 4

/* Per-row quantisation of the SwiGLU output. */
typedef struct {
    const float *h;          /* [rows, n] */
    int8_t *q;
    float *s;
    int rows, n;
    const float *h2;         /* second region (shared expert) or 0 */
    int8_t *q2;
    float *s2;
    int rows2, n2;
} mm_i8_quant_rows_args;

/* out[t] (=|+=) sum_r w[t,r] * y[t*K + r] + ys[t]; clears the E counters
 * cnt[e * MM_CNT_STRIDE] when cnt is given (the tiled path's per-expert
 * counters, read by then). */
typedef struct {
    const float *y, *ys;
    const float *topk_w;
    float *out;
    int32_t *cnt;
    int T, H, K, E;
    int accumulate;
    int has_shared;
    /* mm_i8_combine_norm: then xn[t] = rmsnorm(out[t], norm_w) (eps) */
    const uint16_t *norm_w;
    float *xn;
    float eps;
    uint16_t *xn_hl;         /* or 0: xn also as bf16 hi/lo planes [2, T, H] */
} mm_i8_combine_args;
#define MM_I8_CN_THREADS 512      /* mm_i8_combine_norm: one block per token */
#define MM_I8_CN_MAXH 4096

/* Pack a row-major int8 [N, K] matrix into 16x64 fragments, optionally
 * interleaving two matrices per 16-row block (gate/up). */
typedef struct {
    const int8_t *src0, *src1;   /* src1 = 0: no interleave */
    int8_t *dst;
    int N, K;
} mm_pack_i8_args;

/* Decode-shaped GEMMs: a block of MM_I8S_W waves serves one 16-row tile of
 * one expert (A tile staged once in LDS); each wave streams MM_I8S_SEG
 * consecutive 16-column blocks of the expert's weights (one contiguous run of
 * fragments), the waves of a block taking column units G apart, G being the
 * number of blocks per expert.  The shared expert's row tiles go to
 * MM_I8S_RT blocks 8 block ids apart (one XCD), so that their identical
 * weight reads meet in that XCD's L2. */
/* Swept on MI355X at the config-4 shape (B = 64, DeepSeek-V2-Lite layer):
 * 6 waves with rings of 3 (gate/up, 2 KB per step) and 6 (down, 1 KB) steps
 * beat 4, 5, 7, 8, 12 and 16 waves and deeper rings by 3-6% per step. */
#ifndef MM_I8S_W
#define MM_I8S_W 6                 /* waves per block */
#endif
#ifndef MM_I8S_SEG
#define MM_I8S_SEG 1               /* column blocks per wave (<= 4) */
#endif
#ifndef MM_I8S_DEPTH_GU
#define MM_I8S_DEPTH_GU 3          /* K steps of weight fragments in flight per wave */
#define MM_I8S_DEPTH_DOWN 6
#endif
#define MM_I8S_RT 4                /* row-tile blocks per shared-expert column group */
#define MM_I8S_XCD 8               /* blocks are dealt to XCDs round robin */

/* Grouped int8 GEMM for prefill sizes (mm_i8_gemm_bt, gemm_i8.hip): block
 * tiles of 128 rows x 16 B fragments over the routed experts' row lists (or
 * all T rows for the shared expert), a persistent grid of two blocks per CU. */
#define MM_I8B_BM 128
#define MM_I8B_FR 16
#define MM_I8B_GRID 512          /* persistent grid: 2 blocks on each of 256 CUs */
/* The tiled GEMMs address activation rows by 32-bit byte offsets from the
 * matrix base: matrices below MM_I8_TILED_A_MAX bytes (the host splits
 * longer calls); offsets from it up read nothing (padding rows, plus less
 * than 2^16 of K) */
#define MM_I8_TILED_A_MAX 0xFFFF0000u
/* One GEMM segment: the routed experts, or the shared expert as one dense
 * GEMM. */
typedef struct {
    const int8_t *b;         /* packed fragments of expert 0 */
    size_t b_expert_stride;  /* bytes between experts' fragment sets */
    const float *sb0, *sb1;  /* per-column weight scales (gate, up) of expert 0 */
    int sb_expert_stride;    /* floats between experts' scale vectors */
    const int32_t *cnt;      /* [E * MM_CNT_STRIDE] rows per expert, or 0: one expert with T rows */
    const int32_t *rows;     /* [E, T] route ids, or 0: identity rows */
    const int8_t *a;         /* A rows (int8), indexed by token (gate/up) or route id (down) */
    const float *sa;         /* A row scales, same index as a */
    int a_by_route;          /* 1: A row = route id; 0: A row = route id / K (token) */
    float *out;              /* [rows, N_out] by route id (or token for identity rows) */
    int32_t *dbg_acc;        /* raw accumulators (routed gate/up: [R,2,I]; down: [R,H]) or 0 */
    int T, K, E;             /* tokens, top-k, experts (E = 1 for the shared expert) */
    int N;                   /* output columns (I or S for gate/up, H for down) */
    int Kd;                  /* reduction length (H for gate/up, I or S for down) */
    int gu;                  /* 1: gate/up with SwiGLU epilogue, 0: plain dequantising GEMM */
    int spare_row;           /* `out` has a spare row here (N + 256 floats) that absorbs
                                the stores of padded rows and columns */
} mm_i8_tiled_args;

/* Big-tile kernel arguments: one launch serves the routed experts and the
 * shared expert (segments 0 and 1, same gate/up flag); nseg = 1 when there
 * is no shared expert. */
typedef struct {
    mm_i8_tiled_args seg[2];
    int nseg;
} mm_i8_bt_args;

/* ---- MLA absorbed decode ----------------------------------------------------- */
#define MM_MLA_KVL 512            /* kv_lora_rank served by the kernels */
#define MM_MLA_QKR 64             /* qk_rope_head_dim served by the kernels */
#define MM_MLA_KVD (MM_MLA_KVL + MM_MLA_QKR)
#define MM_MLA_KC (MM_MLA_KVD / 32) /* 32-wide latent chunks of one cache row */
#ifndef MM_MLA_CHUNK
#define MM_MLA_CHUNK 512          /* keys per attention block (the longest chunk) */
#endif
/* From MM_MLA_WIDE_B rows on, the W_UK and W_UV products take
 * MM_MLA_WIDE_S column tiles per wave (mm_mla_qprep_w, mm_mla_uv_w). */
#ifndef MM_MLA_WIDE_B
#define MM_MLA_WIDE_B 512
#endif
#define MM_MLA_WIDE_S 4
#ifndef MM_MLA_MIN_BLOCKS
#define MM_MLA_MIN_BLOCKS 256     /* chunks shrink (to 16 keys per wave) until the grid has this many blocks */
#endif
#ifndef MM_MLA_AW
#define MM_MLA_AW 4               /* waves per attention block */
#endif
/* Key chunks one (head group, sequence) may have: 512 x 512 = 262,144 keys at
 * the longest chunk, above the reference's KV_CACHE_CAP of 163,840
 * (src/model_load.c:237). */
#define MM_MLA_MAXCH 512
#ifndef MM_MLA_PART_MAX
#define MM_MLA_PART_MAX ((size_t)512 << 20)   /* bytes of attention chunk partials per launch */
#endif
#define MM_MLA_TILE_B (16 * 1056 + 16 * 128)   /* LDS bytes of one 16-key sub-tile */
/* mm_mla_attn_rows' dynamic LDS: each wave's row output, 16 heads of
 * MM_MLA_KVL + 4 floats (it also holds the shared sub-tile ring) */
#define MM_MLA_ROWS_LDS (MM_MLA_AW * 16 * (MM_MLA_KVL + 4) * 4)

/* qabs = q_nope . W_UK per head. */
typedef struct {
    const float *q;           /* [B, NH, QKN + QKR] */
    const uint16_t *wukT;     /* [NH, KVL, QKN] bf16: W_UK per head, transposed */
    float *qabs;              /* [B, NH, KVL], or 0: not written */
    uint16_t *qhl;            /* [B, NH, 2, KVL] bf16: qabs split into hi (row 0) + lo (row 1) */
    int B, NH, QKN;
} mm_mla_qprep_args;

/* Load-time preparation of W_UK^T from the head-interleaved kv_b. */
typedef struct {
    const uint16_t *kv_b;
    uint16_t *wukT;
    int NH, QKN, VHD;
} mm_mla_wprep_args;

/* Flash-decoding partials of (row b, head group, chunk) triples, N = B * HG
 * * nchunks of them, in that order (row-major): a 1-D grid of 8 * ceil(N / 8)
 * blocks, block L taking triple (L % 8) * ceil(N / 8) + L / 8 (blocks past N
 * exit), so that a row's chunks run on one XCD (blocks are dealt to the 8
 * XCDs in turn) and share its Q in that L2 -- with one length for every
 * row; with kv_lens, block L takes triple N - 1 - L (rows of unequal
 * lengths spread over the XCDs, a prefill's longest first). */
typedef struct {
    const uint16_t *qhl;      /* [B, NH, 2, KVL] bf16: qabs as hi + lo halves (qprep) */
    const float *q;           /* [B, NH, QKN + QKR] (the q_pe part) */
    const uint16_t *cache;    /* [sequences, seq_stride, KVD] bf16 */
    const int32_t *kv_lens;   /* [B] or 0 */
    int kv_len;               /* used when kv_lens == 0 */
    int seq_stride;
    float scale;
    float *part_ml;           /* [B, HG, nchunks, 2, 16]: running max, sum */
    float *part_o;            /* [B, HG, nchunks, 16, KVL] unnormalised */
    float *scores;            /* [B, NH, probs_stride] scaled scores (debug) or 0 */
    int probs_stride;
    int NH, HG, nchunks, QKN;
    int chunk;                /* keys per block: a multiple of 16 * MM_MLA_AW, <= MM_MLA_CHUNK
                                 (mm_mla_attn_rows: any length, up to a whole context) */
    const int32_t *slots;     /* [B] cache sequence of row b, or 0: sequence b */
    float *clat;              /* one chunk (nchunks == 1, no probabilities): clat [B, NH, KVL]
                                 written here, O / l as the merge computes it; else 0 */
    int B;
} mm_mla_attn_args;

/* Merge the chunk partials, normalise (clat); then ctx = W_UV . clat. */
typedef struct {
    const float *part_ml, *part_o;
    const uint16_t *kv_b;
    const int32_t *kv_lens;
    int kv_len;
    float *ctx;               /* [B, NH * VHD] */
    float *clat;              /* [B, NH, KVL] (written by the merge, read by the W_UV product) */
    float *probs;             /* [B, NH, probs_stride]: scores in, probabilities out, or 0 */
    int probs_stride;
    int B, NH, QKN, VHD, HG, nchunks;
    uint16_t *ctx_hl;         /* or 0: ctx also as bf16 hi/lo planes [2, B, NH * VHD] */
} mm_mla_combine_args;

/* ---- dense bf16 matmul --------------------------------------------------------- */
/* y[t, d] (=|+=) sum_i x[t, i] * W[d, i]; W bf16 row-major [d_out, n_in].  x
 * is first converted to bf16 rows of a padded stride kp (a multiple of 64,
 * zeros past n_in): truncated, or split into hi + lo halves. */
typedef struct {
    const float *x;          /* [T, n_in] */
    uint16_t *xh, *xl;       /* [T, kp]; xl only for the split */
    int T, n_in, kp;
    int split;               /* 1: hi/lo split (RNE); 0: truncation */
} mm_cvt_bf16_args;

typedef struct {
    const uint16_t *xh, *xl; /* [T, kp] converted x (xl: split mode) */
    const uint16_t *w;       /* [d_out, n_in] */
    float *y;                /* [T, d_out] */
    int T, d_out, n_in, kp;
    int split;               /* 1: two MFMAs per product (x = hi + lo) */
    int accumulate;
    int bn;                  /* block tile columns: 128, 64 or 32 */
} mm_gemm_bf16_args;

/* Skinny-M GEMM (T <= MM_SKINNY_T rows of x): block (MM_SKINNY_BN output columns,
 * one K split); partials [nsplit, T, d_out] when nsplit > 1. */
#define MM_SKINNY_T 64
#ifndef MM_SKINNY_BN
#define MM_SKINNY_BN 64           /* output columns per block (4 waves x 16) */
#endif
#ifndef MM_SKINNY_WIDE_WC
#define MM_SKINNY_WIDE_WC 2       /* mm_gemm_skinny_wide: 16-column groups per wave */
#endif
/* outputs of at least this many 64-column blocks take the wide form */
#ifndef MM_SKINNY_WIDE_MIN_NB
#define MM_SKINNY_WIDE_MIN_NB 1024
#endif
typedef struct {
    const float *x;          /* [T, n_in] fp32, converted while staged */
    const uint16_t *w;       /* [d_out, n_in] */
    float *y;                /* [T, d_out], written when nsplit == 1 */
    float *part;             /* [nsplit, T, d_out] when nsplit > 1 */
    int T, d_out, n_in, nsplit, kr;   /* kr: inputs per split, a multiple of 64 */
    int split;               /* 1: x as a bf16 hi/lo pair; 0: x truncated to bf16 */
    int accumulate;
    /* an optional second matrix over the same x: column blocks >= nb0 are
     * its (w1 [d_out1, n_in] -> y1 [T, d_out1], partials after the first's) */
    const uint16_t *w1;
    float *y1;
    int d_out1, nb0;
    int part_out;            /* 1: partials even when nsplit == 1 (a fused reduce reads them) */
} mm_gemm_skinny_args;

/* As mm_gemm_skinny_args, with x given as bf16 hi/lo planes ([2, T, n_in]:
 * rne16(x), then rne16(x - hi)) instead of fp32 rows; always split. */
typedef struct {
    const uint16_t *xhl;
    const uint16_t *w;
    float *y;
    float *part;
    int T, d_out, n_in, nsplit, kr;
    int accumulate;
    const uint16_t *w1;
    float *y1;
    int d_out1, nb0;
    int part_out;
} mm_gemm_hl_args;

typedef struct {
    const float *part;       /* [nsplit, T, d_out], then [nsplit, T, d_out1] */
    float *y;                /* [T, d_out] */
    int T, d_out, nsplit, accumulate;
    float *y1;               /* [T, d_out1] (second matrix) or NULL */
    int d_out1;
} mm_skinny_reduce_args;

/* ---- LM head (final RMSNorm, logits, greedy argmax) ------------------------- */
#define MM_LM_NB 4                /* tokens served by the logits GEMV (more: the MFMA GEMM) */
#define MM_LM_HMAX 2048           /* hidden sizes served by the logits GEMV */
typedef struct {
    const float *x;          /* [T, n] */
    const uint16_t *w;       /* [n] bf16 */
    float *y;                /* [T, n] */
    int n;
    float eps;
} mm_rmsnorm_args;

#define MM_RRN_THREADS 1024      /* mm_reduce_rmsnorm: threads per row block */
#define MM_RRN_PT 4              /* row elements per thread (rows up to 4096) */
/* Split-K partials summed into the residual rows, then their RMSNorm: per
 * row t, v = part[0][t] + part[1][t] + ... (split order), x[t] += v, then
 * xn[t] = rmsnorm(x[t], w) -- mm_skinny_reduce followed by mm_rmsnorm in
 * one pass (the norm's sum of squares reduced over the block's 1024
 * threads). */
typedef struct {
    const float *part;       /* [nsplit, T, n] */
    float *x;                /* [T, n] residual rows, updated */
    const uint16_t *w;       /* [n] bf16 norm weight */
    float *xn;               /* [T, n] */
    int T, n, nsplit;
    float eps;
} mm_reduce_rmsnorm_args;

typedef struct {
    const float *x;          /* [B, H] activations before the final norm */
    const uint16_t *norm;    /* [H] bf16 final RMSNorm weight */
    float eps;
    const uint16_t *w;       /* [V, H] bf16 */
    float *y;                /* [B, V] logits */
    float *part_v;           /* [B, waves] per-wave best logit */
    int32_t *part_i;         /* [B, waves] its row */
    int B, V, H;
} mm_lm_gemv_args;

/* RMSNorm rows written as bf16 hi/lo planes (the LM head GEMM's operand). */
typedef struct {
    const float *x;          /* [T, n] */
    const uint16_t *w;       /* [n] bf16 */
    uint16_t *yhl;           /* [2, T, n]: rne16(y), then rne16(y - hi) */
    int n;
    float eps;
} mm_rmsnorm_hl_args;

/* Logits GEMM for MM_LM_NB < T <= 64 rows: y[T, N] = x . W^T with x given
 * as bf16 hi/lo planes; MM_LMG_BN columns per block. */
#define MM_LMG_BN 256
#define MM_LMG_NS 3                                  /* ring stages (two chunks ahead) */
#define MM_LMG_STAGE (MM_LMG_BN * 128 + 2 * 64 * 128) /* LDS bytes per stage: W, x hi, x lo */
typedef struct {
    const uint16_t *xhl;     /* [2, T, K] */
    const uint16_t *w;       /* [N, K] bf16 */
    float *y;                /* [T, N] */
    int T, N, K;             /* K a multiple of 64 */
} mm_lm_gemm_args;

#define MM_ARGMAX_SEG 1024       /* row elements per argmax segment (block) */
#define MM_LM_GEMV_BLOCKS 2048   /* GEMV grid (4 waves each): argmax partials per token */
typedef struct {
    const float *logits;     /* [T, n] */
    int32_t *tokens;         /* [T] */
    float *part_v;           /* [T, nseg] segment maxima */
    int32_t *part_i;         /* [T, nseg] their indices */
    int n, T, nseg;
} mm_argmax_args;

/* ---- dense GEMV for a few tokens (decode projections) ----------------------- */
/* Up to two weight matrices ("segments") over one activation row set: rows
 * [0, rows0) of the row space are W0's, [rows0, rows0 + rows1) W1's;
 * y_s[t * ys_s + r] receives token t's output row r of segment s. */
typedef struct {
    const float *x;          /* [B, H] */
    const uint16_t *norm;    /* [H] rmsnorm weight applied to x first, or NULL */
    float eps;
    const uint16_t *w0, *w1; /* [rows_s, H] bf16 */
    float *y0, *y1;
    int rows0, rows1, ys0, ys1;
    int B, H;
    int accumulate;          /* y += x' . W^T */
    int x_bf16;              /* x' = bf16(x) by truncation (no norm) */
} mm_gemv_args;
#define MM_GEMV_NB 4              /* tokens served by the GEMV (more: the MFMA GEMM) */
#ifndef MM_GEMV_RPW
#define MM_GEMV_RPW 2             /* GEMV rows per wave per turn (4 waves per block) */
#endif

/* ---- MLA decode front: RoPE, kv norm, latent-cache append -------------------- */
#define MM_ROPE_PAIRS_MAX 2048    /* q_pe pairs per token (NH * QKR / 2) */
typedef struct {
    float *q;                /* [B, NH * (QKN + QKR)]: RoPE applied to each q_pe in place */
    const float *comp;       /* [B, KVL + QKR] kv_a output: c_kv | k_pe before norm/RoPE */
    const uint16_t *kv_norm; /* [KVL] kv_a_layernorm */
    const float *inv_freq;   /* [QKR / 2] */
    const int32_t *pos;      /* [B] positions */
    uint16_t *cache;         /* [sequences, seq_stride, KVL + QKR] bf16 latent cache */
    float *kv_out;           /* [B, KVL + QKR] fp32 copy of the appended rows, or NULL */
    int B, nh, qkn, qkr, kvl, seq_stride, interleaved;
    float eps;               /* kv_a_layernorm eps */
    const int32_t *slots;    /* [B] cache sequence of token b, or 0: sequence b */
} mm_mla_rope_args;

/* RoPE / kv norm / cache append (one block per token) and the absorbed
 * queries in one launch: blocks [0, B) are mm_mla_rope's, the rest
 * mm_mla_qprep's grid (KVL / 64, NH, ceil(B / 32)) in x-fastest order. */
typedef struct {
    mm_mla_rope_args r;
    mm_mla_qprep_args qp;
} mm_mla_rope_qprep_args;

/* ---- routing for more than MM_EMAX_FAST experts ------------------------------- */
/* mm_router_wide: logits [T, E] (mm_router_args' logits mode: logits_out,
 * logit_bias), grid (ceil(T / 4), ceil(E / 64)).  mm_route_wide: scores,
 * top-k and weights from logits_in, one wave per token (4 per block), E up
 * to MM_EMAX; with qx set also the per-token int8 quantisation of x, with
 * cnt/rows also the tiled path's per-expert row lists. */
#define MM_RW_EJ (MM_EMAX / 64)  /* experts per lane */
typedef struct {
    mm_router_args r;
    int32_t *cnt;            /* [E * MM_CNT_STRIDE] rows per expert (zero on entry), or 0 */
    int32_t *rows;           /* [E, T] route ids (t*K + r) per expert, or 0 */
    const float *x;          /* [T, H], with qx */
    int8_t *qx;              /* [T, H] or 0 */
    float *sx;               /* [T] */
} mm_route_wide_args;

#endif /* MLAMOE_KERNEL_PARAMS_H */
