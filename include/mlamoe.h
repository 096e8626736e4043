/* mlamoe.h -- C-ABI of the MI355X (gfx950) mla-moe matmul hot path.
 *
 * A drop-in for the reference engine's CPU hot path:
 *   - the MoE FFN, ffn_compute (src/run.c:116-162), batched over T tokens,
 *     with bf16 weights (GEMV, T small) or int8 weights (MFMA, any T);
 *   - the dense bf16 matmul
 *     (src/run.c:29-37) and the MLA absorbed-decode chain (src/run.c:430-460).
 *
 * Conventions
 *   - Plain C types only; every function returns an int status (0 = MM_OK)
 *     and never exits the process.  mm_last_error() describes the last
 *     failure on the calling thread.  The reference calls exit() instead
 *     (src/model_load.c:15-22, src/kernels/utils.h:9-19).
 *   - A context (mm_ctx) owns one HIP stream on one device plus all
 *     device-side weights it was given; it is used by one host thread at a
 *     time.  The reference keeps this state in a process-global GpuContext
 *     (src/getp_run.hip:26, src/kernels/getp_state.h:57-96).
 *   - Functions named *_dev take device pointers and are asynchronous on the
 *     context stream.  mm_moe_forward / mm_ffn_compute, mm_matmul_bf16 and
 *     mm_mla_absorbed_decode take host pointers and return with the result
 *     in host memory, like the reference functions they replace.
 *   - Weights are uploaded (and quantised, for int8) once per layer, outside
 *     any timed region, like the reference's warm_up (src/getp_run.hip:703-880).
 */
#ifndef MLAMOE_H
#define MLAMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Every entry point below is exported from libmlamoe.so; nothing else is. */
#define MM_API __attribute__((visibility("default")))

/* ---- status ------------------------------------------------------------ */
#define MM_OK 0
#define MM_ERR_INVALID (-1)     /* bad argument or shape */
#define MM_ERR_UNSUPPORTED (-2) /* valid request this build cannot serve */
#define MM_ERR_HIP (-3)         /* HIP runtime error */
#define MM_ERR_NOMEM (-4)       /* device or host allocation failed */
#define MM_ERR_STATE (-5)       /* call order (e.g. layer not loaded) */

/* Message for the last failed call on this thread ("" if none). */
MM_API const char *mm_last_error(void);

/* ---- context ----------------------------------------------------------- */
typedef struct mm_ctx mm_ctx;

/* Create a context on HIP device `device`: loads the gfx950 code objects and
 * creates the context's stream (default priority). */
MM_API int mm_ctx_create(int device, mm_ctx **out);
MM_API void mm_ctx_destroy(mm_ctx *ctx);
/* The hipStream_t the context currently queues on, as an opaque pointer. */
MM_API void *mm_ctx_stream(mm_ctx *ctx);
/* Queue the context's work on a caller-owned hipStream_t (passed as an
 * opaque pointer) from now on; NULL returns to the context's own stream.
 * Work already queued on the previous stream stays ordered before anything
 * queued afterwards (the new stream waits on an event of the old one), so
 * the switch is safe at any point.  The caller keeps the stream alive while
 * it is set, and synchronous entry points then wait on it.  The reference
 * runs everything on one hipStreamNonBlocking stream of its own
 * (src/getp_run.hip:735); this lets a host engine put the hot path on the
 * stream it already orders its other work on. */
MM_API int mm_ctx_set_stream(mm_ctx *ctx, void *stream);
/* Wait for all work queued on the context stream. */
MM_API int mm_ctx_sync(mm_ctx *ctx);
/* Bytes of device workspace the context holds now: the *_dev entry points
 * grow it on demand (after a stream sync) and keep it until the context is
 * destroyed; mm_moe_forward_noalloc_dev never touches it. */
MM_API int mm_ctx_workspace_bytes(mm_ctx *ctx, size_t *bytes);

/* ---- device memory and timing helpers ------------------------------------ */
MM_API int mm_dev_alloc(mm_ctx *ctx, size_t bytes, void **dptr);
MM_API int mm_dev_free(mm_ctx *ctx, void *dptr);
/* Synchronous copies (ordered after the context stream's queued work). */
MM_API int mm_h2d(mm_ctx *ctx, void *dst, const void *src, size_t bytes);
MM_API int mm_d2h(mm_ctx *ctx, void *dst, const void *src, size_t bytes);
MM_API int mm_d2d(mm_ctx *ctx, void *dst, const void *src, size_t bytes);

#define MM_FILL_BF16_NORMAL 0   /* uint16 bf16, N(0, std), truncated */
#define MM_FILL_F32_NORMAL 1    /* float N(0, std) */
#define MM_FILL_F32_UNIFORM 2   /* float U[0, 1) */
/* Fill n elements with seeded synthetic data on the device (asynchronous). */
MM_API int mm_fill_synthetic(mm_ctx *ctx, void *dst, size_t n, int kind, uint64_t seed, float stdev);

/* HIP events on the context stream: mm_timer_start, queue work,
 * mm_timer_stop -> elapsed milliseconds (synchronises). */
MM_API int mm_timer_start(mm_ctx *ctx);
MM_API int mm_timer_stop(mm_ctx *ctx, float *ms);

/* Per-kernel timing: while enabled, every kernel this context launches is
 * bracketed by HIP events on its stream.  mm_prof_query synchronises and
 * returns the summed duration and launch count of kernels named `kernel`. */
MM_API int mm_prof_enable(mm_ctx *ctx, int on);
MM_API int mm_prof_reset(mm_ctx *ctx);
MM_API int mm_prof_query(mm_ctx *ctx, const char *kernel, double *total_ms, long long *launches);

/* ---- MoE FFN ----------------------------------------------------------- */

/* The MoE fields of the reference Config (include/model.h:12-42). */
typedef struct {
    int hidden_size;        /* H */
    int n_routed_experts;   /* E (<= 1024, src/run.c:133-134) */
    int n_shared_experts;   /* shared MLP width = n_shared_experts * moe_inter_size */
    int n_experts_per_tok;  /* K (<= 16) */
    int moe_inter_size;     /* I */
    int router_sigmoid;     /* 0: softmax scores (dsv2), 1: sigmoid (GLM noaux_tc) */
    int norm_topk;          /* normalise the top-k weights */
    float routed_scaling;   /* multiply the routed weights */
} mm_moe_config;

/* One MoE layer's weights, as the reference's ModelWeights holds them
 * (include/model.h:84-96): bf16 row-major, one pointer per expert. */
typedef struct {
    const uint16_t *moe_gate;              /* [E, H] */
    const float *moe_gate_bias;            /* [E] or NULL (GLM e_score_correction_bias) */
    const uint16_t *const *expert_gate;    /* E pointers to [I, H] */
    const uint16_t *const *expert_up;      /* E pointers to [I, H] */
    const uint16_t *const *expert_down;    /* E pointers to [H, I] */
    const uint16_t *shared_gate;           /* [S, H], S = n_shared_experts * I */
    const uint16_t *shared_up;             /* [S, H] */
    const uint16_t *shared_down;           /* [H, S] */
} mm_moe_layer_weights;

/* Configure the MoE geometry for `n_layers` layers (once per context). */
MM_API int mm_moe_init(mm_ctx *ctx, const mm_moe_config *cfg, int n_layers);

#define MM_LOAD_BF16 1u          /* keep bf16 expert weights (GEMV path) */
#define MM_LOAD_INT8 2u          /* keep int8 per-output-channel weights (MFMA path) */
#define MM_LOAD_DEVICE_PTRS 4u   /* the weight pointers are device pointers */
/* Upload one layer's weights (synchronous). */
MM_API int mm_moe_load_layer(mm_ctx *ctx, int layer, const mm_moe_layer_weights *w, unsigned flags);

/* Load layer `layer` as a dense SwiGLU layer, the first_k_dense layers of
 * the reference (ffn_compute's dense branch, src/run.c:119-122: ModelWeights
 * dense_gate / dense_up [dense_inter, H], dense_down [H, dense_inter], bf16,
 * include/model.h:79-81); dense_inter % 8 == 0.  The forward calls then
 * compute out = down . (silu(gate . xn) * (up . xn)) for it, with bf16
 * weights and fp32 activations whatever the MM_FWD_* format flag, and leave
 * topk_idx, topk_w and probs untouched (the reference returns before its
 * router).  Host pointers, or device pointers with MM_LOAD_DEVICE_PTRS (the
 * weights are copied).  Synchronous. */
MM_API int mm_moe_load_dense_layer(mm_ctx *ctx, int layer, const uint16_t *gate,
                                   const uint16_t *up, const uint16_t *down, int dense_inter,
                                   unsigned flags);

/* ---- the packed int8 expert format (offline quantisation) ------------------ */
/* One layer's int8 experts as the MFMA kernels read them: a pool of 16-row x
 * 64-byte fragments -- routed gate/up [E][I/16][H/64][gate, up], routed down
 * [E][H/16][I/64], shared gate/up [S/16][H/64][gate, up], shared down
 * [H/16][S/64]; fragment byte 16 l + b = row 16 nb + (l % 16), column
 * 64 kb + 16 (l / 16) + b -- and a scale table s_g [E*I] | s_u [E*I] |
 * s_d [E*H] | ss_g [S] | ss_u [S] | ss_d [H] (fp32, per output row: q =
 * clamp(rint(w / s), -127, 127), s = max|w| / 127).  The reference packs its
 * bf16 experts at start-up (src/getp_run.hip:58-113, 797-808); this format
 * holds the int8 pack so a loader uploads it without quantising.  Written by
 * mlamoe.weights (safetensors container, format "mlamoe-i8"). */
MM_API int mm_moe_i8_layer_size(const mm_moe_config *cfg, size_t *pool_bytes, size_t *n_scales);
/* Copy a layer loaded with MM_LOAD_INT8 (quantised on the device) to host
 * buffers of mm_moe_i8_layer_size.  Synchronous. */
MM_API int mm_moe_export_layer_i8(mm_ctx *ctx, int layer, void *pool, float *scales);
/* Load a layer from its packed pool and scales plus the router weight
 * (moe_gate [E, H] bf16, moe_gate_bias [E] or NULL), host pointers or, with
 * MM_LOAD_DEVICE_PTRS, device pointers: no quantisation, int8 format only
 * (MM_FWD_INT8).  Synchronous. */
MM_API int mm_moe_load_layer_i8_packed(mm_ctx *ctx, int layer, const uint16_t *moe_gate,
                                       const float *moe_gate_bias, const void *pool,
                                       const float *scales, unsigned flags);

#define MM_FWD_BF16 0u           /* bf16 weights, fp32 activations */
#define MM_FWD_INT8 1u           /* int8 weights, per-token int8 activations */
#define MM_FWD_ACCUMULATE 2u     /* out += ffn(x) (residual fused) instead of out = */

/* T tokens through MoE layer `layer` (ffn_compute, src/run.c:116-162, per
 * token; the prefill loop of src/run.c:291-313).  Device pointers, queued on
 * the context stream:
 *   xn      [T, H] fp32 input (post-attention-norm hidden)
 *   out     [T, H] fp32 output (overwritten, or accumulated with
 *           MM_FWD_ACCUMULATE; may alias xn only with MM_FWD_INT8)
 *   logits  [T, E] fp32 router logits to route instead of computing them
 *           from xn, or NULL
 *   topk_idx/topk_w [T, K] selected experts / weights out, or NULL
 *   probs   [T, E] router scores out (s->moe_logits after the call), or NULL */
MM_API int mm_moe_forward_dev(mm_ctx *ctx, int layer, int T, const float *xn, float *out,
                       const float *logits, int32_t *topk_idx, float *topk_w, float *probs,
                       unsigned flags);

/* mm_moe_forward_dev without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results; the call's workspace is a static
 * device array of MM_NOALLOC_SCRATCH_BYTES per device (32 MiB: e.g. up to
 * ~280 tokens of a DeepSeek-V2-Lite int8 layer, 64 for the bench's decode
 * batch) instead of the context's growable buffer.  A call that would need
 * more fails with MM_ERR_UNSUPPORTED before launching anything.  Every call
 * on a device shares that
 * device's array: calls that overlap on one device (two streams, two host
 * threads) race.  While per-kernel profiling is on (mm_prof_enable) it
 * returns MM_ERR_STATE: the profiler's records are host allocations. */
#define MM_NOALLOC_SCRATCH_BYTES (32u << 20)
MM_API int mm_moe_forward_noalloc_dev(mm_ctx *ctx, int layer, int T, const float *xn, float *out,
                                      const float *logits, int32_t *topk_idx, float *topk_w,
                                      float *probs, unsigned flags);

/* Router logits alone: logits[t, e] = sum_i xn[t, i] * moe_gate[e, i] in the
 * reference's sequential fp32 order (the matmul at src/run.c:124), plus
 * logit_bias[e] when logit_bias != NULL (a per-expert prior; not in the
 * reference, used to build skewed synthetic workloads).  Device pointers,
 * asynchronous.  The result can be passed as `logits` to mm_moe_forward_dev. */
MM_API int mm_moe_router_logits_dev(mm_ctx *ctx, int layer, int T, const float *xn,
                                    const float *logit_bias, float *logits);

/* Intermediates of the int8 path, for parity checking (no reference
 * counterpart: the reference has no int8 path).  Device pointers; any may be
 * NULL.  R = T * K routed rows, row t*K + r is token t's slot r.
 *   qx [T, H] int8, sx [T]        per-token quantised input
 *   acc_gu [R, 2, I] int32        raw gate (0) and up (1) accumulators
 *   h [R, I]                      SwiGLU output, fp32
 *   qh [R, I] int8, sh [R]        its per-row quantisation
 *   acc_d [R, H] int32            raw down-projection accumulators
 *   y [R, H]                      dequantised expert outputs (before the route weight)
 *   hs, qhs [T, S], shs [T], ys [T, H]   the same for the shared expert */
typedef struct {
    int8_t *qx;
    float *sx;
    int32_t *acc_gu;
    float *h;
    int8_t *qh;
    float *sh;
    int32_t *acc_d;
    float *y;
    float *hs;
    int8_t *qhs;
    float *shs;
    float *ys;
} mm_moe_i8_debug;

/* mm_moe_forward_dev with MM_FWD_INT8, also filling the debug intermediates. */
MM_API int mm_moe_forward_i8_debug_dev(mm_ctx *ctx, int layer, int T, const float *xn, float *out,
                                       const float *logits, int32_t *topk_idx, float *topk_w,
                                       float *probs, unsigned flags,
                                       const mm_moe_i8_debug *dbg);

/* mm_moe_forward_dev with host pointers (the prefill loop of
 * src/run.c:291-313 in one call): xn, out [T, H], topk_idx / topk_w [T, K],
 * probs [T, E] (any of the last three may be NULL).  Routes from the layer's
 * own router (no logits argument).  Synchronous: returns with the results in
 * host memory. */
MM_API int mm_moe_forward(mm_ctx *ctx, int layer, int T, const float *xn, float *out,
                          int32_t *topk_idx, float *topk_w, float *probs, unsigned flags);

/* Host-pointer mirror of ffn_compute (src/run.c:116-117) for one token:
 * out [H] overwritten (MM_FWD_ACCUMULATE is ignored, as the reference
 * overwrites); topk_idx / topk_w [K] receive the selected experts and
 * weights, probs [E] the router's softmax (or sigmoid) scores -- what the
 * reference leaves in s->moe_logits (src/run.c:124-129) --, each may be
 * NULL.  A dense layer (mm_moe_load_dense_layer) leaves all three untouched,
 * as the reference's dense branch does.  Synchronous. */
MM_API int mm_ffn_compute(mm_ctx *ctx, int layer, const float *xn, float *out, int *topk_idx,
                          float *topk_w, float *probs, unsigned flags);

/* ---- dense bf16 matmul ------------------------------------------------------ */

#define MM_MATMUL_X_BF16 1u       /* cast x to bf16 (truncation, include/tensor.h:16-20) */
#define MM_MATMUL_ACCUMULATE 2u   /* y += x . W^T (the GPU gemv "add" variant) */

/* matmul (src/run.c:29-37) over T rows: y[t, d] = sum_i x[t, i] * W[d, i],
 * W bf16 row-major [d_out, n_in] (nn.Linear layout), x/y fp32.  Without
 * MM_MATMUL_X_BF16 the fp32 x is carried as a bf16 hi/lo pair (two MFMAs),
 * tracking the fp32 reference to ~1e-5.  Up to 4 rows with n_in <= 2048 take
 * a GEMV that reads each weight row once with x in fp32 registers (the decode
 * step's o_proj, src/run.c:463-464).  n_in % 8 == 0.  Device pointers,
 * asynchronous. */
MM_API int mm_matmul_bf16_dev(mm_ctx *ctx, float *y, const float *x, const uint16_t *w,
                              int d_out, int n_in, int T, unsigned flags);

#define MM_MATMUL_W_HOST 4u       /* mm_matmul_bf16: w is host memory (uploaded once, kept) */

/* matmul (src/run.c:29-37) with host x [T, n_in] and y [T, d_out]: the
 * reference call matmul(y, x, w, d_out, n_in) is mm_matmul_bf16(ctx, y, x,
 * w, d_out, n_in, 1, MM_MATMUL_W_HOST).  w is a device pointer, or with
 * MM_MATMUL_W_HOST a host pointer whose matrix is copied to the device on
 * its first use and looked up by (pointer, size) afterwards -- the
 * reference's weights are read-only mappings of the checkpoint
 * (include/model.h:44-46), so a host matrix must not change while the
 * context holds its copy (mm_host_weights_release drops every copy).
 * Other flags as mm_matmul_bf16_dev.  Synchronous. */
MM_API int mm_matmul_bf16(mm_ctx *ctx, float *y, const float *x, const uint16_t *w, int d_out,
                          int n_in, int T, unsigned flags);
/* Free the device copies of host weights that mm_matmul_bf16 keeps. */
MM_API int mm_host_weights_release(mm_ctx *ctx);

/* The same product over T <= 64 rows (the batched decode step's
 * projections) with x given already split: xhl [2, T, n_in] bf16, plane 0
 * the round-to-nearest-even bf16 of each x, plane 1 that of x minus it (the
 * pair mm_matmul_bf16_dev carries fp32 x as).  Same results, bit for bit, as
 * mm_matmul_bf16_dev on the fp32 rows from 5 rows on; n_in % 64 == 0.  No
 * counterpart in the reference: it serves callers whose kernels write their
 * rows in this form (the engine's norms and W_UV product) and the parity
 * tests of that path.  Device pointers, asynchronous. */
MM_API int mm_matmul_bf16_hl_dev(mm_ctx *ctx, float *y, const uint16_t *xhl, const uint16_t *w,
                                 int d_out, int n_in, int T, unsigned flags);

/* ---- LM head: final RMSNorm, logits, greedy sampling ------------------------- */

/* rmsnorm (src/run.c:22-27) of T rows: y[t] = (x[t] * inv) * w with
 * inv = 1 / sqrtf(sum(x[t]^2) / n + eps); w bf16 [n].  Device pointers,
 * asynchronous; y may equal x. */
MM_API int mm_rmsnorm_dev(mm_ctx *ctx, int T, const float *x, const uint16_t *w, int n, float eps,
                          float *y);

/* sample (src/run.c:503-508) of T rows of logits: tokens[t] = the first index
 * of the maximum (strict '>' scan from index 0; NaNs never win; a NaN at
 * index 0 selects 0).  Device pointers, asynchronous. */
MM_API int mm_argmax_dev(mm_ctx *ctx, int T, const float *logits, int n, int32_t *tokens);

/* The decode step's LM head for B tokens (src/run.c:493-494 followed by
 * sample, run.c:503-508): xb = rmsnorm(x, norm, eps), logits = xb . lm_head^T
 * (lm_head bf16 [vocab, hidden]), tokens = greedy argmax.  `logits` may be
 * NULL (not returned).  Up to 4 tokens with hidden <= 2048 take a GEMV that
 * reads each weight row once; more take the bf16 MFMA GEMM with x carried as
 * a hi/lo pair.  hidden % 8 == 0.  Device pointers, asynchronous.  Replaces
 * the reference's CPU tail of forward_absorbed / forward_unabsorbed and its
 * GPU lm_head GEMV + argmax (src/getp_run.hip:550-554). */
MM_API int mm_lm_head_dev(mm_ctx *ctx, int B, const float *x, const uint16_t *norm, float eps,
                          const uint16_t *lm_head, int vocab, int hidden, float *logits,
                          int32_t *tokens);

/* ---- MLA absorbed decode --------------------------------------------------- */

/* The attention fields of the reference Config (include/model.h:12-42). */
typedef struct {
    int n_heads;            /* NH */
    int qk_nope_head_dim;   /* QKN */
    int qk_rope_head_dim;   /* QKR (64) */
    int kv_lora_rank;       /* KVL (512) */
    int v_head_dim;         /* VHD */
    float softmax_scale;    /* (QKN + QKR)^-0.5 (src/model_load.c:270) */
} mm_mla_config;

/* Configure MLA for `n_layers` layers; kv_lora_rank 512 and qk_rope_head_dim
 * 64 are served (DeepSeek-V2-Lite, GLM-4.7-Flash). */
MM_API int mm_mla_init(mm_ctx *ctx, const mm_mla_config *cfg, int n_layers);

/* Upload one layer's kv_b_proj weight, [NH * (QKN + VHD), KVL] bf16,
 * head-interleaved [W_UK_h | W_UV_h] per head as the reference splits it
 * (src/model_load.c:80-86; include/model.h:56-65).  Synchronous. */
MM_API int mm_mla_load_layer(mm_ctx *ctx, int layer, const uint16_t *kv_b, unsigned flags);

/* Longest context the absorbed chain serves (512 chunks of 512 keys); the
 * reference caps its cache at KV_CACHE_CAP = 163,840 (src/model_load.c:237). */
#define MM_MAX_KV_LEN 262144

/* The absorbed per-head decode chain of forward_absorbed (src/run.c:430-460)
 * for B sequences, kv_len <= MM_MAX_KV_LEN.  Device pointers, asynchronous:
 *   q      [B, NH, QKN + QKR] fp32, q_nope | q_pe (RoPE applied)
 *   cache  [B, seq_stride, KVL + QKR] bf16 latent cache (c_kv | k_pe), the
 *          first kv_len (or kv_lens[b]) rows of each sequence attended
 *   kv_lens [B] per-sequence lengths <= kv_len, or NULL (all kv_len)
 *   ctx    [B, NH * VHD] fp32 output (ctx_h of run.c:460, heads concatenated)
 *   qabs   [B, NH, KVL], probs [B, NH, kv_len], clat [B, NH, KVL]: the
 *          q_absorbed, softmax weights and latent context, or NULL */
MM_API int mm_mla_absorbed_decode_dev(mm_ctx *ctx, int layer, int B, const float *q,
                                      const uint16_t *cache, int seq_stride,
                                      const int32_t *kv_lens, int kv_len, float *ctx_out,
                                      float *qabs, float *probs, float *clat);

/* The absorbed chain with host pointers and the reference's own fp32 latent
 * cache (RunState kv_cache rows c_kv | k_pe, include/model.h:117):
 * q [B, NH, QKN + QKR], cache [B, seq_stride, KVL + QKR] fp32 (the first
 * kv_len rows of each sequence are read), kv_lens [B] host or NULL, and the
 * outputs of mm_mla_absorbed_decode_dev in host memory (qabs, probs, clat
 * may be NULL).  The cache rows are rounded to bf16 (nearest even) on the
 * device, the element type the attention kernels read: the results are
 * those of mm_mla_absorbed_decode_dev on the rounded cache, and differ from
 * the fp32 reference by what that rounding moves (at most 2^-9 of each
 * element; normwise below 2^-8).  Synchronous. */
MM_API int mm_mla_absorbed_decode(mm_ctx *ctx, int layer, int B, const float *q,
                                  const float *cache, int seq_stride, const int32_t *kv_lens,
                                  int kv_len, float *ctx_out, float *qabs, float *probs,
                                  float *clat);

/* ---- MLA decode front: projections, RoPE, latent-cache append -------------- */

/* The RoPE inverse-frequency table of build_rope_inv_freq
 * (src/model_load.c:299-325): inv_freq[j], j < rope_dim / 2, blends the
 * extrapolated 1 / theta^(2j / rope_dim) with the interpolated (that /
 * factor) over the YaRN correction range of beta_fast / beta_slow at
 * orig_max positions; factor 1 is plain RoPE.  The reference reads the
 * parameters from config.json's rope_theta / rope_scaling
 * (src/model_load.c:271-279).  Host computation, fp32, the reference's steps. */
MM_API int mm_rope_inv_freq(int rope_dim, float theta, float factor, float beta_fast,
                            float beta_slow, float orig_max, float *inv_freq);

/* The Config fields of the decode front beyond mm_mla_config
 * (include/model.h:12-42). */
typedef struct {
    int hidden_size;            /* H */
    int q_lora_rank;            /* 0: q_proj (DeepSeek-V2-Lite); > 0: q_a_proj ->
                                   q_a_layernorm -> q_b_proj (GLM) */
    float rms_eps;              /* input_layernorm */
    float mla_norm_eps;         /* q_a / kv_a layernorms (1e-6, src/model_load.c:269) */
    int rope_interleaved;       /* 0: rotate adjacent pairs in place (dsv2); 1: rotated
                                   evens then rotated odds (glm) -- src/run.c:40-67 */
    const float *rope_inv_freq; /* host [qk_rope_head_dim / 2]: the engine's
                                   t->rope_inv_freq, or mm_rope_inv_freq */
} mm_mla_front_config;

/* Configure the decode front (after mm_mla_init); copies the RoPE table to
 * the device.  hidden_size and q_lora_rank must be multiples of 8. */
MM_API int mm_mla_front_init(mm_ctx *ctx, const mm_mla_front_config *cfg);

/* One layer's front weights, device pointers, bf16 row-major [out, in]
 * (ModelWeights, include/model.h:44-96). */
typedef struct {
    const uint16_t *input_norm; /* [H] input_layernorm */
    const uint16_t *q_proj;     /* [NH*(QKN+QKR), H]        q_lora_rank == 0 */
    const uint16_t *q_a_proj;   /* [q_lora_rank, H]         q_lora_rank > 0 */
    const uint16_t *q_a_norm;   /* [q_lora_rank]            q_a_layernorm */
    const uint16_t *q_b_proj;   /* [NH*(QKN+QKR), q_lora_rank] */
    const uint16_t *kv_a_proj;  /* [KVL+QKR, H] */
    const uint16_t *kv_a_norm;  /* [KVL] kv_a_layernorm */
} mm_mla_front_weights;

/* The decode step's attention front for B tokens, token b of sequence b at
 * position pos[b] (forward_absorbed, src/run.c:418-428, and its GPU form,
 * src/getp_run.hip:494-520):
 *   xb = rmsnorm(x[b], input_norm, rms_eps)
 *   q[b] = project_q(xb) (run.c:73-83), RoPE on each head's q_pe slice
 *   comp = kv_a_proj . xb
 *   cache[b, pos[b]] = rmsnorm(comp[:KVL], kv_a_norm, mla_norm_eps) | RoPE(comp[KVL:])
 * x [B, H] fp32; q [B, NH*(QKN+QKR)] fp32 out (the input of
 * mm_mla_absorbed_decode_dev); cache the [B, seq_stride, KVL+QKR] bf16 latent
 * cache of mm_mla_absorbed_decode_dev (round to nearest even; the reference
 * keeps fp32, include/model.h:117); kv_rows [B, KVL+QKR] fp32 copy of the
 * appended rows, or NULL.  A pos[b] outside [0, seq_stride) writes no cache
 * row.  Up to 4 tokens with H <= 2048 take fused GEMVs (norm in registers,
 * q and kv_a projections in one pass); more take the MFMA GEMM.  Device
 * pointers, asynchronous. */
MM_API int mm_mla_front_dev(mm_ctx *ctx, int B, const float *x, const mm_mla_front_weights *w,
                            const int32_t *pos, float *q, uint16_t *cache, int seq_stride,
                            float *kv_rows);

/* ---- batched decode engine ------------------------------------------------- */

/* The model-level fields of Config (include/model.h:12-42) the decode step
 * needs beyond mm_moe_config / mm_mla_config / mm_mla_front_config, and the
 * engine's capacity. */
typedef struct {
    int n_layers;
    int first_k_dense;       /* layers [0, first_k_dense) have a dense SwiGLU MLP */
    int hidden_size;
    int dense_inter_size;
    int vocab_size;
    float rms_eps;           /* post_attention_layernorm and the final norm */
    int max_batch;           /* sequence slots decoded together */
    int max_seq;             /* positions per slot at most (Config.max_seq_len) */
    unsigned moe_flags;      /* MM_FWD_BF16 or MM_FWD_INT8 for the MoE layers */
    int init_seq;            /* positions per slot allocated at creation (0: the
                                smaller of max_seq and 1024); the latent caches
                                grow on demand up to max_seq */
    int max_rows;            /* token rows one step may carry, prompt chunks
                                included (0: the larger of max_batch and 1024) */
} mm_engine_config;

/* One layer's non-expert weights, device pointers (ModelWeights,
 * include/model.h:44-96); the experts and kv_b live in the context
 * (mm_moe_load_layer*, mm_mla_load_layer). */
typedef struct {
    mm_mla_front_weights front;
    const uint16_t *o_proj;       /* [H, NH*VHD] */
    const uint16_t *post_norm;    /* [H] post_attention_layernorm */
    const uint16_t *dense_gate;   /* [dense_inter, H], dense layers only */
    const uint16_t *dense_up;     /* [dense_inter, H] */
    const uint16_t *dense_down;   /* [H, dense_inter] */
} mm_engine_layer;

typedef struct mm_engine mm_engine;

/* An engine over ctx, whose MoE layers (mm_moe_init with n_layers layers,
 * every MoE layer loaded), MLA layers (mm_mla_init, every layer loaded) and
 * front (mm_mla_front_init) are set up.  Allocates the latent caches
 * (n_layers x max_batch x init_seq x (KVL+QKR) bf16) and step buffers.
 * max_seq may exceed what fits in device memory: the caches grow only as
 * far as requests need (mm_engine_reserve). */
MM_API int mm_engine_create(mm_ctx *ctx, const mm_engine_config *cfg, mm_engine **out);
MM_API void mm_engine_destroy(mm_engine *e);
/* Positions per slot the latent caches hold now. */
MM_API int mm_engine_capacity(const mm_engine *e);
/* Grow the latent caches to hold at least `positions` per slot (<= max_seq),
 * doubling the capacity up to max_seq as the reference's
 * ensure_sequence_capacity does (src/getp_run.hip:269-290); every slot's
 * rows are kept.  Layers grow one at a time, so the extra memory during a
 * growth is one layer's new cache; if an allocation fails the engine keeps
 * working at its previous capacity.  Synchronous.  mm_engine_step and
 * mm_engine_generate call it themselves. */
MM_API int mm_engine_reserve(mm_engine *e, int positions);
MM_API int mm_engine_set_layer(mm_engine *e, int layer, const mm_engine_layer *w);
/* embed [vocab, H], final norm [H], lm_head [vocab, H]: device bf16. */
MM_API int mm_engine_set_head(mm_engine *e, const uint16_t *embed, const uint16_t *final_norm,
                              const uint16_t *lm_head);

/* One decode step (forward_absorbed, src/run.c:379-501) for batch rows
 * b < B: slot b takes token tokens[b] at position pos[b] (host arrays,
 * 0 <= pos[b] < max_seq; the caches grow when a position is past their
 * capacity) and next[b] (host) receives the greedy next token; logits
 * (device [B, vocab]) may be NULL.  Slot b's cache rows [0, pos[b]) must
 * hold its earlier positions.  Synchronous. */
MM_API int mm_engine_step(mm_engine *e, int B, const int32_t *tokens, const int32_t *pos,
                          int32_t *next, float *logits);

/* One step over R token rows (R <= max_rows), the batched prefill of
 * forward_unabsorbed (src/run.c:189-370; its GPU form, gpu_forward_unabsorbed
 * + batched_gpu_ffn, src/getp_run.hip:394-460, 558-701) and decode rows in
 * one pass: row r is token tokens[r] at position pos[r] of slot slots[r]
 * (host arrays).  Every row's latent-cache entry is written before any row
 * attends, so a slot may contribute several consecutive positions (a prompt
 * chunk, attended causally: row r sees positions [0, pos[r]] of its slot),
 * and other slots may decode in the same step.  A (slot, position) pair may
 * appear once per step; a slot's positions below its rows must hold its
 * earlier tokens.  The attention is the absorbed form, equal to the
 * reference's unabsorbed prefill in exact arithmetic (src/run.c:375-378).
 * The n_want rows listed in want_rows (ascending) are normed, projected to
 * the vocabulary and sampled: next[j] receives row want_rows[j]'s greedy
 * token, logits (device [n_want, vocab]) its logits, or NULL.  Synchronous. */
MM_API int mm_engine_step_rows(mm_engine *e, int R, const int32_t *slots, const int32_t *tokens,
                               const int32_t *pos, int n_want, const int32_t *want_rows,
                               int32_t *next, float *logits);

/* Continuous-batching greedy generation, the work of the reference's
 * inference() (src/getp_run.hip:920-995) for n_req prompts (token ids):
 * every step carries one decode row per slot past its prompt (the previous
 * step's sample) and, in the rows left up to max_rows, the next chunk of
 * the prompts still being prefilled (mm_engine_step_rows); a slot whose
 * prompt ends in a step samples its first token there, and a finished slot
 * takes the next waiting request.  Request r stops after max_steps
 * generated tokens, at eos (not stored; eos < 0: none) or when max_seq
 * positions are used.
 * out_tokens[r] (capacity max_steps) and out_lens[r] receive its tokens.
 * Returns the total generated (>= 0) or a negative status. */
MM_API long long mm_engine_generate(mm_engine *e, int n_req, const int32_t *const *prompts,
                                    const int32_t *prompt_lens, int max_steps, int eos,
                                    int32_t *const *out_tokens, int32_t *out_lens);

#ifdef __cplusplus
}
#endif
#endif /* MLAMOE_H */
