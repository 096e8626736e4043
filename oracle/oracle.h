/* oracle.h -- CPU oracle for the mla-moe matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker (or as the timed CPU
 * baseline), never as a fallback for the GPU path.
 *
 * Every function restates the reference algorithm in plain scalar C11 and
 * cites the reference file:line it follows (paths relative to the reference
 * repository root).  Build flags: -std=c11 -O2 -ffp-contract=off, i.e. the
 * reference's own C flags plus an explicit "no FMA contraction" so the
 * restatement rounds exactly like the reference on any x86-64 host.
 *
 * Parity pinning (how each function is checked, see tests/test_oracle_*.py):
 *   - bf16 conversions, or_matmul, or_silu, or_swiglu, or_softmax, or_route,
 *     or_ffn_compute, or_absorbed_*, or_rmsnorm, or_argmax: bit-exact against
 *     golden vectors written
 *     by the reference's own compiled run.c (tests/golden/), against
 *     oracle/_ref/libref.so where it is built, and against closed forms
 *     (integer-valued operands, one-hot weights, equal logits, kv_len == 1).
 *   - int8 pieces (or_quant_*, or_gemm_i8, or_ffn_i8): the reference has no
 *     int8 path; they are pinned by closed forms (exact integer dot products
 *     compared against numpy int64 matmul and against or_matmul on
 *     integer-valued operands, quantiser invariants, and reduction to
 *     or_ffn_compute when every operand is exactly representable).
 */
#ifndef MLAMOE_ORACLE_H
#define MLAMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 storage (include/tensor.h:7-20) ---------------------------- */
float    or_bf16_to_f32(uint16_t v);
uint16_t or_f32_to_bf16(float f);               /* truncation, no rounding */
void     or_bf16_to_f32_n(const uint16_t *src, float *dst, size_t n);
void     or_f32_to_bf16_n(const float *src, uint16_t *dst, size_t n);

/* ---- dense math (src/run.c:29-105) ----------------------------------- */
void  or_matmul(float *y, const float *x, const uint16_t *w, int d_out, int n_in);
/* T independent rows: y[t] = matmul(x[t]) (the reference calls matmul once
 * per position, run.c:293-311). */
void  or_matmul_rows(float *y, const float *x, const uint16_t *w, int T, int d_out, int n_in);
float or_silu(float x);
void  or_swiglu(float *dst, const float *x, const uint16_t *gate, const uint16_t *up,
                const uint16_t *down, int inter, int hidden, float *hb, float *hb2);
void  or_softmax(float *x, int n);

/* ---- LM head (src/run.c:22-27, 493-494, 503-508) ---------------------- */
/* y = (x / rms(x)) * w over n elements: sequential sum of squares, one
 * 1/sqrtf(ss/n + eps), then (x[i] * inv) * w[i]. */
void  or_rmsnorm(float *y, const float *x, const uint16_t *w, int n, float eps);
/* greedy argmax: the first index of the maximum under a strict '>' scan
 * from index 0 (a NaN never wins; logits[0] = NaN selects 0). */
int   or_argmax(const float *logits, int n);
/* T tokens: xb = rmsnorm(x[t]), logits[t] = matmul(xb), tokens[t] = argmax. */
void  or_lm_head_rows(const float *x, const uint16_t *norm, float eps, const uint16_t *lm_head,
                      int T, int vocab, int hidden, float *logits, int32_t *tokens);

/* ---- MoE FFN (src/run.c:107-162) ------------------------------------- */
/* Mirrors the MoE fields of Config (include/model.h:12-42). */
typedef struct {
    int   hidden;              /* H */
    int   n_routed_experts;    /* E */
    int   n_shared_experts;
    int   n_experts_per_tok;   /* K */
    int   moe_inter_size;      /* I */
    int   router_sigmoid;      /* 0: softmax (dsv2), 1: sigmoid (GLM noaux_tc) */
    int   norm_topk;
    float routed_scaling;
} or_moe_cfg;

/* bf16 MoE layer weights, contiguous per family (ModelWeights
 * include/model.h:84-96 keeps one pointer per expert; here expert e of the
 * gate family starts at eg + e*I*H). */
typedef struct {
    const uint16_t *moe_gate;      /* [E, H] */
    const float    *moe_gate_bias; /* [E] or NULL */
    const uint16_t *eg, *eu;       /* [E, I, H] */
    const uint16_t *ed;            /* [E, H, I] */
    const uint16_t *sg, *su;       /* [S, H], S = n_shared*I */
    const uint16_t *sd;            /* [H, S] */
} or_moe_weights;

/* Router on one token (run.c:124-150).  `scores` holds the E logits on
 * entry and the softmax/sigmoid scores on return (as s->moe_logits does). */
void or_route(const or_moe_cfg *c, float *scores, const float *bias,
              int *idx, float *w);
/* One token's MoE FFN (run.c:116-162); out is overwritten.  probs (E floats),
 * idx/w (K each) may be NULL. */
void or_ffn_compute(const or_moe_cfg *c, const or_moe_weights *wt, const float *xn,
                    float *out, int *idx, float *w, float *probs);
/* T tokens, each as or_ffn_compute (the prefill FFN loop, run.c:291-313).
 * If logits_in != NULL the router GEMV is skipped and row t of logits_in is
 * routed instead (batched-decode configuration). */
void or_ffn_compute_rows(const or_moe_cfg *c, const or_moe_weights *wt, int T,
                         const float *xn, const float *logits_in, float *out,
                         int *idx, float *w, float *probs);

/* ---- int8 path (no reference counterpart; see header comment) -------- */
/* s = max|x| / 127; q[i] = clamp(rint(x[i] / s), -127, 127); s == 0 -> q = 0 */
void or_quant_row_i8(const float *x, int n, int8_t *q, float *s);
void or_quant_rows_i8(const float *x, int rows, int n, int8_t *q, float *s);
/* per-output-channel weight quantisation of a bf16 [N, K] matrix */
void or_quant_weight_i8(const uint16_t *w, int N, int K, int8_t *q, float *s);
/* c[m, n] = sum_k a[m, k] * b[n, k]   (int32, exact: |c| < 2^31 for K <= 2^17) */
void or_gemm_i8(const int8_t *a, const int8_t *b, int32_t *c, int M, int N, int K);
/* dequantised row: y[n] = ((float)acc[n] * sa) * sb[n] */
void or_dequant_row(const int32_t *acc, float sa, const float *sb, int N, float *y);

typedef struct {
    const int8_t *qg, *qu;  const float *sg, *su;   /* routed gate/up [E, I, H], scales [E, I] */
    const int8_t *qd;       const float *sd;        /* routed down [E, H, I], scales [E, H] */
    const int8_t *qsg, *qsu; const float *ssg, *ssu;/* shared gate/up [S, H], scales [S] */
    const int8_t *qsd;      const float *ssd;       /* shared down [H, S], scales [H] */
} or_moe_i8_weights;

/* Optional intermediates of or_ffn_i8 (any member may be NULL):
 *   qx [T,H], sx [T]              per-token quantised activations
 *   acc_gu [T,K,2,I]              int32 gate/up accumulators per route
 *   qh [T,K,I], sh [T,K]          per-route quantised SwiGLU output
 *   acc_d [T,K,H]                 int32 down accumulators per route
 *   qhs [T,S], shs [T]            shared expert quantised hidden
 */
typedef struct {
    int8_t  *qx;  float *sx;
    int32_t *acc_gu;
    int8_t  *qh;  float *sh;
    int32_t *acc_d;
    int8_t  *qhs; float *shs;
} or_i8_debug;

/* T tokens through the int8 MoE layer.  Routing is the reference router on
 * the fp32 input (or on logits_in when given), exactly as or_ffn_compute;
 * experts run as: quantise x per token -> int8 gate/up GEMM (int32 acc) ->
 * dequantise -> SwiGLU (run.c:39, 86-93) -> quantise h per route -> int8 down
 * GEMM -> dequantise -> combine in slot order then shared (run.c:151-160). */
void or_ffn_i8(const or_moe_cfg *c, const uint16_t *moe_gate, const float *gate_bias,
               const or_moe_i8_weights *wt, int T, const float *xn,
               const float *logits_in, float *out, int *idx, float *w,
               float *probs, or_i8_debug *dbg);

/* ---- MLA absorbed decode (src/run.c:430-460) ------------------------- */
/* One (sequence, head).  wuk: [QKN, KVL], wuv: [VHD, KVL] (bf16 head slices of
 * kv_b, model_load.c:80-86).  cache: kv_len rows of KVL+QKR fp32.  Writes
 * qabs[KVL], score[kv_len] (the softmax probabilities), clat[KVL], ctx[VHD]. */
void or_absorbed_head(const float *qnope, const float *qpe, const uint16_t *wuk,
                      const uint16_t *wuv, const float *cache, int kv_len, int QKN,
                      int QKR, int KVL, int VHD, float scale, float *qabs,
                      float *score, float *clat, float *ctx);

/* B sequences x NH heads.  q: [B, NH, QKN+QKR] (RoPE applied).  kv_b: bf16
 * [NH*(QKN+VHD), KVL], head-interleaved.  cache: B sequences of `seq_stride`
 * rows (>= kv_len) of KVL+QKR values, bf16 when cache_bf16 != 0 (then it is a
 * uint16_t array) else fp32.  Outputs (any of the last three may be NULL):
 * ctx [B, NH*VHD], qabs [B, NH, KVL], probs [B, NH, kv_len], clat [B, NH, KVL]. */
void or_absorbed_decode(const float *q, const uint16_t *kv_b, const void *cache,
                        int cache_bf16, int B, int NH, int QKN, int QKR, int KVL,
                        int VHD, int kv_len, int seq_stride, float scale, float *ctx,
                        float *qabs, float *probs, float *clat);

/* ---- MLA decode front: norms, projections, RoPE, latent-cache row ----- */
/* DeepSeek-V2 YaRN inverse frequencies (src/model_load.c:299-325): inv[j]
 * for j < dim/2 blends 1/theta^(2j/dim) (extrapolated) and that / factor
 * (interpolated) by a ramp over the correction range set by beta_fast /
 * beta_slow and orig_max.  factor == 1 gives plain RoPE. */
void or_rope_inv_freq(int dim, float theta, float factor, float beta_fast, float beta_slow,
                      float orig_max, float *inv);
/* In-place RoPE of a dim-long slice at `pos` (src/run.c:47-67): angle
 * pos * inv[j]; interleaved == 0 rotates (v[2j], v[2j+1]) in place,
 * interleaved == 1 writes the rotated evens then the rotated odds. */
void or_rope_apply(float *v, int pos, const float *inv, int dim, int interleaved);

/* The attention fields of Config the decode front needs. */
typedef struct {
    int   hidden;        /* H */
    int   n_heads;       /* NH */
    int   qk_nope;       /* QKN */
    int   qk_rope;       /* QKR */
    int   kv_lora;       /* KVL */
    int   q_lora;        /* 0: q_proj; > 0: q_a_proj -> q_a_layernorm -> q_b_proj */
    float rms_eps;       /* input_layernorm */
    float mla_eps;       /* q_a / kv_a layernorms (model_load.c:269) */
    int   interleaved;   /* RoPE layout */
} or_front_cfg;

typedef struct {
    const uint16_t *in_norm;     /* [H] */
    const uint16_t *q_proj;      /* [NH*(QKN+QKR), H]   (q_lora == 0) */
    const uint16_t *q_a_proj;    /* [q_lora, H]          (q_lora > 0) */
    const uint16_t *q_a_norm;    /* [q_lora] */
    const uint16_t *q_b_proj;    /* [NH*(QKN+QKR), q_lora] */
    const uint16_t *kv_a;        /* [KVL+QKR, H] */
    const uint16_t *kv_a_norm;   /* [KVL] */
} or_front_weights;

/* One token of forward_absorbed up to the latent-cache append
 * (src/run.c:418-428, project_q run.c:73-83): xb = rmsnorm(x); q =
 * project_q(xb) with RoPE on each head's q_pe; comp = kv_a . xb; kv =
 * rmsnorm(comp[:KVL], kv_a_norm, mla_eps) | rope(comp[KVL:]).  q is
 * [NH*(QKN+QKR)], kv [KVL+QKR] (the cache row); comp [KVL+QKR] may be NULL. */
void or_mla_front(const or_front_cfg *c, const or_front_weights *w, const float *inv,
                  const float *x, int pos, float *q, float *kv, float *comp);

#ifdef __cplusplus
}
#endif
#endif /* MLAMOE_ORACLE_H */
