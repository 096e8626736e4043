/* oracle.c -- scalar CPU restatement of the mla-moe matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP path and
 * the timed CPU baseline, never part of the product.
 *
 * Loop orders, accumulation types and the order of every floating-point
 * operation follow the reference functions cited beside each definition, so
 * that results are bit-identical to the reference compiled with its own
 * flags (-std=c11 -O2; x86-64 baseline has no FMA, and -ffp-contract=off
 * makes that explicit here).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* include/tensor.h:9-14: bf16 -> fp32 is a 16-bit left shift. */
float or_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* include/tensor.h:16-20: fp32 -> bf16 keeps the top 16 bits (truncation). */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

void or_bf16_to_f32_n(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = or_bf16_to_f32(src[i]);
}

void or_f32_to_bf16_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = or_f32_to_bf16(src[i]);
}

/* src/run.c:29-37: y[d] = sum_i x[i]*bf16(W[d,i]); i ascending, fp32
 * accumulator starting at 0, separate multiply and add. */
void or_matmul(float *y, const float *x, const uint16_t *w, int d_out, int n_in) {
    for (int d = 0; d < d_out; d++) {
        const uint16_t *row = w + (size_t)d * n_in;
        float acc = 0.0f;
        for (int i = 0; i < n_in; i++) acc += x[i] * or_bf16_to_f32(row[i]);
        y[d] = acc;
    }
}

void or_matmul_rows(float *y, const float *x, const uint16_t *w, int T, int d_out, int n_in) {
    for (int t = 0; t < T; t++)
        or_matmul(y + (size_t)t * d_out, x + (size_t)t * n_in, w, d_out, n_in);
}

/* src/run.c:22-27 (rmsnorm). */
void or_rmsnorm(float *y, const float *x, const uint16_t *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv * or_bf16_to_f32(w[i]);
}

/* src/run.c:503-508 (sample: greedy argmax). */
int or_argmax(const float *logits, int n) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > bv) {
            bv = logits[i];
            best = i;
        }
    return best;
}

/* src/run.c:493-494 (final rmsnorm + lm_head matmul) followed by sample(). */
void or_lm_head_rows(const float *x, const uint16_t *norm, float eps, const uint16_t *lm_head,
                     int T, int vocab, int hidden, float *logits, int32_t *tokens) {
    float *xb = malloc((size_t)hidden * sizeof(float));
    for (int t = 0; t < T; t++) {
        float *lg = logits + (size_t)t * vocab;
        or_rmsnorm(xb, x + (size_t)t * hidden, norm, hidden, eps);
        or_matmul(lg, xb, lm_head, vocab, hidden);
        tokens[t] = or_argmax(lg, vocab);
    }
    free(xb);
}

/* src/run.c:39 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* src/run.c:85-93: gate, up, silu(gate)*up, down. */
void or_swiglu(float *dst, const float *x, const uint16_t *gate, const uint16_t *up,
               const uint16_t *down, int inter, int hidden, float *hb, float *hb2) {
    or_matmul(hb, x, gate, inter, hidden);
    or_matmul(hb2, x, up, inter, hidden);
    for (int i = 0; i < inter; i++) hb[i] = or_silu(hb[i]) * hb2[i];
    or_matmul(dst, hb, down, hidden, inter);
}

/* src/run.c:95-105: max, exp(x - max) with -inf -> 0, sequential sum, divide. */
void or_softmax(float *x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = (x[i] == -INFINITY) ? 0.0f : expf(x[i] - mx);
        sum += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

/* src/run.c:125-149: scores (sigmoid or softmax), K greedy passes over the
 * unused experts selecting on score+bias with strict '>' (lowest index wins a
 * tie), weight = raw score, optional normalisation seeded with 1e-20, then
 * the routed scaling factor. */
void or_route(const or_moe_cfg *c, float *scores, const float *bias, int *idx, float *w) {
    const int E = c->n_routed_experts, K = c->n_experts_per_tok;
    if (c->router_sigmoid)
        for (int e = 0; e < E; e++) scores[e] = 1.0f / (1.0f + expf(-scores[e]));
    else
        or_softmax(scores, E);
    char used[1024] = {0};
    for (int r = 0; r < K; r++) {
        int best = -1;
        float bv = -INFINITY;
        for (int e = 0; e < E; e++) {
            if (used[e]) continue;
            float sel = scores[e] + (bias ? bias[e] : 0.0f);
            if (sel > bv) { bv = sel; best = e; }
        }
        if (best < 0) best = 0;   /* only reachable with NaN scores */
        used[best] = 1;
        idx[r] = best;
        w[r] = scores[best];
    }
    if (c->norm_topk) {
        float sum = 1e-20f;
        for (int r = 0; r < K; r++) sum += w[r];
        for (int r = 0; r < K; r++) w[r] /= sum;
    }
    for (int r = 0; r < K; r++) w[r] *= c->routed_scaling;
}

/* Shared by the bf16 and int8 paths: router logits for one token
 * (run.c:124) unless they are supplied. */
static void route_token(const or_moe_cfg *c, const uint16_t *moe_gate, const float *bias,
                        const float *xn, const float *logits_in, float *scores,
                        int *idx, float *w) {
    const int E = c->n_routed_experts, H = c->hidden;
    if (logits_in)
        memcpy(scores, logits_in, (size_t)E * sizeof(float));
    else
        or_matmul(scores, xn, moe_gate, E, H);
    or_route(c, scores, bias, idx, w);
}

/* src/run.c:116-162 (MoE branch): route, then for each slot r in order run the
 * expert's SwiGLU and accumulate out += w_r * e, then add the shared expert
 * (one SwiGLU of width n_shared * moe_inter). */
static void ffn_token(const or_moe_cfg *c, const or_moe_weights *wt, const float *xn,
                      const float *logits_in, float *out, int *idx_out, float *w_out,
                      float *probs_out) {
    const int H = c->hidden, I = c->moe_inter_size, K = c->n_experts_per_tok;
    const int S = c->n_shared_experts * I;
    const int maxi = S > I ? S : I;
    float scores[1024];
    int idx[16];
    float w[16];
    route_token(c, wt->moe_gate, wt->moe_gate_bias, xn, logits_in, scores, idx, w);

    float *hb = malloc((size_t)maxi * sizeof(float));
    float *hb2 = malloc((size_t)maxi * sizeof(float));
    float *eo = malloc((size_t)H * sizeof(float));
    for (int i = 0; i < H; i++) out[i] = 0.0f;
    for (int r = 0; r < K; r++) {
        size_t e = (size_t)idx[r];
        or_swiglu(eo, xn, wt->eg + e * I * H, wt->eu + e * I * H, wt->ed + e * H * I, I, H,
                  hb, hb2);
        for (int i = 0; i < H; i++) out[i] += w[r] * eo[i];
    }
    if (S > 0) {
        or_swiglu(eo, xn, wt->sg, wt->su, wt->sd, S, H, hb, hb2);
        for (int i = 0; i < H; i++) out[i] += eo[i];
    }
    free(hb); free(hb2); free(eo);
    if (idx_out)
        for (int r = 0; r < K; r++) { idx_out[r] = idx[r]; w_out[r] = w[r]; }
    if (probs_out) memcpy(probs_out, scores, (size_t)c->n_routed_experts * sizeof(float));
}

void or_ffn_compute(const or_moe_cfg *c, const or_moe_weights *wt, const float *xn,
                    float *out, int *idx, float *w, float *probs) {
    ffn_token(c, wt, xn, NULL, out, idx, w, probs);
}

void or_ffn_compute_rows(const or_moe_cfg *c, const or_moe_weights *wt, int T,
                         const float *xn, const float *logits_in, float *out,
                         int *idx, float *w, float *probs) {
    const int H = c->hidden, E = c->n_routed_experts, K = c->n_experts_per_tok;
    for (int t = 0; t < T; t++)
        ffn_token(c, wt, xn + (size_t)t * H, logits_in ? logits_in + (size_t)t * E : NULL,
                  out + (size_t)t * H, idx ? idx + (size_t)t * K : NULL,
                  w ? w + (size_t)t * K : NULL, probs ? probs + (size_t)t * E : NULL);
}

/* ---- int8 ------------------------------------------------------------ */

void or_quant_row_i8(const float *x, int n, int8_t *q, float *s) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float sc = amax / 127.0f;
    *s = sc;
    for (int i = 0; i < n; i++) {
        if (sc == 0.0f) { q[i] = 0; continue; }
        float v = rintf(x[i] / sc);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q[i] = (int8_t)v;
    }
}

void or_quant_rows_i8(const float *x, int rows, int n, int8_t *q, float *s) {
    for (int r = 0; r < rows; r++)
        or_quant_row_i8(x + (size_t)r * n, n, q + (size_t)r * n, s + r);
}

void or_quant_weight_i8(const uint16_t *w, int N, int K, int8_t *q, float *s) {
    float *row = malloc((size_t)K * sizeof(float));
    for (int n = 0; n < N; n++) {
        or_bf16_to_f32_n(w + (size_t)n * K, row, (size_t)K);
        or_quant_row_i8(row, K, q + (size_t)n * K, s + n);
    }
    free(row);
}

void or_gemm_i8(const int8_t *a, const int8_t *b, int32_t *c, int M, int N, int K) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            const int8_t *ar = a + (size_t)m * K, *br = b + (size_t)n * K;
            int32_t acc = 0;
            for (int k = 0; k < K; k++) acc += (int32_t)ar[k] * (int32_t)br[k];
            c[(size_t)m * N + n] = acc;
        }
}

void or_dequant_row(const int32_t *acc, float sa, const float *sb, int N, float *y) {
    for (int n = 0; n < N; n++) y[n] = ((float)acc[n] * sa) * sb[n];
}

/* One int8 expert on one quantised token: gate/up GEMV (int32), dequantise,
 * SwiGLU as run.c:86-93, quantise the hidden row, down GEMV, dequantise. */
static void expert_i8(const int8_t *qx, float sx, const int8_t *qg, const float *sg,
                      const int8_t *qu, const float *su, const int8_t *qd, const float *sd,
                      int inter, int H, float *y, int32_t *acc_g, int32_t *acc_u,
                      int8_t *qh, float *sh, int32_t *acc_d, float *hb, float *hb2) {
    or_gemm_i8(qx, qg, acc_g, 1, inter, H);
    or_gemm_i8(qx, qu, acc_u, 1, inter, H);
    or_dequant_row(acc_g, sx, sg, inter, hb);
    or_dequant_row(acc_u, sx, su, inter, hb2);
    for (int i = 0; i < inter; i++) hb[i] = or_silu(hb[i]) * hb2[i];
    or_quant_row_i8(hb, inter, qh, sh);
    or_gemm_i8(qh, qd, acc_d, 1, H, inter);
    or_dequant_row(acc_d, *sh, sd, H, y);
}

void or_ffn_i8(const or_moe_cfg *c, const uint16_t *moe_gate, const float *gate_bias,
               const or_moe_i8_weights *wt, int T, const float *xn,
               const float *logits_in, float *out, int *idx_out, float *w_out,
               float *probs, or_i8_debug *dbg) {
    const int H = c->hidden, I = c->moe_inter_size, K = c->n_experts_per_tok;
    const int E = c->n_routed_experts, S = c->n_shared_experts * I;
    const int maxi = S > I ? S : I;
    int8_t *qx = malloc((size_t)H);
    int32_t *ag = malloc((size_t)maxi * sizeof(int32_t));
    int32_t *au = malloc((size_t)maxi * sizeof(int32_t));
    int32_t *ad = malloc((size_t)H * sizeof(int32_t));
    int8_t *qh = malloc((size_t)maxi);
    float *hb = malloc((size_t)maxi * sizeof(float));
    float *hb2 = malloc((size_t)maxi * sizeof(float));
    float *eo = malloc((size_t)H * sizeof(float));
    float scores[1024];
    int idx[16];
    float w[16];
    for (int t = 0; t < T; t++) {
        const float *x = xn + (size_t)t * H;
        float *o = out + (size_t)t * H;
        route_token(c, moe_gate, gate_bias, x, logits_in ? logits_in + (size_t)t * E : NULL,
                    scores, idx, w);
        float sx;
        or_quant_row_i8(x, H, qx, &sx);
        if (dbg && dbg->qx) memcpy(dbg->qx + (size_t)t * H, qx, (size_t)H);
        if (dbg && dbg->sx) dbg->sx[t] = sx;
        for (int i = 0; i < H; i++) o[i] = 0.0f;
        for (int r = 0; r < K; r++) {
            size_t e = (size_t)idx[r];
            float sh;
            expert_i8(qx, sx, wt->qg + e * I * H, wt->sg + e * I, wt->qu + e * I * H,
                      wt->su + e * I, wt->qd + e * H * I, wt->sd + e * H, I, H, eo, ag, au,
                      qh, &sh, ad, hb, hb2);
            size_t route = (size_t)t * K + r;
            if (dbg && dbg->acc_gu) {
                memcpy(dbg->acc_gu + route * 2 * I, ag, (size_t)I * sizeof(int32_t));
                memcpy(dbg->acc_gu + route * 2 * I + I, au, (size_t)I * sizeof(int32_t));
            }
            if (dbg && dbg->qh) memcpy(dbg->qh + route * I, qh, (size_t)I);
            if (dbg && dbg->sh) dbg->sh[route] = sh;
            if (dbg && dbg->acc_d) memcpy(dbg->acc_d + route * H, ad, (size_t)H * sizeof(int32_t));
            for (int i = 0; i < H; i++) o[i] += w[r] * eo[i];
        }
        if (S > 0) {
            float sh;
            expert_i8(qx, sx, wt->qsg, wt->ssg, wt->qsu, wt->ssu, wt->qsd, wt->ssd, S, H, eo,
                      ag, au, qh, &sh, ad, hb, hb2);
            if (dbg && dbg->qhs) memcpy(dbg->qhs + (size_t)t * S, qh, (size_t)S);
            if (dbg && dbg->shs) dbg->shs[t] = sh;
            for (int i = 0; i < H; i++) o[i] += eo[i];
        }
        if (idx_out)
            for (int r = 0; r < K; r++) {
                idx_out[(size_t)t * K + r] = idx[r];
                w_out[(size_t)t * K + r] = w[r];
            }
        if (probs) memcpy(probs + (size_t)t * E, scores, (size_t)E * sizeof(float));
    }
    free(qx); free(ag); free(au); free(ad); free(qh); free(hb); free(hb2); free(eo);
}

/* ---- MLA absorbed decode --------------------------------------------- */

/* src/run.c:430-460 for one head:
 *   qabs[r]  = sum_d q_nope[d] * W_UK[d, r]   (d outer, r inner, :437-442)
 *   score[k] = (qabs . c_kv[k] + q_pe . k_pe[k]) * scale          (:444-451)
 *   softmax(score)                                                (:452)
 *   clat[r]  = sum_k a_k * c_kv[k, r]         (k outer, r inner, :454-459)
 *   ctx      = matmul(clat, W_UV, VHD, KVL)                       (:460)   */
void or_absorbed_head(const float *qnope, const float *qpe, const uint16_t *wuk,
                      const uint16_t *wuv, const float *cache, int kv_len, int QKN,
                      int QKR, int KVL, int VHD, float scale, float *qabs,
                      float *score, float *clat, float *ctx) {
    const int KVD = KVL + QKR;
    for (int r = 0; r < KVL; r++) qabs[r] = 0.0f;
    for (int d = 0; d < QKN; d++) {
        float qd = qnope[d];
        const uint16_t *row = wuk + (size_t)d * KVL;
        for (int r = 0; r < KVL; r++) qabs[r] += qd * or_bf16_to_f32(row[r]);
    }
    for (int k = 0; k < kv_len; k++) {
        const float *ckv = cache + (size_t)k * KVD;
        const float *kpe = ckv + KVL;
        float sn = 0.0f, sp = 0.0f;
        for (int r = 0; r < KVL; r++) sn += qabs[r] * ckv[r];
        for (int d = 0; d < QKR; d++) sp += qpe[d] * kpe[d];
        score[k] = (sn + sp) * scale;
    }
    or_softmax(score, kv_len);
    for (int r = 0; r < KVL; r++) clat[r] = 0.0f;
    for (int k = 0; k < kv_len; k++) {
        float a = score[k];
        const float *ckv = cache + (size_t)k * KVD;
        for (int r = 0; r < KVL; r++) clat[r] += a * ckv[r];
    }
    or_matmul(ctx, clat, wuv, VHD, KVL);
}

/* Per-head W_UK/W_UV live at kv_b + h*(QKN+VHD)*KVL and that + QKN*KVL
 * (head-interleaved split, src/model_load.c:80-86; include/model.h:56-65). */
void or_absorbed_decode(const float *q, const uint16_t *kv_b, const void *cache,
                        int cache_bf16, int B, int NH, int QKN, int QKR, int KVL,
                        int VHD, int kv_len, int seq_stride, float scale, float *ctx,
                        float *qabs, float *probs, float *clat) {
    const int KVD = KVL + QKR, QHD = QKN + QKR;
    const size_t head_stride = (size_t)(QKN + VHD) * KVL;
    float *cf = malloc((size_t)kv_len * KVD * sizeof(float));
    float *qa = malloc((size_t)KVL * sizeof(float));
    float *sc = malloc((size_t)kv_len * sizeof(float));
    float *cl = malloc((size_t)KVL * sizeof(float));
    for (int b = 0; b < B; b++) {
        size_t base = (size_t)b * seq_stride * KVD;
        if (cache_bf16)
            or_bf16_to_f32_n((const uint16_t *)cache + base, cf, (size_t)kv_len * KVD);
        else
            memcpy(cf, (const float *)cache + base, (size_t)kv_len * KVD * sizeof(float));
        for (int h = 0; h < NH; h++) {
            const float *qh = q + ((size_t)b * NH + h) * QHD;
            const uint16_t *wuk = kv_b + (size_t)h * head_stride;
            const uint16_t *wuv = wuk + (size_t)QKN * KVL;
            float *ch = ctx + ((size_t)b * NH + h) * VHD;
            or_absorbed_head(qh, qh + QKN, wuk, wuv, cf, kv_len, QKN, QKR, KVL, VHD, scale,
                             qa, sc, cl, ch);
            size_t bh = (size_t)b * NH + h;
            if (qabs) memcpy(qabs + bh * KVL, qa, (size_t)KVL * sizeof(float));
            if (probs) memcpy(probs + bh * kv_len, sc, (size_t)kv_len * sizeof(float));
            if (clat) memcpy(clat + bh * KVL, cl, (size_t)KVL * sizeof(float));
        }
    }
    free(cf); free(qa); free(sc); free(cl);
}

/* ---- MLA decode front -------------------------------------------------- */

/* src/model_load.c:299-325, step for step (float arithmetic throughout,
 * left-to-right products as written there). */
void or_rope_inv_freq(int dim, float theta, float factor, float beta_fast, float beta_slow,
                      float orig_max, float *inv) {
    const int half = dim / 2;
    const float pi = 3.14159265358979323846f;
    const float lo_d = ((float)dim * logf(orig_max / (beta_fast * 2.0f * pi))) / (2.0f * logf(theta));
    const float hi_d = ((float)dim * logf(orig_max / (beta_slow * 2.0f * pi))) / (2.0f * logf(theta));
    float low = floorf(lo_d), high = ceilf(hi_d);
    if (low < 0) low = 0;
    if (high > dim - 1) high = (float)(dim - 1);
    const float denom = high == low ? 0.001f : high - low;
    for (int j = 0; j < half; j++) {
        const float extra = 1.0f / powf(theta, (float)(2 * j) / (float)dim);
        const float inter = extra / factor;
        float ramp = ((float)j - low) / denom;
        ramp = ramp < 0 ? 0 : ramp > 1 ? 1 : ramp;
        const float keep = 1.0f - ramp;
        inv[j] = inter * (1.0f - keep) + extra * keep;
    }
}

/* src/run.c:47-67 */
void or_rope_apply(float *v, int pos, const float *inv, int dim, int interleaved) {
    const int half = dim / 2;
    float tmp[512];
    for (int j = 0; j < half; j++) {
        const float ang = (float)pos * inv[j];
        const float c = cosf(ang), s = sinf(ang);
        const float a = v[2 * j], b = v[2 * j + 1];
        if (interleaved) {
            tmp[j] = a * c - b * s;
            tmp[half + j] = b * c + a * s;
        } else {
            v[2 * j] = a * c - b * s;
            v[2 * j + 1] = a * s + b * c;
        }
    }
    if (interleaved) memcpy(v, tmp, (size_t)dim * sizeof(float));
}

/* src/run.c:418-428 with project_q (run.c:73-83) */
void or_mla_front(const or_front_cfg *c, const or_front_weights *w, const float *inv,
                  const float *x, int pos, float *q, float *kv, float *comp) {
    const int H = c->hidden, QHD = c->qk_nope + c->qk_rope, QD = c->n_heads * QHD;
    const int KVD = c->kv_lora + c->qk_rope;
    float *xb = malloc((size_t)H * sizeof(float));
    float *cp = malloc((size_t)KVD * sizeof(float));
    or_rmsnorm(xb, x, w->in_norm, H, c->rms_eps);
    if (c->q_lora > 0) {
        float *qa = malloc((size_t)c->q_lora * sizeof(float));
        or_matmul(qa, xb, w->q_a_proj, c->q_lora, H);
        or_rmsnorm(qa, qa, w->q_a_norm, c->q_lora, c->mla_eps);
        or_matmul(q, qa, w->q_b_proj, QD, c->q_lora);
        free(qa);
    } else {
        or_matmul(q, xb, w->q_proj, QD, H);
    }
    for (int h = 0; h < c->n_heads; h++)
        or_rope_apply(q + (size_t)h * QHD + c->qk_nope, pos, inv, c->qk_rope, c->interleaved);
    or_matmul(cp, xb, w->kv_a, KVD, H);
    if (comp) memcpy(comp, cp, (size_t)KVD * sizeof(float));
    or_rmsnorm(kv, cp, w->kv_a_norm, c->kv_lora, c->mla_eps);
    memcpy(kv + c->kv_lora, cp + c->kv_lora, (size_t)c->qk_rope * sizeof(float));
    or_rope_apply(kv + c->kv_lora, pos, inv, c->qk_rope, c->interleaved);
    free(xb);
    free(cp);
}
