/* ref_harness.c -- expose the reference's own hot-path functions for
 * golden-vector generation and oracle cross-checks.
 *
 * TEST INFRASTRUCTURE ONLY.  This file contains no reference code.  It is
 * compiled by oracle/Makefile (target `ref`) with -I pointing at
 * /root/reference/src and /root/reference/include. That makes the
 * `#include "run.c"` below pull in the reference's src/run.c from where it
 * lies, unmodified, and that is the only way to reach its `static`
 * functions (matmul, swiglu, softmax, rmsnorm, ffn_compute). `main` is renamed to an
 * unused static function on the command line, so the library needs nothing
 * beyond libc/libm and the reference's src/dump.c.  The output goes only to
 * oracle/_ref/ (git-ignored).
 */
#include "run.c"

#include <stdint.h>

void ref_matmul(float *y, const float *x, const uint16_t *w, int d_out, int n_in) {
    matmul(y, x, w, d_out, n_in);
}

float ref_silu(float x) { return silu(x); }

void ref_softmax(float *x, int n) { softmax(x, n); }

void ref_rmsnorm(float *y, const float *x, const uint16_t *w, int n, float eps) {
    rmsnorm(y, x, w, n, eps);
}

int ref_sample(float *logits, int n) { return sample(logits, n); }

void ref_swiglu(float *dst, const float *x, const uint16_t *gate, const uint16_t *up,
                const uint16_t *down, int inter, int hidden, float *hb, float *hb2) {
    swiglu(dst, x, gate, up, down, inter, hidden, hb, hb2);
}

/* One token through the reference ffn_compute (run.c:116-162) on layer 0 of a
 * one-layer MoE model whose expert weights are contiguous [E, I, H] / [E, H, I]
 * blocks.  probs receives s->moe_logits (the router scores) after the call. */
void ref_ffn_compute(int H, int E, int n_shared, int K, int I, int router_sigmoid,
                     int norm_topk, float routed_scaling, const uint16_t *moe_gate,
                     const float *bias, const uint16_t *eg, const uint16_t *eu,
                     const uint16_t *ed, const uint16_t *sg, const uint16_t *su,
                     const uint16_t *sd, const float *xn, float *out, int *idx, float *w,
                     float *probs) {
    Config c;
    memset(&c, 0, sizeof(c));
    c.n_layers = 1;
    c.hidden_size = H;
    c.first_k_dense = 0;
    c.n_routed_experts = E;
    c.n_shared_experts = n_shared;
    c.n_experts_per_tok = K;
    c.moe_inter_size = I;
    c.router_sigmoid = router_sigmoid;
    c.norm_topk = norm_topk;
    c.routed_scaling = routed_scaling;

    int S = n_shared * I, maxi = S > I ? S : I;
    ModelWeights mw;
    memset(&mw, 0, sizeof(mw));
    bf16_t *gate_p[1] = {(bf16_t *)moe_gate};
    float *bias_p[1] = {(float *)bias};
    bf16_t **egp = malloc((size_t)E * sizeof(bf16_t *));
    bf16_t **eup = malloc((size_t)E * sizeof(bf16_t *));
    bf16_t **edp = malloc((size_t)E * sizeof(bf16_t *));
    for (int e = 0; e < E; e++) {
        egp[e] = (bf16_t *)eg + (size_t)e * I * H;
        eup[e] = (bf16_t *)eu + (size_t)e * I * H;
        edp[e] = (bf16_t *)ed + (size_t)e * H * I;
    }
    bf16_t **eg_l[1] = {egp}, **eu_l[1] = {eup}, **ed_l[1] = {edp};
    bf16_t *sg_p[1] = {(bf16_t *)sg}, *su_p[1] = {(bf16_t *)su}, *sd_p[1] = {(bf16_t *)sd};
    mw.moe_gate = gate_p;
    mw.moe_gate_bias = bias_p;
    mw.expert_gate = eg_l;
    mw.expert_up = eu_l;
    mw.expert_down = ed_l;
    mw.shared_gate = sg_p;
    mw.shared_up = su_p;
    mw.shared_down = sd_p;

    RunState s;
    memset(&s, 0, sizeof(s));
    s.moe_logits = malloc((size_t)E * sizeof(float));
    s.expert_out = malloc((size_t)H * sizeof(float));
    s.hb = malloc((size_t)maxi * sizeof(float));
    s.hb2 = malloc((size_t)maxi * sizeof(float));

    ffn_compute(&c, &mw, &s, 0, xn, out, idx, w);
    if (probs) memcpy(probs, s.moe_logits, (size_t)E * sizeof(float));

    free(s.moe_logits); free(s.expert_out); free(s.hb); free(s.hb2);
    free(egp); free(eup); free(edp);
}

/* Drive the reference forward_absorbed (run.c:379-501) on a one-layer,
 * dense-FFN (first_k_dense = 1) model at position `pos`, with the layer-0
 * dumps written to dump_dir (reference build with -DMLA_ENABLE_DUMP).  The
 * latent cache rows [0, pos) are taken from `cache_in` ([pos][KVL+QKR] fp32);
 * row pos is produced by the reference itself.  Before the call, q_out
 * receives the post-RoPE query of every head, computed with the reference's
 * own rmsnorm/project_q/rope_apply exactly as forward_absorbed does
 * (run.c:418-421), because the dumps do not include q. */
int ref_absorbed_decode_ex(int NH, int QKN, int QKR, int KVL, int VHD, int H, int dense_inter,
                           int vocab, int pos, float rms_eps, const float *inv_freq,
                           int q_lora, int interleaved, const uint16_t *q_a_proj,
                           const uint16_t *q_a_norm, const uint16_t *q_b_proj,
                           const uint16_t *embed, const uint16_t *in_norm, const uint16_t *q_proj,
                           const uint16_t *kv_a, const uint16_t *kv_a_norm, const uint16_t *kv_b,
                           const uint16_t *o_proj, const uint16_t *post_norm,
                           const uint16_t *dgate, const uint16_t *dup, const uint16_t *ddown,
                           const uint16_t *final_norm, const uint16_t *lm_head,
                           const float *cache_in, const char *dump_dir, float *q_out) {
    const int KVD = KVL + QKR, QHD = QKN + QKR;
    Transformer t;
    memset(&t, 0, sizeof(t));
    Config *c = &t.config;
    c->n_layers = 1;
    c->hidden_size = H;
    c->n_heads = NH;
    c->n_kv_heads = NH;
    c->q_lora_rank = q_lora;
    c->first_k_dense = 1;
    c->kv_lora_rank = KVL;
    c->qk_rope_head_dim = QKR;
    c->qk_nope_head_dim = QKN;
    c->v_head_dim = VHD;
    c->dense_inter_size = dense_inter;
    c->vocab_size = vocab;
    c->max_seq_len = pos + 1;
    c->rms_eps = rms_eps;
    c->mla_norm_eps = 1e-6f;                             /* model_load.c:269 */
    c->softmax_scale = 1.0f / sqrtf((float)(QKN + QKR)); /* model_load.c:270 */
    c->rope_interleaved = interleaved;

    ModelWeights *w = &t.weights;
    bf16_t *qp[1] = {(bf16_t *)q_proj};
    bf16_t *qa[1] = {(bf16_t *)q_a_proj}, *qan[1] = {(bf16_t *)q_a_norm};
    bf16_t *qb[1] = {(bf16_t *)q_b_proj};
    bf16_t *kva[1] = {(bf16_t *)kv_a}, *kvan[1] = {(bf16_t *)kv_a_norm};
    bf16_t *wuk[1] = {(bf16_t *)kv_b};
    bf16_t *wuv[1] = {(bf16_t *)kv_b + (size_t)QKN * KVL};   /* model_load.c:80-86 */
    bf16_t *op[1] = {(bf16_t *)o_proj}, *inn[1] = {(bf16_t *)in_norm};
    bf16_t *pn[1] = {(bf16_t *)post_norm};
    bf16_t *dg[1] = {(bf16_t *)dgate}, *du[1] = {(bf16_t *)dup}, *dd[1] = {(bf16_t *)ddown};
    w->embed_tokens = (bf16_t *)embed;
    w->q_proj = qp;
    w->q_a_proj = qa;
    w->q_b_proj = qb;
    w->q_a_layernorm = qan;
    w->kv_a_proj = kva;
    w->kv_a_layernorm = kvan;
    w->W_UK = wuk;
    w->W_UV = wuv;
    w->o_proj = op;
    w->input_layernorm = inn;
    w->post_attn_norm = pn;
    w->dense_gate = dg;
    w->dense_up = du;
    w->dense_down = dd;
    w->norm = (bf16_t *)final_norm;
    w->lm_head = (bf16_t *)lm_head;

    RunState *s = &t.state;
    s->kv_cache = calloc((size_t)(pos + 1) * KVD, sizeof(float));
    memcpy(s->kv_cache, cache_in, (size_t)pos * KVD * sizeof(float));
    s->hb = malloc((size_t)dense_inter * sizeof(float));
    s->hb2 = malloc((size_t)dense_inter * sizeof(float));
    s->logits = malloc((size_t)vocab * sizeof(float));
    s->q_a = q_lora > 0 ? malloc((size_t)q_lora * sizeof(float)) : NULL;
    t.rope_inv_freq = (float *)inv_freq;

    /* q for token 0 at `pos`, as forward_absorbed computes it (run.c:414-421). */
    float *x = malloc((size_t)H * sizeof(float));
    float *xb = malloc((size_t)H * sizeof(float));
    for (int i = 0; i < H; i++) x[i] = bf16_to_f32(w->embed_tokens[i]);
    rmsnorm(xb, x, w->input_layernorm[0], H, c->rms_eps);
    project_q(c, w, s, 0, xb, q_out);
    for (int h = 0; h < NH; h++)
        rope_apply(&q_out[(size_t)h * QHD + QKN], pos, inv_freq, QKR, c->rope_interleaved);
    free(x);
    free(xb);

    run_set_dump(dump_dir);
    forward_absorbed(&t, 0, pos);
    run_set_dump(NULL);

    free(s->kv_cache); free(s->hb); free(s->hb2); free(s->logits); free(s->q_a);
    return 0;
}

/* The dsv2 form: single q_proj, adjacent-pair RoPE. */
int ref_absorbed_decode(int NH, int QKN, int QKR, int KVL, int VHD, int H, int dense_inter,
                        int vocab, int pos, float rms_eps, const float *inv_freq,
                        const uint16_t *embed, const uint16_t *in_norm, const uint16_t *q_proj,
                        const uint16_t *kv_a, const uint16_t *kv_a_norm, const uint16_t *kv_b,
                        const uint16_t *o_proj, const uint16_t *post_norm,
                        const uint16_t *dgate, const uint16_t *dup, const uint16_t *ddown,
                        const uint16_t *final_norm, const uint16_t *lm_head,
                        const float *cache_in, const char *dump_dir, float *q_out) {
    return ref_absorbed_decode_ex(NH, QKN, QKR, KVL, VHD, H, dense_inter, vocab, pos, rms_eps,
                                  inv_freq, 0, 0, NULL, NULL, NULL, embed, in_norm, q_proj, kv_a,
                                  kv_a_norm, kv_b, o_proj, post_norm, dgate, dup, ddown,
                                  final_norm, lm_head, cache_in, dump_dir, q_out);
}

void ref_rope_apply(float *v, int pos, const float *inv_freq, int rope_dim, int interleaved) {
    rope_apply(v, pos, inv_freq, rope_dim, interleaved);
}
