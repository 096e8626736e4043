/* ref_model.c -- expose the reference's config parsing and RoPE frequency
 * table for golden-vector generation.
 *
 * TEST INFRASTRUCTURE ONLY.  This file contains no reference code.  Like
 * ref_harness.c it is compiled by oracle/Makefile (target `ref`) with -I at
 * /root/reference/src, so the `#include "model_load.c"` below pulls in the
 * reference's src/model_load.c from where it lies, unmodified: the only way
 * to reach its `static` config_from_json (model_load.c:242-292) and
 * build_rope_inv_freq (model_load.c:299-325).  It links against the
 * reference's own vendor/cJSON.c, src/safetensors_loader.c and src/tensor.c;
 * the output goes only to oracle/_ref/ (git-ignored).
 */
#include "model_load.c"

/* Parse <model_dir>/config.json as the engine does and build its RoPE
 * inverse-frequency table.  ints[] receives qk_rope_head_dim,
 * rope_interleaved, q_lora_rank, n_heads, qk_nope_head_dim, kv_lora_rank,
 * v_head_dim, hidden_size; flts[] receives rms_eps, mla_norm_eps,
 * softmax_scale, rope_theta, rope_factor, rope_beta_fast, rope_beta_slow,
 * rope_orig_max.  inv must hold qk_rope_head_dim / 2 floats. */
int ref_config_rope(const char *model_dir, float *inv, int *ints, float *flts) {
    Config c = config_from_json(model_dir);
    float *f = build_rope_inv_freq(&c);
    memcpy(inv, f, (size_t)(c.qk_rope_head_dim / 2) * sizeof(float));
    free(f);
    const int iv[8] = {c.qk_rope_head_dim, c.rope_interleaved, c.q_lora_rank, c.n_heads,
                       c.qk_nope_head_dim, c.kv_lora_rank, c.v_head_dim, c.hidden_size};
    const float fv[8] = {c.rms_eps, c.mla_norm_eps, c.softmax_scale, c.rope_theta,
                         c.rope_factor, c.rope_beta_fast, c.rope_beta_slow, c.rope_orig_max};
    memcpy(ints, iv, sizeof(iv));
    memcpy(flts, fv, sizeof(fv));
    return 0;
}

#include "dump.h"
#include "engine.h"

/* A small model for whole-step golden vectors: n_layers layers, the first
 * first_k_dense of them dense, the rest MoE (experts contiguous per layer:
 * eg/eu [E, I, H], ed [E, H, I]); q_proj, or with q_lora > 0 the q-LoRA
 * chain; RoPE layout `interleaved`.  Pointer arrays are indexed by layer
 * (NULL where a layer has no such tensor). */
typedef struct {
    int n_layers, first_k_dense, H, NH, QKN, QKR, KVL, VHD, dense_inter, E, n_shared, K, I,
        vocab, router_sigmoid, norm_topk, max_seq, q_lora, interleaved;
    float routed_scaling, rms_eps;
    const float *inv_freq;
    const uint16_t *embed, *final_norm, *lm_head;
    const uint16_t *const *in_norm, *const *q_proj, *const *kv_a, *const *kv_a_norm,
        *const *kv_b, *const *o_proj, *const *post_norm, *const *dgate, *const *dup,
        *const *ddown, *const *moe_gate, *const *eg, *const *eu, *const *ed, *const *sg,
        *const *su, *const *sd, *const *q_a_proj, *const *q_a_norm, *const *q_b_proj;
    const float *const *moe_bias;
} ref_model_spec;

/* A Transformer over the spec's arrays (borrowed), run state allocated. */
static void ref_build(const ref_model_spec *m, Transformer *t) {
    memset(t, 0, sizeof(*t));
    Config *c = &t->config;
    const int L = m->n_layers;
    c->n_layers = L;
    c->hidden_size = m->H;
    c->n_heads = c->n_kv_heads = m->NH;
    c->first_k_dense = m->first_k_dense;
    c->kv_lora_rank = m->KVL;
    c->qk_rope_head_dim = m->QKR;
    c->qk_nope_head_dim = m->QKN;
    c->v_head_dim = m->VHD;
    c->n_routed_experts = m->E;
    c->n_shared_experts = m->n_shared;
    c->n_experts_per_tok = m->K;
    c->dense_inter_size = m->dense_inter;
    c->moe_inter_size = m->I;
    c->vocab_size = m->vocab;
    c->max_seq_len = m->max_seq;
    c->rms_eps = m->rms_eps;
    c->mla_norm_eps = 1e-6f;
    c->softmax_scale = 1.0f / sqrtf((float)(m->QKN + m->QKR));
    c->router_sigmoid = m->router_sigmoid;
    c->norm_topk = m->norm_topk;
    c->routed_scaling = m->routed_scaling;
    c->q_lora_rank = m->q_lora;
    c->rope_interleaved = m->interleaved;
    ModelWeights *w = &t->weights;
#define PA(field) w->field = calloc((size_t)L, sizeof(*w->field))
    PA(q_proj); PA(q_a_proj); PA(q_b_proj); PA(kv_a_proj); PA(W_UK); PA(W_UV); PA(o_proj);
    PA(input_layernorm); PA(post_attn_norm); PA(q_a_layernorm); PA(kv_a_layernorm);
    PA(dense_gate); PA(dense_up); PA(dense_down); PA(moe_gate); PA(moe_gate_bias);
    PA(expert_gate); PA(expert_up); PA(expert_down); PA(shared_gate); PA(shared_up); PA(shared_down);
#undef PA
    w->embed_tokens = (bf16_t *)m->embed;
    w->norm = (bf16_t *)m->final_norm;
    w->lm_head = (bf16_t *)m->lm_head;
    const size_t ne = (size_t)m->I * m->H;
    for (int l = 0; l < L; l++) {
        w->q_proj[l] = m->q_proj ? (bf16_t *)m->q_proj[l] : NULL;
        if (m->q_lora > 0) {
            w->q_a_proj[l] = (bf16_t *)m->q_a_proj[l];
            w->q_a_layernorm[l] = (bf16_t *)m->q_a_norm[l];
            w->q_b_proj[l] = (bf16_t *)m->q_b_proj[l];
        }
        w->kv_a_proj[l] = (bf16_t *)m->kv_a[l];
        w->kv_a_layernorm[l] = (bf16_t *)m->kv_a_norm[l];
        w->W_UK[l] = (bf16_t *)m->kv_b[l];                              /* model_load.c:80-86 */
        w->W_UV[l] = (bf16_t *)m->kv_b[l] + (size_t)m->QKN * m->KVL;
        w->o_proj[l] = (bf16_t *)m->o_proj[l];
        w->input_layernorm[l] = (bf16_t *)m->in_norm[l];
        w->post_attn_norm[l] = (bf16_t *)m->post_norm[l];
        if (l < m->first_k_dense) {
            w->dense_gate[l] = (bf16_t *)m->dgate[l];
            w->dense_up[l] = (bf16_t *)m->dup[l];
            w->dense_down[l] = (bf16_t *)m->ddown[l];
            continue;
        }
        w->moe_gate[l] = (bf16_t *)m->moe_gate[l];
        w->moe_gate_bias[l] = m->moe_bias ? (float *)m->moe_bias[l] : NULL;
        w->expert_gate[l] = malloc((size_t)m->E * sizeof(bf16_t *));
        w->expert_up[l] = malloc((size_t)m->E * sizeof(bf16_t *));
        w->expert_down[l] = malloc((size_t)m->E * sizeof(bf16_t *));
        for (int e = 0; e < m->E; e++) {
            w->expert_gate[l][e] = (bf16_t *)m->eg[l] + e * ne;
            w->expert_up[l][e] = (bf16_t *)m->eu[l] + e * ne;
            w->expert_down[l][e] = (bf16_t *)m->ed[l] + e * ne;
        }
        w->shared_gate[l] = (bf16_t *)m->sg[l];
        w->shared_up[l] = (bf16_t *)m->su[l];
        w->shared_down[l] = (bf16_t *)m->sd[l];
    }
    /* the RoPE table stays the caller's */
    t->rope_inv_freq = (float *)m->inv_freq;
    malloc_run_state(&t->state, c);
}

static void ref_release(Transformer *t) {
    ModelWeights *w = &t->weights;
    free_run_state(&t->state);
    for (int l = 0; l < t->config.n_layers; l++) {
        free(w->expert_gate[l]); free(w->expert_up[l]); free(w->expert_down[l]);
    }
    void *arrs[] = {w->q_proj, w->q_a_proj, w->q_b_proj, w->kv_a_proj, w->W_UK, w->W_UV, w->o_proj,
                    w->input_layernorm, w->post_attn_norm, w->q_a_layernorm, w->kv_a_layernorm,
                    w->dense_gate, w->dense_up, w->dense_down, w->moe_gate, w->moe_gate_bias,
                    w->expert_gate, w->expert_up, w->expert_down, w->shared_gate, w->shared_up,
                    w->shared_down};
    for (size_t i = 0; i < sizeof(arrs) / sizeof(arrs[0]); i++) free(arrs[i]);
}

/* forward_absorbed (src/run.c:379-501) at positions 0..n-1 on tokens[p]
 * (teacher forcing): logits[p] = the step's logits. */
int ref_forward_tokens(const ref_model_spec *m, const int *tokens, int n, float *logits) {
    Transformer t;
    ref_build(m, &t);
    for (int p = 0; p < n; p++) {
        const float *lg = forward_absorbed(&t, tokens[p], p);
        memcpy(logits + (size_t)p * m->vocab, lg, (size_t)m->vocab * sizeof(float));
    }
    ref_release(&t);
    return 0;
}

/* forward_unabsorbed (src/run.c:189-370), the whole-prompt prefill, on
 * tokens[0..n): logits[p] = the logits at every prompt position, as the
 * reference dumps them ("prefill_logits", run.c:356-364) into dump_dir (a
 * writable directory; the file is read back and left there).  The
 * reference's router dump keeps n * n_experts_per_tok <= 128
 * (run.c:324-330): callers keep n within that. */
int ref_prefill_tokens(const ref_model_spec *m, const int *tokens, int n, const char *dump_dir,
                       float *logits) {
    Transformer t;
    ref_build(m, &t);
    run_set_dump(dump_dir);
    forward_unabsorbed(&t, tokens, n, NULL, NULL);
    run_set_dump(NULL);
    ref_release(&t);
    char path[512];
    snprintf(path, sizeof(path), "%s/prefill_logits.bin", dump_dir);
    FILE *f = fopen(path, "rb");
    if (!f) return -1;
    const size_t want = (size_t)n * m->vocab;
    const size_t got = fread(logits, sizeof(float), want, f);
    fclose(f);
    return got == want ? 0 : -2;
}
