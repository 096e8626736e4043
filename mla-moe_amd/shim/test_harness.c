/* test_harness.c -- runs the getp shim (getp_mlamoe.c) end to end on a
 * model given as host arrays, for the GPU test of the shim.
 *
 * TEST SUPPORT.  Built with the shim against the reference's headers
 * (include/model.h, getp.h, tokenizer.h: types only) by the Makefile beside
 * it, into libgetp_shim_test.so.  It fills a reference Transformer the way
 * the reference's loader does (src/model_load.c:80-86 for the kv_b split,
 * include/model.h:44-96 for the pointer layout), then calls warm_up,
 * inference and finish as the reference's getp() harness does
 * (src/getp_eval.c).  The tokenizer is a test double: a prompt is its token
 * ids written as decimal numbers separated by spaces, so requests can be
 * checked token by token against the oracle.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "getp.h"
#include "model.h"
#include "tokenizer.h"

/* ---- test-double tokenizer (the two functions the shim calls) ------------- */
struct Tokenizer {
    int eos;
};

int tokenizer_encode(const Tokenizer *t, const char *text, int add_bos, int *out_ids, int max_ids) {
    (void)t;
    (void)add_bos;
    int n = 0;
    const char *p = text;
    while (n < max_ids) {
        char *end;
        long v = strtol(p, &end, 10);
        if (end == p) break;
        out_ids[n++] = (int)v;
        p = end;
    }
    return n;
}

int tokenizer_eos_id(const Tokenizer *t) { return t ? t->eos : -1; }

/* ---- the model --------------------------------------------------------------- */
/* Layer pointer arrays are indexed by layer (NULL where a layer has no such
 * tensor); experts are contiguous per layer: eg/eu [E, I, H], ed [E, H, I]. */
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
} shim_model_spec;

/* Build a Transformer over the spec (borrowed arrays), run warm_up, one
 * inference over n_req prompts (space-separated token ids) with max_steps
 * and end-of-sequence id eos, then finish.  out_tokens [n_req][max_steps]
 * and out_lens [n_req] receive the generated ids; *max_seq_after the
 * Transformer's max_seq_len after warm_up.  Returns inference's total. */
long long shim_run(const shim_model_spec *m, int n_req, char **prompts, int max_steps, int eos,
                   int *out_tokens, int *out_lens, int *max_seq_after) {
    Transformer t;
    memset(&t, 0, sizeof(t));
    Config *c = &t.config;
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
    ModelWeights *w = &t.weights;
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
        w->q_proj[l] = m->q_lora > 0 ? NULL : (bf16_t *)m->q_proj[l];
        if (m->q_lora > 0) {
            w->q_a_proj[l] = (bf16_t *)m->q_a_proj[l];
            w->q_a_layernorm[l] = (bf16_t *)m->q_a_norm[l];
            w->q_b_proj[l] = (bf16_t *)m->q_b_proj[l];
        }
        w->kv_a_proj[l] = (bf16_t *)m->kv_a[l];
        w->kv_a_layernorm[l] = (bf16_t *)m->kv_a_norm[l];
        w->W_UK[l] = (bf16_t *)m->kv_b[l];
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
    t.rope_inv_freq = (float *)m->inv_freq;
    Tokenizer tok = {eos};
    t.tokenizer = &tok;

    int **outs = malloc((size_t)(n_req > 0 ? n_req : 1) * sizeof(int *));
    for (int r = 0; r < n_req; r++) outs[r] = out_tokens + (size_t)r * max_steps;
    Requests req = {n_req, max_steps, prompts, outs, out_lens};
    warm_up(&t);
    *max_seq_after = t.config.max_seq_len;
    const long long total = inference(&t, &req);
    finish(&t);
    free(outs);
    for (int l = 0; l < L; l++) {
        free(w->expert_gate[l]); free(w->expert_up[l]); free(w->expert_down[l]);
    }
    void *arrs[] = {w->q_proj, w->q_a_proj, w->q_b_proj, w->kv_a_proj, w->W_UK, w->W_UV, w->o_proj,
                    w->input_layernorm, w->post_attn_norm, w->q_a_layernorm, w->kv_a_layernorm,
                    w->dense_gate, w->dense_up, w->dense_down, w->moe_gate, w->moe_gate_bias,
                    w->expert_gate, w->expert_up, w->expert_down, w->shared_gate, w->shared_up,
                    w->shared_down};
    for (size_t i = 0; i < sizeof(arrs) / sizeof(arrs[0]); i++) free(arrs[i]);
    return total;
}
