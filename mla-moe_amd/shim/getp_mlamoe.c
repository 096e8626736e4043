/* getp_mlamoe.c -- the reference's batch-throughput interface (warm_up /
 * inference / finish, include/getp.h) implemented on libmlamoe.
 *
 * Built by a maintainer INSIDE the reference tree, in place of
 * src/getp_run.hip, against the reference's own headers:
 *
 *   gcc -std=c11 -O2 -c getp_mlamoe.c -I<ref>/include -I<repo>/include
 *   ... link with -L<repo>/mla-moe_amd -lmlamoe -Wl,-rpath,<repo>/mla-moe_amd
 *
 * warm_up uploads the Transformer's weights (host pointers into the
 * checkpoint mmaps, include/model.h:44-96) once: the experts as int8
 * (quantised on the device), every other tensor as bf16; it applies the
 * reference's GLM position cap (src/getp_run.hip:709-710) and starts the
 * latent caches at MLAMOE_GETP_INIT_SEQ positions per slot.  inference
 * encodes the prompts with the reference's tokenizer (prompt cap as
 * src/getp_run.hip:932-953) and runs mm_engine_generate: all requests
 * decode together in slots of a batch instead of one after another
 * (src/getp_run.hip:958-993), the caches growing as requests need
 * (src/getp_run.hip:269-290), each prompt prefilled in batched chunks of up
 * to MLAMOE_GETP_ROWS rows beside the decoding slots (the reference's
 * gpu_forward_unabsorbed, src/getp_run.hip:558-701).  Generated ids stop at
 * EOS as there.  Errors print the library's
 * message and exit, as the reference's harness does (src/getp_run.hip:480-484).
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "getp.h"
#include "mlamoe.h"
#include "model.h"
#include "tokenizer.h"

#ifndef MLAMOE_GETP_BATCH
#define MLAMOE_GETP_BATCH 64    /* decode slots */
#endif
#ifndef MLAMOE_GETP_INIT_SEQ
#define MLAMOE_GETP_INIT_SEQ 256  /* positions per slot the caches start with */
#endif
#ifndef MLAMOE_GETP_ROWS
#define MLAMOE_GETP_ROWS 2048   /* token rows per step: prompt chunks and decode rows */
#endif

static mm_ctx *g_ctx;
static mm_engine *g_eng;
static const Transformer *g_owner;
static void **g_dev;            /* device copies to free in finish() */
static size_t g_ndev, g_capdev;

static void die(const char *what) {
    fprintf(stderr, "getp_mlamoe: %s: %s\n", what, mm_last_error());
    exit(EXIT_FAILURE);
}

/* Device copy of a host tensor (NULL stays NULL). */
static const uint16_t *up(const void *h, size_t bytes) {
    if (!h) return NULL;
    void *d = NULL;
    if (mm_dev_alloc(g_ctx, bytes, &d) || mm_h2d(g_ctx, d, h, bytes)) die("upload");
    if (g_ndev == g_capdev) {
        g_capdev = g_capdev ? 2 * g_capdev : 256;
        g_dev = realloc(g_dev, g_capdev * sizeof(void *));
        if (!g_dev) die("realloc");
    }
    g_dev[g_ndev++] = d;
    return d;
}

void warm_up(Transformer *t) {
    if (g_owner) {
        fprintf(stderr, "getp_mlamoe: warm_up: already initialised\n");
        exit(EXIT_FAILURE);
    }
    /* the reference's GLM runtime caps its positions (src/getp_run.hip:709-710) */
    if (t->config.rope_interleaved && t->config.q_lora_rank > 0) t->config.max_seq_len = 512 + 64;
    const Config *c = &t->config;
    const ModelWeights *w = &t->weights;
    const size_t H = (size_t)c->hidden_size, QD = (size_t)c->n_heads * (c->qk_nope_head_dim + c->qk_rope_head_dim);
    const size_t KVD = (size_t)c->kv_lora_rank + c->qk_rope_head_dim, QL = (size_t)c->q_lora_rank;
    if (mm_ctx_create(0, &g_ctx)) die("mm_ctx_create");
    mm_mla_config ac = {c->n_heads, c->qk_nope_head_dim, c->qk_rope_head_dim, c->kv_lora_rank,
                        c->v_head_dim, c->softmax_scale};
    if (mm_mla_init(g_ctx, &ac, c->n_layers)) die("mm_mla_init");
    mm_mla_front_config fc = {c->hidden_size, c->q_lora_rank, c->rms_eps, c->mla_norm_eps,
                              c->rope_interleaved, t->rope_inv_freq};
    if (mm_mla_front_init(g_ctx, &fc)) die("mm_mla_front_init");
    mm_moe_config mc = {c->hidden_size, c->n_routed_experts, c->n_shared_experts,
                        c->n_experts_per_tok, c->moe_inter_size, c->router_sigmoid,
                        c->norm_topk, c->routed_scaling};
    if (c->first_k_dense < c->n_layers && mm_moe_init(g_ctx, &mc, c->n_layers)) die("mm_moe_init");
    /* positions per slot: the model's max_seq_len (163,840 for DeepSeek-V2-Lite,
     * src/model_load.c:237), at most what the absorbed chain serves; the
     * latent caches start small and grow with the requests, as the
     * reference's ensure_sequence_capacity does (src/getp_run.hip:269-290) */
    const int max_seq = c->max_seq_len < MM_MAX_KV_LEN ? c->max_seq_len : MM_MAX_KV_LEN;
    mm_engine_config ec = {c->n_layers, c->first_k_dense, c->hidden_size, c->dense_inter_size,
                           c->vocab_size, c->rms_eps, MLAMOE_GETP_BATCH, max_seq, MM_FWD_INT8,
                           MLAMOE_GETP_INIT_SEQ < max_seq ? MLAMOE_GETP_INIT_SEQ : max_seq,
                           MLAMOE_GETP_ROWS};
    mm_engine_layer *ls = calloc((size_t)c->n_layers, sizeof(*ls));
    if (!ls) die("calloc");
    for (int l = 0; l < c->n_layers; l++) {
        /* W_UK[l] is head 0 of the head-interleaved kv_b_proj (model_load.c:80-86) */
        if (mm_mla_load_layer(g_ctx, l, w->W_UK[l], 0)) die("mm_mla_load_layer");
        mm_engine_layer *L = &ls[l];
        L->front.input_norm = up(w->input_layernorm[l], H * 2);
        L->front.q_proj = QL ? NULL : up(w->q_proj[l], QD * H * 2);
        L->front.q_a_proj = QL ? up(w->q_a_proj[l], QL * H * 2) : NULL;
        L->front.q_a_norm = QL ? up(w->q_a_layernorm[l], QL * 2) : NULL;
        L->front.q_b_proj = QL ? up(w->q_b_proj[l], QD * QL * 2) : NULL;
        L->front.kv_a_proj = up(w->kv_a_proj[l], KVD * H * 2);
        L->front.kv_a_norm = up(w->kv_a_layernorm[l], (size_t)c->kv_lora_rank * 2);
        L->o_proj = up(w->o_proj[l], H * (size_t)c->n_heads * c->v_head_dim * 2);
        L->post_norm = up(w->post_attn_norm[l], H * 2);
        if (l < c->first_k_dense) {
            const size_t DI = (size_t)c->dense_inter_size;
            L->dense_gate = up(w->dense_gate[l], DI * H * 2);
            L->dense_up = up(w->dense_up[l], DI * H * 2);
            L->dense_down = up(w->dense_down[l], H * DI * 2);
        } else {
            mm_moe_layer_weights mw = {w->moe_gate[l], w->moe_gate_bias ? w->moe_gate_bias[l] : NULL,
                                       (const uint16_t *const *)w->expert_gate[l],
                                       (const uint16_t *const *)w->expert_up[l],
                                       (const uint16_t *const *)w->expert_down[l],
                                       w->shared_gate[l], w->shared_up[l], w->shared_down[l]};
            if (mm_moe_load_layer(g_ctx, l, &mw, MM_LOAD_INT8)) die("mm_moe_load_layer");
        }
    }
    if (mm_engine_create(g_ctx, &ec, &g_eng)) die("mm_engine_create");
    for (int l = 0; l < c->n_layers; l++)
        if (mm_engine_set_layer(g_eng, l, &ls[l])) die("mm_engine_set_layer");
    free(ls);
    if (mm_engine_set_head(g_eng, up(w->embed_tokens, (size_t)c->vocab_size * H * 2),
                           up(w->norm, H * 2), up(w->lm_head, (size_t)c->vocab_size * H * 2)))
        die("mm_engine_set_head");
    g_owner = t;
}

long long inference(Transformer *t, Requests *reqs) {
    if (g_owner != t) {
        fprintf(stderr, "getp_mlamoe: warm_up() was not called for this Transformer\n");
        exit(EXIT_FAILURE);
    }
    if (!t->tokenizer) {
        fprintf(stderr, "getp_mlamoe: model_dir has no tokenizer.json\n");
        exit(EXIT_FAILURE);
    }
    const int n = reqs->num_reqs;
    const int max_seq = t->config.max_seq_len < MM_MAX_KV_LEN ? t->config.max_seq_len : MM_MAX_KV_LEN;
    /* prompt cap of the reference's GLM runtime (src/getp_run.hip:932-936) */
    const int glm = t->config.rope_interleaved && t->config.q_lora_rank > 0;
    const int steps_cap = reqs->max_steps < 64 ? reqs->max_steps : 64;
    const int cap = glm ? (max_seq - steps_cap > 1 ? max_seq - steps_cap : 1) : max_seq;
    int32_t **prompts = calloc((size_t)n + 1, sizeof(int32_t *));
    int32_t *lens = calloc((size_t)n + 1, sizeof(int32_t));
    if (!prompts || !lens) die("calloc");
    for (int r = 0; r < n; r++) {
        prompts[r] = malloc((size_t)(cap > 0 ? cap : 1) * sizeof(int32_t));
        if (!prompts[r]) die("malloc");
        const int k = tokenizer_encode(t->tokenizer, reqs->prompts[r], 0, (int *)prompts[r], cap);
        lens[r] = k < 0 ? 0 : k;
    }
    const long long total =
        mm_engine_generate(g_eng, n, (const int32_t *const *)prompts, lens, reqs->max_steps,
                           tokenizer_eos_id(t->tokenizer), (int32_t *const *)reqs->out_tokens,
                           (int32_t *)reqs->out_lens);
    if (total < 0) die("mm_engine_generate");
    for (int r = 0; r < n; r++) free(prompts[r]);
    free(prompts);
    free(lens);
    return total;
}

void finish(Transformer *t) {
    (void)t;
    mm_engine_destroy(g_eng);
    g_eng = NULL;
    for (size_t i = 0; i < g_ndev; i++) mm_dev_free(g_ctx, g_dev[i]);
    free(g_dev);
    g_dev = NULL;
    g_ndev = g_capdev = 0;
    mm_ctx_destroy(g_ctx);
    g_ctx = NULL;
    g_owner = NULL;
}
