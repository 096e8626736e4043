/* mm_engine.c -- batched greedy decoding over the library's kernels.
 *
 * One decode step (forward_absorbed, src/run.c:379-501) for B sequence
 * slots at once: embedding, then per layer the attention front
 * (mm_mla_front_dev: input norm, q / kv_a projections, RoPE, kv_a norm, the
 * bf16 latent-cache append), the absorbed chain (mm_mla_absorbed_decode_dev
 * with per-slot lengths), o_proj with the residual add, the post-attention
 * norm and the FFN (dense SwiGLU for the first layers, the MoE layer with
 * its residual add), then the LM head's norm, logits and greedy argmax.
 *
 * mm_engine_generate is the scheduler: the reference's inference()
 * (src/getp_run.hip:920-995) prefills and decodes one request at a time;
 * here every active slot advances one position per step (prompt tokens
 * first, then its own samples) and a slot that finishes takes the next
 * waiting request, so the weights stream once per step for the whole batch.
 * Slot b is batch row b; a step covers rows [0, 1 + the highest active
 * slot), an idle row inside that range decodes token 0 at position 0 of its
 * own (free) cache.
 */
#include <stdlib.h>
#include <string.h>

#include "mm_internal.h"

struct mm_engine {
    mm_ctx *c;
    mm_engine_config cfg;
    mm_engine_layer *layers;
    unsigned char *layer_set;
    const uint16_t *embed, *final_norm, *lm_head;
    uint16_t **cache;          /* [n_layers] device [max_batch, lcap[l], KVL+QKR] bf16 */
    int *lcap;                 /* [n_layers] positions per slot of each layer's cache */
    int cap;                   /* positions every layer holds: min of lcap */
    int max_rows;              /* token rows per step */
    float *x, *xn, *q, *ctxo, *g, *u;   /* [max_rows, ...] step activations */
    float *fcomp;              /* [MM_SKINNY_T, KVL + QKR]: kv_a's output of steps of up to
                                  MM_SKINNY_T rows, read by the RoPE / qprep launch */
    uint16_t *xn_hl, *ctx_hl;  /* xn and ctxo of steps of 5..MM_SKINNY_T rows as bf16 hi/lo
                                  planes [2, rows, n]: the projections' operands */
    int32_t *d_io;             /* device [IO_ARRAYS][max_rows]: see IO_* */
    int32_t *h_io;             /* pinned host, same layout */
    int32_t *last_pos;         /* [max_batch] host: a step's check of its rows' positions */
};

/* the per-row arrays of a step, device and pinned host */
enum { IO_TOK, IO_POS, IO_LEN, IO_SLOT, IO_WANT, IO_NEXT, IO_ARRAYS };

void mm_engine_destroy(mm_engine *e) {
    if (!e) return;
    if (e->c) mm_set_device(e->c);
    if (e->cache) {
        for (int l = 0; l < e->cfg.n_layers; l++)
            if (e->cache[l]) hipFree(e->cache[l]);
        free(e->cache);
    }
    void *dev[] = {e->x, e->xn, e->q, e->ctxo, e->g, e->u, e->d_io, e->fcomp, e->xn_hl, e->ctx_hl};
    for (size_t i = 0; i < sizeof(dev) / sizeof(dev[0]); i++)
        if (dev[i]) hipFree(dev[i]);
    if (e->h_io) hipHostFree(e->h_io);
    free(e->last_pos);
    free(e->lcap);
    free(e->layers);
    free(e->layer_set);
    free(e);
}

/* Bytes of one layer's latent cache at `cap` positions per slot. */
static size_t cache_bytes(const mm_engine *e, int cap) {
    const mm_mla_config *g = &e->c->mla;
    return (size_t)e->cfg.max_batch * (size_t)cap * ((size_t)g->kv_lora_rank + g->qk_rope_head_dim) * 2;
}

int mm_engine_capacity(const mm_engine *e) { return e ? e->cap : 0; }

int mm_engine_reserve(mm_engine *e, int positions) {
    if (!e) return mm_fail(MM_ERR_INVALID, "mm_engine_reserve: NULL engine");
    if (positions <= e->cap) return MM_OK;
    if (positions > e->cfg.max_seq)
        return mm_fail(MM_ERR_INVALID, "mm_engine_reserve: %d positions > max_seq %d", positions,
                       e->cfg.max_seq);
    mm_ctx *c = e->c;
    int st = mm_set_device(c);
    if (st) return st;
    /* doubling up to max_seq, as ensure_sequence_capacity (getp_run.hip:269-290) */
    int cap = e->cap > 0 ? e->cap : 1;
    while (cap < positions && cap < e->cfg.max_seq)
        cap = (long long)cap * 2 < e->cfg.max_seq ? cap * 2 : e->cfg.max_seq;
    if (cap < positions) cap = positions;
    const size_t row = (size_t)(c->mla.kv_lora_rank + c->mla.qk_rope_head_dim) * 2;
    MM_HIP(hipStreamSynchronize(c->stream));
    for (int l = 0; l < e->cfg.n_layers; l++) {
        if (e->lcap[l] >= cap) continue;
        uint16_t *nc = NULL;
        if (hipMalloc((void **)&nc, cache_bytes(e, cap)) != hipSuccess) {
            (void)hipGetLastError();
            return mm_fail(MM_ERR_NOMEM, "mm_engine_reserve: latent cache of layer %d at %d "
                           "positions (%zu bytes); the engine keeps %d positions", l, cap,
                           cache_bytes(e, cap), e->cap);
        }
        /* every slot's rows [0, lcap) to the new stride */
        hipError_t he = hipMemcpy2DAsync(nc, (size_t)cap * row, e->cache[l], (size_t)e->lcap[l] * row,
                                         (size_t)e->lcap[l] * row, (size_t)e->cfg.max_batch,
                                         hipMemcpyDeviceToDevice, c->stream);
        if (he == hipSuccess) he = hipStreamSynchronize(c->stream);
        if (he != hipSuccess) {
            hipFree(nc);
            return mm_hip_fail(he, "mm_engine_reserve: copying the cache");
        }
        hipFree(e->cache[l]);
        e->cache[l] = nc;
        e->lcap[l] = cap;
    }
    e->cap = cap;
    return MM_OK;
}

int mm_engine_create(mm_ctx *c, const mm_engine_config *cfg, mm_engine **out) {
    if (!c || !cfg || !out) return mm_fail(MM_ERR_INVALID, "mm_engine_create: NULL argument");
    *out = NULL;
    if (!c->mla_ready || !c->front_ready)
        return mm_fail(MM_ERR_STATE, "mm_engine_create: call mm_mla_init and mm_mla_front_init first");
    if (cfg->first_k_dense < cfg->n_layers && !c->moe_ready)
        return mm_fail(MM_ERR_STATE, "mm_engine_create: call mm_moe_init first");
    if (cfg->n_layers <= 0 || cfg->n_layers > c->mla_layers ||
        (cfg->first_k_dense < cfg->n_layers && cfg->n_layers > c->n_layers) || cfg->first_k_dense < 0 ||
        cfg->max_batch <= 0 || cfg->max_seq <= 0 || cfg->vocab_size <= 0 ||
        cfg->hidden_size != c->front.hidden_size ||
        (cfg->first_k_dense < cfg->n_layers && cfg->hidden_size != c->moe.hidden_size) ||
        (cfg->first_k_dense > 0 && (cfg->dense_inter_size <= 0 || cfg->dense_inter_size % 8)))
        return mm_fail(MM_ERR_INVALID, "mm_engine_create: configuration does not match the context");
    if (cfg->moe_flags & ~(unsigned)MM_FWD_INT8)
        return mm_fail(MM_ERR_INVALID, "mm_engine_create: moe_flags must be MM_FWD_BF16 or MM_FWD_INT8");
    for (int l = cfg->first_k_dense; l < cfg->n_layers; l++)
        if (!c->layers[l].loaded)
            return mm_fail(MM_ERR_STATE, "mm_engine_create: MoE layer %d not loaded", l);
    for (int l = 0; l < cfg->n_layers; l++)
        if (!c->mla_kvb[l]) return mm_fail(MM_ERR_STATE, "mm_engine_create: MLA layer %d not loaded", l);
    int st = mm_set_device(c);
    if (st) return st;
    mm_engine *e = calloc(1, sizeof(*e));
    if (!e) return mm_fail(MM_ERR_NOMEM, "mm_engine_create: calloc");
    e->c = c;
    e->cfg = *cfg;
    e->layers = calloc((size_t)cfg->n_layers, sizeof(mm_engine_layer));
    e->layer_set = calloc((size_t)cfg->n_layers, 1);
    e->cache = calloc((size_t)cfg->n_layers, sizeof(uint16_t *));
    e->lcap = calloc((size_t)cfg->n_layers, sizeof(int));
    if (!e->layers || !e->layer_set || !e->cache || !e->lcap) {
        mm_engine_destroy(e);
        return mm_fail(MM_ERR_NOMEM, "mm_engine_create: calloc");
    }
    const mm_mla_config *g = &c->mla;
    const size_t B = (size_t)cfg->max_batch, H = (size_t)cfg->hidden_size;
    if (cfg->max_rows < 0) {
        mm_engine_destroy(e);
        return mm_fail(MM_ERR_INVALID, "mm_engine_create: max_rows < 0");
    }
    e->max_rows = cfg->max_rows ? cfg->max_rows : (cfg->max_batch > 1024 ? cfg->max_batch : 1024);
    if (e->max_rows < cfg->max_batch) e->max_rows = cfg->max_batch;
    const size_t MR = (size_t)e->max_rows;
    const size_t KVD = (size_t)g->kv_lora_rank + g->qk_rope_head_dim;
    const size_t QD = (size_t)g->n_heads * (g->qk_nope_head_dim + g->qk_rope_head_dim);
    const size_t DI = cfg->first_k_dense > 0 ? (size_t)cfg->dense_inter_size : 8;
    struct { void **p; size_t n; } bufs[] = {
        {(void **)&e->x, MR * H * 4}, {(void **)&e->xn, MR * H * 4}, {(void **)&e->q, MR * QD * 4},
        {(void **)&e->ctxo, MR * (size_t)g->n_heads * g->v_head_dim * 4},
        {(void **)&e->g, MR * DI * 4}, {(void **)&e->u, MR * DI * 4},
        {(void **)&e->d_io, IO_ARRAYS * MR * 4},
        {(void **)&e->fcomp, (size_t)MM_SKINNY_T * KVD * 4},
        {(void **)&e->xn_hl, (size_t)MM_SKINNY_T * H * 4},
        {(void **)&e->ctx_hl, (size_t)MM_SKINNY_T * g->n_heads * g->v_head_dim * 4}};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
        if (hipMalloc(bufs[i].p, bufs[i].n) != hipSuccess) {
            mm_engine_destroy(e);
            return mm_fail(MM_ERR_NOMEM, "mm_engine_create: step buffers for %zu rows", MR);
        }
    if (hipHostMalloc((void **)&e->h_io, IO_ARRAYS * MR * 4, 0) != hipSuccess) {
        mm_engine_destroy(e);
        return mm_fail(MM_ERR_NOMEM, "mm_engine_create: pinned host buffer");
    }
    e->last_pos = malloc(B * sizeof(int32_t));
    if (!e->last_pos) {
        mm_engine_destroy(e);
        return mm_fail(MM_ERR_NOMEM, "mm_engine_create: malloc");
    }
    if (cfg->init_seq < 0 || cfg->init_seq > cfg->max_seq) {
        mm_engine_destroy(e);
        return mm_fail(MM_ERR_INVALID, "mm_engine_create: init_seq outside [0, max_seq]");
    }
    e->cap = cfg->init_seq ? cfg->init_seq : (cfg->max_seq < 1024 ? cfg->max_seq : 1024);
    for (int l = 0; l < cfg->n_layers; l++) {
        if (hipMalloc((void **)&e->cache[l], B * (size_t)e->cap * KVD * 2) != hipSuccess) {
            (void)hipGetLastError();
            mm_engine_destroy(e);
            return mm_fail(MM_ERR_NOMEM, "mm_engine_create: latent cache of layer %d (%zu bytes)", l,
                           B * (size_t)e->cap * KVD * 2);
        }
        e->lcap[l] = e->cap;
    }
    *out = e;
    return MM_OK;
}

int mm_engine_set_layer(mm_engine *e, int layer, const mm_engine_layer *w) {
    if (!e || !w) return mm_fail(MM_ERR_INVALID, "mm_engine_set_layer: NULL argument");
    if (layer < 0 || layer >= e->cfg.n_layers)
        return mm_fail(MM_ERR_INVALID, "mm_engine_set_layer: layer %d out of range", layer);
    if (!w->o_proj || !w->post_norm ||
        (layer < e->cfg.first_k_dense && (!w->dense_gate || !w->dense_up || !w->dense_down)))
        return mm_fail(MM_ERR_INVALID, "mm_engine_set_layer: NULL weight");
    e->layers[layer] = *w;
    e->layer_set[layer] = 1;
    return MM_OK;
}

int mm_engine_set_head(mm_engine *e, const uint16_t *embed, const uint16_t *final_norm,
                       const uint16_t *lm_head) {
    if (!e || !embed || !final_norm || !lm_head) return mm_fail(MM_ERR_INVALID, "mm_engine_set_head: NULL argument");
    e->embed = embed;
    e->final_norm = final_norm;
    e->lm_head = lm_head;
    return MM_OK;
}

/* GEMV sizes: the post-attention norm is fused into the consumer's GEMV
 * (dense gate/up) or runs on its own; larger batches fuse it into o_proj's
 * reduce instead. */
static int gemv_rows(const mm_engine *e, int B) {
    return B <= MM_GEMV_NB && e->cfg.hidden_size <= MM_LM_HMAX;
}

/* Steps whose projections read their x as bf16 hi/lo planes (5 to
 * MM_SKINNY_T rows, both widths multiples of 64). */
static int hl_rows(const mm_engine *e, int R) {
    const mm_mla_config *g = &e->c->mla;
    return !gemv_rows(e, R) && R <= MM_SKINNY_T && e->cfg.hidden_size % 64 == 0 &&
           (g->n_heads * g->v_head_dim) % 64 == 0;
}

/* o_proj with its residual add, x += ctxo . o_proj^T (src/run.c:462-468),
 * then xn = rmsnorm(x, post_norm) (src/run.c:470-472) unless the dense
 * GEMV path applies it itself: one GEMM + one reduce-and-norm pass for
 * more than MM_GEMV_NB rows. */
static int oproj_post_norm(mm_engine *e, const mm_engine_layer *L, int R, int dense) {
    mm_ctx *c = e->c;
    const mm_mla_config *g = &c->mla;
    const int H = e->cfg.hidden_size, NIN = g->n_heads * g->v_head_dim;
    int st;
    if (gemv_rows(e, R)) {
        if ((st = mm_matmul_bf16_dev(c, e->x, e->ctxo, L->o_proj, H, NIN, R, MM_MATMUL_ACCUMULATE)))
            return st;
        if (dense && gemv_rows(e, R)) return MM_OK;
        mm_rmsnorm_args ra = {e->x, L->post_norm, e->xn, H, e->cfg.rms_eps};
        return mm_launch(c, K_RMSNORM, (unsigned)R, 1, 1, 256, 0, &ra);
    }
    char *ws;
    if ((st = mm_workspace(c, mm_gemm_bf16_add_rmsnorm_ws_bytes(R, NIN, H), (void **)&ws))) return st;
    if (hl_rows(e, R))   /* ctx as the hi/lo planes the W_UV product wrote */
        return mm_gemm_bf16_add_rmsnorm_hl(c, e->x, e->ctx_hl, L->o_proj, H, NIN, R, L->post_norm,
                                           e->cfg.rms_eps, e->xn, ws);
    return mm_gemm_bf16_add_rmsnorm(c, e->x, e->ctxo, L->o_proj, H, NIN, R, L->post_norm,
                                    e->cfg.rms_eps, e->xn, ws);
}

/* The dense SwiGLU MLP with its residual add: x += down . (silu(gate . xn) * (up . xn)),
 * xn = rmsnorm(x, post_norm) (src/run.c:470-472, 86-93): computed by
 * oproj_post_norm, or here by the gate/up GEMV at GEMV sizes. */
static int dense_ffn(mm_engine *e, const mm_engine_layer *L, int B) {
    mm_ctx *c = e->c;
    const int H = e->cfg.hidden_size, DI = e->cfg.dense_inter_size;
    int st;
    if (gemv_rows(e, B)) {
        mm_gemv_args a = {e->x, L->post_norm, e->cfg.rms_eps, L->dense_gate, L->dense_up, e->g, e->u,
                          DI, DI, DI, DI, B, H, 0, 0};
        if ((st = mm_gemv_launch(c, &a))) return st;
    } else {
        /* gate and up over the same xn in one pass */
        char *ws;
        if ((st = mm_workspace(c, mm_gemm_bf16_ws2_bytes(B, H, DI, DI, 0), (void **)&ws))) return st;
        if ((st = mm_gemm_bf16_ws2(c, e->g, L->dense_gate, DI, e->u, L->dense_up, DI, e->xn, H, B, 0, ws)))
            return st;
    }
    const size_t n = (size_t)B * DI;
    mm_swiglu_args sa = {e->g, e->u, e->g, n};
    const size_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    if ((st = mm_launch(c, K_SWIGLU, (unsigned)blocks, 1, 1, 256, 0, &sa))) return st;
    return mm_matmul_bf16_dev(c, e->x, e->g, L->dense_down, H, DI, B, MM_MATMUL_ACCUMULATE);
}

/* One step over R rows (h_io filled: tokens, positions, slots; want rows):
 * embedding, every layer over all rows, the LM head over the wanted rows. */
static int engine_run(mm_engine *e, int R, int n_want, int32_t *next, float *logits) {
    mm_ctx *c = e->c;
    const mm_engine_config *f = &e->cfg;
    const int MR = e->max_rows;
    int32_t *hio = e->h_io;
    int kvmax = 1;
    for (int b = 0; b < f->max_batch; b++) e->last_pos[b] = -1;
    for (int r = 0; r < R; r++) {
        const int s = hio[IO_SLOT * MR + r], p = hio[IO_POS * MR + r];
        if (s < 0 || s >= f->max_batch)
            return mm_fail(MM_ERR_INVALID, "mm_engine_step: row %d: slot %d outside [0, %d)", r, s,
                           f->max_batch);
        if (p < 0 || p >= f->max_seq)
            return mm_fail(MM_ERR_INVALID, "mm_engine_step: row %d: pos %d outside [0, %d)", r, p,
                           f->max_seq);
        /* a slot's rows in ascending positions: no cache row written twice */
        if (p <= e->last_pos[s])
            return mm_fail(MM_ERR_INVALID, "mm_engine_step: row %d: slot %d position %d not above "
                           "its previous row's", r, s, p);
        e->last_pos[s] = p;
        hio[IO_LEN * MR + r] = p + 1;
        if (p + 1 > kvmax) kvmax = p + 1;
    }
    for (int j = 0; j < n_want; j++) {
        const int w = hio[IO_WANT * MR + j];
        if (w < 0 || w >= R || (j > 0 && w <= hio[IO_WANT * MR + j - 1]))
            return mm_fail(MM_ERR_INVALID, "mm_engine_step: want_rows must ascend within [0, %d)", R);
    }
    /* every group of 4 rows in one slot (a prefill's positions): the
     * attention reads each group's keys once */
    int rows4 = R > 1;
    for (int r = 0; r < R && rows4; r++) rows4 = hio[IO_SLOT * MR + r] == hio[IO_SLOT * MR + (r & ~3)];
    int st = mm_engine_reserve(e, kvmax);
    if (st) return st;
    if ((st = mm_set_device(c))) return st;
    int32_t *d_tok = e->d_io + IO_TOK * MR, *d_pos = e->d_io + IO_POS * MR;
    int32_t *d_len = e->d_io + IO_LEN * MR, *d_slot = e->d_io + IO_SLOT * MR;
    int32_t *d_want = e->d_io + IO_WANT * MR, *d_next = e->d_io + IO_NEXT * MR;
    MM_HIP(hipMemcpyAsync(e->d_io, hio, (size_t)IO_NEXT * MR * 4, hipMemcpyHostToDevice, c->stream));
    const int H = f->hidden_size;
    mm_embed_args ea = {e->embed, d_tok, e->x, H, f->vocab_size};
    if ((st = mm_launch(c, K_EMBED, (unsigned)((H + 2047) / 2048), (unsigned)R, 1, 256, 0, &ea))) return st;
    int xn_ready = 0;   /* xn holds rmsnorm(x, this layer's input_norm) */
    for (int l = 0; l < f->n_layers; l++) {
        const mm_engine_layer *L = &e->layers[l];
        const int pre = xn_ready;
        xn_ready = 0;
        /* up to MM_SKINNY_T rows the RoPE / cache append runs in the absorbed
         * queries' launch (one launch fewer per layer) */
        mm_mla_rope_args ra;
        const int fuse = R <= MM_SKINNY_T;
        if ((st = mm_mla_front_rows(c, R, e->x, &L->front, d_pos, d_slot, e->q, e->cache[l], e->lcap[l],
                                    NULL, pre ? e->xn : NULL, pre && hl_rows(e, R) ? e->xn_hl : NULL,
                                    fuse ? e->fcomp : NULL,
                                    fuse ? &ra : NULL)))
            return st;
        if ((st = mm_mla_decode_rows(c, l, R, e->q, e->cache[l], e->lcap[l], d_slot, d_len, kvmax,
                                     e->ctxo, NULL, NULL, NULL, fuse ? &ra : NULL,
                                     hl_rows(e, R) ? e->ctx_hl : NULL, rows4)))
            return st;
        const int dense = l < f->first_k_dense;
        if ((st = oproj_post_norm(e, L, R, dense))) return st;
        if (dense) {
            if ((st = dense_ffn(e, L, R))) return st;
        } else {
            /* above GEMV sizes the next layer's input norm is computed by
             * the MoE's combine pass (int8 experts) into xn, which the MoE
             * no longer reads by then */
            const int next_norm = l + 1 < f->n_layers && !gemv_rows(e, R);
            int fused = 0;
            if ((st = mm_moe_forward_norm(c, l, R, e->xn, e->x, f->moe_flags | MM_FWD_ACCUMULATE,
                                          next_norm ? e->layers[l + 1].front.input_norm : NULL,
                                          c->front.rms_eps, e->xn, hl_rows(e, R) ? e->xn_hl : NULL,
                                          &fused)))
                return st;
            xn_ready = fused;
        }
    }
    if (n_want > 0) {
        /* the sampled rows, gathered (xn is free by now) unless they are all rows */
        const float *xs = e->x;
        if (n_want < R) {
            mm_gather_rows_args ga = {e->x, d_want, e->xn, n_want, H};
            if ((st = mm_launch(c, K_GATHER_ROWS, (unsigned)n_want, 1, 1, 256, 0, &ga))) return st;
            xs = e->xn;
        }
        if ((st = mm_lm_head_dev(c, n_want, xs, e->final_norm, f->rms_eps, e->lm_head, f->vocab_size,
                                 H, logits, d_next)))
            return st;
        MM_HIP(hipMemcpyAsync(hio + IO_NEXT * MR, d_next, (size_t)n_want * 4, hipMemcpyDeviceToHost,
                              c->stream));
    }
    MM_HIP(hipStreamSynchronize(c->stream));
    if (n_want > 0) memcpy(next, hio + IO_NEXT * MR, (size_t)n_want * 4);
    return MM_OK;
}

static int engine_ready(const mm_engine *e, const char *fn) {
    if (!e->embed) return mm_fail(MM_ERR_STATE, "%s: call mm_engine_set_head first", fn);
    for (int l = 0; l < e->cfg.n_layers; l++)
        if (!e->layer_set[l]) return mm_fail(MM_ERR_STATE, "%s: layer %d not set", fn, l);
    return MM_OK;
}

int mm_engine_step(mm_engine *e, int B, const int32_t *tokens, const int32_t *pos, int32_t *next,
                   float *logits) {
    if (!e || !tokens || !pos || !next) return mm_fail(MM_ERR_INVALID, "mm_engine_step: NULL argument");
    if (B < 1 || B > e->cfg.max_batch)
        return mm_fail(MM_ERR_INVALID, "mm_engine_step: B = %d outside [1, %d]", B, e->cfg.max_batch);
    int st = engine_ready(e, "mm_engine_step");
    if (st) return st;
    const int MR = e->max_rows;
    for (int b = 0; b < B; b++) {
        e->h_io[IO_TOK * MR + b] = tokens[b];
        e->h_io[IO_POS * MR + b] = pos[b];
        e->h_io[IO_SLOT * MR + b] = b;
        e->h_io[IO_WANT * MR + b] = b;
    }
    return engine_run(e, B, B, next, logits);
}

int mm_engine_step_rows(mm_engine *e, int R, const int32_t *slots, const int32_t *tokens,
                        const int32_t *pos, int n_want, const int32_t *want_rows, int32_t *next,
                        float *logits) {
    if (!e || !slots || !tokens || !pos || (n_want > 0 && (!want_rows || !next)))
        return mm_fail(MM_ERR_INVALID, "mm_engine_step_rows: NULL argument");
    if (R < 1 || R > e->max_rows || n_want < 0 || n_want > R)
        return mm_fail(MM_ERR_INVALID, "mm_engine_step_rows: R = %d outside [1, %d] or n_want = %d "
                       "outside [0, R]", R, e->max_rows, n_want);
    int st = engine_ready(e, "mm_engine_step_rows");
    if (st) return st;
    const int MR = e->max_rows;
    memcpy(e->h_io + IO_TOK * MR, tokens, (size_t)R * 4);
    memcpy(e->h_io + IO_POS * MR, pos, (size_t)R * 4);
    memcpy(e->h_io + IO_SLOT * MR, slots, (size_t)R * 4);
    if (n_want) memcpy(e->h_io + IO_WANT * MR, want_rows, (size_t)n_want * 4);
    return engine_run(e, R, n_want, next, logits);
}

long long mm_engine_generate(mm_engine *e, int n_req, const int32_t *const *prompts,
                             const int32_t *prompt_lens, int max_steps, int eos,
                             int32_t *const *out_tokens, int32_t *out_lens) {
    if (!e || n_req < 0 || (n_req > 0 && (!prompts || !prompt_lens || !out_tokens || !out_lens)))
        return mm_fail(MM_ERR_INVALID, "mm_engine_generate: NULL argument");
    int st = engine_ready(e, "mm_engine_generate");
    if (st) return st;
    const int MB = e->cfg.max_batch, MR = e->max_rows;
    /* per slot: request, token budget, next position to feed, last sample */
    int *req = malloc((size_t)MB * sizeof(int)), *limit = malloc((size_t)MB * sizeof(int));
    int *npos = malloc((size_t)MB * sizeof(int)), *wslot = malloc((size_t)MR * sizeof(int));
    int32_t *last = malloc((size_t)MB * 4), *nxt = malloc((size_t)MR * 4);
    if (!req || !limit || !npos || !wslot || !last || !nxt) {
        free(req); free(limit); free(npos); free(wslot); free(last); free(nxt);
        return mm_fail(MM_ERR_NOMEM, "mm_engine_generate: malloc");
    }
    int32_t *rtok = e->h_io + IO_TOK * MR, *rpos = e->h_io + IO_POS * MR;
    int32_t *rslot = e->h_io + IO_SLOT * MR, *rwant = e->h_io + IO_WANT * MR;
    for (int s = 0; s < MB; s++) req[s] = -1;
    for (int r = 0; r < n_req; r++) out_lens[r] = 0;
    long long total = 0;
    int next_req = 0;
    for (;;) {
        /* admit waiting requests into free slots (lowest first) */
        for (int s = 0; s < MB && next_req < n_req && !st; s++) {
            if (req[s] >= 0) continue;
            while (next_req < n_req) {
                const int r = next_req++;
                const int n = prompt_lens[r];
                /* generated tokens: max_steps, and no more than the positions
                 * left after the prompt (getp_run.hip:946-952) */
                const int lim = max_steps < e->cfg.max_seq - n ? max_steps : e->cfg.max_seq - n;
                if (n < 1 || lim < 1 || !prompts[r]) continue;
                /* the positions this request will use: its prompt and all
                 * but the last generated token */
                if ((st = mm_engine_reserve(e, n + lim - 1))) break;
                req[s] = r;
                limit[s] = lim;
                npos[s] = 0;
                break;
            }
        }
        if (st) break;
        /* the step's rows: one decode row per slot past its prompt, then the
         * prompts' next chunks in the rows left */
        int R = 0, nw = 0;
        for (int s = 0; s < MB; s++) {
            if (req[s] < 0 || npos[s] < prompt_lens[req[s]]) continue;
            rslot[R] = s;
            rpos[R] = npos[s];
            rtok[R] = last[s];
            wslot[nw] = s;
            rwant[nw++] = R++;
        }
        for (int s = 0; s < MB && R < MR; s++) {
            if (req[s] < 0) continue;
            const int n = prompt_lens[req[s]];
            if (npos[s] >= n) continue;
            const int k = n - npos[s] < MR - R ? n - npos[s] : MR - R;
            for (int i = 0; i < k; i++) {
                rslot[R + i] = s;
                rpos[R + i] = npos[s] + i;
                rtok[R + i] = prompts[req[s]][npos[s] + i];
            }
            R += k;
            if (npos[s] + k == n) {          /* the prompt's last row samples */
                wslot[nw] = s;
                rwant[nw++] = R - 1;
            }
        }
        if (R == 0) break;
        if ((st = engine_run(e, R, nw, nxt, NULL))) break;
        /* positions fed this step */
        for (int i = 0; i < R; i++) npos[rslot[i]] = rpos[i] + 1;
        for (int j = 0; j < nw; j++) {
            const int s = wslot[j], r = req[s];
            int done;
            if (eos >= 0 && nxt[j] == eos) {
                done = 1;
            } else {
                out_tokens[r][out_lens[r]++] = nxt[j];
                total++;
                last[s] = nxt[j];
                done = out_lens[r] >= limit[s];
            }
            if (done) req[s] = -1;
        }
    }
    free(req); free(limit); free(npos); free(wslot); free(last); free(nxt);
    return st ? (long long)st : total;
}
