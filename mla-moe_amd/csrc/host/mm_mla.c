/* mm_mla.c -- MLA absorbed decode (host side).
 *
 * Replaces the absorbed per-head loop of forward_absorbed (src/run.c:430-460)
 * for B sequences at once.  kv_b is the reference's kv_b_proj weight,
 * head-interleaved [W_UK_h | W_UV_h] per head (src/model_load.c:80-86).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "mm_internal.h"

void mm_mla_release(mm_ctx *c) {
    if (c->front_inv) hipFree(c->front_inv);
    c->front_inv = NULL;
    c->front_ready = 0;
    if (!c->mla_kvb) return;
    for (int l = 0; l < c->mla_layers; l++)
        if (c->mla_kvb[l]) hipFree(c->mla_kvb[l]);
    free(c->mla_kvb);
    c->mla_kvb = NULL;
    c->mla_ready = 0;
}

int mm_mla_init(mm_ctx *c, const mm_mla_config *cfg, int n_layers) {
    if (!c || !cfg) return mm_fail(MM_ERR_INVALID, "mm_mla_init: NULL argument");
    if (c->mla_ready) return mm_fail(MM_ERR_STATE, "mm_mla_init: already initialised");
    if (n_layers <= 0 || cfg->n_heads <= 0 || cfg->qk_nope_head_dim <= 0 || cfg->v_head_dim <= 0)
        return mm_fail(MM_ERR_INVALID, "mm_mla_init: non-positive dimension");
    if (cfg->qk_nope_head_dim % 32)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_mla_init: qk_nope_head_dim must be a multiple of 32");
    if (cfg->kv_lora_rank != MM_MLA_KVL || cfg->qk_rope_head_dim != MM_MLA_QKR)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_mla_init: kernels serve kv_lora_rank %d and "
                       "qk_rope_head_dim %d", MM_MLA_KVL, MM_MLA_QKR);
    c->mla_kvb = calloc((size_t)n_layers, sizeof(uint16_t *));
    if (!c->mla_kvb) return mm_fail(MM_ERR_NOMEM, "mm_mla_init: calloc");
    c->mla = *cfg;
    c->mla_layers = n_layers;
    c->mla_ready = 1;
    return MM_OK;
}

int mm_mla_load_layer(mm_ctx *c, int layer, const uint16_t *kv_b, unsigned flags) {
    if (!c || !kv_b) return mm_fail(MM_ERR_INVALID, "mm_mla_load_layer: NULL argument");
    if (!c->mla_ready) return mm_fail(MM_ERR_STATE, "mm_mla_load_layer: call mm_mla_init first");
    if (layer < 0 || layer >= c->mla_layers)
        return mm_fail(MM_ERR_INVALID, "mm_mla_load_layer: layer %d out of range", layer);
    if (c->mla_kvb[layer]) return mm_fail(MM_ERR_STATE, "mm_mla_load_layer: layer %d loaded", layer);
    int st = mm_set_device(c);
    if (st) return st;
    const mm_mla_config *g = &c->mla;
    /* one pool per layer: kv_b as given, then W_UK^T per head [NH][KVL][QKN] */
    const size_t n = (size_t)g->n_heads * (g->qk_nope_head_dim + g->v_head_dim) * g->kv_lora_rank;
    const size_t nt = (size_t)g->n_heads * g->kv_lora_rank * g->qk_nope_head_dim;
    MM_HIP(hipMalloc((void **)&c->mla_kvb[layer], (n + nt) * 2));
    MM_HIP(hipMemcpyAsync(c->mla_kvb[layer], kv_b, n * 2,
                          (flags & MM_LOAD_DEVICE_PTRS) ? hipMemcpyDeviceToDevice
                                                        : hipMemcpyHostToDevice,
                          c->stream));
    mm_mla_wprep_args wa = {c->mla_kvb[layer], c->mla_kvb[layer] + n, g->n_heads,
                            g->qk_nope_head_dim, g->v_head_dim};
    if ((st = mm_launch(c, K_MLA_WPREP, 1024, 1, 1, 256, 0, &wa))) return st;
    MM_HIP(hipStreamSynchronize(c->stream));
    return MM_OK;
}

int mm_mla_absorbed_decode_dev(mm_ctx *c, int layer, int B, const float *q,
                               const uint16_t *cache, int seq_stride, const int32_t *kv_lens,
                               int kv_len, float *ctx_out, float *qabs, float *probs,
                               float *clat) {
    return mm_mla_decode_rows(c, layer, B, q, cache, seq_stride, NULL, kv_lens, kv_len, ctx_out,
                              qabs, probs, clat, NULL, NULL, 0);
}

static int decode_rows(mm_ctx *c, int layer, int B, const float *q, const uint16_t *cache,
                       int seq_stride, const int32_t *slots, const int32_t *kv_lens, int kv_len,
                       float *ctx_out, float *qabs, float *probs, float *clat,
                       const mm_mla_rope_args *rope, uint16_t *ctx_hl, int chunk_in, unsigned zc_in,
                       int rows4);

int mm_mla_decode_rows(mm_ctx *c, int layer, int B, const float *q, const uint16_t *cache,
                       int seq_stride, const int32_t *slots, const int32_t *kv_lens, int kv_len,
                       float *ctx_out, float *qabs, float *probs, float *clat,
                       const mm_mla_rope_args *rope, uint16_t *ctx_hl, int rows4) {
    return decode_rows(c, layer, B, q, cache, seq_stride, slots, kv_lens, kv_len, ctx_out, qabs,
                       probs, clat, rope, ctx_hl, 0, 0, rows4 && slots && c->mla_rows4);
}

/* The merge's blocks per (head, sequence): the latent columns over 4 blocks
 * when the grid would otherwise have fewer than 128 blocks (each block's
 * chunk groups then meet in group order). */
static unsigned merge_z(int NH, int B) { return (size_t)NH * B < 128 ? MM_MLA_KVL / 128 : 1; }

/* chunk_in > 0: a group of a larger call's rows, with that call's chunk
 * length and merge split zc_in (the same partition of every row's keys and
 * the same order of their sums, so the same results) and no further
 * grouping. */
static int decode_rows(mm_ctx *c, int layer, int B, const float *q, const uint16_t *cache,
                       int seq_stride, const int32_t *slots, const int32_t *kv_lens, int kv_len,
                       float *ctx_out, float *qabs, float *probs, float *clat,
                       const mm_mla_rope_args *rope, uint16_t *ctx_hl, int chunk_in, unsigned zc_in,
                       int rows4) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode_dev: NULL context");
    if (!c->mla_ready || layer < 0 || layer >= c->mla_layers || !c->mla_kvb[layer])
        return mm_fail(MM_ERR_STATE, "mm_mla_absorbed_decode_dev: layer %d not loaded", layer);
    if (B < 0 || (B > 0 && (!q || !cache || !ctx_out)))
        return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode_dev: NULL argument");
    if (B == 0) return MM_OK;
    if (kv_len < 1 || seq_stride < kv_len)
        return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode_dev: need 1 <= kv_len <= seq_stride");
    const int g_nh = c->mla.n_heads, HG0 = (g_nh + 15) / 16;
    /* chunk length: MM_MLA_CHUNK keys per block, halved (down to 16 keys per
     * wave) while the grid has fewer than MM_MLA_MIN_BLOCKS blocks and the
     * chunk count stays <= 64 -- small batches then spread the cache read
     * over more CUs; long contexts keep the longest chunk, up to
     * MM_MLA_MAXCH of them (the merge's limit) */
    int chunk = MM_MLA_CHUNK;
    const size_t Bblk = rows4 ? (size_t)(B + MM_MLA_AW - 1) / MM_MLA_AW : (size_t)B;   /* blocks per chunk */
    while (chunk > 16 * MM_MLA_AW &&
           Bblk * HG0 * ((kv_len + chunk - 1) / chunk) < MM_MLA_MIN_BLOCKS &&
           (kv_len + chunk / 2 - 1) / (chunk / 2) <= 64)
        chunk /= 2;
    /* a second chunk of under half a chunk (short contexts): one chunk of
     * twice the length instead, whose block writes clat itself (no merge
     * launch) */
    if (chunk < MM_MLA_CHUNK && kv_len > chunk && kv_len <= chunk + chunk / 2) chunk *= 2;
    /* row groups numerous enough to fill the CUs twice over (a prefill's
     * causal rows): one block per group takes the whole context and writes
     * clat itself -- no chunk partials, no merge launch; dealt longest
     * first, the groups' unequal lengths even out over the CUs */
    if (rows4 && Bblk * HG0 >= 2 * MM_MLA_MIN_BLOCKS)
        chunk = (kv_len + 16 * MM_MLA_AW - 1) / (16 * MM_MLA_AW) * (16 * MM_MLA_AW);
    if (chunk_in > 0) chunk = chunk_in;
    const int nchunks = (kv_len + chunk - 1) / chunk;
    const int direct = nchunks == 1 && !probs;
    if (kv_len > MM_MAX_KV_LEN || nchunks > MM_MLA_MAXCH)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_mla_absorbed_decode_dev: kv_len %d > %d", kv_len,
                       MM_MAX_KV_LEN);
    if ((uintptr_t)cache % 16)
        return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode_dev: cache must be 16-byte aligned");
    int st = mm_set_device(c);
    if (st) return st;
    const mm_mla_config *g = &c->mla;
    const int NH = g->n_heads, HG = (NH + 15) / 16;
    /* The chunk partials take B HG nchunks (16 x 512 + 32) floats: every row
     * is sized for the longest context of the step (kv_len).  Above
     * c->mla_part_max bytes (MM_MLA_PART_MAX) the rows go in groups, one
     * after another on the stream, each within the cap and with this call's
     * chunk length (the RoPE / cache append of a front step first, for all
     * rows).  Not with ctx_hl, whose lo plane sits B rows after the hi plane
     * (its callers pass at most MM_SKINNY_T rows). */
    const size_t part_row = direct ? 0 : (size_t)HG * nchunks * (16 * MM_MLA_KVL + 32) * 4;
    if (!chunk_in && !ctx_hl && (size_t)B * part_row > c->mla_part_max) {
        if (rope && (st = mm_launch(c, K_MLA_ROPE, (unsigned)B, 1, 1, 256, 0, (void *)rope))) return st;
        int G = (int)(c->mla_part_max / part_row) > 0 ? (int)(c->mla_part_max / part_row) : 1;
        if (rows4) G = G >= MM_MLA_AW ? G / MM_MLA_AW * MM_MLA_AW : MM_MLA_AW;   /* whole row groups */
        const int QKD = g->qk_nope_head_dim + MM_MLA_QKR;
        for (int r0 = 0; r0 < B; r0 += G) {
            const int n = B - r0 < G ? B - r0 : G;
            const size_t rq = (size_t)r0 * NH;
            /* without slots row b reads cache sequence b */
            if ((st = decode_rows(
                     c, layer, n, q + rq * QKD,
                     slots ? cache : cache + (size_t)r0 * seq_stride * MM_MLA_KVD, seq_stride,
                     slots ? slots + r0 : NULL, kv_lens ? kv_lens + r0 : NULL, kv_len,
                     ctx_out + rq * g->v_head_dim, qabs ? qabs + rq * MM_MLA_KVL : NULL,
                     probs ? probs + rq * kv_len : NULL, clat ? clat + rq * MM_MLA_KVL : NULL, NULL,
                     NULL, chunk, merge_z(NH, B), rows4)))
                return st;
        }
        return MM_OK;
    }
    /* qabs in fp32 only for a caller that asks for it (the attention reads
     * its bf16 hi / lo rows) */
    const size_t qa_b = 0;
    /* chunk partials (none when one block takes a row's whole context) */
    const size_t ml_b = direct ? 0 : (size_t)B * HG * nchunks * 32 * 4;
    const size_t po_b = direct ? 0 : (size_t)B * HG * nchunks * 16 * MM_MLA_KVL * 4;
    const size_t cl_b = clat ? 0 : (size_t)B * NH * MM_MLA_KVL * 4;
    const size_t qhl_b = (size_t)B * NH * 2 * MM_MLA_KVL * 2;   /* qabs as bf16 hi + lo */
    char *ws;
    const size_t a1 = 0, a2 = (qa_b + 255) & ~(size_t)255;
    const size_t a3 = (ml_b + 255) & ~(size_t)255, a4 = (po_b + 255) & ~(size_t)255;
    const size_t a5 = (cl_b + 255) & ~(size_t)255;
    if ((st = mm_workspace(c, a1 + a2 + a3 + a4 + a5 + qhl_b, (void **)&ws))) return st;
    float *part_ml = (float *)(ws + a1 + a2), *part_o = (float *)(ws + a1 + a2 + a3);
    if (!clat) clat = (float *)(ws + a1 + a2 + a3 + a4);
    uint16_t *qhl = (uint16_t *)(ws + a1 + a2 + a3 + a4 + a5);

    const int QKN = g->qk_nope_head_dim;
    const size_t nkvb = (size_t)NH * (QKN + g->v_head_dim) * MM_MLA_KVL;
    mm_mla_qprep_args qa = {q, c->mla_kvb[layer] + nkvb, qabs, qhl, B, NH, QKN};
    /* many rows (a prefill): MM_MLA_WIDE_S column tiles per wave in the W_UK
     * and W_UV products, a 32-row tile of their fp32 operand read and split
     * once for all of them */
    const int wide = B >= MM_MLA_WIDE_B;
    if (rope) {   /* the front's RoPE / cache append in the same launch */
        mm_mla_rope_qprep_args rq;
        rq.r = *rope;
        rq.qp = qa;
        const unsigned nq = (unsigned)(MM_MLA_KVL / 64 * NH * ((B + 31) / 32));
        if ((st = mm_launch(c, K_MLA_ROPE_QPREP, (unsigned)B + nq, 1, 1, 256, 0, &rq))) return st;
    } else if ((st = mm_launch(c, wide ? K_MLA_QPREP_W : K_MLA_QPREP,
                               MM_MLA_KVL / (wide ? 64 * MM_MLA_WIDE_S : 64), (unsigned)NH,
                               (unsigned)((B + 31) / 32), 256, 0, &qa))) {
        return st;
    }
    mm_mla_attn_args aa = {qhl, q, cache, kv_lens, kv_len, seq_stride, g->softmax_scale, part_ml,
                           part_o, probs, kv_len, NH, HG, nchunks, QKN, chunk, slots,
                           direct ? clat : NULL, B};
    /* dynamic LDS: two 16-key cache tiles per wave (c_kv rows padded to 1056 B,
     * then the k_pe parts); also holds the waves' partial states for the merge */
    const size_t alds = (size_t)MM_MLA_AW * 2 * MM_MLA_TILE_B;   /* two sub-tile stages per wave */
    /* a row's chunks on one XCD: see mm_mla_attn_args; row groups sharing
     * a sequence: one block per group, in index order */
    const unsigned ntrip = (unsigned)Bblk * (unsigned)HG * (unsigned)nchunks;
    if ((st = mm_launch(c, rows4 ? K_MLA_ATTN_ROWS : K_MLA_ATTN, rows4 ? ntrip : 8 * ((ntrip + 7) / 8), 1, 1,
                        64 * MM_MLA_AW, rows4 ? (size_t)MM_MLA_ROWS_LDS : alds, &aa)))
        return st;
    mm_mla_combine_args ca = {part_ml, part_o, c->mla_kvb[layer], kv_lens, kv_len, ctx_out, clat,
                              probs, kv_len, B, NH, g->qk_nope_head_dim, g->v_head_dim, HG, nchunks,
                              ctx_hl};
    const unsigned zc = chunk_in > 0 ? zc_in : merge_z(NH, B);
    if (!direct && (st = mm_launch(c, K_MLA_COMBINE, (unsigned)NH, (unsigned)B, zc, 256, 0, &ca)))
        return st;
    const int vt = wide ? 16 * MM_MLA_WIDE_S : 16;
    return mm_launch(c, wide ? K_MLA_UV_W : K_MLA_UV, (unsigned)((g->v_head_dim + vt - 1) / vt), (unsigned)NH,
                     (unsigned)((B + 31) / 32), 256, 0, &ca);
}

/* ---- decode front ---------------------------------------------------------- */

/* build_rope_inv_freq (src/model_load.c:299-325), step for step in fp32. */
int mm_rope_inv_freq(int rope_dim, float theta, float factor, float beta_fast, float beta_slow,
                     float orig_max, float *inv) {
    if (!inv) return mm_fail(MM_ERR_INVALID, "mm_rope_inv_freq: NULL argument");
    if (rope_dim <= 0 || rope_dim % 2 || !(theta > 1.0f) || !(factor > 0.0f) ||
        !(beta_fast > 0.0f) || !(beta_slow > 0.0f) || !(orig_max > 0.0f))
        return mm_fail(MM_ERR_INVALID, "mm_rope_inv_freq: bad parameter");
    const float pi = 3.14159265358979323846f;
    const float lo_d = ((float)rope_dim * logf(orig_max / (beta_fast * 2.0f * pi))) /
                       (2.0f * logf(theta));
    const float hi_d = ((float)rope_dim * logf(orig_max / (beta_slow * 2.0f * pi))) /
                       (2.0f * logf(theta));
    float low = floorf(lo_d), high = ceilf(hi_d);
    if (low < 0) low = 0;
    if (high > rope_dim - 1) high = (float)(rope_dim - 1);
    const float span = high == low ? 0.001f : high - low;
    for (int j = 0; j < rope_dim / 2; j++) {
        const float f_ex = 1.0f / powf(theta, (float)(2 * j) / (float)rope_dim);
        const float f_in = f_ex / factor;
        float t = ((float)j - low) / span;
        if (t < 0) t = 0;
        if (t > 1) t = 1;
        const float m = 1.0f - t;
        inv[j] = f_in * (1.0f - m) + f_ex * m;
    }
    return MM_OK;
}

int mm_mla_front_init(mm_ctx *c, const mm_mla_front_config *cfg) {
    if (!c || !cfg || !cfg->rope_inv_freq) return mm_fail(MM_ERR_INVALID, "mm_mla_front_init: NULL argument");
    if (!c->mla_ready) return mm_fail(MM_ERR_STATE, "mm_mla_front_init: call mm_mla_init first");
    if (c->front_ready) return mm_fail(MM_ERR_STATE, "mm_mla_front_init: already initialised");
    if (cfg->hidden_size <= 0 || cfg->hidden_size % 8 || cfg->q_lora_rank < 0 || cfg->q_lora_rank % 8)
        return mm_fail(MM_ERR_INVALID, "mm_mla_front_init: hidden_size and q_lora_rank must be "
                       "multiples of 8");
    if (cfg->rope_interleaved != 0 && cfg->rope_interleaved != 1)
        return mm_fail(MM_ERR_INVALID, "mm_mla_front_init: rope_interleaved must be 0 or 1");
    const mm_mla_config *g = &c->mla;
    if (g->n_heads * g->qk_rope_head_dim / 2 > MM_ROPE_PAIRS_MAX)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_mla_front_init: n_heads * qk_rope_head_dim / 2 > %d",
                       MM_ROPE_PAIRS_MAX);
    int st = mm_set_device(c);
    if (st) return st;
    const size_t nb = (size_t)g->qk_rope_head_dim / 2 * sizeof(float);
    MM_HIP(hipMalloc((void **)&c->front_inv, nb));
    MM_HIP(hipMemcpy(c->front_inv, cfg->rope_inv_freq, nb, hipMemcpyHostToDevice));
    c->front = *cfg;
    c->front.rope_inv_freq = c->front_inv;
    c->front_ready = 1;
    return MM_OK;
}

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

int mm_mla_front_dev(mm_ctx *c, int B, const float *x, const mm_mla_front_weights *w,
                     const int32_t *pos, float *q, uint16_t *cache, int seq_stride,
                     float *kv_rows) {
    return mm_mla_front_rows(c, B, x, w, pos, NULL, q, cache, seq_stride, kv_rows, NULL, NULL, NULL,
                             NULL);
}

int mm_mla_front_rows(mm_ctx *c, int B, const float *x, const mm_mla_front_weights *w,
                      const int32_t *pos, const int32_t *slots, float *q, uint16_t *cache,
                      int seq_stride, float *kv_rows, const float *xn_pre,
                      const uint16_t *xn_pre_hl, float *comp_buf, mm_mla_rope_args *defer) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_mla_front_dev: NULL context");
    if (!c->front_ready) return mm_fail(MM_ERR_STATE, "mm_mla_front_dev: call mm_mla_front_init first");
    if (B < 0) return mm_fail(MM_ERR_INVALID, "mm_mla_front_dev: B < 0");
    if (B == 0) return MM_OK;
    const mm_mla_front_config *f = &c->front;
    const int ql = f->q_lora_rank;
    if (!x || !w || !pos || !q || !cache || !w->input_norm || !w->kv_a_proj || !w->kv_a_norm ||
        (ql ? (!w->q_a_proj || !w->q_a_norm || !w->q_b_proj) : !w->q_proj))
        return mm_fail(MM_ERR_INVALID, "mm_mla_front_dev: NULL argument");
    if (seq_stride < 1) return mm_fail(MM_ERR_INVALID, "mm_mla_front_dev: seq_stride < 1");
    const void *al[] = {x, w->input_norm, w->q_proj, w->q_a_proj, w->q_a_norm, w->q_b_proj,
                        w->kv_a_proj, w->kv_a_norm, cache};
    for (size_t i = 0; i < sizeof(al) / sizeof(al[0]); i++)
        if ((uintptr_t)al[i] % 16)
            return mm_fail(MM_ERR_INVALID, "mm_mla_front_dev: x, weights and cache must be "
                           "16-byte aligned");
    int st = mm_set_device(c);
    if (st) return st;
    const mm_mla_config *g = &c->mla;
    const int H = f->hidden_size, NH = g->n_heads;
    const int QD = NH * (g->qk_nope_head_dim + g->qk_rope_head_dim);
    const int KVD = g->kv_lora_rank + g->qk_rope_head_dim;
    const int gemv = B <= MM_GEMV_NB && H <= MM_LM_HMAX && ql <= MM_LM_HMAX;
    /* workspace: comp [B, KVD], q_a [B, q_lora]; the GEMM path adds xb [B, H]
     * and the GEMM staging */
    const size_t o_cp = 0, o_qa = al256((size_t)B * KVD * 4);
    const size_t o_xb = o_qa + al256((size_t)B * ql * 4);
    /* GEMM staging: the larger of the two passes' needs */
    size_t gw = mm_gemm_bf16_ws2_bytes(B, H, ql ? ql : QD, KVD, 0), g2;
    if (ql && (g2 = mm_gemm_bf16_ws_bytes(B, ql, QD, 0)) > gw) gw = g2;
    /* up to MM_SKINNY_T rows without q-LoRA the projections read x as bf16
     * hi/lo planes (the caller's, or this norm's), both operands through
     * one direct-to-LDS ring: the same results as the fp32-row GEMM */
    const int hl = !gemv && !ql && B <= MM_SKINNY_T && H % 64 == 0;
    if (hl && (g2 = mm_gemm_bf16_hl_ws_bytes(B, H, QD, KVD)) > gw) gw = g2;
    const size_t o_gm = o_xb + (gemv ? 0 : al256((size_t)B * H * 4));
    char *ws;
    if ((st = mm_workspace(c, o_gm + (gemv ? 0 : gw), (void **)&ws))) return st;
    float *comp = (float *)(ws + o_cp), *qa = (float *)(ws + o_qa);
    if (defer) {
        /* the deferred launch runs after later calls have reused the
         * workspace: comp lives in the caller's buffer instead */
        if (!comp_buf || B > MM_SKINNY_T)
            return mm_fail(MM_ERR_INVALID, "mm_mla_front_rows: a deferred RoPE needs comp_buf and "
                           "B <= %d", MM_SKINNY_T);
        comp = comp_buf;
    }
    if (gemv) {
        /* input norm fused; the query projection (or q_a) and kv_a in one row space */
        mm_gemv_args a = {x, w->input_norm, f->rms_eps, ql ? w->q_a_proj : w->q_proj, w->kv_a_proj,
                          ql ? qa : q, comp, ql ? ql : QD, KVD, ql ? ql : QD, KVD, B, H, 0, 0};
        if ((st = mm_gemv_launch(c, &a))) return st;
        if (ql) {
            mm_gemv_args b = {qa, w->q_a_norm, f->mla_norm_eps, w->q_b_proj, NULL, q, NULL,
                              QD, 0, QD, 0, B, ql, 0, 0};
            if ((st = mm_gemv_launch(c, &b))) return st;
        }
    } else if (hl && (xn_pre_hl || !xn_pre)) {
        char *gws = ws + o_gm;
        const uint16_t *xhl = xn_pre_hl;
        if (!xhl) {   /* the norm writes the planes (the o_xb region holds them) */
            uint16_t *p = (uint16_t *)(ws + o_xb);
            mm_rmsnorm_hl_args rh = {x, w->input_norm, p, H, f->rms_eps};
            if ((st = mm_launch(c, K_RMSNORM_HL, (unsigned)B, 1, 1, 256, 0, &rh))) return st;
            xhl = p;
        }
        if ((st = mm_gemm_bf16_hl(c, q, w->q_proj, QD, comp, w->kv_a_proj, KVD, xhl, H, B, 0, gws)))
            return st;
    } else {
        const float *xb = (float *)(ws + o_xb);
        char *gws = ws + o_gm;
        if (xn_pre) {
            xb = (float *)xn_pre;      /* rmsnorm(x, input_norm), computed by the caller */
        } else {
            mm_rmsnorm_args ra = {x, w->input_norm, (float *)xb, H, f->rms_eps};
            if ((st = mm_launch(c, K_RMSNORM, (unsigned)B, 1, 1, 256, 0, &ra))) return st;
        }
        /* the query projection (or q_a) and kv_a over the same xb: one pass */
        if ((st = mm_gemm_bf16_ws2(c, ql ? qa : q, ql ? w->q_a_proj : w->q_proj, ql ? ql : QD, comp,
                                   w->kv_a_proj, KVD, xb, H, B, 0, gws)))
            return st;
        if (ql) {
            mm_rmsnorm_args qn = {qa, w->q_a_norm, qa, ql, f->mla_norm_eps};
            if ((st = mm_launch(c, K_RMSNORM, (unsigned)B, 1, 1, 256, 0, &qn))) return st;
            if ((st = mm_gemm_bf16_ws(c, q, qa, w->q_b_proj, QD, ql, B, 0, gws))) return st;
        }
    }
    mm_mla_rope_args r = {q, comp, w->kv_a_norm, c->front_inv, pos, cache, kv_rows, B, NH,
                          g->qk_nope_head_dim, g->qk_rope_head_dim, g->kv_lora_rank, seq_stride,
                          f->rope_interleaved, f->mla_norm_eps, slots};
    if (defer) {
        *defer = r;
        return MM_OK;
    }
    return mm_launch(c, K_MLA_ROPE, (unsigned)B, 1, 1, 256, 0, &r);
}
