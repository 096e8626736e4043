/* mm_host.c -- the synchronous host-pointer entry points.
 *
 * The reference's hot-path functions take host arrays and return with the
 * result in them: matmul (src/run.c:29-37), ffn_compute (src/run.c:116-162)
 * and the absorbed per-head chain of forward_absorbed (src/run.c:430-460).
 * These entry points keep that contract over the device paths: the inputs
 * are staged into a device buffer owned by the context, the *_dev entry
 * point runs on the context stream, the outputs are copied back and the
 * call returns after the stream has drained.  Host weights passed to
 * mm_matmul_bf16 are uploaded once and kept (the reference's weights are
 * read-only mappings of the checkpoint, include/model.h:44-46).
 */
#include <stdlib.h>
#include <string.h>

#include "mm_internal.h"

struct mm_wcache_entry {
    const void *host;
    size_t bytes;
    void *dev;
};

void mm_host_release(mm_ctx *c) {
    for (size_t i = 0; i < c->wcache_n; i++) hipFree(c->wcache[i].dev);
    free(c->wcache);
    c->wcache = NULL;
    c->wcache_n = c->wcache_cap = 0;
}

int mm_host_weights_release(mm_ctx *c) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_host_weights_release: NULL context");
    int st = mm_set_device(c);
    if (st) return st;
    MM_HIP(hipStreamSynchronize(c->stream));
    mm_host_release(c);
    return MM_OK;
}

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

/* Queue a host -> device (or back) copy on the context stream. */
static int put(mm_ctx *c, void *d, const void *h, size_t bytes) {
    if (bytes) MM_HIP(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, c->stream));
    return MM_OK;
}
static int get(mm_ctx *c, void *h, const void *d, size_t bytes) {
    if (h && bytes) MM_HIP(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, c->stream));
    return MM_OK;
}

/* Wait for the stream; the first error of the call wins. */
static int drain(mm_ctx *c, int st) {
    hipError_t e = hipStreamSynchronize(c->stream);
    if (!st && e != hipSuccess) st = mm_hip_fail(e, "hipStreamSynchronize");
    return st;
}

/* ---- MoE FFN --------------------------------------------------------------- */

int mm_moe_forward(mm_ctx *c, int layer, int T, const float *xn, float *out, int32_t *topk_idx,
                   float *topk_w, float *probs, unsigned flags) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: NULL context");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_forward: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers || !c->layers[layer].loaded)
        return mm_fail(MM_ERR_STATE, "mm_moe_forward: layer %d not loaded", layer);
    if (T < 0 || (T > 0 && (!xn || !out))) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: bad arguments");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    const size_t H = c->moe.hidden_size, E = c->moe.n_routed_experts, K = c->moe.n_experts_per_tok;
    const int dense = c->layers[layer].dense;
    const int acc = (flags & MM_FWD_ACCUMULATE) != 0;
    const size_t bx = (size_t)T * H * 4, bk = (size_t)T * K * 4, be = (size_t)T * E * 4;
    const size_t o_x = 0, o_o = al256(bx), o_i = o_o + al256(bx), o_w = o_i + al256(bk);
    const size_t o_p = o_w + al256(bk);
    char *io;
    if ((st = mm_io_buffer(c, o_p + al256(be), (void **)&io))) return st;
    float *dx = (float *)(io + o_x), *dout = (float *)(io + o_o), *dw = (float *)(io + o_w);
    int32_t *didx = (int32_t *)(io + o_i);
    float *dp = (float *)(io + o_p);
    if (!(st = put(c, dx, xn, bx)) && acc) st = put(c, dout, out, bx);
    if (!st)
        st = mm_moe_forward_dev(c, layer, T, dx, dout, NULL, topk_idx ? didx : NULL,
                                topk_w ? dw : NULL, probs ? dp : NULL, flags);
    if (!st) st = get(c, out, dout, bx);
    if (!st && !dense) {   /* a dense layer leaves them as they were (src/run.c:119-122) */
        if (!(st = get(c, topk_idx, didx, bk)) && !(st = get(c, topk_w, dw, bk)))
            st = get(c, probs, dp, be);
    }
    return drain(c, st);
}

int mm_ffn_compute(mm_ctx *c, int layer, const float *xn, float *out, int *topk_idx,
                   float *topk_w, float *probs, unsigned flags) {
    if (!c || !xn || !out) return mm_fail(MM_ERR_INVALID, "mm_ffn_compute: NULL argument");
    return mm_moe_forward(c, layer, 1, xn, out, topk_idx, topk_w, probs,
                          flags & ~(unsigned)MM_FWD_ACCUMULATE);
}

/* ---- dense matmul ------------------------------------------------------------ */

/* The device copy of host weight w ([d_out, n_in] bf16), uploaded on first use. */
static int cached_weight(mm_ctx *c, const uint16_t *w, size_t bytes, const uint16_t **dw) {
    for (size_t i = 0; i < c->wcache_n; i++)
        if (c->wcache[i].host == w && c->wcache[i].bytes == bytes) {
            *dw = c->wcache[i].dev;
            return MM_OK;
        }
    if (c->wcache_n == c->wcache_cap) {
        const size_t cap = c->wcache_cap ? 2 * c->wcache_cap : 64;
        struct mm_wcache_entry *p = realloc(c->wcache, cap * sizeof(*p));
        if (!p) return mm_fail(MM_ERR_NOMEM, "mm_matmul_bf16: weight cache");
        c->wcache = p;
        c->wcache_cap = cap;
    }
    void *d = NULL;
    MM_HIP(hipMalloc(&d, bytes));
    hipError_t e = hipMemcpyAsync(d, w, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        hipFree(d);
        return mm_hip_fail(e, "mm_matmul_bf16: weight upload");
    }
    c->wcache[c->wcache_n++] = (struct mm_wcache_entry){w, bytes, d};
    *dw = d;
    return MM_OK;
}

int mm_matmul_bf16(mm_ctx *c, float *y, const float *x, const uint16_t *w, int d_out, int n_in,
                   int T, unsigned flags) {
    if (!c || (T > 0 && (!y || !x || !w))) return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16: NULL argument");
    if (T < 0 || d_out <= 0 || n_in <= 0) return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16: bad shape");
    if (n_in % 8) return mm_fail(MM_ERR_UNSUPPORTED, "mm_matmul_bf16: n_in must be a multiple of 8");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    const uint16_t *dw = w;
    if ((flags & MM_MATMUL_W_HOST) &&
        (st = cached_weight(c, w, (size_t)d_out * n_in * sizeof(uint16_t), &dw)))
        return st;
    const size_t bx = (size_t)T * n_in * 4, by = (size_t)T * d_out * 4;
    char *io;
    if ((st = mm_io_buffer(c, al256(bx) + by, (void **)&io))) return st;
    float *dx = (float *)io, *dy = (float *)(io + al256(bx));
    if (!(st = put(c, dx, x, bx)) && (flags & MM_MATMUL_ACCUMULATE)) st = put(c, dy, y, by);
    if (!st)
        st = mm_matmul_bf16_dev(c, dy, dx, dw, d_out, n_in, T,
                                flags & (MM_MATMUL_X_BF16 | MM_MATMUL_ACCUMULATE));
    if (!st) st = get(c, y, dy, by);
    return drain(c, st);
}

/* ---- MLA absorbed decode ------------------------------------------------------- */

int mm_mla_absorbed_decode(mm_ctx *c, int layer, int B, const float *q, const float *cache,
                           int seq_stride, const int32_t *kv_lens, int kv_len, float *ctx_out,
                           float *qabs, float *probs, float *clat) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode: NULL context");
    if (!c->mla_ready || layer < 0 || layer >= c->mla_layers || !c->mla_kvb[layer])
        return mm_fail(MM_ERR_STATE, "mm_mla_absorbed_decode: layer %d not loaded", layer);
    if (B < 0 || (B > 0 && (!q || !cache || !ctx_out)))
        return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode: NULL argument");
    if (B == 0) return MM_OK;
    if (kv_len < 1 || kv_len > MM_MAX_KV_LEN || seq_stride < kv_len)
        return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode: need 1 <= kv_len <= seq_stride and "
                       "kv_len <= %d", MM_MAX_KV_LEN);
    if (kv_lens)
        for (int b = 0; b < B; b++)
            if (kv_lens[b] < 1 || kv_lens[b] > kv_len)
                return mm_fail(MM_ERR_INVALID, "mm_mla_absorbed_decode: kv_lens[%d] = %d outside "
                               "[1, kv_len]", b, kv_lens[b]);
    int st = mm_set_device(c);
    if (st) return st;
    const mm_mla_config *g = &c->mla;
    const size_t NH = g->n_heads, QD = g->qk_nope_head_dim + g->qk_rope_head_dim;
    const size_t KVD = g->kv_lora_rank + g->qk_rope_head_dim, KVL = g->kv_lora_rank;
    const size_t rows = (size_t)B * kv_len;
    const size_t bq = B * NH * QD * 4, bcf = rows * KVD * 4, bcb = rows * KVD * 2;
    const size_t bl = (size_t)B * 4, bo = B * NH * g->v_head_dim * 4, bla = B * NH * KVL * 4;
    const size_t bp = B * NH * (size_t)kv_len * 4;
    size_t off[8], n = 0;
    const size_t sz[8] = {bq, bcf, bcb, bl, bo, bla, bp, bla};
    for (int i = 0; i < 8; i++) {
        off[i] = n;
        n += al256(sz[i]);
    }
    char *io;
    if ((st = mm_io_buffer(c, n, (void **)&io))) return st;
    float *dq = (float *)(io + off[0]), *dcf = (float *)(io + off[1]);
    uint16_t *dcb = (uint16_t *)(io + off[2]);
    int32_t *dl = (int32_t *)(io + off[3]);
    float *dctx = (float *)(io + off[4]), *dqa = (float *)(io + off[5]);
    float *dp = (float *)(io + off[6]), *dcl = (float *)(io + off[7]);
    /* the first kv_len rows of each sequence, packed at stride kv_len */
    if (!(st = put(c, dq, q, bq)) && !(st = put(c, dl, kv_lens, kv_lens ? bl : 0))) {
        hipError_t e = hipMemcpy2DAsync(dcf, (size_t)kv_len * KVD * 4, cache,
                                        (size_t)seq_stride * KVD * 4, (size_t)kv_len * KVD * 4,
                                        (size_t)B, hipMemcpyHostToDevice, c->stream);
        if (e != hipSuccess) st = mm_hip_fail(e, "mm_mla_absorbed_decode: cache upload");
    }
    if (!st) {
        mm_f32_bf16_args ca = {dcf, dcb, (uint64_t)rows * KVD};
        const size_t blocks = (rows * KVD + 255) / 256 < 8192 ? (rows * KVD + 255) / 256 : 8192;
        st = mm_launch(c, K_F32_BF16, (unsigned)blocks, 1, 1, 256, 0, &ca);
    }
    if (!st)
        st = mm_mla_absorbed_decode_dev(c, layer, B, dq, dcb, kv_len, kv_lens ? dl : NULL, kv_len,
                                        dctx, qabs ? dqa : NULL, probs ? dp : NULL,
                                        clat ? dcl : NULL);
    if (!st && !(st = get(c, ctx_out, dctx, bo)) && !(st = get(c, qabs, dqa, bla)) &&
        !(st = get(c, probs, dp, bp)))
        st = get(c, clat, dcl, bla);
    return drain(c, st);
}
