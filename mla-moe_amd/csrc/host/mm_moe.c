/* mm_moe.c -- MoE FFN layer registry and forward pass (host side).
 *
 * Mirrors the reference's ffn_compute (src/run.c:116-162) over T tokens.
 * Weight upload replaces the reference GPU driver's warm_up packing
 * (src/getp_run.hip:58-113, 781-808): every layer owns one device pool per
 * weight format, and the router weight is kept transposed in fp32 for the
 * sequential-order router.
 */
#include <stdlib.h>
#include <string.h>

#include "mm_internal.h"

#define BF16_NT_MAX 8         /* tokens per pass of the bf16 GEMV path */
#define GU_ROWS_PER_BLOCK 4   /* one gate/up row pair per wave */
#define DOWN_ROWS_PER_BLOCK 4 /* one output row per wave */
#define ROUTER_TOKENS_PER_BLOCK 8

void mm_moe_release(mm_ctx *c) {
    if (!c->layers) return;
    for (int l = 0; l < c->n_layers; l++) {
        mm_moe_layer *L = &c->layers[l];
        if (L->wgT) hipFree(L->wgT);
        if (L->bias) hipFree(L->bias);
        if (L->bf16_pool) hipFree(L->bf16_pool);
    }
    free(c->layers);
    c->layers = NULL;
    c->moe_ready = 0;
}

int mm_moe_init(mm_ctx *c, const mm_moe_config *cfg, int n_layers) {
    if (!c || !cfg) return mm_fail(MM_ERR_INVALID, "mm_moe_init: NULL argument");
    if (c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_init: already initialised");
    const int H = cfg->hidden_size, E = cfg->n_routed_experts, K = cfg->n_experts_per_tok;
    const int I = cfg->moe_inter_size, NS = cfg->n_shared_experts;
    if (n_layers <= 0 || H <= 0 || E <= 0 || K <= 0 || I <= 0 || NS < 0)
        return mm_fail(MM_ERR_INVALID, "mm_moe_init: non-positive dimension");
    /* run.c:133-134 limits K <= 16 and E <= 1024; this build routes E <= 256 */
    if (K > 16 || K > E) return mm_fail(MM_ERR_INVALID, "mm_moe_init: need K <= min(16, E)");
    if (E > 256) return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_init: E > 256 experts");
    if (H % 8 || I % 8)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_init: hidden and moe_inter must be multiples of 8");
    c->layers = calloc((size_t)n_layers, sizeof(mm_moe_layer));
    if (!c->layers) return mm_fail(MM_ERR_NOMEM, "mm_moe_init: calloc");
    c->moe = *cfg;
    c->n_layers = n_layers;
    c->moe_ready = 1;
    return MM_OK;
}

static int upload(mm_ctx *c, void *dst, const void *src, size_t bytes, int dev) {
    if (!src) return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: NULL weight pointer");
    MM_HIP(hipMemcpyAsync(dst, src, bytes, dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                          c->stream));
    return MM_OK;
}

int mm_moe_load_layer(mm_ctx *c, int layer, const mm_moe_layer_weights *w, unsigned flags) {
    if (!c || !w) return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: NULL argument");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_load_layer: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: layer %d out of range", layer);
    if (!(flags & (MM_LOAD_BF16 | MM_LOAD_INT8)))
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: no weight format requested");
    if (flags & MM_LOAD_INT8)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_load_layer: int8 format not built yet");
    if (!w->moe_gate || !w->expert_gate || !w->expert_up || !w->expert_down)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: NULL weight pointer");
    int st = mm_set_device(c);
    if (st) return st;
    const mm_moe_config *g = &c->moe;
    const size_t H = g->hidden_size, E = g->n_routed_experts, I = g->moe_inter_size;
    const size_t S = (size_t)g->n_shared_experts * I;
    const int dev = (flags & MM_LOAD_DEVICE_PTRS) != 0;
    mm_moe_layer *L = &c->layers[layer];
    if (L->loaded) return mm_fail(MM_ERR_STATE, "mm_moe_load_layer: layer %d already loaded", layer);

    uint16_t *gate_tmp = NULL;
    MM_HIP(hipMalloc((void **)&L->wgT, H * E * sizeof(float)));
    MM_HIP(hipMalloc((void **)&gate_tmp, H * E * sizeof(uint16_t)));
    if ((st = upload(c, gate_tmp, w->moe_gate, H * E * 2, dev))) goto out;
    mm_transpose_gate_args ta = {gate_tmp, L->wgT, (int)E, (int)H};
    if ((st = mm_launch(c, K_TRANSPOSE_GATE, 1024, 1, 1, 256, 0, &ta))) goto out;
    if (w->moe_gate_bias) {
        if (hipMalloc((void **)&L->bias, E * sizeof(float)) != hipSuccess) {
            st = mm_fail(MM_ERR_NOMEM, "mm_moe_load_layer: bias");
            goto out;
        }
        if ((st = upload(c, L->bias, w->moe_gate_bias, E * sizeof(float), dev))) goto out;
    }
    if (flags & MM_LOAD_BF16) {
        const size_t ne = I * H;   /* elements per expert matrix */
        const size_t total = 3 * E * ne + 3 * S * H;
        if (hipMalloc((void **)&L->bf16_pool, total * sizeof(uint16_t)) != hipSuccess) {
            st = mm_fail(MM_ERR_NOMEM, "mm_moe_load_layer: bf16 pool of %zu bytes", total * 2);
            goto out;
        }
        L->eg = L->bf16_pool;
        L->eu = L->eg + E * ne;
        L->ed = L->eu + E * ne;
        L->sg = L->ed + E * ne;
        L->su = L->sg + S * H;
        L->sd = L->su + S * H;
        for (size_t e = 0; e < E && !st; e++) {
            st = upload(c, L->eg + e * ne, w->expert_gate[e], ne * 2, dev);
            if (!st) st = upload(c, L->eu + e * ne, w->expert_up[e], ne * 2, dev);
            if (!st) st = upload(c, L->ed + e * ne, w->expert_down[e], ne * 2, dev);
        }
        if (!st && S) {
            st = upload(c, L->sg, w->shared_gate, S * H * 2, dev);
            if (!st) st = upload(c, L->su, w->shared_up, S * H * 2, dev);
            if (!st) st = upload(c, L->sd, w->shared_down, S * H * 2, dev);
        }
        if (st) goto out;
    }
    L->formats = flags & (MM_LOAD_BF16 | MM_LOAD_INT8);
    L->loaded = 1;
out:;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (gate_tmp) hipFree(gate_tmp);
    if (!st && e != hipSuccess) st = mm_hip_fail(e, "mm_moe_load_layer");
    return st;
}

/* bf16 weights, GEMV stages (kernels/moe_bf16.hip), BF16_NT_MAX tokens per pass. */
static int forward_bf16(mm_ctx *c, const mm_moe_layer *L, int T, const float *xn, float *out,
                        const float *logits, int32_t *idx, float *wts, float *probs, int acc) {
    const mm_moe_config *g = &c->moe;
    const int H = g->hidden_size, E = g->n_routed_experts, K = g->n_experts_per_tok;
    const int I = g->moe_inter_size, S = g->n_shared_experts * I;
    const size_t hw = (size_t)K * I + S;
    void *ws;
    int st = mm_workspace(c, (size_t)BF16_NT_MAX * hw * sizeof(float), &ws);
    if (st) return st;
    float *hcat = ws;
    for (int t0 = 0; t0 < T; t0 += BF16_NT_MAX) {
        const int Tc = T - t0 < BF16_NT_MAX ? T - t0 : BF16_NT_MAX;
        mm_gu_bf16_args a;
        memset(&a, 0, sizeof(a));
        a.r.x = xn + (size_t)t0 * H;
        a.r.wgT = L->wgT;
        a.r.logits_in = logits ? logits + (size_t)t0 * E : NULL;
        a.r.bias = L->bias;
        a.r.probs = probs ? probs + (size_t)t0 * E : NULL;
        a.r.topk_idx = idx + (size_t)t0 * K;
        a.r.topk_w = wts + (size_t)t0 * K;
        a.r.T = Tc;
        a.r.H = H;
        a.r.E = E;
        a.r.K = K;
        a.r.sigmoid = g->router_sigmoid;
        a.r.norm_topk = g->norm_topk;
        a.r.scale = g->routed_scaling;
        a.r.n_router_blocks = (Tc + ROUTER_TOKENS_PER_BLOCK - 1) / ROUTER_TOKENS_PER_BLOCK;
        a.x = xn + (size_t)t0 * H;
        a.gate = L->sg;
        a.up = L->su;
        a.hcat = hcat;
        a.T = Tc;
        a.H = H;
        a.I = I;
        a.S = S;
        a.K = K;
        a.rows_per_block = GU_ROWS_PER_BLOCK;
        unsigned nb1 = a.r.n_router_blocks + (S + GU_ROWS_PER_BLOCK - 1) / GU_ROWS_PER_BLOCK;
        if ((st = mm_launch(c, K_MOE_BF16_S1, nb1, 1, 1, 256, 0, &a))) return st;

        a.gate = L->eg;
        a.up = L->eu;
        a.n_blocks_per_token = (I + GU_ROWS_PER_BLOCK - 1) / GU_ROWS_PER_BLOCK;
        if ((st = mm_launch(c, K_MOE_BF16_S2, a.n_blocks_per_token, Tc * K, 1, 256, 0, &a)))
            return st;

        mm_down_bf16_args d = {hcat, L->ed, L->sd, idx + (size_t)t0 * K, out + (size_t)t0 * H,
                               Tc, H, I, S, K, E, acc, DOWN_ROWS_PER_BLOCK};
        if ((st = mm_launch(c, K_MOE_BF16_S3, (H + DOWN_ROWS_PER_BLOCK - 1) / DOWN_ROWS_PER_BLOCK,
                            Tc, 1, 256, 0, &d)))
            return st;
    }
    return MM_OK;
}

/* Device scratch for the routing results the caller did not ask for. */
static int routing_scratch(mm_ctx *c, int T, int32_t **idx, float **w) {
    const int K = c->moe.n_experts_per_tok, H = c->moe.hidden_size;
    const int I = c->moe.moe_inter_size, S = c->moe.n_shared_experts * I;
    const size_t hbytes = (size_t)BF16_NT_MAX * ((size_t)K * I + S) * sizeof(float);
    const size_t rbytes = (size_t)T * K * (sizeof(int32_t) + sizeof(float));
    (void)H;
    void *ws;
    int st = mm_workspace(c, hbytes + rbytes, &ws);
    if (st) return st;
    char *p = (char *)ws + hbytes;
    if (!*idx) *idx = (int32_t *)p;
    if (!*w) *w = (float *)(p + (size_t)T * K * sizeof(int32_t));
    return MM_OK;
}

int mm_moe_forward_dev(mm_ctx *c, int layer, int T, const float *xn, float *out,
                       const float *logits, int32_t *topk_idx, float *topk_w, float *probs,
                       unsigned flags) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_moe_forward_dev: NULL context");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_forward_dev: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers || !c->layers[layer].loaded)
        return mm_fail(MM_ERR_STATE, "mm_moe_forward_dev: layer %d not loaded", layer);
    if (T < 0 || !out || (!xn && T > 0))
        return mm_fail(MM_ERR_INVALID, "mm_moe_forward_dev: bad arguments");
    if (T == 0) return MM_OK;
    if ((uintptr_t)xn % 16 || (uintptr_t)out % 16)
        return mm_fail(MM_ERR_INVALID, "mm_moe_forward_dev: xn/out must be 16-byte aligned");
    const mm_moe_layer *L = &c->layers[layer];
    int st = mm_set_device(c);
    if (st) return st;
    const int acc = (flags & MM_FWD_ACCUMULATE) != 0;
    if (flags & MM_FWD_INT8)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_forward_dev: int8 path not built yet");
    if (!(L->formats & MM_LOAD_BF16))
        return mm_fail(MM_ERR_STATE, "mm_moe_forward_dev: layer %d has no bf16 weights", layer);
    if (xn == out) return mm_fail(MM_ERR_INVALID, "mm_moe_forward_dev: bf16 path needs out != xn");
    int32_t *idx = topk_idx;
    float *w = topk_w;
    if ((st = routing_scratch(c, T, &idx, &w))) return st;
    return forward_bf16(c, L, T, xn, out, logits, idx, w, probs, acc);
}

int mm_ffn_compute(mm_ctx *c, int layer, const float *xn, float *out, int *topk_idx,
                   float *topk_w, unsigned flags) {
    if (!c || !xn || !out) return mm_fail(MM_ERR_INVALID, "mm_ffn_compute: NULL argument");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_ffn_compute: call mm_moe_init first");
    const int H = c->moe.hidden_size, K = c->moe.n_experts_per_tok;
    int st = mm_set_device(c);
    if (st) return st;
    /* private device staging: [x | out | idx | w] */
    char *buf = NULL;
    const size_t bytes = 2 * (size_t)H * sizeof(float) + (size_t)K * 8;
    MM_HIP(hipMalloc((void **)&buf, bytes));
    float *dx = (float *)buf, *dout = dx + H;
    int32_t *didx = (int32_t *)(dout + H);
    float *dw = (float *)(didx + K);
    if (!(st = mm_h2d(c, dx, xn, (size_t)H * sizeof(float))))
        st = mm_moe_forward_dev(c, layer, 1, dx, dout, NULL, didx, dw, NULL,
                                flags & ~(unsigned)MM_FWD_ACCUMULATE);
    if (!st) st = mm_d2h(c, out, dout, (size_t)H * sizeof(float));
    if (!st && topk_idx) st = mm_d2h(c, topk_idx, didx, (size_t)K * sizeof(int32_t));
    if (!st && topk_w) st = mm_d2h(c, topk_w, dw, (size_t)K * sizeof(float));
    hipStreamSynchronize(c->stream);
    hipFree(buf);
    return st;
}
