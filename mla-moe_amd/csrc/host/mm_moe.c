/* mm_moe.c -- MoE FFN layer registry and forward pass (host side).
 *
 * Mirrors the reference's ffn_compute (src/run.c:116-162) over T tokens.
 * Weight upload replaces the reference GPU driver's warm_up packing
 * (src/getp_run.hip:58-113, 781-808): every layer owns one device pool per
 * weight format; the router weight is kept as the checkpoint's bf16 [E, H]
 * for the sequential-order router.
 */
#include <stdlib.h>
#include <string.h>

#include "mm_internal.h"

#define BF16_NT_MAX 8         /* tokens per pass of the bf16 GEMV path */
#define GU_ROWS_PER_BLOCK 4   /* stage 1: one gate/up row pair per wave */
#define GU2_ROWS_PER_BLOCK 8  /* stage 2: two row pairs per wave (one round of loads) */
#define RSH_ROWS_PER_BLOCK 16 /* shared gate/up beside the router: four row pairs per wave */
#define RSH_TMAX 4            /* tokens up to which the shared gate/up joins the router launch */
#define DOWN_ROWS_PER_BLOCK 4 /* one output row per wave (the LDS-staged form needs exactly this) */
#define DN_LDS_MAX 65536      /* stage 3 stages the hidden row in LDS up to this many bytes */
#define ROUTER_TOKENS_PER_BLOCK (4 * MM_ROUTER_TPW)

void mm_moe_release(mm_ctx *c) {
    if (!c->layers) return;
    for (int l = 0; l < c->n_layers; l++) {
        mm_moe_layer *L = &c->layers[l];
        if (L->wg) hipFree(L->wg);
        if (L->bias) hipFree(L->bias);
        if (L->bf16_pool) hipFree(L->bf16_pool);
        if (L->i8_pool) hipFree(L->i8_pool);
        if (L->i8_scales) hipFree(L->i8_scales);
    }
    free(c->layers);
    c->layers = NULL;
    if (c->moe_cnt) hipFree(c->moe_cnt);
    c->moe_cnt = NULL;
    c->moe_ready = 0;
}

int mm_moe_init(mm_ctx *c, const mm_moe_config *cfg, int n_layers) {
    if (!c || !cfg) return mm_fail(MM_ERR_INVALID, "mm_moe_init: NULL argument");
    if (c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_init: already initialised");
    const int H = cfg->hidden_size, E = cfg->n_routed_experts, K = cfg->n_experts_per_tok;
    const int I = cfg->moe_inter_size, NS = cfg->n_shared_experts;
    if (n_layers <= 0 || H <= 0 || E <= 0 || K <= 0 || I <= 0 || NS < 0)
        return mm_fail(MM_ERR_INVALID, "mm_moe_init: non-positive dimension");
    /* run.c:133-134 limits K <= 16 and E <= 1024 (above MM_EMAX_FAST experts
     * the wide routers serve) */
    if (K > 16 || K > E) return mm_fail(MM_ERR_INVALID, "mm_moe_init: need K <= min(16, E)");
    if (E > MM_EMAX) return mm_fail(MM_ERR_INVALID, "mm_moe_init: E > %d experts", MM_EMAX);
    if (H % 8 || I % 8)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_init: hidden and moe_inter must be multiples of 8");
    int st = mm_set_device(c);
    if (st) return st;
    /* per-expert counters of the tiled int8 path, or per-token counters of
     * the bf16 router + shared launch (RSH_TMAX tokens): zero between calls */
    const size_t ncnt = (size_t)E * MM_CNT_STRIDE;   /* >= RSH_TMAX */
    MM_HIP(hipMalloc((void **)&c->moe_cnt, ncnt * sizeof(int32_t)));
    MM_HIP(hipMemsetAsync(c->moe_cnt, 0, ncnt * sizeof(int32_t), c->stream));
    MM_HIP(hipStreamSynchronize(c->stream));
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

/* ---- int8 weights -------------------------------------------------------- */

/* Device copy of one expert family (E matrices of n elements). */
static int gather_family(mm_ctx *c, uint16_t *dst, const uint16_t *const *src, size_t E,
                         size_t n, int dev) {
    for (size_t e = 0; e < E; e++) {
        int st = upload(c, dst + e * n, src[e], n * 2, dev);
        if (st) return st;
    }
    return MM_OK;
}

static int quant_rows_dev(mm_ctx *c, const uint16_t *src, size_t rows, size_t K, int8_t *q,
                          float *s) {
    mm_quant_w_args a = {src, q, s, (int)rows, (int)K};
    return mm_launch(c, K_QUANT_W, (unsigned)((rows + 3) / 4), 1, 1, 256, 0, &a);
}

static int pack_dev(mm_ctx *c, const int8_t *s0, const int8_t *s1, int8_t *dst, size_t N, size_t K) {
    mm_pack_i8_args a = {s0, s1, dst, (int)N, (int)K};
    size_t threads = (N / 16) * (s1 ? 2 : 1) * (K / 64) * 64;
    size_t blocks = (threads + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    return mm_launch(c, K_PACK_I8, (unsigned)blocks, 1, 1, 256, 0, &a);
}

/* Quantise every expert matrix per output channel (s = max|w|/127) and pack
 * it into MFMA fragment order (kernel_params.h, mm_i8_weights). */
/* The packed int8 layer: one pool of fragments, gate/up [E][I/16][H/64][2]
 * then down [E][H/16][I/64], then the shared expert's gate/up and down
 * likewise (16 x 64-byte fragments, mm_pack_i8), and one scale table
 * s_g [E*I] | s_u [E*I] | s_d [E*H] | ss_g [S] | ss_u [S] | ss_d [H]. */
static void i8_sizes(const mm_moe_config *g, size_t *pool, size_t *nsc) {
    const size_t H = g->hidden_size, E = g->n_routed_experts, I = g->moe_inter_size;
    const size_t S = (size_t)g->n_shared_experts * I;
    *pool = 3 * E * I * H + 3 * S * H;
    *nsc = 2 * E * I + E * H + 2 * S + H;
}

/* Allocate the pool and scales of L and point L->i8 into them. */
static int i8_alloc(mm_ctx *c, mm_moe_layer *L) {
    const mm_moe_config *g = &c->moe;
    const size_t H = g->hidden_size, E = g->n_routed_experts, I = g->moe_inter_size;
    const size_t S = (size_t)g->n_shared_experts * I;
    size_t pool, nsc;
    i8_sizes(g, &pool, &nsc);
    MM_HIP(hipMalloc((void **)&L->i8_pool, pool));
    MM_HIP(hipMalloc((void **)&L->i8_scales, nsc * sizeof(float)));
    mm_i8_weights *q = &L->i8;
    q->gu = L->i8_pool;
    q->d = q->gu + 2 * E * I * H;
    q->sgu = q->d + E * I * H;
    q->sdn = q->sgu + 2 * S * H;
    float *sc = L->i8_scales;
    q->s_g = sc;
    q->s_u = sc + E * I;
    q->s_d = sc + 2 * E * I;
    q->ss_g = sc + 2 * E * I + E * H;
    q->ss_u = q->ss_g + S;
    q->ss_d = q->ss_u + S;
    return MM_OK;
}

static int load_int8(mm_ctx *c, mm_moe_layer *L, const mm_moe_layer_weights *w, int dev) {
    const mm_moe_config *g = &c->moe;
    const size_t H = g->hidden_size, E = g->n_routed_experts, I = g->moe_inter_size;
    const size_t S = (size_t)g->n_shared_experts * I;
    const size_t ne = I * H;
    int st = i8_alloc(c, L);
    if (st) return st;
    mm_i8_weights *q = &L->i8;

    const size_t fam = E * ne > S * H ? E * ne : S * H;
    uint16_t *tb = NULL;
    int8_t *t0 = NULL, *t1 = NULL;
    if (hipMalloc((void **)&tb, fam * 2) != hipSuccess || hipMalloc((void **)&t0, fam) != hipSuccess ||
        hipMalloc((void **)&t1, fam) != hipSuccess) {
        st = mm_fail(MM_ERR_NOMEM, "mm_moe_load_layer: int8 staging buffers");
        goto out;
    }
    /* routed gate / up: [E*I, H] rows, interleaved per 16-row block */
    const uint16_t *src;
    if (L->eg) src = L->eg;
    else if (!(st = gather_family(c, tb, w->expert_gate, E, ne, dev))) src = tb;
    if (st || (st = quant_rows_dev(c, src, E * I, H, t0, (float *)q->s_g))) goto out;
    if (L->eu) src = L->eu;
    else if (!(st = gather_family(c, tb, w->expert_up, E, ne, dev))) src = tb;
    if (st || (st = quant_rows_dev(c, src, E * I, H, t1, (float *)q->s_u))) goto out;
    for (size_t e = 0; e < E && !st; e++)
        st = pack_dev(c, t0 + e * ne, t1 + e * ne, (int8_t *)q->gu + e * 2 * ne, I, H);
    if (st) goto out;
    /* routed down: [E*H, I] */
    if (L->ed) src = L->ed;
    else if (!(st = gather_family(c, tb, w->expert_down, E, ne, dev))) src = tb;
    if (st || (st = quant_rows_dev(c, src, E * H, I, t0, (float *)q->s_d))) goto out;
    for (size_t e = 0; e < E && !st; e++)
        st = pack_dev(c, t0 + e * ne, NULL, (int8_t *)q->d + e * ne, H, I);
    if (st) goto out;
    /* shared expert */
    if (S) {
        if (L->sg) src = L->sg;
        else if (!(st = upload(c, tb, w->shared_gate, S * H * 2, dev))) src = tb;
        if (st || (st = quant_rows_dev(c, src, S, H, t0, (float *)q->ss_g))) goto out;
        if (L->su) src = L->su;
        else if (!(st = upload(c, tb, w->shared_up, S * H * 2, dev))) src = tb;
        if (st || (st = quant_rows_dev(c, src, S, H, t1, (float *)q->ss_u))) goto out;
        if ((st = pack_dev(c, t0, t1, (int8_t *)q->sgu, S, H))) goto out;
        if (L->sd) src = L->sd;
        else if (!(st = upload(c, tb, w->shared_down, S * H * 2, dev))) src = tb;
        if (st || (st = quant_rows_dev(c, src, H, S, t0, (float *)q->ss_d))) goto out;
        if ((st = pack_dev(c, t0, NULL, (int8_t *)q->sdn, H, S))) goto out;
    } else if (hipMemsetAsync((void *)q->ss_d, 0, H * sizeof(float), c->stream) != hipSuccess) {
        /* no shared expert: its scale slot holds zeros, as in the packed format */
        st = mm_fail(MM_ERR_HIP, "mm_moe_load_layer: clearing the shared scales");
        goto out;
    }
out:;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (tb) hipFree(tb);
    if (t0) hipFree(t0);
    if (t1) hipFree(t1);
    if (!st && e != hipSuccess) st = mm_hip_fail(e, "mm_moe_load_layer(int8)");
    return st;
}

/* Shapes the int8 kernels take: K dimensions (hidden, moe_inter and the
 * shared experts' concatenated inter size) multiples of 64 and below 2^16
 * (the tiled GEMMs' 32-bit activation offsets leave 2^16 past the matrix
 * for padding rows). */
static int i8_cfg_ok(const mm_moe_config *g) {
    return g->hidden_size > 0 && g->n_routed_experts > 0 && g->moe_inter_size > 0 &&
           g->n_shared_experts >= 0 && g->hidden_size % 64 == 0 && g->moe_inter_size % 64 == 0 &&
           g->hidden_size < 65536 && g->moe_inter_size < 65536 &&
           (size_t)g->n_shared_experts * g->moe_inter_size < 65536;
}
#define I8_CFG_MSG "needs hidden and moe_inter multiples of 64, and hidden, moe_inter and " \
                   "n_shared x moe_inter below 65536"

int mm_moe_load_layer(mm_ctx *c, int layer, const mm_moe_layer_weights *w, unsigned flags) {
    if (!c || !w) return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: NULL argument");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_load_layer: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: layer %d out of range", layer);
    if (!(flags & (MM_LOAD_BF16 | MM_LOAD_INT8)))
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer: no weight format requested");
    if ((flags & MM_LOAD_INT8) && !i8_cfg_ok(&c->moe))
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_load_layer: int8 format " I8_CFG_MSG);
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

    /* router weight in its checkpoint layout [E, H] bf16 */
    MM_HIP(hipMalloc((void **)&L->wg, H * E * sizeof(uint16_t)));
    if ((st = upload(c, L->wg, w->moe_gate, H * E * 2, dev))) goto out;
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
    if (flags & MM_LOAD_INT8) {
        if ((st = load_int8(c, L, w, dev))) goto out;
    }
    L->formats = flags & (MM_LOAD_BF16 | MM_LOAD_INT8);
    L->loaded = 1;
out:;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (!st && e != hipSuccess) st = mm_hip_fail(e, "mm_moe_load_layer");
    return st;
}

/* ---- dense layers (l < first_k_dense) --------------------------------------- */

int mm_moe_load_dense_layer(mm_ctx *c, int layer, const uint16_t *gate, const uint16_t *up,
                            const uint16_t *down, int dense_inter, unsigned flags) {
    if (!c || !gate || !up || !down)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_dense_layer: NULL argument");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_load_dense_layer: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_dense_layer: layer %d out of range", layer);
    if (dense_inter <= 0 || dense_inter % 8)
        return mm_fail(MM_ERR_UNSUPPORTED,
                       "mm_moe_load_dense_layer: dense_inter must be a positive multiple of 8");
    mm_moe_layer *L = &c->layers[layer];
    if (L->loaded) return mm_fail(MM_ERR_STATE, "mm_moe_load_dense_layer: layer %d already loaded", layer);
    int st = mm_set_device(c);
    if (st) return st;
    const size_t H = c->moe.hidden_size, DI = dense_inter, ne = DI * H;
    const int dev = (flags & MM_LOAD_DEVICE_PTRS) != 0;
    if (hipMalloc((void **)&L->bf16_pool, 3 * ne * sizeof(uint16_t)) != hipSuccess)
        return mm_fail(MM_ERR_NOMEM, "mm_moe_load_dense_layer: %zu bytes", 3 * ne * 2);
    L->sg = L->bf16_pool;
    L->su = L->sg + ne;
    L->sd = L->su + ne;
    if (!(st = upload(c, L->sg, gate, ne * 2, dev)) && !(st = upload(c, L->su, up, ne * 2, dev)))
        st = upload(c, L->sd, down, ne * 2, dev);
    hipError_t e = hipStreamSynchronize(c->stream);
    if (!st && e != hipSuccess) st = mm_hip_fail(e, "mm_moe_load_dense_layer");
    if (st) {
        hipFree(L->bf16_pool);
        L->bf16_pool = L->sg = L->su = L->sd = NULL;
        return st;
    }
    L->dense = 1;
    L->dense_inter = dense_inter;
    L->formats = MM_LOAD_BF16;
    L->loaded = 1;
    return MM_OK;
}

/* ---- packed int8 layers (the offline expert format) ------------------------ */

int mm_moe_i8_layer_size(const mm_moe_config *cfg, size_t *pool_bytes, size_t *n_scales) {
    if (!cfg || !pool_bytes || !n_scales) return mm_fail(MM_ERR_INVALID, "mm_moe_i8_layer_size: NULL argument");
    if (!i8_cfg_ok(cfg))
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_i8_layer_size: int8 format needs positive sizes, "
                       I8_CFG_MSG);
    i8_sizes(cfg, pool_bytes, n_scales);
    return MM_OK;
}

int mm_moe_export_layer_i8(mm_ctx *c, int layer, void *pool, float *scales) {
    if (!c || !pool || !scales) return mm_fail(MM_ERR_INVALID, "mm_moe_export_layer_i8: NULL argument");
    if (!c->moe_ready || layer < 0 || layer >= c->n_layers || !c->layers[layer].loaded ||
        !(c->layers[layer].formats & MM_LOAD_INT8))
        return mm_fail(MM_ERR_STATE, "mm_moe_export_layer_i8: layer %d has no int8 weights", layer);
    int st = mm_set_device(c);
    if (st) return st;
    size_t pb, nsc;
    i8_sizes(&c->moe, &pb, &nsc);
    MM_HIP(hipStreamSynchronize(c->stream));
    MM_HIP(hipMemcpy(pool, c->layers[layer].i8_pool, pb, hipMemcpyDeviceToHost));
    MM_HIP(hipMemcpy(scales, c->layers[layer].i8_scales, nsc * sizeof(float), hipMemcpyDeviceToHost));
    return MM_OK;
}

int mm_moe_load_layer_i8_packed(mm_ctx *c, int layer, const uint16_t *moe_gate,
                                const float *moe_gate_bias, const void *pool, const float *scales,
                                unsigned flags) {
    if (!c || !moe_gate || !pool || !scales)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer_i8_packed: NULL argument");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_load_layer_i8_packed: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers)
        return mm_fail(MM_ERR_INVALID, "mm_moe_load_layer_i8_packed: layer %d out of range", layer);
    if (!i8_cfg_ok(&c->moe))
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_load_layer_i8_packed: int8 format " I8_CFG_MSG);
    mm_moe_layer *L = &c->layers[layer];
    if (L->loaded) return mm_fail(MM_ERR_STATE, "mm_moe_load_layer_i8_packed: layer %d already loaded", layer);
    int st = mm_set_device(c);
    if (st) return st;
    const mm_moe_config *g = &c->moe;
    const size_t H = g->hidden_size, E = g->n_routed_experts;
    const int dev = (flags & MM_LOAD_DEVICE_PTRS) != 0;
    size_t pb, nsc;
    i8_sizes(g, &pb, &nsc);
    MM_HIP(hipMalloc((void **)&L->wg, H * E * sizeof(uint16_t)));
    if ((st = upload(c, L->wg, moe_gate, H * E * 2, dev))) goto out;
    if (moe_gate_bias) {
        if (hipMalloc((void **)&L->bias, E * sizeof(float)) != hipSuccess) {
            st = mm_fail(MM_ERR_NOMEM, "mm_moe_load_layer_i8_packed: bias");
            goto out;
        }
        if ((st = upload(c, L->bias, moe_gate_bias, E * sizeof(float), dev))) goto out;
    }
    if ((st = i8_alloc(c, L))) goto out;
    if ((st = upload(c, L->i8_pool, pool, pb, dev))) goto out;
    if ((st = upload(c, L->i8_scales, scales, nsc * sizeof(float), dev))) goto out;
    L->formats = MM_LOAD_INT8;
    L->loaded = 1;
out:;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (!st && e != hipSuccess) st = mm_hip_fail(e, "mm_moe_load_layer_i8_packed");
    return st;
}

/* ---- workspace planning --------------------------------------------------- */

typedef struct {
    size_t off;
} mm_plan;

/* Reserve `bytes` (256-byte aligned) in the plan; returns the offset. */
static size_t plan_take(mm_plan *p, size_t bytes) {
    size_t o = p->off;
    p->off = (o + bytes + 255) & ~(size_t)255;
    return o;
}

/* The device workspace of one forward call: the context's growable one, or
 * a fixed region (the no-allocation entry point's scratch) that must hold
 * the whole plan. */
static int take_ws(mm_ctx *c, const mm_fixed_ws *fx, size_t need, char **ws) {
    if (fx) {
        if (need > fx->cap)
            return mm_fail(MM_ERR_UNSUPPORTED, "mm_moe_forward_noalloc_dev: this call needs %zu bytes "
                           "of scratch, the entry point holds %zu (use mm_moe_forward_dev)", need,
                           fx->cap);
        *ws = fx->base;
        return MM_OK;
    }
    return mm_workspace(c, need, (void **)ws);
}

/* The dense branch of ffn_compute (src/run.c:119-122, swiglu at :86-93):
 * out = down . (silu(gate . xn) * (up . xn)) over T rows, fp32 activations
 * and bf16 weights whatever the expert format (the reference's dense MLP
 * is bf16), out overwritten or accumulated.  Gate and up in one pass (the
 * fused GEMV up to MM_GEMV_NB rows, the skinny or tiled MFMA GEMM above),
 * SwiGLU in place over the gate rows, then the down projection. */
static int forward_dense(mm_ctx *c, const mm_moe_layer *L, int T, const float *xn, float *out,
                         int acc, const mm_fixed_ws *fx) {
    const int H = c->moe.hidden_size, DI = L->dense_inter;
    const int gv_gu = T <= MM_GEMV_NB && H <= MM_LM_HMAX;
    const int gv_d = T <= MM_GEMV_NB && DI <= MM_LM_HMAX;
    const unsigned dflags = acc ? MM_MATMUL_ACCUMULATE : 0;
    size_t wsb = gv_gu ? 0 : mm_gemm_bf16_ws2_bytes(T, H, DI, DI, 0);
    const size_t wsd = gv_d ? 0 : mm_gemm_bf16_ws_bytes(T, DI, H, dflags);
    if (wsd > wsb) wsb = wsd;
    mm_plan p = {0};
    const size_t o_g = plan_take(&p, (size_t)T * DI * 4), o_u = plan_take(&p, (size_t)T * DI * 4);
    const size_t o_ws = plan_take(&p, wsb);
    char *ws;
    int st = take_ws(c, fx, p.off, &ws);
    if (st) return st;
    float *g = (float *)(ws + o_g), *u = (float *)(ws + o_u);
    if (gv_gu) {
        mm_gemv_args a = {xn, NULL, 0.0f, L->sg, L->su, g, u, DI, DI, DI, DI, T, H, 0, 0};
        if ((st = mm_gemv_launch(c, &a))) return st;
    } else if ((st = mm_gemm_bf16_ws2(c, g, L->sg, DI, u, L->su, DI, xn, H, T, 0, ws + o_ws))) {
        return st;
    }
    const size_t n = (size_t)T * DI;
    mm_swiglu_args sa = {g, u, g, n};
    const size_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    if ((st = mm_launch(c, K_SWIGLU, (unsigned)blocks, 1, 1, 256, 0, &sa))) return st;
    if (gv_d) {
        mm_gemv_args a = {g, NULL, 0.0f, L->sd, NULL, out, NULL, H, 0, H, 0, T, DI, acc, 0};
        return mm_gemv_launch(c, &a);
    }
    return mm_gemm_bf16_ws(c, out, g, L->sd, H, DI, T, dflags, ws + o_ws);
}

/* ---- routing for more than MM_EMAX_FAST experts --------------------------------- */

/* Logits (computed from xn into lg_buf unless given) and the wide router
 * over all T tokens: idx, wts and probs (or NULL); with ra (int8) also the
 * quantisation of x and the tiled path's row lists.  */
static int route_wide(mm_ctx *c, const mm_moe_layer *L, int T, const float *xn,
                      const float *logits, float *lg_buf, int32_t *idx, float *wts, float *probs,
                      const mm_i8_route_args *ra) {
    const mm_moe_config *g = &c->moe;
    int st;
    if (!logits) {
        mm_router_args la;
        memset(&la, 0, sizeof(la));
        la.x = xn;
        la.wg = L->wg;
        la.logits_out = lg_buf;
        la.T = T;
        la.H = g->hidden_size;
        la.E = g->n_routed_experts;
        la.K = g->n_experts_per_tok;
        if ((st = mm_launch(c, K_ROUTER_WIDE, (unsigned)((T + 3) / 4),
                            (unsigned)((la.E + 63) / 64), 1, 256, 0, &la)))
            return st;
        logits = lg_buf;
    }
    mm_route_wide_args wa;
    memset(&wa, 0, sizeof(wa));
    wa.r.x = xn;
    wa.r.logits_in = logits;
    wa.r.bias = L->bias;
    wa.r.probs = probs;
    wa.r.topk_idx = idx;
    wa.r.topk_w = wts;
    wa.r.T = T;
    wa.r.H = g->hidden_size;
    wa.r.E = g->n_routed_experts;
    wa.r.K = g->n_experts_per_tok;
    wa.r.sigmoid = g->router_sigmoid;
    wa.r.norm_topk = g->norm_topk;
    wa.r.scale = g->routed_scaling;
    if (ra) {
        wa.cnt = ra->cnt;
        wa.rows = ra->rows;
        wa.x = ra->x;
        wa.qx = ra->qx;
        wa.sx = ra->sx;
    }
    return mm_launch(c, K_ROUTE_WIDE, (unsigned)((T + 3) / 4), 1, 1, 256, 0, &wa);
}

/* ---- bf16 forward ------------------------------------------------------------ */

/* Stage 2 (routed gate/up, shared parts): blocks of GU2_ROWS_PER_BLOCK rows,
 * one row group per wave, so the form that stages x once per block in LDS
 * (H * 4 bytes rounded up to 1 KB) applies whenever x fits 64 KB. */
static int launch_s2(mm_ctx *c, unsigned gx, unsigned gy, mm_gu_bf16_args *a) {
    const size_t xl = ((size_t)a->H * 4 + 1023) / 1024 * 1024;
    const int staged = a->rows_per_block == GU2_ROWS_PER_BLOCK && xl <= 65536;
    return mm_launch(c, staged ? K_MOE_BF16_S2L : K_MOE_BF16_S2, gx, gy, 1, 256, staged ? xl : 0, a);
}

/* bf16 weights, GEMV stages (kernels/moe_bf16.hip), BF16_NT_MAX tokens per pass. */
static int forward_bf16(mm_ctx *c, const mm_moe_layer *L, int T, const float *xn, float *out,
                        const float *logits, int32_t *idx, float *wts, float *probs, int acc,
                        const mm_fixed_ws *fx) {
    const mm_moe_config *g = &c->moe;
    const int H = g->hidden_size, E = g->n_routed_experts, K = g->n_experts_per_tok;
    const int I = g->moe_inter_size, S = g->n_shared_experts * I;
    const size_t hw = (size_t)K * I + S;
    const int wide = E > MM_EMAX_FAST;
    mm_plan p = {0};
    const size_t o_h = plan_take(&p, (size_t)BF16_NT_MAX * hw * sizeof(float));
    const size_t o_i = plan_take(&p, (size_t)T * K * sizeof(int32_t));
    const size_t o_w = plan_take(&p, (size_t)T * K * sizeof(float));
    /* router logits scratch: the wide routers', or the split router's of
     * the router + shared launch (computed logits, T <= RSH_TMAX) */
    const int rsh = !wide && E <= 64 && H % 8 == 0 && S % I == 0;
    const size_t o_lg = plan_take(&p, !logits && (wide || rsh) ? (size_t)T * E * sizeof(float) : 0);
    char *ws;
    int st = take_ws(c, fx, p.off, &ws);
    if (st) return st;
    float *hcat = (float *)(ws + o_h);
    if (!idx) idx = (int32_t *)(ws + o_i);
    if (!wts) wts = (float *)(ws + o_w);
    if (wide) {
        /* more than MM_EMAX_FAST experts: every token routed up front by
         * the wide routers, then the stages below without their router */
        if ((st = route_wide(c, L, T, xn, logits, (float *)(ws + o_lg), idx, wts, probs, NULL)))
            return st;
    }
    for (int t0 = 0; t0 < T; t0 += BF16_NT_MAX) {
        const int Tc = T - t0 < BF16_NT_MAX ? T - t0 : BF16_NT_MAX;
        mm_gu_bf16_args a;
        memset(&a, 0, sizeof(a));
        a.r.x = xn + (size_t)t0 * H;
        a.r.wg = L->wg;
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
        a.x = xn + (size_t)t0 * H;
        a.hcat = hcat;
        a.T = Tc;
        a.H = H;
        a.I = I;
        a.S = S;
        a.K = K;
        a.rows_per_block = GU2_ROWS_PER_BLOCK;
        a.n_blocks_per_token = (I + GU2_ROWS_PER_BLOCK - 1) / GU2_ROWS_PER_BLOCK;
        if (wide) {
            a.r.n_router_blocks = 0;   /* routed above: stage 1 runs the shared gate/up only */
            a.gate = L->sg;
            a.up = L->su;
            a.rows_per_block = GU_ROWS_PER_BLOCK;
            const unsigned nb1 = (unsigned)((S + GU_ROWS_PER_BLOCK - 1) / GU_ROWS_PER_BLOCK);
            if ((st = mm_launch(c, K_MOE_BF16_S1, nb1, 1, 1, 256, 0, &a))) return st;
            a.rows_per_block = GU2_ROWS_PER_BLOCK;
            a.gate = L->eg;
            a.up = L->eu;
            if ((st = launch_s2(c, a.n_blocks_per_token, Tc * K, &a)))
                return st;
        } else if (rsh && Tc <= MM_ROUTER_PC_TMAX) {
            /* small T: the router in product / chain form; up to RSH_TMAX
             * tokens the shared expert's gate/up runs in the same launch (it
             * does not wait on the routing), else with the routed gate/up */
            a.r.n_router_blocks = Tc;
            a.gate = L->eg;
            a.up = L->eu;
            a.sgate = L->sg;
            a.sup = L->su;
            a.nsh_parts = S / I;
            const unsigned nsh = (unsigned)(Tc * a.nsh_parts);
            if (Tc <= RSH_TMAX) {
                /* computed logits: MM_RSH_EB experts per router block */
                const unsigned ngr = logits ? 1u : (unsigned)((E + MM_RSH_EB - 1) / MM_RSH_EB);
                a.lg = (float *)(ws + o_lg);
                a.cnt = c->moe_cnt;
                /* the shared rows beside the router in blocks of RSH_ROWS_PER_BLOCK
                 * (measured: fewer, longer blocks there; more, shorter ones for
                 * the routed gate/up after it) */
                mm_gu_bf16_args ar = a;
                ar.rows_per_block = RSH_ROWS_PER_BLOCK;
                ar.n_blocks_per_token = (I + RSH_ROWS_PER_BLOCK - 1) / RSH_ROWS_PER_BLOCK;
                if ((st = mm_launch(c, K_MOE_BF16_RSH, (unsigned)Tc * ngr + ar.n_blocks_per_token * nsh,
                                    1, 1, 256, 0, &ar)))
                    return st;
                if ((st = launch_s2(c, a.n_blocks_per_token, (unsigned)(Tc * K), &a)))
                    return st;
            } else {
                if ((st = mm_launch(c, K_ROUTER_PC, (unsigned)Tc, 1, 1, 256, 0, &a.r))) return st;
                if ((st = launch_s2(c, a.n_blocks_per_token, (unsigned)(Tc * K) + nsh, &a)))
                    return st;
            }
        } else {
            a.r.n_router_blocks = (Tc + ROUTER_TOKENS_PER_BLOCK - 1) / ROUTER_TOKENS_PER_BLOCK;
            a.gate = L->sg;
            a.up = L->su;
            a.rows_per_block = GU_ROWS_PER_BLOCK;
            unsigned nb1 = a.r.n_router_blocks + (S + GU_ROWS_PER_BLOCK - 1) / GU_ROWS_PER_BLOCK;
            if ((st = mm_launch(c, K_MOE_BF16_S1, nb1, 1, 1, 256, 0, &a))) return st;
            a.rows_per_block = GU2_ROWS_PER_BLOCK;
            a.gate = L->eg;
            a.up = L->eu;
            if ((st = launch_s2(c, a.n_blocks_per_token, Tc * K, &a)))
                return st;
        }

        mm_down_bf16_args d = {hcat, L->ed, L->sd, idx + (size_t)t0 * K, out + (size_t)t0 * H,
                               Tc, H, I, S, K, E, acc, DOWN_ROWS_PER_BLOCK};
        /* the hidden row staged in LDS per block when it fits DN_LDS_MAX */
        const size_t hl_b = ((size_t)hw * 4 + 1023) / 1024 * 1024;
        const int staged = hl_b <= DN_LDS_MAX;
        if ((st = mm_launch(c, staged ? K_MOE_BF16_S3L : K_MOE_BF16_S3,
                            (H + DOWN_ROWS_PER_BLOCK - 1) / DOWN_ROWS_PER_BLOCK, Tc, 1, 256,
                            staged ? hl_b : 0, &d)))
            return st;
    }
    return MM_OK;
}

/* Router logits only (a->logits_out set): for small batches, where the
 * chain-per-lane form leaves most CUs idle, one token per block row and
 * MM_ROUTER_PC_EB experts per block (the token's products spread over
 * several CUs' LDS). */
static int launch_router_logits(mm_ctx *c, mm_router_args *a) {
    if (a->E > MM_EMAX_FAST)
        return mm_launch(c, K_ROUTER_WIDE, (unsigned)((a->T + 3) / 4), (unsigned)((a->E + 63) / 64), 1,
                         256, 0, a);
    if (a->E <= 64 && a->H % 8 == 0 && a->T <= MM_ROUTER_PC_TMAX)
        return mm_launch(c, K_ROUTER_PC_SPLIT, (unsigned)a->T,
                         (unsigned)((a->E + MM_ROUTER_PC_EB - 1) / MM_ROUTER_PC_EB), 1, 256, 0, a);
    const int tpb = MM_ROUTER_WAVES_LOGITS * MM_ROUTER_TPW;
    return mm_launch(c, K_ROUTER, (unsigned)((a->T + tpb - 1) / tpb), 1, 1, 64 * MM_ROUTER_WAVES_LOGITS, 0,
                     a);
}

/* ---- int8 forward ----------------------------------------------------------- */

/* Blocks of a decode GEMM that serve the shared expert's `groups` column
 * groups: MM_I8S_RT row-tile waves each, dealt in sets of MM_I8S_XCD. */
static size_t sh_blocks(size_t groups) {
    return (groups + MM_I8S_XCD - 1) / MM_I8S_XCD * MM_I8S_XCD * MM_I8S_RT;
}

static size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }
static size_t al16(size_t b) { return (b + 15) & ~(size_t)15; }
/* LDS of the K split's partials: MM_I8S_W waves x n accumulators x 64 lanes x 16 B */
#define KSPLIT_RED(n) ((size_t)MM_I8S_W * (n) * 64 * 16)

/* One grouped GEMM over the routed experts (ta) and, when ts is not NULL,
 * the shared expert: one persistent launch of the big-tile kernel. */
static int launch_tiled(mm_ctx *c, const mm_i8_tiled_args *ta, const mm_i8_tiled_args *ts) {
    mm_i8_bt_args ba;
    memset(&ba, 0, sizeof(ba));
    ba.seg[0] = *ta;
    if (ts) ba.seg[1] = *ts;
    ba.nseg = ts ? 2 : 1;
    const mm_kernel_id k = ta->gu ? (ta->dbg_acc ? K_I8_BT_GU_DBG : K_I8_BT_GU)
                                  : (ta->dbg_acc ? K_I8_BT_DN_DBG : K_I8_BT_DN);
    return mm_launch(c, k, MM_I8B_GRID, 1, 1, 256, 0, &ba);
}

/* A tiled call that fails after its routing launch leaves rows counted in
 * the per-expert counters that its combine would have cleared: clear them
 * here (best effort: the launch itself may be what fails) and return st. */
static int clear_counters(mm_ctx *c, int st) {
    mm_zero32_args za = {(uint32_t *)c->moe_cnt,
                         (uint64_t)c->moe.n_routed_experts * MM_CNT_STRIDE};
    (void)mm_launch(c, K_ZERO32, 1, 1, 1, 256, 0, &za);
    return st;
}

static int forward_int8(mm_ctx *c, const mm_moe_layer *L, int T, const float *xn, float *out,
                        const float *logits, int32_t *idx, float *wts, float *probs, int acc,
                        const mm_moe_i8_debug *dbg, const mm_fixed_ws *fx) {
    const mm_moe_config *g = &c->moe;
    const size_t H = g->hidden_size, E = g->n_routed_experts, K = g->n_experts_per_tok;
    const size_t I = g->moe_inter_size, S = (size_t)g->n_shared_experts * I;
    const size_t R = (size_t)T * K;   /* routed rows */
    mm_plan p = {0};
    const size_t o_rows = plan_take(&p, E * T * 4), o_qx = plan_take(&p, (size_t)T * H);
    /* GEMM outputs carry one spare row (+256 floats) that absorbs the
     * big-tile kernel's stores of padded rows and columns */
#define SPARE(rows, n) ((((size_t)(rows) + 1) * (n) + 256) * 4)
    const size_t o_sx = plan_take(&p, (size_t)T * 4), o_h = plan_take(&p, SPARE(R, I));
    const size_t o_hs = plan_take(&p, SPARE(T, S)), o_qh = plan_take(&p, R * I);
    const size_t o_sh = plan_take(&p, R * 4), o_qhs = plan_take(&p, (size_t)T * S);
    const size_t o_shs = plan_take(&p, (size_t)T * 4), o_y = plan_take(&p, SPARE(R, H));
    const size_t o_ys = plan_take(&p, SPARE(T, H)), o_i = plan_take(&p, R * 4);
#undef SPARE
    const size_t o_w = plan_take(&p, R * 4), o_lg = plan_take(&p, logits ? 0 : (size_t)T * E * 4);
    char *ws;
    int st = take_ws(c, fx, p.off, &ws);
    if (st) return st;
    if (!idx) idx = (int32_t *)(ws + o_i);
    if (!wts) wts = (float *)(ws + o_w);
    int32_t *rows = (int32_t *)(ws + o_rows);
    int8_t *qx = (int8_t *)(ws + o_qx), *qh = (int8_t *)(ws + o_qh), *qhs = (int8_t *)(ws + o_qhs);
    float *sx = (float *)(ws + o_sx), *h = (float *)(ws + o_h), *hs = (float *)(ws + o_hs);
    float *sh = (float *)(ws + o_sh), *shs = (float *)(ws + o_shs);
    float *y = (float *)(ws + o_y), *ys = (float *)(ws + o_ys);

    if (!logits) {
        /* router logits in the reference's order, then routing from them */
        mm_router_args la;
        memset(&la, 0, sizeof(la));
        la.x = xn;
        la.wg = L->wg;
        la.logits_out = (float *)(ws + o_lg);
        la.T = T;
        la.H = (int)H;
        la.E = (int)E;
        la.K = (int)K;
        if ((st = launch_router_logits(c, &la))) return st;
        logits = la.logits_out;
    }
    mm_i8_route_args ra;
    memset(&ra, 0, sizeof(ra));
    ra.r.x = xn;
    ra.r.wg = L->wg;
    ra.r.logits_in = logits;
    ra.r.bias = L->bias;
    ra.r.probs = probs;
    ra.r.topk_idx = idx;
    ra.r.topk_w = wts;
    ra.r.T = T;
    ra.r.H = (int)H;
    ra.r.E = (int)E;
    ra.r.K = (int)K;
    ra.r.sigmoid = g->router_sigmoid;
    ra.r.norm_topk = g->norm_topk;
    ra.r.scale = g->routed_scaling;
    /* decode-shaped GEMMs stage a 16-row A tile (16 * K bytes) and a row list
     * (T ints) in LDS; shapes beyond 64 KB of it take the tiled GEMMs */
    const size_t lds_dec = 16 * (H > (I > S ? I : S) ? H : (I > S ? I : S)) + 4 * (size_t)T;
    const int tiled = T >= c->i8_tiled_min_t || lds_dec > 65536;
    /* per-expert row lists only for the tiled path; the decode-shaped GEMMs
     * build theirs from the routing */
    ra.cnt = tiled ? c->moe_cnt : NULL;
    ra.rows = tiled ? rows : NULL;
    ra.x = xn;
    ra.qx = qx;
    ra.sx = sx;
    /* the route kernel appends to the per-expert counters (zero on entry:
     * cleared at init and by every tiled call's combine); a failure after it
     * clears them itself (FAIL_ROUTED) */
    /* routing waves and as many x-quantising waves per block */
    if (E > MM_EMAX_FAST)   /* the wide router (logits are given or computed above) */
        st = route_wide(c, L, T, xn, logits, NULL, idx, wts, probs, &ra);
    else
        st = mm_launch(c, K_I8_ROUTE, (T + MM_I8_RT_TOKENS - 1) / MM_I8_RT_TOKENS, 1, 1,
                       2 * 64 * MM_I8_RT_WAVES, 0, &ra);
    if (st) return tiled ? clear_counters(c, st) : st;
#define FAIL_ROUTED(call)                                   \
    do {                                                    \
        if ((st = (call))) return tiled ? clear_counters(c, st) : st; \
    } while (0)

    mm_i8_gemm_args ga;
    memset(&ga, 0, sizeof(ga));
    ga.w = L->i8;
    ga.cnt = c->moe_cnt;
    ga.rows = rows;
    ga.topk = idx;
    ga.a = qx;
    ga.sa = sx;
    ga.h = h;
    ga.hs = hs;
    ga.dbg_acc = dbg ? dbg->acc_gu : NULL;
    ga.T = T;
    ga.H = (int)H;
    ga.I = (int)I;
    ga.S = (int)S;
    ga.E = (int)E;
    ga.K = (int)K;
    /* few tokens: few experts hold rows, so the gate/up GEMM splits K
     * (the hidden size) over a block's waves to have enough blocks */
    ga.ksplit = !tiled && T <= MM_I8_KSPLIT_TMAX && H / 64 >= MM_I8S_W;
    if (tiled) {
        /* routed experts, then the shared expert as one dense GEMM */
        mm_i8_tiled_args ta = {L->i8.gu, 2 * I * H, L->i8.s_g, L->i8.s_u, (int)I, c->moe_cnt,
                               rows, qx, sx, 0, h, dbg ? dbg->acc_gu : NULL, T, (int)K,
                               (int)E, (int)I, (int)H, 1, (int)R};
        mm_i8_tiled_args ts = {L->i8.sgu, 0, L->i8.ss_g, L->i8.ss_u, 0, NULL, NULL, qx, sx, 0,
                               hs, NULL, T, (int)K, 1, (int)S, (int)H, 1, T};
        FAIL_ROUTED(launch_tiled(c, &ta, S ? &ts : NULL));
    } else {
        /* shared-expert blocks (row-tile waves), then every routed unit */
        const size_t per_blk = ga.ksplit ? 1 : (size_t)MM_I8S_W * MM_I8S_SEG;
        /* routed block rows: one per expert, or per route slot with the K
         * split (few slots; a slot repeating an earlier slot's expert exits) */
        const size_t rrows = ga.ksplit ? R : E;
        const unsigned nb = (unsigned)((S ? sh_blocks(ceil_div(S / 16, per_blk)) : 0) +
                                       rrows * ceil_div(I / 16, per_blk));
        /* dynamic LDS: the 16-row A tile (16 * K bytes), the row list, the
         * K split's partials */
        FAIL_ROUTED(mm_launch(c, ga.ksplit ? K_I8_GU_KS : K_I8_GU, nb, 1, 1, 64 * MM_I8S_W,
                              16 * H + al16(4 * (size_t)T) + (ga.ksplit ? KSPLIT_RED(2) : 0), &ga));
    }

    mm_i8_quant_rows_args qa = {h, qh, sh, (int)R, (int)I, S ? hs : NULL, qhs, shs,
                                S ? T : 0, (int)S};
    FAIL_ROUTED(mm_launch(c, K_I8_QUANT_H, (unsigned)((R + (S ? T : 0) + 3) / 4), 1, 1, 256, 0, &qa));

    if (tiled) {
        mm_i8_tiled_args td = {L->i8.d, H * I, L->i8.s_d, NULL, (int)H, c->moe_cnt, rows, qh, sh,
                               1, y, dbg ? dbg->acc_d : NULL, T, (int)K, (int)E, (int)H, (int)I,
                               0, (int)R};
        mm_i8_tiled_args tsd = {L->i8.sdn, 0, L->i8.ss_d, NULL, 0, NULL, NULL, qhs, shs, 1, ys,
                                NULL, T, (int)K, 1, (int)H, (int)S, 0, T};
        FAIL_ROUTED(launch_tiled(c, &td, S ? &tsd : NULL));
    } else {
        ga.a = qh;
        ga.sa = sh;
        ga.a_sh = qhs;
        ga.sa_sh = shs;
        ga.y = y;
        ga.ys = ys;
        ga.dbg_acc = dbg ? dbg->acc_d : NULL;
        /* the down GEMM keeps its column groups: its K (the intermediate
         * size, 22 steps at I = 1408) split six ways left each wave too
         * short a stream (14.3 against 13.2 us per layer at one token) */
        ga.ksplit = 0;
        const size_t gpe = ceil_div(H / 16, (size_t)MM_I8S_W * MM_I8S_SEG);
        const unsigned nb = (unsigned)((S ? sh_blocks(gpe) : 0) + E * gpe);
        FAIL_ROUTED(mm_launch(c, K_I8_DOWN, nb, 1, 1, 64 * MM_I8S_W,
                              16 * (S > I ? S : I) + 4 * (size_t)T, &ga));
    }

    mm_i8_combine_args ca = {y, ys, wts, out, tiled ? c->moe_cnt : NULL, T, (int)H, (int)K,
                             (int)E, acc, S > 0, c->norm_w, c->norm_xn, c->norm_eps,
                             c->norm_w ? c->norm_xn_hl : NULL};
    if (c->norm_w)   /* one block per token, the row's norm in the same pass */
        FAIL_ROUTED(mm_launch(c, K_I8_COMBINE_NORM, (unsigned)T, 1, 1, MM_I8_CN_THREADS, 0, &ca));
    else             /* two blocks per token: one round of loads per thread at H = 2048 */
        FAIL_ROUTED(mm_launch(c, K_I8_COMBINE, (unsigned)T, 2, 1, 256, 0, &ca));
#undef FAIL_ROUTED

    if (dbg) {
        struct {
            void *dst;
            const void *src;
            size_t n;
        } cp[] = {{dbg->qx, qx, (size_t)T * H},       {dbg->sx, sx, (size_t)T * 4},
                  {dbg->h, h, R * I * 4},             {dbg->qh, qh, R * I},
                  {dbg->sh, sh, R * 4},               {dbg->y, y, R * H * 4},
                  {dbg->hs, hs, (size_t)T * S * 4},   {dbg->qhs, qhs, (size_t)T * S},
                  {dbg->shs, shs, (size_t)T * 4},     {dbg->ys, ys, (size_t)T * H * 4}};
        for (size_t i = 0; i < sizeof(cp) / sizeof(cp[0]); i++)
            if (cp[i].dst && cp[i].n)
                MM_HIP(hipMemcpyAsync(cp[i].dst, cp[i].src, cp[i].n, hipMemcpyDeviceToDevice,
                                      c->stream));
    }
    return MM_OK;
}

/* Rows of one forward pass.  Every token's routing and expert rows are its
 * own, so a longer call runs as consecutive chunks with identical results;
 * the chunk keeps each int8 activation matrix of the tiled GEMMs (T x H,
 * T K x I and T x S bytes) below the 32-bit range of their row offsets
 * (MM_I8_TILED_A_MAX) and the workspace to the chunk's rows. */
#define MM_MOE_T_CHUNK 65536
static int moe_t_chunk(const mm_ctx *c) {
    const mm_moe_config *g = &c->moe;
    size_t w = g->hidden_size;
    const size_t ki = (size_t)g->n_experts_per_tok * g->moe_inter_size;
    const size_t s = (size_t)g->n_shared_experts * g->moe_inter_size;
    if (ki > w) w = ki;
    if (s > w) w = s;
    size_t n = c->moe_t_chunk > 0 ? (size_t)c->moe_t_chunk : MM_MOE_T_CHUNK;
    if (w && n > (MM_I8_TILED_A_MAX - 1) / w) n = (MM_I8_TILED_A_MAX - 1) / w;
    return n > 0 ? (int)n : 1;
}

static int forward(mm_ctx *c, int layer, int T, const float *xn, float *out, const float *logits,
                   int32_t *topk_idx, float *topk_w, float *probs, unsigned flags,
                   const mm_moe_i8_debug *dbg, const mm_fixed_ws *fx) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: NULL context");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_forward: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers || !c->layers[layer].loaded)
        return mm_fail(MM_ERR_STATE, "mm_moe_forward: layer %d not loaded", layer);
    if (T < 0 || !out || (!xn && T > 0))
        return mm_fail(MM_ERR_INVALID, "mm_moe_forward: bad arguments");
    if (T == 0) return MM_OK;
    if ((uintptr_t)xn % 16 || (uintptr_t)out % 16)
        return mm_fail(MM_ERR_INVALID, "mm_moe_forward: xn/out must be 16-byte aligned");
    const mm_moe_layer *L = &c->layers[layer];
    const int tc = moe_t_chunk(c);
    if (T > tc) {
        /* the debug block and the fused next-layer norm (its lo plane at row
         * T + t) are laid out for the whole call */
        if (dbg || c->norm_w)
            return mm_fail(MM_ERR_INVALID, "mm_moe_forward: %d rows with debug outputs or the "
                           "fused norm (at most %d)", T, tc);
        const size_t H = c->moe.hidden_size, E = c->moe.n_routed_experts;
        const size_t K = c->moe.n_experts_per_tok;
        for (int t0 = 0; t0 < T; t0 += tc) {
            const int n = T - t0 < tc ? T - t0 : tc;
            const int st = forward(c, layer, n, xn + (size_t)t0 * H, out + (size_t)t0 * H,
                                   logits ? logits + (size_t)t0 * E : NULL,
                                   topk_idx ? topk_idx + (size_t)t0 * K : NULL,
                                   topk_w ? topk_w + (size_t)t0 * K : NULL,
                                   probs ? probs + (size_t)t0 * E : NULL, flags, NULL, fx);
            if (st) return st;
        }
        return MM_OK;
    }
    int st = mm_set_device(c);
    if (st) return st;
    const int acc = (flags & MM_FWD_ACCUMULATE) != 0;
    if (L->dense) {
        /* the reference returns before routing: topk_idx, topk_w, probs untouched */
        if (dbg) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: layer %d is dense (no int8 "
                                "intermediates)", layer);
        return forward_dense(c, L, T, xn, out, acc, fx);
    }
    if (flags & MM_FWD_INT8) {
        if (!(L->formats & MM_LOAD_INT8))
            return mm_fail(MM_ERR_STATE, "mm_moe_forward: layer %d has no int8 weights", layer);
        return forward_int8(c, L, T, xn, out, logits, topk_idx, topk_w, probs, acc, dbg, fx);
    }
    if (dbg) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: debug outputs need MM_FWD_INT8");
    if (!(L->formats & MM_LOAD_BF16))
        return mm_fail(MM_ERR_STATE, "mm_moe_forward: layer %d has no bf16 weights", layer);
    if (xn == out) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: bf16 path needs out != xn");
    return forward_bf16(c, L, T, xn, out, logits, topk_idx, topk_w, probs, acc, fx);
}

int mm_moe_forward_norm(mm_ctx *c, int layer, int T, const float *xn, float *out, unsigned flags,
                        const uint16_t *norm_w, float eps, float *xn_next, uint16_t *xn_next_hl,
                        int *fused) {
    *fused = 0;
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_moe_forward: NULL context");
    const int can = (flags & MM_FWD_INT8) && c->moe.hidden_size <= MM_I8_CN_MAXH &&
                    c->moe.hidden_size % 4 == 0 && norm_w && xn_next && T <= moe_t_chunk(c);
    if (can) {
        c->norm_w = norm_w;
        c->norm_xn = xn_next;
        c->norm_xn_hl = xn_next_hl;
        c->norm_eps = eps;
    }
    const int st = forward(c, layer, T, xn, out, NULL, NULL, NULL, NULL, flags, NULL, NULL);
    c->norm_w = NULL;
    c->norm_xn = NULL;
    c->norm_xn_hl = NULL;
    if (!st) *fused = can;
    return st;
}

int mm_moe_router_logits_dev(mm_ctx *c, int layer, int T, const float *xn,
                             const float *logit_bias, float *logits) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_moe_router_logits_dev: NULL context");
    if (!c->moe_ready) return mm_fail(MM_ERR_STATE, "mm_moe_router_logits_dev: call mm_moe_init first");
    if (layer < 0 || layer >= c->n_layers || !c->layers[layer].loaded || c->layers[layer].dense)
        return mm_fail(MM_ERR_STATE, "mm_moe_router_logits_dev: layer %d is not a loaded MoE layer",
                       layer);
    if (T < 0 || (T > 0 && (!xn || !logits)))
        return mm_fail(MM_ERR_INVALID, "mm_moe_router_logits_dev: bad arguments");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    const mm_moe_layer *L = &c->layers[layer];
    mm_router_args a;
    memset(&a, 0, sizeof(a));
    a.x = xn;
    a.wg = L->wg;
    a.logit_bias = logit_bias;
    a.logits_out = logits;
    a.T = T;
    a.H = c->moe.hidden_size;
    a.E = c->moe.n_routed_experts;
    a.K = c->moe.n_experts_per_tok;
    return launch_router_logits(c, &a);
}

int mm_moe_forward_dev(mm_ctx *c, int layer, int T, const float *xn, float *out,
                       const float *logits, int32_t *topk_idx, float *topk_w, float *probs,
                       unsigned flags) {
    return forward(c, layer, T, xn, out, logits, topk_idx, topk_w, probs, flags, NULL, NULL);
}

int mm_moe_forward_fixed(mm_ctx *c, int layer, int T, const float *xn, float *out,
                         const float *logits, int32_t *topk_idx, float *topk_w, float *probs,
                         unsigned flags, const mm_fixed_ws *fx) {
    return forward(c, layer, T, xn, out, logits, topk_idx, topk_w, probs, flags, NULL, fx);
}

int mm_moe_forward_i8_debug_dev(mm_ctx *c, int layer, int T, const float *xn, float *out,
                                const float *logits, int32_t *topk_idx, float *topk_w,
                                float *probs, unsigned flags, const mm_moe_i8_debug *dbg) {
    if (!dbg) return mm_fail(MM_ERR_INVALID, "mm_moe_forward_i8_debug_dev: NULL debug block");
    return forward(c, layer, T, xn, out, logits, topk_idx, topk_w, probs, flags | MM_FWD_INT8,
                   dbg, NULL);
}
