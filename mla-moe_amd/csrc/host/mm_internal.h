/* mm_internal.h -- private state of the C11 host library. */
#ifndef MLAMOE_INTERNAL_H
#define MLAMOE_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "../kernel_params.h"
#include "mlamoe.h"

/* Kernels, one entry per extern "C" __global__ in csrc/kernels. */
typedef enum {
    K_ROUTER,
    K_ROUTER_PC,
    K_ROUTER_PC_SPLIT,
    K_MOE_BF16_RSH,
    K_MOE_BF16_S1,
    K_MOE_BF16_S2,
    K_MOE_BF16_S2L,
    K_MOE_BF16_S3,
    K_MOE_BF16_S3L,
    K_FILL,
    K_QUANT_W,
    K_I8_ROUTE,
    K_I8_GU,
    K_I8_GU_KS,
    K_I8_QUANT_H,
    K_I8_DOWN,
    K_I8_COMBINE,
    K_I8_COMBINE_NORM,
    K_PACK_I8,
    K_I8_BT_GU,
    K_I8_BT_DN,
    K_I8_BT_GU_DBG,
    K_I8_BT_DN_DBG,
    K_MLA_QPREP,
    K_MLA_ROPE_QPREP,
    K_MLA_ATTN,
    K_MLA_ATTN_ROWS,
    K_MLA_COMBINE,
    K_MLA_UV,
    K_MLA_QPREP_W,
    K_MLA_UV_W,
    K_MLA_WPREP,
    K_GEMM_BF16,
    K_CVT_BF16,
    K_RMSNORM,
    K_RMSNORM_HL,
    K_LM_GEMM,
    K_LM_GEMV1,
    K_LM_GEMV2,
    K_LM_GEMV4,
    K_ARGMAX_PART,
    K_ARGMAX_FINAL,
    K_GEMV1,
    K_GEMV2,
    K_GEMV4,
    K_MLA_ROPE,
    K_EMBED,
    K_SWIGLU,
    K_GEMM_SKINNY,
    K_GEMM_SKINNY_WIDE,
    K_GEMM_HL,
    K_SKINNY_REDUCE,
    K_REDUCE_RMSNORM,
    K_ZERO32,
    K_GATHER_ROWS,
    K_F32_BF16,
    K_ROUTER_WIDE,
    K_ROUTE_WIDE,
    K_COUNT
} mm_kernel_id;

typedef struct {
    int id;
    hipEvent_t ev[2];
} mm_prof_rec;

typedef struct {
    int loaded;
    int dense;                  /* a dense SwiGLU layer (l < first_k_dense, src/run.c:119-122) */
    int dense_inter;            /* its intermediate size */
    unsigned formats;
    uint16_t *wg;               /* [E, H] bf16 router weight */
    float *bias;                /* [E] or NULL */
    uint16_t *bf16_pool;        /* one allocation holding the six bf16 families */
    uint16_t *eg, *eu, *ed, *sg, *su, *sd;   /* dense layer: sg, su, sd = gate, up, down */
    int8_t *i8_pool;            /* packed int8 fragments (kernel_params.h) */
    float *i8_scales;
    mm_i8_weights i8;
} mm_moe_layer;

struct mm_ctx {
    int device;
    hipStream_t stream;         /* where work is queued: own_stream or the caller's */
    hipStream_t own_stream;     /* created with the context */
    hipEvent_t ev_switch;       /* orders work across a stream switch */
    hipModule_t *modules;
    int n_modules;
    hipFunction_t fn[K_COUNT];
    hipEvent_t t0, t1;

    int prof_on;
    mm_prof_rec *prof;
    size_t prof_n, prof_cap;
    hipEvent_t *ev_pool;
    size_t ev_pool_n, ev_pool_cap;

    /* MoE */
    int moe_ready;
    mm_moe_config moe;
    int n_layers;
    mm_moe_layer *layers;
    int32_t *moe_cnt;           /* [E * MM_CNT_STRIDE]: per-expert row counters of the
                                   tiled int8 path (one per 128-byte line), or per-token
                                   counters (the first RSH_TMAX entries) of the bf16
                                   router + shared launch; zero between calls */
    /* set by mm_moe_forward_norm for the duration of one forward: the int8
     * combine also writes rmsnorm(out, norm_w) into norm_xn */
    const uint16_t *norm_w;
    float *norm_xn;
    uint16_t *norm_xn_hl;
    float norm_eps;

    /* MLA */
    int mla_ready;
    mm_mla_config mla;
    int mla_layers;
    uint16_t **mla_kvb;         /* [layers] device kv_b_proj weights */
    int front_ready;
    mm_mla_front_config front;  /* rope_inv_freq points at front_inv (device) */
    float *front_inv;           /* [qk_rope_head_dim / 2] device RoPE table */

    int i8_tiled_min_t;         /* token count from which the tiled int8 GEMM is used */
    size_t mla_part_max;        /* attention chunk partials per launch (bytes) */
    int mla_rows4;              /* row groups sharing a sequence read its keys once
                                   (MLAMOE_MLA_ROWS4=0: per row, for comparisons) */
    int moe_t_chunk;            /* cap on the rows of one MoE forward pass (0: MM_MOE_T_CHUNK) */

    /* growable device workspace */
    void *ws;
    size_t ws_bytes;
    /* growable device staging of the synchronous host-pointer entry points */
    void *io;
    size_t io_bytes;
    /* device copies of host weights passed to mm_matmul_bf16 (MM_MATMUL_W_HOST) */
    struct mm_wcache_entry *wcache;
    size_t wcache_n, wcache_cap;

    /* this device's copy of the no-allocation entry point's static scratch
     * array (its device address, from hipGetSymbolAddress at set-up) */
    void *scratch;
    size_t scratch_bytes;
};

/* A fixed device workspace region (no growth). */
typedef struct {
    char *base;
    size_t cap;
} mm_fixed_ws;

/* mm_moe_forward_dev on the fixed workspace fx: fails with
 * MM_ERR_UNSUPPORTED before any launch when the call needs more than
 * fx->cap bytes; allocates nothing. */
/* mm_moe_forward_dev whose output rows are also normalised into xn_next
 * (rmsnorm with norm_w, eps) in the combine pass when the int8 path runs
 * (returns 1 in *fused then; else the caller normalises); xn_next_hl (or
 * NULL) also receives them as bf16 hi/lo planes [2, T, H]. */
int mm_moe_forward_norm(mm_ctx *c, int layer, int T, const float *xn, float *out, unsigned flags,
                        const uint16_t *norm_w, float eps, float *xn_next, uint16_t *xn_next_hl,
                        int *fused);
int mm_moe_forward_fixed(mm_ctx *ctx, int layer, int T, const float *xn, float *out,
                         const float *logits, int32_t *topk_idx, float *topk_w, float *probs,
                         unsigned flags, const mm_fixed_ws *fx);

/* Set-up of the no-allocation scratch for the context's device (with that
 * device current): its device address and size. */
int mm_noalloc_setup(mm_ctx *ctx);

/* error reporting (thread-local message) */
int mm_fail(int status, const char *fmt, ...);
int mm_hip_fail(hipError_t e, const char *what);
#define MM_HIP(call)                                              \
    do {                                                          \
        hipError_t mm_e_ = (call);                                \
        if (mm_e_ != hipSuccess) return mm_hip_fail(mm_e_, #call); \
    } while (0)

int mm_set_device(mm_ctx *ctx);
/* Launch kernel `id` with its argument block `args` (the struct is copied). */
int mm_launch(mm_ctx *ctx, mm_kernel_id id, unsigned gx, unsigned gy, unsigned gz,
              unsigned block, size_t shmem, void *args);
/* Device workspace of at least `bytes`, reallocated (after a stream sync)
 * when too small. */
int mm_workspace(mm_ctx *ctx, size_t bytes, void **out);
/* Device staging of at least `bytes` for the host-pointer entry points (a
 * buffer of its own: the forward calls they make use the workspace). */
int mm_io_buffer(mm_ctx *ctx, size_t bytes, void **out);
void mm_host_release(mm_ctx *ctx);

/* Dense bf16 GEMM (mm_matmul_bf16_dev) on a caller-provided workspace of at
 * least mm_gemm_bf16_ws_bytes(T, n_in, d_out, flags) bytes. */
size_t mm_gemm_bf16_ws_bytes(int T, int n_in, int d_out, unsigned flags);
/* Two matrices over the same x (y0 = x . W0^T, y1 = x . W1^T; w1 may be
 * NULL): one skinny-M launch when that path applies. */
size_t mm_gemm_bf16_ws2_bytes(int T, int n_in, int d0, int d1, unsigned flags);
/* The skinny-M GEMM (T <= MM_SKINNY_T, n_in % 64 == 0) over x given as bf16
 * hi/lo planes [2, T, n_in]; y0 (and y1 over w1 when d1 > 0) as
 * mm_gemm_bf16_ws2 computes them from the fp32 rows the planes split. */
size_t mm_gemm_bf16_hl_ws_bytes(int T, int n_in, int d0, int d1);
int mm_gemm_bf16_hl(mm_ctx *ctx, float *y0, const uint16_t *w0, int d0, float *y1,
                    const uint16_t *w1, int d1, const uint16_t *xhl, int n_in, int T, int acc,
                    char *ws);
/* x += a . w^T (bf16 w [d_out, n_in]) then xn = rmsnorm(x, norm_w) over rows
 * of d_out; ws of mm_gemm_bf16_add_rmsnorm_ws_bytes bytes. */
size_t mm_gemm_bf16_add_rmsnorm_ws_bytes(int T, int n_in, int d_out);
int mm_gemm_bf16_add_rmsnorm(mm_ctx *c, float *x, const float *a, const uint16_t *w, int d_out,
                             int n_in, int T, const uint16_t *norm_w, float eps, float *xn,
                             char *ws);
/* The same with a given as bf16 hi/lo planes [2, T, n_in]: T <= MM_SKINNY_T,
 * n_in % 64 == 0, d_out <= MM_RRN_THREADS * MM_RRN_PT (ws as above). */
int mm_gemm_bf16_add_rmsnorm_hl(mm_ctx *c, float *x, const uint16_t *ahl, const uint16_t *w,
                                int d_out, int n_in, int T, const uint16_t *norm_w, float eps,
                                float *xn, char *ws);
int mm_gemm_bf16_ws2(mm_ctx *ctx, float *y0, const uint16_t *w0, int d0, float *y1,
                     const uint16_t *w1, int d1, const float *x, int n_in, int T, unsigned flags,
                     char *ws);
int mm_gemm_bf16_ws(mm_ctx *ctx, float *y, const float *x, const uint16_t *w, int d_out, int n_in,
                    int T, unsigned flags, char *ws);

/* GEMV over up to MM_GEMV_NB tokens (hidden <= GV_HMAX): the launch shape
 * for `rows` output rows in total. */
unsigned mm_gemv_blocks(int rows);
int mm_gemv_launch(mm_ctx *ctx, const mm_gemv_args *a);

/* mm_mla_front_dev / mm_mla_absorbed_decode_dev with row b on cache
 * sequence slots[b] (slots NULL: sequence b): rows of one sequence may share
 * a call (prefill chunks), causality coming from each row's position /
 * kv_lens[b].  xn_pre: rmsnorm(x, input_norm) already computed by the
 * caller (used above MM_GEMV_NB rows), or NULL; xn_pre_hl (or NULL) the
 * same rows as bf16 hi/lo planes, which the projections then read. */
/* defer (or NULL; B <= MM_SKINNY_T): the RoPE / cache-append launch is not
 * made; its arguments go to *defer for mm_mla_decode_rows to run with the
 * absorbed queries in one launch, and kv_a's output goes to comp_buf
 * ([B, KVL + QKR] fp32, the caller's) instead of the workspace, which later
 * calls reuse before that launch runs. */
int mm_mla_front_rows(mm_ctx *ctx, int B, const float *x, const mm_mla_front_weights *w,
                      const int32_t *pos, const int32_t *slots, float *q, uint16_t *cache,
                      int seq_stride, float *kv_rows, const float *xn_pre,
                      const uint16_t *xn_pre_hl, float *comp_buf, mm_mla_rope_args *defer);
/* rope (or NULL): the deferred RoPE of mm_mla_front_rows, run with qprep;
 * ctx_hl (or NULL): ctx_out also as bf16 hi/lo planes [2, B, NH * VHD].
 * rows4: slots given and rows 4 j .. 4 j + 3 of every group share a cache
 * sequence (a prefill's consecutive positions): the attention reads each
 * group's keys once (mm_mla_attn_rows). */
int mm_mla_decode_rows(mm_ctx *ctx, int layer, int B, const float *q, const uint16_t *cache,
                       int seq_stride, const int32_t *slots, const int32_t *kv_lens, int kv_len,
                       float *ctx_out, float *qabs, float *probs, float *clat,
                       const mm_mla_rope_args *rope, uint16_t *ctx_hl, int rows4);

void mm_moe_release(mm_ctx *ctx);
void mm_mla_release(mm_ctx *ctx);

#endif
