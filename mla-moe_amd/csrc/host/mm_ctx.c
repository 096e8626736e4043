/* mm_ctx.c -- context, code-object loading, launches, memory and timing.
 *
 * The gfx950 kernels are compiled to code objects (hipcc --genco) that are
 * embedded in this library (embed.S) and loaded with hipModuleLoadData when
 * a context is created; kernels are launched with hipModuleLaunchKernel.
 * The host side therefore stays plain C11 over the HIP runtime API.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mm_internal.h"

/* ---- embedded code objects (embed.S) ------------------------------------ */
extern const unsigned char mm_co_moe_bf16[];
extern const unsigned char mm_co_util[];
extern const unsigned char mm_co_moe_i8[];
extern const unsigned char mm_co_mla[];
extern const unsigned char mm_co_gemm_bf16[];
extern const unsigned char mm_co_gemm_i8[];
extern const unsigned char mm_co_lm_head[];
extern const unsigned char mm_co_gemv[];

enum { MOD_MOE_BF16, MOD_UTIL, MOD_MOE_I8, MOD_MLA, MOD_GEMM_BF16, MOD_GEMM_I8, MOD_LM_HEAD,
       MOD_GEMV, MOD_COUNT };
static const unsigned char *const mod_blob[MOD_COUNT] = {mm_co_moe_bf16, mm_co_util,
                                                          mm_co_moe_i8, mm_co_mla,
                                                          mm_co_gemm_bf16, mm_co_gemm_i8,
                                                          mm_co_lm_head, mm_co_gemv};

static const struct {
    const char *name;
    int module;
} kinfo[K_COUNT] = {
    [K_ROUTER] = {"mm_router", MOD_MOE_BF16},
    [K_ROUTER_PC] = {"mm_router_pc", MOD_MOE_BF16},
    [K_ROUTER_PC_SPLIT] = {"mm_router_pc_split", MOD_MOE_BF16},
    [K_MOE_BF16_RSH] = {"mm_moe_bf16_router_sh", MOD_MOE_BF16},
    [K_MOE_BF16_S1] = {"mm_moe_bf16_stage1", MOD_MOE_BF16},
    [K_MOE_BF16_S2] = {"mm_moe_bf16_stage2", MOD_MOE_BF16},
    [K_MOE_BF16_S2L] = {"mm_moe_bf16_stage2_lds", MOD_MOE_BF16},
    [K_MOE_BF16_S3] = {"mm_moe_bf16_stage3", MOD_MOE_BF16},
    [K_MOE_BF16_S3L] = {"mm_moe_bf16_stage3_lds", MOD_MOE_BF16},
    [K_FILL] = {"mm_fill", MOD_UTIL},
    [K_QUANT_W] = {"mm_quant_weight", MOD_UTIL},
    [K_I8_ROUTE] = {"mm_i8_route", MOD_MOE_I8},
    [K_I8_GU] = {"mm_i8_gu", MOD_MOE_I8},
    [K_I8_GU_KS] = {"mm_i8_gu_ks", MOD_MOE_I8},
    [K_I8_QUANT_H] = {"mm_i8_quant_h", MOD_MOE_I8},
    [K_I8_DOWN] = {"mm_i8_down", MOD_MOE_I8},
    [K_I8_COMBINE] = {"mm_i8_combine", MOD_MOE_I8},
    [K_I8_COMBINE_NORM] = {"mm_i8_combine_norm", MOD_MOE_I8},
    [K_PACK_I8] = {"mm_pack_i8", MOD_MOE_I8},
    [K_I8_BT_GU] = {"mm_i8_gemm_gu", MOD_GEMM_I8},
    [K_I8_BT_DN] = {"mm_i8_gemm_dn", MOD_GEMM_I8},
    [K_I8_BT_GU_DBG] = {"mm_i8_gemm_gu_dbg", MOD_GEMM_I8},
    [K_I8_BT_DN_DBG] = {"mm_i8_gemm_dn_dbg", MOD_GEMM_I8},
    [K_MLA_QPREP] = {"mm_mla_qprep", MOD_MLA},
    [K_MLA_ROPE_QPREP] = {"mm_mla_rope_qprep", MOD_MLA},
    [K_MLA_ATTN] = {"mm_mla_attn", MOD_MLA},
    [K_MLA_ATTN_ROWS] = {"mm_mla_attn_rows", MOD_MLA},
    [K_MLA_COMBINE] = {"mm_mla_combine", MOD_MLA},
    [K_MLA_UV] = {"mm_mla_uv", MOD_MLA},
    [K_MLA_QPREP_W] = {"mm_mla_qprep_w", MOD_MLA},
    [K_MLA_UV_W] = {"mm_mla_uv_w", MOD_MLA},
    [K_MLA_WPREP] = {"mm_mla_wprep", MOD_MLA},
    [K_GEMM_BF16] = {"mm_gemm_bf16", MOD_GEMM_BF16},
    [K_CVT_BF16] = {"mm_cvt_bf16", MOD_GEMM_BF16},
    [K_RMSNORM] = {"mm_rmsnorm", MOD_LM_HEAD},
    [K_RMSNORM_HL] = {"mm_rmsnorm_hl", MOD_LM_HEAD},
    [K_LM_GEMM] = {"mm_lm_gemm", MOD_LM_HEAD},
    [K_LM_GEMV1] = {"mm_lm_gemv_1", MOD_LM_HEAD},
    [K_LM_GEMV2] = {"mm_lm_gemv_2", MOD_LM_HEAD},
    [K_LM_GEMV4] = {"mm_lm_gemv_4", MOD_LM_HEAD},
    [K_ARGMAX_PART] = {"mm_argmax_part", MOD_LM_HEAD},
    [K_ARGMAX_FINAL] = {"mm_argmax_final", MOD_LM_HEAD},
    [K_GEMV1] = {"mm_gemv_1", MOD_GEMV},
    [K_GEMV2] = {"mm_gemv_2", MOD_GEMV},
    [K_GEMV4] = {"mm_gemv_4", MOD_GEMV},
    [K_MLA_ROPE] = {"mm_mla_rope", MOD_MLA},
    [K_EMBED] = {"mm_embed", MOD_UTIL},
    [K_SWIGLU] = {"mm_swiglu", MOD_UTIL},
    [K_GEMM_SKINNY] = {"mm_gemm_skinny", MOD_GEMM_BF16},
    [K_GEMM_SKINNY_WIDE] = {"mm_gemm_skinny_wide", MOD_GEMM_BF16},
    [K_GEMM_HL] = {"mm_gemm_hl", MOD_GEMM_BF16},
    [K_SKINNY_REDUCE] = {"mm_skinny_reduce", MOD_GEMM_BF16},
    [K_REDUCE_RMSNORM] = {"mm_reduce_rmsnorm", MOD_LM_HEAD},
    [K_ZERO32] = {"mm_zero32", MOD_UTIL},
    [K_GATHER_ROWS] = {"mm_gather_rows", MOD_UTIL},
    [K_F32_BF16] = {"mm_f32_bf16", MOD_UTIL},
    [K_ROUTER_WIDE] = {"mm_router_wide", MOD_MOE_BF16},
    [K_ROUTE_WIDE] = {"mm_route_wide", MOD_MOE_I8},
};

/* ---- errors ------------------------------------------------------------- */
static _Thread_local char g_err[512];

const char *mm_last_error(void) { return g_err; }

int mm_fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int mm_hip_fail(hipError_t e, const char *what) {
    return mm_fail(e == hipErrorOutOfMemory ? MM_ERR_NOMEM : MM_ERR_HIP, "%s: %s (%d)", what,
                   hipGetErrorString(e), (int)e);
}

int mm_set_device(mm_ctx *ctx) {
    MM_HIP(hipSetDevice(ctx->device));
    return MM_OK;
}

/* ---- context ------------------------------------------------------------ */
int mm_ctx_create(int device, mm_ctx **out) {
    if (!out) return mm_fail(MM_ERR_INVALID, "mm_ctx_create: out is NULL");
    *out = NULL;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return mm_fail(MM_ERR_HIP, "mm_ctx_create: no HIP device");
    if (device < 0 || device >= n)
        return mm_fail(MM_ERR_INVALID, "mm_ctx_create: device %d out of range [0,%d)", device, n);
    hipDeviceProp_t prop;
    MM_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_ctx_create: device %d is %s, this build is gfx950",
                       device, prop.gcnArchName);
    if (prop.warpSize != 64)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_ctx_create: wave64 required");

    mm_ctx *c = calloc(1, sizeof(*c));
    if (!c) return mm_fail(MM_ERR_NOMEM, "mm_ctx_create: calloc");
    c->device = device;
    int st = MM_OK;
    if ((e = hipSetDevice(device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&c->t0)) != hipSuccess || (e = hipEventCreate(&c->t1)) != hipSuccess ||
        (e = hipEventCreateWithFlags(&c->ev_switch, hipEventDisableTiming)) != hipSuccess) {
        st = mm_hip_fail(e, "mm_ctx_create");
        goto fail;
    }
    c->stream = c->own_stream;
    c->modules = calloc(MOD_COUNT, sizeof(hipModule_t));
    if (!c->modules) {
        st = mm_fail(MM_ERR_NOMEM, "mm_ctx_create: calloc");
        goto fail;
    }
    for (int m = 0; m < MOD_COUNT; m++) {
        if ((e = hipModuleLoadData(&c->modules[m], mod_blob[m])) != hipSuccess) {
            st = mm_hip_fail(e, "hipModuleLoadData");
            goto fail;
        }
        c->n_modules = m + 1;
    }
    for (int k = 0; k < K_COUNT; k++) {
        if ((e = hipModuleGetFunction(&c->fn[k], c->modules[kinfo[k].module], kinfo[k].name)) !=
            hipSuccess) {
            st = mm_fail(MM_ERR_HIP, "hipModuleGetFunction(%s): %s", kinfo[k].name,
                         hipGetErrorString(e));
            goto fail;
        }
    }
    /* MLAMOE_I8_TILED_MIN_T overrides the token count from which the int8
     * path switches to the tiled GEMM (for measuring the crossover). */
    c->i8_tiled_min_t = 256;
    const char *ev = getenv("MLAMOE_I8_TILED_MIN_T");
    if (ev && *ev) c->i8_tiled_min_t = atoi(ev);
    /* MLAMOE_MLA_PART_MAX (bytes) overrides the cap on the attention chunk
     * partials of one launch, above which rows go in groups */
    c->mla_part_max = MM_MLA_PART_MAX;
    {
        const char *r4 = getenv("MLAMOE_MLA_ROWS4");
        c->mla_rows4 = !(r4 && r4[0] == '0');
    }
    ev = getenv("MLAMOE_MLA_PART_MAX");
    if (ev && *ev && atoll(ev) > 0) c->mla_part_max = (size_t)atoll(ev);
    /* MLAMOE_MOE_T_CHUNK lowers the rows of one MoE forward pass (longer
     * calls run in chunks of it; for testing that the chunks agree) */
    c->moe_t_chunk = 0;
    ev = getenv("MLAMOE_MOE_T_CHUNK");
    if (ev && *ev && atoi(ev) > 0) c->moe_t_chunk = atoi(ev);
    if ((st = mm_noalloc_setup(c))) goto fail;
    *out = c;
    return MM_OK;
fail:
    mm_ctx_destroy(c);
    return st;
}

void mm_ctx_destroy(mm_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    if (c->own_stream && c->own_stream != c->stream) hipStreamSynchronize(c->own_stream);
    mm_moe_release(c);
    mm_mla_release(c);
    mm_host_release(c);
    if (c->ws) hipFree(c->ws);
    if (c->io) hipFree(c->io);
    for (size_t i = 0; i < c->ev_pool_n; i++) hipEventDestroy(c->ev_pool[i]);
    free(c->ev_pool);
    free(c->prof);
    for (int m = 0; m < c->n_modules; m++) hipModuleUnload(c->modules[m]);
    free(c->modules);
    if (c->t0) hipEventDestroy(c->t0);
    if (c->t1) hipEventDestroy(c->t1);
    if (c->ev_switch) hipEventDestroy(c->ev_switch);
    if (c->own_stream) hipStreamDestroy(c->own_stream);
    free(c);
}

void *mm_ctx_stream(mm_ctx *c) { return c ? (void *)c->stream : NULL; }

int mm_ctx_set_stream(mm_ctx *c, void *stream) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_ctx_set_stream: NULL context");
    hipStream_t s = stream ? (hipStream_t)stream : c->own_stream;
    if (s == c->stream) return MM_OK;
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipEventRecord(c->ev_switch, c->stream));
    MM_HIP(hipStreamWaitEvent(s, c->ev_switch, 0));
    c->stream = s;
    return MM_OK;
}

int mm_ctx_sync(mm_ctx *c) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_ctx_sync: NULL context");
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipStreamSynchronize(c->stream));
    return MM_OK;
}

/* ---- launches and per-kernel timing ------------------------------------- */
/* Event `i` of the profiling pool (record r uses events 2r and 2r+1). */
static int pool_event(mm_ctx *c, size_t i, hipEvent_t *ev) {
    while (i >= c->ev_pool_n) {
        if (c->ev_pool_n == c->ev_pool_cap) {
            size_t cap = c->ev_pool_cap ? 2 * c->ev_pool_cap : 256;
            hipEvent_t *p = realloc(c->ev_pool, cap * sizeof(*p));
            if (!p) return mm_fail(MM_ERR_NOMEM, "profiler events");
            c->ev_pool = p;
            c->ev_pool_cap = cap;
        }
        MM_HIP(hipEventCreate(&c->ev_pool[c->ev_pool_n]));
        c->ev_pool_n++;
    }
    *ev = c->ev_pool[i];
    return MM_OK;
}

int mm_launch(mm_ctx *c, mm_kernel_id id, unsigned gx, unsigned gy, unsigned gz,
              unsigned block, size_t shmem, void *args) {
    if (gx == 0 || gy == 0 || gz == 0) return MM_OK;
    void *params[1] = {args};
    mm_prof_rec rec = {id, {0, 0}};
    if (c->prof_on) {
        if (c->prof_n == c->prof_cap) {
            size_t cap = c->prof_cap ? 2 * c->prof_cap : 128;
            mm_prof_rec *p = realloc(c->prof, cap * sizeof(*p));
            if (!p) return mm_fail(MM_ERR_NOMEM, "profiler records");
            c->prof = p;
            c->prof_cap = cap;
        }
        int st = pool_event(c, 2 * c->prof_n, &rec.ev[0]);
        if (!st) st = pool_event(c, 2 * c->prof_n + 1, &rec.ev[1]);
        if (st) return st;
        MM_HIP(hipEventRecord(rec.ev[0], c->stream));
    }
    hipError_t e = hipModuleLaunchKernel(c->fn[id], gx, gy, gz, block, 1, 1, (unsigned)shmem,
                                         c->stream, params, NULL);
    if (e != hipSuccess)
        return mm_fail(MM_ERR_HIP, "launch %s: %s", kinfo[id].name, hipGetErrorString(e));
    if (c->prof_on) {
        MM_HIP(hipEventRecord(rec.ev[1], c->stream));
        c->prof[c->prof_n++] = rec;
    }
    return MM_OK;
}

int mm_prof_enable(mm_ctx *c, int on) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_prof_enable: NULL context");
    c->prof_on = on != 0;
    return MM_OK;
}

int mm_prof_reset(mm_ctx *c) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_prof_reset: NULL context");
    int st = mm_ctx_sync(c);
    c->prof_n = 0;
    return st;
}

int mm_prof_query(mm_ctx *c, const char *kernel, double *total_ms, long long *launches) {
    if (!c || !kernel) return mm_fail(MM_ERR_INVALID, "mm_prof_query: bad argument");
    int st = mm_ctx_sync(c);
    if (st) return st;
    double tot = 0.0;
    long long n = 0;
    for (size_t i = 0; i < c->prof_n; i++) {
        if (strcmp(kinfo[c->prof[i].id].name, kernel) != 0) continue;
        float ms = 0.0f;
        MM_HIP(hipEventElapsedTime(&ms, c->prof[i].ev[0], c->prof[i].ev[1]));
        tot += ms;
        n++;
    }
    if (total_ms) *total_ms = tot;
    if (launches) *launches = n;
    return MM_OK;
}

int mm_timer_start(mm_ctx *c) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_timer_start: NULL context");
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipEventRecord(c->t0, c->stream));
    return MM_OK;
}

int mm_timer_stop(mm_ctx *c, float *ms) {
    if (!c || !ms) return mm_fail(MM_ERR_INVALID, "mm_timer_stop: bad argument");
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipEventRecord(c->t1, c->stream));
    MM_HIP(hipEventSynchronize(c->t1));
    MM_HIP(hipEventElapsedTime(ms, c->t0, c->t1));
    return MM_OK;
}

/* ---- memory --------------------------------------------------------------- */
int mm_dev_alloc(mm_ctx *c, size_t bytes, void **dptr) {
    if (!c || !dptr) return mm_fail(MM_ERR_INVALID, "mm_dev_alloc: bad argument");
    *dptr = NULL;
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipMalloc(dptr, bytes ? bytes : 1));
    return MM_OK;
}

int mm_dev_free(mm_ctx *c, void *dptr) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_dev_free: NULL context");
    if (!dptr) return MM_OK;
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipStreamSynchronize(c->stream));
    MM_HIP(hipFree(dptr));
    return MM_OK;
}

static int copy(mm_ctx *c, void *dst, const void *src, size_t bytes, hipMemcpyKind k) {
    if (!c || (bytes && (!dst || !src))) return mm_fail(MM_ERR_INVALID, "copy: bad argument");
    if (!bytes) return MM_OK;
    MM_HIP(hipSetDevice(c->device));
    MM_HIP(hipMemcpyAsync(dst, src, bytes, k, c->stream));
    MM_HIP(hipStreamSynchronize(c->stream));
    return MM_OK;
}

int mm_h2d(mm_ctx *c, void *dst, const void *src, size_t bytes) {
    return copy(c, dst, src, bytes, hipMemcpyHostToDevice);
}
int mm_d2h(mm_ctx *c, void *dst, const void *src, size_t bytes) {
    return copy(c, dst, src, bytes, hipMemcpyDeviceToHost);
}
int mm_d2d(mm_ctx *c, void *dst, const void *src, size_t bytes) {
    return copy(c, dst, src, bytes, hipMemcpyDeviceToDevice);
}

int mm_workspace(mm_ctx *c, size_t bytes, void **out) {
    if (bytes > c->ws_bytes) {
        MM_HIP(hipStreamSynchronize(c->stream));
        if (c->ws) MM_HIP(hipFree(c->ws));
        c->ws = NULL;
        c->ws_bytes = 0;
        size_t nb = bytes + bytes / 4;
        MM_HIP(hipMalloc(&c->ws, nb));
        c->ws_bytes = nb;
    }
    *out = c->ws;
    return MM_OK;
}

int mm_io_buffer(mm_ctx *c, size_t bytes, void **out) {
    if (bytes > c->io_bytes) {
        MM_HIP(hipStreamSynchronize(c->stream));
        if (c->io) MM_HIP(hipFree(c->io));
        c->io = NULL;
        c->io_bytes = 0;
        MM_HIP(hipMalloc(&c->io, bytes));
        c->io_bytes = bytes;
    }
    *out = c->io;
    return MM_OK;
}

int mm_ctx_workspace_bytes(mm_ctx *c, size_t *bytes) {
    if (!c || !bytes) return mm_fail(MM_ERR_INVALID, "mm_ctx_workspace_bytes: bad argument");
    *bytes = c->ws_bytes;
    return MM_OK;
}

int mm_fill_synthetic(mm_ctx *c, void *dst, size_t n, int kind, uint64_t seed, float stdev) {
    if (!c || (n && !dst) || kind < 0 || kind > 2)
        return mm_fail(MM_ERR_INVALID, "mm_fill_synthetic: bad argument");
    int st = mm_set_device(c);
    if (st) return st;
    mm_fill_args a = {dst, (uint64_t)n, seed, stdev, kind};
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    return mm_launch(c, K_FILL, (unsigned)blocks, 1, 1, 256, 0, &a);
}
