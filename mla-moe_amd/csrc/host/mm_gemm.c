/* mm_gemm.c -- dense bf16 matmul (host side): the reference's matmul
 * (src/run.c:29-37) batched over T rows. */
#include "mm_internal.h"

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

/* Skinny-M plan: T <= MM_SKINNY_T rows and n_in a multiple of 64.  Blocks of
 * MM_SKINNY_BN output columns; the K range splits until the grid has about one block
 * per CU (partials summed by mm_skinny_reduce). */
static int skinny_ok(int T, int n_in) { return T <= MM_SKINNY_T && n_in % 64 == 0; }

#ifndef MM_SKINNY_BLOCKS
#define MM_SKINNY_BLOCKS 256      /* target grid: about one block per CU */
#endif
/* nb column blocks in all: split K until the grid has about
 * MM_SKINNY_BLOCKS blocks */
static void skinny_plan(int nb, int n_in, int *nsplit, int *kr) {
    const int nk = n_in / 64;
    int ns = (MM_SKINNY_BLOCKS + nb - 1) / nb;
    if (ns > nk) ns = nk;
    if (ns < 1) ns = 1;
    const int kc = (nk + ns - 1) / ns;          /* 64-input chunks per split */
    *kr = 64 * kc;
    *nsplit = (nk + kc - 1) / kc;
}

static int skinny_nb(int d) { return (d + MM_SKINNY_BN - 1) / MM_SKINNY_BN; }

/* one long matrix (the LM head): the wide form, 64 * MM_SKINNY_WIDE_WC
 * columns per block */
static int skinny_wide(int d0, int d1) { return d1 <= 0 && skinny_nb(d0) >= MM_SKINNY_WIDE_MIN_NB; }
static int skinny_nb_wide(int d) {
    return (d + 64 * MM_SKINNY_WIDE_WC - 1) / (64 * MM_SKINNY_WIDE_WC);
}

size_t mm_gemm_bf16_ws2_bytes(int T, int n_in, int d0, int d1, unsigned flags) {
    if (skinny_ok(T, n_in)) {                    /* only the split partials */
        int ns, kr;
        skinny_plan(skinny_wide(d0, d1) ? skinny_nb_wide(d0)
                                        : skinny_nb(d0) + (d1 > 0 ? skinny_nb(d1) : 0),
                    n_in, &ns, &kr);
        return ns > 1 ? al256((size_t)ns * T * ((size_t)d0 + (d1 > 0 ? d1 : 0)) * 4) : 256;
    }
    const int split = (flags & MM_MATMUL_X_BF16) == 0;
    const size_t xb = (size_t)T * ((n_in + 63) / 64 * 64) * 2;
    return (split ? 2 : 1) * al256(xb);
}

size_t mm_gemm_bf16_ws_bytes(int T, int n_in, int d_out, unsigned flags) {
    return mm_gemm_bf16_ws2_bytes(T, n_in, d_out, 0, flags);
}

static int gemm_bf16_rows(mm_ctx *c, float *y, const uint16_t *xh, const uint16_t *xl,
                          const uint16_t *w, int d_out, int n_in, int kp, int T, int split, int acc);
static int cvt_rows(mm_ctx *c, const float *x, int n_in, int T, int split, char *ws,
                    uint16_t **xh, uint16_t **xl, int *kp);

int mm_gemm_bf16_ws2(mm_ctx *c, float *y0, const uint16_t *w0, int d0, float *y1,
                     const uint16_t *w1, int d1, const float *x, int n_in, int T, unsigned flags,
                     char *ws) {
    const int split = (flags & MM_MATMUL_X_BF16) == 0;
    const int acc = (flags & MM_MATMUL_ACCUMULATE) != 0;
    int st;
    if (!w1) d1 = 0;
    if (skinny_ok(T, n_in)) {
        /* fp32 x converted while staged; ws holds the split partials; both
         * matrices in one launch */
        const int wide = skinny_wide(d0, d1);
        const int nb0 = wide ? skinny_nb_wide(d0) : skinny_nb(d0), nb = nb0 + (d1 ? skinny_nb(d1) : 0);
        int ns, kr;
        skinny_plan(nb, n_in, &ns, &kr);
        mm_gemm_skinny_args k = {x, w0, y0, (float *)ws, T, d0, n_in, ns, kr, split, acc,
                                 w1, y1, d1, nb0, 0};
        if ((st = mm_launch(c, wide ? K_GEMM_SKINNY_WIDE : K_GEMM_SKINNY, (unsigned)nb, (unsigned)ns,
                            1, 256, 0, &k)))
            return st;
        if (ns == 1) return MM_OK;
        mm_skinny_reduce_args r = {(float *)ws, y0, T, d0, ns, acc, d1 ? y1 : NULL, d1};
        const size_t n = (size_t)T * ((size_t)d0 + d1);
        const size_t blocks = (n + 255) / 256 < 2048 ? (n + 255) / 256 : 2048;
        return mm_launch(c, K_SKINNY_REDUCE, (unsigned)blocks, 1, 1, 256, 0, &r);
    }
    /* x converted once for both weights */
    uint16_t *xh, *xl;
    int kp;
    if ((st = cvt_rows(c, x, n_in, T, split, ws, &xh, &xl, &kp))) return st;
    if ((st = gemm_bf16_rows(c, y0, xh, xl, w0, d0, n_in, kp, T, split, acc))) return st;
    return d1 ? gemm_bf16_rows(c, y1, xh, xl, w1, d1, n_in, kp, T, split, acc) : MM_OK;
}

size_t mm_gemm_bf16_hl_ws_bytes(int T, int n_in, int d0, int d1) {
    int ns, kr;
    skinny_plan(skinny_nb(d0) + (d1 > 0 ? skinny_nb(d1) : 0), n_in, &ns, &kr);
    return ns > 1 ? al256((size_t)ns * T * ((size_t)d0 + (d1 > 0 ? d1 : 0)) * 4) : 256;
}

int mm_gemm_bf16_hl(mm_ctx *c, float *y0, const uint16_t *w0, int d0, float *y1,
                    const uint16_t *w1, int d1, const uint16_t *xhl, int n_in, int T, int acc,
                    char *ws) {
    if (!w1) d1 = 0;
    /* the skinny plan: 64-column blocks, K split until ~one block per CU */
    const int nb0 = skinny_nb(d0), nb = nb0 + (d1 ? skinny_nb(d1) : 0);
    int ns, kr, st;
    skinny_plan(nb, n_in, &ns, &kr);
    mm_gemm_hl_args k = {xhl, w0, y0, (float *)ws, T, d0, n_in, ns, kr, acc, w1, y1, d1, nb0, 0};
    if ((st = mm_launch(c, K_GEMM_HL, (unsigned)nb, (unsigned)ns, 1, 256, 0, &k))) return st;
    if (ns == 1) return MM_OK;
    mm_skinny_reduce_args r = {(float *)ws, y0, T, d0, ns, acc, d1 ? y1 : NULL, d1};
    const size_t n = (size_t)T * ((size_t)d0 + d1);
    const size_t blocks = (n + 255) / 256 < 2048 ? (n + 255) / 256 : 2048;
    return mm_launch(c, K_SKINNY_REDUCE, (unsigned)blocks, 1, 1, 256, 0, &r);
}

/* x += a . w^T, then xn = rmsnorm(x, norm_w) -- for T <= MM_SKINNY_T rows
 * the split-K partials are summed by the norm pass itself (one launch fewer;
 * the partial sums and residual adds are the skinny reduce's, the norm's sum
 * of squares is reduced over 1024 threads instead of 256);
 * otherwise the GEMM accumulates and mm_rmsnorm follows.  d_out is the row
 * length of x. */
size_t mm_gemm_bf16_add_rmsnorm_ws_bytes(int T, int n_in, int d_out) {
    if (skinny_ok(T, n_in) && d_out <= MM_RRN_THREADS * MM_RRN_PT) {
        int ns, kr;
        skinny_plan(skinny_nb(d_out), n_in, &ns, &kr);
        return al256((size_t)ns * T * d_out * 4);
    }
    return mm_gemm_bf16_ws_bytes(T, n_in, d_out, 0);
}

int mm_gemm_bf16_add_rmsnorm(mm_ctx *c, float *x, const float *a, const uint16_t *w, int d_out,
                             int n_in, int T, const uint16_t *norm_w, float eps, float *xn,
                             char *ws) {
    int st;
    if (skinny_ok(T, n_in) && d_out <= MM_RRN_THREADS * MM_RRN_PT) {
        const int nb = skinny_nb(d_out);
        int ns, kr;
        skinny_plan(nb, n_in, &ns, &kr);
        mm_gemm_skinny_args k = {a, w, x, (float *)ws, T, d_out, n_in, ns, kr, 1, 0,
                                 NULL, NULL, 0, nb, 1};
        if ((st = mm_launch(c, K_GEMM_SKINNY, (unsigned)nb, (unsigned)ns, 1, 256, 0, &k))) return st;
        mm_reduce_rmsnorm_args r = {(const float *)ws, x, norm_w, xn, T, d_out, ns, eps};
        return mm_launch(c, K_REDUCE_RMSNORM, (unsigned)T, 1, 1, MM_RRN_THREADS, 0, &r);
    }
    if ((st = mm_gemm_bf16_ws(c, x, a, w, d_out, n_in, T, MM_MATMUL_ACCUMULATE, ws))) return st;
    mm_rmsnorm_args r = {x, norm_w, xn, d_out, eps};
    return mm_launch(c, K_RMSNORM, (unsigned)T, 1, 1, 256, 0, &r);
}

int mm_gemm_bf16_add_rmsnorm_hl(mm_ctx *c, float *x, const uint16_t *ahl, const uint16_t *w,
                                int d_out, int n_in, int T, const uint16_t *norm_w, float eps,
                                float *xn, char *ws) {
    const int nb = skinny_nb(d_out);
    int ns, kr, st;
    skinny_plan(nb, n_in, &ns, &kr);
    mm_gemm_hl_args k = {ahl, w, x, (float *)ws, T, d_out, n_in, ns, kr, 0, NULL, NULL, 0, nb, 1};
    if ((st = mm_launch(c, K_GEMM_HL, (unsigned)nb, (unsigned)ns, 1, 256, 0, &k))) return st;
    mm_reduce_rmsnorm_args r = {(const float *)ws, x, norm_w, xn, T, d_out, ns, eps};
    return mm_launch(c, K_REDUCE_RMSNORM, (unsigned)T, 1, 1, MM_RRN_THREADS, 0, &r);
}

/* y = x W^T on x already in bf16 rows of stride kp (xh, and xl with split) */
static int gemm_bf16_rows(mm_ctx *c, float *y, const uint16_t *xh, const uint16_t *xl,
                          const uint16_t *w, int d_out, int n_in, int kp, int T, int split, int acc) {
    /* block tile columns: the widest of 128, 64, 32 that still gives 192
     * tiles (most of the 256 CUs), else 32 -- the projections of this path
     * have too few 128 x 128 tiles to fill the machine (measured per width) */
    const size_t nby = ((size_t)T + 127) / 128;
    int bn = 32;
    for (int cw = 128; cw >= 64; cw /= 2)
        if (((size_t)d_out + cw - 1) / cw * nby >= 192) {
            bn = cw;
            break;
        }
    const size_t nbx = ((size_t)d_out + bn - 1) / bn;
    mm_gemm_bf16_args a = {xh, xl, w, y, T, d_out, n_in, kp, split, acc, bn};
    /* LDS ring: 4 stages (3 for the hi/lo split) of A hi [, A lo] (16 KB
     * each) and bn rows of B (128 B each); a 1-D grid of 8 XCD columns, each
     * with every row block of its column blocks (the kernel maps blocks to
     * tiles) */
    const size_t stage = (size_t)(split ? 2 : 1) * 16384 + (size_t)bn * 128;
    const size_t lds = (split ? 3 : 4) * stage;
    return mm_launch(c, K_GEMM_BF16, (unsigned)(8 * ((nbx + 7) / 8) * nby), 1, 1, 256, lds, &a);
}

/* x as bf16 rows of a stride padded to 64 (zeros past n_in) into ws: hi,
 * then (split) lo */
static int cvt_rows(mm_ctx *c, const float *x, int n_in, int T, int split, char *ws,
                    uint16_t **xh, uint16_t **xl, int *kp) {
    *kp = (n_in + 63) / 64 * 64;
    const size_t xb = (size_t)T * *kp * 2;
    *xh = (uint16_t *)ws;
    *xl = split ? (uint16_t *)(ws + al256(xb)) : NULL;
    mm_cvt_bf16_args ca = {x, *xh, *xl, T, n_in, *kp, split};
    const size_t chunks = (size_t)T * *kp / 8;
    return mm_launch(c, K_CVT_BF16, (unsigned)((chunks + 255) / 256), 1, 1, 256, 0, &ca);
}

int mm_gemm_bf16_ws(mm_ctx *c, float *y, const float *x, const uint16_t *w, int d_out, int n_in,
                    int T, unsigned flags, char *ws) {
    if (skinny_ok(T, n_in)) return mm_gemm_bf16_ws2(c, y, w, d_out, NULL, NULL, 0, x, n_in, T, flags, ws);
    const int split = (flags & MM_MATMUL_X_BF16) == 0;
    const int acc = (flags & MM_MATMUL_ACCUMULATE) != 0;
    uint16_t *xh, *xl;
    int kp, st;
    if ((st = cvt_rows(c, x, n_in, T, split, ws, &xh, &xl, &kp))) return st;
    return gemm_bf16_rows(c, y, xh, xl, w, d_out, n_in, kp, T, split, acc);
}

unsigned mm_gemv_blocks(int rows) {
    /* 4 waves per block, MM_GEMV_RPW rows per wave per turn: one turn covers
     * every row when the grid allows */
    const unsigned b = (unsigned)((rows + 4 * MM_GEMV_RPW - 1) / (4 * MM_GEMV_RPW));
    return b < 2048 ? b : 2048;
}

int mm_gemv_launch(mm_ctx *c, const mm_gemv_args *a) {
    mm_gemv_args k = *a;
    const mm_kernel_id id = a->B <= 1 ? K_GEMV1 : a->B <= 2 ? K_GEMV2 : K_GEMV4;
    return mm_launch(c, id, mm_gemv_blocks(a->rows0 + a->rows1), 1, 1, 256, 0, &k);
}

int mm_matmul_bf16_hl_dev(mm_ctx *c, float *y, const uint16_t *xhl, const uint16_t *w, int d_out,
                          int n_in, int T, unsigned flags) {
    if (!c || (T > 0 && (!y || !xhl || !w)))
        return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16_hl_dev: NULL argument");
    if (T < 0 || T > MM_SKINNY_T || d_out <= 0 || n_in <= 0)
        return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16_hl_dev: need 0 <= T <= %d", MM_SKINNY_T);
    if (n_in % 64)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_matmul_bf16_hl_dev: n_in must be a multiple of 64");
    if ((uintptr_t)xhl % 16 || (uintptr_t)w % 16)
        return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16_hl_dev: xhl and w must be 16-byte aligned");
    if (flags & MM_MATMUL_X_BF16)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_matmul_bf16_hl_dev: x is a hi/lo pair");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    char *ws;
    if ((st = mm_workspace(c, mm_gemm_bf16_hl_ws_bytes(T, n_in, d_out, 0), (void **)&ws))) return st;
    return mm_gemm_bf16_hl(c, y, w, d_out, NULL, NULL, 0, xhl, n_in, T,
                           (flags & MM_MATMUL_ACCUMULATE) != 0, ws);
}

int mm_matmul_bf16_dev(mm_ctx *c, float *y, const float *x, const uint16_t *w, int d_out,
                       int n_in, int T, unsigned flags) {
    if (!c || (T > 0 && (!y || !x || !w)))
        return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16_dev: NULL argument");
    if (T < 0 || d_out <= 0 || n_in <= 0)
        return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16_dev: bad shape");
    if (n_in % 8)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_matmul_bf16_dev: n_in must be a multiple of 8");
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16)
        return mm_fail(MM_ERR_INVALID, "mm_matmul_bf16_dev: x and w must be 16-byte aligned");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    if (T <= MM_GEMV_NB && n_in <= MM_LM_HMAX) {
        mm_gemv_args a = {x, NULL, 0.0f, w, NULL, y, NULL, d_out, 0, d_out, 0, T, n_in,
                          (flags & MM_MATMUL_ACCUMULATE) != 0, (flags & MM_MATMUL_X_BF16) != 0};
        return mm_gemv_launch(c, &a);
    }
    char *ws;
    if ((st = mm_workspace(c, mm_gemm_bf16_ws_bytes(T, n_in, d_out, flags), (void **)&ws))) return st;
    return mm_gemm_bf16_ws(c, y, x, w, d_out, n_in, T, flags, ws);
}
