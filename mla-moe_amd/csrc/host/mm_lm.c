/* mm_lm.c -- the decode step's LM head (host side): final RMSNorm, logits
 * over the vocabulary, greedy argmax (src/run.c:22-27, 493-494, 503-508). */
#include "mm_internal.h"

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

int mm_rmsnorm_dev(mm_ctx *c, int T, const float *x, const uint16_t *w, int n, float eps, float *y) {
    if (!c || (T > 0 && (!x || !w || !y))) return mm_fail(MM_ERR_INVALID, "mm_rmsnorm_dev: NULL argument");
    if (T < 0 || n <= 0) return mm_fail(MM_ERR_INVALID, "mm_rmsnorm_dev: bad shape");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    mm_rmsnorm_args a = {x, w, y, n, eps};
    return mm_launch(c, K_RMSNORM, (unsigned)T, 1, 1, 256, 0, &a);
}

/* Workspace bytes of the two-pass argmax over T rows of n. */
static size_t argmax_ws(int T, int n) {
    const size_t nseg = ((size_t)n + MM_ARGMAX_SEG - 1) / MM_ARGMAX_SEG;
    return 2 * al256((size_t)T * nseg * 4);
}

static int argmax_launch(mm_ctx *c, int T, const float *logits, int n, int32_t *tokens, char *ws) {
    const int nseg = (n + MM_ARGMAX_SEG - 1) / MM_ARGMAX_SEG;
    mm_argmax_args a = {logits, tokens, (float *)ws,
                        (int32_t *)(ws + al256((size_t)T * nseg * 4)), n, T, nseg};
    int st = mm_launch(c, K_ARGMAX_PART, (unsigned)nseg, (unsigned)T, 1, 256, 0, &a);
    if (st) return st;
    return mm_launch(c, K_ARGMAX_FINAL, (unsigned)T, 1, 1, 256, 0, &a);
}

int mm_argmax_dev(mm_ctx *c, int T, const float *logits, int n, int32_t *tokens) {
    if (!c || (T > 0 && (!logits || !tokens))) return mm_fail(MM_ERR_INVALID, "mm_argmax_dev: NULL argument");
    if (T < 0 || n <= 0) return mm_fail(MM_ERR_INVALID, "mm_argmax_dev: bad shape");
    if (T == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    char *ws;
    if ((st = mm_workspace(c, argmax_ws(T, n), (void **)&ws))) return st;
    return argmax_launch(c, T, logits, n, tokens, ws);
}

int mm_lm_head_dev(mm_ctx *c, int B, const float *x, const uint16_t *norm, float eps,
                   const uint16_t *lm_head, int vocab, int hidden, float *logits, int32_t *tokens) {
    if (!c || (B > 0 && (!x || !norm || !lm_head || !tokens)))
        return mm_fail(MM_ERR_INVALID, "mm_lm_head_dev: NULL argument");
    if (B < 0 || vocab <= 0 || hidden <= 0) return mm_fail(MM_ERR_INVALID, "mm_lm_head_dev: bad shape");
    if (hidden % 8) return mm_fail(MM_ERR_UNSUPPORTED, "mm_lm_head_dev: hidden must be a multiple of 8");
    if ((uintptr_t)lm_head % 16 || (logits && (uintptr_t)logits % 16))
        return mm_fail(MM_ERR_INVALID, "mm_lm_head_dev: lm_head and logits must be 16-byte aligned");
    if (B == 0) return MM_OK;
    int st = mm_set_device(c);
    if (st) return st;
    const int gemv = B <= MM_LM_NB && hidden <= MM_LM_HMAX;
    /* workspace: xb [B, hidden] (GEMM path), logits [B, vocab] when not
     * returned, GEMM staging, argmax partials */
    const size_t rpb = 4 * MM_GEMV_RPW;           /* GEMV rows per block per turn */
    const size_t nb = gemv ? (((size_t)vocab + rpb - 1) / rpb < MM_LM_GEMV_BLOCKS
                                  ? ((size_t)vocab + rpb - 1) / rpb : MM_LM_GEMV_BLOCKS)
                           : 0;
    const size_t o_xb = 0, n_xb = gemv ? 0 : al256((size_t)B * hidden * 4);
    const size_t o_lg = o_xb + n_xb, n_lg = logits ? 0 : al256((size_t)B * vocab * 4);
    const size_t o_gm = o_lg + n_lg, n_gm = gemv ? 0 : al256(mm_gemm_bf16_ws_bytes(B, hidden, vocab, 0));
    const size_t o_am = o_gm + n_gm;
    const size_t n_am = gemv ? 2 * al256((size_t)B * nb * 4) : argmax_ws(B, vocab);
    char *ws;
    if ((st = mm_workspace(c, o_am + n_am, (void **)&ws))) return st;
    float *lg = logits ? logits : (float *)(ws + o_lg);
    if (gemv) {
        /* one pass: norm, logits, per-block argmax partials; then the final
         * reduction over the nb partials of each token */
        float *pv = (float *)(ws + o_am);
        int32_t *pi = (int32_t *)(ws + o_am + al256((size_t)B * nb * 4));
        mm_lm_gemv_args ga = {x, norm, eps, lm_head, lg, pv, pi, B, vocab, hidden};
        const mm_kernel_id id = B <= 1 ? K_LM_GEMV1 : B <= 2 ? K_LM_GEMV2 : K_LM_GEMV4;
        if ((st = mm_launch(c, id, (unsigned)nb, 1, 1, 256, 0, &ga))) return st;
        mm_argmax_args fa = {lg, tokens, pv, pi, vocab, B, (int)nb};
        return mm_launch(c, K_ARGMAX_FINAL, (unsigned)B, 1, 1, 256, 0, &fa);
    }
    if (B <= 64 && hidden % 64 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)norm % 16 == 0) {
        /* the norm writes bf16 hi/lo planes (the same bytes as xb's fp32)
         * for the logits GEMM's direct-to-LDS ring */
        uint16_t *xhl = (uint16_t *)(ws + o_xb);
        mm_rmsnorm_hl_args rh = {x, norm, xhl, hidden, eps};
        if ((st = mm_launch(c, K_RMSNORM_HL, (unsigned)B, 1, 1, 256, 0, &rh))) return st;
        mm_lm_gemm_args lg_a = {xhl, lm_head, lg, B, vocab, hidden};
        if ((st = mm_launch(c, K_LM_GEMM, (unsigned)((vocab + MM_LMG_BN - 1) / MM_LMG_BN), 1, 1, 256,
                            (size_t)MM_LMG_NS * MM_LMG_STAGE, &lg_a)))
            return st;
        return argmax_launch(c, B, lg, vocab, tokens, ws + o_am);
    }
    float *xb = (float *)(ws + o_xb);
    mm_rmsnorm_args ra = {x, norm, xb, hidden, eps};
    if ((st = mm_launch(c, K_RMSNORM, (unsigned)B, 1, 1, 256, 0, &ra))) return st;
    if ((st = mm_gemm_bf16_ws(c, lg, xb, lm_head, vocab, hidden, B, 0, ws + o_gm))) return st;
    return argmax_launch(c, B, lg, vocab, tokens, ws + o_am);
}
