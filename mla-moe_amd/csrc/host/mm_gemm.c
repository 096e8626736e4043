/* mm_gemm.c -- dense bf16 matmul (host side): the reference's matmul
 * (src/run.c:29-37) batched over T rows. */
#include "mm_internal.h"

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
    const int split = (flags & MM_MATMUL_X_BF16) == 0;
    /* x as bf16 rows of a stride padded to 64 (zeros past n_in) */
    const int kp = (n_in + 63) / 64 * 64;
    const size_t xb = (size_t)T * kp * 2;
    char *ws;
    if ((st = mm_workspace(c, (split ? 2 : 1) * ((xb + 255) & ~(size_t)255), (void **)&ws))) return st;
    uint16_t *xh = (uint16_t *)ws, *xl = split ? (uint16_t *)(ws + ((xb + 255) & ~(size_t)255)) : NULL;
    mm_cvt_bf16_args ca = {x, xh, xl, T, n_in, kp, split};
    const size_t chunks = (size_t)T * kp / 8;
    if ((st = mm_launch(c, K_CVT_BF16, (unsigned)((chunks + 255) / 256), 1, 1, 256, 0, &ca))) return st;
    mm_gemm_bf16_args a = {xh, xl, w, y, T, d_out, n_in, kp, split, (flags & MM_MATMUL_ACCUMULATE) != 0};
    /* LDS ring: 4 stages of A and B (32 KB) or 3 of A hi, A lo and B (48 KB);
     * a 1-D grid of 8 XCD columns, each with every row block of its column
     * blocks (the kernel maps blocks to tiles) */
    const size_t lds = split ? (size_t)3 * 49152 : (size_t)4 * 32768;
    const size_t nbx = ((size_t)d_out + 127) / 128, nby = ((size_t)T + 127) / 128;
    return mm_launch(c, K_GEMM_BF16, (unsigned)(8 * ((nbx + 7) / 8) * nby), 1, 1, 256, lds, &a);
}
