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
    mm_gemm_bf16_args a = {x, w, y, T, d_out, n_in, (flags & MM_MATMUL_X_BF16) != 0,
                           (flags & MM_MATMUL_ACCUMULATE) != 0};
    return mm_launch(c, K_GEMM_BF16, (unsigned)((d_out + 63) / 64), (unsigned)((T + 63) / 64), 1,
                     256, 0, &a);
}
