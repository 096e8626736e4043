/* gemm_bf16.hip -- dense y = x . W^T on v_mfma_f32_16x16x32_bf16 (matmul of
 * src/run.c:29-37 batched over T rows).
 *
 * W is bf16 row-major [d_out, n_in] exactly as the reference stores it: a B
 * operand fragment (16 output columns x 32 inputs, lane l holding column
 * l % 16 and inputs 8*(l/16) .. +7) is 16 contiguous bytes of one weight row
 * per lane.  x is fp32: either truncated to bf16 (the config that casts
 * activations on the input side, include/tensor.h:16-20) or split into a
 * bf16 hi/lo pair (two MFMAs, ~2^-17 relative) so the result tracks the fp32
 * reference.  Block tile 64 x 64, four waves of 32 x 32, K step 32; operands
 * are read from L1/L2 directly (the GEMMs of this path are small enough that
 * the block grid, not LDS reuse, is what fills the machine).
 */
#include "common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint16_t rne16(float x) {
    uint32_t u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

extern "C" __global__ __launch_bounds__(256) void mm_gemm_bf16(mm_gemm_bf16_args a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r16 = lane & 15;
    const int m0 = blockIdx.y * 64 + wm * 32, n0 = blockIdx.x * 64 + wn * 32;
    const int K = a.n_in;

    const float *xr[2];
    const uint16_t *wr[2];
    bool mv[2], nv[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int m = m0 + i * 16 + r16, n = n0 + i * 16 + r16;
        mv[i] = m < a.T;
        nv[i] = n < a.d_out;
        xr[i] = a.x + (size_t)(mv[i] ? m : 0) * K + 8 * g;
        wr[i] = a.w + (size_t)(nv[i] ? n : 0) * K + 8 * g;
    }
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    for (int k0 = 0; k0 < K; k0 += 32) {
        const bool kv = k0 + 8 * g < K;   /* K is a multiple of 8 */
        bf16x8 ah[2], al[2], bw[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            u16x8 hi = {0, 0, 0, 0, 0, 0, 0, 0}, lo = {0, 0, 0, 0, 0, 0, 0, 0};
            if (mv[i] && kv) {
                const f32x4 x0 = *(const f32x4 *)(xr[i] + k0), x1 = *(const f32x4 *)(xr[i] + k0 + 4);
                const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (a.x_bf16) {
                        hi[j] = (uint16_t)(__float_as_uint(xs[j]) >> 16);   /* truncation */
                    } else {
                        const uint16_t h = rne16(xs[j]);
                        hi[j] = h;
                        lo[j] = rne16(xs[j] - bf16_f32(h));
                    }
                }
            }
            ah[i] = __builtin_bit_cast(bf16x8, hi);
            al[i] = __builtin_bit_cast(bf16x8, lo);
            u16x8 wv = {0, 0, 0, 0, 0, 0, 0, 0};
            if (nv[i] && kv) wv = *(const u16x8 *)(wr[i] + k0);
            bw[i] = __builtin_bit_cast(bf16x8, wv);
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bw[j], acc[i][j], 0, 0, 0);
                if (!a.x_bf16)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bw[j], acc[i][j], 0, 0, 0);
            }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + j * 16 + r16;
            if (n >= a.d_out) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + i * 16 + 4 * g + e;
                if (m >= a.T) continue;
                float *o = a.y + (size_t)m * a.d_out + n;
                *o = a.accumulate ? *o + acc[i][j][e] : acc[i][j][e];
            }
        }
}
