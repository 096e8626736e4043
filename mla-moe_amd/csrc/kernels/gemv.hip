/* gemv.hip -- dense bf16 GEMV for up to MM_GEMV_NB tokens on gfx950: the
 * decode step's projections (q_proj / q_a_proj with kv_a_proj in one pass,
 * q_b_proj, o_proj) and the reference's matmul (src/run.c:29-37) at T <= 4.
 *
 * HBM-bound: 2 bytes per weight, every row read once (gemv.h).  Two weight
 * matrices that share the activations run as one row space, as the
 * reference's GPU path pairs q_proj with kv_a_proj (src/getp_run.hip:497-508),
 * so the activations are loaded, and optionally normalised, once per wave
 * for both.  Accumulation is fp32 in a different association than the
 * sequential loop of run.c:29-37 (~1e-6 relative, which the tests bound).
 */
#include "gemv.h"

struct gemv_sink {
    float *y0, *y1;
    int rows0, ys0, ys1, B, accumulate;
    __device__ __forceinline__ void operator()(int row, int t, float v) {
        if ((threadIdx.x & (MM_WAVE - 1)) != 0 || t >= B) return;
        float *y = row < rows0 ? y0 + (size_t)t * ys0 + row : y1 + (size_t)t * ys1 + (row - rows0);
        *y = accumulate ? *y + v : v;
    }
};

template <int NB>
__device__ __forceinline__ void gemv_two(const mm_gemv_args &a) {
    f32x4 xv[NB][GV_PPL][2];
    gemv_load_x<NB>(xv, a.x, a.B, a.H, a.norm, a.eps, a.x_bf16 != 0);
    gemv_sink sk{a.y0, a.y1, a.rows0, a.ys0, a.ys1, a.B, a.accumulate};
    const uint16_t *w0 = a.w0, *w1 = a.w1;
    const int H = a.H, rows0 = a.rows0;
    gemv_rows<NB>(xv, H, a.rows0 + a.rows1,
                  [=](int r) { return r < rows0 ? w0 + (size_t)r * H : w1 + (size_t)(r - rows0) * H; },
                  sk);
}

/* One entry point per token count, so that the register allocation (and
 * with it the occupancy) of the one-token kernel is not that of the four-
 * token one. */
extern "C" __global__ __launch_bounds__(256) void mm_gemv_1(mm_gemv_args a) { gemv_two<1>(a); }
extern "C" __global__ __launch_bounds__(256) void mm_gemv_2(mm_gemv_args a) { gemv_two<2>(a); }
extern "C" __global__ __launch_bounds__(256) void mm_gemv_4(mm_gemv_args a) { gemv_two<4>(a); }
