/* util.hip -- device-side data preparation (synthetic inputs, the int8
 * per-output-channel weight quantiser) and the decode step's elementwise
 * pieces (token embedding, dense SwiGLU). */
#include "common.h"

/* Counter-based generator: splitmix64 of (seed, index), so any element can be
 * produced independently.  Normal samples use Box-Muller on two 32-bit
 * uniforms.  Used for large synthetic benchmark inputs only. */
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float gen_normal(uint64_t seed, uint64_t i) {
    uint64_t h = splitmix64(seed * 0x2545F4914F6CDD1Dull ^ splitmix64(i));
    float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);   /* (0, 1] */
    float u2 = (float)(uint32_t)(h & 0xFFFFFFu) * (1.0f / 16777216.0f);      /* [0, 1) */
    return sqrtf(-2.0f * __logf(u1)) * __cosf(6.28318530718f * u2);
}

extern "C" __global__ __launch_bounds__(256) void mm_fill(mm_fill_args a) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
        if (a.kind == 0) {
            float v = gen_normal(a.seed, i) * a.std;
            ((uint16_t *)a.dst)[i] = (uint16_t)(__float_as_uint(v) >> 16);   /* truncation */
        } else if (a.kind == 1) {
            ((float *)a.dst)[i] = gen_normal(a.seed, i) * a.std;
        } else {
            uint64_t h = splitmix64(a.seed * 0x2545F4914F6CDD1Dull ^ splitmix64(i));
            ((float *)a.dst)[i] = (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
        }
    }
}

/* Zero n 32-bit words in stream order (per-expert counters of the tiled
 * int8 path are cleared this way before every routing pass). */
extern "C" __global__ __launch_bounds__(256) void mm_zero32(mm_zero32_args a) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n;
         i += (uint64_t)gridDim.x * blockDim.x)
        a.dst[i] = 0u;
}

/* One wave per row: s = max|w| / 127, q = clamp(rint(w / s), -127, 127),
 * with IEEE fp32 division and round-half-even, bit-identical to the CPU
 * quantiser; s == 0 gives an all-zero row. */
extern "C" __global__ __launch_bounds__(256) void mm_quant_weight(mm_quant_w_args a) {
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int row = blockIdx.x * (blockDim.x / MM_WAVE) + threadIdx.x / MM_WAVE;
    if (row >= a.rows) return;
    const uint16_t *w = a.w + (size_t)row * a.K;
    int8_t *q = a.q + (size_t)row * a.K;
    float amax = 0.0f;
    for (int i = lane; i < a.K; i += MM_WAVE) amax = fmaxf(amax, fabsf(bf16_f32(w[i])));
    amax = wave_max(amax);
    const float s = amax / 127.0f;
    if (lane == 0) a.s[row] = s;
    for (int i = lane; i < a.K; i += MM_WAVE) {
        float v = 0.0f;
        if (s != 0.0f) v = fminf(fmaxf(rintf(bf16_f32(w[i]) / s), -127.0f), 127.0f);
        q[i] = (int8_t)(int)v;
    }
}


/* x[b] = embed[tokens[b]] widened to fp32 (src/run.c:413, the embedding of
 * forward_absorbed); a token outside [0, vocab) reads row 0.  grid (ceil(H /
 * 2048), B), 256 threads, 8 values per thread. */
extern "C" __global__ __launch_bounds__(256) void mm_embed(mm_embed_args a) {
    const int b = blockIdx.y;
    const int tok = a.tokens[b];
    const uint16_t *src = a.embed + (size_t)(tok >= 0 && tok < a.vocab ? tok : 0) * a.H;
    float *dst = a.x + (size_t)b * a.H;
    for (int i = blockIdx.x * 2048 + threadIdx.x; i < a.H && i < (int)(blockIdx.x + 1) * 2048; i += 256)
        dst[i] = bf16_f32(src[i]);
}

/* dst[j] = src[idx[j]] (rows of H floats): the rows of a step that are
 * sampled, gathered for the LM head.  grid (n), 256 threads. */
extern "C" __global__ __launch_bounds__(256) void mm_gather_rows(mm_gather_rows_args a) {
    const int j = blockIdx.x;
    const float *s = a.src + (size_t)a.idx[j] * a.H;
    float *d = a.dst + (size_t)j * a.H;
    for (int i = threadIdx.x; i < a.H; i += 256) d[i] = s[i];
}

/* h = silu(g) * u with silu(x) = x / (1 + e^-x) (src/run.c:39, 86-93). */
extern "C" __global__ __launch_bounds__(256) void mm_swiglu(mm_swiglu_args a) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n;
         i += (size_t)gridDim.x * blockDim.x) {
        const float g = a.g[i];
        a.h[i] = g / (1.0f + expf(-g)) * a.u[i];
    }
}

/* y = bf16(x) rounded to nearest even (the latent cache's element type). */
extern "C" __global__ __launch_bounds__(256) void mm_f32_bf16(mm_f32_bf16_args a) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n;
         i += (uint64_t)gridDim.x * blockDim.x)
        a.y[i] = rne16(a.x[i]);
}
