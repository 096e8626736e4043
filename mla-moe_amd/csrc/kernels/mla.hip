/* mla.hip -- MLA absorbed decode on gfx950 (src/run.c:430-460, batched).
 *
 * Per sequence b and head h, the reference computes
 *   qabs[r]  = sum_d q_nope[d] * W_UK[d, r]                    (run.c:437-442)
 *   score[k] = (qabs . c_kv[k] + q_pe . k_pe[k]) * scale        (run.c:444-451)
 *   softmax over k < kv_len                                    (run.c:452)
 *   clat[r]  = sum_k a_k * c_kv[k, r]                           (run.c:454-459)
 *   ctx      = W_UV . clat                                     (run.c:460)
 * Here the latent cache (bf16, [B, L, 576] = c_kv | k_pe) is read once per
 * sequence for all heads:
 *   mm_mla_qprep    qabs (fp32) and [qabs | q_pe] as a bf16 hi/lo pair in
 *                   MFMA operand order (x = hi + lo to ~2^-17 relative)
 *   mm_mla_attn     flash decoding over 512-key chunks: the 16 heads of a
 *                   head group are the M dimension of the MFMAs.  Per 16-key
 *                   sub-tile: S = Q . C^T on v_mfma_f32_16x16x32_bf16 (cache
 *                   rows loaded straight into B operands), online softmax in
 *                   registers, O += P . C_kv on v_mfma_f32_16x16x16bf16_1k
 *                   with the key-major B operand built by a per-wave LDS
 *                   transpose of the same cache rows.  Two waves per block,
 *                   merged in LDS into one partial per chunk.
 *   mm_mla_combine  merge the chunk partials, clat = O / l, ctx = W_UV . clat
 */
#include "common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

#define KVL MM_MLA_KVL
#define KVD MM_MLA_KVD
#define KC MM_MLA_KC
#define SUB 16                    /* keys per sub-tile */
#define CT_ROW 20                 /* u16 per transposed row: 16 keys + pad (conflict-free reads) */

__device__ __forceinline__ uint16_t bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* x ~= hi + lo: hi = rne(x), lo = rne(x - hi) (x - hi is exact in fp32). */
__device__ __forceinline__ void split_bf16(float x, uint16_t *hi, uint16_t *lo) {
    const uint16_t h = bf16_rne(x);
    *hi = h;
    *lo = bf16_rne(x - bf16_f32(h));
}

/* One wave's share of a per-head GEMM on bf16 MFMA, Y[m, n] = sum_k
 * X[m, k] W[n, k]: 32 rows of X (fp32, split into bf16 hi + lo so that the
 * products carry fp32-level precision) against 16 rows of W (bf16, K
 * contiguous).  Operand fragments come straight from memory: lane l holds
 * row (l % 16), K values 8 (l / 16) .. +7 of a 32-wide K step.  Rows of X
 * at or past mrows read row 0 (their results are not stored).  On return
 * acc[t][i] = Y[16 t + 4 (l / 16) + i][l % 16]. */
__device__ __forceinline__ void hl_gemm_32x16(const float *X, size_t xs, int mrows,
                                              const uint16_t *W, size_t ws, int k_begin, int k_end,
                                              f32x4 (&acc)[2]) {
    constexpr int GB = 4;   /* K steps whose loads are issued together */
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int r16 = lane & 15, kq = 8 * (lane >> 4);
    acc[0] = acc[1] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const float *xr[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int m = 16 * t + r16;
        xr[t] = X + (size_t)(m < mrows ? m : 0) * xs + kq;
    }
    const uint16_t *wr = W + (size_t)r16 * ws + kq;
    for (int k0 = k_begin; k0 < k_end; k0 += 32 * GB) {
        u16x8 bw[GB];
        f32x4 xv[GB][2][2];
#pragma unroll
        for (int g = 0; g < GB; g++) {
            const int k = min(k0 + 32 * g, k_end - 32);   /* steps past the end: not used */
            bw[g] = *(const u16x8 *)(wr + k);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                xv[g][t][0] = *(const f32x4 *)(xr[t] + k);
                xv[g][t][1] = *(const f32x4 *)(xr[t] + k + 4);
            }
        }
#pragma unroll
        for (int g = 0; g < GB; g++) {
            if (k0 + 32 * g >= k_end) break;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                u16x8 hi, lo;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint16_t h16, l16;
                    split_bf16(xv[g][t][j >> 2][j & 3], &h16, &l16);
                    hi[j] = h16;
                    lo[j] = l16;
                }
                const bf16x8 b8 = __builtin_bit_cast(bf16x8, bw[g]);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, hi), b8, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, lo), b8, acc[t], 0, 0, 0);
            }
        }
    }
}

/* Absorbed queries, qabs[b, h, r] = sum_d q_nope[b, h, d] W_UK_h[d, r], as a
 * per-head GEMM with W_UK_h kept transposed ([r][d], prepared at load
 * time); then the bf16 hi/lo halves of [qabs | q_pe] in MFMA A-operand
 * order for the score MFMA.  grid (KVD / 64 column slabs, HG * 16 head
 * slots, ceil(B / 32)), 4 waves of 16 columns.  The last slab is q_pe (no
 * product); head slots >= NH write zero operands so a partial head group
 * contributes nothing. */
extern "C" __global__ __launch_bounds__(256) void mm_mla_qprep(mm_mla_qprep_args a) {
    const int slab = blockIdx.x, hs = blockIdx.y, b0 = blockIdx.z * 32;
    const int hg = hs >> 4, hl = hs & 15;
    const int QKR = MM_MLA_QKR, QKN = a.QKN;
    const bool real = hs < a.NH;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int e = slab * 64 + 16 * wave + (lane & 15);     /* latent index of this lane */
    const int mrows = min(32, a.B - b0);
    f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    if (real && slab < KVL / 64)
        hl_gemm_32x16(a.q + ((size_t)b0 * a.NH + hs) * (QKN + QKR), (size_t)a.NH * (QKN + QKR), mrows,
                      a.wukT + ((size_t)hs * KVL + slab * 64 + 16 * wave) * QKN, QKN, 0, QKN, acc);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int bb = 16 * t + 4 * (lane >> 4) + i;
            if (bb >= mrows) continue;
            const int b = b0 + bb;
            float v = 0.0f;
            if (real) {
                if (e < KVL) {
                    v = acc[t][i];
                    a.qabs[((size_t)b * a.NH + hs) * KVL + e] = v;
                } else {
                    v = a.q[((size_t)b * a.NH + hs) * (QKN + QKR) + QKN + (e - KVL)];
                }
            }
            uint16_t hi, lo;
            split_bf16(v, &hi, &lo);
            uint16_t *qf = a.qfrag + (size_t)(b * a.HG + hg) * 2 * KC * 64 * 8;
            const int c = e >> 5, L = hl + 16 * ((e & 31) >> 3), j = e & 7;
            qf[((size_t)(0 * KC + c) * 64 + L) * 8 + j] = hi;
            qf[((size_t)(1 * KC + c) * 64 + L) * 8 + j] = lo;
        }
}

/* Load-time: W_UK_h transposed, wukT[h][r][d] = kv_b[h (QKN + VHD) + d][r]. */
extern "C" __global__ __launch_bounds__(256) void mm_mla_wprep(mm_mla_wprep_args a) {
    const size_t n = (size_t)a.NH * KVL * a.QKN;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t d = i % a.QKN, r = (i / a.QKN) % KVL, h = i / ((size_t)a.QKN * KVL);
        a.wukT[i] = a.kv_b[(h * (a.QKN + a.VHD) + d) * KVL + r];
    }
}

__device__ __forceinline__ float grp16_max(float v) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, MM_WAVE));
    return v;
}
__device__ __forceinline__ float grp16_sum(float v) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, MM_WAVE);
    return v;
}

/* grid (nchunks, B, HG), 128 threads (2 waves); wave w handles keys
 * [chunk*512 + w*256, +256). */
extern "C" __global__ __launch_bounds__(128) void mm_mla_attn(mm_mla_attn_args a) {
    __shared__ __attribute__((aligned(16))) uint16_t qlds[2 * KC * 64 * 8];          /* 36 KB */
    __shared__ __attribute__((aligned(16))) uint16_t ctlds[2][KVL * CT_ROW];        /* 40 KB */
    __shared__ __attribute__((aligned(16))) uint16_t plds[2][2][16 * 16];           /* 2 KB */
    __shared__ float mlds[2][32];

    const int chunk = blockIdx.x, b = blockIdx.y, hg = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, kl = lane & 15;
    const int L = a.kv_lens ? min(a.kv_lens[b], a.kv_len) : a.kv_len;

    {   /* Q operands for this (b, head group) into LDS */
        const u16x8 *src = (const u16x8 *)(a.qfrag + (size_t)(b * a.HG + hg) * 2 * KC * 64 * 8);
        u16x8 *dst = (u16x8 *)qlds;
        for (int i = tid; i < 2 * KC * 64; i += 128) dst[i] = src[i];
    }
    __syncthreads();

    float m[4], l[4];
    f32x4 O[KVL / 16];
#pragma unroll
    for (int i = 0; i < 4; i++) { m[i] = -INFINITY; l[i] = 0.0f; }
#pragma unroll
    for (int nb = 0; nb < KVL / 16; nb++) O[nb] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    uint16_t *ct = ctlds[w];
    const int kbeg = chunk * MM_MLA_CHUNK + w * (MM_MLA_CHUNK / 2);
    const int kend = min(kbeg + MM_MLA_CHUNK / 2, L);
    const uint16_t *cseq = a.cache + (size_t)b * a.seq_stride * KVD;
    for (int k0 = kbeg; k0 < kend; k0 += SUB) {
        const int key = k0 + kl;
        const bool valid = key < L;
        const uint16_t *rp = cseq + (size_t)(valid ? key : k0) * KVD + 8 * g;
        bf16x8 bfr[KC];
#pragma unroll
        for (int c = 0; c < KC; c++) {
            u16x8 v = *(const u16x8 *)(rp + 32 * c);
            if (!valid) v = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
            bfr[c] = __builtin_bit_cast(bf16x8, v);
        }
        /* S[head 4g+i][key kl] */
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const bf16x8 qh = __builtin_bit_cast(bf16x8, *(const u16x8 *)&qlds[((0 * KC + c) * 64 + lane) * 8]);
            const bf16x8 ql = __builtin_bit_cast(bf16x8, *(const u16x8 *)&qlds[((1 * KC + c) * 64 + lane) * 8]);
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh, bfr[c], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql, bfr[c], s, 0, 0, 0);
        }
        float p[4], cr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float sv = valid ? s[i] * a.scale : -INFINITY;
            const int head = hg * 16 + 4 * g + i;
            if (a.scores && valid && head < a.NH)
                a.scores[((size_t)b * a.NH + head) * a.probs_stride + key] = sv;
            const float mnew = fmaxf(m[i], grp16_max(sv));
            cr[i] = m[i] == -INFINITY ? 0.0f : __expf(m[i] - mnew);
            p[i] = sv == -INFINITY ? 0.0f : __expf(sv - mnew);
            l[i] = l[i] * cr[i] + grp16_sum(p[i]);
            m[i] = mnew;
        }
#pragma unroll
        for (int nb = 0; nb < KVL / 16; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++) O[nb][i] *= cr[i];
        /* P (hi/lo) as [head][key]; the sub-tile's c_kv transposed [r][key] */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint16_t hi, lo;
            split_bf16(p[i], &hi, &lo);
            plds[w][0][(4 * g + i) * 16 + kl] = hi;
            plds[w][1][(4 * g + i) * 16 + kl] = lo;
        }
#pragma unroll
        for (int c = 0; c < KVL / 32; c++) {
            const u16x8 v = __builtin_bit_cast(u16x8, bfr[c]);
#pragma unroll
            for (int j = 0; j < 8; j++) ct[(32 * c + 8 * g + j) * CT_ROW + kl] = v[j];
        }
        /* O[head][r] += P[head][keys] . C[keys][r]  (K = 16 keys, 4 per lane) */
        const s16x4 ph = *(const s16x4 *)&plds[w][0][kl * 16 + 4 * g];
        const s16x4 pl = *(const s16x4 *)&plds[w][1][kl * 16 + 4 * g];
#pragma unroll
        for (int nb = 0; nb < KVL / 16; nb++) {
            const s16x4 bv = *(const s16x4 *)&ct[(nb * 16 + kl) * CT_ROW + 4 * g];
            O[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ph, bv, O[nb], 0, 0, 0);
            O[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pl, bv, O[nb], 0, 0, 0);
        }
    }

    /* merge the two waves: wave 1 parks its state in LDS, wave 0 merges */
    __syncthreads();
    float *ob = (float *)ctlds;   /* 16 x 512 fp32 = 32 KB fits in the 40 KB transpose area */
    if (w == 1) {
#pragma unroll
        for (int nb = 0; nb < KVL / 16; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++) ob[(4 * g + i) * KVL + nb * 16 + kl] = O[nb][i];
        if (kl == 0)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                mlds[0][4 * g + i] = m[i];
                mlds[1][4 * g + i] = l[i];
            }
    }
    __syncthreads();
    if (w == 0) {
        const size_t pidx = ((size_t)(b * a.HG + hg) * a.nchunks + chunk);
        float *po = a.part_o + pidx * 16 * KVL;
        float w0[4], w1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int hrow = 4 * g + i;
            const float m1 = mlds[0][hrow], l1 = mlds[1][hrow];
            const float mm = fmaxf(m[i], m1);
            w0[i] = m[i] == -INFINITY ? 0.0f : __expf(m[i] - mm);
            w1[i] = m1 == -INFINITY ? 0.0f : __expf(m1 - mm);
            if (kl == 0) {
                a.part_ml[pidx * 32 + hrow] = mm;
                a.part_ml[pidx * 32 + 16 + hrow] = l[i] * w0[i] + l1 * w1[i];
            }
        }
#pragma unroll
        for (int nb = 0; nb < KVL / 16; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int idx = (4 * g + i) * KVL + nb * 16 + kl;
                po[idx] = O[nb][i] * w0[i] + ob[idx] * w1[i];
            }
    }
}

/* Merge the chunk partials of (head h, sequence b): clat = sum_c w_c O_c / l
 * with w_c = e^(m_c - m); also turns the debug scores into probabilities.
 * grid (NH, B), 256 threads. */
extern "C" __global__ __launch_bounds__(256) void mm_mla_combine(mm_mla_combine_args a) {
    __shared__ float wch[64];
    __shared__ float stat[2];
    const int h = blockIdx.x, b = blockIdx.y;
    const int hg = h >> 4, hl = h & 15;
    const int tid = threadIdx.x;
    const int L = a.kv_lens ? min(a.kv_lens[b], a.kv_len) : a.kv_len;
    const size_t pbase = (size_t)(b * a.HG + hg) * a.nchunks;
    if (tid < MM_WAVE) {
        /* chunk maxima and sums, one lane per chunk (nchunks <= 64) */
        const bool ok = tid < a.nchunks;
        const float mc = ok ? a.part_ml[(pbase + tid) * 32 + hl] : -INFINITY;
        const float lc = ok ? a.part_ml[(pbase + tid) * 32 + 16 + hl] : 0.0f;
        const float mx = wave_max(mc);
        const float wc = mc == -INFINITY ? 0.0f : __expf(mc - mx);
        const float ls = wave_sum(lc * wc);
        if (ok) wch[tid] = wc;
        if (tid == 0) {
            stat[0] = mx;
            stat[1] = ls;
        }
    }
    __syncthreads();
    const float mx = stat[0], inv = 1.0f / stat[1];
    float *cl = a.clat + ((size_t)b * a.NH + h) * KVL;
    for (int r = tid; r < KVL; r += blockDim.x) {
        float o = 0.0f;
        for (int c = 0; c < a.nchunks; c++)
            o += wch[c] * a.part_o[((pbase + c) * 16 + hl) * KVL + r];
        cl[r] = o * inv;
    }
    if (a.probs) {
        float *pr = a.probs + ((size_t)b * a.NH + h) * a.probs_stride;
        for (int k = tid; k < L; k += blockDim.x) pr[k] = __expf(pr[k] - mx) * inv;
    }
}

/* ctx[b, h, v] = sum_r W_UV_h[v, r] clat[b, h, r], a per-head GEMM on bf16
 * MFMA (clat split hi/lo).  grid (ceil(VHD / 16), NH, ceil(B / 32)), 4 waves
 * splitting K = KVL; the partial sums meet in LDS. */
extern "C" __global__ __launch_bounds__(256) void mm_mla_uv(mm_mla_combine_args a) {
    __shared__ f32x4 red[3][2][MM_WAVE];
    const int vw = blockIdx.x * 16, h = blockIdx.y, b0 = blockIdx.z * 32;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int mrows = min(32, a.B - b0);
    const int nv = min(16, a.VHD - vw);
    const uint16_t *wuv = a.kv_b + ((size_t)h * (a.QKN + a.VHD) + a.QKN + vw) * KVL;
    f32x4 acc[2];
    /* rows of W_UV past VHD: read row vw instead (results not stored) */
    hl_gemm_32x16(a.clat + ((size_t)b0 * a.NH + h) * KVL, (size_t)a.NH * KVL, mrows,
                  (lane & 15) < nv ? wuv : wuv - (size_t)(lane & 15) * KVL, KVL,
                  wave * (KVL / 4), (wave + 1) * (KVL / 4), acc);
    if (wave > 0) {
        red[wave - 1][0][lane] = acc[0];
        red[wave - 1][1][lane] = acc[1];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < 3; w++) {
        acc[0] += red[w][0][lane];
        acc[1] += red[w][1][lane];
    }
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int bb = 16 * t + 4 * (lane >> 4) + i;
            if (bb < mrows && (lane & 15) < nv)
                a.ctx[((size_t)(b0 + bb) * a.NH + h) * a.VHD + vw + (lane & 15)] = acc[t][i];
        }
}
