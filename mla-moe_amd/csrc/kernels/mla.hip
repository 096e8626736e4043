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
 *   mm_mla_qprep    qabs (fp32), a per-head GEMM on bf16 MFMA; q is split
 *                   into bf16 hi + lo halves (x = hi + lo to ~2^-17 relative)
 *                   wherever an fp32 operand meets a bf16 MFMA
 *   mm_mla_attn     flash decoding over 512-key chunks, all 16 heads of a
 *                   head group per MFMA (see the kernel)
 *   mm_mla_combine  merge the chunk partials, clat = O / l
 *   mm_mla_uv       ctx = W_UV . clat
 */
#include "common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

#define KVL MM_MLA_KVL
#define KVD MM_MLA_KVD
#define KC MM_MLA_KC

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

/* hl_gemm_32x16 for S column tiles at once (large batches): lane l's W
 * row of tile s starts at wr[s] (row l % 16 of the tile, chosen by the
 * caller); each K step's X fragments are loaded and split into hi + lo once
 * for the S tiles, so a wave reads its 32 rows of X once per S x 16 columns.
 * On return acc[s][t][i] = Y[16 t + 4 (l / 16) + i][tile s, column l % 16]. */
template <int S>
__device__ __forceinline__ void hl_gemm_32x16s(const float *X, size_t xs, int mrows,
                                               const uint16_t *const (&wr)[S], int k_begin,
                                               int k_end, f32x4 (&acc)[S][2]) {
    constexpr int GB = S >= 4 ? 2 : 4;   /* K steps whose loads are issued together */
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int r16 = lane & 15, kq = 8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < S; s++) acc[s][0] = acc[s][1] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const float *xr[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int m = 16 * t + r16;
        xr[t] = X + (size_t)(m < mrows ? m : 0) * xs + kq;
    }
    for (int k0 = k_begin; k0 < k_end; k0 += 32 * GB) {
        u16x8 bw[GB][S];
        f32x4 xv[GB][2][2];
#pragma unroll
        for (int g = 0; g < GB; g++) {
            const int k = min(k0 + 32 * g, k_end - 32);   /* steps past the end: not used */
#pragma unroll
            for (int s = 0; s < S; s++) bw[g][s] = *(const u16x8 *)(wr[s] + kq + k);
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
#pragma unroll
                for (int s = 0; s < S; s++) {
                    const bf16x8 b8 = __builtin_bit_cast(bf16x8, bw[g][s]);
                    acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, hi), b8, acc[s][t], 0, 0, 0);
                    acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, lo), b8, acc[s][t], 0, 0, 0);
                }
            }
        }
    }
}

/* Absorbed queries, qabs[b, h, r] = sum_d q_nope[b, h, d] W_UK_h[d, r], as a
 * per-head GEMM with W_UK_h kept transposed ([r][d], prepared at load
 * time), also written split into bf16 hi + lo (the attention's Q operands,
 * split once here rather than by each of its waves).  grid (KVL / 64
 * column slabs, NH, ceil(B / 32)), 4 waves of 16 columns. */
__device__ __forceinline__ void qprep_block(const mm_mla_qprep_args &a, int slab, int h, int b0) {
    const int QKR = MM_MLA_QKR, QKN = a.QKN;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int e = slab * 64 + 16 * wave + (lane & 15);     /* latent index of this lane */
    const int mrows = min(32, a.B - b0);
    f32x4 acc[2];
    hl_gemm_32x16(a.q + ((size_t)b0 * a.NH + h) * (QKN + QKR), (size_t)a.NH * (QKN + QKR), mrows,
                  a.wukT + ((size_t)h * KVL + slab * 64 + 16 * wave) * QKN, QKN, 0, QKN, acc);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int bb = 16 * t + 4 * (lane >> 4) + i;
            if (bb < mrows) {
                const size_t row = (size_t)(b0 + bb) * a.NH + h;
                uint16_t hi, lo;
                split_bf16(acc[t][i], &hi, &lo);
                if (a.qabs) a.qabs[row * KVL + e] = acc[t][i];
                a.qhl[row * 2 * KVL + e] = hi;
                a.qhl[(row * 2 + 1) * KVL + e] = lo;
            }
        }
}

extern "C" __global__ __launch_bounds__(256) void mm_mla_qprep(mm_mla_qprep_args a) {
    qprep_block(a, blockIdx.x, blockIdx.y, blockIdx.z * 32);
}

/* mm_mla_qprep for large batches (a prefill's rows): grid (KVL / (64 S),
 * NH, ceil(B / 32)), wave w taking columns (slab S + s) 64 + 16 w .. +15 of
 * each tile s < S -- the 32 rows of q are read and split once per S tiles
 * instead of once per tile. */
static_assert(KVL % (64 * MM_MLA_WIDE_S) == 0, "qprep column slabs");
extern "C" __global__ __launch_bounds__(256) void mm_mla_qprep_w(mm_mla_qprep_args a) {
    constexpr int S = MM_MLA_WIDE_S;
    const int slab = blockIdx.x, h = blockIdx.y, b0 = blockIdx.z * 32;
    const int QKR = MM_MLA_QKR, QKN = a.QKN;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int mrows = min(32, a.B - b0);
    const uint16_t *wr[S];
#pragma unroll
    for (int s = 0; s < S; s++)
        wr[s] = a.wukT + ((size_t)h * KVL + (slab * S + s) * 64 + 16 * wave + (lane & 15)) * QKN;
    f32x4 acc[S][2];
    hl_gemm_32x16s<S>(a.q + ((size_t)b0 * a.NH + h) * (QKN + QKR), (size_t)a.NH * (QKN + QKR), mrows,
                      wr, 0, QKN, acc);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int e = (slab * S + s) * 64 + 16 * wave + (lane & 15);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int bb = 16 * t + 4 * (lane >> 4) + i;
                if (bb < mrows) {
                    const size_t row = (size_t)(b0 + bb) * a.NH + h;
                    uint16_t hi, lo;
                    split_bf16(acc[s][t][i], &hi, &lo);
                    if (a.qabs) a.qabs[row * KVL + e] = acc[s][t][i];
                    a.qhl[row * 2 * KVL + e] = hi;
                    a.qhl[(row * 2 + 1) * KVL + e] = lo;
                }
            }
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

/* Transposing LDS read (ds_read_b64_tr_b16) at addr + off (off a constant
 * after unrolling) as inline assembly (the compiler does not track it;
 * callers wait with lgkmcnt): within each
 * 16-lane group, lane 4k + c supplies the address of 4 consecutive 16-bit
 * values of row k (k, c = 0..3); lane i receives column i of the 4 rows,
 * i.e. a row-major [4][16] block read as the B operand of
 * v_mfma_f32_16x16x16bf16_1k. */
__device__ __forceinline__ s16x4 ds_read_tr16(uint32_t addr, int off) {
    s16x4 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off));
    return r;
}

#define AW MM_MLA_AW               /* waves per attention block */
#define CROW_B 1056               /* bytes per LDS c_kv row: 1024 + 32 pad */
#define TILE_B (16 * CROW_B + 16 * 128)   /* 16 keys: c_kv rows, then the k_pe parts */
static_assert(TILE_B == MM_MLA_TILE_B, "sub-tile size");
#define OROW (KVL + 4)            /* floats per head row of the merge buffer */
/* Rescaling is lazy: a head's running maximum m moves only when a score
 * exceeds it by more than RESCALE_TAU, so exp(s - m) <= e^RESCALE_TAU and the
 * accumulator is rescaled on few sub-tiles.  The final O / l is the same
 * quantity for any m. */
#define RESCALE_TAU 8.0f
static_assert((AW * 16 * OROW + AW * 32 + 16) * 4 <= AW * 2 * TILE_B, "merge buffer exceeds the staging LDS");
static_assert((16 * KVL) % (4 * AW * MM_WAVE) == 0, "merge loop");

/* A operand of the score product: cache row kl of the sub-tile at LDS
 * address t, latent 32 c + 8 g .. +7 (c_kv, then the k_pe part) */
__device__ __forceinline__ i32x4 mla_read_a(uint32_t t, int c, int kl, int g) {
    return c < KVL / 32 ? ds_read16(t + kl * CROW_B + 16 * g, 64 * c)
                        : ds_read16(t + 16 * CROW_B + kl * 128 + 16 * g, 64 * (c - KVL / 32));
}

/* S^T[key 4g+i][head kl] for the sub-tile at LDS address t: A = cache
 * row kl, latent 32 c + 8 g .. +7; LDS reads run one batch of 6 ahead of
 * the MFMAs.  Returns the scaled scores, -inf past kend. */
__device__ __forceinline__ void mla_score(const mm_mla_attn_args &a, uint32_t t, int k0, int kend, int b,
                                          int hg, int kl, int g, const bf16x8 (&qh)[KC],
                                          const bf16x8 (&ql)[KC], float *sv) {
    /* the hi and lo products in two independent MFMA chains (one chain
     * of 36 dependent MFMAs waits out each one's latency), added at the
     * end */
    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f}, s2 = {0.0f, 0.0f, 0.0f, 0.0f};
    i32x4 af[2][6];
#pragma unroll
    for (int c = 0; c < 6; c++) af[0][c] = mla_read_a(t, c, kl, g);
#pragma unroll
    for (int bt = 0; bt < KC / 6; bt++) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[bt & 1][0]), "+v"(af[bt & 1][1]), "+v"(af[bt & 1][2]),
                     "+v"(af[bt & 1][3]), "+v"(af[bt & 1][4]), "+v"(af[bt & 1][5]));
        if (bt + 1 < KC / 6) {
#pragma unroll
            for (int c = 0; c < 6; c++) af[(bt + 1) & 1][c] = mla_read_a(t, 6 * (bt + 1) + c, kl, g);
        }
#pragma unroll
        for (int c = 0; c < 6; c++) {
            const bf16x8 ab = __builtin_bit_cast(bf16x8, af[bt & 1][c]);
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, qh[6 * bt + c], s, 0, 0, 0);
            s2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, ql[6 * bt + c], s2, 0, 0, 0);
        }
    }
    s += s2;
    const int head = hg * 16 + kl;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int key = k0 + 4 * g + i;
        sv[i] = key < kend ? s[i] * a.scale : -INFINITY;
        if (a.scores && key < kend && head < a.NH)
            a.scores[((size_t)b * a.NH + head) * a.probs_stride + key] = sv[i];
    }
}

/* P = e^(s - m) into the sums and O[head][r] += P . C_kv.  P[head kl][keys
 * 4g .. 4g+3] is a bf16 hi/lo pair of A operands; the B operands come by
 * transposing reads (lane 4k + c of group g reads row 4g + k, columns
 * 16 nb + 4c .. +3), one batch of 8 ahead of the MFMAs. */
__device__ __forceinline__ void mla_accumulate(uint32_t t, const float *sv, float m, float &l,
                                               f32x4 (&O)[KVL / 16], int kl, int g) {
    const uint32_t tb = t + (4 * g + (kl >> 2)) * CROW_B + 8 * (kl & 3);
    s16x4 bv[2][8];
#pragma unroll
    for (int j = 0; j < 8; j++) bv[0][j] = ds_read_tr16(tb, 32 * j);
    s16x4 ph, pl;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float p = sv[i] == -INFINITY ? 0.0f : __expf(sv[i] - m);
        l += p;
        uint16_t hi, lo;
        split_bf16(p, &hi, &lo);
        ph[i] = (short)hi;
        pl[i] = (short)lo;
    }
    const bf16x8 pa = __builtin_bit_cast(bf16x8, (s16x8){ph[0], ph[1], ph[2], ph[3], pl[0], pl[1], pl[2], pl[3]});
#pragma unroll
    for (int bt = 0; bt < KVL / 128; bt++) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(bv[bt & 1][0]), "+v"(bv[bt & 1][1]), "+v"(bv[bt & 1][2]), "+v"(bv[bt & 1][3]),
                       "+v"(bv[bt & 1][4]), "+v"(bv[bt & 1][5]), "+v"(bv[bt & 1][6]), "+v"(bv[bt & 1][7]));
        if (bt + 1 < KVL / 128) {
#pragma unroll
            for (int j = 0; j < 8; j++) bv[(bt + 1) & 1][j] = ds_read_tr16(tb, 32 * (8 * (bt + 1) + j));
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int nb = 8 * bt + j;
            /* K = 32 as (key 4g + i, hi) at 8g + i and (key 4g + i, lo)
             * at 8g + 4 + i: the hi and lo products in one MFMA */
            const s16x4 c = bv[bt & 1][j];
            const bf16x8 bb = __builtin_bit_cast(bf16x8, (s16x8){c[0], c[1], c[2], c[3], c[0], c[1], c[2], c[3]});
            O[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, bb, O[nb], 0, 0, 0);
        }
    }
}

/* one block per (row b, head group hg, chunk) triple (the 1-D grid and its
 * XCD-grouped order: mm_mla_attn_args), AW waves; row b attends to the first kv_lens[b]
 * rows of cache sequence slots[b] (b without slots); with KPW = a.chunk / AW
 * keys per wave,
 * wave w handles keys [chunk * a.chunk + w * KPW, + KPW) in 16-key
 * sub-tiles, each staged into LDS by direct global -> LDS
 * loads one sub-tile ahead of its use (two LDS stages per wave):
 *   S^T[key][head] = C[key] . Q[head]^T on v_mfma_f32_16x16x32_bf16 with the
 *     cache rows as the A operand and Q (hi and lo halves, in registers) as
 *     B, so lane (head = l % 16, l / 16) holds the scores of keys
 *     4 (l / 16) .. +3;
 *   online softmax per head with lazy rescaling; the sums l stay per lane
 *     (4 keys each) until the merge;
 *   P[head][keys] is then already in A-operand order for
 *   O[head][r] += P . C_kv on v_mfma_f32_16x16x16bf16_1k, whose B operand
 *   ([keys][r] row-major) comes from the same LDS rows by transposing reads.
 * The AW waves' partial states merge in LDS into one partial per chunk.
 * Dynamic LDS: AW * 2 * TILE_B bytes (the merge reuses it). */
extern "C" __global__ __launch_bounds__(AW * MM_WAVE) void mm_mla_attn(mm_mla_attn_args a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t alds[];
    /* XCD-grouped order for rows of one length; rows of their own lengths
     * (kv_lens) last row first, in index order over the XCDs in turn, so
     * that long and short rows spread over the XCDs and a prefill's longest
     * rows start first */
    const int ntrip = a.B * a.HG * a.nchunks, per = (ntrip + 7) / 8;
    const int trip = a.kv_lens ? ntrip - 1 - (int)blockIdx.x
                               : (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (trip < 0 || trip >= ntrip) return;   /* the grid is rounded up to 8 blocks */
    const int chunk = trip % a.nchunks, hg = (trip / a.nchunks) % a.HG, b = trip / (a.nchunks * a.HG);
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, kl = lane & 15;
    const int L = a.kv_lens ? min(a.kv_lens[b], a.kv_len) : a.kv_len;
    /* stage st of wave w at (st AW + w) TILE_B: the second stages of all
     * waves are one region, which holds the block's Q before their loads */
    auto stage = [&](int st) { return alds + (size_t)(st * AW + w) * TILE_B; };

    const int kpw = a.chunk / AW;                     /* keys per wave */
    const int kbeg = chunk * a.chunk + w * kpw;
    const int kend = min(kbeg + kpw, L);
    const int seq = a.slots ? a.slots[b] : b;
    const uint8_t *cseq = (const uint8_t *)(a.cache + (size_t)seq * a.seq_stride * KVD);
    /* sub-tile at key k0 -> stage st: row p's c_kv (1 KB, one load per lane
     * of 16 B) at p * CROW_B; the k_pe parts (128 B per row) of rows 0..7 and
     * 8..15 as two 1 KB pieces after the c_kv rows.  Rows past L load row
     * L - 1 (masked in the softmax; row 0 when L = 0). */
    const int klast = max(L - 1, 0);
#define ISSUE_LOADS 18            /* direct loads per issue(): 16 c_kv rows + 2 k_pe pieces */
    auto issue = [&](int st, int k0) {
        uint8_t *t = stage(st);
#pragma unroll
        for (int p = 0; p < 16; p++) {
            const int key = __builtin_amdgcn_readfirstlane(min(k0 + p, klast));
            lds_dma16(cseq + (uint32_t)(key * KVD * 2) + lane * 16, t + p * CROW_B);
        }
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const int key = min(k0 + 8 * p + (lane >> 3), klast);
            lds_dma16(cseq + (uint32_t)(key * KVD * 2 + KVL * 2 + (lane & 7) * 16),
                      t + 16 * CROW_B + p * 1024);
        }
    };
    /* both stages from the start: the first two sub-tiles' loads are in
     * flight while Q is prepared, and each later sub-tile is issued one
     * sub-tile of compute before its use.  The Q loads go out first: the
     * counter completes in issue order, and behind both sub-tiles (every
     * wave of the launch asking for its first two at once) Q arrived ~8 us
     * after the block's start, ~5 us after the first sub-tile. */

    /* Q operands in registers: lane (head kl, g) holds [qabs | q_pe] of its
     * head, latent 32 c + 8 g .. +7, as bf16 hi + lo; head slots past NH are
     * zero.  qabs comes split by qprep (splitting all 16 heads' 576 values
     * in every wave cost ~3-4 us of VALU per block); the 64 q_pe values
     * are split here, after the cache loads are issued. */
    bf16x8 qh[KC], ql[KC];
    f32x4 qpe[KC - KVL / 32][2];
    static_assert(KC - KVL / 32 == 2, "q_pe: two 32-value K steps");
    const bool qreal = hg * 16 + kl < a.NH;
    /* qabs (hi and lo rows of the group's 16 heads, 32 KB) is staged once
     * per block in the second-stage region, each wave loading 8 of its 32
     * 1 KB rows (head h, half p at h QROW_B + 1024 p: the 16-byte pad
     * between heads puts the 16 heads of a ds_read_b128 on distinct banks);
     * every wave then reads all of it into registers.  Loaded per wave
     * from global memory, the same 36 KB went out 32 times per row (4
     * waves x 8 chunks) in 64-byte pieces and took ~5 us to arrive. */
    constexpr int QROW_B = 2 * KVL * 2 + 16;
    static_assert(16 * QROW_B <= AW * TILE_B, "Q staging exceeds the second stages");
    uint8_t *qlds = alds + (size_t)AW * TILE_B;
    {
        /* q_pe per wave as assembly loads (after a direct-to-LDS load the
         * compiler waits for every load in flight at the first use of a
         * loaded register; these waits are counted by hand below) */
        const int qhd = qreal ? hg * 16 + kl : 0;
        const float *qp = a.q + ((size_t)b * a.NH + qhd) * (a.QKN + MM_MLA_QKR) + a.QKN + 8 * g;
#pragma unroll
        for (int c = 0; c < KC - KVL / 32; c++) {
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(qpe[c][0]) : "v"(qp), "i"(128 * c));
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(qpe[c][1]) : "v"(qp), "i"(128 * c + 16));
        }
        static_assert(AW == 4, "8 qabs rows per wave");
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int row = 8 * w + j, h = row >> 1, p = row & 1;
            const int qhd2 = hg * 16 + h < a.NH ? hg * 16 + h : 0;   /* head slots past NH: zeroed below */
            lds_dma16(a.qhl + (((size_t)b * a.NH + qhd2) * 2 + p) * KVL + 8 * lane, qlds + h * QROW_B + p * 1024);
        }
    }
    /* the first stage, then the wait for Q, then the second stage (into
     * the region Q leaves): Q meets one stage's loads of every wave.  Both
     * stages whatever the wave's key count (clamped rows of its own LDS,
     * waited for before the merge), so that the counts hold */
    __builtin_amdgcn_sched_barrier(0);
    issue(0, kbeg);
    __builtin_amdgcn_sched_barrier(0);
    /* this wave's part of Q has landed once at most the first stage's
     * loads are outstanding; the barrier waits for the other waves' parts */
    static_assert(ISSUE_LOADS == 18, "wait count");
    asm volatile("s_waitcnt vmcnt(18)" : "+v"(qpe[0][0]), "+v"(qpe[0][1]), "+v"(qpe[1][0]), "+v"(qpe[1][1]));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    {
        const uint32_t qa = lds_addr(qlds) + (uint32_t)(kl * QROW_B + 16 * g);
#pragma unroll
        for (int c = 0; c < KVL / 32; c++) {
            qh[c] = __builtin_bit_cast(bf16x8, ds_read16(qa, 64 * c));
            ql[c] = __builtin_bit_cast(bf16x8, ds_read16(qa, 1024 + 64 * c));
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(qh[0]), "+v"(qh[1]), "+v"(qh[2]), "+v"(qh[3]), "+v"(qh[4]), "+v"(qh[5]), "+v"(qh[6]),
                   "+v"(qh[7]), "+v"(qh[8]), "+v"(qh[9]), "+v"(qh[10]), "+v"(qh[11]), "+v"(qh[12]), "+v"(qh[13]),
                   "+v"(qh[14]), "+v"(qh[15]));
    asm volatile(""
                 : "+v"(ql[0]), "+v"(ql[1]), "+v"(ql[2]), "+v"(ql[3]), "+v"(ql[4]), "+v"(ql[5]), "+v"(ql[6]),
                   "+v"(ql[7]), "+v"(ql[8]), "+v"(ql[9]), "+v"(ql[10]), "+v"(ql[11]), "+v"(ql[12]), "+v"(ql[13]),
                   "+v"(ql[14]), "+v"(ql[15]));
    /* every wave has read Q: the region takes the second stages */
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(1, kbeg + 16);
    __builtin_amdgcn_sched_barrier(0);
    {
        const bf16x8 z8 = __builtin_bit_cast(bf16x8, (u16x8){});
#pragma unroll
        for (int c = 0; c < KVL / 32; c++) {
            qh[c] = qreal ? qh[c] : z8;
            ql[c] = qreal ? ql[c] : z8;
        }
#pragma unroll
        for (int c = KVL / 32; c < KC; c++) {
            const f32x4 x0 = qpe[c - KVL / 32][0], x1 = qpe[c - KVL / 32][1];
            u16x8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint16_t h16, l16;
                split_bf16(qreal ? (j < 4 ? x0[j & 3] : x1[j & 3]) : 0.0f, &h16, &l16);
                hi[j] = h16;
                lo[j] = l16;
            }
            qh[c] = __builtin_bit_cast(bf16x8, hi);
            ql[c] = __builtin_bit_cast(bf16x8, lo);
        }
    }

    float m = -INFINITY, l = 0.0f;        /* head kl: running max; this lane's share of the sum */
    f32x4 O[KVL / 16];
#pragma unroll
    for (int nb = 0; nb < KVL / 16; nb++) O[nb] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    /* The inner loop touches O only through MFMAs (it stays in accumulation
     * registers); a sub-tile that needs a rescale leaves it, and the outer
     * loop rescales and accumulates that sub-tile. */
    int k0 = kbeg, st = 0;
    while (k0 < kend) {
        float sv[4];
        bool moved = false;
        for (;;) {
            /* this sub-tile's rows are in LDS: the loads of the next one
             * (ISSUE_LOADS, issued later) may stay outstanding, as may
             * nothing else (the score stores of the previous sub-tile were
             * issued before them) */
            if (k0 + 16 < kend) VMCNT_WAIT(ISSUE_LOADS);
            else VMCNT_WAIT(0);
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t t = lds_addr(stage(st));
            mla_score(a, t, k0, kend, b, hg, kl, g, qh, ql, sv);
            const float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            if (__builtin_amdgcn_ballot_w64(mx > m + RESCALE_TAU)) {
                moved = true;
                break;
            }
            mla_accumulate(t, sv, m, l, O, kl, g);
            __builtin_amdgcn_sched_barrier(0);
            /* this stage's LDS reads are complete (accumulate waits for them
             * before its last MFMAs): refill it with the sub-tile after next */
            if (k0 + 32 < kend) issue(st, k0 + 32);
            __builtin_amdgcn_sched_barrier(0);
            k0 += 16;
            st ^= 1;
            if (k0 >= kend) break;
        }
        if (!moved) break;
        /* some head's maximum moved: new m = the head's max over the
         * sub-tile (across the 4 lane groups) */
        float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, MM_WAVE));
        mx = fmaxf(mx, __shfl_xor(mx, 32, MM_WAVE));
        const float mnew = fmaxf(m, mx);
        /* m is uniform over the wave's lanes of a head, and -inf for every
         * head until the wave's first sub-tile: O and l are still zero then
         * and need no rescale */
        if (__builtin_amdgcn_ballot_w64(m != -INFINITY)) {
            const float cr = m == -INFINITY ? 0.0f : __expf(m - mnew);
            l *= cr;
            /* rescale O rows: lane (r, g) holds heads 4g + i, whose factor
             * sits in lane 4g + i */
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float ci = __shfl(cr, 4 * g + i, MM_WAVE);
#pragma unroll
                for (int nb = 0; nb < KVL / 16; nb++) O[nb][i] *= ci;
            }
        }
        m = mnew;
        mla_accumulate(lds_addr(stage(st)), sv, m, l, O, kl, g);
        __builtin_amdgcn_sched_barrier(0);
        if (k0 + 32 < kend) issue(st, k0 + 32);
        __builtin_amdgcn_sched_barrier(0);
        k0 += 16;
        st ^= 1;
    }
    VMCNT_WAIT(0);

    /* merge the waves (LDS of the stages is free after the barrier):
     * per head, mm = max over waves of m, each wave's weight e^(m_w - mm);
     * every wave parks its weighted O; all threads then sum the AW parts */
    l += __shfl_xor(l, 16, MM_WAVE);
    l += __shfl_xor(l, 32, MM_WAVE);
    __syncthreads();
    float *ob = (float *)alds;                       /* [AW][16 heads][OROW] */
    float *mlb = ob + AW * 16 * OROW;                /* [AW][2][16] */
    if (g == 0) {
        mlb[w * 32 + kl] = m;
        mlb[w * 32 + 16 + kl] = l;
    }
    __syncthreads();
    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < AW; j++) mm = fmaxf(mm, mlb[j * 32 + kl]);
    const float wself = m == -INFINITY ? 0.0f : __expf(m - mm);
    {
        float *o = ob + (size_t)w * 16 * OROW;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float wi = __shfl(wself, 4 * g + i, MM_WAVE);
#pragma unroll
            for (int nb = 0; nb < KVL / 16; nb++) o[(4 * g + i) * OROW + nb * 16 + kl] = O[nb][i] * wi;
        }
    }
    const size_t pidx = ((size_t)(b * a.HG + hg) * a.nchunks + chunk);
    float *linv = mlb + AW * 32;                     /* [16]: one chunk, 1 / l per head */
    if (w == 0 && g == 0) {
        float lsum = 0.0f;
#pragma unroll
        for (int j = 0; j < AW; j++) {
            const float mj = mlb[j * 32 + kl];
            lsum += mj == -INFINITY ? 0.0f : mlb[j * 32 + 16 + kl] * __expf(mj - mm);
        }
        if (a.clat) {
            linv[kl] = 1.0f / lsum;
        } else {
            a.part_ml[pidx * 32 + kl] = mm;
            a.part_ml[pidx * 32 + 16 + kl] = lsum;
        }
    }
    __syncthreads();
    if (a.clat) {   /* the whole context in this block: clat = O (1 / l), the merge's values */
#pragma unroll
        for (int j = 0; j < 16 * KVL / (4 * AW * MM_WAVE); j++) {
            const int e = 4 * (tid + j * AW * MM_WAVE);
            const int hh = e / KVL, col = e % KVL;
            f32x4 v = *(const f32x4 *)(ob + hh * OROW + col);
#pragma unroll
            for (int k = 1; k < AW; k++) v += *(const f32x4 *)(ob + (size_t)k * 16 * OROW + hh * OROW + col);
            const int head = hg * 16 + hh;
            if (head < a.NH) *(f32x4 *)(a.clat + ((size_t)b * a.NH + head) * KVL + col) = v * linv[hh];
        }
        return;
    }
    float *po = a.part_o + pidx * 16 * KVL;
#pragma unroll
    for (int j = 0; j < 16 * KVL / (4 * AW * MM_WAVE); j++) {
        const int e = 4 * (tid + j * AW * MM_WAVE);
        const int hh = e / KVL, col = e % KVL;
        f32x4 v = *(const f32x4 *)(ob + hh * OROW + col);
#pragma unroll
        for (int k = 1; k < AW; k++) v += *(const f32x4 *)(ob + (size_t)k * 16 * OROW + hh * OROW + col);
        *(f32x4 *)(po + e) = v;
    }
}

/* Rows that read one cache sequence in groups of AW (a prefill's
 * consecutive positions): one block per (row group, head group, chunk), a
 * 1-D grid of ceil(B / AW) HG nchunks blocks, the last group's first;
 * wave w is row AW grp + w and takes every key of the chunk below
 * its own length.  The chunk's 16-key sub-tiles go through a ring of NSR
 * stages shared by the block -- each wave loads 5 of a sub-tile's 18
 * pieces (the two k_pe pieces twice, identical bytes) -- so the group's
 * rows read their common keys once instead of once per row; one barrier
 * per sub-tile (every wave's pieces of it landed, every wave done with the
 * stage the refill takes).  No merge across waves: each wave leaves its
 * row's partial (or, with one chunk, clat) through its own LDS region.
 * a.slots is required and the host guarantees that a group's rows share a
 * sequence.  Dynamic LDS: AW * 16 * OROW * 4 bytes (>= NSR * TILE_B). */
#define NSR 4                      /* shared sub-tile stages */
#define RPIECES 5                  /* pieces per wave per sub-tile */
static_assert(NSR * TILE_B <= AW * 16 * OROW * 4 && AW * 16 * OROW * 4 == MM_MLA_ROWS_LDS, "row-group LDS");
static_assert(AW == 4, "pieces of a sub-tile over four waves");
extern "C" __global__ __launch_bounds__(AW * MM_WAVE) void mm_mla_attn_rows(mm_mla_attn_args a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t alds[];
    /* last group first (a prefill's longest rows), blocks in index order
     * over the XCDs in turn: with a prefill's causal lengths, the XCD-grouped
     * order of mm_mla_attn gave the last XCD every long row (measured: its
     * blocks ended ~600 us after the first while the others idled) */
    const int ngrp = (a.B + AW - 1) / AW;
    const int ntrip = ngrp * a.HG * a.nchunks;
    const int trip = (int)blockIdx.x;
    if (trip >= ntrip) return;
    const int rem = trip % (a.HG * a.nchunks);
    const int grp = ngrp - 1 - trip / (a.HG * a.nchunks), hg = rem / a.nchunks, chunk = rem % a.nchunks;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, kl = lane & 15;
    const int b = grp * AW + w;                       /* this wave's row */
    const bool brow = b < a.B;
    const int bc = min(b, a.B - 1);
    auto len = [&](int r) { return a.kv_lens ? min(a.kv_lens[r], a.kv_len) : a.kv_len; };
    int lmax = 0;
#pragma unroll
    for (int r = 0; r < AW; r++) lmax = max(lmax, len(min(grp * AW + r, a.B - 1)));
    const int kbeg = chunk * a.chunk;
    const int kend = brow ? min(kbeg + a.chunk, len(bc)) : kbeg;   /* this wave's keys */
    const int nsub = max(min(kbeg + a.chunk, lmax) - kbeg + 15, 0) / 16;   /* the block's sub-tiles */
    const int klast = max(lmax - 1, 0);
    const uint8_t *cseq = (const uint8_t *)(a.cache + (size_t)a.slots[grp * AW] * a.seq_stride * KVD);
    auto stage = [&](int st) { return alds + (size_t)st * TILE_B; };
    /* pieces w, w + 4, w + 8, w + 12 (c_kv rows) and k_pe piece w & 1 of
     * the sub-tile at key k0 (rows past the group's longest row load row
     * lmax - 1, masked in the softmax) */
    auto issue = [&](int st, int k0) {
        uint8_t *t = stage(st);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int p = w + 4 * j;
            const int key = __builtin_amdgcn_readfirstlane(min(k0 + p, klast));
            lds_dma16(cseq + (uint32_t)(key * KVD * 2) + lane * 16, t + p * CROW_B);
        }
        const int q = w & 1;
        const int key = min(k0 + 8 * q + (lane >> 3), klast);
        lds_dma16(cseq + (uint32_t)(key * KVD * 2 + KVL * 2 + (lane & 7) * 16), t + 16 * CROW_B + q * 1024);
    };

    /* Q of this wave's row (as mm_mla_attn, from global memory: a row's Q
     * is read by its chunks' blocks only), then the ring's first NSR - 1
     * sub-tiles; assembly loads, waited for by hand (after a direct-to-LDS
     * load the compiler waits for every load in flight at the first use of
     * a loaded register) */
    bf16x8 qh[KC], ql[KC];
    f32x4 qpe[KC - KVL / 32][2];
    static_assert(KC - KVL / 32 == 2, "q_pe: two 32-value K steps");
    const bool qreal = hg * 16 + kl < a.NH;
    {
        const int qhd = qreal ? hg * 16 + kl : 0;
        const uint16_t *qa = a.qhl + ((size_t)bc * a.NH + qhd) * 2 * KVL + 8 * g;
        const float *qp = a.q + ((size_t)bc * a.NH + qhd) * (a.QKN + MM_MLA_QKR) + a.QKN + 8 * g;
#pragma unroll
        for (int c = 0; c < KVL / 32; c++) {
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(qh[c]) : "v"(qa), "i"(64 * c));
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(ql[c]) : "v"(qa), "i"(2 * KVL + 64 * c));
        }
#pragma unroll
        for (int c = 0; c < KC - KVL / 32; c++) {
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(qpe[c][0]) : "v"(qp), "i"(128 * c));
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(qpe[c][1]) : "v"(qp), "i"(128 * c + 16));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < NSR - 1; st++) issue(st, kbeg + 16 * st);
    __builtin_amdgcn_sched_barrier(0);
    static_assert((NSR - 1) * RPIECES == 15, "wait count");
    asm volatile("s_waitcnt vmcnt(15)"
                 : "+v"(qh[0]), "+v"(qh[1]), "+v"(qh[2]), "+v"(qh[3]), "+v"(qh[4]), "+v"(qh[5]), "+v"(qh[6]),
                   "+v"(qh[7]), "+v"(qh[8]), "+v"(qh[9]), "+v"(qh[10]), "+v"(qh[11]), "+v"(qh[12]), "+v"(qh[13]),
                   "+v"(qh[14]), "+v"(qh[15]), "+v"(qpe[0][0]), "+v"(qpe[0][1]));
    asm volatile(""
                 : "+v"(ql[0]), "+v"(ql[1]), "+v"(ql[2]), "+v"(ql[3]), "+v"(ql[4]), "+v"(ql[5]), "+v"(ql[6]),
                   "+v"(ql[7]), "+v"(ql[8]), "+v"(ql[9]), "+v"(ql[10]), "+v"(ql[11]), "+v"(ql[12]), "+v"(ql[13]),
                   "+v"(ql[14]), "+v"(ql[15]), "+v"(qpe[1][0]), "+v"(qpe[1][1]));
    {
        const bf16x8 z8 = __builtin_bit_cast(bf16x8, (u16x8){});
#pragma unroll
        for (int c = 0; c < KVL / 32; c++) {
            qh[c] = qreal ? qh[c] : z8;
            ql[c] = qreal ? ql[c] : z8;
        }
#pragma unroll
        for (int c = KVL / 32; c < KC; c++) {
            const f32x4 x0 = qpe[c - KVL / 32][0], x1 = qpe[c - KVL / 32][1];
            u16x8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint16_t h16, l16;
                split_bf16(qreal ? (j < 4 ? x0[j & 3] : x1[j & 3]) : 0.0f, &h16, &l16);
                hi[j] = h16;
                lo[j] = l16;
            }
            qh[c] = __builtin_bit_cast(bf16x8, hi);
            ql[c] = __builtin_bit_cast(bf16x8, lo);
        }
    }

    float m = -INFINITY, l = 0.0f;        /* head kl: running max; this lane's share of the sum */
    f32x4 O[KVL / 16];
#pragma unroll
    for (int nb = 0; nb < KVL / 16; nb++) O[nb] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < nsub; i++) {
        /* this wave's pieces of sub-tile i have landed once at most those of
         * the next NSR - 2 sub-tiles are outstanding (every step issues one
         * sub-tile, past the chunk at clamped keys: the count holds to the
         * end); the barrier: every wave's pieces, and every wave done with
         * sub-tile i - 1, whose stage the refill below takes */
        static_assert((NSR - 2) * RPIECES == 10, "wait count");
        VMCNT_WAIT(10);
        /* a bare barrier: __syncthreads() would also wait for every load
         * in flight (the ring's later sub-tiles) */
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue((i + NSR - 1) % NSR, kbeg + 16 * (i + NSR - 1));
        __builtin_amdgcn_sched_barrier(0);
        const int k0 = kbeg + 16 * i;
        const uint32_t t = lds_addr(stage(i % NSR));
        float sv[4];
        mla_score(a, t, k0, kend, bc, hg, kl, g, qh, ql, sv);
        float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        if (__builtin_amdgcn_ballot_w64(mx > m + RESCALE_TAU)) {
            /* some head's maximum moved: new m = the head's max over the
             * sub-tile (across the 4 lane groups); O and l rescaled unless
             * still empty */
            mx = fmaxf(mx, __shfl_xor(mx, 16, MM_WAVE));
            mx = fmaxf(mx, __shfl_xor(mx, 32, MM_WAVE));
            const float mnew = fmaxf(m, mx);
            if (__builtin_amdgcn_ballot_w64(m != -INFINITY)) {
                const float cr = m == -INFINITY ? 0.0f : __expf(m - mnew);
                l *= cr;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float ci = __shfl(cr, 4 * g + r, MM_WAVE);
#pragma unroll
                    for (int nb = 0; nb < KVL / 16; nb++) O[nb][r] *= ci;
                }
            }
            m = mnew;
        }
        mla_accumulate(t, sv, m, l, O, kl, g);
    }
    VMCNT_WAIT(0);
    __syncthreads();   /* every stage read: the LDS takes the waves' outputs */

    /* this wave's row: (m, l) per head and O, scaled by 1 / l for clat */
    l += __shfl_xor(l, 16, MM_WAVE);
    l += __shfl_xor(l, 32, MM_WAVE);
    float *ob = (float *)alds + (size_t)w * 16 * OROW;
    const float fself = a.clat ? (l > 0.0f ? 1.0f / l : 0.0f) : 1.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float fr = __shfl(fself, 4 * g + r, MM_WAVE);
#pragma unroll
        for (int nb = 0; nb < KVL / 16; nb++) ob[(4 * g + r) * OROW + nb * 16 + kl] = O[nb][r] * fr;
    }
    if (!brow) return;
    const size_t pidx = ((size_t)(b * a.HG + hg) * a.nchunks + chunk);
    if (!a.clat && g == 0) {
        a.part_ml[pidx * 32 + kl] = m;
        a.part_ml[pidx * 32 + 16 + kl] = l;
    }
#pragma unroll 4
    for (int j = 0; j < 16 * KVL / (4 * MM_WAVE); j++) {
        const int e = 4 * (lane + j * MM_WAVE);
        const int hh = e / KVL, col = e % KVL;
        const f32x4 v = *(const f32x4 *)(ob + hh * OROW + col);
        if (a.clat) {
            const int head = hg * 16 + hh;
            if (head < a.NH) *(f32x4 *)(a.clat + ((size_t)b * a.NH + head) * KVL + col) = v;
        } else {
            *(f32x4 *)(a.part_o + pidx * 16 * KVL + e) = v;
        }
    }
}

/* Merge the chunk partials of (head h, sequence b): clat = sum_c w_c O_c / l
 * with w_c = e^(m_c - m); also turns the debug scores into probabilities.
 * grid (NH, B, Z) with Z = 1 or KVL / 128, 256 threads: block z owns the
 * latent columns [z KVL / Z, (z + 1) KVL / Z); thread t sums the column pair
 * t % (pairs per block) over the chunks of its group t / (pairs per block)
 * (16 loads in flight); with Z > 1 the chunk groups meet in LDS in group
 * order (small batches: more blocks, fewer chunks each). */
extern "C" __global__ __launch_bounds__(256) void mm_mla_combine(mm_mla_combine_args a) {
    __shared__ float wch[MM_MLA_MAXCH];
    __shared__ float stat[2];
    __shared__ float2 red[256];
    const int h = blockIdx.x, b = blockIdx.y, z = blockIdx.z;
    const int hg = h >> 4, hl = h & 15;
    const int tid = threadIdx.x;
    const int L = a.kv_lens ? min(a.kv_lens[b], a.kv_len) : a.kv_len;
    const size_t pbase = (size_t)(b * a.HG + hg) * a.nchunks;
    if (tid < MM_WAVE) {
        /* chunk maxima and sums: lane l takes chunks l, l + 64, ...
         * (nchunks <= MM_MLA_MAXCH) */
        float mx = -INFINITY;
        for (int c = tid; c < a.nchunks; c += MM_WAVE)
            mx = fmaxf(mx, a.part_ml[(pbase + c) * 32 + hl]);
        mx = wave_max(mx);
        float ls = 0.0f;
        for (int c = tid; c < a.nchunks; c += MM_WAVE) {
            const float mc = a.part_ml[(pbase + c) * 32 + hl];
            const float wc = mc == -INFINITY ? 0.0f : __expf(mc - mx);
            ls += a.part_ml[(pbase + c) * 32 + 16 + hl] * wc;
            wch[c] = wc;
        }
        ls = wave_sum(ls);
        if (tid == 0) {
            stat[0] = mx;
            stat[1] = ls;
        }
    }
    __syncthreads();
    const float mx = stat[0], inv = 1.0f / stat[1];
    static_assert(KVL == 512, "combine: 256 column pairs per sequence and head");
    const int npair = (KVL / 2) / gridDim.z, ng = 256 / npair;   /* pairs per block, chunk groups */
    const int cp = tid % npair, cg = tid / npair;
    const int col = z * (KVL / gridDim.z) + 2 * cp;
    const float *po = a.part_o + (pbase * 16 + hl) * KVL + col;
    float o0 = 0.0f, o1 = 0.0f;
    for (int c0 = cg; c0 < a.nchunks; c0 += ng * 16) {
        float2 v[16];
#pragma unroll
        for (int k = 0; k < 16; k++)
            v[k] = *(const float2 *)(po + (size_t)min(c0 + ng * k, a.nchunks - 1) * 16 * KVL);
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (c0 + ng * k < a.nchunks) {
                o0 += wch[c0 + ng * k] * v[k].x;
                o1 += wch[c0 + ng * k] * v[k].y;
            }
    }
    red[tid] = make_float2(o0, o1);
    __syncthreads();
    if (cg == 0) {
        float2 s2 = red[cp];
        for (int g = 1; g < ng; g++) {
            s2.x += red[g * npair + cp].x;
            s2.y += red[g * npair + cp].y;
        }
        float *cl = a.clat + ((size_t)b * a.NH + h) * KVL;
        *(float2 *)(cl + col) = make_float2(s2.x * inv, s2.y * inv);
    }
    if (a.probs && z == 0) {
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
            if (bb < mrows && (lane & 15) < nv) {
                const size_t o = ((size_t)(b0 + bb) * a.NH + h) * a.VHD + vw + (lane & 15);
                a.ctx[o] = acc[t][i];
                if (a.ctx_hl) {   /* o_proj's operand split once here */
                    const uint16_t hi = rne16(acc[t][i]);
                    a.ctx_hl[o] = hi;
                    a.ctx_hl[(size_t)a.B * a.NH * a.VHD + o] = rne16(acc[t][i] - bf16_f32(hi));
                }
            }
        }
}

/* mm_mla_uv for large batches: grid (ceil(VHD / (16 S)), NH, ceil(B / 32)),
 * each wave S column tiles of its K quarter (clat read and split once per
 * S tiles); W_UV rows past VHD read row VHD - 1 (results not stored). */
extern "C" __global__ __launch_bounds__(256) void mm_mla_uv_w(mm_mla_combine_args a) {
    constexpr int S = MM_MLA_WIDE_S;
    __shared__ f32x4 red[3][S][2][MM_WAVE];
    const int v0 = blockIdx.x * 16 * S, h = blockIdx.y, b0 = blockIdx.z * 32;
    const int lane = threadIdx.x & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / MM_WAVE);
    const int mrows = min(32, a.B - b0);
    const uint16_t *wuv = a.kv_b + ((size_t)h * (a.QKN + a.VHD) + a.QKN) * KVL;
    const uint16_t *wr[S];
#pragma unroll
    for (int s = 0; s < S; s++) wr[s] = wuv + (size_t)min(v0 + 16 * s + (lane & 15), a.VHD - 1) * KVL;
    f32x4 acc[S][2];
    hl_gemm_32x16s<S>(a.clat + ((size_t)b0 * a.NH + h) * KVL, (size_t)a.NH * KVL, mrows, wr,
                      wave * (KVL / 4), (wave + 1) * (KVL / 4), acc);
    if (wave > 0) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            red[wave - 1][s][0][lane] = acc[s][0];
            red[wave - 1][s][1][lane] = acc[s][1];
        }
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int s = 0; s < S; s++) {
#pragma unroll
        for (int w = 0; w < 3; w++) {
            acc[s][0] += red[w][s][0][lane];
            acc[s][1] += red[w][s][1][lane];
        }
        const int v = v0 + 16 * s + (lane & 15);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int bb = 16 * t + 4 * (lane >> 4) + i;
                if (bb < mrows && v < a.VHD) {
                    const size_t o = ((size_t)(b0 + bb) * a.NH + h) * a.VHD + v;
                    a.ctx[o] = acc[s][t][i];
                    if (a.ctx_hl) {
                        const uint16_t hi = rne16(acc[s][t][i]);
                        a.ctx_hl[o] = hi;
                        a.ctx_hl[(size_t)a.B * a.NH * a.VHD + o] = rne16(acc[s][t][i] - bf16_f32(hi));
                    }
                }
            }
    }
}

/* ---- decode front: RoPE, kv_a_layernorm, latent-cache append ----------------- */

/* One block per token b at position p = pos[b] of cache sequence slots[b]
 * (b without slots) (src/run.c:420-428):
 *   q_pe of every head   rope_apply(q_h + QKN, p)                (run.c:420-421)
 *   c_kv                 rmsnorm(comp[0:KVL], kv_a_layernorm, eps) (run.c:426)
 *   k_pe                 rope_apply(comp[KVL:KVL+QKR], p)         (run.c:427-428)
 * The row c_kv | k_pe goes to the bf16 cache at (b, p), rounded to nearest
 * even (the reference keeps an fp32 cache, include/model.h:117), and, when
 * kv_out is given, to kv_out in fp32.  A position outside [0, seq_stride)
 * writes no cache row.  cos / sin of the angle p * inv_freq[j] are evaluated
 * in fp64 and rounded once, so they are the correctly rounded fp32 values
 * except for angles within ~2^-29 relative of a rounding boundary; the
 * rotations are unfused multiply / add, in the reference's order. */
__device__ __forceinline__ uint16_t bf16_rne_keepnan(float x) {
    return x != x ? (uint16_t)0x7fc0u : bf16_rne(x);
}

__device__ __forceinline__ void rope_token(const mm_mla_rope_args &a, int b) {
#pragma clang fp contract(off)
    __shared__ float cs[2][128];
    __shared__ float red[256 / MM_WAVE];
    static_assert(KVL == 512 && MM_MLA_QKR <= 256, "one c_kv pair per thread, one k_pe pair per thread");
    const int tid = threadIdx.x;
    const int half = MM_MLA_QKR / 2, kvd = KVL + MM_MLA_QKR;
    const int qhd = a.qkn + MM_MLA_QKR, npairs = a.nh * half;
    constexpr int QK = MM_ROPE_PAIRS_MAX / 256;
    /* Every load of the block goes out first, at clamped addresses (no load
     * under a condition: each would be waited for on its own), so the block
     * pays one round trip: the position, the cache slot, the frequency, this
     * thread's c_kv pair with its norm weights, its k_pe pair and its q_pe
     * pairs.  Thread t owns c_kv values 2t, 2t + 1 and k_pe pair t (t < 32). */
    const int p = a.pos[b];
    const int seq = a.slots ? a.slots[b] : b;
    const float invf = a.inv_freq[min(tid, half - 1)];
    const float *comp = a.comp + (size_t)b * kvd;
    const f32x2 cv = *(const f32x2 *)(comp + 2 * tid);
    const uint32_t nw = *(const uint32_t *)(a.kv_norm + 2 * tid);
    const f32x2 kp = *(const f32x2 *)(comp + KVL + 2 * min(tid, half - 1));
    float *q = a.q + (size_t)b * a.nh * qhd + a.qkn;
    float qe[QK], qo[QK];
#pragma unroll
    for (int k = 0; k < QK; k++) {
        const int i = min(tid + 256 * k, npairs - 1);
        const int h = i / half, j = i - h * half;
        const f32x2 v = *(const f32x2 *)(q + (size_t)h * qhd + 2 * j);   /* adjacent pair, both layouts */
        qe[k] = v.x;
        qo[k] = v.y;
    }
    if (tid < half) {
        const double ang = (double)((float)p * invf);
        cs[0][tid] = (float)cos(ang);
        cs[1][tid] = (float)sin(ang);
    }
    float ss = cv.x * cv.x + cv.y * cv.y;
    ss = wave_sum(ss);
    if ((tid & (MM_WAVE - 1)) == 0) red[tid / MM_WAVE] = ss;
    __syncthreads();   /* red and cs; every thread has read its q pairs */
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < 256 / MM_WAVE; w++) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)KVL + a.eps);

    /* q_pe of every head, in place (all pairs were read before the barrier:
     * the split-half layout moves values across pairs) */
#pragma unroll
    for (int k = 0; k < QK; k++) {
        const int i = tid + 256 * k;
        if (i < npairs) {
            const int h = i / half, j = i - h * half;
            const float c = cs[0][j], s = cs[1][j];
            float *v = q + (size_t)h * qhd;
            if (!a.interleaved) {
                v[2 * j] = qe[k] * c - qo[k] * s;
                v[2 * j + 1] = qe[k] * s + qo[k] * c;
            } else {
                v[j] = qe[k] * c - qo[k] * s;
                v[half + j] = qo[k] * c + qe[k] * s;
            }
        }
    }

    /* the cache row */
    const bool wr = p >= 0 && p < a.seq_stride;
    uint16_t *dst = a.cache + ((size_t)seq * a.seq_stride + (wr ? p : 0)) * kvd;
    float *ko = a.kv_out ? a.kv_out + (size_t)b * kvd : nullptr;
    {
        const int i = 2 * tid;
        const float y0 = cv.x * inv * bf16_lo(nw);
        const float y1 = cv.y * inv * bf16_hi(nw);
        if (wr) *(uint32_t *)(dst + i) = (uint32_t)bf16_rne_keepnan(y0) | (uint32_t)bf16_rne_keepnan(y1) << 16;
        if (ko) { ko[i] = y0; ko[i + 1] = y1; }
    }
    if (tid < half) {
        const int j = tid;
        const float c = cs[0][j], s = cs[1][j];
        const float x0 = kp.x, x1 = kp.y;
        const int o0 = KVL + (a.interleaved ? j : 2 * j);
        const int o1 = KVL + (a.interleaved ? half + j : 2 * j + 1);
        const float r0 = x0 * c - x1 * s;
        const float r1 = a.interleaved ? x1 * c + x0 * s : x0 * s + x1 * c;
        if (wr) { dst[o0] = bf16_rne_keepnan(r0); dst[o1] = bf16_rne_keepnan(r1); }
        if (ko) { ko[o0] = r0; ko[o1] = r1; }
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_mla_rope(mm_mla_rope_args a) {
    rope_token(a, blockIdx.x);
}

/* mm_mla_rope and mm_mla_qprep in one launch (independent: RoPE writes the
 * q_pe parts and the cache row, qprep reads the q_nope parts): one launch
 * fewer per decode layer. */
extern "C" __global__ __launch_bounds__(256) void mm_mla_rope_qprep(mm_mla_rope_qprep_args a) {
    const int b = blockIdx.x;
    if (b < a.r.B) {
        rope_token(a.r, b);
        return;
    }
    const int v = b - a.r.B, nx = KVL / 64;
    qprep_block(a.qp, v % nx, (v / nx) % a.qp.NH, v / (nx * a.qp.NH) * 32);
}
