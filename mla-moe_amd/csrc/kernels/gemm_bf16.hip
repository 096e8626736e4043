/* gemm_bf16.hip -- dense y = x . W^T on v_mfma_f32_16x16x32_bf16 (matmul of
 * src/run.c:29-37 batched over T rows).
 *
 * W is bf16 row-major [d_out, n_in] exactly as the reference stores it: a B
 * operand fragment (16 output columns x 32 inputs, lane l holding column
 * l % 16 and inputs 8*(l/16) .. +7) is 16 contiguous bytes of one weight row
 * per lane, so B stages into LDS by direct global -> LDS loads in operand
 * order.  x is fp32: mm_cvt_bf16 first writes it as bf16 rows, either
 * truncated (the config that casts activations on the input side,
 * include/tensor.h:16-20) or split into a bf16 hi/lo pair (two MFMAs, ~2^-17
 * relative) so the result tracks the fp32 reference; A then stages exactly
 * like B.
 *
 * Block tile 128 x 128, K step 64; four waves in a 2 x 2 grid, each a 64 x
 * 64 tile (16 MFMAs per 32 of K).  Both operands stage through an LDS ring
 * (4 stages, 3 for the split) by direct loads issued three (two) steps
 * ahead of the MFMAs.
 */
#include "common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

#define GB_BM 128
#define GB_BK 64
#define GB_COPY (128 * 128)             /* A of one stage: 128 rows x 128 B */

/* x -> bf16 rows of stride kp (zeros past n_in), 8 values per thread:
 * truncation (the reference's cast, include/tensor.h:16-20) or the RNE
 * hi/lo split. */
extern "C" __global__ __launch_bounds__(256) void mm_cvt_bf16(mm_cvt_bf16_args a) {
    const size_t i8 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   /* 8-value chunk */
    const int cpr = a.kp / 8;
    if (i8 >= (size_t)a.T * cpr) return;
    const int t = (int)(i8 / cpr), k = (int)(i8 % cpr) * 8;
    u16x8 hi = {0, 0, 0, 0, 0, 0, 0, 0}, lo = {0, 0, 0, 0, 0, 0, 0, 0};
    if (k < a.n_in) {   /* n_in is a multiple of 8 */
        const float *p = a.x + (size_t)t * a.n_in + k;
        const f32x4 x0 = *(const f32x4 *)p, x1 = *(const f32x4 *)(p + 4);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = e < 4 ? x0[e] : x1[e - 4];
            if (a.split) {
                const uint16_t h16 = rne16(v);
                hi[e] = h16;
                lo[e] = rne16(v - bf16_f32(h16));
            } else {
                hi[e] = (uint16_t)(__float_as_uint(v) >> 16);
            }
        }
    }
    *(u16x8 *)(a.xh + i8 * 8) = hi;
    if (a.split) *(u16x8 *)(a.xl + i8 * 8) = lo;
}

/* Stage layout: [A hi][A lo (split mode)][B], each 128 rows (A) or output
 * columns (B) x 64 K = 16 KB.  A load instruction moves 8 rows x 128 B
 * (whole cache lines; half-line accesses measured ~2.6x slower): lane l
 * carries row 8 i + l / 8 and stores at position p = l % 8 of that row's
 * 128 B the 16 B chunk q = p ^ s(row), s(R) = (R / 2) % 8.  The XOR swizzle
 * makes the operand reads below (16 rows, one chunk each) conflict-free. */
__device__ __forceinline__ int gb_swz(int R) { return (R >> 1) & 7; }

template <bool HL, int GB_BN>
__device__ __forceinline__ void gemm_block(const mm_gemm_bf16_args &a, uint8_t *lds) {
    constexpr int GB_NC = GB_BN / 32;             /* B fragments of 16 columns per wave */
    constexpr int NA = HL ? 2 : 1;                /* A copies: hi (and lo) */
    constexpr int BOFF = NA * GB_COPY;
    constexpr int SB = BOFF + GB_BN * 128;        /* stage bytes */
    constexpr int NS = HL ? 3 : 4;                /* stages */
    constexpr int D = NS - 1;                     /* steps issued ahead */
    constexpr int G = 4 * NA + GB_NC;             /* transfers per wave per step */
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    /* 1-D grid: blocks are dealt to the 8 XCDs round robin (block b -> XCD
     * b % 8).  XCD x takes the column blocks x, x + 8, ... for every row
     * block: its weight columns are fetched into its L2 once and reused by
     * all row blocks, and the x rows (small) are shared by its tiles */
    const int nbx = (a.d_out + GB_BN - 1) / GB_BN, nby = (a.T + GB_BM - 1) / GB_BM;
    const int b = blockIdx.x, slot = b / 8;
    const int cb = b % 8 + 8 * (slot / nby), rb = slot % nby;
    if (cb >= nbx) return;
    const int m0 = rb * GB_BM, n0 = cb * GB_BN;
    const int K = a.n_in, KB = a.kp / GB_BK;

    /* wave w issues A instructions 4 w .. 4 w + 3 (rows 32 w .. 32 w + 31)
     * (hi, lo) and B instructions GB_NC w .. GB_NC w + GB_NC - 1; rows past
     * T / columns past d_out read the last one (results discarded); B chunks
     * past n_in re-read chunk 0 of the row (A is zero there) */
    const uint16_t *ah_src[4], *al_src[4], *b_src[GB_NC];
    int bq[GB_NC];
#pragma unroll
    for (int h = 0; h < 4; h++) {
        const int R = 8 * (4 * wave + h) + (lane >> 3);
        const int kq = 8 * ((lane & 7) ^ gb_swz(R));      /* element offset in the step */
        const int m = min(m0 + R, a.T - 1);
        ah_src[h] = a.xh + (size_t)m * a.kp + kq;
        al_src[h] = HL ? a.xl + (size_t)m * a.kp + kq : nullptr;
    }
#pragma unroll
    for (int h = 0; h < GB_NC; h++) {
        const int R = 8 * (GB_NC * wave + h) + (lane >> 3);
        const int n = min(n0 + R, a.d_out - 1);
        b_src[h] = a.w + (size_t)n * K;
        bq[h] = 8 * ((lane & 7) ^ gb_swz(R));
    }
    auto issue = [&](int kb, int st) {
        uint8_t *s0 = lds + st * SB;
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const int i = 4 * wave + h;
            lds_dma16(ah_src[h] + kb * GB_BK, s0 + i * 1024);
            if (HL) lds_dma16(al_src[h] + kb * GB_BK, s0 + GB_COPY + i * 1024);
        }
#pragma unroll
        for (int h = 0; h < GB_NC; h++) {
            const int k = kb * GB_BK + bq[h];
            lds_dma16(b_src[h] + (k < K ? k : 0), s0 + BOFF + (GB_NC * wave + h) * 1024);
        }
    };
    /* operand read of lane (c = l % 16, g = l / 16) for fragment row block r
     * and K half kh: row 16 r + c, chunk q = 4 kh + g, at (16 r + c) * 128 +
     * 16 (q ^ s(c)); the r part is a compile-time offset */
    const int c16 = lane & 15, g4 = lane >> 4;
    const uint32_t rd0 = c16 * 128 + 16 * ((0 + g4) ^ gb_swz(c16));
    const uint32_t rd1 = c16 * 128 + 16 * ((4 + g4) ^ gb_swz(c16));

    f32x4 acc[4][GB_NC];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int c = 0; c < GB_NC; c++) acc[r][c] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    /* every step issues one group (steps past the end re-load the last, so
     * that the wait counts are static) */
#pragma unroll
    for (int s = 0; s < D; s++) issue(min(s, KB - 1), s);
    __builtin_amdgcn_sched_barrier(0);
    auto step = [&](int kb, int j) {   /* j = kb % NS */
        VMCNT_WAIT(G * (D - 1));       /* this wave's step-kb group has landed */
        __builtin_amdgcn_s_barrier();  /* ... every wave's, and stage kb-1 is free */
        __builtin_amdgcn_sched_barrier(0);
        issue(min(kb + D, KB - 1), (j + D) % NS);
        __builtin_amdgcn_sched_barrier(0);
        /* this wave's A rows 64 wm .. and B columns GB_BN / 2 * wn .. */
        const uint32_t st0 = lds_addr(lds + j * SB);
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const uint32_t sa = st0 + (kh ? rd1 : rd0) + wm * 64 * 128;
            const uint32_t sb = st0 + BOFF + (kh ? rd1 : rd0) + wn * (GB_BN / 2) * 128;
            i32x4 ah[4], al[4], bw[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                ah[r] = ds_read16(sa, r * 2048);
                if (HL) al[r] = ds_read16(sa, GB_COPY + r * 2048);
            }
#pragma unroll
            for (int c = 0; c < GB_NC; c++) bw[c] = ds_read16(sb, c * 2048);
            if (HL)
                asm volatile("s_waitcnt lgkmcnt(0)"
                             : "+v"(ah[0]), "+v"(ah[1]), "+v"(ah[2]), "+v"(ah[3]), "+v"(al[0]), "+v"(al[1]),
                               "+v"(al[2]), "+v"(al[3]), "+v"(bw[0]), "+v"(bw[1]), "+v"(bw[2]), "+v"(bw[3]));
            else
                asm volatile("s_waitcnt lgkmcnt(0)"
                             : "+v"(ah[0]), "+v"(ah[1]), "+v"(ah[2]), "+v"(ah[3]), "+v"(bw[0]), "+v"(bw[1]),
                               "+v"(bw[2]), "+v"(bw[3]));
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int c = 0; c < GB_NC; c++) {
                    const bf16x8 bb = __builtin_bit_cast(bf16x8, bw[c]);
                    acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[r]), bb,
                                                                        acc[r][c], 0, 0, 0);
                    if (HL)
                        acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al[r]), bb,
                                                                            acc[r][c], 0, 0, 0);
                }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int k0 = 0;
    for (; k0 + NS <= KB; k0 += NS) {
#pragma unroll
        for (int j = 0; j < NS; j++) step(k0 + j, j);
    }
#pragma unroll
    for (int j = 0; j < NS - 1; j++)
        if (k0 + j < KB) step(k0 + j, j);
    VMCNT_WAIT(0);

    /* lane holds D[4 (l / 16) + i][l % 16] of each 16 x 16 tile.  With
     * accumulate, a row block's old outputs are all loaded (clamped
     * addresses, unconditionally) before any is added: a load under the
     * row / column conditions would be a branch of its own, each waited
     * for before the next is issued. */
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float prev[GB_NC][4];
        if (a.accumulate) {   /* uniform */
#pragma unroll
            for (int c = 0; c < GB_NC; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = min(n0 + (GB_BN / 2) * wn + 16 * c + (lane & 15), a.d_out - 1);
                    const int m = min(m0 + 64 * wm + 16 * r + 4 * (lane >> 4) + i, a.T - 1);
                    prev[c][i] = a.y[(size_t)m * a.d_out + n];
                }
        }
#pragma unroll
        for (int c = 0; c < GB_NC; c++) {
            const int n = n0 + (GB_BN / 2) * wn + 16 * c + (lane & 15);
            if (n >= a.d_out) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 64 * wm + 16 * r + 4 * (lane >> 4) + i;
                if (m >= a.T) continue;
                a.y[(size_t)m * a.d_out + n] = a.accumulate ? prev[c][i] + acc[r][c][i] : acc[r][c][i];
            }
        }
    }
}

/* 1-D grid of 8 * ceil(ceil(d_out / 128) / 8) * ceil(T / 128) blocks, 256
 * threads, dynamic LDS: 4 stages x 32 KB (truncated x) or
 * 3 x 48 KB (hi/lo x). */
extern "C" __global__ __launch_bounds__(256) void mm_gemm_bf16(mm_gemm_bf16_args a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t glds[];
    if (a.split) {
        if (a.bn == 128) gemm_block<true, 128>(a, glds);
        else if (a.bn == 64) gemm_block<true, 64>(a, glds);
        else gemm_block<true, 32>(a, glds);
    } else {
        if (a.bn == 128) gemm_block<false, 128>(a, glds);
        else if (a.bn == 64) gemm_block<false, 64>(a, glds);
        else gemm_block<false, 32>(a, glds);
    }
}

/* ---- skinny-M GEMM: T <= 64 rows of x (batched decode) ------------------------
 *
 * Every weight row is read from HBM once per K split.  Block = 4 waves x
 * 16 SK_WC output columns; a wave holds C[64 tokens][16 SK_WC columns] (4
 * token groups x SK_WC column groups of v_mfma_f32_16x16x32_bf16, x as the
 * A operand -- each x fragment read from LDS feeds SK_WC MFMAs -- and W as
 * the B operand).  The
 * W fragments of the block's K range stream straight into registers, SK_D
 * 64-input chunks ahead of their MFMAs; fp32 x is loaded two chunks ahead
 * into registers and staged into LDS as bf16 (hi and lo) one 64-input chunk
 * at a time, so no separate conversion pass runs (double-buffered; rows
 * padded to 72 bf16 against bank conflicts; token rows past T read row
 * T - 1 and are not stored).  With
 * nsplit > 1 the K range is split over grid.y and mm_skinny_reduce sums the
 * partials in split order. */
/* Two forms: 64 output columns per block (one 16-column group per wave,
 * 4 chunks of W in flight), and for long outputs (the LM head) 64 *
 * MM_SKINNY_WIDE_WC columns per block (MM_SKINNY_WIDE_WC groups per wave, 2
 * chunks in flight), which stages each x chunk (64 rows x 64 inputs, fp32:
 * twice the bytes of one wave-group's weights) once for more weights.  LM
 * head at 64 rows (102400 x 2048): 154.6 -> ~136 us with 2 or 4 groups. */
#define SK_WC1 (MM_SKINNY_BN / 64)   /* 16-column groups per wave */
#define SK_D1 4                      /* chunks of W in flight per wave */
#define SK_DW 2
#define SK_ROW 72                    /* LDS row stride (bf16) of a staged x chunk */
#define SK_STAGE (2 * 64 * SK_ROW)   /* bf16 per stage: hi rows then lo rows */

template <bool SPLIT, int SK_WC, int SK_D>
__device__ __forceinline__ void skinny(const mm_gemm_skinny_args &a, uint16_t (*xs)[SK_STAGE]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    /* column block bx of matrix `seg` (the second one past nb0 blocks) */
    const bool seg = (int)blockIdx.x >= a.nb0;
    const int bx = seg ? blockIdx.x - a.nb0 : blockIdx.x;
    const int d_out = seg ? a.d_out1 : a.d_out;
    const uint16_t *wm = seg ? a.w1 : a.w;
    const int n0 = bx * (64 * SK_WC) + wave * (16 * SK_WC);
    const int kb = blockIdx.y * a.kr;
    const int nch = (min(a.n_in, kb + a.kr) - kb) / 64;    /* 64-input chunks of this split */
    const uint16_t *wrow[SK_WC];
#pragma unroll
    for (int j = 0; j < SK_WC; j++) {
        const int col = min(n0 + 16 * j + (lane & 15), d_out - 1);   /* past d_out: not stored */
        wrow[j] = wm + (size_t)col * a.n_in + kb + 8 * (lane >> 4);
    }

    /* x chunk c (fp32) -> registers, two slots: chunks are loaded two ahead
     * of their use.  Thread t holds the 16 B pieces p = t + 256 j (64 rows x
     * 16 pieces); staging converts them to bf16 -- the hi/lo pair of
     * mm_cvt_bf16 (RNE hi, RNE of the remainder) or the truncation -- and
     * writes hi rows then lo rows. */
    f32x4 xr[2][4];
    auto load_x = [&](int slot, int c) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int p = tid + 256 * j, r = p >> 4, q = p & 15;
            xr[slot][j] = *(const f32x4 *)(a.x + (size_t)min(r, a.T - 1) * a.n_in + kb + 64 * c + 4 * q);
        }
    };
    auto store_x = [&](int slot, int st) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int p = tid + 256 * j, r = p >> 4, q = p & 15;
            typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
            u16x4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v = xr[slot][j][e];
                if (SPLIT) {
                    hi[e] = rne16(v);
                    lo[e] = rne16(v - bf16_f32(hi[e]));
                } else {
                    hi[e] = (uint16_t)(__float_as_uint(v) >> 16);
                }
            }
            *(u16x4 *)&xs[st][r * SK_ROW + 4 * q] = hi;
            if (SPLIT) *(u16x4 *)&xs[st][(64 + r) * SK_ROW + 4 * q] = lo;
        }
    };
    bf16x8 wr[SK_D][SK_WC][2];
    auto load_w = [&](int slot, int c) {
        const int cc = min(c, nch - 1);                     /* past the end: reload the last */
#pragma unroll
        for (int j = 0; j < SK_WC; j++)
#pragma unroll
            for (int s = 0; s < 2; s++)
                wr[slot][j][s] = __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(
                                                                (const u16x8 *)(wrow[j] + 64 * cc + 32 * s)));
    };
#pragma unroll
    for (int d = 0; d < SK_D; d++) load_w(d, d);
    load_x(0, 0);
    if (nch > 1) load_x(1, 1);
    store_x(0, 0);
    __syncthreads();

    f32x4 acc[SK_WC][4];
#pragma unroll
    for (int j = 0; j < SK_WC; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) acc[j][g] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    static_assert(SK_D % 2 == 0, "the x slots alternate with the chunk parity");
    for (int c0 = 0; c0 < nch; c0 += SK_D) {
#pragma unroll
        for (int d = 0; d < SK_D; d++) {
            const int c = c0 + d;
            /* slot d & 1 held chunk c (in LDS since the last barrier): refill it with c + 2 */
            if (c + 2 < nch) load_x(d & 1, c + 2);
            if (c < nch) {
                const uint16_t *xb = xs[d & 1];
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const int ko = 32 * s + 8 * (lane >> 4);
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int r = 16 * g + (lane & 15);
                        const bf16x8 ah = *(const bf16x8 *)&xb[r * SK_ROW + ko];
                        bf16x8 al;
                        if (SPLIT) al = *(const bf16x8 *)&xb[(64 + r) * SK_ROW + ko];
#pragma unroll
                        for (int j = 0; j < SK_WC; j++) {
                            acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wr[d][j][s], acc[j][g], 0, 0, 0);
                            if (SPLIT)
                                acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, wr[d][j][s], acc[j][g], 0, 0, 0);
                        }
                    }
                }
            }
            load_w(d, c + SK_D);
            if (c + 1 < nch) store_x((d + 1) & 1, (d + 1) & 1);
            __syncthreads();
        }
    }
    /* C[token 16 g + 4 (l / 16) + i][column n0 + 16 j + l % 16] */
#pragma unroll
    for (int j = 0; j < SK_WC; j++) {
        const int n = n0 + 16 * j + (lane & 15);
        if (n >= d_out) continue;
        float *part = a.part + (seg ? (size_t)a.nsplit * a.T * a.d_out : 0);
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * g + 4 * (lane >> 4) + i;
                if (t >= a.T) continue;
                if (a.nsplit > 1 || a.part_out) {
                    part[((size_t)blockIdx.y * a.T + t) * d_out + n] = acc[j][g][i];
                } else {
                    float *y = (seg ? a.y1 : a.y) + (size_t)t * d_out + n;
                    *y = a.accumulate ? *y + acc[j][g][i] : acc[j][g][i];
                }
            }
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_gemm_skinny(mm_gemm_skinny_args a) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][SK_STAGE];
    if (a.split)
        skinny<true, SK_WC1, SK_D1>(a, xs);
    else
        skinny<false, SK_WC1, SK_D1>(a, xs);
}

extern "C" __global__ __launch_bounds__(256) void mm_gemm_skinny_wide(mm_gemm_skinny_args a) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][SK_STAGE];
    if (a.split)
        skinny<true, MM_SKINNY_WIDE_WC, SK_DW>(a, xs);
    else
        skinny<false, MM_SKINNY_WIDE_WC, SK_DW>(a, xs);
}

/* y (+)= sum over splits s = 0 .. nsplit-1 of part[s], in that order. */
/* ---- skinny-M GEMM over pre-split x ------------------------------------------
 *
 * The mm_gemm_skinny computation (same column blocks, K splits, partials and
 * MFMA sequence per output: per 32-wide K step the hi product, then the lo
 * product) with x arriving as bf16 hi/lo planes written by its producer.
 * Both operands then go global -> LDS by direct loads into one ring of
 * HL_NS stages of a 64-wide K chunk (W: 64 rows x 128 B; x: 64 rows x 128 B
 * per plane), two chunks ahead: every load of the loop belongs to the ring,
 * so no wait for an x chunk (an L2 hit) also waits for weight loads issued
 * before it, as the register staging of fp32 x did (vector memory counts
 * complete in order; measured 0.75 us per chunk at q_proj + kv_a_proj,
 * B = 64).  Wave w owns token rows 16 w .. + 15 and the block's 64 columns
 * (4 x 16-column MFMA tiles).  LDS rows are 128 B of 8 pieces; piece p of
 * row r sits in slot p ^ swz(r) (16 consecutive rows, one piece: 16
 * distinct bank groups).  Two blocks per CU. */
#define HL_NS 3
#define HL_WB (64 * 128)                 /* W bytes per stage */
#define HL_STAGE (HL_WB + 2 * 64 * 128)  /* + the x planes: 24 KB */
#define HL_LPW 6                         /* direct loads per wave per stage: 2 of W, 4 of x */

__device__ __forceinline__ int hl_swz(int r) { return (r >> 1) & 7; }

extern "C" __global__ __launch_bounds__(256) void mm_gemm_hl(mm_gemm_hl_args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[HL_NS * HL_STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    /* column block bx of matrix `seg` (the second one past nb0 blocks) */
    const bool seg = (int)blockIdx.x >= a.nb0;
    const int bx = seg ? blockIdx.x - a.nb0 : blockIdx.x;
    const int d_out = seg ? a.d_out1 : a.d_out;
    const uint16_t *wm = seg ? a.w1 : a.w;
    const int n0 = bx * 64, K = a.n_in, T = a.T, q = lane & 7;
    const int kb = blockIdx.y * a.kr;
    const int nch = (min(K, kb + a.kr) - kb) / 64;      /* 64-input chunks of this split */

    /* direct loads of a chunk: W instruction 2 wave + u covers weight rows
     * (output columns) 8 (2 wave + u) .. + 7 of the block, x instruction
     * 4 wave + u plane (4 wave + u) / 8, token rows 8 ((4 wave + u) % 8) ..
     * + 7; lane l loads row + l / 8, slot q = l % 8, i.e. piece q ^ swz(row).
     * Rows past d_out or T load the last one (not stored). */
    const uint16_t *wp[2], *xp[4];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int c = 8 * (2 * wave + u) + (lane >> 3);
        wp[u] = wm + (size_t)min(n0 + c, d_out - 1) * K + kb + 8 * (q ^ hl_swz(c));
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int i = 4 * wave + u, r = 8 * (i & 7) + (lane >> 3);
        xp[u] = a.xhl + (size_t)(i >> 3) * T * K + (size_t)min(r, T - 1) * K + kb + 8 * (q ^ hl_swz(r));
    }
    auto issue = [&](int c, int st) {
        uint8_t *sb = lds + st * HL_STAGE;
#pragma unroll
        for (int u = 0; u < 2; u++) lds_dma16(wp[u] + 64 * c, sb + (2 * wave + u) * 1024);
#pragma unroll
        for (int u = 0; u < 4; u++) lds_dma16(xp[u] + 64 * c, sb + HL_WB + (4 * wave + u) * 1024);
    };
    /* operand reads (bytes within a stage), K half s: A row 16 wave + l % 16,
     * B row (column) 16 j + l % 16, piece 4 s + l / 16 */
    uint32_t ao[2], bo[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int p = 4 * s + (lane >> 4), r = 16 * wave + (lane & 15);
        ao[s] = HL_WB + r * 128 + 16 * (p ^ hl_swz(r));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = 16 * j + (lane & 15);
            bo[s][j] = c * 128 + 16 * (p ^ hl_swz(c));
        }
    }
    f32x4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t l0 = lds_addr(lds);
    issue(0, 0);
    if (nch > 1) issue(1, 1);
    for (int c = 0; c < nch; c++) {
        /* chunk c landed (chunk c + 1's loads, issued after, may stay out);
         * the barrier shows every wave's loads of chunk c and frees the stage
         * of chunk c - 1 for chunk c + 2 */
        if (c + 1 < nch) VMCNT_WAIT(HL_LPW);
        else VMCNT_WAIT(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (c + 2 < nch) issue(c + 2, (c + 2) % HL_NS);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t sb = l0 + (uint32_t)((c % HL_NS) * HL_STAGE);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            i32x4 xa[2], wb[4];
            xa[0] = ds_read16(sb + ao[s]);
            xa[1] = ds_read16(sb + ao[s] + 64 * 128);
#pragma unroll
            for (int j = 0; j < 4; j++) wb[j] = ds_read16(sb + bo[s][j]);
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(xa[0]), "+v"(xa[1]), "+v"(wb[0]), "+v"(wb[1]), "+v"(wb[2]), "+v"(wb[3]));
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, xa[h]), __builtin_bit_cast(bf16x8, wb[j]), acc[j], 0, 0, 0);
        }
    }
    /* C[token 16 wave + 4 (l / 16) + i][column n0 + 16 j + l % 16] */
    float *part = a.part + (seg ? (size_t)a.nsplit * T * a.d_out : 0);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + 16 * j + (lane & 15);
        if (n >= d_out) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * wave + 4 * (lane >> 4) + i;
            if (t >= T) continue;
            if (a.nsplit > 1 || a.part_out) {
                part[((size_t)blockIdx.y * T + t) * d_out + n] = acc[j][i];
            } else {
                float *y = (seg ? a.y1 : a.y) + (size_t)t * d_out + n;
                *y = a.accumulate ? *y + acc[j][i] : acc[j][i];
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void mm_skinny_reduce(mm_skinny_reduce_args a) {
    const size_t n0 = (size_t)a.T * a.d_out, n1 = a.y1 ? (size_t)a.T * a.d_out1 : 0;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < n0 + n1;
         k += (size_t)gridDim.x * blockDim.x) {
        const bool seg = k >= n0;
        const size_t n = seg ? n1 : n0, i = seg ? k - n0 : k;
        const float *part = a.part + (seg ? (size_t)a.nsplit * n0 : 0);
        float *y = seg ? a.y1 : a.y;
        float v = part[i];
        for (int s = 1; s < a.nsplit; s++) v += part[(size_t)s * n + i];
        y[i] = a.accumulate ? y[i] + v : v;
    }
}
