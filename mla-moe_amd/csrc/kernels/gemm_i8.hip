/* gemm_i8.hip -- big-tile grouped int8 GEMM for the prefill MoE FFN on
 * v_mfma_i32_32x32x32_i8 (int32 accumulation).
 *
 * The prefill-sized counterpart of mm_i8_gu / mm_i8_down (moe_i8.hip): for
 * each routed expert (and the shared expert as one dense GEMM, in the same
 * launch) and each of its rows, out[rid] = dequant(qa[row] . qW^T), with the
 * SwiGLU epilogue for gate/up; the weights are the packed 16-column x 64-K
 * fragments of kernel_params.h.
 *
 * Block tile MM_I8B_BM = 128 rows x MM_I8B_FR = 16 fragments (gate/up: the
 * gate and up fragments of 8 column blocks, 128 output columns; plain: 256
 * output columns), K step 64 bytes.  The four waves split the columns: wave
 * w owns all 128 rows and fragments 4 w .. 4 w + 3, i.e. four 32-row blocks
 * x two 32-column MFMA tiles (gate/up: the gate and the up tile of one
 * 32-column pair), 8 accumulators of 16 registers.
 *
 * The 32x32x32 MFMA is used because it keeps the pipe 85-90% busy at one or
 * two waves per SIMD, where the 16x16x64 form is limited by issue to 58-75%
 * (measured on MI355X).  Two blocks share a CU, so one block's set-up, load
 * latency and epilogue overlap the other's MFMAs.
 *
 * Data path: the A rows go global -> LDS by direct loads in stages of
 * BT_KB = 128 bytes of K per row (16 KB: whole cache lines of every row,
 * 16-byte chunks XOR-swizzled by row), two LDS slots, read by all four
 * waves; each wave loads its own B operands (4 KB per 64-byte K step)
 * straight into registers, as the decode GEMMs do, through a ring of BT_NSB
 * slots two steps ahead.  A tile's head (its first two A stages and B
 * steps) goes out before the previous tile's stores; the output tile is
 * restaged through LDS so that the stores are whole 128-byte lines.
 *
 * Waits: only the hand-counted partial vmcnt waits order the ring.  The
 * compiler adds a wait for every load and store in flight wherever a load
 * was issued under a condition, a branch joins a value still being loaded,
 * a register still being loaded is copied, or an LDS read follows a
 * direct-to-LDS load it knows of.  So the loads of whole K turns and of
 * every head are unconditional (clamped indices past a tile's end), the A
 * stages are assembly, the tile metadata loads are issued by every thread
 * and used only after the K loop, and the first tile and first K turn are
 * copies of their own (their entry follows a different history of loads).
 *
 * A 32x32x32 B operand (lane l: column l % 32, K bytes 16 (l / 32) .. + 15)
 * is one 16-byte load per lane
 * out of two packed 16x64 fragments: the 16 bytes of (column c, K chunk q)
 * sit at byte (16 q + c % 16) * 16 of fragment c / 16.  Measured on MI355X
 * against staging both operands in LDS (which costs each wave 12 LDS reads
 * per stage instead of 8): gate/up 10-15% faster at config 3's skewed
 * routing; with its MFMAs, A loads or B loads switched off in a test build,
 * the kernel is bound by the loads a CU can take in from L2, not by MFMA
 * issue or load latency (a deeper ring changes nothing).
 *
 * MFMA 32x32x32 i8 layout: src0 lane l = row l % 32, K bytes 16 (l / 32) .. + 15;
 * src1 likewise by column; result register 4 g + i of lane l is row
 * 8 g + 4 (l / 32) + i, column l % 32.  The weights go in as src0 and the
 * activation rows as src1, so the result is the output tile transposed:
 * lane l holds activation row l % 32 and, in registers 4 g .. 4 g + 3, four
 * consecutive output columns 8 g + 4 (l / 32) .. + 3, which the epilogue
 * writes to its LDS staging tile as one 16-byte write (a quarter of the
 * writes of the other operand order, whose lanes hold one column of four
 * rows).
 */
#include <type_traits>

#include "i8_tile.h"

typedef int32_t v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32_i8(i32x4 a, i32x4 b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

#define BT_KB 128                /* K bytes per A stage: whole 128-byte lines of every A row */
#define BT_A_BYTES (MM_I8B_BM * BT_KB)
#define BT_NSA 2                 /* A ring (LDS): one stage in flight, one consumed */
#define BT_NSB 3                 /* B ring (registers): 64-byte K steps, two in flight */
#define BT_LB 4                  /* B loads per wave per 64-byte K step */
#define BT_NST_GU 16             /* epilogue stores per wave: gate/up, plain */
#define BT_NST_PLAIN 32
static_assert(MM_I8B_BM == 128 && MM_I8B_FR == 16, "block tile shape is fixed by the wave grid");

/* s_waitcnt vmcnt(n) for a wave-uniform n, a multiple of 4 below 64 (the
 * instruction takes the count as an immediate) */
__device__ __forceinline__ void vmcnt_wait_rt(int n) {
    switch (__builtin_amdgcn_readfirstlane(n) >> 2) {
    case 0: VMCNT_WAIT(0); break;
    case 1: VMCNT_WAIT(4); break;
    case 2: VMCNT_WAIT(8); break;
    case 3: VMCNT_WAIT(12); break;
    case 4: VMCNT_WAIT(16); break;
    case 5: VMCNT_WAIT(20); break;
    case 6: VMCNT_WAIT(24); break;
    case 7: VMCNT_WAIT(28); break;
    case 8: VMCNT_WAIT(32); break;
    case 9: VMCNT_WAIT(36); break;
    case 10: VMCNT_WAIT(40); break;
    case 11: VMCNT_WAIT(44); break;
    default: VMCNT_WAIT(0); break;
    }
}

/* Epilogue staging: per wave one 32 x 32 fp32 tile, rows of BT_EP_LD floats */
#define BT_EP_LD 36

/* ds_write_b128 of an f32x4 at an LDS byte address, and the wait for the
 * wave's outstanding LDS operations (the staging round trip is one wave's
 * own rows: no barrier).  No memory clobber: they serve the epilogue's
 * staging rows only, which only assembly reads (volatile, so kept in order
 * with these); with a clobber the compiler would read every LDS value it
 * uses (scales, row ids) again after each of them. */
__device__ __forceinline__ void ds_write16(uint32_t addr, f32x4 v) {
    asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v));
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)"); }

/* registers 4 g .. 4 g + 3 of an accumulator */
__device__ __forceinline__ i32x4 acc4(const v16i &c, int g) {
    return (i32x4){c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]};
}

/* position of 16-byte chunk q of staged A row R (128 bytes per row): q ^ swz128(R).
 * A ds_read_b128 serves 16 lanes per cycle: rows R .. R + 15 at one chunk q
 * then fall on 16 distinct 16-byte bank groups (the row's parity picks the
 * half of the 256-byte bank space, swz128 the group within it). */
__device__ __forceinline__ int swz128(int R) { return (R >> 1) & 7; }

/* s_waitcnt lgkmcnt(0), tied to the operand registers it makes valid */
template <int N>
__device__ __forceinline__ void lds_wait_regs(i32x4 (&A)[N]) {
    if constexpr (N == 1) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(A[0]));
    if constexpr (N == 2) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(A[0]), "+v"(A[1]));
    if constexpr (N == 3) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]));
    if constexpr (N == 4)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]));
}

/* ds_read_b32 at addr + off (a constant), as inline assembly: the caller
 * waits (lgkmcnt) before using the result */
__device__ __forceinline__ int ds_read4(uint32_t addr, int off) {
    int r;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off));
    return r;
}

/* A wave-uniform pointer held in scalar registers. */
template <class P>
__device__ __forceinline__ P *uniform_ptr(P *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (P *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

/* Per-block schedule and row tables in LDS. */
struct bt_shared {
    int gstart[MM_EMAX + 1];                 /* segment 0: exclusive prefix of 128-row groups */
    int cnt[MM_EMAX];                        /* segment 0: rows of each expert (<= T) */
    int g1;                                  /* segment 1 (one expert): its row groups */
    int m1;                                  /* segment 1: its rows */
    int n0, n;                               /* tiles of segment 0, of both */
    int arow[2][MM_I8B_BM];                  /* A row of each tile row (two tiles in flight) */
    __attribute__((aligned(16))) int rid[2][MM_I8B_BM];     /* output row id, -1 = padding */
    __attribute__((aligned(16))) float sa[2][MM_I8B_BM];    /* A row scale */
    /* column scales of the slab: gate/up [gate 128 | up 128], plain 256 */
    __attribute__((aligned(16))) float cs[2][2 * MM_I8B_BM];
};

/* A tile of the grouped GEMM: segment si, expert e, column slab, rows
 * m0 .. m0 + 127 of the expert's M rows. */
struct bt_tile_id {
    int si, e, slab, m0, M;
};

__device__ __forceinline__ int bt_nslab(const mm_i8_tiled_args &g) {
    return ((g.gu ? 2 : 1) * (g.N / 16) + MM_I8B_FR - 1) / MM_I8B_FR;
}

/* Tiles are ordered (segment, expert, slab, row group): expert e of
 * segment 0 owns tiles [nslab gstart[e], nslab gstart[e + 1]); segment 1
 * follows.  Uniform over the block (made explicit, so that the segment's
 * fields are scalar loads).  Reads LDS only: no global load here whose
 * wait would also wait for the stores and loads in flight. */
__device__ __forceinline__ bt_tile_id bt_decode(const mm_i8_bt_args &a, const bt_shared &sh,
                                                int t) {
    bt_tile_id id;
    if (t < sh.n0) {
        const mm_i8_tiled_args &g = a.seg[0];
        const int nslab = bt_nslab(g);
        int lo = 0, hi = g.cnt ? g.E : 1;    /* largest e with nslab * gstart[e] <= t */
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (nslab * sh.gstart[mid] <= t) lo = mid; else hi = mid;
        }
        const int ge = sh.gstart[lo + 1] - sh.gstart[lo];
        const int loc = t - nslab * sh.gstart[lo];
        id.si = 0;
        id.e = lo;
        id.slab = loc / ge;
        id.m0 = (loc % ge) * MM_I8B_BM;
        id.M = sh.cnt[lo];
    } else {
        const int loc = t - sh.n0;
        id.si = 1;
        id.e = 0;
        id.slab = loc / sh.g1;
        id.m0 = (loc % sh.g1) * MM_I8B_BM;
        id.M = sh.m1;
    }
    id.si = __builtin_amdgcn_readfirstlane(id.si);
    id.e = __builtin_amdgcn_readfirstlane(id.e);
    id.slab = __builtin_amdgcn_readfirstlane(id.slab);
    id.m0 = __builtin_amdgcn_readfirstlane(id.m0);
    id.M = __builtin_amdgcn_readfirstlane(id.M);
    return id;
}

/* Row id and A row of tile row `r` (r < 128) in two parts: the load (always
 * issued, from the scale array where the segment has no row list, so that
 * no branch joins a value still in flight) and, where the value is used,
 * the ids. */
__device__ __forceinline__ int bt_row_load(const mm_i8_tiled_args &g, const bt_tile_id &id, int r) {
    const int m = id.m0 + r < id.M ? id.m0 + r : id.m0;
    const int *p = g.rows ? g.rows + (size_t)id.e * g.T + m : (const int *)g.sa;
    return *p;
}
__device__ __forceinline__ void bt_row_ids(const mm_i8_tiled_args &g, const bt_tile_id &id, int r,
                                           int raw, int *rid, int *arow) {
    const int m = id.m0 + r < id.M ? id.m0 + r : id.m0;
    const int q = g.rows ? raw : m;
    *arow = (g.a_by_route || !g.rows) ? q : q / g.K;
    *rid = id.m0 + r < id.M ? q : -1;
}

/* The tiles of one XCD: its eighth of segment 0 followed by its eighth of
 * segment 1; local index t -> global tile index. */
struct bt_xcd_list {
    int lo0, len0, lo1, len;
    __device__ int operator()(int t) const { return t < len0 ? lo0 + t : lo1 + (t - len0); }
};

template <bool GU, bool DBG>
__device__ __forceinline__ void bt_run(const mm_i8_bt_args &a, int8_t *lds, float *ep, bt_shared &sh,
                                       const bt_xcd_list &xl, int t, int t_step) {
    const int t_end = xl.len;
    const int tid = threadIdx.x, lane = tid & (MM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / MM_WAVE);
    const int l32 = lane & 31, hi = lane >> 5;
    const uint32_t lds0 = lds_addr(lds);
    constexpr int NT = GU ? 1 : 2;          /* output column tiles of 32 per wave */

    /* ---- load parameters of the tile whose stages are being issued ----
     * K advances in 64-byte steps h (one packed fragment of every column
     * block); A is staged 128 bytes of K at a time (stage s = steps 2 s,
     * 2 s + 1), so that every A load covers whole 128-byte cache lines.
     * A (DMA into LDS): wave w issues instructions 4 w .. 4 w + 3 of a stage
     * (8 rows x 128 B each); lane l carries row R = 8 i + l / 8 and stores at
     * position l % 8 of the row's 128 B the chunk (l % 8) ^ swz128(R).  With
     * an odd number of steps the last stage is half a stage: its A loads
     * re-read the row's first 64 bytes (within the row; never multiplied).
     * B (into registers): column tile cj, K half ks of step h: lane l reads
     * column l % 32 of the tile, K chunk 2 ks + l / 32: the 16 bytes at
     * (16 (2 ks + l / 32) + l % 16) * 16 of the tile's fragment (l % 32) / 16
     * for K block h.  gate/up: the wave's column blocks are 2 w, 2 w + 1 of
     * the slab; tile 0 is their gate fragments, tile 1 their up fragments.
     * plain: column blocks 4 w .. 4 w + 3, tile cj = blocks 4 w + 2 cj, + 1.
     * Column blocks past the last are clamped (results not stored). */
    uint32_t arow_off[4];
    int aq[4];
    __amdgpu_buffer_rsrc_t brs;
    rsrc_t ars;
    uint32_t boff[2];
    int lkb, bstep;
    auto set_tile = [&](const bt_tile_id &id, int buf) {
        const mm_i8_tiled_args &g = a.seg[id.si];
        lkb = g.Kd / 64;
        /* A rows past the tile's valid rows: an offset past the range (no
         * memory read, zeros staged; their results are not stored) */
        ars = raw_rsrc(g.a, MM_I8_TILED_A_MAX);
        const int vrows = min(id.M - id.m0, MM_I8B_BM);
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const int R = 8 * (4 * wave + h) + (lane >> 3);
            arow_off[h] = R < vrows ? (uint32_t)sh.arow[buf][R] * (uint32_t)g.Kd : MM_I8_TILED_A_MAX;
            aq[h] = (lane & 7) ^ swz128(R);
        }
        const int ncb = g.N / 16;
        const uint32_t in_frag = (uint32_t)((16 * hi + (lane & 15)) * 16);
#pragma unroll
        for (int cj = 0; cj < 2; cj++) {
            if (GU) {
                const int cb = min(id.slab * 8 + 2 * wave + (l32 >> 4), ncb - 1);
                boff[cj] = (uint32_t)((cb * 2 * lkb + cj) * 1024) + in_frag;
            } else {
                const int cb = min(id.slab * 16 + 4 * wave + 2 * cj + (l32 >> 4), ncb - 1);
                boff[cj] = (uint32_t)(cb * lkb * 1024) + in_frag;
            }
        }
        bstep = GU ? 2048 : 1024;
        brs = __builtin_amdgcn_make_buffer_rsrc((void *)(g.b + (size_t)id.e * g.b_expert_stride), 0,
                                                (int)((uint32_t)((GU ? 2 : 1) * ncb * lkb) * 1024u),
                                                0x00020000);
    };
    /* B operands of the ring slots: [slot][column tile][K half] */
    i32x4 bq[BT_NSB][2][2];
    auto issue_a = [&](int s, int slot) {
        const uint32_t st = (uint32_t)(slot * BT_A_BYTES);
        const bool full = 2 * s + 1 < lkb;
#pragma unroll
        for (int h = 0; h < 4; h++)
            lds_dma16_buf(arow_off[h] + (uint32_t)(s * BT_KB + 16 * (full ? aq[h] : aq[h] & 3)), ars,
                          lds0 + st + (uint32_t)((4 * wave + h) * 1024));
    };
    auto issue_b = [&](int slot, int h) {
        const int so = __builtin_amdgcn_readfirstlane(h * bstep);
#pragma unroll
        for (int cj = 0; cj < 2; cj++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
                bq[slot][cj][ks] = __builtin_bit_cast(
                    i32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, boff[cj] + 512 * ks, so, 0));
    };

    /* a tile's head: its first two A stages and first two B steps, issued
     * before the previous tile's epilogue stores so that the tile's first
     * two steps wait for none of those stores.  Always four groups of loads
     * (a tile of one K step re-reads B(0) into slot 1, one of at most two
     * steps A(0) into slot 1, neither read by the tile): loads under a
     * condition would leave the ring registers defined on some paths only,
     * and the compiler's copies at the join wait for every load in flight. */
    auto issue_head = [&]() {
        issue_a(0, 0);
        issue_b(0, 0);
        issue_b(1, min(1, lkb - 1));
        issue_a(min(1, (lkb - 1) >> 1), 1);
    };

    /* A operand of row block ri, K step h, half ks: row 32 ri + l % 32,
     * chunk 4 (h % 2) + 2 ks + l / 32 of the stage (the swizzle depends on
     * l % 32 only) */
    uint32_t rdA[4];
#pragma unroll
    for (int c = 0; c < 4; c++) rdA[c] = l32 * BT_KB + 16 * ((2 * c + hi) ^ swz128(l32));

    /* ---- first tile ---- */
    bt_tile_id cur = bt_decode(a, sh, xl(t));
    int buf = 0;
    if (tid < MM_I8B_BM) {
        int rid, arow;
        bt_row_ids(a.seg[cur.si], cur, tid, bt_row_load(a.seg[cur.si], cur, tid), &rid, &arow);
        sh.rid[0][tid] = rid;
        sh.arow[0][tid] = arow;
    }
    __syncthreads();
    set_tile(cur, 0);
    issue_head();

    /* one tile: K loop, then the next tile's head and this tile's epilogue;
     * false after the last.  The first tile is a copy of its own (FIRST: no
     * epilogue stores follow its head), so that every entry into the
     * loop's copy comes after the same loads and stores and the compiler's
     * own wait counts there stay exact. */
    auto tile = [&](auto first_c) -> bool {
        constexpr bool FIRST = decltype(first_c)::value;
        const mm_i8_tiled_args &g = a.seg[cur.si];
        const int tn = t + t_step;
        const bool has_next = tn < t_end;
        const bt_tile_id nxt = has_next ? bt_decode(a, sh, xl(tn)) : cur;

        /* loads whose results are used after the K loop: this tile's row
         * scales and column scales (thread tid: slab column tid, gate/up:
         * gate column tid or up column tid - 128), the next tile's row ids.
         * Every thread issues them (tile row clamped to 127) and the values
         * are first used after the K loop: the first use of a load, or a
         * branch joining its value, is where the compiler waits for it, and
         * that wait would also take the previous tile's stores and this
         * tile's head. */
        const int trow = min(tid, MM_I8B_BM - 1);
        const float sa_r = g.sa[sh.arow[buf][trow]];
        const int nraw = bt_row_load(a.seg[nxt.si], nxt, trow);
        const int N = g.N;
        const int slab_c0 = cur.slab * (GU ? 128 : 256);   /* first output column of the slab */
        float cs_r;
        {
            /* both pointers in scalar registers before the per-thread choice
             * (else the choice is made on the fields' addresses: a divergent
             * load of the pointer, then a dependent load) */
            const float *sb = (GU && tid >= 128 ? uniform_ptr(g.sb1) : uniform_ptr(g.sb0)) +
                              (size_t)cur.e * g.sb_expert_stride;
            cs_r = ((const __attribute__((address_space(1))) float *)sb)[min(slab_c0 + (GU ? (tid & 127) : tid), N - 1)];
        }

        /* ---- K loop ---- */
        v16i acc[4][2];
#pragma unroll
        for (int ri = 0; ri < 4; ri++)
#pragma unroll
            for (int cj = 0; cj < 2; cj++) acc[ri][cj] = (v16i){};
        /* One form of the loop for every tile: 32-row blocks made only of
         * padding (A rows staged as zeros without a memory read, results to
         * the spare row) skip their MFMAs by a uniform branch.  With a form
         * per row-block count the compiler copies the head's ring registers
         * on entry, and a copy of a register still being loaded waits for
         * every load and store in flight. */
        const int nri = __builtin_amdgcn_readfirstlane((min(cur.M - cur.m0, MM_I8B_BM) + 31) >> 5);
        /* step h (64 bytes of K): A stage s = h / 2 in LDS slot s % 2, B in
         * register slot h % 3.  Loads are issued in this order: the tile's
         * head A(0), B(0), B(1), A(1), B(2); then at each even step 2 s >= 2,
         * after its wait and barrier, A(s + 1) and B(2 s + 2); at each odd
         * step h, B(h + 2).  The vmcnt counter completes in issue order, so a
         * step waits until only the operations issued after the loads it
         * needs are outstanding: even step 2 s >= 2 needs A(s) and B(2 s),
         * after which only B(2 s + 1) was issued (BT_LB loads); odd step
         * 2 s + 1 >= 3 needs B(2 s + 1), after which A(s + 1) and B(2 s + 2)
         * were issued (2 BT_LB).  The tile's head is A(0), B(0), B(1), A(1),
         * followed on a later tile by the previous tile's epilogue stores
         * (exactly NST per wave); step 0 issues B(2) (and, in a whole turn,
         * A(1) again).  Steps 0 and 1 need head loads issued before the
         * stores, which may stay outstanding until step 2.  Near the end of
         * the tile
         * fewer loads follow, and the counts shrink accordingly (0: wait for
         * all).  The barrier of an even step makes every wave's A rows of
         * stage s visible and frees slot (s + 1) % 2, read by every wave
         * during steps 2 s - 2 and 2 s - 1 (or by the previous tile). */
        constexpr int NST = GU ? BT_NST_GU : BT_NST_PLAIN;
        constexpr int NSTF = FIRST ? 0 : NST;   /* stores issued after the head */
        auto kloop = [&](auto nri_c) {
            constexpr int NRI = decltype(nri_c)::value;
            /* FULL: a step of a whole turn of 6 (h0 + 6 <= lkb), whose
             * loads are issued unconditionally.  A load under a condition is
             * a branch, and the compiler then waits for every outstanding
             * load (vmcnt(0)) before the next MFMAs, draining the B ring at
             * each step.  In a whole turn: step 0 of the tile re-issues A(1)
             * (same bytes into the same slot as the head's, read from step 2
             * on), and near the tile's end B and A are issued at clamped
             * indices (a B step into the free register slot, an A stage into
             * the LDS slot that no later step of the tile reads; the tile ends
             * with vmcnt(0) before the next head).  Extra later loads only
             * make a hand-counted wait stricter, except at step 1, whose
             * count includes the re-issued A(1). */
            auto kstep = [&](auto d_c, int h, auto full_c, auto ft_c) {
                constexpr int D = decltype(d_c)::value;     /* h % 6 */
                constexpr bool FULL = decltype(full_c)::value;
                constexpr bool FT = decltype(ft_c)::value;  /* the tile's first whole turn */
                constexpr int J = D & 1, SB = D % BT_NSB;
                const int sa_slot = (h >> 1) & 1;
                const bool more = h + 1 < lkb;
                if (FULL) {
                    if (FT && D == 0) VMCNT_WAIT(2 * BT_LB + NSTF);
                    else if (FT && D == 1) VMCNT_WAIT(3 * BT_LB + NSTF);
                    else if (J == 0) VMCNT_WAIT(BT_LB);
                    else VMCNT_WAIT(2 * BT_LB);
                } else if (D == 0 && h == 0) {
                    VMCNT_WAIT(2 * BT_LB + NSTF);
                } else if (D == 1 && h == 1) {
                    vmcnt_wait_rt(BT_LB + BT_LB * (lkb > 2) + NSTF);
                } else if (J == 0) {
                    if (more) VMCNT_WAIT(BT_LB); else VMCNT_WAIT(0);
                } else {
                    if (more) VMCNT_WAIT(2 * BT_LB); else VMCNT_WAIT(0);
                }
                if (J == 0) __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if (FULL) {
                    if (J == 0) issue_a(min((h >> 1) + 1, (lkb - 1) >> 1), sa_slot ^ 1);
                    issue_b((D + 2) % BT_NSB, min(h + 2, lkb - 1));
                } else {
                    /* A(1) is part of the head */
                    if (J == 0 && h > 0 && h + 2 < lkb) issue_a((h >> 1) + 1, sa_slot ^ 1);
                    if (h + 2 < lkb) issue_b((D + 2) % BT_NSB, h + 2);
                }
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t sb = lds0 + (uint32_t)(sa_slot * BT_A_BYTES);
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    i32x4 A[NRI];
#pragma unroll
                    for (int ri = 0; ri < NRI; ri++)
                        A[ri] = ds_read16(sb + rdA[2 * J + ks], ri * 32 * BT_KB);
                    lds_wait_regs(A);
#pragma unroll
                    for (int ri = 0; ri < NRI; ri++)
                        if (ri == 0 || ri < nri)   /* uniform: padding-only blocks skip */
#pragma unroll
                            for (int cj = 0; cj < 2; cj++)
                                acc[ri][cj] = mfma32_i8(bq[SB][cj][ks], A[ri], acc[ri][cj]);
                }
            };
            using std::integral_constant;
            using T_ = std::true_type;
            using F_ = std::false_type;
            /* the first whole turn is a copy of its own (its waits count the
             * head and the stores after it), so that every entry into the
             * turn loop follows a whole turn and the compiler's own counts
             * there stay exact */
            auto turn = [&](int h0, auto ft_c) {
                kstep(integral_constant<int, 0>(), h0, T_(), ft_c);
                kstep(integral_constant<int, 1>(), h0 + 1, T_(), ft_c);
                kstep(integral_constant<int, 2>(), h0 + 2, T_(), ft_c);
                kstep(integral_constant<int, 3>(), h0 + 3, T_(), ft_c);
                kstep(integral_constant<int, 4>(), h0 + 4, T_(), ft_c);
                kstep(integral_constant<int, 5>(), h0 + 5, T_(), ft_c);
            };
            int h0 = 0;
            if (lkb >= 6) {
                turn(0, T_());
                for (h0 = 6; h0 + 6 <= lkb; h0 += 6) turn(h0, F_());
            }
            if (h0 < lkb) kstep(integral_constant<int, 0>(), h0, F_(), F_());
            if (h0 + 1 < lkb) kstep(integral_constant<int, 1>(), h0 + 1, F_(), F_());
            if (h0 + 2 < lkb) kstep(integral_constant<int, 2>(), h0 + 2, F_(), F_());
            if (h0 + 3 < lkb) kstep(integral_constant<int, 3>(), h0 + 3, F_(), F_());
            if (h0 + 4 < lkb) kstep(integral_constant<int, 4>(), h0 + 4, F_(), F_());
        };
        kloop(std::integral_constant<int, 4>());
        VMCNT_WAIT(0);

        /* row tables: this tile's scales, the next tile's rows */
        if (tid < MM_I8B_BM) {
            int nrid = -1, narow = 0;
            if (has_next) bt_row_ids(a.seg[nxt.si], nxt, tid, nraw, &nrid, &narow);
            sh.sa[buf][tid] = sa_r;
            sh.rid[buf ^ 1][tid] = nrid;
            sh.arow[buf ^ 1][tid] = narow;
        }
        sh.cs[buf][tid] = cs_r;
        __syncthreads();
        /* the next tile's head goes out before this tile's stores (its third
         * B step after them); after the last tile a head of this tile again
         * (nxt == cur, row 0 of the segment for every row: valid addresses
         * into LDS slots and registers nothing reads, waited for at the end),
         * so that the head's loads are never under a condition */
        set_tile(nxt, buf ^ 1);
        issue_head();

        /* ---- epilogue ----
         * accumulator register 4 g + i of lane l is row 32 ri + l % 32,
         * column 8 g + 4 (l / 32) + i of the wave's 32-column tile q
         * (gate/up: slab columns 32 w .., tile 0 gate, tile 1 up, one output
         * tile; plain: slab columns 64 w + 32 q ..).  Each 32 x 32 output
         * tile goes through the wave's own LDS staging rows (row stride 36
         * floats: both access patterns below are free of bank conflicts
         * but for one pair of lanes), written as the MFMA left it and read
         * back row-major, so that each 16-byte store instruction writes 8
         * whole 128-byte rows instead of 32-byte pieces of 32 rows (L2
         * requests, not bytes, bound this kernel).  Stores are unconditional
         * (exactly NST per wave): padded rows and columns past N go to the
         * spare row of `out`. */
        float *out = g.out;
        const size_t spare = (size_t)g.spare_row * N;
        float *stg = ep + wave * (32 * BT_EP_LD);
        const uint32_t stg_w = lds_addr(stg) + (uint32_t)(l32 * BT_EP_LD + 4 * hi) * 4;
        const int er = lane >> 3, ec = 4 * (lane & 7);      /* read back: row er + 8 k, columns ec .. */
        const uint32_t stg_r = lds_addr(stg) + (uint32_t)(er * BT_EP_LD + ec) * 4;
        {
            int32_t *dbg = g.dbg_acc;
            /* the output rows: assembly reads beside the staging reads,
             * under one wait */
            const uint32_t rid_r = lds_addr(&sh.rid[buf][er]);
#pragma unroll
            for (int ri = 0; ri < 4; ri++) {
                const float sa = sh.sa[buf][32 * ri + l32];
#pragma unroll
                for (int q = 0; q < NT; q++) {
                    const int ct = (GU ? 32 * wave : 64 * wave + 32 * q);   /* tile's first slab column */
#pragma unroll
                    for (int gq = 0; gq < 4; gq++) {
                        const int cl = ct + 8 * gq + 4 * hi;
                        const f32x4 c0 = *(const f32x4 *)(&sh.cs[buf][cl]);
                        f32x4 v;
                        if (GU) {
                            const f32x4 c1 = *(const f32x4 *)(&sh.cs[buf][128 + cl]);
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                v[i] = silu_mul_fast(((float)acc[ri][0][4 * gq + i] * sa) * c0[i],
                                                     ((float)acc[ri][1][4 * gq + i] * sa) * c1[i]);
                            if (DBG && dbg) {
                                const int rid = sh.rid[buf][32 * ri + l32], col = slab_c0 + cl;
                                if (rid >= 0 && col < N) {
                                    int32_t *d = dbg + ((size_t)rid * 2) * N + col;
                                    *(i32x4 *)d = acc4(acc[ri][0], gq);
                                    *(i32x4 *)(d + N) = acc4(acc[ri][1], gq);
                                }
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; i++) v[i] = ((float)acc[ri][q][4 * gq + i] * sa) * c0[i];
                            if (DBG && dbg) {
                                const int rid = sh.rid[buf][32 * ri + l32], col = slab_c0 + cl;
                                if (rid >= 0 && col < N)
                                    *(i32x4 *)(dbg + (size_t)rid * N + col) = acc4(acc[ri][q], gq);
                            }
                        }
                        ds_write16(stg_w + 32 * gq, v);
                    }
                    lds_wait();
                    i32x4 rv[4];
                    int ridk[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) rv[k] = ds_read16(stg_r, 8 * k * BT_EP_LD * 4);
#pragma unroll
                    for (int k = 0; k < 4; k++) ridk[k] = ds_read4(rid_r, (32 * ri + 8 * k) * 4);
                    asm volatile("s_waitcnt lgkmcnt(0)"
                                 : "+v"(rv[0]), "+v"(rv[1]), "+v"(rv[2]), "+v"(rv[3]), "+v"(ridk[0]),
                                   "+v"(ridk[1]), "+v"(ridk[2]), "+v"(ridk[3]));
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const f32x4 v = __builtin_bit_cast(f32x4, rv[k]);
                        const int rid = ridk[k];
                        const int col = slab_c0 + ct + ec;
                        const bool ok = rid >= 0 && col < N;
                        *(f32x4 *)(out + (ok ? (size_t)rid * N + col : spare + col)) = v;
                    }
                    lds_wait();
                }
            }
        }
        if (!has_next) return false;
        t = tn;
        cur = nxt;
        buf ^= 1;
        return true;
    };
    if (tile(std::true_type{}))
        while (tile(std::false_type{})) {
        }
    VMCNT_WAIT(0);
}

/* Persistent grid of 2 blocks per CU (the host launches a multiple of 8).
 * Blocks are dealt to the 8 XCDs round robin (block b runs on XCD b % 8);
 * XCD x owns the x-th eighth of each segment's tile list and its blocks take
 * those tiles in turn, so the blocks of one XCD work on neighbouring tiles at
 * the same time: row groups of the same expert and slab, whose weights then
 * come from HBM once and from that XCD's L2 for the others. */
template <bool GU, bool DBG>
__device__ __forceinline__ void bt_kernel(const mm_i8_bt_args &a) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[BT_NSA * BT_A_BYTES];
    __shared__ __attribute__((aligned(16))) float ep[4 * 32 * BT_EP_LD];
    __shared__ bt_shared sh;
    const mm_i8_tiled_args &g0 = a.seg[0];
    const int E = g0.cnt ? g0.E : 1;
    /* segment 0: exclusive prefix of row groups per expert (wave 0) */
    if (threadIdx.x < MM_WAVE) {
        const int lane = threadIdx.x;
        int base = 0;
        for (int e0 = 0; e0 < E; e0 += MM_WAVE) {
            const int e = e0 + lane;
            const int M = e < E ? (g0.cnt ? min(g0.cnt[e * MM_CNT_STRIDE], g0.T) : g0.T) : 0;
            const int nt = (M + MM_I8B_BM - 1) / MM_I8B_BM;
            if (e < E) sh.cnt[e] = M;
            int incl = nt;
#pragma unroll
            for (int off = 1; off < MM_WAVE; off <<= 1) {
                const int v = __shfl_up(incl, off, MM_WAVE);
                if (lane >= off) incl += v;
            }
            if (e < E) sh.gstart[e] = base + incl - nt;
            base += __shfl(incl, MM_WAVE - 1, MM_WAVE);
        }
        if (lane == 0) {
            sh.gstart[E] = base;
            sh.n0 = base * bt_nslab(g0);
            sh.g1 = a.nseg > 1 ? (a.seg[1].T + MM_I8B_BM - 1) / MM_I8B_BM : 0;
            sh.m1 = a.nseg > 1 ? a.seg[1].T : 0;
            sh.n = sh.n0 + (a.nseg > 1 ? sh.g1 * bt_nslab(a.seg[1]) : 0);
        }
    }
    __syncthreads();
    /* XCD x takes the x-th eighth of each segment's tiles */
    const int n0 = sh.n0, n1 = sh.n - sh.n0;
    const int xcd = blockIdx.x % MM_I8S_XCD, j = blockIdx.x / MM_I8S_XCD;
    const int nbx = gridDim.x / MM_I8S_XCD;
    bt_xcd_list xl;
    xl.lo0 = n0 * xcd / MM_I8S_XCD;
    xl.len0 = n0 * (xcd + 1) / MM_I8S_XCD - xl.lo0;
    xl.lo1 = n0 + n1 * xcd / MM_I8S_XCD;
    xl.len = xl.len0 + n0 + n1 * (xcd + 1) / MM_I8S_XCD - xl.lo1;
    if (j >= xl.len) return;
    bt_run<GU, DBG>(a, lds, ep, sh, xl, j, nbx);
}

/* One kernel per epilogue form, so that each holds only its own code:
 * gate/up (SwiGLU, segments' gu = 1) and down (plain dequantisation). */
extern "C" __global__ __launch_bounds__(256, 2) void mm_i8_gemm_gu(mm_i8_bt_args a) {
    bt_kernel<true, false>(a);
}
extern "C" __global__ __launch_bounds__(256, 2) void mm_i8_gemm_dn(mm_i8_bt_args a) {
    bt_kernel<false, false>(a);
}

/* As mm_i8_gemm_gu / _dn, also writing the raw accumulators of each segment
 * whose dbg_acc is set (the shared segment's is not); debug entry points
 * only: kernels of their own keep these stores and their registers out of
 * the product kernels. */
extern "C" __global__ __launch_bounds__(256, 2) void mm_i8_gemm_gu_dbg(mm_i8_bt_args a) {
    bt_kernel<true, true>(a);
}
extern "C" __global__ __launch_bounds__(256, 2) void mm_i8_gemm_dn_dbg(mm_i8_bt_args a) {
    bt_kernel<false, true>(a);
}
