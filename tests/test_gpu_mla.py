"""GPU parity of the MLA absorbed decode (run.c:430-460, batched) against the
CPU oracle fed the same bf16 cache, up-converted exactly.

Bars: ctx, clat and the softmax weights within max-abs-rel 2e-3 (the score
and context products run on bf16 MFMA with fp32 accumulation, operands split
into bf16 hi/lo pairs); qabs within 1e-5 (fp32 FMA vs the sequential sum).
"""
import numpy as np
import pytest

import mlamoe
from conftest import load_golden, max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture
def ctx():
    c = mlamoe.Context(0)
    yield c
    c.close()


def run_case(ctx, oracle, NH, B, L, kv_len, seed, kv_lens=None, QKN=128, VHD=128):
    print(f"mla case NH={NH} B={B} L={L} kv_len={kv_len} lens={kv_lens}", flush=True)
    rng = np.random.default_rng(seed)
    KVL, QKR = 512, 64
    kv_b = synth.normal_bf16(rng, (NH * (QKN + VHD), KVL), 0.02)
    q = synth.normal_f32(rng, (B, NH, QKN + QKR))
    cache = synth.normal_bf16(rng, (B, L, KVL + QKR), 1.0)
    ctx.mla_init(NH, QKN, QKR, KVL, VHD)
    ctx.mla_load_layer(0, kv_b)
    got = ctx.mla_absorbed_decode(0, q, cache, kv_len, kv_lens)
    lens = kv_lens if kv_lens is not None else [kv_len] * B
    for b in range(B):
        n = int(lens[b])
        rc, rq, rp, rl = oracle.absorbed_decode(q[b:b + 1], kv_b, cache[b:b + 1, :n], n, NH, QKN,
                                                QKR, KVL, VHD)
        assert max_abs_rel(got[1][b], rq[0]) < 1e-5, ("qabs", b)
        assert max_abs_rel(got[2][b][:, :n], rp[0]) < TOL, ("probs", b)
        assert max_abs_rel(got[3][b], rl[0]) < TOL, ("clat", b)
        assert max_abs_rel(got[0][b], rc[0]) < TOL, ("ctx", b)
    return got


def test_mla_golden_dims(ctx, oracle):
    """The reference forward_absorbed's layer-0 case (real head dims,
    kv_len 41): GPU on the bf16-rounded cache vs the oracle on the same."""
    g = load_golden("absorbed.npz")
    NH, QKN, QKR, KVL, VHD, kv_len = (int(v) for v in g["dsv2_dims"])
    kv_b = synth.normal_bf16(np.random.default_rng(int(g["dsv2_kvb_seed"])),
                             (NH * (QKN + VHD), KVL), 0.02)
    assert synth.checksum_u16(kv_b) == int(g["dsv2_kvb_sum"])
    cache = synth.bf16_from_f32(g["dsv2_cache"])[None]
    q = g["dsv2_q"][None]
    ctx.mla_init(NH, QKN, QKR, KVL, VHD)
    ctx.mla_load_layer(0, kv_b)
    c, qa, p, cl = ctx.mla_absorbed_decode(0, q, cache, kv_len)
    rc, rq, rp, rl = oracle.absorbed_decode(q, kv_b, cache, kv_len, NH, QKN, QKR, KVL, VHD)
    assert max_abs_rel(qa, rq) < 1e-5
    # qabs does not depend on the cache: it also matches the reference dump
    assert max_abs_rel(qa[0], g["dsv2_qabs"]) < 1e-5
    assert max_abs_rel(p, rp) < TOL and max_abs_rel(cl, rl) < TOL and max_abs_rel(c, rc) < TOL
    # and the bf16 rounding of the one fp32 row keeps us near the fp32 reference
    assert max_abs_rel(c[0].reshape(NH, VHD), g["dsv2_ctx"]) < 1e-2


@pytest.mark.parametrize("kv_len", [1, 16, 37, 512, 777])
def test_mla_lengths(ctx, oracle, kv_len):
    run_case(ctx, oracle, 16, 2, max(kv_len, 1), kv_len, 600 + kv_len)


def test_mla_longest_context(ctx, oracle):
    """kv_len = 64 chunks x 512 keys (the last length whose chunks may still
    shrink for a small batch)."""
    run_case(ctx, oracle, 16, 1, 32768, 32768, 640)


@pytest.mark.parametrize("B,kv_len", [(2, 1), (2, 37), (2, 80), (64, 65), (64, 90)])
def test_mla_one_chunk_without_probs(ctx, oracle, B, kv_len):
    """Without the probabilities a context of one chunk (at most 1.5 of the
    small-grid chunk of 64 keys) has its attention block write clat: the
    same values as the merge's (bit for bit) and the oracle's."""
    got = run_case(ctx, oracle, 16, B, kv_len, kv_len, 700 + B + kv_len)
    rng = np.random.default_rng(700 + B + kv_len)
    KVL, QKR, QKN, VHD, NH = 512, 64, 128, 128, 16
    synth.normal_bf16(rng, (NH * (QKN + VHD), KVL), 0.02)
    q = synth.normal_f32(rng, (B, NH, QKN + QKR))
    cache = synth.normal_bf16(rng, (B, kv_len, KVL + QKR), 1.0)
    c2, _, p2, cl2 = ctx.mla_absorbed_decode(0, q, cache, kv_len, want_probs=False)
    assert p2 is None
    assert np.array_equal(cl2, got[3]) and np.array_equal(c2, got[0])


@pytest.mark.parametrize("kv_len", [32769, 163840])
def test_mla_beyond_64_chunks(ctx, oracle, kv_len):
    """Past 64 chunks the merge strides over up to 512 chunk partials:
    one key past 32768, and the reference's KV_CACHE_CAP of 163,840
    positions (src/model_load.c:237; 320 chunks of 512 keys)."""
    run_case(ctx, oracle, 16, 1, kv_len, kv_len, 641)


def test_mla_ragged_batch(ctx, oracle):
    """Per-sequence lengths, including one sequence shorter than a sub-tile
    and chunks with no valid keys."""
    run_case(ctx, oracle, 16, 4, 1100, 1100, 611, kv_lens=[1100, 5, 600, 513])


@pytest.mark.parametrize("NH", [8, 20])
def test_mla_head_groups(ctx, oracle, NH):
    """Fewer than 16 heads (padded group) and more than 16 (two groups)."""
    run_case(ctx, oracle, NH, 2, 300, 300, 620 + NH)


def test_mla_closed_forms(ctx, oracle):
    """kv_len = 1: weights exactly 1 and clat = c_kv[0] (to bf16 precision of
    the hi/lo split); q = 0: uniform weights and clat = mean of the rows."""
    NH, B, L = 16, 2, 64
    rng = np.random.default_rng(630)
    kv_b = synth.normal_bf16(rng, (NH * 256, 512), 0.02)
    cache = synth.normal_bf16(rng, (B, L, 576), 1.0)
    ctx.mla_init(NH)
    ctx.mla_load_layer(0, kv_b)
    q = synth.normal_f32(rng, (B, NH, 192))
    c, qa, p, cl = ctx.mla_absorbed_decode(0, q, cache, 1)
    assert np.allclose(p, 1.0)
    cf = synth.bf16_to_f32(cache)
    for b in range(B):
        assert max_abs_rel(cl[b], np.stack([cf[b, 0, :512]] * NH)) < 1e-4
    c, qa, p, cl = ctx.mla_absorbed_decode(0, np.zeros_like(q), cache, L)
    assert np.allclose(p, 1.0 / L, rtol=1e-5)
    for b in range(B):
        assert max_abs_rel(cl[b, 0], cf[b, :, :512].astype(np.float64).mean(axis=0)) < 1e-4


def test_mla_config5_subset(ctx, oracle):
    """BASELINE config-5 geometry (16 heads, 4096 context) on 3 sequences."""
    run_case(ctx, oracle, 16, 3, 4096, 4096, 640)


def test_mla_config5_full(ctx, oracle):
    """BASELINE config 5 at its own size: B = 32 sequences x 16 heads over
    4096 positions, every sequence checked.  This is the shape the bench
    times: 512-key chunks (32 x 8 = 256 blocks, no halving), the one-block
    merge per (head, sequence) (NH * B = 512 >= 128) and full 32-row tiles in
    the W_UK and W_UV products."""
    run_case(ctx, oracle, 16, 32, 4096, 4096, 650)


def test_mla_two_row_tiles_ragged(ctx, oracle):
    """B = 40 (> 32: a second, partial row tile in the W_UK / W_UV products)
    with ragged lengths up to 1500 and NH * B = 640 (one-block merge)."""
    lens = [1500 - 37 * b for b in range(40)]
    lens[3], lens[17], lens[39] = 1, 16, 513
    run_case(ctx, oracle, 16, 40, 1500, 1500, 651, kv_lens=lens)


@pytest.mark.parametrize("NH,B,VHD", [(16, 520, 128), (20, 516, 80)])
def test_mla_wide_products(ctx, oracle, NH, B, VHD):
    """From 512 rows on (a prefill's) the W_UK and W_UV products take four
    column tiles per wave: a partial last row tile, two head groups, and a
    V head dimension of 80 (the second column block's tiles past it read a
    clamped W_UV row and store nothing), ragged short contexts."""
    lens = [1 + (37 * b) % 60 for b in range(B)]
    run_case(ctx, oracle, NH, B, 60, 60, 655 + NH, kv_lens=lens, VHD=VHD)


def test_mla_rows_in_groups(monkeypatch, oracle):
    """Chunk partials over the per-launch cap (MLAMOE_MLA_PART_MAX, here
    three rows' worth): the rows go in groups of 3, 3, 3 and 1, one after
    another.  Every row against the oracle and bit-identical to the
    ungrouped call (ragged lengths; B * HG * chunks = 10 x 24)."""
    B, L, NH = 10, 1500, 16
    lens = [1500, 7, 900, 64, 1, 1499, 300, 16, 1024, 777]
    per_row = 24 * (16 * 512 + 32) * 4            # 24 chunks of 64 keys
    with mlamoe.Context(0) as c0:
        ref = run_case(c0, oracle, NH, B, L, L, 660, kv_lens=lens)
    monkeypatch.setenv("MLAMOE_MLA_PART_MAX", str(3 * per_row))
    with mlamoe.Context(0) as c1:
        got = run_case(c1, oracle, NH, B, L, L, 660, kv_lens=lens)
    same = lambda x, y: np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32))  # noqa: E731
    for name, i in (("ctx", 0), ("qabs", 1), ("clat", 3)):
        assert same(ref[i], got[i]), name
    for b, n in enumerate(lens):   # the weights of each row's own keys (the rest is not written)
        assert same(ref[2][b][:, :n], got[2][b][:, :n]), ("probs", b)
