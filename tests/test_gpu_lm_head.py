"""GPU parity of the LM head (final RMSNorm, logits, greedy argmax) against
the CPU oracle, which the reference's own compiled run.c pins bit for bit
(tests/golden/lm_head.npz).

Bars:
  - argmax: identical to the oracle on the same logits (exact integer result);
  - rmsnorm: normwise error <= 1e-6 (the GPU reduces the sum of squares in a
    different order than the sequential loop of run.c:22-27);
  - logits: max-abs-rel (normwise) <= 2e-3, the north-star bf16 bar; measured
    ~1e-6 since x is carried as fp32 (GEMV) or a bf16 hi/lo pair (GEMM);
  - sampled token: equal to the oracle's, or, where the GPU's rounding moved a
    near-tie, a token whose oracle logit is within 1e-5 (normwise) of the
    oracle maximum.
"""
import numpy as np
import pytest

import mlamoe
from conftest import load_golden, max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def ctx():
    c = mlamoe.Context(0)
    yield c
    c.close()


def _check_tokens(tok, ref_logits, ref_tok):
    for t, (a, b) in enumerate(zip(tok, ref_tok)):
        if a != b:
            lg = ref_logits[t]
            assert lg[a] >= lg.max() - 1e-5 * np.abs(lg).max(), (t, a, b)


def test_argmax_rules(ctx, oracle):
    g = load_golden("lm_head.npz")
    for name in ("random", "tie", "nan0", "nanmid", "ninf", "pinf"):
        v = g[f"sample_{name}_in"]
        assert int(ctx.argmax(v[None])[0]) == int(g[f"sample_{name}_out"]), name
    rng = np.random.default_rng(5)
    rows = synth.normal_f32(rng, (7, 102400))
    rows[1, [10, 90000]] = rows[1].max() + 1.0          # tie far apart: lower index
    rows[2, 0] = np.nan                                  # NaN at 0 never replaced
    rows[3, rng.integers(0, 102400, 500)] = np.nan       # scattered NaNs never win
    rows[4, :] = -np.inf
    rows[5, :] = np.nan
    assert np.array_equal(ctx.argmax(rows), oracle.argmax(rows))


def test_rmsnorm(ctx, oracle):
    rng = np.random.default_rng(6)
    for T, n, eps, scale in ((1, 2048, 1e-6, 1.0), (5, 512, 1e-5, 30.0), (3, 8, 1e-6, 1e-3)):
        x = synth.normal_f32(rng, (T, n), scale)
        w = synth.bf16_from_f32(1.0 + synth.normal_f32(rng, (n,), 0.1))
        assert max_abs_rel(ctx.rmsnorm(x, w, eps), oracle.rmsnorm(x, w, eps)) < 1e-6
    # constant rows: ss is exact, so every step is correctly rounded on both sides
    x = np.full((2, 64), 2.0, np.float32)
    one = synth.bf16_from_f32(np.ones(64, np.float32))
    assert np.array_equal(ctx.rmsnorm(x, one, 1e-6), oracle.rmsnorm(x, one, 1e-6))


def test_lm_head_golden(ctx):
    g = load_golden("lm_head.npz")
    logits, tokens = ctx.lm_head(g["lm_x"], g["lm_norm"], float(g["lm_eps"]), g["lm_w"])
    assert max_abs_rel(logits, g["lm_logits"]) < TOL
    _check_tokens(tokens, g["lm_logits"], g["lm_tokens"])


@pytest.mark.parametrize("B,V,H", [(1, 1000, 256), (3, 4099, 2048), (4, 777, 64),
                                   (5, 4096, 2048), (8, 1001, 512), (17, 300, 136)])
def test_lm_head_shapes(ctx, oracle, B, V, H):
    """Both paths (B <= 4: GEMV, else the MFMA GEMM), vocabularies that are
    not multiples of the tile sizes, hidden sizes below the GEMV's maximum."""
    print(f"lm_head B={B} V={V} H={H}", flush=True)
    rng = np.random.default_rng(B * 1000 + V)
    x = synth.normal_f32(rng, (B, H))
    norm = synth.bf16_from_f32(1.0 + synth.normal_f32(rng, (H,), 0.1))
    lm = synth.normal_bf16(rng, (V, H), 0.02)
    logits, tokens = ctx.lm_head(x, norm, 1e-6, lm)
    rl, rt = oracle.lm_head_rows(x, norm, 1e-6, lm)
    assert max_abs_rel(logits, rl) < TOL
    assert max_abs_rel(logits, rl) < 1e-5            # fp32-level, not bf16-level
    _check_tokens(tokens, rl, rt)
    # tokens without returning the logits
    _, t2 = ctx.lm_head(x, norm, 1e-6, lm, want_logits=False)
    assert np.array_equal(t2, tokens)


def test_lm_head_dsv2_vocab(ctx, oracle):
    """DeepSeek-V2-Lite's LM head: vocab 102400 x hidden 2048, one decode
    token (GEMV), five and 64 (the logits GEMM)."""
    rng = np.random.default_rng(77)
    V, H = 102400, 2048
    lm = synth.normal_bf16(rng, (V, H), 0.02)
    norm = synth.bf16_from_f32(1.0 + synth.normal_f32(rng, (H,), 0.1))
    for B in (1, 5, 64):
        print(f"lm_head dsv2 B={B}", flush=True)
        x = synth.normal_f32(rng, (B, H))
        logits, tokens = ctx.lm_head(x, norm, 1e-6, lm)
        rl, rt = oracle.lm_head_rows(x, norm, 1e-6, lm)
        assert max_abs_rel(logits, rl) < 1e-5
        _check_tokens(tokens, rl, rt)


def test_lm_head_gemm_matches_skinny(ctx):
    """5..64 rows: the logits GEMM (bf16 hi/lo planes written by the norm,
    both operands through a direct-to-LDS ring) gives the same bits as the
    skinny GEMM's wide form over the fp32 norm output (the same split, the
    same MFMA sequence per output, one pass over K: the wide form takes
    vocabularies past 65536); V = 65600 is not a multiple of the 256-row
    tile."""
    rng = np.random.default_rng(90)
    V, H = 65600, 2048
    lm = synth.normal_bf16(rng, (V, H), 0.02)
    norm = synth.bf16_from_f32(1.0 + synth.normal_f32(rng, (H,), 0.1))
    for B in (5, 64):
        print(f"lm_head gemm vs skinny B={B} V={V}", flush=True)
        x = synth.normal_f32(rng, (B, H))
        logits, _ = ctx.lm_head(x, norm, 1e-6, lm)
        ref = ctx.matmul(ctx.rmsnorm(x, norm, 1e-6), lm)
        assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32)), B


def test_lm_head_errors(ctx):
    L = mlamoe.lib()
    assert L.mm_lm_head_dev(ctx.h, 1, None, None, 1e-6, None, 10, 16, None, None) != 0
    assert b"NULL" in L.mm_last_error()
    buf = ctx.empty((64,), np.float32)
    assert L.mm_lm_head_dev(ctx.h, 1, buf.ptr, buf.ptr, 1e-6, buf.ptr, 10, 12, None, buf.ptr) != 0
    assert b"multiple of 8" in L.mm_last_error()
    assert L.mm_lm_head_dev(ctx.h, 0, None, None, 1e-6, None, 10, 16, None, None) == 0  # no-op
