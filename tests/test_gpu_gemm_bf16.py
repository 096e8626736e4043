"""GPU parity of the dense bf16 matmul (run.c:29-37 over T rows) against the
oracle's matmul: max-abs-rel 2e-3 (fp32 accumulation in MFMA order)."""
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


def test_matmul_golden(ctx, oracle):
    """Against the reference matmul's own outputs (tests/golden/matmul.npz);
    the tiny shapes have n_in not a multiple of 8, which this build rejects."""
    g = load_golden("matmul.npz")
    for name in ("router", "expert"):
        r = np.random.default_rng(int(g[f"{name}_seed"]))
        d_out, n_in = (int(v) for v in g[f"{name}_shape"])
        w = synth.normal_bf16(r, (d_out, n_in), 0.02)
        x = synth.normal_f32(r, (n_in,))
        y = ctx.matmul(x[None], w)[0]
        assert max_abs_rel(y, g[f"{name}_y"]) < 1e-5, name
    with pytest.raises(mlamoe.MMError):
        ctx.matmul(g["tiny_x"][None], g["tiny_w"])


@pytest.mark.parametrize("T,d_out,n_in", [(1, 64, 2048), (37, 100, 264), (512, 576, 2048),
                                          (512, 4096, 512), (512, 3072, 2048),
                                          (512, 2048, 2048), (70, 3072, 2048),
                                          (1024, 3072, 136),    # 128-column tiles
                                          # skinny-M GEMM (5 <= T <= 64, n_in % 64 == 0):
                                          # one split, many splits, ragged columns
                                          (64, 102400 // 16, 2048), (5, 3072, 2048),
                                          (33, 576, 2048), (17, 100, 64), (64, 2048, 10944),
                                          (8, 130, 1408)])
def test_matmul_shapes(ctx, oracle, T, d_out, n_in):
    print(f"matmul T={T} d_out={d_out} n_in={n_in}", flush=True)
    rng = np.random.default_rng(T + d_out)
    w = synth.normal_bf16(rng, (d_out, n_in), 0.02)
    x = synth.normal_f32(rng, (T, n_in))
    ref = oracle.matmul(x, w)
    assert max_abs_rel(ctx.matmul(x, w), ref) < 1e-5      # fp32 x as a bf16 hi/lo pair
    xb = synth.bf16_to_f32(synth.bf16_from_f32(x))         # the config-2 input cast
    ref_b = oracle.matmul(xb, w)
    got_b = ctx.matmul(x, w, mlamoe.MM_MATMUL_X_BF16)
    assert max_abs_rel(got_b, ref_b) < TOL
    # accumulate: y += x . W^T
    y0 = synth.normal_f32(rng, (T, d_out))
    got_acc = ctx.matmul(x, w, mlamoe.MM_MATMUL_ACCUMULATE, y0=y0)
    assert max_abs_rel(got_acc - y0, ref) < 1e-5


def test_skinny_integer_exact(ctx):
    """The skinny-M path with integer-valued operands (every summation order
    exact): bit for bit, with and without splits of K, and the wide form
    of long outputs (65600 columns)."""
    rng = np.random.default_rng(4)
    for T, d_out, n_in in ((64, 640, 256), (7, 96, 4096), (33, 65600, 128)):
        w = rng.integers(-8, 9, size=(d_out, n_in)).astype(np.float32)
        x = rng.integers(-8, 9, size=(T, n_in)).astype(np.float32)
        got = ctx.matmul(x, synth.bf16_from_f32(w))
        assert np.array_equal(got, x @ w.T), (T, d_out, n_in)


def test_matmul_integer_exact(ctx):
    """Integer-valued operands with sums < 2^24: every order gives the exact
    integer result, so the GPU must match it bit for bit."""
    rng = np.random.default_rng(3)
    w = rng.integers(-8, 9, size=(96, 256)).astype(np.float32)
    x = rng.integers(-8, 9, size=(33, 256)).astype(np.float32)
    exact = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    got = ctx.matmul(x, synth.bf16_from_f32(w), mlamoe.MM_MATMUL_X_BF16)
    assert np.array_equal(got, exact)


def test_matmul_empty_is_a_no_op(ctx):
    """T = 0: no launch, y untouched."""
    y = ctx.empty((1, 64), np.float32)
    ctx.fill(y, 64, mlamoe.MM_FILL_F32_NORMAL, 5, 1.0)
    before = y.download()
    x = ctx.empty((1, 128), np.float32)
    w = ctx.empty((64, 128), np.uint16)
    ctx.matmul_dev(y, x, w, 64, 128, 0)
    ctx.sync()
    assert np.array_equal(y.download(), before)


def _rne16(x):
    """fp32 -> bf16 bits, round to nearest even (the GPU's rne16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def _split_hl(x):
    """The bf16 hi/lo planes of fp32 rows: hi = rne(x), lo = rne(x - hi)."""
    hi = _rne16(x)
    lo = _rne16((x - synth.bf16_to_f32(hi)).astype(np.float32))
    return np.stack([hi, lo])


@pytest.mark.parametrize("T,d,n", [(5, 3648, 2048), (33, 2048, 2048), (64, 3648, 2048),
                                   (64, 576, 512), (64, 2000, 2048)])
def test_gemm_hl_matches_skinny(ctx, T, d, n):
    """x given as bf16 hi/lo planes (mm_matmul_bf16_hl_dev: both operands
    through a direct-to-LDS ring) gives the skinny GEMM's bits on the fp32
    rows: the same split, K splits, partial order and MFMA sequence; plain
    and accumulating, d not a multiple of the 64-column block."""
    print(f"gemm hl T={T} d={d} n={n}", flush=True)
    rng = np.random.default_rng(500 + T + d)
    x = synth.normal_f32(rng, (T, n))
    w = synth.normal_bf16(rng, (d, n), 0.02)
    ref = ctx.matmul(x, w)
    got = ctx.matmul_hl(_split_hl(x), w)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    y0 = synth.normal_f32(rng, (T, d))
    ref = ctx.matmul(x, w, mlamoe.MM_MATMUL_ACCUMULATE, y0)
    got = ctx.matmul_hl(_split_hl(x), w, mlamoe.MM_MATMUL_ACCUMULATE, y0)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
