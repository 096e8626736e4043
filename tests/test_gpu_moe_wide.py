"""GPU parity of routing over more than 256 experts (the wide routers), up to
the reference's limit of 1024 (src/run.c:133-134: `char used[1024]`).

Above 256 experts the logits come from mm_router_wide (the reference's
sequential fp32 order, bit for bit) and the selection from mm_route_wide
(K passes of a wave-wide argmax in the CPU scan's order).  Checked for the
bf16 experts, the int8 decode-shaped GEMMs and the int8 tiled GEMM: routing
identical to the oracle's router (which restates run.c:124-150 and is
pinned to the compiled reference), scores within 2 ulp, layer outputs
within 2e-3 of the oracle; ties, a NaN logit and E not a multiple of 64.
"""
import numpy as np
import pytest

import mlamoe
from conftest import max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


def ulp_diff(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


@pytest.fixture(params=["decode", "tiled"])
def path(request, monkeypatch):
    monkeypatch.setenv("MLAMOE_I8_TILED_MIN_T", "1" if request.param == "tiled" else "1000000000")
    return request.param


@pytest.mark.parametrize("E,glm", [(1024, 0), (1024, 1), (300, 0)])
def test_wide_routing_and_layer(oracle, path, E, glm):
    H, K, I, NS, T = 256, 8, 64, 1, 37
    print(f"wide routing E={E} glm={glm} int8 path {path}", flush=True)
    w = synth.moe_layer(700 + E + glm, H, E, I, NS, gate_bias=bool(glm))
    x = synth.activations(701 + E, T, H)
    sig, norm, scale = (1, 1, 2.5) if glm else (0, 0, 1.0)
    cfg = oracle.moe_cfg(H, E, NS, K, I, sig, norm, scale)
    qw = oracle.quantize_moe_weights(w)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I, sig, norm, scale)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_BF16 | mlamoe.MM_LOAD_INT8)
        lg = ctx.router_logits(0, x)
        o16, i16, w16, p16 = ctx.moe_forward(0, x, flags=mlamoe.MM_FWD_BF16)
        o8, i8, w8, p8 = ctx.moe_forward(0, x, flags=mlamoe.MM_FWD_INT8)
        g8, gi8, *_ = ctx.moe_forward(0, x, lg, flags=mlamoe.MM_FWD_INT8)   # logits given
    # logits: the reference's sequential fp32 order, bit for bit
    assert np.array_equal(lg.view(np.uint32), oracle.matmul(x, w["moe_gate"]).view(np.uint32))
    ro, ri, rw, rp = oracle.ffn_compute_rows(cfg, w, x)
    for idx, wt, pr in ((i16, w16, p16), (i8, w8, p8)):
        assert np.array_equal(idx, ri)
        assert ulp_diff(wt, rw).max() <= 4 and ulp_diff(pr, rp).max() <= 2
    assert np.array_equal(gi8, ri) and np.array_equal(g8.view(np.uint32), o8.view(np.uint32))
    assert max_abs_rel(o16, ro) < TOL
    r8, ri8, *_ = oracle.ffn_i8(cfg, w, qw, x)
    assert np.array_equal(ri8, ri)
    assert max_abs_rel(o8, r8) < TOL


def test_wide_ties_and_nan(oracle, path):
    """All-equal logits pick experts 0 .. K-1 (the lowest index wins a tie,
    run.c:140); a NaN logit makes every score of its token NaN: the token
    still gets K distinct experts (NaN ranks after every number), and the
    other tokens route as the oracle."""
    H, E, K, I, NS, T = 128, 1024, 6, 64, 0, 5
    w = synth.moe_layer(720, H, E, I, NS)
    x = synth.activations(721, T, H)
    lg = np.random.default_rng(722).random((T, E)).astype(np.float32)
    lg[0, :] = 0.5
    lg[1, 17] = np.nan
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_BF16 | mlamoe.MM_LOAD_INT8)
        for flags in (mlamoe.MM_FWD_BF16, mlamoe.MM_FWD_INT8):
            _, idx, wt, _ = ctx.moe_forward(0, x, lg, flags)
            assert np.array_equal(idx[0], np.arange(K)), (flags, idx[0])
            row = idx[1].tolist()
            assert len(set(row)) == K and min(row) >= 0 and max(row) < E, (flags, row)
            for t in (0, 2, 3, 4):
                assert np.array_equal(idx[t], oracle.route(cfg, lg[t])[1]), (flags, t)


def test_wide_expert_count_limit():
    """E = 1025 is past the reference's limit: refused at set-up."""
    with mlamoe.Context(0) as ctx:
        with pytest.raises(mlamoe.MMError) as e:
            ctx.moe_init(128, 1025, 1, 6, 64)
        assert e.value.status == -1
