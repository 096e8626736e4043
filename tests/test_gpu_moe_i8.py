"""GPU parity of the int8 MoE path (MFMA) against the CPU oracle.

Bars (stated per check below):
  - routing identical to the reference router;
  - quantised activations, weights and every int32 accumulator bit-exact
    against scalar CPU int8 dot products on the same int8 operands;
  - dequantised outputs bit-exact where the GPU performs the same fp32
    operations, otherwise within max-abs-rel 2e-3 of the CPU on the same
    quantised operands.
"""
import numpy as np
import pytest

import mlamoe
from conftest import max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(params=["decode", "tiled"])
def ctx(request, monkeypatch):
    """A context whose int8 GEMMs take the decode-shaped path or the tiled
    (prefill, big-tile) path for every T."""
    monkeypatch.setenv("MLAMOE_I8_TILED_MIN_T", "1" if request.param == "tiled" else "1000000000")
    print(f"int8 GEMM path: {request.param}", flush=True)
    c = mlamoe.Context(0)
    yield c
    c.close()


def _dot_exact(qa, qb):
    """int8 [M, K] x int8 [N, K]^T in float64: exact for |acc| < 2^53."""
    return (qa.astype(np.float64) @ qb.astype(np.float64).T).astype(np.int64)


def _silu_mul(g, u, oracle):
    L = oracle.lib()
    s = np.array([L.or_silu(float(v)) for v in g.ravel()], np.float32).reshape(g.shape)
    return s * u


def run_case(ctx, oracle, H, E, K, I, NS, T, seed, logits=None, sig=0, norm=0, scale=1.0,
             bias=False, check_all=True):
    print(f"int8 case H={H} E={E} K={K} I={I} NS={NS} T={T} seed={seed}", flush=True)
    w = synth.moe_layer(seed, H, E, I, NS, gate_bias=bias)
    ctx.moe_init(H, E, NS, K, I, sig, norm, scale)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
    x = synth.activations(seed + 1, T, H)
    out, idx, wt, probs, d = ctx.moe_forward_i8_debug(0, x, logits)
    cfg = oracle.moe_cfg(H, E, NS, K, I, sig, norm, scale)
    qw = oracle.quantize_moe_weights(w)
    ro, ri, rw, rp, rd = oracle.ffn_i8(cfg, w, qw, x, logits, debug=True)
    S = NS * I

    # routing: identical selection, scores within 2 ulp (e^x rounding)
    assert np.array_equal(idx, ri)
    assert np.max(np.abs(wt.view(np.int32).astype(np.int64) - rw.view(np.int32))) <= 4
    # per-token activation quantisation: bit-exact
    assert np.array_equal(d["qx"], rd["qx"]) and np.array_equal(d["sx"], rd["sx"])
    if check_all:
        for t in range(T):
            for r in range(K):
                e, rid = idx[t, r], t * K + r
                # int32 gate/up accumulators: bit-exact vs scalar int8 dots
                ag = _dot_exact(d["qx"][t:t + 1], qw["qeg"][e])[0]
                au = _dot_exact(d["qx"][t:t + 1], qw["qeu"][e])[0]
                assert np.array_equal(d["acc_gu"][rid, 0], ag), (t, r)
                assert np.array_equal(d["acc_gu"][rid, 1], au), (t, r)
                # dequantise + SwiGLU: same fp32 ops, e^x may differ by an ulp
                g = (ag.astype(np.float32) * d["sx"][t]) * qw["seg"][e]
                u = (au.astype(np.float32) * d["sx"][t]) * qw["seu"][e]
                assert max_abs_rel(d["h"][rid], _silu_mul(g, u, oracle)) < 1e-5
                # down accumulators on the GPU's own quantised hidden row
                adr = _dot_exact(d["qh"][rid:rid + 1], qw["qed"][e])[0]
                assert np.array_equal(d["acc_d"][rid], adr), (t, r)
                y = (adr.astype(np.float32) * d["sh"][rid]) * qw["sed"][e]
                assert np.array_equal(d["y"][rid], y)
                # dequantised output vs an fp32 matmul on the dequantised operands
                hq = d["qh"][rid].astype(np.float32) * d["sh"][rid]
                wd = qw["qed"][e].astype(np.float32) * qw["sed"][e][:, None]
                assert max_abs_rel(d["y"][rid], wd.astype(np.float64) @ hq) < TOL
    # hidden-row quantisation: bit-exact on the GPU's own h
    qh, sh = oracle.quant_rows(d["h"])
    assert np.array_equal(d["qh"], qh) and np.array_equal(d["sh"], sh)
    if S:
        qs, ss = oracle.quant_rows(d["hs"])
        assert np.array_equal(d["qhs"], qs) and np.array_equal(d["shs"], ss)
        acs = _dot_exact(d["qhs"], qw["qsd"])
        ys = (acs.astype(np.float32) * d["shs"][:, None]) * qw["ssd"][None, :]
        assert np.array_equal(d["ys"], ys)
    # whole layer against the CPU int8 pipeline
    assert max_abs_rel(out, ro) < TOL
    return out, ro, idx, x, w


def test_i8_small_computed_logits(ctx, oracle):
    run_case(ctx, oracle, 256, 16, 4, 128, 2, 1, 51)


def test_i8_small_glm_router(ctx, oracle):
    run_case(ctx, oracle, 256, 16, 4, 128, 2, 37, 52, sig=1, norm=1, scale=1.8, bias=True)


def test_i8_skewed_rows_over_64(ctx, oracle):
    """Three experts take every token (M = 200 > one 64-row pass), most get
    none: exercises the row-pass loop and empty experts."""
    T, E = 200, 16
    lg = synth.uniform_logits(60, T, E)
    lg[:, :3] += 5.0
    out, ro, idx, *_ = run_case(ctx, oracle, 256, E, 4, 128, 1, T, 61, logits=lg)
    assert np.all(np.isin([0, 1, 2], idx))


def test_i8_no_shared_expert(ctx, oracle):
    run_case(ctx, oracle, 128, 8, 2, 64, 0, 9, 62)


def test_i8_odd_k_blocks(ctx, oracle):
    """Reduction lengths of an odd number of 64-byte K blocks (H = 192:
    three; I = S = 320: five): the tiled GEMM's last 128-byte stage is half
    a stage."""
    run_case(ctx, oracle, 192, 16, 4, 320, 1, 37, 63)


def test_i8_dsv2_decode_batch(ctx, oracle):
    """DeepSeek-V2-Lite shape, batched decode with given uniform logits
    (config 4's routing), T = 16 (routed and shared accumulators checked on
    the tiled path's larger tiles too)."""
    d = synth.DSV2
    T = 16
    lg = synth.uniform_logits(70, T, d["E"])
    run_case(ctx, oracle, d["H"], d["E"], d["K"], d["I"], d["n_shared"], T, 71, logits=lg,
             check_all=False)


@pytest.mark.parametrize("T", [1, 3])
def test_i8_dsv2_few_tokens(ctx, oracle, T):
    """DeepSeek-V2-Lite shape at 1 and 3 tokens: the decode-shaped gate/up
    GEMM splits K over a block's waves there (few experts hold rows); the
    int32 accumulators of every route and of the shared expert stay
    bit-exact."""
    d = synth.DSV2
    run_case(ctx, oracle, d["H"], d["E"], d["K"], d["I"], d["n_shared"], T, 72 + T)


def test_i8_accumulate_in_place(ctx, oracle):
    """MM_FWD_ACCUMULATE with out aliasing xn: x += ffn(x) (residual stream)."""
    H, E, K, I, NS, T = 256, 16, 4, 128, 2, 23
    w = synth.moe_layer(80, H, E, I, NS)
    ctx.moe_init(H, E, NS, K, I)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
    x = synth.activations(81, T, H)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    ro, *_ = oracle.ffn_i8(cfg, w, oracle.quantize_moe_weights(w), x)
    dx = ctx.to_device(x)
    ctx.moe_forward_dev(0, T, dx, dx, flags=mlamoe.MM_FWD_INT8 | mlamoe.MM_FWD_ACCUMULATE)
    got = dx.download(np.float32, (T, H))
    assert max_abs_rel(got - x, ro) < TOL


def test_i8_repeat_calls_reset_counters(ctx, oracle):
    """Back-to-back calls with different T: per-expert counters start at zero."""
    H, E, K, I, NS = 128, 8, 2, 64, 1
    w = synth.moe_layer(90, H, E, I, NS)
    ctx.moe_init(H, E, NS, K, I)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    qw = oracle.quantize_moe_weights(w)
    for T in (40, 3, 17):
        x = synth.activations(91 + T, T, H)
        out, idx, *_ = ctx.moe_forward(0, x, flags=mlamoe.MM_FWD_INT8)
        ro, ri, *_ = oracle.ffn_i8(cfg, w, qw, x)
        assert np.array_equal(idx, ri) and max_abs_rel(out, ro) < TOL


def test_i8_vs_bf16_drift_reported(ctx, oracle):
    """The int8 layer against the bf16 reference ffn_compute: reported, not
    gated by the 2e-3 bar (quantisation error), but must stay small."""
    H, E, K, I, NS, T = 256, 16, 4, 128, 2, 8
    w = synth.moe_layer(95, H, E, I, NS)
    ctx.moe_init(H, E, NS, K, I)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8 | mlamoe.MM_LOAD_BF16)
    x = synth.activations(96, T, H)
    o8, i8, *_ = ctx.moe_forward(0, x, flags=mlamoe.MM_FWD_INT8)
    o16, i16, *_ = ctx.moe_forward(0, x, flags=mlamoe.MM_FWD_BF16)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    ro, ri, *_ = oracle.ffn_compute_rows(cfg, w, x)
    assert np.array_equal(i8, ri) and np.array_equal(i16, ri)
    assert max_abs_rel(o16, ro) < TOL
    drift = max_abs_rel(o8, ro)
    print(f"int8 vs bf16 reference drift (max-abs-rel): {drift:.3e}")
    assert drift < 5e-2


def test_i8_dsv2_prefill_skewed(ctx, oracle):
    """Config-3 routing on a shorter prompt: DeepSeek-V2-Lite shapes, T=300,
    router logits W_g x plus the Zipf(1.1) prior, so some experts get more
    than one 128-row tile and others none."""
    d = synth.DSV2
    H, E, K, I, NS, T = d["H"], d["E"], d["K"], d["I"], d["n_shared"], 300
    w = synth.moe_layer(120, H, E, I, NS)
    ctx.moe_init(H, E, NS, K, I)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
    x = synth.activations(121, T, H)
    z = synth.zipf_prior(122, E)
    lg = ctx.router_logits(0, x, z)
    assert np.array_equal(lg.view(np.uint32), (oracle.matmul(x, w["moe_gate"]) + z).view(np.uint32))
    out, idx, wt, probs, dd = ctx.moe_forward_i8_debug(0, x, lg)
    # the product GEMM kernel (the debug call runs its twin): the same bits
    po, pi, pw, _ = ctx.moe_forward(0, x, lg, mlamoe.MM_FWD_INT8)
    assert np.array_equal(pi, idx) and np.array_equal(pw.view(np.uint32), wt.view(np.uint32))
    assert np.array_equal(po.view(np.uint32), out.view(np.uint32))
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    qw = oracle.quantize_moe_weights(w)
    ro, ri, *_ = oracle.ffn_i8(cfg, w, qw, x, lg)
    assert np.array_equal(idx, ri)
    counts = np.bincount(idx.ravel(), minlength=E)
    assert counts.max() > 128
    # spot-check int32 accumulators of the busiest expert's rows
    e = int(counts.argmax())
    rids = [t * K + r for t in range(T) for r in range(K) if idx[t, r] == e][:40]
    for rid in rids:
        t = rid // K
        assert np.array_equal(dd["acc_gu"][rid, 0], _dot_exact(dd["qx"][t:t + 1], qw["qeg"][e])[0])
        assert np.array_equal(dd["acc_d"][rid], _dot_exact(dd["qh"][rid:rid + 1], qw["qed"][e])[0])
    assert max_abs_rel(out, ro) < TOL


@pytest.mark.parametrize("E", [100, 160])
def test_i8_many_experts(ctx, oracle, E):
    """More than 64 experts (two or four per router lane), top-8, with the
    row lists of the tiled path spread over all of them."""
    run_case(ctx, oracle, 256, E, 8, 128, 1, 40, 97, check_all=False)


def test_i8_empty_batch_is_a_no_op(ctx):
    """T = 0: nothing is launched and the output is untouched."""
    H, E, K, I, NS = 128, 8, 2, 64, 1
    w = synth.moe_layer(98, H, E, I, NS)
    ctx.moe_init(H, E, NS, K, I)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
    out = ctx.empty((1, H), np.float32)
    ctx.fill(out, H, mlamoe.MM_FILL_F32_NORMAL, 99, 1.0)
    before = out.download()
    ctx.moe_forward_dev(0, 0, None, out, flags=mlamoe.MM_FWD_INT8)
    ctx.sync()
    assert np.array_equal(out.download(), before)


@pytest.mark.parametrize("T", [3, 6])
def test_nan_router_scores_route_distinct_experts(ctx, oracle, T):
    """A NaN logit makes every softmax score of its token NaN.  The
    reference's strict '>' scan never picks a NaN (its index is then
    undefined); here a NaN score ranks after every number, so each token
    still routes to K distinct experts in range -- the GEMMs' per-expert row
    lists hold at most T rows -- and tokens without NaN route as the
    oracle's router.  int8 (this fixture's decode or tiled GEMMs; the K-split
    gate/up at 3 tokens) and bf16 experts."""
    H, E, K, I, NS = 256, 16, 4, 128, 1
    print(f"NaN router scores T={T}", flush=True)
    w = synth.moe_layer(810 + T, H, E, I, NS)
    ctx.moe_init(H, E, NS, K, I)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8 | mlamoe.MM_LOAD_BF16)
    x = synth.activations(811 + T, T, H)
    logits = np.random.default_rng(812 + T).random((T, E)).astype(np.float32)
    logits[0, :] = np.nan                  # every logit NaN
    logits[1, 3] = np.nan                  # one NaN logit
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    for flags in (mlamoe.MM_FWD_INT8, mlamoe.MM_FWD_BF16):
        _, idx, _, _ = ctx.moe_forward(0, x, logits, flags)
        for t in range(T):
            row = idx[t].tolist()
            assert len(set(row)) == K and min(row) >= 0 and max(row) < E, (flags, t, row)
            if t >= 2:   # the oracle's scan only on NaN-free tokens
                assert np.array_equal(idx[t], oracle.route(cfg, logits[t])[1]), (flags, t)


def test_i8_rows_in_chunks(ctx, oracle, monkeypatch):
    """A call longer than the forward pass's row cap runs as consecutive
    chunks: outputs, routing and scores bit-identical to one pass (the cap
    lowered to 37 rows through MLAMOE_MOE_T_CHUNK; by default it keeps every
    int8 activation matrix of the tiled GEMMs below their 32-bit offsets)."""
    H, E, K, I, NS, T = 256, 16, 4, 128, 2, 100
    w = synth.moe_layer(120, H, E, I, NS)
    x = synth.activations(121, T, H)
    monkeypatch.setenv("MLAMOE_MOE_T_CHUNK", "37")
    cc = mlamoe.Context(0)
    try:
        for c in (ctx, cc):
            c.moe_init(H, E, NS, K, I)
            c.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8 | mlamoe.MM_LOAD_BF16)
        for flags in (mlamoe.MM_FWD_INT8, mlamoe.MM_FWD_BF16):
            one = ctx.moe_forward(0, x, flags=flags)
            chunked = cc.moe_forward(0, x, flags=flags)
            for a, b in zip(one, chunked):
                assert np.array_equal(a, b), flags
        ro, ri, *_ = oracle.ffn_i8(oracle.moe_cfg(H, E, NS, K, I), w,
                                   oracle.quantize_moe_weights(w), x)
        out, idx, *_ = cc.moe_forward(0, x, flags=mlamoe.MM_FWD_INT8)
        assert np.array_equal(idx, ri) and max_abs_rel(out, ro) < TOL
    finally:
        cc.close()


@pytest.mark.parametrize("H,I,NS", [(384, 448, 1), (768, 704, 2), (832, 576, 1)])
def test_i8_k_turn_boundaries(ctx, oracle, H, I, NS):
    """Reduction lengths around the tiled GEMM's whole turns of 6 K steps:
    gate/up 6, 12 and 13 steps (one turn, two, two plus one), down 7, 11 and
    9 (a turn plus a tail of 1, 5 and 3, odd: a half last stage), the shared
    down 7, 22 and 9.  Every accumulator against the oracle through the
    debug entry, and the product kernels' output bit-identical to it."""
    T, E, K = 40, 16, 4
    out, ro, idx, x, w = run_case(ctx, oracle, H, E, K, I, NS, T, 130 + H // 64)
    prod, pidx, *_ = ctx.moe_forward(0, x, flags=mlamoe.MM_FWD_INT8)
    assert np.array_equal(pidx, idx) and np.array_equal(prod, out)
