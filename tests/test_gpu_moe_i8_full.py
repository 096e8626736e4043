"""GPU parity of the int8 MoE path at the BASELINE configs' own sizes.

Config 3: one DeepSeek-V2-Lite-shaped layer at prefill T = 2048 with the
router's logits W_g x plus the Zipf(1.1) prior (the bench's workload: the
hot expert holds ~2000 rows, i.e. ~16 of the big-tile kernel's 128-row
tiles; 15 experts are hot, most are cold).
Config 4: batched decode B = 64 with uniform-random logits through one layer
against the oracle, and through three chained layers with the residual
carried (x += ffn(x)) as the bench runs its 26-layer stack.

The CPU oracle's full layer costs ~69 M scalar MACs per token, so whole-layer
outputs are compared on token subsets (tokens are independent in
ffn_compute, src/run.c:116-162, and in its int8 restatement: the subset's
results equal the full run's).  Every int32 accumulator of the checked rows
is compared with exact integer dots (float64 products of |q| <= 127 over
K <= 2816 stay below 2^53, so they are exact).

Bars: routing identical; int32 accumulators and per-row quantisation
bit-exact; dequantised outputs max-abs-rel <= 2e-3 of the oracle on the same
quantised operands.
"""
import numpy as np
import pytest

import mlamoe
from conftest import max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3
D = synth.DSV2
H, E, K, I, NS = D["H"], D["E"], D["K"], D["I"], D["n_shared"]
S = NS * I


@pytest.fixture(scope="module")
def layer0():
    """One DeepSeek-V2-Lite-shaped layer (bf16 host weights) and its int8
    quantisation by the oracle."""
    import pyoracle
    w = synth.moe_layer(130, H, E, I, NS)
    return w, pyoracle.quantize_moe_weights(w)


def _exact(qa, qb):
    return (qa.astype(np.float64) @ qb.astype(np.float64).T).astype(np.int64)


def _check_routes(dd, qw, idx, rids, label):
    """Gate/up and down accumulators (and the dequantised down outputs) of
    the routed rows `rids` bit-exact, one expert at a time."""
    rids = np.asarray(rids)
    flat = idx.ravel()
    for e in np.unique(flat[rids]):
        r = rids[flat[rids] == e]
        t = r // K
        ag = _exact(dd["qx"][t], qw["qeg"][e])
        au = _exact(dd["qx"][t], qw["qeu"][e])
        assert np.array_equal(dd["acc_gu"][r, 0], ag), (label, "gate", int(e))
        assert np.array_equal(dd["acc_gu"][r, 1], au), (label, "up", int(e))
        ad = _exact(dd["qh"][r], qw["qed"][e])
        assert np.array_equal(dd["acc_d"][r], ad), (label, "down", int(e))
        y = (ad.astype(np.float32) * dd["sh"][r][:, None]) * qw["sed"][e][None, :]
        assert np.array_equal(dd["y"][r], y), (label, "y", int(e))


def test_i8_config3_full_size(oracle, layer0):
    """T = 2048 prefill through the big-tile grouped GEMM (the path the bench
    times): top-k identical for every token, every accumulator of the
    hottest and of a cold expert bit-exact, all of the shared expert's
    outputs bit-exact, and the layer output on 48 tokens (including tokens
    routed to the hottest expert) within 2e-3 of the oracle.  The debug call
    runs the GEMM's accumulator-writing twin; the product kernel then runs on
    the same inputs and must give the same bits (output, routing, scores)."""
    w, qw = layer0
    T = 2048
    print(f"config 3 full size: T={T}", flush=True)
    x = synth.activations(131, T, H)
    z = synth.zipf_prior(132, E)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
        lg = ctx.router_logits(0, x, z)
        out, idx, wt, probs, dd = ctx.moe_forward_i8_debug(0, x, lg)
        # the product kernel (the one the bench times; the debug call runs
        # its accumulator-writing twin) on the same inputs: the same bits
        po, pi, pw, pp = ctx.moe_forward(0, x, lg, mlamoe.MM_FWD_INT8)
    assert np.array_equal(pi, idx) and np.array_equal(pw.view(np.uint32), wt.view(np.uint32))
    assert np.array_equal(po.view(np.uint32), out.view(np.uint32))
    assert np.array_equal(pp.view(np.uint32), probs.view(np.uint32))
    # router logits: the reference's sequential fp32 order, bit for bit
    assert np.array_equal(lg.view(np.uint32), (oracle.matmul(x, w["moe_gate"]) + z).view(np.uint32))
    # routing of every token identical to the CPU router
    for t in range(T):
        _, ri, rw = oracle.route(cfg, lg[t])
        assert np.array_equal(idx[t], ri), t
        assert np.max(np.abs(wt[t].view(np.int32).astype(np.int64) - rw.view(np.int32))) <= 4, t
    counts = np.bincount(idx.ravel(), minlength=E)
    hot = int(counts.argmax())
    cold = int(np.flatnonzero((counts > 0) & (counts < 32))[0])
    print(f"rows: hot expert {hot} {counts[hot]}, cold expert {cold} {counts[cold]}, "
          f"experts with rows {(counts > 0).sum()}", flush=True)
    assert counts[hot] > 16 * 64          # many 128-row tiles
    # per-token quantisation of x and of the hidden rows: bit-exact
    qx, sx = oracle.quant_rows(x)
    assert np.array_equal(dd["qx"], qx) and np.array_equal(dd["sx"], sx)
    qh, sh = oracle.quant_rows(dd["h"])
    assert np.array_equal(dd["qh"], qh) and np.array_equal(dd["sh"], sh)
    # every route of the hottest and of a cold expert
    rids = np.flatnonzero(idx.ravel() == hot)
    _check_routes(dd, qw, idx, rids, "hot")
    _check_routes(dd, qw, idx, np.flatnonzero(idx.ravel() == cold), "cold")
    # SwiGLU epilogue of the hot expert: same fp32 ops as the oracle's
    # dequantisation, e^x within an ulp
    for rid in rids[:64]:
        t = rid // K
        ag = dd["acc_gu"][rid, 0].astype(np.float32)
        au = dd["acc_gu"][rid, 1].astype(np.float32)
        g = (ag * dd["sx"][t]) * qw["seg"][hot]
        u = (au * dd["sx"][t]) * qw["seu"][hot]
        ref = g / (np.float32(1) + np.exp(-g)) * u
        assert max_abs_rel(dd["h"][rid], ref) < 1e-5, rid
    # shared expert over all T tokens: its quantised rows and outputs bit-exact
    qs, ss = oracle.quant_rows(dd["hs"])
    assert np.array_equal(dd["qhs"], qs) and np.array_equal(dd["shs"], ss)
    acs = _exact(dd["qhs"], qw["qsd"])
    ys = (acs.astype(np.float32) * dd["shs"][:, None]) * qw["ssd"][None, :]
    assert np.array_equal(dd["ys"], ys)
    # whole layer on a token subset: 24 tokens of the hot expert, 24 spread out
    hot_tok = np.unique(rids // K)[:24]
    sub = np.unique(np.concatenate([hot_tok, np.linspace(0, T - 1, 24).astype(int)]))
    ro, ri, *_ = oracle.ffn_i8(cfg, w, qw, x[sub], lg[sub])
    assert np.array_equal(idx[sub], ri)
    err = max_abs_rel(out[sub], ro)
    print(f"config 3 layer output on {len(sub)} tokens: max-abs-rel {err:.2e}", flush=True)
    assert err < TOL


def test_i8_config4_layer_B64(oracle, layer0):
    """B = 64 decode (uniform-random logits, the decode-shaped GEMMs): every
    route's accumulators bit-exact and the layer output within 2e-3 for all
    64 tokens."""
    w, qw = layer0
    T = 64
    print(f"config 4 layer: B={T}", flush=True)
    x = synth.activations(141, T, H)
    lg = synth.uniform_logits(142, T, E)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
        out, idx, wt, probs, dd = ctx.moe_forward_i8_debug(0, x, lg)
    ro, ri, rw, rp, rd = oracle.ffn_i8(cfg, w, qw, x, lg, debug=True)
    assert np.array_equal(idx, ri)
    assert np.array_equal(dd["qx"], rd["qx"]) and np.array_equal(dd["sx"], rd["sx"])
    # every int32 accumulator of every route, against the oracle's own
    assert np.array_equal(dd["acc_gu"].reshape(T, K, 2, I), rd["acc_gu"])
    _check_routes(dd, qw, idx, range(T * K), "decode")
    qh, sh = oracle.quant_rows(dd["h"])
    assert np.array_equal(dd["qh"], qh) and np.array_equal(dd["sh"], sh)
    acs = _exact(dd["qhs"], qw["qsd"])
    assert np.array_equal(dd["ys"], (acs.astype(np.float32) * dd["shs"][:, None]) * qw["ssd"][None, :])
    err = max_abs_rel(out, ro)
    print(f"config 4 layer output: max-abs-rel {err:.2e}", flush=True)
    assert err < TOL


def test_i8_config4_chain_three_layers(oracle, layer0):
    """Three DeepSeek-V2-Lite-shaped layers chained at B = 64 with the
    residual carried in place (MM_FWD_ACCUMULATE, out aliasing xn: the
    bench's step).  Per layer: the layer's update x_{l+1} - x_l within 2e-3
    of the oracle fed the GPU's own x_l (16 tokens); end to end: the summed
    update of the three layers within 2e-3 of the oracle's own chain."""
    T, L = 64, 3
    print(f"config 4 chain: B={T}, {L} layers", flush=True)
    ws = [layer0[0]] + [synth.moe_layer(150 + l, H, E, I, NS) for l in range(1, L)]
    qws = [layer0[1]] + [oracle.quantize_moe_weights(w) for w in ws[1:]]
    lgs = [synth.uniform_logits(160 + l, T, E) for l in range(L)]
    x0 = synth.activations(170, T, H)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    xs = [x0]
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I, n_layers=L)
        for l, w in enumerate(ws):
            ctx.moe_load_layer(l, w, mlamoe.MM_LOAD_INT8)
        dx = ctx.to_device(x0)
        dl = [ctx.to_device(lg) for lg in lgs]
        for l in range(L):
            ctx.moe_forward_dev(l, T, dx, dx, logits=dl[l],
                                flags=mlamoe.MM_FWD_INT8 | mlamoe.MM_FWD_ACCUMULATE)
            xs.append(dx.download(np.float32, (T, H)))
    sub = np.arange(0, T, 4)
    xr = x0[sub]
    for l in range(L):
        ro, *_ = oracle.ffn_i8(cfg, ws[l], qws[l], xs[l][sub], lgs[l][sub])
        err = max_abs_rel(xs[l + 1][sub] - xs[l][sub], ro)
        print(f"layer {l}: update max-abs-rel {err:.2e}", flush=True)
        assert err < TOL, l
        rc, *_ = oracle.ffn_i8(cfg, ws[l], qws[l], xr, lgs[l][sub])
        xr = (xr + rc).astype(np.float32)
    err = max_abs_rel(xs[L][sub] - x0[sub], xr - x0[sub])
    print(f"three-layer chain: summed update max-abs-rel {err:.2e}", flush=True)
    assert err < TOL
