"""GPU parity of the router and the bf16-weight MoE FFN (GEMV path) against
the CPU oracle and the reference golden vectors.

Bars: router top-k identical; router scores within 2 ulp (the softmax's e^x
is correctly rounded on the GPU, glibc's expf is within 0.5 ulp); FFN output
within max-abs-rel 2e-3 of the reference (fp32 accumulation in a different
order on the GPU).
"""
import numpy as np
import pytest

import mlamoe
from conftest import load_golden, max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


@pytest.fixture
def ctx():
    c = mlamoe.Context(0)
    yield c
    c.close()


def _layer_ctx(ctx, w, H, E, NS, K, I, sig=0, norm=0, scale=1.0):
    ctx.moe_init(H, E, NS, K, I, sig, norm, scale)
    ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_BF16)


@pytest.mark.parametrize("T", [1, 7, 37])
def test_router_given_logits(ctx, oracle, T):
    """Routing of caller-supplied logits (the batched-decode configuration)."""
    print(f"router given logits T={T}", flush=True)
    H, E, K, I = 64, 64, 6, 16
    w = synth.moe_layer(21, H, E, I, 1)
    _layer_ctx(ctx, w, H, E, 1, K, I)
    lg = synth.uniform_logits(22 + T, T, E)
    lg[0, :] = 0.5            # an all-equal row: lowest indices win
    out, idx, wt, probs = ctx.moe_forward(0, synth.activations(1, T, H), logits=lg)
    cfg = oracle.moe_cfg(H, E, 1, K, I)
    for t in range(T):
        p, i, ww = oracle.route(cfg, lg[t])
        assert np.array_equal(idx[t], i), t
        assert ulp_diff(probs[t], p).max() <= 2
        assert ulp_diff(wt[t], ww).max() <= 2
    assert list(idx[0]) == [0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("sig", [0, 1])
def test_router_sequential_logits(ctx, oracle, sig):
    """Router logits from x in the reference's sequential fp32 order: the
    selected experts must be identical."""
    print(f"router sequential sig={sig}", flush=True)
    H, E, K, I, T = 2048, 64, 6, 8, 21
    w = synth.moe_layer(31 + sig, H, E, I, 1, gate_bias=bool(sig))
    _layer_ctx(ctx, w, H, E, 1, K, I, sig, sig, 1.0 + 0.8 * sig)
    x = synth.activations(33, T, H)
    out, idx, wt, probs = ctx.moe_forward(0, x)
    cfg = oracle.moe_cfg(H, E, 1, K, I, sig, sig, 1.0 + 0.8 * sig)
    logits = oracle.matmul(x, w["moe_gate"])
    for t in range(T):
        p, i, ww = oracle.route(cfg, logits[t], w["moe_gate_bias"])
        assert np.array_equal(idx[t], i), t
        assert ulp_diff(probs[t], p).max() <= 2
        assert ulp_diff(wt[t], ww).max() <= 4


@pytest.mark.parametrize("flavour", ["dsv2", "glm", "tie"])
def test_ffn_tiny_golden(ctx, flavour):
    print(f"ffn tiny golden {flavour}", flush=True)
    g = load_golden("ffn_tiny.npz")
    H, E, NS, K, I, sig, norm = (int(v) for v in g[f"{flavour}_cfg"])
    w = {k: g[f"{flavour}_{k}"] for k in ("moe_gate", "eg", "eu", "ed", "sg", "su", "sd")}
    w["moe_gate_bias"] = g.get(f"{flavour}_bias")
    _layer_ctx(ctx, w, H, E, NS, K, I, sig, norm, float(g[f"{flavour}_scale"]))
    out, idx, wt, probs = ctx.moe_forward(0, g[f"{flavour}_x"])
    assert np.array_equal(idx, g[f"{flavour}_idx"])
    assert ulp_diff(probs, g[f"{flavour}_probs"]).max() <= 2
    assert max_abs_rel(out, g[f"{flavour}_out"]) < TOL


@pytest.fixture(scope="module")
def dsv2_layer():
    g = load_golden("ffn_dsv2.npz")
    d = synth.DSV2
    w = synth.moe_layer(int(g["seed"]), d["H"], d["E"], d["I"], d["n_shared"])
    for k in ("moe_gate", "eg", "sd"):
        assert synth.checksum_u16(w[k]) == int(g[f"sum_{k}"])
    return g, w


def test_ffn_dsv2_golden(ctx, dsv2_layer):
    """Config 1 (T=1 decode layer, DeepSeek-V2-Lite shape) against the
    reference's own ffn_compute output."""
    print("ffn dsv2 golden", flush=True)
    g, w = dsv2_layer
    d = synth.DSV2
    _layer_ctx(ctx, w, d["H"], d["E"], d["n_shared"], d["K"], d["I"])
    x = synth.activations(int(g["xseed"]), int(g["T"]), d["H"])
    out, idx, wt, probs = ctx.moe_forward(0, x)
    assert np.array_equal(idx, g["idx"])
    assert ulp_diff(probs, g["probs"]).max() <= 2
    assert max_abs_rel(out, g["out"]) < TOL
    # the host-pointer mirror of ffn_compute gives the same result
    o1, i1, w1, p1 = ctx.ffn_compute(0, x[0])
    assert np.array_equal(i1, g["idx"][0]) and max_abs_rel(o1, g["out"][0]) < TOL
    assert ulp_diff(p1, g["probs"][0]).max() <= 2     # s->moe_logits after ffn_compute


def test_ffn_multi_token_and_accumulate(ctx, oracle):
    """T=11 crosses the 8-token pass boundary; MM_FWD_ACCUMULATE adds to out."""
    print("ffn multi-token accumulate", flush=True)
    H, E, K, I, NS, T = 256, 16, 4, 64, 2, 11
    w = synth.moe_layer(41, H, E, I, NS)
    _layer_ctx(ctx, w, H, E, NS, K, I)
    x = synth.activations(42, T, H)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    ro, ri, rw, rp = oracle.ffn_compute_rows(cfg, w, x)
    out, idx, wt, probs = ctx.moe_forward(0, x)
    assert np.array_equal(idx, ri)
    assert max_abs_rel(out, ro) < TOL
    base = synth.activations(43, T, H)
    dx, dout = ctx.to_device(x), ctx.to_device(base)
    ctx.moe_forward_dev(0, T, dx, dout, flags=mlamoe.MM_FWD_ACCUMULATE)
    acc = dout.download(np.float32, (T, H))
    assert max_abs_rel(acc - base, ro) < TOL


@pytest.mark.parametrize("K,I,NS", [(4, 72, 1), (8, 2304, 1)])
def test_ffn_down_hidden_row_forms(ctx, oracle, K, I, NS):
    """The down stage stages a token's concatenated hidden row (K I + NS I
    floats) in LDS up to 64 KB, in 1 KB pieces (360 floats: the second piece
    partly past the row), and reads it from global memory beyond (20736
    floats)."""
    print(f"ffn down hidden row K={K} I={I}", flush=True)
    H, E, T = 128, 8, 3
    w = synth.moe_layer(51 + K, H, E, I, NS)
    _layer_ctx(ctx, w, H, E, NS, K, I)
    x = synth.activations(52 + K, T, H)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    ro, ri, rw, rp = oracle.ffn_compute_rows(cfg, w, x)
    out, idx, wt, probs = ctx.moe_forward(0, x)
    assert np.array_equal(idx, ri)
    assert max_abs_rel(out, ro) < TOL


@pytest.mark.parametrize("H", [1032, 4096])
def test_ffn_gate_up_x_forms(ctx, oracle, H):
    """The gate/up stage stages x in LDS in 1 KB pieces: 1032 values (the
    last piece partly past x, chunks past the row clamped) and 4096 (two
    groups of chunks per row pair, the second reading the staged x)."""
    print(f"ffn gate/up x H={H}", flush=True)
    E, K, I, NS, T = 8, 2, 64, 1, 2
    w = synth.moe_layer(61 + H, H, E, I, NS)
    _layer_ctx(ctx, w, H, E, NS, K, I)
    x = synth.activations(62 + H, T, H)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    ro, ri, rw, rp = oracle.ffn_compute_rows(cfg, w, x)
    out, idx, wt, probs = ctx.moe_forward(0, x)
    assert np.array_equal(idx, ri)
    assert max_abs_rel(out, ro) < TOL


def test_rejects_bad_shapes(ctx):
    with pytest.raises(mlamoe.MMError):
        ctx.moe_init(100, 8, 1, 2, 12)          # H not a multiple of 8
    ctx.moe_init(64, 8, 1, 2, 16)
    with pytest.raises(mlamoe.MMError):        # layer not loaded
        ctx.moe_forward(0, np.zeros((1, 64), np.float32))


@pytest.mark.parametrize("H,E,T", [(2048, 64, 29), (1000, 40, 29), (256, 160, 29), (2048, 64, 1),
                                   (2048, 64, 300)])
def test_router_logits_bit_exact(ctx, oracle, H, E, T):
    """Logits-only router: bit-identical to the reference matmul (run.c:29-37,
    sequential fp32, no FMA), for a partial last chunk (H=1000), more than 64
    experts per wave (E=160), one token, and more tokens than the
    one-token-per-block form takes (T=300, the chain-per-lane form); the
    optional prior is a plain fp32 add."""
    print(f"router logits H={H} E={E} T={T}", flush=True)
    K, I = 4, 8
    w = synth.moe_layer(55 + E, H, E, I, 0)
    _layer_ctx(ctx, w, H, E, 0, K, I)
    x = synth.activations(56, T, H)
    ref = oracle.matmul(x, w["moe_gate"])
    got = ctx.router_logits(0, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    z = synth.zipf_prior(57, E)
    got2 = ctx.router_logits(0, x, z)
    assert np.array_equal(got2.view(np.uint32), (ref + z).view(np.uint32))
    # routing from those logits equals routing from x
    out_a, idx_a, *_ = ctx.moe_forward(0, x)
    out_b, idx_b, *_ = ctx.moe_forward(0, x, logits=got)
    assert np.array_equal(idx_a, idx_b) and np.array_equal(out_a, out_b)
