"""GPU parity of the synchronous host-pointer entry points, which replace the
reference's call sites one for one:

  - ffn_compute (src/run.c:116-162) at the decode step's call site
    (src/run.c:472), for every layer of a model with first_k_dense = 1: the
    dense SwiGLU branch (src/run.c:119-122) on layer 0 and the MoE branch on
    layer 1, with the router's scores that the reference leaves in
    s->moe_logits (src/run.c:124-129);
  - the prefill loop over T tokens (src/run.c:291-313) as one mm_moe_forward;
  - matmul (src/run.c:29-37) with host x, y and host weights (kv_a_proj at
    src/run.c:424, o_proj at src/run.c:468);
  - the absorbed per-head chain (src/run.c:430-460) on the reference's own
    fp32 latent cache.

Bars: routing identical; scores within 2 ulp (e^x rounding); outputs
max-abs-rel (normwise) <= 2e-3 of the CPU oracle, which is bit-exact to the
reference's compiled C; where two device paths do the same arithmetic, the
same bits.
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
DI = 10944                    # DeepSeek-V2-Lite's dense_inter_size (layer 0)


def ulp_diff(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


@pytest.fixture(scope="module")
def model():
    """Layer 0 dense (gate/up [DI, H], down [H, DI]), layer 1 MoE, bf16."""
    r = np.random.default_rng(900)
    dense = dict(gate=synth.normal_bf16(r, (DI, H)), up=synth.normal_bf16(r, (DI, H)),
                 down=synth.normal_bf16(r, (H, DI)))
    return dense, synth.moe_layer(901, H, E, I, NS)


def _ctx(model, flags=mlamoe.MM_LOAD_BF16):
    dense, moe = model
    c = mlamoe.Context(0)
    c.moe_init(H, E, NS, K, I, n_layers=2)
    c.moe_load_dense_layer(0, dense["gate"], dense["up"], dense["down"])
    c.moe_load_layer(1, moe, flags)
    return c


def test_ffn_compute_call_site_dense_and_moe(oracle, model):
    """run.c:472, ffn_compute(c, w, s, l, xb, mo, NULL, NULL), replayed for
    l = 0 (dense) and l = 1 (MoE) on three tokens through mm_ffn_compute."""
    dense, moe = model
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    xs = synth.activations(902, 3, H)
    with _ctx(model) as ctx:
        for t in range(3):
            print(f"ffn_compute call site: token {t}", flush=True)
            out0, i0, w0, p0 = ctx.ffn_compute(0, xs[t])
            ref0 = oracle.swiglu_rows(xs[t], dense["gate"], dense["up"], dense["down"])[0]
            assert max_abs_rel(out0, ref0) < TOL
            # the dense branch returns before the router: nothing written
            assert np.all(i0 == -1) and np.all(np.isnan(w0)) and np.all(np.isnan(p0))
            out1, i1, w1, p1 = ctx.ffn_compute(1, xs[t])
            ro, ri, rw, rp = oracle.ffn_compute_rows(cfg, moe, xs[t][None])
            assert np.array_equal(i1, ri[0])
            assert ulp_diff(w1, rw[0]).max() <= 2 and ulp_diff(p1, rp[0]).max() <= 2
            assert max_abs_rel(out1, ro[0]) < TOL
            # the reference's own compiled ffn_compute, where it is built here
            if oracle.ref_available():
                so, si, sw, sp = oracle.ref_ffn_compute(cfg, moe, xs[t])
                assert np.array_equal(i1, si) and ulp_diff(p1, sp).max() <= 2
                assert max_abs_rel(out1, so) < TOL


@pytest.mark.parametrize("T", [1, 4, 70])
def test_moe_forward_host_dense_layer(oracle, model, T):
    """The dense branch over T tokens (GEMV up to 4 rows, the skinny MFMA
    GEMM above), overwrite and accumulate, against the oracle's swiglu on a
    row subset (tokens are independent)."""
    dense, _ = model
    print(f"dense layer host forward T={T}", flush=True)
    x = synth.activations(903 + T, T, H)
    y0 = synth.activations(904 + T, T, H)
    sub = np.unique(np.linspace(0, T - 1, min(T, 6)).astype(int))
    ref = oracle.swiglu_rows(x[sub], dense["gate"], dense["up"], dense["down"])
    with _ctx(model) as ctx:
        out, idx, w, p = ctx.moe_forward_host(0, x, mlamoe.MM_FWD_BF16)
        acc, *_ = ctx.moe_forward_host(0, x, mlamoe.MM_FWD_BF16 | mlamoe.MM_FWD_ACCUMULATE, out=y0)
        # the format flag does not apply to the dense layer (bf16 weights)
        o8, *_ = ctx.moe_forward_host(0, x, mlamoe.MM_FWD_INT8)
        # the device entry point, in place (out aliasing xn)
        dx = ctx.to_device(x)
        ctx.moe_forward_dev(0, T, dx, dx, flags=mlamoe.MM_FWD_ACCUMULATE)
        inplace = dx.download()
    assert np.all(idx == -1) and np.all(np.isnan(w)) and np.all(np.isnan(p))
    assert max_abs_rel(out[sub], ref) < TOL
    assert max_abs_rel(acc[sub] - y0[sub], ref) < TOL
    assert np.array_equal(o8.view(np.uint32), out.view(np.uint32))
    assert max_abs_rel(inplace[sub] - x[sub], ref) < TOL


@pytest.mark.parametrize("fmt", ["bf16", "int8"])
def test_moe_forward_host_matches_device(oracle, model, fmt):
    """The prefill loop (run.c:291-313) as one host-pointer call: T = 300
    tokens of the MoE layer (int8: the tiled grouped GEMM) give the same
    bits as the device entry point, and the bf16 experts match the oracle's
    ffn_compute on a token subset."""
    _, moe = model
    T = 300
    print(f"MoE host forward T={T} {fmt}", flush=True)
    flags = mlamoe.MM_FWD_INT8 if fmt == "int8" else mlamoe.MM_FWD_BF16
    x = synth.activations(905, T, H)
    with _ctx(model, mlamoe.MM_LOAD_BF16 | mlamoe.MM_LOAD_INT8) as ctx:
        out, idx, w, p = ctx.moe_forward_host(1, x, flags)
        do, di, dw, dp = ctx.moe_forward(1, x, flags=flags)
    assert np.array_equal(idx, di) and np.array_equal(w.view(np.uint32), dw.view(np.uint32))
    assert np.array_equal(p.view(np.uint32), dp.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), do.view(np.uint32))
    if fmt == "bf16":
        cfg = oracle.moe_cfg(H, E, NS, K, I)
        sub = np.arange(0, T, 37)
        ro, ri, *_ = oracle.ffn_compute_rows(cfg, moe, x[sub])
        assert np.array_equal(idx[sub], ri)
        assert max_abs_rel(out[sub], ro) < TOL


@pytest.mark.parametrize("T,d_out,n_in", [(1, 576, 2048), (1, 2048, 2048), (3, 3072, 2048),
                                          (64, 576, 2048), (512, 2048, 2048)])
def test_matmul_host(oracle, T, d_out, n_in):
    """matmul(y, x, w, d_out, n_in) with host pointers throughout: kv_a_proj
    (run.c:424) and o_proj (run.c:468) at one token, and batched rows.  The
    host weight is uploaded on first use and reused (a second call gives the
    same bits); with the weight already on the device, the same bits again."""
    print(f"host matmul T={T} d_out={d_out} n_in={n_in}", flush=True)
    r = np.random.default_rng(T * 7 + d_out)
    w = synth.normal_bf16(r, (d_out, n_in))
    x = synth.normal_f32(r, (T, n_in))
    y0 = synth.normal_f32(r, (T, d_out))
    ref = oracle.matmul(x, w)
    with mlamoe.Context(0) as ctx:
        y = ctx.matmul_host(x, w)
        y2 = ctx.matmul_host(x, w)
        ya = ctx.matmul_host(x, w, mlamoe.MM_MATMUL_W_HOST | mlamoe.MM_MATMUL_ACCUMULATE, y0=y0)
        yd = ctx.matmul_host(x, ctx.to_device(w), 0)
        ctx.host_weights_release()
        y3 = ctx.matmul_host(x, w)
    assert max_abs_rel(y, ref) < 1e-5
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    assert np.array_equal(y.view(np.uint32), yd.view(np.uint32))
    assert np.array_equal(y.view(np.uint32), y3.view(np.uint32))
    assert max_abs_rel(ya - y0, ref) < 1e-5


@pytest.mark.parametrize("B,kv_len,stride", [(1, 1, 1), (2, 100, 130), (4, 1100, 1100)])
def test_absorbed_decode_host_fp32_cache(oracle, B, kv_len, stride):
    """The absorbed chain (run.c:430-460) on the reference's fp32 latent
    cache through the host-pointer entry point: the same bits as the device
    entry point fed the cache rounded to bf16 (the element type the kernels
    read), within 2e-3 of the oracle on that rounded cache, and within the
    rounding's own 2^-8 of the oracle on the fp32 cache."""
    NH, QKN, QKR, KVL, VHD = 16, 128, 64, 512, 128
    print(f"host absorbed decode B={B} kv_len={kv_len} stride={stride}", flush=True)
    r = np.random.default_rng(B * 1000 + kv_len)
    kv_b = synth.normal_bf16(r, (NH * (QKN + VHD), KVL))
    q = synth.normal_f32(r, (B, NH, QKN + QKR))
    cache = synth.normal_f32(r, (B, stride, KVL + QKR))
    lens = np.array([max(1, kv_len - 7 * b) for b in range(B)], np.int32)
    with mlamoe.Context(0) as ctx:
        ctx.mla_init(NH, QKN, QKR, KVL, VHD)
        ctx.mla_load_layer(0, kv_b)
        ctx_o, qabs, probs, clat = ctx.mla_absorbed_decode_host(0, q, cache, kv_len, kv_lens=lens)
        rne = np.asarray(cache[:, :kv_len], np.float32).view(np.uint32)
        rne = ((rne + 0x7FFF + ((rne >> 16) & 1)) >> 16).astype(np.uint16)
        d_ctx, d_qabs, d_probs, d_clat = ctx.mla_absorbed_decode(0, q, rne, kv_len, kv_lens=lens)
    assert np.array_equal(ctx_o.view(np.uint32), d_ctx.view(np.uint32))
    assert np.array_equal(clat.view(np.uint32), d_clat.view(np.uint32))
    for b in range(B):
        n = int(lens[b])
        # the oracle on the rounded cache: the BASELINE bar, 2e-3
        rc, rq, rp, rl = oracle.absorbed_decode(q[b:b + 1], kv_b, rne[b:b + 1], n, NH, QKN, QKR,
                                                KVL, VHD)
        assert max_abs_rel(qabs[b], rq[0]) < 1e-5
        assert max_abs_rel(probs[b, :, :n], rp[0]) < TOL
        assert max_abs_rel(clat[b], rl[0]) < TOL
        assert max_abs_rel(ctx_o[b], rc[0]) < TOL, b
        # the oracle on the fp32 cache itself: rounding a cache element to
        # bf16 moves it by up to 2^-9 of its magnitude (half a unit in the
        # 8-bit significand's last place), which kv_len = 1 (clat = c_kv[0])
        # passes straight through: bar 2^-8
        fc, fq, fp, fl = oracle.absorbed_decode(q[b:b + 1], kv_b, cache[b:b + 1], n, NH, QKN, QKR,
                                                KVL, VHD)
        assert max_abs_rel(probs[b, :, :n], fp[0]) < 2.0 ** -8
        assert max_abs_rel(clat[b], fl[0]) < 2.0 ** -8
        assert max_abs_rel(ctx_o[b], fc[0]) < 2.0 ** -8, b


def test_boundary_errors(model):
    """Call-order and argument errors come back as status codes."""
    dense, moe = model
    with _ctx(model) as ctx:
        with pytest.raises(mlamoe.MMError) as e:
            ctx.moe_load_dense_layer(0, dense["gate"], dense["up"], dense["down"])
        assert e.value.status == -5                      # already loaded
        dx = ctx.to_device(synth.activations(906, 2, H))
        dl = ctx.empty((2, E), np.float32)
        with pytest.raises(mlamoe.MMError) as e:
            ctx.router_logits_dev(0, 2, dx, dl)           # a dense layer has no router
        assert e.value.status == -5
        with pytest.raises(mlamoe.MMError) as e:
            ctx.moe_forward_i8_debug(0, synth.activations(907, 2, H))
        assert e.value.status == -1
    with mlamoe.Context(0) as ctx:
        ctx.mla_init(16)
        with pytest.raises(mlamoe.MMError):
            ctx.mla_absorbed_decode_host(0, np.zeros((1, 16, 192), np.float32),
                                         np.zeros((1, 4, 576), np.float32), 4)   # not loaded
