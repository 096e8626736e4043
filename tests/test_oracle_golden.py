"""The CPU oracle against golden vectors written by the reference's own
compiled src/run.c (tests/golden/make_golden.py), bit for bit, and against
the compiled reference itself on fresh random inputs where it is built."""
import json
import os
import tempfile

import numpy as np
import pytest

from conftest import load_golden
from mlamoe import synth


def test_bf16_conversions(oracle):
    # include/tensor.h:9-20: shift up, truncate down (no round-to-nearest)
    L = oracle.lib()
    assert L.or_bf16_to_f32(0x3F80) == 1.0
    assert L.or_bf16_to_f32(0xC000) == -2.0
    assert L.or_f32_to_bf16(1.0) == 0x3F80
    # 1 + 2^-8 + 2^-9 would round up to 0x3F81 under RNE; truncation keeps 0x3F80
    assert L.or_f32_to_bf16(1.0 + 2 ** -8 + 2 ** -9) == 0x3F80
    assert L.or_f32_to_bf16(-1.0 - 2 ** -8 - 2 ** -9) == 0xBF80
    rng = np.random.default_rng(0)
    x = rng.standard_normal(1000).astype(np.float32)
    u = synth.bf16_from_f32(x)
    assert all(L.or_f32_to_bf16(float(v)) == b for v, b in zip(x[:100], u[:100]))
    back = synth.bf16_to_f32(u)
    assert np.all(np.abs(back) <= np.abs(x)) and np.all(np.sign(back) == np.sign(x))


def test_matmul_golden(oracle):
    g = load_golden("matmul.npz")
    for name in ("tiny", "odd"):
        y = oracle.matmul(g[f"{name}_x"], g[f"{name}_w"])
        assert np.array_equal(y.view(np.uint32), g[f"{name}_y"].view(np.uint32)), name
    for name in ("router", "expert"):
        r = np.random.default_rng(int(g[f"{name}_seed"]))
        d_out, n_in = (int(v) for v in g[f"{name}_shape"])
        w = synth.normal_bf16(r, (d_out, n_in), 0.02)
        x = synth.normal_f32(r, (n_in,))
        assert synth.checksum_u16(w) == int(g[f"{name}_wsum"])
        y = oracle.matmul(x, w)
        assert np.array_equal(y.view(np.uint32), g[f"{name}_y"].view(np.uint32)), name


def test_softmax_silu_golden(oracle):
    g = load_golden("softmax_silu.npz")
    for k in ("router", "ctx", "masked", "equal"):
        y = oracle.softmax(g[f"softmax_{k}_in"])
        assert np.array_equal(y.view(np.uint32), g[f"softmax_{k}_out"].view(np.uint32)), k
    L = oracle.lib()
    s = np.array([L.or_silu(float(v)) for v in g["silu_in"]], np.float32)
    assert np.array_equal(s.view(np.uint32), g["silu_out"].view(np.uint32))


@pytest.mark.parametrize("flavour", ["dsv2", "glm", "tie"])
def test_ffn_tiny_golden(oracle, flavour):
    g = load_golden("ffn_tiny.npz")
    H, E, NS, K, I, sig, norm = (int(v) for v in g[f"{flavour}_cfg"])
    cfg = oracle.moe_cfg(H, E, NS, K, I, sig, norm, float(g[f"{flavour}_scale"]))
    w = {k: g[f"{flavour}_{k}"] for k in ("moe_gate", "eg", "eu", "ed", "sg", "su", "sd")}
    w["moe_gate_bias"] = g.get(f"{flavour}_bias")
    out, idx, wt, probs = oracle.ffn_compute_rows(cfg, w, g[f"{flavour}_x"])
    assert np.array_equal(idx, g[f"{flavour}_idx"])
    for a, b in ((out, "out"), (wt, "w"), (probs, "probs")):
        assert np.array_equal(a.view(np.uint32), g[f"{flavour}_{b}"].view(np.uint32)), b
    if flavour == "tie":
        # all logits equal: strict '>' keeps the lowest index (run.c:140)
        assert np.all(idx == np.arange(K))
        assert np.all(probs == np.float32(1.0 / E))


def test_ffn_dsv2_golden(oracle):
    """Config-1 layer (H=2048, 64 experts, I=1408, top-6, 2 shared), regenerated
    from its seed; output, routing and scores bit-identical to the reference."""
    g = load_golden("ffn_dsv2.npz")
    d = synth.DSV2
    w = synth.moe_layer(int(g["seed"]), d["H"], d["E"], d["I"], d["n_shared"])
    for k in ("moe_gate", "eg", "eu", "ed", "sg", "su", "sd"):
        assert synth.checksum_u16(w[k]) == int(g[f"sum_{k}"]), k
    x = synth.activations(int(g["xseed"]), int(g["T"]), d["H"])
    cfg = oracle.moe_cfg(d["H"], d["E"], d["n_shared"], d["K"], d["I"])
    out, idx, wt, probs = oracle.ffn_compute_rows(cfg, w, x)
    assert np.array_equal(idx, g["idx"])
    assert np.array_equal(out.view(np.uint32), g["out"].view(np.uint32))
    assert np.array_equal(wt.view(np.uint32), g["w"].view(np.uint32))
    assert np.array_equal(probs.view(np.uint32), g["probs"].view(np.uint32))


@pytest.mark.parametrize("case", ["tiny", "dsv2"])
def test_absorbed_golden(oracle, case):
    """The absorbed per-head chain against the reference forward_absorbed's
    own layer-0 dumps (run.c:430-490)."""
    g = load_golden("absorbed.npz")
    NH, QKN, QKR, KVL, VHD, kv_len = (int(v) for v in g[f"{case}_dims"])
    if f"{case}_kvb" in g:
        kv_b = g[f"{case}_kvb"]
    else:
        kv_b = synth.normal_bf16(np.random.default_rng(int(g[f"{case}_kvb_seed"])),
                                 (NH * (QKN + VHD), KVL), 0.02)
    assert synth.checksum_u16(kv_b) == int(g[f"{case}_kvb_sum"])
    q = g[f"{case}_q"][None]
    cache = g[f"{case}_cache"][None].astype(np.float32)
    ctx, qabs, probs, clat = oracle.absorbed_decode(q, kv_b, cache, kv_len, NH, QKN, QKR,
                                                    KVL, VHD)
    for a, b in ((qabs[0], "qabs"), (probs[0], "probs"), (clat[0], "clat"),
                 (ctx[0].reshape(NH, VHD), "ctx")):
        assert np.array_equal(a.view(np.uint32), g[f"{case}_{b}"].view(np.uint32)), b


needs_ref = pytest.mark.skipif(
    not __import__("pyoracle").ref_available(),
    reason="oracle/_ref/libref.so is built only where /root/reference exists")


@needs_ref
def test_matmul_vs_reference_random(oracle):
    rng = np.random.default_rng(7)
    for d_out, n_in in ((3, 1), (17, 255), (64, 2048), (2048, 1408)):
        x = synth.normal_f32(rng, (n_in,))
        w = synth.normal_bf16(rng, (d_out, n_in), 0.05)
        a, b = oracle.matmul(x, w), oracle.ref_matmul(x, w)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("seed", [11, 12, 13])
def test_ffn_vs_reference_random(oracle, seed):
    H, E, K, I, NS = 128, 16, 4, 40, 1
    sig = seed % 2
    w = synth.moe_layer(seed, H, E, I, NS, gate_bias=bool(sig))
    cfg = oracle.moe_cfg(H, E, NS, K, I, sig, sig, 1.0 + 0.4 * sig)
    x = synth.activations(seed + 100, 3, H)
    out, idx, wt, probs = oracle.ffn_compute_rows(cfg, w, x)
    for t in range(3):
        ro, ri, rw, rp = oracle.ref_ffn_compute(cfg, w, x[t])
        assert np.array_equal(idx[t], ri)
        assert np.array_equal(out[t].view(np.uint32), ro.view(np.uint32))
        assert np.array_equal(wt[t].view(np.uint32), rw.view(np.uint32))
        assert np.array_equal(probs[t].view(np.uint32), rp.view(np.uint32))


def test_rmsnorm_golden(oracle):
    g = load_golden("lm_head.npz")
    for name in ("small", "hidden", "glm", "tiny"):
        y = oracle.rmsnorm(g[f"rms_{name}_x"], g[f"rms_{name}_w"], float(g[f"rms_{name}_eps"]))
        assert np.array_equal(y.view(np.uint32), g[f"rms_{name}_y"].view(np.uint32)), name


def test_argmax_golden(oracle):
    g = load_golden("lm_head.npz")
    for name in ("random", "tie", "nan0", "nanmid", "ninf", "pinf"):
        assert oracle.argmax(g[f"sample_{name}_in"]) == int(g[f"sample_{name}_out"]), name


def test_lm_head_golden(oracle):
    g = load_golden("lm_head.npz")
    logits, tokens = oracle.lm_head_rows(g["lm_x"], g["lm_norm"], float(g["lm_eps"]), g["lm_w"])
    assert np.array_equal(logits.view(np.uint32), g["lm_logits"].view(np.uint32))
    assert np.array_equal(tokens, g["lm_tokens"])


@needs_ref
def test_rmsnorm_argmax_vs_reference_random(oracle):
    rng = np.random.default_rng(17)
    for n, eps, scale in ((1, 1e-6, 1.0), (100, 1e-5, 7.0), (2048, 1e-6, 0.01)):
        x = synth.normal_f32(rng, (n,), scale)
        w = synth.normal_bf16(rng, (n,), 1.0)
        a, b = oracle.rmsnorm(x, w, eps), oracle.ref_rmsnorm(x, w, eps)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for n in (1, 2, 1000, 102400):
        lg = synth.normal_f32(rng, (n,))
        assert oracle.argmax(lg) == oracle.ref_sample(lg)


# ---- MLA decode front (mla_front.npz) -----------------------------------------

def test_rope_inv_freq_golden(oracle):
    """The YaRN table as the reference's config_from_json + build_rope_inv_freq
    produce it from a config.json (model_load.c:242-325), bit for bit, from
    the oracle and from the library's own host code."""
    import mlamoe
    g = load_golden("mla_front.npz")
    for name in ("dsv2", "glm", "yarn2"):
        f = g[f"cfg_{name}_flts"]
        dim = int(g[f"cfg_{name}_ints"][0])
        args = (dim, *(float(v) for v in f[3:8]))
        assert np.array_equal(oracle.rope_inv_freq(*args), g[f"cfg_{name}_inv"]), name
        assert np.array_equal(mlamoe.rope_inv_freq(*args), g[f"cfg_{name}_inv"]), name
    # the parsed fields the front uses
    assert list(g["cfg_dsv2_ints"][:3]) == [64, 0, 0] and list(g["cfg_glm_ints"][:3]) == [64, 1, 96]
    assert g["cfg_glm_flts"][0] == np.float32(1e-5) and g["cfg_dsv2_flts"][1] == np.float32(1e-6)


def test_rope_apply_golden(oracle):
    g = load_golden("mla_front.npz")
    for il in (0, 1):
        for pos in (0, 1, 7, 4095, 163839):
            out = oracle.rope_apply(g["rope_in"], pos, g["rope_inv"], il)
            assert np.array_equal(out.view(np.uint32), g[f"rope_il{il}_p{pos}_out"].view(np.uint32))


@pytest.mark.parametrize("name", ["dsv2", "glm"])
def test_mla_front_golden(oracle, name):
    """q after RoPE and the latent-cache row that forward_absorbed appends
    (run.c:418-428), then the attention output behind them (run.c:430-468:
    absorbed chain on the fp32 cache, o_proj), all bit for bit."""
    from conftest import front_case
    g = load_golden("mla_front.npz")
    c = front_case(g, name)
    cfg = oracle.front_cfg(c["H"], c["NH"], c["QKN"], c["QKR"], c["KVL"], c["q_lora"],
                           c["rms_eps"], c["mla_eps"], c["il"])
    q, kv, _ = oracle.mla_front(cfg, c["w"], c["inv"], c["x"], c["pos"])
    assert np.array_equal(q[0].view(np.uint32), g[f"{name}_q"].view(np.uint32))
    assert np.array_equal(kv[0].view(np.uint32), g[f"{name}_kv"].view(np.uint32))
    cache = np.concatenate([synth.bf16_to_f32(c["cache_in"]), kv], axis=0)[None]
    ctx, _, _, _ = oracle.absorbed_decode(q.reshape(1, c["NH"], -1), c["w"]["kv_b"], cache,
                                          c["pos"] + 1, c["NH"], c["QKN"], c["QKR"], c["KVL"],
                                          c["VHD"])
    ao = oracle.matmul(ctx[0], c["w"]["o_proj"])
    assert np.array_equal(ao.view(np.uint32), g[f"{name}_attn_out"].view(np.uint32))


@pytest.mark.skipif(not __import__("pyoracle").ref_available(),
                    reason="compiled reference (oracle/_ref) not built here")
def test_rope_against_reference_random(oracle):
    rng = np.random.default_rng(31)
    for _ in range(20):
        dim = int(rng.choice([8, 32, 64, 128]))
        theta = float(rng.choice([10000.0, 50000.0, 1e6]))
        factor = float(rng.choice([1.0, 4.0, 40.0]))
        bf, bs = float(rng.choice([16.0, 32.0])), float(rng.choice([1.0, 2.0]))
        om = float(rng.choice([2048.0, 4096.0]))
        inv = oracle.rope_inv_freq(dim, theta, factor, bf, bs, om)
        # the reference's own table for the same config.json fields
        with tempfile.TemporaryDirectory() as td:
            with open(os.path.join(td, "config.json"), "w") as f:
                json.dump(dict(num_hidden_layers=1, hidden_size=64, kv_lora_rank=512,
                               qk_rope_head_dim=dim, rope_theta=theta,
                               rope_scaling=dict(type="yarn", factor=factor, beta_fast=bf,
                                                 beta_slow=bs,
                                                 original_max_position_embeddings=om)), f)
            ref_inv, _, _ = oracle.ref_config_rope(td)
        assert np.array_equal(inv, ref_inv), (dim, theta, factor, bf, bs, om)
        v = synth.normal_f32(rng, (3, dim))
        for il in (0, 1):
            pos = int(rng.integers(0, 200000))
            assert np.array_equal(oracle.rope_apply(v, pos, inv, il),
                                  oracle.ref_rope_apply(v, pos, inv, il))


# ---- whole decode steps (engine.npz) -----------------------------------------

@pytest.mark.parametrize("name", ["dsv2", "glm"])
def test_model_logits_golden(oracle, name):
    """The oracle's composition of a decode step (front, absorbed chain,
    o_proj, dense / MoE FFN, final norm, lm_head) equals the reference's
    forward_absorbed bit for bit at every position of a teacher-forced
    sequence on a dense + MoE model, in the DeepSeek-V2 flavour and the GLM
    one (q-LoRA, split-half RoPE, sigmoid router with bias, normalised and
    scaled top-k)."""
    from conftest import engine_case
    c, m, g = engine_case(name)
    lg = oracle.model_logits(c, m, g["tokens"], g["inv"])
    assert np.array_equal(lg.view(np.uint32), g["logits"].view(np.uint32))


@pytest.mark.parametrize("name", ["dsv2", "glm"])
def test_model_logits_vs_reference_prefill(oracle, name):
    """The reference's whole-prompt prefill, forward_unabsorbed (run.c:189-370:
    K/V decompressed per head, causal scores), gives the same logits at every
    prompt position as the absorbed composition the oracle (and the engine)
    uses: the two are equal in exact arithmetic (run.c:375-378), and measured
    within 3.2e-7 normwise in fp32 on both flavours (prefill.npz, written by
    the reference's own dump, run.c:356-364)."""
    from conftest import engine_case, max_abs_rel
    c, m, _ = engine_case(name)
    g = load_golden("prefill.npz")
    lg = oracle.model_logits(c, m, g[f"{name}_tokens"], g[f"{name}_inv"])
    assert max_abs_rel(lg, g[f"{name}_logits"]) < 1e-6
