"""Shared pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X; everything else runs on the CPU.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "mla-moe_amd"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def max_abs_rel(y, r):
    """Normwise error max|y - r| / max|r|, the tolerance metric of this path."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(y - r)) / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    pyoracle.lib()
    return pyoracle


def front_case(g, name):
    """Rebuild one decode-front golden case of mla_front.npz: its dimensions,
    the weights (synth.attn_layer, checked against the stored checksums) and
    the earlier latent-cache rows, exactly as tests/golden/make_golden.py
    drew them."""
    from mlamoe import synth
    H, NH, QKN, QKR, KVL, VHD, q_lora, il, pos, seed = (int(v) for v in g[f"{name}_cfg"])
    w = synth.attn_layer(seed, H, NH, QKN, QKR, KVL, VHD, q_lora)
    for k, v in w.items():
        if v is not None:
            assert synth.checksum_u16(v) == int(g[f"{name}_sum_{k}"]), k
    r = np.random.default_rng(seed + 1)
    for shape, std in (((2, H), 1.0), ((4, H), 0.02), ((4, H), 0.02), ((H, 4), 0.02),
                       ((2, H), 0.02)):
        synth.normal_bf16(r, shape, std)   # embed, dense FFN and lm_head draws
    cache_in = synth.normal_bf16(r, (pos, KVL + QKR), 1.0)
    assert synth.checksum_u16(cache_in) == int(g[f"{name}_sum_cache"])
    eps = g[f"{name}_eps"]
    return dict(H=H, NH=NH, QKN=QKN, QKR=QKR, KVL=KVL, VHD=VHD, q_lora=q_lora, il=il, pos=pos,
                rms_eps=float(eps[0]), mla_eps=float(eps[1]), inv=g[f"{name}_inv"],
                x=g[f"{name}_x"], w=w, cache_in=cache_in)


def engine_case(name="dsv2"):
    """One engine golden model (tests/golden/engine.npz: "dsv2" or "glm"),
    rebuilt from its seed and checked against the stored checksums:
    (config dict, model, {tokens, inv, logits})."""
    sys.path.insert(0, GOLDEN)
    from make_golden import ENGINE_CASES, engine_model
    from mlamoe import synth
    g = load_golden("engine.npz")
    m = engine_model(name)
    for k in ("embed", "final_norm", "lm_head"):
        assert synth.checksum_u16(m[k]) == int(g[f"{name}_sum_{k}"]), k
    for l, lw in enumerate(m["layers"]):
        for k, v in lw.items():
            if v is not None and v.dtype == np.uint16:
                assert synth.checksum_u16(v) == int(g[f"{name}_sum_l{l}_{k}"]), (l, k)
    return (dict(ENGINE_CASES[name][0]), m,
            {k: g[f"{name}_{k}"] for k in ("tokens", "inv", "logits")})
