"""Write the golden vectors under tests/golden/ from the reference's own code.

Runs only in the build container, where /root/reference exists: it calls the
reference's src/run.c compiled from its own sources into oracle/_ref/libref.so
(`make -C oracle ref`) and stores inputs and outputs as .npz fixtures
(numpy, no pickles).  Large weight tensors are not stored; they are
regenerated from the recorded seed with mlamoe.synth, and a checksum of each
regenerated tensor is stored so a test can prove it rebuilt the same bytes.

    python tests/golden/make_golden.py [fixture ...]
"""
from __future__ import annotations

import ctypes as C
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "mla-moe_amd"))

import pyoracle as O  # noqa: E402
from mlamoe import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def gen_matmul():
    rng = np.random.default_rng(101)
    d = {}
    for name, (d_out, n_in) in dict(tiny=(7, 13), odd=(5, 129)).items():
        x = synth.normal_f32(rng, (n_in,))
        w = synth.normal_bf16(rng, (d_out, n_in), 0.02)
        d[f"{name}_x"], d[f"{name}_w"], d[f"{name}_y"] = x, w, O.ref_matmul(x, w)
    # router-shaped [64, 2048] and expert-shaped [1408, 2048], by seed
    for name, (seed, d_out, n_in) in dict(router=(102, 64, 2048),
                                          expert=(103, 1408, 2048)).items():
        r = np.random.default_rng(seed)
        w = synth.normal_bf16(r, (d_out, n_in), 0.02)
        x = synth.normal_f32(r, (n_in,))
        d[f"{name}_seed"] = np.int64(seed)
        d[f"{name}_shape"] = np.array([d_out, n_in], np.int64)
        d[f"{name}_wsum"] = np.uint64(synth.checksum_u16(w))
        d[f"{name}_y"] = O.ref_matmul(x, w)
    np.savez_compressed(os.path.join(OUT, "matmul.npz"), **d)


def gen_softmax_silu():
    rng = np.random.default_rng(201)
    d = {}
    cases = {
        "router": synth.normal_f32(rng, (64,)),
        "ctx": synth.normal_f32(rng, (4096,), 3.0),
        "masked": np.where(rng.random(33) < 0.3, -np.inf, synth.normal_f32(rng, (33,))),
        "equal": np.full(64, 0.25, np.float32),
    }
    for k, v in cases.items():
        v = v.astype(np.float32)
        d[f"softmax_{k}_in"] = v
        d[f"softmax_{k}_out"] = O.ref_softmax(v)
    xs = np.concatenate([synth.normal_f32(rng, (256,), 4.0),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 87.0, -87.0,
                                   100.0, -100.0], np.float32)]).astype(np.float32)
    d["silu_in"] = xs
    d["silu_out"] = np.array([O.ref().ref_silu(C.c_float(float(v))) for v in xs], np.float32)
    np.savez_compressed(os.path.join(OUT, "softmax_silu.npz"), **d)


def gen_ffn_tiny():
    """ffn_compute on tiny layers, three router flavours, 5 tokens each."""
    H, E, K, I, NS, T = 64, 8, 3, 24, 2, 5
    d = {}
    flavours = {
        "dsv2": dict(sig=0, norm=0, scale=1.0, bias=False, zero_gate=False),
        "glm": dict(sig=1, norm=1, scale=1.8, bias=True, zero_gate=False),
        "tie": dict(sig=0, norm=0, scale=1.0, bias=False, zero_gate=True),
    }
    for i, (name, f) in enumerate(flavours.items()):
        w = synth.moe_layer(300 + i, H, E, I, NS, gate_bias=f["bias"])
        if f["zero_gate"]:
            w["moe_gate"] = np.zeros_like(w["moe_gate"])
        x = synth.activations(310 + i, T, H)
        cfg = O.moe_cfg(H, E, NS, K, I, f["sig"], f["norm"], f["scale"])
        outs = [O.ref_ffn_compute(cfg, w, x[t]) for t in range(T)]
        for k in ("moe_gate", "eg", "eu", "ed", "sg", "su", "sd"):
            d[f"{name}_{k}"] = w[k]
        if w["moe_gate_bias"] is not None:
            d[f"{name}_bias"] = w["moe_gate_bias"]
        d[f"{name}_cfg"] = np.array([H, E, NS, K, I, f["sig"], f["norm"]], np.int64)
        d[f"{name}_scale"] = np.float32(f["scale"])
        d[f"{name}_x"] = x
        d[f"{name}_out"] = np.stack([o[0] for o in outs])
        d[f"{name}_idx"] = np.stack([o[1] for o in outs])
        d[f"{name}_w"] = np.stack([o[2] for o in outs])
        d[f"{name}_probs"] = np.stack([o[3] for o in outs])
    np.savez_compressed(os.path.join(OUT, "ffn_tiny.npz"), **d)


def gen_ffn_dsv2():
    """One DeepSeek-V2-Lite-shaped MoE layer (config 1), two tokens, by seed."""
    g = synth.DSV2
    seed, xseed, T = 401, 402, 2
    w = synth.moe_layer(seed, g["H"], g["E"], g["I"], g["n_shared"])
    x = synth.activations(xseed, T, g["H"])
    cfg = O.moe_cfg(g["H"], g["E"], g["n_shared"], g["K"], g["I"])
    outs = [O.ref_ffn_compute(cfg, w, x[t]) for t in range(T)]
    d = dict(seed=np.int64(seed), xseed=np.int64(xseed), T=np.int64(T),
             out=np.stack([o[0] for o in outs]), idx=np.stack([o[1] for o in outs]),
             w=np.stack([o[2] for o in outs]), probs=np.stack([o[3] for o in outs]))
    for k in ("moe_gate", "eg", "eu", "ed", "sg", "su", "sd"):
        d[f"sum_{k}"] = np.uint64(synth.checksum_u16(w[k]))
    np.savez_compressed(os.path.join(OUT, "ffn_dsv2.npz"), **d)


def _absorbed_case(name, NH, QKN, QKR, KVL, VHD, pos, seed, store_kvb):
    H = NH * VHD                    # so that an identity o_proj returns ctx exactly
    KVD, QHD = KVL + QKR, QKN + QKR
    DI, V = 4, 2
    r = np.random.default_rng(seed)
    kv_b = synth.normal_bf16(np.random.default_rng(seed + 1), (NH * (QKN + VHD), KVL), 0.02)
    one = np.uint16(0x3F80)                                      # bf16 1.0
    embed = synth.normal_bf16(r, (V, H), 1.0)
    in_norm = np.full(H, one, np.uint16)
    q_proj = synth.normal_bf16(r, (NH * QHD, H), 0.02)
    kv_a = synth.normal_bf16(r, (KVD, H), 0.02)
    kv_a_norm = np.full(KVL, one, np.uint16)
    o_proj = np.zeros((H, NH * VHD), np.uint16)
    o_proj[np.arange(H), np.arange(H)] = one
    post_norm = np.full(H, one, np.uint16)
    dg = synth.normal_bf16(r, (DI, H), 0.02)
    du = synth.normal_bf16(r, (DI, H), 0.02)
    dd = synth.normal_bf16(r, (H, DI), 0.02)
    final_norm = np.full(H, one, np.uint16)
    lm_head = synth.normal_bf16(r, (V, H), 0.02)
    # earlier cache rows: bf16-representable values, as a bf16 cache would hold
    cache_in = synth.bf16_to_f32(synth.normal_bf16(r, (pos, KVD), 1.0))
    inv_freq = (1.0 / (10000.0 ** (np.arange(0, QKR, 2, dtype=np.float64) / QKR))).astype(np.float32)
    q = np.empty(NH * QHD, np.float32)
    f32p, u16p = C.POINTER(C.c_float), C.POINTER(C.c_uint16)
    with tempfile.TemporaryDirectory() as td:
        rc = O.ref().ref_absorbed_decode(
            NH, QKN, QKR, KVL, VHD, H, DI, V, pos, C.c_float(1e-6), _p(inv_freq, f32p),
            _p(embed, u16p), _p(in_norm, u16p), _p(q_proj, u16p), _p(kv_a, u16p),
            _p(kv_a_norm, u16p), _p(kv_b, u16p), _p(o_proj, u16p), _p(post_norm, u16p),
            _p(dg, u16p), _p(du, u16p), _p(dd, u16p), _p(final_norm, u16p), _p(lm_head, u16p),
            _p(np.ascontiguousarray(cache_in), f32p), td.encode(), _p(q, f32p))
        assert rc == 0

        def rd(n):
            return np.fromfile(os.path.join(td, f"decode_layer0_{n}.bin"), np.float32)
        kv_len = pos + 1
        ckv = rd("c_kv_cache").reshape(kv_len, KVL)
        kpe = rd("k_pe_cache").reshape(kv_len, QKR)
        d = {
            f"{name}_dims": np.array([NH, QKN, QKR, KVL, VHD, kv_len], np.int64),
            f"{name}_q": q.reshape(NH, QHD),
            f"{name}_cache": np.concatenate([ckv, kpe], axis=1),
            f"{name}_qabs": rd("q_absorbed").reshape(NH, KVL),
            f"{name}_probs": rd("attn_weights").reshape(NH, kv_len),
            f"{name}_clat": rd("ctx_latent").reshape(NH, KVL),
            f"{name}_ctx": rd("attn_out").reshape(NH, VHD),
            f"{name}_kvb_seed": np.int64(seed + 1),
            f"{name}_kvb_sum": np.uint64(synth.checksum_u16(kv_b)),
        }
        assert np.array_equal(d[f"{name}_cache"][:pos], cache_in)
        if store_kvb:
            d[f"{name}_kvb"] = kv_b
        return d


def gen_absorbed():
    d = {}
    d.update(_absorbed_case("tiny", 2, 16, 8, 32, 16, 6, 501, True))
    d.update(_absorbed_case("dsv2", 16, 128, 64, 512, 128, 40, 511, False))
    np.savez_compressed(os.path.join(OUT, "absorbed.npz"), **d)


def gen_lm_head():
    """rmsnorm (run.c:22-27), sample (run.c:503-508) and the final norm +
    lm_head matmul + sample of one small decode step (run.c:493-494)."""
    rng = np.random.default_rng(601)
    d = {}
    for name, (n, eps, xs) in dict(small=(8, 1e-6, 1.0), hidden=(2048, 1e-6, 1.0),
                                   glm=(64, 1e-5, 30.0), tiny=(64, 1e-6, 1e-3)).items():
        x = synth.normal_f32(rng, (n,), xs)
        w = synth.bf16_from_f32(1.0 + synth.normal_f32(rng, (n,), 0.1))
        d[f"rms_{name}_x"], d[f"rms_{name}_w"] = x, w
        d[f"rms_{name}_eps"] = np.float32(eps)
        d[f"rms_{name}_y"] = O.ref_rmsnorm(x, w, eps)
    lg = synth.normal_f32(rng, (1000,))
    tie = synth.normal_f32(rng, (50,))
    tie[7] = tie[31] = np.float32(tie.max() + 1.0)
    nan0 = synth.normal_f32(rng, (40,))
    nan0[0] = np.nan
    nanmid = synth.normal_f32(rng, (40,))
    nanmid[[3, 17]] = np.nan
    ninf = np.full(20, -np.inf, np.float32)
    pinf = synth.normal_f32(rng, (30,))
    pinf[[12, 20]] = np.inf
    for name, v in dict(random=lg, tie=tie, nan0=nan0, nanmid=nanmid, ninf=ninf,
                        pinf=pinf).items():
        v = v.astype(np.float32)
        d[f"sample_{name}_in"] = v
        d[f"sample_{name}_out"] = np.int32(O.ref_sample(v))
    T, V, H = 3, 512, 256
    x = synth.normal_f32(rng, (T, H))
    norm = synth.bf16_from_f32(1.0 + synth.normal_f32(rng, (H,), 0.1))
    lm = synth.normal_bf16(rng, (V, H), 0.02)
    logits = np.stack([O.ref_matmul(O.ref_rmsnorm(x[t], norm, 1e-6), lm) for t in range(T)])
    d.update(lm_x=x, lm_norm=norm, lm_w=lm, lm_eps=np.float32(1e-6), lm_logits=logits,
             lm_tokens=np.array([O.ref_sample(r) for r in logits], np.int32))
    np.savez_compressed(os.path.join(OUT, "lm_head.npz"), **d)


# config.json fields the reference's config_from_json reads (model_load.c:242-292)
_CFG_BASE = dict(num_hidden_layers=1, first_k_dense_replace=1, n_routed_experts=64,
                 n_shared_experts=2, num_experts_per_tok=6, intermediate_size=10944,
                 moe_intermediate_size=1408, vocab_size=102400, topk_method="greedy",
                 norm_topk_prob=False, routed_scaling_factor=1.0)
ROPE_CONFIGS = {
    # DeepSeek-V2-Lite's published attention/RoPE fields (YaRN, factor 40)
    "dsv2": dict(model_type="deepseek_v2", hidden_size=2048, num_attention_heads=16,
                 q_lora_rank=None, kv_lora_rank=512, qk_nope_head_dim=128, qk_rope_head_dim=64,
                 v_head_dim=128, max_position_embeddings=163840, rms_norm_eps=1e-6,
                 rope_theta=10000, rope_scaling=dict(
                     type="yarn", factor=40, beta_fast=32, beta_slow=1, mscale=0.707,
                     mscale_all_dim=0.707, original_max_position_embeddings=4096)),
    # GLM-style: q-LoRA, split-half RoPE, no rope_scaling (plain RoPE)
    "glm": dict(model_type="glm4_moe_lite", hidden_size=512, num_attention_heads=4,
                q_lora_rank=96, kv_lora_rank=512, qk_nope_head_dim=64, qk_rope_head_dim=64,
                v_head_dim=64, max_position_embeddings=202752, rms_norm_eps=1e-5,
                rope_theta=1000000, rope_scaling=None, topk_method="noaux_tc"),
    # a second YaRN correction range (low/high inside (0, dim-1), small factor)
    "yarn2": dict(model_type="deepseek_v2", hidden_size=256, num_attention_heads=2,
                  kv_lora_rank=512, qk_nope_head_dim=32, qk_rope_head_dim=64, v_head_dim=32,
                  rms_norm_eps=1e-6, rope_theta=50000, rope_scaling=dict(
                      type="yarn", factor=4, beta_fast=16, beta_slow=2,
                      original_max_position_embeddings=2048)),
}


def _ref_config(name):
    import json
    with tempfile.TemporaryDirectory() as td:
        with open(os.path.join(td, "config.json"), "w") as f:
            json.dump(dict(_CFG_BASE, **ROPE_CONFIGS[name]), f)
        return O.ref_config_rope(td)


def _front_case(name, cfg_name, seed, pos):
    """One decode token through the reference's forward_absorbed on a
    one-layer model (ref_absorbed_decode_ex): the post-RoPE q, the latent-cache
    row the reference appends at `pos`, and attn_out (o_proj . ctx)."""
    inv, ints, flts = _ref_config(cfg_name)
    QKR, inter, q_lora, NH, QKN, KVL, VHD, H = (int(v) for v in ints)
    rms_eps = float(flts[0])
    KVD, QHD = KVL + QKR, QKN + QKR
    w = synth.attn_layer(seed, H, NH, QKN, QKR, KVL, VHD, q_lora)
    r = np.random.default_rng(seed + 1)
    DI, V = 4, 2
    embed = synth.normal_bf16(r, (V, H), 1.0)
    dg = synth.normal_bf16(r, (DI, H), 0.02)
    du = synth.normal_bf16(r, (DI, H), 0.02)
    dd = synth.normal_bf16(r, (H, DI), 0.02)
    one = np.full(H, np.uint16(0x3F80), np.uint16)
    lm_head = synth.normal_bf16(r, (V, H), 0.02)
    cache_in = synth.bf16_to_f32(synth.normal_bf16(r, (pos, KVD), 1.0))
    q = np.empty(NH * QHD, np.float32)
    u16p, f32p = C.POINTER(C.c_uint16), C.POINTER(C.c_float)
    z = np.zeros(1, np.uint16)

    def u(a):
        return _p(z if a is None else a, u16p)
    with tempfile.TemporaryDirectory() as td:
        rc = O.ref().ref_absorbed_decode_ex(
            NH, QKN, QKR, KVL, VHD, H, DI, V, pos, C.c_float(rms_eps), _p(inv, f32p),
            q_lora, inter, u(w["q_a_proj"]), u(w["q_a_norm"]), u(w["q_b_proj"]),
            u(embed), u(w["in_norm"]), u(w["q_proj"]), u(w["kv_a"]), u(w["kv_a_norm"]),
            u(w["kv_b"]), u(w["o_proj"]), u(one), u(dg), u(du), u(dd), u(one), u(lm_head),
            _p(np.ascontiguousarray(cache_in), f32p), td.encode(), _p(q, f32p))
        assert rc == 0

        def rd(n):
            return np.fromfile(os.path.join(td, f"decode_layer0_{n}.bin"), np.float32)
        ckv = rd("c_kv_cache").reshape(pos + 1, KVL)
        kpe = rd("k_pe_cache").reshape(pos + 1, QKR)
        ao = rd("attn_out")
    assert np.array_equal(ckv[:pos], cache_in[:, :KVL])
    d = {f"{name}_{k}": v for k, v in dict(
        cfg=np.array([H, NH, QKN, QKR, KVL, VHD, q_lora, inter, pos, seed], np.int64),
        eps=np.array([rms_eps, flts[1]], np.float32), inv=inv,
        x=synth.bf16_to_f32(embed[0]), q=q, kv=np.concatenate([ckv[pos], kpe[pos]]),
        attn_out=ao).items()}
    for k, v in w.items():
        if v is not None:
            d[f"{name}_sum_{k}"] = np.uint64(synth.checksum_u16(v))
    d[f"{name}_sum_cache"] = np.uint64(synth.checksum_u16(synth.bf16_from_f32(cache_in)))
    return d


def gen_mla_front():
    """RoPE (run.c:47-67), the YaRN table as config_from_json +
    build_rope_inv_freq make it (model_load.c:242-325), and whole decode
    fronts (run.c:418-428) with the attention behind them (attn_out)."""
    d = {}
    rng = np.random.default_rng(700)
    for name in ROPE_CONFIGS:
        inv, ints, flts = _ref_config(name)
        d[f"cfg_{name}_inv"], d[f"cfg_{name}_ints"], d[f"cfg_{name}_flts"] = inv, ints, flts
    inv = d["cfg_dsv2_inv"]
    v = synth.normal_f32(rng, (6, 64))
    for il in (0, 1):
        for pos in (0, 1, 7, 4095, 163839):
            d[f"rope_il{il}_p{pos}_out"] = O.ref_rope_apply(v, pos, inv, il)
    d["rope_in"], d["rope_inv"] = v, inv
    d.update(_front_case("dsv2", "dsv2", 701, 1000))
    d.update(_front_case("glm", "glm", 702, 37))
    np.savez_compressed(os.path.join(OUT, "mla_front.npz"), **d)


ENGINE_CFG = dict(n_layers=3, first_dense=1, H=256, NH=2, QKN=32, QKR=64, KVL=512, VHD=32,
                  dense_inter=192, E=8, n_shared=1, K=2, I=128, vocab=384, router_sigmoid=0,
                  norm_topk=0, routed_scaling=1.0, rms_eps=1e-6)
# GLM-style: q-LoRA, split-half RoPE, sigmoid router with a score bias,
# normalised top-k, routed scaling, eps 1e-5
ENGINE_GLM_CFG = dict(ENGINE_CFG, NH=4, q_lora=96, interleaved=1, router_sigmoid=1, norm_topk=1,
                      routed_scaling=1.8, rms_eps=1e-5, K=3)
ENGINE_CASES = {"dsv2": (ENGINE_CFG, 900, False), "glm": (ENGINE_GLM_CFG, 950, True)}


def engine_model(name):
    c, seed, bias = ENGINE_CASES[name]
    return synth.model(seed, c["n_layers"], c["first_dense"], c["H"], c["NH"], c["QKN"], c["QKR"],
                       c["KVL"], c["VHD"], c["dense_inter"], c["E"], c["I"], c["n_shared"],
                       c["vocab"], gate_bias=bias, q_lora=c.get("q_lora", 0))


def gen_engine():
    """Whole decode steps of the reference's forward_absorbed (run.c:379-501)
    on three-layer models (dense layer 0, MoE layers 1-2) of both flavours,
    teacher forced on a token sequence: the logits at every position."""
    d = {}
    for name, (c, seed, _) in ENGINE_CASES.items():
        m = engine_model(name)
        inv = O.rope_inv_freq(c["QKR"], 10000.0)
        tokens = np.random.default_rng(seed + 1).integers(0, c["vocab"], 16).astype(np.int32)
        d[f"{name}_tokens"], d[f"{name}_inv"] = tokens, inv
        d[f"{name}_logits"] = O.ref_forward_tokens(c, m, tokens, inv)
        for k in ("embed", "final_norm", "lm_head"):
            d[f"{name}_sum_{k}"] = np.uint64(synth.checksum_u16(m[k]))
        for l, lw in enumerate(m["layers"]):
            for k, v in lw.items():
                if v is not None and v.dtype == np.uint16:
                    d[f"{name}_sum_l{l}_{k}"] = np.uint64(synth.checksum_u16(v))
    np.savez_compressed(os.path.join(OUT, "engine.npz"), **d)


def gen_prefill():
    """The reference's whole-prompt prefill, forward_unabsorbed (run.c:189-370),
    on the two engine models: every position's logits of a 24-token prompt
    (the reference's own dump, run.c:356-364; its router dump limits a
    prompt to 128 / n_experts_per_tok positions, run.c:324-330)."""
    d = {}
    for name, (c, seed, _) in ENGINE_CASES.items():
        m = engine_model(name)
        inv = O.rope_inv_freq(c["QKR"], 10000.0)
        tokens = np.random.default_rng(seed + 7).integers(0, c["vocab"], 24).astype(np.int32)
        d[f"{name}_tokens"], d[f"{name}_inv"] = tokens, inv
        d[f"{name}_logits"] = O.ref_forward_tokens(c, m, tokens, inv, prefill=True)
    np.savez_compressed(os.path.join(OUT, "prefill.npz"), **d)


GENERATORS = dict(prefill=lambda: gen_prefill(), engine=lambda: gen_engine(), mla_front=lambda: gen_mla_front(), matmul=lambda: gen_matmul(), softmax_silu=lambda: gen_softmax_silu(),
                  ffn_tiny=lambda: gen_ffn_tiny(), absorbed=lambda: gen_absorbed(),
                  ffn_dsv2=lambda: gen_ffn_dsv2(), lm_head=lambda: gen_lm_head())

if __name__ == "__main__":
    if not O.ref_available():
        O.build(ref=True)
    # python make_golden.py [name ...]: only the named fixtures
    for name in (sys.argv[1:] or list(GENERATORS)):
        GENERATORS[name]()
    for f in sorted(os.listdir(OUT)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(OUT, f)))
