"""Benchmark of the MI355X mla-moe hot path (one JSON line on stdout).

Default workload: batched decode, B=64 tokens through a
26-layer stack of DeepSeek-V2-Lite-shaped MoE FFN layers with int8
per-output-channel weights (from bf16 N(0, 0.02)), uniform-random fp32 router
logits per layer, residual carried through the stack (x += ffn(x)), weights
resident in HBM.  A step is one pass of the 64 tokens through the 26 layers.

The same line carries, under "extra", the other configurations measured in
the same run: config 3 (prefill T=2048, int8, Zipf-skewed routing, router
GEMV included), config 1 (T=1 decode layer, bf16 weights), config 5 (MLA
absorbed decode), config 2 (dense bf16 projections) and the LM head of a
decode step (vocabulary 102400, B = 1 and 64).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mla-moe_amd"))

import mlamoe  # noqa: E402
from mlamoe import synth  # noqa: E402

METRIC = "MoE FFN tok/s; decode HBM GB/s & prefill int8 TOPS vs MI355X roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
INT8_PEAK_TOPS = 5033.0        # MI355X dense int8 MFMA (no sparsity)
G = synth.DSV2                 # H=2048, E=64, K=6, I=1408, n_shared=2
H, E, K, I, NS = G["H"], G["E"], G["K"], G["I"], G["n_shared"]
S = NS * I


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def fill_layer_bf16(ctx, bufs, seed):
    for i, (k, b) in enumerate(bufs.items()):
        ctx.fill(b, int(np.prod(b.shape)), mlamoe.MM_FILL_BF16_NORMAL, seed * 16 + i, 0.02)


def bf16_buffers(ctx):
    shapes = dict(moe_gate=(E, H), eg=(E, I, H), eu=(E, I, H), ed=(E, H, I), sg=(S, H),
                  su=(S, H), sd=(H, S))
    return {k: ctx.empty(v, np.uint16) for k, v in shapes.items()}


def load_layers(ctx, n_layers, seed0, flags):
    """Synthetic bf16 weights generated on the device, then loaded (and
    quantised for int8) layer by layer through the C-ABI."""
    ctx.moe_init(H, E, NS, K, I, n_layers=n_layers)
    bufs = bf16_buffers(ctx)
    w = dict(bufs)
    w["moe_gate_bias"] = None
    for l in range(n_layers):
        fill_layer_bf16(ctx, bufs, seed0 + l)
        ctx.moe_load_layer(l, w, flags | mlamoe.MM_LOAD_DEVICE_PTRS)
    for b in bufs.values():
        b.free()
        ctx._bufs.remove(b)


def i8_gu_bytes(touched, T, R):
    """Algorithmic HBM bytes of one mm_i8_gu launch: int8 gate/up weights of
    the touched experts and the shared expert, their scales, the quantised
    activations, and the fp32 SwiGLU rows written."""
    w = touched * 2 * I * H + 2 * S * H
    sc = touched * 2 * I * 4 + 2 * S * 4
    act = T * H + T * 4
    out = R * I * 4 + T * S * 4
    return w + sc + act + out


def i8_layer_bytes(touched, T, R):
    """Algorithmic HBM bytes of a whole int8 MoE layer (all kernels): every
    touched expert's int8 weights and scales read once, activations in and
    out, and the intermediate rows each written and read once."""
    w = touched * 3 * I * H + 3 * S * H
    sc = touched * (2 * I + H) * 4 + (2 * S + H) * 4
    io = 2 * T * H * 4 + T * E * 4
    inter = (R * I * 4) * 2 + R * I + (T * S * 4) * 2 + T * S + (R * H * 4) * 2 + (T * H * 4) * 2
    return w + sc + io + inter


def kernel_avg_ms(ctx, name):
    tot, n = ctx.prof_query(name)
    return tot / max(n, 1), n


def timed(ctx, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    ctx.sync()                                    # barrier + synchronize (N = 1)
    t0 = time.perf_counter()
    ctx.timer_start()
    for _ in range(steps):
        fn()
    ms = ctx.timer_stop()                         # HIP events on the context stream
    ctx.sync()
    wall = (time.perf_counter() - t0) * 1e3
    return ms / steps, wall / steps


def profile_kernels(ctx, fn, steps, names):
    ctx.prof_enable(True)
    ctx.prof_reset()
    for _ in range(steps):
        fn()
    res = {n: kernel_avg_ms(ctx, n) for n in names}
    ctx.prof_enable(False)
    ctx.prof_reset()
    return res


def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    p = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


# ---------------------------------------------------------------------------

def bench_decode_i8(ctx, steps, warmup, B=64, L=26):
    """Config 4: B tokens through L int8 MoE layers, residual carried."""
    log(f"[decode_i8] loading {L} int8 layers")
    load_layers(ctx, L, 1000, mlamoe.MM_LOAD_INT8)
    x0 = ctx.empty((B, H), np.float32)
    ctx.fill(x0, B * H, mlamoe.MM_FILL_F32_NORMAL, 7, 1.0)
    x = ctx.empty((B, H), np.float32)
    logits = [ctx.empty((B, E), np.float32) for _ in range(L)]
    for l, lg in enumerate(logits):
        ctx.fill(lg, B * E, mlamoe.MM_FILL_F32_UNIFORM, 500 + l)
    idx = [ctx.empty((B, K), np.int32) for _ in range(L)]
    wts = ctx.empty((B, K), np.float32)
    flags = mlamoe.MM_FWD_INT8 | mlamoe.MM_FWD_ACCUMULATE
    lib, h = mlamoe.lib(), ctx.h

    def step():
        mlamoe._check(lib.mm_d2d(h, x.ptr, x0.ptr, B * H * 4))
        for l in range(L):
            mlamoe._check(lib.mm_moe_forward_dev(h, l, B, x.ptr, x.ptr, logits[l].ptr,
                                                 idx[l].ptr, wts.ptr, None, flags))
    log("[decode_i8] timing")
    ms, wall = timed(ctx, step, steps, warmup)
    touched = [len(np.unique(i.download())) for i in idx]
    R = B * K
    names = ["mm_i8_route", "mm_i8_gu", "mm_i8_quant_h", "mm_i8_down", "mm_i8_combine"]
    prof = profile_kernels(ctx, step, max(2, steps // 4), names)
    # one gate/up launch per layer covers the routed and the shared expert
    gu_ms = prof["mm_i8_gu"][0]
    gu_bytes = float(np.mean([i8_gu_bytes(t, B, R) for t in touched]))
    step_bytes = float(sum(i8_layer_bytes(t, B, R) for t in touched))
    res = dict(
        ms_per_step=ms, wall_ms_per_step=wall, tok_s=B / (ms * 1e-3),
        step_gbs=step_bytes / (ms * 1e-3) / 1e9, step_bytes=step_bytes,
        touched_experts_per_layer=float(np.mean(touched)),
        kernels_us={n: round(v[0] * 1e3, 2) for n, v in prof.items()},
        roofline=dict(bound="hbm", kernel="mm_i8_gu (gate/up GEMM, routed + shared)",
                      achieved=gu_bytes / (gu_ms * 1e-3) / 1e9, peak=HBM_PEAK_GBS,
                      unit="GB/s", bytes_per_launch=gu_bytes, avg_launch_us=gu_ms * 1e3))
    res["roofline"]["frac"] = res["roofline"]["achieved"] / HBM_PEAK_GBS
    res["roofline"]["traffic"] = traffic_from_profiles("mm_i8_gu", "decode_i8")
    return res


def bench_prefill_i8(ctx, steps, warmup, T=2048):
    """Config 3: T tokens through one int8 layer, router logits W_g x plus a
    Zipf(1.1) prior computed inside the step."""
    log("[prefill_i8] loading int8 layer")
    load_layers(ctx, 1, 3000, mlamoe.MM_LOAD_INT8)
    x = ctx.empty((T, H), np.float32)
    ctx.fill(x, T * H, mlamoe.MM_FILL_F32_NORMAL, 11, 1.0)
    prior = ctx.to_device(synth.zipf_prior(12, E, 1.1))
    logits = ctx.empty((T, E), np.float32)
    out = ctx.empty((T, H), np.float32)
    idx = ctx.empty((T, K), np.int32)
    wts = ctx.empty((T, K), np.float32)
    lib, h = mlamoe.lib(), ctx.h

    def step():
        mlamoe._check(lib.mm_moe_router_logits_dev(h, 0, T, x.ptr, prior.ptr, logits.ptr))
        mlamoe._check(lib.mm_moe_forward_dev(h, 0, T, x.ptr, out.ptr, logits.ptr, idx.ptr,
                                             wts.ptr, None, mlamoe.MM_FWD_INT8))
    log("[prefill_i8] timing")
    ms, wall = timed(ctx, step, steps, warmup)
    ii = idx.download()
    counts = np.bincount(ii.ravel(), minlength=E)
    names = ["mm_router", "mm_i8_route", "mm_i8_gemm_gu", "mm_i8_quant_h", "mm_i8_gemm_dn",
             "mm_i8_combine"]
    psteps = max(2, steps // 4)
    prof = profile_kernels(ctx, step, psteps, names)
    gk = "mm_i8_gemm_gu"
    R = T * K
    gu_ops = 2.0 * R * 2 * I * H + 2.0 * T * 2 * S * H
    dn_ops = 2.0 * R * H * I + 2.0 * T * H * S
    # grouped GEMM time per layer: one gate/up and one down launch (routed
    # and shared experts in one launch each)
    gemm_ms = prof["mm_i8_gemm_gu"][0] + prof["mm_i8_gemm_dn"][0]
    res = dict(
        ms_per_step=ms, wall_ms_per_step=wall, tok_s=T / (ms * 1e-3),
        layer_tops=(gu_ops + dn_ops) / (ms * 1e-3) / 1e12,
        gemm_tops=(gu_ops + dn_ops) / (gemm_ms * 1e-3) / 1e12,
        expert_rows_max=int(counts.max()), expert_rows_min=int(counts.min()),
        experts_touched=int((counts > 0).sum()),
        kernels_us={n: round(v[0] * 1e3, 2) for n, v in prof.items()},
        gemm_tops_gu=gu_ops / (prof["mm_i8_gemm_gu"][0] * 1e-3) / 1e12,
        gemm_tops_dn=dn_ops / (prof["mm_i8_gemm_dn"][0] * 1e-3) / 1e12,
        roofline=dict(bound="mfma", kernel="mm_i8_gemm_gu + mm_i8_gemm_dn (one launch each "
                      "per layer)",
                      achieved=(gu_ops + dn_ops) / (gemm_ms * 1e-3) / 1e12,
                      peak=INT8_PEAK_TOPS, unit="TOPS", ops_per_layer=gu_ops + dn_ops,
                      avg_launch_us=gemm_ms * 1e3 / 2))
    res["roofline"]["frac"] = res["roofline"]["achieved"] / INT8_PEAK_TOPS
    res["roofline"]["traffic"] = traffic_from_profiles("mm_i8_gemm", "prefill_i8")
    return res


def bench_decode_bf16(ctx, steps, warmup):
    """Config 1: one T=1 decode token through a bf16 MoE layer (router GEMV
    from x, top-6 softmax, 2 shared experts)."""
    log("[decode_bf16] loading bf16 layer")
    load_layers(ctx, 1, 5000, mlamoe.MM_LOAD_BF16)
    x = ctx.empty((1, H), np.float32)
    ctx.fill(x, H, mlamoe.MM_FILL_F32_NORMAL, 13, 1.0)
    out = ctx.empty((1, H), np.float32)
    idx = ctx.empty((1, K), np.int32)
    wts = ctx.empty((1, K), np.float32)
    lib, h = mlamoe.lib(), ctx.h

    def step():
        mlamoe._check(lib.mm_moe_forward_dev(h, 0, 1, x.ptr, out.ptr, None, idx.ptr, wts.ptr,
                                             None, mlamoe.MM_FWD_BF16))
    ms, wall = timed(ctx, step, steps * 20, warmup * 5)
    names = ["mm_moe_bf16_router_sh", "mm_moe_bf16_stage2_lds", "mm_moe_bf16_stage3_lds"]
    prof = profile_kernels(ctx, step, 50, names)
    nbytes = 262144 + 103809024 + 34603008      # router + 6 experts + shared (bf16)
    return dict(ms_per_step=ms, tok_s=1.0 / (ms * 1e-3), layer_gbs=nbytes / (ms * 1e-3) / 1e9,
                frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                kernels_us={n: round(v[0] * 1e3, 2) for n, v in prof.items()})


def bench_mla_decode(ctx, steps, warmup, B=32, NH=16, L=4096):
    """Config 5: MLA absorbed decode, B sequences x NH heads over a bf16
    latent cache of L positions."""
    log("[mla_decode] setup")
    QKN, QKR, KVL, VHD = 128, 64, 512, 128
    ctx.mla_init(NH, QKN, QKR, KVL, VHD)
    kvb = ctx.empty((NH * (QKN + VHD), KVL), np.uint16)
    ctx.fill(kvb, NH * (QKN + VHD) * KVL, mlamoe.MM_FILL_BF16_NORMAL, 21, 0.02)
    ctx.mla_load_layer(0, kvb, mlamoe.MM_LOAD_DEVICE_PTRS)
    cache = ctx.empty((B, L, KVL + QKR), np.uint16)
    ctx.fill(cache, B * L * (KVL + QKR), mlamoe.MM_FILL_BF16_NORMAL, 22, 1.0)
    q = ctx.empty((B, NH, QKN + QKR), np.float32)
    ctx.fill(q, B * NH * (QKN + QKR), mlamoe.MM_FILL_F32_NORMAL, 23, 1.0)
    out = ctx.empty((B, NH * VHD), np.float32)
    lib, h = mlamoe.lib(), ctx.h

    def step():
        mlamoe._check(lib.mm_mla_absorbed_decode_dev(h, 0, B, q.ptr, cache.ptr, L, None, L,
                                                     out.ptr, None, None, None))
    ms, wall = timed(ctx, step, steps * 5, warmup)
    names = ["mm_mla_qprep", "mm_mla_attn", "mm_mla_combine", "mm_mla_uv"]
    prof = profile_kernels(ctx, step, 20, names)
    nbytes = B * L * (KVL + QKR) * 2 + 2 * NH * QKN * KVL * 2   # cache + W_UK + W_UV
    attn_bytes = B * L * (KVL + QKR) * 2
    at_ms = prof["mm_mla_attn"][0]
    return dict(ms_per_step=ms, seq_per_s=B / (ms * 1e-3), gbs=nbytes / (ms * 1e-3) / 1e9,
                frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                attn_kernel_gbs=attn_bytes / (at_ms * 1e-3) / 1e9,
                kernels_us={n: round(v[0] * 1e3, 2) for n, v in prof.items()})


def bench_dense_bf16(ctx, steps, warmup, T=512):
    """Config 2: the four MLA projection GEMMs at prefill T=512, activations
    cast to bf16 on the input side, fp32 accumulation."""
    log("[dense_bf16] setup")
    shapes = dict(q_proj=(3072, 2048), kv_a=(576, 2048), kv_b=(4096, 512), o_proj=(2048, 2048))
    bufs = {}
    for i, (k, (d, n)) in enumerate(shapes.items()):
        w = ctx.empty((d, n), np.uint16)
        ctx.fill(w, d * n, mlamoe.MM_FILL_BF16_NORMAL, 31 + i, 0.02)
        x = ctx.empty((T, n), np.float32)
        ctx.fill(x, T * n, mlamoe.MM_FILL_F32_NORMAL, 41 + i, 1.0)
        y = ctx.empty((T, d), np.float32)
        bufs[k] = (w, x, y, d, n)
    lib, h = mlamoe.lib(), ctx.h

    def step():
        for w, x, y, d, n in bufs.values():
            mlamoe._check(lib.mm_matmul_bf16_dev(h, y.ptr, x.ptr, w.ptr, d, n, T,
                                                 mlamoe.MM_MATMUL_X_BF16))
    ms, wall = timed(ctx, step, steps * 5, warmup)
    prof = profile_kernels(ctx, step, 20, ["mm_gemm_bf16"])
    flops = sum(2.0 * T * d * n for _, _, _, d, n in bufs.values())
    return dict(ms_per_step=ms, tflops=flops / (ms * 1e-3) / 1e12,
                frac_bf16_peak=flops / (ms * 1e-3) / 1e12 / 2516.6,
                kernel_avg_us=round(prof["mm_gemm_bf16"][0] * 1e3, 2), gflop=flops / 1e9)


def bench_attn_layer(ctx_unused, steps, warmup, L=4096, NH=16):
    """The attention half of a DeepSeek-V2-Lite decode layer (src/run.c:418-469)
    for B sequences, each appending at position L-1 and attending all L
    positions: input norm + q_proj/kv_a projections + RoPE + kv_a_layernorm
    into the bf16 latent cache (mm_mla_front_dev), the absorbed chain
    (mm_mla_absorbed_decode_dev), o_proj with the residual add
    (mm_matmul_bf16_dev, MM_MATMUL_ACCUMULATE).  B = 1 (latency) and B = 32
    (the config-5 batch)."""
    Hd, QKN, QKR, KVL, VHD = 2048, 128, 64, 512, 128
    QD, KVD = NH * (QKN + QKR), KVL + QKR
    lib = mlamoe.lib()
    res = {}
    for B in (1, 32):
        log(f"[attn_layer] B={B} setup")
        with mlamoe.Context(0) as ctx:
            h = ctx.h
            ctx.mla_init(NH, QKN, QKR, KVL, VHD)
            ctx.mla_front_init(Hd, mlamoe.rope_inv_freq(QKR, 10000.0, 40.0, 32.0, 1.0, 4096.0))
            kvb = ctx.empty((NH * (QKN + VHD), KVL), np.uint16)
            ctx.fill(kvb, NH * (QKN + VHD) * KVL, mlamoe.MM_FILL_BF16_NORMAL, 71, 0.02)
            ctx.mla_load_layer(0, kvb, mlamoe.MM_LOAD_DEVICE_PTRS)
            shapes = dict(input_norm=(Hd,), q_proj=(QD, Hd), kv_a_proj=(KVD, Hd),
                          kv_a_norm=(KVL,), o_proj=(Hd, NH * VHD))
            wd = {}
            for i, (k, shp) in enumerate(shapes.items()):
                wd[k] = ctx.empty(shp, np.uint16)
                ctx.fill(wd[k], int(np.prod(shp)), mlamoe.MM_FILL_BF16_NORMAL, 72 + i,
                         0.1 if len(shp) == 1 else 0.02)
            ws = mlamoe.MlaFrontWeights(*[wd[k].ptr if k in wd else None
                                          for k in mlamoe.FRONT_WEIGHTS])
            cache = ctx.empty((B, L, KVD), np.uint16)
            ctx.fill(cache, B * L * KVD, mlamoe.MM_FILL_BF16_NORMAL, 80, 1.0)
            x = ctx.empty((B, Hd), np.float32)
            ctx.fill(x, B * Hd, mlamoe.MM_FILL_F32_NORMAL, 81, 1.0)
            pos = ctx.to_device(np.full(B, L - 1, np.int32))
            q = ctx.empty((B, QD), np.float32)
            co = ctx.empty((B, NH * VHD), np.float32)

            def step():
                mlamoe._check(lib.mm_mla_front_dev(h, B, x.ptr, C.byref(ws), pos.ptr, q.ptr,
                                                   cache.ptr, L, None))
                mlamoe._check(lib.mm_mla_absorbed_decode_dev(h, 0, B, q.ptr, cache.ptr, L, None,
                                                             L, co.ptr, None, None, None))
                mlamoe._check(lib.mm_matmul_bf16_dev(h, x.ptr, co.ptr, wd["o_proj"].ptr, Hd,
                                                     NH * VHD, B, mlamoe.MM_MATMUL_ACCUMULATE))
            ms, _ = timed(ctx, step, steps * 5, warmup)
            names = ["mm_gemv_1", "mm_gemv_4", "mm_rmsnorm", "mm_rmsnorm_hl", "mm_cvt_bf16", "mm_gemm_bf16",
                     "mm_gemm_skinny", "mm_gemm_hl", "mm_skinny_reduce",
                     "mm_mla_rope", "mm_mla_qprep", "mm_mla_attn", "mm_mla_combine", "mm_mla_uv"]
            prof = profile_kernels(ctx, step, 20, names)
            wbytes = 2 * (QD * Hd + KVD * Hd + Hd * NH * VHD + 2 * NH * QKN * KVL + Hd + KVL)
            nbytes = wbytes + B * L * KVD * 2
            res[f"B{B}"] = dict(ms_per_step=ms, tok_s=B / (ms * 1e-3), mb=nbytes / 1e6,
                                gbs=nbytes / (ms * 1e-3) / 1e9,
                                frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                kernels_us={n: [round(v[0] * 1e3, 2), v[1]]
                                            for n, v in prof.items() if v[1]})
    return res


def bench_engine(steps, warmup, B=64, prompt=64, gen=64, prefill_len=2048):
    """End-to-end greedy decoding of a DeepSeek-V2-Lite-shaped model (27
    layers: a dense SwiGLU layer 0 (intermediate 10944), 26 MoE layers with
    int8 experts, vocabulary 102400; random weights generated on the device)
    through the batched engine: (1) one decode step of B slots at context
    `prompt` (the steady-state step) and of one slot (latency), (2) the
    batched prefill of one `prefill_len`-token prompt in one step
    (mm_engine_step_rows: every layer over all prompt rows, the int8 grouped
    GEMM at T = prefill_len), (3) mm_engine_generate over B requests of
    `prompt` tokens generating `gen` tokens each (prompts prefilled in
    chunks beside the decode rows, continuous batching over B slots)."""
    from mlamoe.engine import Engine
    NL, DI, V, NH, QKN, QKR, KVL, VHD = 27, 10944, 102400, 16, 128, 64, 512, 128
    QD, KVD = NH * (QKN + QKR), KVL + QKR
    log("[engine] building a 27-layer DeepSeek-V2-Lite-shaped model on the device")
    lib = mlamoe.lib()
    with mlamoe.Context(0) as ctx:
        ctx.mla_init(NH, QKN, QKR, KVL, VHD, n_layers=NL)
        ctx.mla_front_init(H, mlamoe.rope_inv_freq(QKR, 10000.0, 40.0, 32.0, 1.0, 4096.0))
        ctx.moe_init(H, E, NS, K, I, n_layers=NL)
        stage = bf16_buffers(ctx)
        wst = dict(stage)
        wst["moe_gate_bias"] = None
        kvb = ctx.empty((NH * (QKN + VHD), KVL), np.uint16)
        seed = [1000]

        def filled(shape, std=0.02):
            b = ctx.empty(shape, np.uint16)
            seed[0] += 1
            ctx.fill(b, int(np.prod(shape)), mlamoe.MM_FILL_BF16_NORMAL, seed[0], std)
            return b
        layers = []
        for l in range(NL):
            ctx.fill(kvb, int(np.prod(kvb.shape)), mlamoe.MM_FILL_BF16_NORMAL, 5000 + l, 0.02)
            ctx.mla_load_layer(l, kvb, mlamoe.MM_LOAD_DEVICE_PTRS)
            fr = mlamoe.MlaFrontWeights(filled((H,), 0.1).ptr, filled((QD, H)).ptr, None, None, None,
                                        filled((KVD, H)).ptr, filled((KVL,), 0.1).ptr)
            ly = mlamoe.EngineLayer(fr, filled((H, NH * VHD)).ptr, filled((H,), 0.1).ptr)
            if l == 0:
                ly.dense_gate, ly.dense_up = filled((DI, H)).ptr, filled((DI, H)).ptr
                ly.dense_down = filled((H, DI)).ptr
            else:
                fill_layer_bf16(ctx, stage, 7000 + l)
                ctx.moe_load_layer(l, wst, mlamoe.MM_LOAD_INT8 | mlamoe.MM_LOAD_DEVICE_PTRS)
            layers.append(ly)
        for b in list(stage.values()) + [kvb]:
            b.free()
            ctx._bufs.remove(b)
        max_seq = max(prompt + gen + 8, prefill_len + 8)
        cfg = mlamoe.EngineConfig(NL, 1, H, DI, V, 1e-6, B, max_seq, mlamoe.MM_FWD_INT8, 0,
                                  prefill_len)
        h = C.c_void_p()
        mlamoe._check(lib.mm_engine_create(ctx.h, C.byref(cfg), C.byref(h)))
        eng = Engine(ctx, h.value, cfg, [])
        try:
            for l, ly in enumerate(layers):
                mlamoe._check(lib.mm_engine_set_layer(eng.h, l, C.byref(ly)))
            mlamoe._check(lib.mm_engine_set_head(eng.h, filled((V, H), 1.0).ptr, filled((H,), 0.1).ptr,
                                                 filled((V, H)).ptr))
            rng = np.random.default_rng(11)
            toks = rng.integers(0, V, B).astype(np.int32)
            pos = np.full(B, prompt, np.int32)
            log(f"[engine] decode step B={B} at context {prompt}")
            for _ in range(warmup):
                eng.step(toks, pos)
            t0 = time.perf_counter()
            for _ in range(steps):
                eng.step(toks, pos)
            step_ms = (time.perf_counter() - t0) * 1e3 / steps
            log(f"[engine] decode step B=1 at context {prompt}")
            for _ in range(warmup):
                eng.step(toks[:1], pos[:1])
            t0 = time.perf_counter()
            for _ in range(steps):
                eng.step(toks[:1], pos[:1])
            step1_ms = (time.perf_counter() - t0) * 1e3 / steps
            log(f"[engine] prefill of one {prefill_len}-token prompt in one step")
            ptoks = rng.integers(0, V, prefill_len).astype(np.int32)
            pslots = np.zeros(prefill_len, np.int32)
            ppos = np.arange(prefill_len, dtype=np.int32)
            last = np.array([prefill_len - 1], np.int32)
            for _ in range(max(1, warmup)):
                eng.step_rows(pslots, ptoks, ppos, last)
            t0 = time.perf_counter()
            for _ in range(max(2, steps // 4)):
                eng.step_rows(pslots, ptoks, ppos, last)
            prefill_ms = (time.perf_counter() - t0) * 1e3 / max(2, steps // 4)
            prompts = [rng.integers(0, V, prompt).astype(np.int32) for _ in range(B)]
            log(f"[engine] generate: {B} requests x ({prompt} prompt + {gen} generated) tokens")
            eng.generate(prompts[:2], 2)                      # warm the generate path
            t0 = time.perf_counter()
            outs, total = eng.generate(prompts, gen)
            gen_s = time.perf_counter() - t0
        finally:
            eng.close()
    return dict(model="DeepSeek-V2-Lite shape, 27 layers, int8 experts, random weights",
                step_B=B, step_context=prompt + 1, step_ms=step_ms, step_tok_s=B / (step_ms * 1e-3),
                step_B1_ms=step1_ms, step_B1_tok_s=1.0 / (step1_ms * 1e-3),
                prefill_tokens=prefill_len, prefill_ms=prefill_ms,
                prefill_tok_s=prefill_len / (prefill_ms * 1e-3),
                generate_requests=B, generate_prompt=prompt, generate_new=gen,
                generate_tokens=total, generate_s=gen_s, generate_tok_s=total / gen_s,
                generate_steps=prompt + gen - 1,
                generate_positions_per_s=B * (prompt + gen - 1) / gen_s)


def bench_lm_head(ctx, steps, warmup, V=102400, H=2048):
    """LM head of a decode step on DeepSeek-V2-Lite's vocabulary: final
    RMSNorm, logits over V (bf16 [V, H] weight), greedy argmax, for B = 1
    (GEMV) and B = 64 (the config-4 batch; MFMA GEMM)."""
    log("[lm_head] setup")
    w = ctx.empty((V, H), np.uint16)
    ctx.fill(w, V * H, mlamoe.MM_FILL_BF16_NORMAL, 61, 0.02)
    norm = ctx.empty((H,), np.uint16)
    ctx.fill(norm, H, mlamoe.MM_FILL_BF16_NORMAL, 62, 1.0)
    lib, h = mlamoe.lib(), ctx.h
    res = {}
    for B in (1, 64):
        x = ctx.empty((B, H), np.float32)
        ctx.fill(x, B * H, mlamoe.MM_FILL_F32_NORMAL, 63 + B, 1.0)
        lg = ctx.empty((B, V), np.float32)
        tok = ctx.empty((B,), np.int32)

        def step():
            mlamoe._check(lib.mm_lm_head_dev(h, B, x.ptr, norm.ptr, 1e-6, w.ptr, V, H, lg.ptr,
                                             tok.ptr))
        ms, _ = timed(ctx, step, steps * 5, warmup)
        names = ["mm_rmsnorm", "mm_rmsnorm_hl", "mm_lm_gemv_1", "mm_lm_gemv_4", "mm_cvt_bf16",
                 "mm_gemm_bf16", "mm_gemm_skinny", "mm_gemm_skinny_wide", "mm_lm_gemm",
                 "mm_argmax_part", "mm_argmax_final"]
        prof = profile_kernels(ctx, step, 20, names)
        nbytes = V * H * 2 + B * V * 4 + B * H * 4 + H * 2  # weights, logits out, x, norm
        flops = 2.0 * B * V * H
        res[f"B{B}"] = dict(ms_per_step=ms, tok_s=B / (ms * 1e-3), gbs=nbytes / (ms * 1e-3) / 1e9,
                            frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                            tflops=flops / (ms * 1e-3) / 1e12,
                            kernels_us={n: round(v[0] * 1e3, 2) for n, v in prof.items() if v[1]})
    return res


# ---------------------------------------------------------------------------

def cpu_baseline_decode(B=64, seconds_hint=True):
    """Reference CPU path (ffn_compute on bf16 experts, the oracle's
    restatement, bit-identical to the reference's golden vectors), single
    thread, on a bounded sample: all B tokens through ONE of the 26 layers;
    the step time is that times 26."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    log("[cpu_baseline] generating one host layer")
    w = _host_layer()
    rng = np.random.default_rng(9002)
    x = synth.normal_f32(rng, (B, H))
    lg = synth.uniform_logits(9003, B, E)
    cfg = pyoracle.moe_cfg(H, E, NS, K, I)
    pyoracle.ffn_compute_rows(cfg, w, x[:1], lg[:1])          # warm-up (page in)
    log("[cpu_baseline] timing")
    t0 = time.perf_counter()
    pyoracle.ffn_compute_rows(cfg, w, x, lg)
    dt = time.perf_counter() - t0
    step_s = dt * 26
    return dict(value=B / step_s, unit="tok/s", cores=1, kind="port",
                sample=f"{B} tokens x 1 of 26 layers ({dt:.1f} s single-threaded, "
                       f"x26 for a step); oracle ffn_compute on bf16 experts",
                cpu=_cpu_name(), nproc=os.cpu_count())


_HOST_LAYER = []


def _host_layer():
    """One DeepSeek-V2-Lite-shaped bf16 host layer for the CPU timings
    (generated once per run)."""
    if not _HOST_LAYER:
        _HOST_LAYER.append(synth.moe_layer(9001, H, E, I, NS))
    return _HOST_LAYER[0]


def _median_timed(fn, reps):
    """run.c:548-608's convention: rep 0 is a warm-up, the median of the rest."""
    ts = []
    for r in range(reps + 1):
        t0 = time.perf_counter()
        fn()
        if r:
            ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baselines_extra():
    """CPU timings beside configs 1 and 3 and the scalar int8 oracle on its
    own (BASELINE's plan), single-threaded, bounded samples:
    config 1: one token through one bf16 layer (oracle ffn_compute);
    config 3: 16 tokens of the Zipf-routed T = 2048 prefill through the
    bf16 reference path (what the reference executes for this layer) and
    through the scalar int8 oracle, each scaled x128 to the 2048 tokens
    (tokens are independent in ffn_compute); config 4: the int8 oracle on
    16 of the 64 tokens of one layer, x4 x26 for a step."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    log("[cpu_baseline] configs 1 and 3, int8 oracle")
    w = _host_layer()
    qw = pyoracle.quantize_moe_weights(w)
    cfg = pyoracle.moe_cfg(H, E, NS, K, I)
    common = dict(cores=1, cpu=_cpu_name(), nproc=os.cpu_count())
    x1 = synth.activations(9102, 1, H)
    t1 = _median_timed(lambda: pyoracle.ffn_compute_rows(cfg, w, x1), 3)
    c1 = dict(value=1.0 / t1, unit="tok/s", kind="port", ms_per_token=t1 * 1e3,
              sample="1 token x 1 layer, median of 3 after a warm-up; oracle ffn_compute "
                     "on bf16 experts", **common)
    n3 = 16
    x3 = synth.activations(9103, n3, H)
    lg3 = pyoracle.matmul(x3, w["moe_gate"]) + synth.zipf_prior(9104, E, 1.1)[None, :]
    t3 = _median_timed(lambda: pyoracle.ffn_compute_rows(cfg, w, x3, lg3), 1)
    t3i = _median_timed(lambda: pyoracle.ffn_i8(cfg, w, qw, x3, lg3), 1)
    scale = 2048 / n3
    c3 = dict(value=2048 / (t3 * scale), unit="tok/s", kind="port", ms_per_layer=t3 * scale * 1e3,
              sample=f"{n3} of the 2048 Zipf-routed tokens x 1 layer, x{scale:.0f}; oracle "
                     "ffn_compute on bf16 experts (the reference's path)",
              int8_oracle=dict(value=2048 / (t3i * scale), unit="tok/s",
                               ms_per_layer=t3i * scale * 1e3,
                               sample=f"the same {n3} tokens through the scalar int8 oracle "
                                      "(or_ffn_i8: int8 quantisation, exact int32 dots)"),
              **common)
    x4 = synth.activations(9105, 16, H)
    lg4 = synth.uniform_logits(9106, 16, E)
    t4i = _median_timed(lambda: pyoracle.ffn_i8(cfg, w, qw, x4, lg4), 1)
    c4 = dict(value=64 / (t4i * 4 * 26), unit="tok/s", kind="port", cores=1,
              sample="16 of the 64 tokens x 1 of 26 layers through the scalar int8 oracle, "
                     "x4 x26 for a step")
    return c1, c3, c4


def _cpu_name():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", choices=["decode_i8", "prefill_i8", "decode_bf16", "mla", "dense",
                                       "lm_head", "attn_layer", "engine", "calib"],
                    help="run one workload and print its result dict (profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first copy 1 GiB device-to-device (reference kernel for the "
                         "FETCH_SIZE/WRITE_SIZE counter scale)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding plan is a design, not built here.", file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        with mlamoe.Context(0) as ctx:
            n = 1 << 30
            src, dst = ctx.alloc(n, keep=True), ctx.alloc(n, keep=True)
            ctx.fill(src, n // 4, mlamoe.MM_FILL_F32_UNIFORM, 1)
            for _ in range(3):
                mlamoe._check(mlamoe.lib().mm_d2d(ctx.h, dst.ptr, src.ptr, n))
            log(f"[calibrate] copied {n} bytes x3 device-to-device")
    if args.only == "calib":
        return
    if args.only:
        fn = dict(decode_i8=bench_decode_i8, prefill_i8=bench_prefill_i8,
                  decode_bf16=bench_decode_bf16, mla=bench_mla_decode,
                  dense=bench_dense_bf16, lm_head=bench_lm_head,
                  attn_layer=bench_attn_layer, engine=None)[args.only]
        if args.only == "attn_layer":
            print(json.dumps({args.only: fn(None, args.steps, args.warmup)}, default=float),
                  flush=True)
            return
        if args.only == "engine":
            print(json.dumps({args.only: bench_engine(args.steps, args.warmup)}, default=float),
                  flush=True)
            return
        with mlamoe.Context(0) as ctx:
            print(json.dumps({args.only: fn(ctx, args.steps, args.warmup)}, default=float), flush=True)
        return

    extra = {}
    with mlamoe.Context(0) as ctx:
        dec = bench_decode_i8(ctx, args.steps, args.warmup)
    if not args.no_extra:
        with mlamoe.Context(0) as ctx:
            extra["prefill_i8_config3"] = bench_prefill_i8(ctx, args.steps, args.warmup)
        with mlamoe.Context(0) as ctx:
            extra["decode_bf16_config1"] = bench_decode_bf16(ctx, args.steps, args.warmup)
        with mlamoe.Context(0) as ctx:
            extra["mla_decode_config5"] = bench_mla_decode(ctx, args.steps, args.warmup)
        with mlamoe.Context(0) as ctx:
            extra["dense_bf16_config2"] = bench_dense_bf16(ctx, args.steps, args.warmup)
        with mlamoe.Context(0) as ctx:
            extra["lm_head_dsv2"] = bench_lm_head(ctx, args.steps, args.warmup)
        extra["attn_layer_dsv2"] = bench_attn_layer(None, args.steps, args.warmup)
        extra["engine_dsv2"] = bench_engine(args.steps, args.warmup)
    roof = dec.pop("roofline")
    cpu = None if args.no_cpu_baseline else cpu_baseline_decode()
    if not args.no_cpu_baseline and not args.no_extra:
        c1, c3, c4 = cpu_baselines_extra()
        extra["decode_bf16_config1"]["cpu_baseline"] = c1
        extra["prefill_i8_config3"]["cpu_baseline"] = c3
        cpu["int8_oracle"] = c4
    line = {
        "metric": METRIC,
        "value": round(dec["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded device RNG; bf16 N(0,0.02) weights quantised to int8, "
                "U(0,1) router logits, N(0,1) activations)",
        "config": {"workload": "config4: MoE decode B=64 x 26 layers, int8 weights, "
                               "DeepSeek-V2-Lite shapes",
                   "batch": 64, "layers": 26, "hidden": H, "experts": E, "top_k": K,
                   "moe_inter": I, "shared_experts": NS, "parallelism": "single-gpu"},
        "roofline": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in roof.items()},
        "cpu_baseline": cpu,
        "decode_detail": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in dec.items()},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
