"""GPU parity of the decode attention front (mm_mla_front_dev) and the
few-token GEMV path of mm_matmul_bf16_dev against the CPU oracle, which the
reference's own compiled run.c / model_load.c pin bit for bit
(tests/golden/mla_front.npz).

Bars:
  - q (after RoPE) and the fp32 appended rows (kv_rows): normwise <= 1e-5
    (fp32 dot products in a different association than run.c:29-37; cos/sin
    correctly rounded on the GPU);
  - the bf16 cache row: exactly the nearest-even bf16 of the kernel's fp32
    row, and within half a bf16 ulp of the oracle's value plus the fp32 bar;
  - attn_out behind the front (absorbed chain on the bf16 cache, o_proj):
    normwise <= 2e-3, the north-star bf16 bar (the reference's cache row is
    fp32, this build's bf16).
"""
import numpy as np
import pytest

import mlamoe
from conftest import front_case, load_golden, max_abs_rel
from mlamoe import synth

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-5


def rne(x):
    """fp32 -> bf16, round to nearest even (the cache's rounding)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def check_cache_row(got, got_f32, ref):
    """got (bf16) is exactly the nearest-even bf16 of the kernel's own fp32
    row got_f32, and within half a bf16 ulp of the oracle's ref plus the
    fp32 bar (normwise)."""
    assert np.array_equal(got, rne(got_f32))
    g = synth.bf16_to_f32(got).astype(np.float64)
    lo = synth.bf16_to_f32(synth.bf16_from_f32(ref)).astype(np.float64)
    ulp = np.abs(synth.bf16_to_f32((synth.bf16_from_f32(ref) + 1).astype(np.uint16)) - lo)
    assert np.all(np.abs(g - ref) <= 0.5 * ulp + TOL_F32 * np.abs(ref).max())


def make_ctx(NH, QKN, QKR, KVL, VHD, H, inv, q_lora=0, rms_eps=1e-6, mla_eps=1e-6, il=0,
             kv_b=None):
    c = mlamoe.Context(0)
    c.mla_init(NH, QKN, QKR, KVL, VHD)
    c.mla_front_init(H, inv, q_lora, rms_eps, mla_eps, il)
    if kv_b is not None:
        c.mla_load_layer(0, kv_b)
    return c


@pytest.mark.parametrize("name", ["dsv2", "glm"])
def test_front_golden(oracle, name):
    """One decode token of the reference's forward_absorbed: q, the appended
    cache row, and the attention output behind them."""
    g = load_golden("mla_front.npz")
    c = front_case(g, name)
    print(f"front golden {name}", flush=True)
    ctx = make_ctx(c["NH"], c["QKN"], c["QKR"], c["KVL"], c["VHD"], c["H"], c["inv"], c["q_lora"],
                   c["rms_eps"], c["mla_eps"], c["il"], c["w"]["kv_b"])
    try:
        L = c["pos"] + 8
        cache = np.zeros((1, L, c["KVL"] + c["QKR"]), np.uint16)
        cache[0, :c["pos"]] = c["cache_in"]
        q, kv, cache2 = ctx.mla_front(c["x"][None], c["w"], [c["pos"]], cache)
        assert max_abs_rel(q[0], g[f"{name}_q"]) < TOL_F32
        assert max_abs_rel(kv[0], g[f"{name}_kv"]) < TOL_F32
        check_cache_row(cache2[0, c["pos"]], kv[0], g[f"{name}_kv"])
        assert np.array_equal(cache2[0, :c["pos"]], c["cache_in"])       # earlier rows kept
        assert not np.any(cache2[0, c["pos"] + 1:])                      # later rows untouched
        ctx_out, _, _, _ = ctx.mla_absorbed_decode(0, q.reshape(1, c["NH"], -1), cache2,
                                                   c["pos"] + 1)
        ao = ctx.matmul(ctx_out, c["w"]["o_proj"])
        assert max_abs_rel(ao[0], g[f"{name}_attn_out"]) < 2e-3
    finally:
        ctx.close()


CASES = [  # B, q_lora, interleaved, H  (B <= 4: fused GEMVs; more: MFMA GEMMs; above
    #          64 rows the tiled GEMM, x converted to bf16 rows once for q and kv_a)
    (1, 0, 0, 2048), (3, 0, 1, 2048), (4, 96, 1, 512), (5, 0, 0, 2048), (9, 96, 0, 512),
    (2, 0, 0, 4096), (70, 0, 0, 2048), (66, 96, 1, 512),
]


@pytest.mark.parametrize("B,q_lora,il,H", CASES)
def test_front_random(oracle, B, q_lora, il, H):
    """B tokens at their own positions (one out of range: no cache write)
    against the oracle token by token."""
    print(f"front random B={B} q_lora={q_lora} il={il} H={H}", flush=True)
    NH, QKN, QKR, KVL, VHD, L = 16 if H == 2048 else 4, 128 if H == 2048 else 64, 64, 512, 64, 40
    rng = np.random.default_rng(B * 7 + q_lora + il)
    w = synth.attn_layer(100 + B, H, NH, QKN, QKR, KVL, VHD, q_lora)
    inv = oracle.rope_inv_freq(QKR, 10000.0, 40.0, 32.0, 1.0, 4096.0)
    x = synth.normal_f32(rng, (B, H), 3.0)
    pos = rng.integers(0, L, B).astype(np.int32)
    pos[-1] = L if B > 1 else pos[-1]                    # out of range: not written
    cache = synth.normal_bf16(rng, (B, L, KVL + QKR), 1.0)
    ctx = make_ctx(NH, QKN, QKR, KVL, VHD, H, inv, q_lora, 1e-5, 1e-6, il)
    try:
        q, kv, cache2 = ctx.mla_front(x, w, pos, cache)
    finally:
        ctx.close()
    cfg = oracle.front_cfg(H, NH, QKN, QKR, KVL, q_lora, 1e-5, 1e-6, il)
    for b in range(B):
        rq, rkv, _ = oracle.mla_front(cfg, w, inv, x[b], int(pos[b]))
        assert max_abs_rel(q[b], rq[0]) < TOL_F32, b
        assert max_abs_rel(kv[b], rkv[0]) < TOL_F32, b
        keep = np.ones(L, bool)
        if pos[b] < L:
            check_cache_row(cache2[b, pos[b]], kv[b], rkv[0])
            keep[pos[b]] = False
        assert np.array_equal(cache2[b, keep], cache[b, keep]), b


def test_front_errors():
    L = mlamoe.lib()
    c = mlamoe.Context(0)
    try:
        ws = mlamoe.MlaFrontWeights()
        assert L.mm_mla_front_dev(c.h, 1, None, ws, None, None, None, 8, None) != 0
        assert b"mm_mla_front_init" in L.mm_last_error()
        c.mla_init(16)
        inv = np.ones(32, np.float32)
        with pytest.raises(mlamoe.MMError, match="multiples of 8"):
            c.mla_front_init(2044, inv)
        c.mla_front_init(2048, inv)
        buf = c.empty((1 << 16,), np.float32)
        assert L.mm_mla_front_dev(c.h, 1, buf.ptr, ws, buf.ptr, buf.ptr, buf.ptr, 8, None) != 0
        assert b"NULL" in L.mm_last_error()
        ws = mlamoe.MlaFrontWeights(*([buf.ptr] * 7))
        assert L.mm_mla_front_dev(c.h, 1, buf.ptr + 4, ws, buf.ptr, buf.ptr, buf.ptr, 8, None) != 0
        assert b"aligned" in L.mm_last_error()
        assert L.mm_mla_front_dev(c.h, 0, None, None, None, None, None, 8, None) == 0  # no-op
    finally:
        c.close()


@pytest.mark.parametrize("T,d_out,n_in,flags", [(1, 2048, 2048, 0), (2, 300, 136, 0),
                                                (3, 1001, 512, 1), (4, 77, 2048, 2),
                                                (1, 576, 2048, 3)])
def test_matmul_gemv_path(oracle, T, d_out, n_in, flags):
    """mm_matmul_bf16_dev at T <= 4 (the GEMV): plain, x truncated to bf16
    (MM_MATMUL_X_BF16), and y += (MM_MATMUL_ACCUMULATE, the residual add of
    run.c:468-469)."""
    rng = np.random.default_rng(T * 1000 + d_out)
    x = synth.normal_f32(rng, (T, n_in))
    w = synth.normal_bf16(rng, (d_out, n_in), 0.02)
    y0 = synth.normal_f32(rng, (T, d_out))
    with mlamoe.Context(0) as c:
        y = c.matmul(x, w, flags, y0=y0)
    xr = synth.bf16_to_f32(synth.bf16_from_f32(x)) if flags & 1 else x
    ref = oracle.matmul(xr, w) + (y0 if flags & 2 else 0)
    assert max_abs_rel(y, ref) < TOL_F32
