"""mm_moe_forward_noalloc_dev (the MoE FFN entry point that allocates
nothing: its workspace is a static per-device scratch array) against
mm_moe_forward_dev: identical outputs, routing and scores on two calls in a
row, the second with fewer tokens, for the int8 decode-shaped path at the
bench's B = 64 DeepSeek-V2-Lite shape, the int8 tiled path, the bf16 GEMV
path and a dense SwiGLU layer; on a fresh context the no-allocation calls
leave the context's workspace unallocated; a call needing more than the array holds, and a call while per-kernel
profiling is on, fail with a message before launching anything."""
import numpy as np
import pytest

import mlamoe
from mlamoe import synth

pytestmark = pytest.mark.gpu


def _call(ctx, fn, layer, T, x, lg, flags, E, K, H):
    L = mlamoe.lib()
    out = ctx.empty((T, H), np.float32)
    idx = ctx.empty((T, K), np.int32)
    wt = ctx.empty((T, K), np.float32)
    pr = ctx.empty((T, E), np.float32)
    # the same preset contents for both entry points (a dense layer leaves
    # the routing outputs as they were)
    for b, n in ((idx, T * K), (wt, T * K), (pr, T * E)):
        ctx.fill(b, n, mlamoe.MM_FILL_F32_UNIFORM, 7)
    mlamoe._check(getattr(L, fn)(ctx.h, layer, T, x.ptr, out.ptr, lg.ptr if lg is not None else None,
                                 idx.ptr, wt.ptr, pr.ptr, flags))
    res = (out.download(), idx.download(), wt.download(), pr.download())
    ctx._tmp((out, idx, wt, pr))
    return res


def _compare(ctx, layer, xs, lgs, flags, E, K, H):
    """Both entry points on each (x, logits) in turn, the no-allocation one
    first: on a fresh context it must leave the context's growable
    workspace unallocated (the property itself, not only equal results),
    and it never changes the workspace's size; the regular one then runs
    (it may grow its workspace; the scratch array is untouched by it)."""
    for x, lg in zip(xs, lgs):
        T = x.shape[0]
        print(f"noalloc T={T} flags={flags}", flush=True)
        dx = ctx.to_device(x)
        dl = ctx.to_device(lg) if lg is not None else None
        ws0 = ctx.workspace_bytes()
        b = _call(ctx, "mm_moe_forward_noalloc_dev", layer, T, dx, dl, flags, E, K, H)
        assert ctx.workspace_bytes() == ws0
        a = _call(ctx, "mm_moe_forward_dev", layer, T, dx, dl, flags, E, K, H)
        for u, v in zip(a, b):
            assert np.array_equal(u, v)
        ctx._tmp((dx,) + ((dl,) if dl is not None else ()))


def _fresh(ctx):
    """A context that has not run a forward call holds no workspace."""
    assert ctx.workspace_bytes() == 0


def test_noalloc_int8_decode_dsv2():
    d = synth.DSV2
    H, E, K, I, NS = d["H"], d["E"], d["K"], d["I"], d["n_shared"]
    w = synth.moe_layer(400, H, E, I, NS)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
        _fresh(ctx)
        xs = [synth.activations(401, 64, H), synth.activations(402, 9, H)]
        lgs = [synth.uniform_logits(403, 64, E), synth.uniform_logits(404, 9, E)]
        _compare(ctx, 0, xs, lgs, mlamoe.MM_FWD_INT8, E, K, H)
        # router logits computed from x (the router kernel's output also
        # lives in the scratch array)
        _compare(ctx, 0, xs, [None, None], mlamoe.MM_FWD_INT8, E, K, H)
        # too many tokens for the array: refused before any launch
        big = ctx.to_device(synth.activations(405, 512, H))
        out = ctx.empty((512, H), np.float32)
        st = mlamoe.lib().mm_moe_forward_noalloc_dev(ctx.h, 0, 512, big.ptr, out.ptr, None, None,
                                                     None, None, mlamoe.MM_FWD_INT8)
        assert st == -2 and b"scratch" in mlamoe.lib().mm_last_error()
        # per-kernel profiling allocates records: refused
        ctx.prof_enable(True)
        st = mlamoe.lib().mm_moe_forward_noalloc_dev(ctx.h, 0, 9, big.ptr, out.ptr, None, None,
                                                     None, None, mlamoe.MM_FWD_INT8)
        ctx.prof_enable(False)
        assert st == -5 and b"profiling" in mlamoe.lib().mm_last_error()


def test_noalloc_int8_tiled(monkeypatch):
    monkeypatch.setenv("MLAMOE_I8_TILED_MIN_T", "1")
    H, E, K, I, NS = 256, 16, 4, 128, 2
    w = synth.moe_layer(410, H, E, I, NS)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
        _fresh(ctx)
        xs = [synth.activations(411, 300, H), synth.activations(412, 7, H)]
        _compare(ctx, 0, xs, [None, None], mlamoe.MM_FWD_INT8, E, K, H)


def test_noalloc_bf16():
    H, E, K, I, NS = 256, 16, 4, 128, 2
    w = synth.moe_layer(420, H, E, I, NS)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_BF16)
        _fresh(ctx)
        xs = [synth.activations(421, 11, H), synth.activations(422, 2, H)]
        _compare(ctx, 0, xs, [None, None], mlamoe.MM_FWD_BF16, E, K, H)


def test_noalloc_dense_layer():
    """A dense SwiGLU layer (the reference's first_k_dense layers) through
    the no-allocation entry point: the GEMV (2 rows) and the skinny GEMM
    (40 rows) with their split partials in the scratch array."""
    H, E, K, I, NS, DI = 256, 16, 4, 128, 2, 512
    r = np.random.default_rng(430)
    with mlamoe.Context(0) as ctx:
        ctx.moe_init(H, E, NS, K, I)
        ctx.moe_load_dense_layer(0, synth.normal_bf16(r, (DI, H)), synth.normal_bf16(r, (DI, H)),
                                 synth.normal_bf16(r, (H, DI)))
        _fresh(ctx)
        xs = [synth.activations(431, 40, H), synth.activations(432, 2, H)]
        _compare(ctx, 0, xs, [None, None], mlamoe.MM_FWD_BF16, E, K, H)
