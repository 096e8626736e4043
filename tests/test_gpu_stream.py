"""A caller-supplied HIP stream (mm_ctx_set_stream): the context queues its
work on the caller's stream, results are bit-identical to those on its own
stream, and switching back restores it.  The reference runs on one stream of
its own (src/getp_run.hip:735); the boundary lets a host engine pass the
stream it orders its other work on."""
import ctypes as C

import numpy as np
import pytest

import mlamoe
from mlamoe import synth

pytestmark = pytest.mark.gpu


def _hip():
    h = C.CDLL("libamdhip64.so")
    h.hipStreamCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
    h.hipStreamDestroy.argtypes = [C.c_void_p]
    h.hipStreamSynchronize.argtypes = [C.c_void_p]
    return h


def test_caller_stream_int8_moe():
    H, E, K, I, NS, T = 256, 16, 4, 128, 2, 300     # T >= 256: the tiled path too
    w = synth.moe_layer(300, H, E, I, NS)
    x = synth.activations(301, T, H)
    hip = _hip()
    s = C.c_void_p()
    assert hip.hipStreamCreateWithFlags(C.byref(s), 1) == 0      # hipStreamNonBlocking
    try:
        with mlamoe.Context(0) as ctx:
            own = ctx.stream()
            ctx.moe_init(H, E, NS, K, I)
            ctx.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
            for t in (T, 7):
                a = ctx.moe_forward(0, x[:t], flags=mlamoe.MM_FWD_INT8)
                ctx.set_stream(s.value)
                assert ctx.stream() == s.value
                b = ctx.moe_forward(0, x[:t], flags=mlamoe.MM_FWD_INT8)
                assert hip.hipStreamSynchronize(s) == 0
                ctx.set_stream(None)
                assert ctx.stream() == own
                for u, v in zip(a, b):
                    assert np.array_equal(u, v)
    finally:
        hip.hipStreamDestroy(s)
