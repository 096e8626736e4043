"""GPU checks of the offline int8 expert format: the host packer
(mlamoe.weights) is bit-identical to the device quantise + pack of
mm_moe_load_layer(MM_LOAD_INT8), and a layer uploaded from an mlamoe-i8 file
(mm_moe_load_layer_i8_packed, no quantisation at load) computes exactly
what the device-quantised layer computes."""
import numpy as np
import pytest

import mlamoe
from mlamoe import synth, weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,E,I,NS", [(256, 8, 128, 2), (2048, 3, 1408, 2), (512, 4, 192, 0)])
def test_device_pack_equals_host_pack(H, E, I, NS):
    print(f"pack H={H} E={E} I={I} NS={NS}", flush=True)
    w = synth.moe_layer(7 + H, H, E, I, max(NS, 1))
    if NS == 0:
        w.update(sg=np.zeros((0, H), np.uint16), su=np.zeros((0, H), np.uint16),
                 sd=np.zeros((H, 0), np.uint16))
    with mlamoe.Context(0) as c:
        c.moe_init(H, E, NS, 2, I)
        c.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
        pb, ns = weights.layer_size(c._moe_cfg)
        pool, sc = np.empty(pb, np.int8), np.empty(ns, np.float32)
        mlamoe._check(mlamoe.lib().mm_moe_export_layer_i8(c.h, 0, pool.ctypes.data, sc.ctypes.data))
    hp, hs = weights.pack_layer(w, H, E, I, NS)
    assert np.array_equal(pool, hp)
    assert np.array_equal(sc.view(np.uint32), hs.view(np.uint32))


@pytest.mark.parametrize("T", [3, 64, 300])
def test_packed_file_forward_identical(tmp_path, T):
    """Decode (T <= 64) and prefill-tiled (T = 300) int8 paths, GLM-style
    router (sigmoid, bias, normalised top-k)."""
    print(f"packed forward T={T}", flush=True)
    H, E, I, NS, K = 256, 16, 128, 1, 4
    w = synth.moe_layer(11, H, E, I, NS, gate_bias=True)
    pool, scales = weights.pack_layer(w, H, E, I, NS)
    path = str(tmp_path / "experts.i8.safetensors")
    weights.save_packed(path, H, E, I, NS, {5: (pool, scales, w["moe_gate"], w["moe_gate_bias"])})
    x = synth.normal_f32(np.random.default_rng(T), (T, H))
    outs = []
    for from_file in (False, True):
        with mlamoe.Context(0) as c:
            c.moe_init(H, E, NS, K, I, router_sigmoid=1, norm_topk=1, routed_scaling=2.5)
            if from_file:
                assert weights.load(c, path, {5: 0}) == [5]
            else:
                c.moe_load_layer(0, w, mlamoe.MM_LOAD_INT8)
            outs.append(c.moe_forward(0, x, flags=mlamoe.MM_FWD_INT8))
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b)


def test_packed_errors(tmp_path):
    L = mlamoe.lib()
    with mlamoe.Context(0) as c:
        z = np.zeros(16, np.float32)
        assert L.mm_moe_load_layer_i8_packed(c.h, 0, z.ctypes.data, None, z.ctypes.data,
                                             z.ctypes.data, 0) != 0
        assert b"mm_moe_init" in L.mm_last_error()
        c.moe_init(256, 4, 1, 2, 128)
        assert L.mm_moe_load_layer_i8_packed(c.h, 0, None, None, None, None, 0) != 0
        assert b"NULL" in L.mm_last_error()
        assert L.mm_moe_export_layer_i8(c.h, 0, z.ctypes.data, z.ctypes.data) != 0
        assert b"no int8 weights" in L.mm_last_error()
        w = synth.moe_layer(3, 256, 4, 128, 1)
        path = str(tmp_path / "a.safetensors")
        weights.save_packed(path, 256, 4, 128, 1, {0: (*weights.pack_layer(w, 256, 4, 128, 1),
                                                        w["moe_gate"], None)})
        weights.load(c, path)
        with pytest.raises(mlamoe.MMError, match="already loaded"):
            weights.load(c, path)
    with mlamoe.Context(0) as c:
        c.moe_init(256, 8, 1, 2, 128)
        with pytest.raises(ValueError, match="geometry"):
            weights.load(c, path)
