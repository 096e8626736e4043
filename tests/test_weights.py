"""The offline int8 expert format (mlamoe.weights) on the CPU: the host
quantiser against the oracle's (or_quant_weight_i8), the fragment packing
against its inverse and against the per-element layout rule the int8 kernels
read, the safetensors container, and conversion of a checkpoint laid out
with the reference's tensor names (src/model_load.c:118-148)."""
import json
import os

import numpy as np
import pytest

import mlamoe
from mlamoe import synth, weights


def test_quantize_rows_matches_oracle(oracle):
    rng = np.random.default_rng(1)
    w = synth.normal_bf16(rng, (37, 256), 0.02)
    w[3] = 0                                                   # zero row: s = 0, q = 0
    # a row with exact halves: max 127 -> s = 1, w / s = 63.5, -62.5 (ties to even)
    w[5] = synth.bf16_from_f32(np.array([127.0, 63.5, -62.5, 0.5] + [0.0] * 252, np.float32))
    q, s = weights.quantize_rows(w)
    qo, so = oracle.quant_weight(w)
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert list(q[5, :4]) == [127, 64, -62, 0] and not q[3].any() and s[3] == 0


def test_pack_layout_and_inverse():
    rng = np.random.default_rng(2)
    q0 = rng.integers(-127, 128, (48, 192), dtype=np.int8)
    q1 = rng.integers(-127, 128, (48, 192), dtype=np.int8)
    p1, p2 = weights.pack(q0), weights.pack(q0, q1)
    assert np.array_equal(weights.unpack(p1, 48, 192), q0)
    a, b = weights.unpack(p2, 48, 192, two=True)
    assert np.array_equal(a, q0) and np.array_equal(b, q1)
    # the element rule of the int8 kernels' B operand (moe_i8.hip, mm_pack_i8):
    # fragment f = (nb * KB + kb) * NS + which, byte 16 l + b -> row 16 nb + l % 16,
    # column 64 kb + 16 (l // 16) + b
    KB = 192 // 64
    for _ in range(200):
        r, c, which = int(rng.integers(48)), int(rng.integers(192)), int(rng.integers(2))
        nb, kb, l = r // 16, c // 64, (r % 16) + 16 * ((c % 64) // 16)
        off = (((nb * KB + kb) * 2 + which) * 64 + l) * 16 + c % 16
        assert p2[off] == (q1 if which else q0)[r, c]
        if which == 0:
            assert p1[((nb * KB + kb) * 64 + l) * 16 + c % 16] == q0[r, c]
    # a batch of matrices packs as the concatenation of each
    qs = rng.integers(-127, 128, (3, 32, 64), dtype=np.int8)
    assert np.array_equal(weights.pack(qs).reshape(-1),
                          np.concatenate([weights.pack(m) for m in qs]))


def test_pack_layer_pieces(oracle):
    H, E, I, NS = 128, 3, 64, 2
    w = synth.moe_layer(5, H, E, I, NS)
    pool, scales = weights.pack_layer(w, H, E, I, NS)
    qw = oracle.quantize_moe_weights(w)
    S = NS * I
    o = 0
    for e in range(E):
        g, u = weights.unpack(pool[o:o + 2 * I * H], I, H, two=True)
        assert np.array_equal(g, qw["qeg"][e]) and np.array_equal(u, qw["qeu"][e])
        o += 2 * I * H
    for e in range(E):
        assert np.array_equal(weights.unpack(pool[o:o + H * I], H, I), qw["qed"][e])
        o += H * I
    g, u = weights.unpack(pool[o:o + 2 * S * H], S, H, two=True)
    assert np.array_equal(g, qw["qsg"]) and np.array_equal(u, qw["qsu"])
    o += 2 * S * H
    assert np.array_equal(weights.unpack(pool[o:], H, S), qw["qsd"])
    want = np.concatenate([qw[k].reshape(-1) for k in ("seg", "seu", "sed", "ssg", "ssu", "ssd")])
    assert np.array_equal(scales, want)
    assert (pool.size, scales.size) == weights.layer_sizes(H, E, I, NS)
    # the library's own size function (host code, no GPU)
    cfg = mlamoe.MoeConfig(H, E, NS, 2, I, 0, 0, 1.0)
    assert weights.layer_size(cfg) == (pool.size, scales.size)
    with pytest.raises(mlamoe.MMError, match="multiples of 64"):
        weights.layer_size(mlamoe.MoeConfig(H, E, NS, 2, 100, 0, 0, 1.0))
    # K dimensions of the int8 GEMMs stay below 2^16: moe_inter itself, and the
    # shared experts' concatenated inter size (2 x 32768)
    for ns, inter in ((0, 65536), (2, 32768)):
        with pytest.raises(mlamoe.MMError, match="below 65536"):
            weights.layer_size(mlamoe.MoeConfig(H, E, ns, 2, inter, 0, 0, 1.0))
    assert weights.layer_size(mlamoe.MoeConfig(H, E, 1, 2, 32704, 0, 0, 1.0))[0] > 0


def test_container_roundtrip(tmp_path):
    rng = np.random.default_rng(3)
    t = dict(a=("BF16", synth.normal_bf16(rng, (5, 7))), b=("F32", synth.normal_f32(rng, (3,))),
             c=("I8", rng.integers(-127, 128, 11, dtype=np.int8)))
    p = str(tmp_path / "x.safetensors")
    weights.write_safetensors(p, t, dict(k="v"))
    st = weights.SafeTensors(p)
    assert st.metadata == {"k": "v"} and st.names() == ["a", "b", "c"]
    for k, (dt, a) in t.items():
        assert st.dtype(k) == dt and np.array_equal(st.get(k), a)
    with open(p, "rb") as f:                       # the public layout: u64 header length
        n = int.from_bytes(f.read(8), "little")
        hdr = json.loads(f.read(n))
    assert hdr["b"]["data_offsets"][0] % 8 == 0 and hdr["__metadata__"] == {"k": "v"}
    with pytest.raises(ValueError, match="not an mlamoe-i8"):
        weights.read_packed(p)


def _write_reference_checkpoint(d, H, E, I, NS, layers, first_dense, seed, bias=False):
    """A tiny checkpoint with the reference's tensor names, sharded over two
    files behind model.safetensors.index.json."""
    shards = [{}, {}]
    ws = {}
    for l in range(first_dense, layers):
        w = synth.moe_layer(seed + l, H, E, I, NS, gate_bias=bias)
        ws[l] = w
        p = f"model.layers.{l}.mlp"
        sh = shards[l % 2]
        sh[f"{p}.gate.weight"] = ("BF16", w["moe_gate"])
        if bias:
            sh[f"{p}.gate.e_score_correction_bias"] = ("F32", w["moe_gate_bias"])
        for k, n in (("sg", "gate_proj"), ("su", "up_proj"), ("sd", "down_proj")):
            sh[f"{p}.shared_experts.{n}.weight"] = ("BF16", w[k])
        for e in range(E):
            for k, n in (("eg", "gate_proj"), ("eu", "up_proj"), ("ed", "down_proj")):
                sh[f"{p}.experts.{e}.{n}.weight"] = ("BF16", w[k][e])
    wm = {}
    for i, sh in enumerate(shards):
        name = f"model-{i + 1:05d}-of-00002.safetensors"
        weights.write_safetensors(os.path.join(d, name), sh)
        wm.update({k: name for k in sh})
    json.dump({"metadata": {}, "weight_map": wm}, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    json.dump(dict(hidden_size=H, n_routed_experts=E, moe_intermediate_size=I, n_shared_experts=NS,
                   num_hidden_layers=layers, first_k_dense_replace=first_dense),
              open(os.path.join(d, "config.json"), "w"))
    return ws


def test_convert_reference_checkpoint(tmp_path):
    H, E, I, NS = 128, 4, 64, 1
    ws = _write_reference_checkpoint(str(tmp_path), H, E, I, NS, 3, 1, 40, bias=True)
    out = str(tmp_path / "experts.i8.safetensors")
    assert weights.convert(str(tmp_path), out) == [1, 2]
    geo, st, layers = weights.read_packed(out)
    assert layers == [1, 2] and geo == dict(hidden_size=H, n_routed_experts=E,
                                            moe_intermediate_size=I, n_shared_experts=NS)
    for l in layers:
        pool, scales = weights.pack_layer(ws[l], H, E, I, NS)
        p = f"model.layers.{l}.mlp"
        assert np.array_equal(st.get(f"{p}.experts.i8_pool"), pool)
        assert np.array_equal(st.get(f"{p}.experts.i8_scales"), scales)
        assert np.array_equal(st.get(f"{p}.gate.weight"), ws[l]["moe_gate"])
        assert np.array_equal(st.get(f"{p}.gate.e_score_correction_bias"), ws[l]["moe_gate_bias"])
