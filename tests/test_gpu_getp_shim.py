"""The reference's getp interface (warm_up / inference / finish,
include/getp.h) implemented by mla-moe_amd/shim/getp_mlamoe.c, run end to end
on the engine golden models through mla-moe_amd/shim/libgetp_shim_test.so
(the shim plus a harness that fills a reference Transformer; prompts are
token ids written as text for its test-double tokenizer).

Checks: the model's max_seq_len of 163,840 (the reference's KV_CACHE_CAP)
starts without allocating for it (the caches grow with the requests, as
src/getp_run.hip:269-290); the GLM flavour gets the reference's 576-position
cap (src/getp_run.hip:709-710) and prompt cap (src/getp_run.hip:932-936);
every generated token is the oracle's argmax for its prefix (near-ties within
2e-3 normwise accepted; the oracle runs the int8 expert scheme the shim
serves); lengths follow
min(max_steps, max_seq - prompt) and generation stops at EOS.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT, engine_case

pytestmark = pytest.mark.gpu
TOL = 2e-3
SHIM = os.path.join(ROOT, "mla-moe_amd", "shim", "libgetp_shim_test.so")
_u16p, _f32p = C.POINTER(C.c_uint16), C.POINTER(C.c_float)
KEYS = ("in_norm", "q_proj", "kv_a", "kv_a_norm", "kv_b", "o_proj", "post_norm", "dgate", "dup",
        "ddown", "moe_gate", "eg", "eu", "ed", "sg", "su", "sd", "q_a_proj", "q_a_norm", "q_b_proj")


class Spec(C.Structure):
    _fields_ = [(k, C.c_int) for k in ("n_layers", "first_k_dense", "H", "NH", "QKN", "QKR",
                                        "KVL", "VHD", "dense_inter", "E", "n_shared", "K", "I",
                                        "vocab", "router_sigmoid", "norm_topk", "max_seq",
                                        "q_lora", "interleaved")] + \
        [("routed_scaling", C.c_float), ("rms_eps", C.c_float), ("inv_freq", _f32p),
         ("embed", _u16p), ("final_norm", _u16p), ("lm_head", _u16p)] + \
        [(k, C.POINTER(_u16p)) for k in KEYS] + [("moe_bias", C.POINTER(_f32p))]


def _shim():
    if not os.path.exists(SHIM):
        pytest.skip("libgetp_shim_test.so is built only where the reference headers are "
                    "(__graft_entry__.build)")
    L = C.CDLL(SHIM)
    L.shim_run.argtypes = [C.POINTER(Spec), C.c_int, C.POINTER(C.c_char_p), C.c_int, C.c_int,
                           C.c_void_p, C.c_void_p, C.POINTER(C.c_int)]
    L.shim_run.restype = C.c_longlong
    return L


def run_shim(c, m, inv, prompts, max_steps, eos, max_seq):
    keep = []

    def u16(a):
        a = np.ascontiguousarray(a, np.uint16)
        keep.append(a)
        return a.ctypes.data_as(_u16p)

    def per_layer(key):
        arr = (_u16p * len(m["layers"]))()
        for l, lw in enumerate(m["layers"]):
            if lw.get(key) is not None:
                arr[l] = u16(lw[key])
        return arr
    bias = (_f32p * len(m["layers"]))()
    for l, lw in enumerate(m["layers"]):
        if lw.get("moe_gate_bias") is not None:
            b = np.ascontiguousarray(lw["moe_gate_bias"], np.float32)
            keep.append(b)
            bias[l] = b.ctypes.data_as(_f32p)
    inv = np.ascontiguousarray(inv, np.float32)
    spec = Spec(c["n_layers"], c["first_dense"], c["H"], c["NH"], c["QKN"], c["QKR"], c["KVL"],
                c["VHD"], c["dense_inter"], c["E"], c["n_shared"], c["K"], c["I"], c["vocab"],
                c["router_sigmoid"], c["norm_topk"], max_seq, c.get("q_lora", 0),
                c.get("interleaved", 0), c["routed_scaling"], c["rms_eps"],
                inv.ctypes.data_as(_f32p), u16(m["embed"]), u16(m["final_norm"]), u16(m["lm_head"]),
                *[per_layer(k) for k in KEYS], bias)
    n = len(prompts)
    texts = (C.c_char_p * n)(*[" ".join(str(int(t)) for t in p).encode() for p in prompts])
    out = np.zeros((n, max_steps), np.int32)
    lens = np.zeros(n, np.int32)
    ms = C.c_int()
    total = _shim().shim_run(C.byref(spec), n, texts, max_steps, eos, out.ctypes.data,
                             lens.ctypes.data, C.byref(ms))
    return [out[r, :lens[r]].copy() for r in range(n)], int(total), ms.value


def _check_tokens(oracle, c, m, inv, prompt, out):
    """Each generated id is the argmax of the oracle's logits for its prefix
    (the oracle running the int8 expert scheme the shim serves)."""
    seq = np.concatenate([prompt, out])
    lg = oracle.model_logits(c, m, seq[:-1], inv, int8=True)
    for k, t in enumerate(out):
        row = lg[len(prompt) - 1 + k]
        assert t == row.argmax() or row[t] >= row.max() - TOL * np.abs(row).max(), k


def test_getp_shim_dsv2(oracle):
    c, m, g = engine_case("dsv2")
    inv = g["inv"]
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, c["vocab"], n).astype(np.int32) for n in (3, 1, 7, 2, 5, 9, 4)]
    max_steps = 6
    print("getp shim dsv2: 7 requests, max_seq 163840", flush=True)
    outs, total, ms = run_shim(c, m, inv, prompts, max_steps, -1, 163840)
    assert ms == 163840
    assert total == sum(len(o) for o in outs) == len(prompts) * max_steps
    for p, o in zip(prompts, outs):
        _check_tokens(oracle, c, m, inv, p, o)
    # EOS: the first sampled EOS ends a request and is not stored
    eos = int(outs[0][2])
    outs2, _, _ = run_shim(c, m, inv, prompts[:1], max_steps, eos, 163840)
    assert list(outs2[0]) == list(outs[0][:2])


def test_getp_shim_glm_caps(oracle):
    c, m, g = engine_case("glm")
    inv = g["inv"]
    rng = np.random.default_rng(13)
    prompts = [rng.integers(0, c["vocab"], n).astype(np.int32) for n in (600, 4, 2)]
    max_steps = 6
    print("getp shim glm: 600-token prompt against the 576-position cap", flush=True)
    outs, total, ms = run_shim(c, m, inv, prompts, max_steps, -1, 163840)
    assert ms == 576                              # getp_run.hip:709-710
    cap = 576 - max_steps                         # getp_run.hip:932-936
    assert [len(o) for o in outs] == [max_steps] * 3
    _check_tokens(oracle, c, m, inv, prompts[0][:cap], outs[0])
    for p, o in zip(prompts[1:], outs[1:]):
        _check_tokens(oracle, c, m, inv, p, o)
