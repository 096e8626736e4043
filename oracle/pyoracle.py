"""ctypes bindings for the CPU oracle (liboracle.so) and, where it is built,
the reference's own compiled hot path (_ref/libref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

_f32p = C.POINTER(C.c_float)
_u16p = C.POINTER(C.c_uint16)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_ip = C.POINTER(C.c_int)


def build(ref: bool = False) -> None:
    """Compile liboracle.so (and _ref/libref.so when `ref` and the reference
    tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref and os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _p(a, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


class MoeCfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_routed_experts", C.c_int),
                ("n_shared_experts", C.c_int), ("n_experts_per_tok", C.c_int),
                ("moe_inter_size", C.c_int), ("router_sigmoid", C.c_int),
                ("norm_topk", C.c_int), ("routed_scaling", C.c_float)]


class MoeWeights(C.Structure):
    _fields_ = [("moe_gate", _u16p), ("moe_gate_bias", _f32p), ("eg", _u16p),
                ("eu", _u16p), ("ed", _u16p), ("sg", _u16p), ("su", _u16p),
                ("sd", _u16p)]


class MoeI8Weights(C.Structure):
    _fields_ = [("qg", _i8p), ("qu", _i8p), ("sg", _f32p), ("su", _f32p),
                ("qd", _i8p), ("sd", _f32p), ("qsg", _i8p), ("qsu", _i8p),
                ("ssg", _f32p), ("ssu", _f32p), ("qsd", _i8p), ("ssd", _f32p)]


class I8Debug(C.Structure):
    _fields_ = [("qx", _i8p), ("sx", _f32p), ("acc_gu", _i32p), ("qh", _i8p),
                ("sh", _f32p), ("acc_d", _i32p), ("qhs", _i8p), ("shs", _f32p)]


class FrontCfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_heads", C.c_int), ("qk_nope", C.c_int),
                ("qk_rope", C.c_int), ("kv_lora", C.c_int), ("q_lora", C.c_int),
                ("rms_eps", C.c_float), ("mla_eps", C.c_float), ("interleaved", C.c_int)]


class FrontWeights(C.Structure):
    _fields_ = [(n, _u16p) for n in ("in_norm", "q_proj", "q_a_proj", "q_a_norm", "q_b_proj",
                                     "kv_a", "kv_a_norm")]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.or_bf16_to_f32.restype = C.c_float
        L.or_bf16_to_f32.argtypes = [C.c_uint16]
        L.or_f32_to_bf16.restype = C.c_uint16
        L.or_f32_to_bf16.argtypes = [C.c_float]
        L.or_silu.restype = C.c_float
        L.or_silu.argtypes = [C.c_float]
        L.or_matmul.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_int]
        L.or_matmul_rows.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_int, C.c_int]
        L.or_swiglu.argtypes = [_f32p, _f32p, _u16p, _u16p, _u16p, C.c_int, C.c_int,
                                _f32p, _f32p]
        L.or_softmax.argtypes = [_f32p, C.c_int]
        L.or_rmsnorm.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_float]
        L.or_argmax.restype = C.c_int
        L.or_argmax.argtypes = [_f32p, C.c_int]
        L.or_lm_head_rows.argtypes = [_f32p, _u16p, C.c_float, _u16p, C.c_int, C.c_int, C.c_int,
                                      _f32p, _i32p]
        L.or_route.argtypes = [C.POINTER(MoeCfg), _f32p, _f32p, _ip, _f32p]
        L.or_ffn_compute.argtypes = [C.POINTER(MoeCfg), C.POINTER(MoeWeights), _f32p,
                                     _f32p, _ip, _f32p, _f32p]
        L.or_ffn_compute_rows.argtypes = [C.POINTER(MoeCfg), C.POINTER(MoeWeights),
                                          C.c_int, _f32p, _f32p, _f32p, _ip, _f32p, _f32p]
        L.or_quant_row_i8.argtypes = [_f32p, C.c_int, _i8p, _f32p]
        L.or_quant_rows_i8.argtypes = [_f32p, C.c_int, C.c_int, _i8p, _f32p]
        L.or_quant_weight_i8.argtypes = [_u16p, C.c_int, C.c_int, _i8p, _f32p]
        L.or_gemm_i8.argtypes = [_i8p, _i8p, _i32p, C.c_int, C.c_int, C.c_int]
        L.or_dequant_row.argtypes = [_i32p, C.c_float, _f32p, C.c_int, _f32p]
        L.or_ffn_i8.argtypes = [C.POINTER(MoeCfg), _u16p, _f32p, C.POINTER(MoeI8Weights),
                                C.c_int, _f32p, _f32p, _f32p, _ip, _f32p, _f32p,
                                C.POINTER(I8Debug)]
        L.or_absorbed_head.argtypes = [_f32p, _f32p, _u16p, _u16p, _f32p, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_int, C.c_float, _f32p, _f32p,
                                       _f32p, _f32p]
        L.or_absorbed_decode.argtypes = [_f32p, _u16p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                         C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.c_float, _f32p, _f32p, _f32p, _f32p]
        L.or_rope_inv_freq.argtypes = [C.c_int] + [C.c_float] * 5 + [_f32p]
        L.or_rope_apply.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int]
        L.or_mla_front.argtypes = [C.POINTER(FrontCfg), C.POINTER(FrontWeights), _f32p, _f32p,
                                   C.c_int, _f32p, _f32p, _f32p]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own compiled run.c (only in the build container)."""
    global _ref
    if _ref is None:
        R = C.CDLL(REF_PATH)
        R.ref_matmul.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_int]
        R.ref_silu.restype = C.c_float
        R.ref_silu.argtypes = [C.c_float]
        R.ref_softmax.argtypes = [_f32p, C.c_int]
        R.ref_rmsnorm.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_float]
        R.ref_sample.restype = C.c_int
        R.ref_sample.argtypes = [_f32p, C.c_int]
        R.ref_swiglu.argtypes = [_f32p, _f32p, _u16p, _u16p, _u16p, C.c_int, C.c_int,
                                 _f32p, _f32p]
        R.ref_ffn_compute.argtypes = [C.c_int] * 7 + [C.c_float] + [_u16p, _f32p] + \
            [_u16p] * 6 + [_f32p, _f32p, _ip, _f32p, _f32p]
        R.ref_absorbed_decode.restype = C.c_int
        R.ref_absorbed_decode.argtypes = [C.c_int] * 9 + [C.c_float, _f32p] + [_u16p] * 13 + \
            [_f32p, C.c_char_p, _f32p]
        R.ref_absorbed_decode_ex.restype = C.c_int
        R.ref_absorbed_decode_ex.argtypes = [C.c_int] * 9 + [C.c_float, _f32p, C.c_int, C.c_int] + \
            [_u16p] * 16 + [_f32p, C.c_char_p, _f32p]
        R.ref_rope_apply.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int]
        R.ref_forward_tokens.restype = C.c_int
        R.ref_forward_tokens.argtypes = [C.c_void_p, _ip, C.c_int, _f32p]
        R.ref_prefill_tokens.restype = C.c_int
        R.ref_prefill_tokens.argtypes = [C.c_void_p, _ip, C.c_int, C.c_char_p, _f32p]
        R.ref_config_rope.restype = C.c_int
        R.ref_config_rope.argtypes = [C.c_char_p, _f32p, _ip, _f32p]
        _ref = R
    return _ref


# ---------------------------------------------------------------------------
# numpy-level helpers
# ---------------------------------------------------------------------------

def c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def matmul(x, w):
    """run.c:30 matmul for each row of x ([T, n_in] or [n_in]); w bf16 [d_out, n_in]."""
    x = c32(x)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    d_out, n_in = w.shape
    x2 = x.reshape(-1, n_in)
    y = np.empty((x2.shape[0], d_out), np.float32)
    lib().or_matmul_rows(_p(y, _f32p), _p(x2, _f32p), _p(w, _u16p), x2.shape[0], d_out, n_in)
    return y.reshape(x.shape[:-1] + (d_out,))


def softmax(x):
    x = c32(x).copy()
    lib().or_softmax(_p(x, _f32p), x.size)
    return x


def rmsnorm(x, w, eps):
    """run.c:22-27 on each row of x ([T, n] or [n]); w bf16 [n]."""
    x = c32(x)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    n = w.size
    x2 = x.reshape(-1, n)
    y = np.empty_like(x2)
    for t in range(x2.shape[0]):
        lib().or_rmsnorm(_p(y[t], _f32p), _p(np.ascontiguousarray(x2[t]), _f32p), _p(w, _u16p),
                         n, float(eps))
    return y.reshape(x.shape)


def argmax(logits):
    """run.c:503-508 sample() on each row of logits."""
    lg = c32(logits)
    rows = lg.reshape(-1, lg.shape[-1])
    return np.array([lib().or_argmax(_p(np.ascontiguousarray(r), _f32p), r.size) for r in rows],
                    np.int32).reshape(lg.shape[:-1])


def lm_head_rows(x, norm, eps, lm_head):
    """Final rmsnorm + lm_head matmul + greedy argmax (run.c:493-494, 503-508)
    for T tokens; returns (logits [T, V], tokens [T])."""
    x = c32(x)
    norm = np.ascontiguousarray(norm, dtype=np.uint16)
    lm_head = np.ascontiguousarray(lm_head, dtype=np.uint16)
    V, H = lm_head.shape
    T = x.shape[0]
    logits = np.empty((T, V), np.float32)
    tokens = np.empty(T, np.int32)
    lib().or_lm_head_rows(_p(x, _f32p), _p(norm, _u16p), float(eps), _p(lm_head, _u16p), T, V, H,
                          _p(logits, _f32p), _p(tokens, _i32p))
    return logits, tokens


def moe_cfg(H, E, n_shared, K, I, router_sigmoid=0, norm_topk=0, routed_scaling=1.0):
    return MoeCfg(H, E, n_shared, K, I, router_sigmoid, norm_topk, routed_scaling)


def _weights_struct(w):
    return MoeWeights(_p(w["moe_gate"], _u16p), _p(w.get("moe_gate_bias"), _f32p),
                      _p(w["eg"], _u16p), _p(w["eu"], _u16p), _p(w["ed"], _u16p),
                      _p(w["sg"], _u16p), _p(w["su"], _u16p), _p(w["sd"], _u16p))


def route(cfg, logits, bias=None):
    """Router on one token's logits; returns (probs, idx, w)."""
    s = c32(logits).copy()
    K = cfg.n_experts_per_tok
    idx = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    lib().or_route(C.byref(cfg), _p(s, _f32p), _p(c32(bias) if bias is not None else None, _f32p),
                   _p(idx, _ip), _p(w, _f32p))
    return s, idx, w


def swiglu_rows(xn, gate, up, down):
    """run.c:86-93 swiglu (the dense branch of ffn_compute, run.c:119-122)
    for each row of xn: down . (silu(gate . x) * (up . x))."""
    x2 = c32(xn).reshape(-1, np.shape(gate)[1])
    gate, up, down = (np.ascontiguousarray(a, dtype=np.uint16) for a in (gate, up, down))
    inter, H = gate.shape
    out = np.empty((x2.shape[0], H), np.float32)
    hb = np.empty(inter, np.float32)
    hb2 = np.empty(inter, np.float32)
    for t in range(x2.shape[0]):
        row = np.ascontiguousarray(x2[t])
        lib().or_swiglu(_p(out[t], _f32p), _p(row, _f32p), _p(gate, _u16p), _p(up, _u16p),
                        _p(down, _u16p), inter, H, _p(hb, _f32p), _p(hb2, _f32p))
    return out


def ffn_compute_rows(cfg, w, xn, logits=None):
    """T tokens through the reference MoE FFN; returns out, idx, w, probs."""
    xn = c32(xn)
    T = xn.shape[0]
    H, E, K = cfg.hidden, cfg.n_routed_experts, cfg.n_experts_per_tok
    out = np.empty((T, H), np.float32)
    idx = np.empty((T, K), np.int32)
    wt = np.empty((T, K), np.float32)
    probs = np.empty((T, E), np.float32)
    ws = _weights_struct(w)
    lg = c32(logits) if logits is not None else None
    lib().or_ffn_compute_rows(C.byref(cfg), C.byref(ws), T, _p(xn, _f32p), _p(lg, _f32p),
                              _p(out, _f32p), _p(idx, _ip), _p(wt, _f32p), _p(probs, _f32p))
    return out, idx, wt, probs


def quant_rows(x):
    x = c32(x)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    q = np.empty((rows, n), np.int8)
    s = np.empty(rows, np.float32)
    lib().or_quant_rows_i8(_p(x, _f32p), rows, n, _p(q, _i8p), _p(s, _f32p))
    return q, s


def quant_weight(w):
    w = np.ascontiguousarray(w, dtype=np.uint16)
    K = w.shape[-1]
    q = np.empty(w.shape, np.int8)
    s = np.empty(w.shape[:-1], np.float32)
    if w.size == 0:
        s[...] = 0
        return q, s
    rows = w.size // K
    lib().or_quant_weight_i8(_p(w, _u16p), rows, K, _p(q, _i8p), _p(s, _f32p))
    return q, s


def gemm_i8(a, b):
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    M, K = a.shape
    N = b.shape[0]
    c = np.empty((M, N), np.int32)
    lib().or_gemm_i8(_p(a, _i8p), _p(b, _i8p), _p(c, _i32p), M, N, K)
    return c


def quantize_moe_weights(w):
    """Per-output-channel int8 quantisation of every expert matrix."""
    q = {}
    for k in ("eg", "eu", "ed", "sg", "su", "sd"):
        q["q" + k], q["s" + k] = quant_weight(w[k])
    return q


def ffn_i8(cfg, w, qw, xn, logits=None, debug=False):
    """T tokens through the int8 MoE layer (or_ffn_i8)."""
    xn = c32(xn)
    T = xn.shape[0]
    H, E, K, I = cfg.hidden, cfg.n_routed_experts, cfg.n_experts_per_tok, cfg.moe_inter_size
    S = cfg.n_shared_experts * I
    out = np.empty((T, H), np.float32)
    idx = np.empty((T, K), np.int32)
    wt = np.empty((T, K), np.float32)
    probs = np.empty((T, E), np.float32)
    ws = MoeI8Weights(_p(qw["qeg"], _i8p), _p(qw["qeu"], _i8p), _p(qw["seg"], _f32p),
                      _p(qw["seu"], _f32p), _p(qw["qed"], _i8p), _p(qw["sed"], _f32p),
                      _p(qw["qsg"], _i8p), _p(qw["qsu"], _i8p), _p(qw["ssg"], _f32p),
                      _p(qw["ssu"], _f32p), _p(qw["qsd"], _i8p), _p(qw["ssd"], _f32p))
    dbg = None
    d = {}
    if debug:
        d = dict(qx=np.empty((T, H), np.int8), sx=np.empty(T, np.float32),
                 acc_gu=np.empty((T, K, 2, I), np.int32), qh=np.empty((T, K, I), np.int8),
                 sh=np.empty((T, K), np.float32), acc_d=np.empty((T, K, H), np.int32),
                 qhs=np.empty((T, max(S, 1)), np.int8), shs=np.empty(T, np.float32))
        dbg = I8Debug(_p(d["qx"], _i8p), _p(d["sx"], _f32p), _p(d["acc_gu"], _i32p),
                      _p(d["qh"], _i8p), _p(d["sh"], _f32p), _p(d["acc_d"], _i32p),
                      _p(d["qhs"], _i8p), _p(d["shs"], _f32p))
    lg = c32(logits) if logits is not None else None
    bias = w.get("moe_gate_bias")
    lib().or_ffn_i8(C.byref(cfg), _p(w["moe_gate"], _u16p),
                    _p(c32(bias) if bias is not None else None, _f32p), C.byref(ws), T,
                    _p(xn, _f32p), _p(lg, _f32p), _p(out, _f32p), _p(idx, _ip),
                    _p(wt, _f32p), _p(probs, _f32p), C.byref(dbg) if dbg else None)
    return out, idx, wt, probs, d


def absorbed_decode(q, kv_b, cache, kv_len, NH, QKN, QKR, KVL, VHD, scale=None,
                    seq_stride=None):
    """B sequences x NH heads of the absorbed chain.  cache: [B, L, KVL+QKR]
    uint16 (bf16) or float32.  Returns ctx, qabs, probs, clat."""
    q = c32(q)
    B = q.shape[0]
    kv_b = np.ascontiguousarray(kv_b, dtype=np.uint16)
    is_bf16 = cache.dtype == np.uint16
    cache = np.ascontiguousarray(cache)
    L = cache.shape[1] if seq_stride is None else seq_stride
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(QKN + QKR)))
    ctx = np.empty((B, NH * VHD), np.float32)
    qabs = np.empty((B, NH, KVL), np.float32)
    probs = np.empty((B, NH, kv_len), np.float32)
    clat = np.empty((B, NH, KVL), np.float32)
    lib().or_absorbed_decode(_p(q, _f32p), _p(kv_b, _u16p), cache.ctypes.data_as(C.c_void_p),
                             int(is_bf16), B, NH, QKN, QKR, KVL, VHD, kv_len, L,
                             C.c_float(scale), _p(ctx, _f32p), _p(qabs, _f32p),
                             _p(probs, _f32p), _p(clat, _f32p))
    return ctx, qabs, probs, clat


def rope_inv_freq(dim, theta, factor=1.0, beta_fast=32.0, beta_slow=1.0, orig_max=4096.0):
    inv = np.empty(dim // 2, np.float32)
    lib().or_rope_inv_freq(dim, theta, factor, beta_fast, beta_slow, orig_max, _p(inv, _f32p))
    return inv


def rope_apply(v, pos, inv, interleaved=0):
    """RoPE of every row of v [..., dim] at `pos` (one position for all rows)."""
    v = c32(v).copy()
    inv = c32(inv)
    dim = v.shape[-1]
    for row in v.reshape(-1, dim):
        lib().or_rope_apply(_p(row, _f32p), int(pos), _p(inv, _f32p), dim, int(interleaved))
    return v


def front_cfg(H, NH, QKN, QKR, KVL, q_lora=0, rms_eps=1e-6, mla_eps=1e-6, interleaved=0):
    return FrontCfg(H, NH, QKN, QKR, KVL, q_lora, rms_eps, mla_eps, interleaved)


def _front_struct(w):
    return FrontWeights(*[_p(w.get(n), _u16p) if w.get(n) is not None else None
                          for n, _ in FrontWeights._fields_])


def mla_front(cfg, w, inv, x, pos):
    """B tokens of the decode front, token b at position pos[b].  Returns q
    [B, NH*(QKN+QKR)], kv [B, KVL+QKR] (the fp32 cache rows), comp [B, KVL+QKR]."""
    x = c32(np.atleast_2d(x))
    B = x.shape[0]
    inv = c32(inv)
    QD = cfg.n_heads * (cfg.qk_nope + cfg.qk_rope)
    KVD = cfg.kv_lora + cfg.qk_rope
    q = np.empty((B, QD), np.float32)
    kv = np.empty((B, KVD), np.float32)
    comp = np.empty((B, KVD), np.float32)
    ws = _front_struct({k: np.ascontiguousarray(v, dtype=np.uint16) for k, v in w.items()
                        if v is not None})
    pos = np.broadcast_to(np.asarray(pos), (B,))
    for b in range(B):
        lib().or_mla_front(C.byref(cfg), C.byref(ws), _p(inv, _f32p), _p(x[b], _f32p),
                           int(pos[b]), _p(q[b], _f32p), _p(kv[b], _f32p), _p(comp[b], _f32p))
    return q, kv, comp


# ---------------------------------------------------------------------------
# reference-library helpers (build container only)
# ---------------------------------------------------------------------------

def ref_rmsnorm(x, w, eps):
    x = c32(x)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    y = np.empty_like(x)
    ref().ref_rmsnorm(_p(y, _f32p), _p(x, _f32p), _p(w, _u16p), x.size, float(eps))
    return y


def ref_sample(logits):
    lg = c32(logits).copy()
    return int(ref().ref_sample(_p(lg, _f32p), lg.size))


def ref_matmul(x, w):
    x = c32(x)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    d_out, n_in = w.shape
    y = np.empty(d_out, np.float32)
    ref().ref_matmul(_p(y, _f32p), _p(x, _f32p), _p(w, _u16p), d_out, n_in)
    return y


def ref_softmax(x):
    x = c32(x).copy()
    ref().ref_softmax(_p(x, _f32p), x.size)
    return x


def ref_ffn_compute(cfg, w, xn):
    """One token through the reference's own ffn_compute."""
    xn = c32(xn)
    H, E, K = cfg.hidden, cfg.n_routed_experts, cfg.n_experts_per_tok
    out = np.empty(H, np.float32)
    idx = np.empty(K, np.int32)
    wt = np.empty(K, np.float32)
    probs = np.empty(E, np.float32)
    bias = w.get("moe_gate_bias")
    ref().ref_ffn_compute(cfg.hidden, E, cfg.n_shared_experts, K, cfg.moe_inter_size,
                          cfg.router_sigmoid, cfg.norm_topk, C.c_float(cfg.routed_scaling),
                          _p(w["moe_gate"], _u16p),
                          _p(c32(bias) if bias is not None else None, _f32p),
                          _p(w["eg"], _u16p), _p(w["eu"], _u16p), _p(w["ed"], _u16p),
                          _p(w["sg"], _u16p), _p(w["su"], _u16p), _p(w["sd"], _u16p),
                          _p(xn, _f32p), _p(out, _f32p), _p(idx, _ip), _p(wt, _f32p),
                          _p(probs, _f32p))
    return out, idx, wt, probs


def ref_rope_apply(v, pos, inv, interleaved=0):
    v = c32(v).copy()
    inv = c32(inv)
    dim = v.shape[-1]
    for row in v.reshape(-1, dim):
        ref().ref_rope_apply(_p(row, _f32p), int(pos), _p(inv, _f32p), dim, int(interleaved))
    return v


def ref_config_rope(model_dir):
    """The reference's config_from_json + build_rope_inv_freq on
    <model_dir>/config.json.  Returns (inv_freq, ints, floats) as documented
    in oracle/ref/ref_model.c."""
    ints = np.zeros(8, np.int32)
    flts = np.zeros(8, np.float32)
    inv = np.zeros(512, np.float32)
    ref().ref_config_rope(model_dir.encode(), _p(inv, _f32p), _p(ints, _ip), _p(flts, _f32p))
    return inv[:ints[0] // 2].copy(), ints, flts


# ---------------------------------------------------------------------------
# whole decode steps (src/run.c:379-501)
# ---------------------------------------------------------------------------

def model_logits(c, m, tokens, inv, int8=False):
    """forward_absorbed at positions 0..n-1 on tokens (teacher forcing),
    composed from the restated pieces in the reference's order; c: dict of
    the Config fields (n_layers, first_dense, H, NH, QKN, QKR, KVL, VHD,
    dense_inter, E, n_shared, K, I, vocab, router_sigmoid, norm_topk,
    routed_scaling, rms_eps), m: synth.model().  With int8 the MoE layers
    run the int8 expert scheme (ffn_i8 on per-channel quantised weights,
    the library's MM_FWD_INT8) instead of ffn_compute.  Returns [n, vocab]."""
    H, NH, QKN, QKR, KVL, VHD = (c[k] for k in ("H", "NH", "QKN", "QKR", "KVL", "VHD"))
    KVD, eps, n = KVL + QKR, c["rms_eps"], len(tokens)
    fc = front_cfg(H, NH, QKN, QKR, KVL, c.get("q_lora", 0), eps, 1e-6, c.get("interleaved", 0))
    mc = moe_cfg(H, c["E"], c["n_shared"], c["K"], c["I"], c["router_sigmoid"], c["norm_topk"],
                 c["routed_scaling"])
    caches = [np.zeros((n, KVD), np.float32) for _ in m["layers"]]
    out = np.empty((n, c["vocab"]), np.float32)
    qws = [quantize_moe_weights(lw) if int8 and l >= c["first_dense"] else None
           for l, lw in enumerate(m["layers"])]
    for p, tok in enumerate(tokens):
        x = (m["embed"][tok].astype(np.uint32) << 16).view(np.float32).copy()
        for l, lw in enumerate(m["layers"]):
            q, kv, _ = mla_front(fc, lw, inv, x, p)
            caches[l][p] = kv[0]
            ctx, _, _, _ = absorbed_decode(q.reshape(1, NH, -1), lw["kv_b"], caches[l][None, :p + 1],
                                           p + 1, NH, QKN, QKR, KVL, VHD)
            x = (x + matmul(ctx[0], lw["o_proj"])).astype(np.float32)
            xb = rmsnorm(x, lw["post_norm"], eps)
            if l < c["first_dense"]:
                hb = np.empty(c["dense_inter"], np.float32)
                hb2 = np.empty(c["dense_inter"], np.float32)
                mo = np.empty(H, np.float32)
                lib().or_swiglu(_p(mo, _f32p), _p(c32(xb), _f32p), _p(lw["dgate"], _u16p),
                                _p(lw["dup"], _u16p), _p(lw["ddown"], _u16p), c["dense_inter"], H,
                                _p(hb, _f32p), _p(hb2, _f32p))
            elif int8:
                mo = ffn_i8(mc, lw, qws[l], xb[None])[0][0]
            else:
                mo = ffn_compute_rows(mc, lw, xb[None])[0][0]
            x = (x + mo).astype(np.float32)
        out[p] = matmul(rmsnorm(x, m["final_norm"], eps), m["lm_head"])
    return out


class RefModelSpec(C.Structure):
    _fields_ = [(k, C.c_int) for k in ("n_layers", "first_k_dense", "H", "NH", "QKN", "QKR",
                                        "KVL", "VHD", "dense_inter", "E", "n_shared", "K", "I",
                                        "vocab", "router_sigmoid", "norm_topk", "max_seq",
                                        "q_lora", "interleaved")] + \
        [("routed_scaling", C.c_float), ("rms_eps", C.c_float), ("inv_freq", _f32p),
         ("embed", _u16p), ("final_norm", _u16p), ("lm_head", _u16p)] + \
        [(k, C.POINTER(_u16p)) for k in ("in_norm", "q_proj", "kv_a", "kv_a_norm", "kv_b",
                                         "o_proj", "post_norm", "dgate", "dup", "ddown",
                                         "moe_gate", "eg", "eu", "ed", "sg", "su", "sd",
                                         "q_a_proj", "q_a_norm", "q_b_proj")] + \
        [("moe_bias", C.POINTER(_f32p))]


def ref_forward_tokens(c, m, tokens, inv, prefill=False):
    """The reference's own forward_absorbed over tokens (teacher forcing), or
    with prefill its forward_unabsorbed over the whole prompt (every
    position's logits, from its dump).  Returns [n, vocab]."""
    L = len(m["layers"])
    keep = []

    def arr(key, src="layers"):
        ptrs = (_u16p * L)()
        for l, lw in enumerate(m["layers"]):
            a = lw.get(key)
            if a is not None:
                a = np.ascontiguousarray(a, np.uint16)
                keep.append(a)
                ptrs[l] = _p(a, _u16p)
        return ptrs
    bias = (_f32p * L)()
    for l, lw in enumerate(m["layers"]):
        if lw.get("moe_gate_bias") is not None:
            b = c32(lw["moe_gate_bias"])
            keep.append(b)
            bias[l] = _p(b, _f32p)
    n = len(tokens)
    inv = c32(inv)
    spec = RefModelSpec(L, c["first_dense"], c["H"], c["NH"], c["QKN"], c["QKR"], c["KVL"], c["VHD"],
                        c["dense_inter"], c["E"], c["n_shared"], c["K"], c["I"], c["vocab"],
                        c["router_sigmoid"], c["norm_topk"], max(n, 1), c.get("q_lora", 0),
                        c.get("interleaved", 0), c["routed_scaling"],
                        c["rms_eps"], _p(inv, _f32p), _p(m["embed"], _u16p),
                        _p(m["final_norm"], _u16p), _p(m["lm_head"], _u16p),
                        *[arr(k) for k in ("in_norm", "q_proj", "kv_a", "kv_a_norm", "kv_b",
                                           "o_proj", "post_norm", "dgate", "dup", "ddown",
                                           "moe_gate", "eg", "eu", "ed", "sg", "su", "sd",
                                           "q_a_proj", "q_a_norm", "q_b_proj")],
                        bias)
    out = np.empty((n, c["vocab"]), np.float32)
    tk = np.ascontiguousarray(tokens, np.int32)
    if not prefill:
        assert ref().ref_forward_tokens(C.byref(spec), _p(tk, _ip), n, _p(out, _f32p)) == 0
        return out
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        assert ref().ref_prefill_tokens(C.byref(spec), _p(tk, _ip), n, d.encode(),
                                        _p(out, _f32p)) == 0
    return out
