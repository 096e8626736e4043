"""Python mirror of the libmlamoe C-ABI (include/mlamoe.h), over ctypes.

This is the host-side interface the tests and the benchmark drive; it keeps
the reference's names and argument meanings (ffn_compute, matmul, the
absorbed-decode chain).  Errors are raised as MMError carrying the library's
message.  The HIP library is required: importing works without it, but
creating a Context fails loudly when libmlamoe.so is missing or no gfx950
device is present.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("MLAMOE_LIB") or os.path.join(PKG_DIR, "libmlamoe.so")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "mlamoe.h")

MM_LOAD_BF16, MM_LOAD_INT8, MM_LOAD_DEVICE_PTRS = 1, 2, 4
MM_FWD_BF16, MM_FWD_INT8, MM_FWD_ACCUMULATE = 0, 1, 2
MM_FILL_BF16_NORMAL, MM_FILL_F32_NORMAL, MM_FILL_F32_UNIFORM = 0, 1, 2
MM_MATMUL_X_BF16, MM_MATMUL_ACCUMULATE, MM_MATMUL_W_HOST = 1, 2, 4

_vp = C.c_void_p


class MMError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"mlamoe status {status}: {msg}")
        self.status = status


class MoeConfig(C.Structure):
    """Mirror of mm_moe_config (the MoE fields of the reference Config)."""
    _fields_ = [("hidden_size", C.c_int), ("n_routed_experts", C.c_int),
                ("n_shared_experts", C.c_int), ("n_experts_per_tok", C.c_int),
                ("moe_inter_size", C.c_int), ("router_sigmoid", C.c_int),
                ("norm_topk", C.c_int), ("routed_scaling", C.c_float)]


class MoeLayerWeights(C.Structure):
    _fields_ = [("moe_gate", _vp), ("moe_gate_bias", _vp), ("expert_gate", C.POINTER(_vp)),
                ("expert_up", C.POINTER(_vp)), ("expert_down", C.POINTER(_vp)),
                ("shared_gate", _vp), ("shared_up", _vp), ("shared_down", _vp)]


class MlaConfig(C.Structure):
    """Mirror of mm_mla_config (the attention fields of the reference Config)."""
    _fields_ = [("n_heads", C.c_int), ("qk_nope_head_dim", C.c_int),
                ("qk_rope_head_dim", C.c_int), ("kv_lora_rank", C.c_int),
                ("v_head_dim", C.c_int), ("softmax_scale", C.c_float)]


class MlaFrontConfig(C.Structure):
    """Mirror of mm_mla_front_config."""
    _fields_ = [("hidden_size", C.c_int), ("q_lora_rank", C.c_int), ("rms_eps", C.c_float),
                ("mla_norm_eps", C.c_float), ("rope_interleaved", C.c_int),
                ("rope_inv_freq", C.POINTER(C.c_float))]


FRONT_WEIGHTS = ("input_norm", "q_proj", "q_a_proj", "q_a_norm", "q_b_proj", "kv_a_proj",
                 "kv_a_norm")


class MlaFrontWeights(C.Structure):
    """Mirror of mm_mla_front_weights (device pointers)."""
    _fields_ = [(n, _vp) for n in FRONT_WEIGHTS]


class EngineConfig(C.Structure):
    """Mirror of mm_engine_config."""
    _fields_ = [("n_layers", C.c_int), ("first_k_dense", C.c_int), ("hidden_size", C.c_int),
                ("dense_inter_size", C.c_int), ("vocab_size", C.c_int), ("rms_eps", C.c_float),
                ("max_batch", C.c_int), ("max_seq", C.c_int), ("moe_flags", C.c_uint),
                ("init_seq", C.c_int), ("max_rows", C.c_int)]


class EngineLayer(C.Structure):
    """Mirror of mm_engine_layer (device pointers)."""
    _fields_ = [("front", MlaFrontWeights), ("o_proj", _vp), ("post_norm", _vp),
                ("dense_gate", _vp), ("dense_up", _vp), ("dense_down", _vp)]


class MoeI8Debug(C.Structure):
    _fields_ = [(n, _vp) for n in ("qx", "sx", "acc_gu", "h", "qh", "sh", "acc_d", "y", "hs",
                                   "qhs", "shs", "ys")]


_lib = None


def header_functions():
    """Names of the functions include/mlamoe.h declares."""
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(mm_\w+)\s*\(", src, flags=re.M)))


def lib():
    """Load libmlamoe.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MMError(-2, f"{LIB_PATH} not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        L.mm_last_error.restype = C.c_char_p
        L.mm_ctx_create.argtypes = [C.c_int, C.POINTER(_vp)]
        L.mm_ctx_destroy.argtypes = [_vp]
        L.mm_ctx_destroy.restype = None
        L.mm_ctx_stream.argtypes = [_vp]
        L.mm_ctx_stream.restype = _vp
        L.mm_ctx_sync.argtypes = [_vp]
        L.mm_ctx_set_stream.argtypes = [_vp, _vp]
        L.mm_dev_alloc.argtypes = [_vp, C.c_size_t, C.POINTER(_vp)]
        L.mm_dev_free.argtypes = [_vp, _vp]
        for f in (L.mm_h2d, L.mm_d2h, L.mm_d2d):
            f.argtypes = [_vp, _vp, _vp, C.c_size_t]
        L.mm_fill_synthetic.argtypes = [_vp, _vp, C.c_size_t, C.c_int, C.c_uint64, C.c_float]
        L.mm_timer_start.argtypes = [_vp]
        L.mm_timer_stop.argtypes = [_vp, C.POINTER(C.c_float)]
        L.mm_prof_enable.argtypes = [_vp, C.c_int]
        L.mm_prof_reset.argtypes = [_vp]
        L.mm_prof_query.argtypes = [_vp, C.c_char_p, C.POINTER(C.c_double),
                                    C.POINTER(C.c_longlong)]
        L.mm_moe_init.argtypes = [_vp, C.POINTER(MoeConfig), C.c_int]
        L.mm_moe_load_layer.argtypes = [_vp, C.c_int, C.POINTER(MoeLayerWeights), C.c_uint]
        L.mm_moe_forward_dev.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                         C.c_uint]
        L.mm_ffn_compute.argtypes = [_vp, C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_uint]
        L.mm_moe_forward.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_uint]
        L.mm_moe_load_dense_layer.argtypes = [_vp, C.c_int, _vp, _vp, _vp, C.c_int, C.c_uint]
        L.mm_matmul_bf16.argtypes = [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_uint]
        L.mm_host_weights_release.argtypes = [_vp]
        L.mm_mla_absorbed_decode.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, C.c_int, _vp,
                                             C.c_int, _vp, _vp, _vp, _vp]
        L.mm_ctx_workspace_bytes.argtypes = [_vp, C.POINTER(C.c_size_t)]
        L.mm_moe_forward_noalloc_dev.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                                 _vp, C.c_uint]
        L.mm_matmul_bf16_dev.argtypes = [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_uint]
        L.mm_matmul_bf16_hl_dev.argtypes = [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_uint]
        L.mm_mla_init.argtypes = [_vp, C.POINTER(MlaConfig), C.c_int]
        L.mm_mla_load_layer.argtypes = [_vp, C.c_int, _vp, C.c_uint]
        L.mm_mla_absorbed_decode_dev.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, C.c_int, _vp,
                                                 C.c_int, _vp, _vp, _vp, _vp]
        L.mm_moe_router_logits_dev.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp]
        L.mm_moe_forward_i8_debug_dev.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp,
                                                  _vp, _vp, C.c_uint, C.POINTER(MoeI8Debug)]
        L.mm_rmsnorm_dev.argtypes = [_vp, C.c_int, _vp, _vp, C.c_int, C.c_float, _vp]
        L.mm_argmax_dev.argtypes = [_vp, C.c_int, _vp, C.c_int, _vp]
        L.mm_lm_head_dev.argtypes = [_vp, C.c_int, _vp, _vp, C.c_float, _vp, C.c_int, C.c_int,
                                     _vp, _vp]
        L.mm_moe_i8_layer_size.argtypes = [C.POINTER(MoeConfig), C.POINTER(C.c_size_t),
                                           C.POINTER(C.c_size_t)]
        L.mm_moe_export_layer_i8.argtypes = [_vp, C.c_int, _vp, _vp]
        L.mm_moe_load_layer_i8_packed.argtypes = [_vp, C.c_int, _vp, _vp, _vp, _vp, C.c_uint]
        L.mm_engine_create.argtypes = [_vp, C.POINTER(EngineConfig), C.POINTER(_vp)]
        L.mm_engine_destroy.argtypes = [_vp]
        L.mm_engine_destroy.restype = None
        L.mm_engine_set_layer.argtypes = [_vp, C.c_int, C.POINTER(EngineLayer)]
        L.mm_engine_set_head.argtypes = [_vp, _vp, _vp, _vp]
        L.mm_engine_step.argtypes = [_vp, C.c_int, _vp, _vp, _vp, _vp]
        L.mm_engine_step_rows.argtypes = [_vp, C.c_int, _vp, _vp, _vp, C.c_int, _vp, _vp, _vp]
        L.mm_engine_capacity.argtypes = [_vp]
        L.mm_engine_reserve.argtypes = [_vp, C.c_int]
        L.mm_engine_generate.argtypes = [_vp, C.c_int, C.POINTER(_vp), _vp, C.c_int, C.c_int,
                                         C.POINTER(_vp), _vp]
        L.mm_engine_generate.restype = C.c_longlong
        L.mm_rope_inv_freq.argtypes = [C.c_int] + [C.c_float] * 5 + [C.POINTER(C.c_float)]
        L.mm_mla_front_init.argtypes = [_vp, C.POINTER(MlaFrontConfig)]
        L.mm_mla_front_dev.argtypes = [_vp, C.c_int, _vp, C.POINTER(MlaFrontWeights), _vp, _vp,
                                       _vp, C.c_int, _vp]
        _lib = L
    return _lib


def rope_inv_freq(dim, theta, factor=1.0, beta_fast=32.0, beta_slow=1.0, orig_max=4096.0):
    """The RoPE inverse-frequency table (build_rope_inv_freq,
    src/model_load.c:299-325) from the library's host code."""
    inv = np.empty(dim // 2, np.float32)
    _check(lib().mm_rope_inv_freq(dim, theta, factor, beta_fast, beta_slow, orig_max,
                                  inv.ctypes.data_as(C.POINTER(C.c_float))))
    return inv


def _check(st):
    if st != 0:
        raise MMError(st, lib().mm_last_error().decode())


class DevBuf:
    """A device allocation owned by a Context."""

    def __init__(self, ctx, nbytes, dtype=np.uint8, shape=None):
        self.ctx, self.nbytes, self.dtype = ctx, int(nbytes), np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = _vp()
        _check(lib().mm_dev_alloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            _check(lib().mm_dev_free(self.ctx.h, self.ptr))
            self.ptr = None

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib().mm_h2d(self.ctx.h, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype=None, shape=None):
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        shp = shape if shape is not None else self.shape
        out = np.empty(shp, dt)
        _check(lib().mm_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out


class Context:
    """One mm_ctx: a device, its stream and the weights it holds."""

    def __init__(self, device=0):
        h = _vp()
        _check(lib().mm_ctx_create(device, C.byref(h)))
        self.h = h.value
        self._bufs = []
        self._moe_cfg = None

    def close(self):
        if self.h:
            for b in self._bufs:
                b.free()
            self._bufs = []
            lib().mm_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # memory --------------------------------------------------------------
    def alloc(self, nbytes, dtype=np.uint8, shape=None, keep=True):
        b = DevBuf(self, nbytes, dtype, shape)
        if keep:
            self._bufs.append(b)
        return b

    def to_device(self, a):
        a = np.ascontiguousarray(a)
        return self.alloc(max(a.nbytes, 1), a.dtype, a.shape).upload(a)

    def empty(self, shape, dtype):
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        return self.alloc(max(n, 1), dt, tuple(shape))

    def fill(self, buf, n, kind, seed, std=1.0):
        _check(lib().mm_fill_synthetic(self.h, buf.ptr, n, kind, seed, std))

    def sync(self):
        _check(lib().mm_ctx_sync(self.h))

    def set_stream(self, stream):
        """Queue on a caller-owned hipStream_t (an int handle), or on the
        context's own stream again with None."""
        _check(lib().mm_ctx_set_stream(self.h, stream))

    def stream(self):
        return lib().mm_ctx_stream(self.h)

    def workspace_bytes(self):
        """Device workspace the context holds now (mm_ctx_workspace_bytes)."""
        n = C.c_size_t()
        _check(lib().mm_ctx_workspace_bytes(self.h, C.byref(n)))
        return n.value

    # timing --------------------------------------------------------------
    def timer_start(self):
        _check(lib().mm_timer_start(self.h))

    def timer_stop(self):
        ms = C.c_float()
        _check(lib().mm_timer_stop(self.h, C.byref(ms)))
        return ms.value

    def prof_enable(self, on=True):
        _check(lib().mm_prof_enable(self.h, int(on)))

    def prof_reset(self):
        _check(lib().mm_prof_reset(self.h))

    def prof_query(self, kernel):
        t = C.c_double()
        n = C.c_longlong()
        _check(lib().mm_prof_query(self.h, kernel.encode(), C.byref(t), C.byref(n)))
        return t.value, n.value

    # MoE FFN ---------------------------------------------------------------
    def moe_init(self, H, E, n_shared, K, I, router_sigmoid=0, norm_topk=0,
                 routed_scaling=1.0, n_layers=1):
        cfg = MoeConfig(H, E, n_shared, K, I, router_sigmoid, norm_topk, routed_scaling)
        _check(lib().mm_moe_init(self.h, C.byref(cfg), n_layers))
        self._moe_cfg = cfg

    def moe_load_layer(self, layer, w, flags=MM_LOAD_BF16):
        """w: dict of numpy arrays as mlamoe.synth.moe_layer returns (host
        pointers), or of DevBufs with flags | MM_LOAD_DEVICE_PTRS."""
        cfg = self._moe_cfg
        E, I, H = cfg.n_routed_experts, cfg.moe_inter_size, cfg.hidden_size
        dev = bool(flags & MM_LOAD_DEVICE_PTRS)
        keep = []

        def base(a):
            if a is None:
                return None
            if dev:
                return a.ptr
            a = np.ascontiguousarray(a)
            keep.append(a)
            return a.ctypes.data

        def per_expert(a, rows, cols):
            b = base(a)
            step = rows * cols * 2
            return (_vp * E)(*[b + e * step for e in range(E)])
        eg, eu, ed = per_expert(w["eg"], I, H), per_expert(w["eu"], I, H), per_expert(w["ed"], H, I)
        lw = MoeLayerWeights(base(w["moe_gate"]), base(w.get("moe_gate_bias")), eg, eu, ed,
                             base(w["sg"]), base(w["su"]), base(w["sd"]))
        _check(lib().mm_moe_load_layer(self.h, layer, C.byref(lw), flags))

    def moe_load_dense_layer(self, layer, gate, up, down, flags=0):
        """A dense SwiGLU layer (the reference's first_k_dense layers):
        gate/up [DI, H], down [H, DI] bf16 host arrays (or DevBufs with
        MM_LOAD_DEVICE_PTRS)."""
        if flags & MM_LOAD_DEVICE_PTRS:
            ptrs, di = (gate.ptr, up.ptr, down.ptr), gate.shape[0]
        else:
            gate, up, down = (np.ascontiguousarray(a, np.uint16) for a in (gate, up, down))
            ptrs, di = (gate.ctypes.data, up.ctypes.data, down.ctypes.data), gate.shape[0]
        _check(lib().mm_moe_load_dense_layer(self.h, layer, *ptrs, int(di), flags))

    def moe_forward_host(self, layer, xn, flags=MM_FWD_BF16, out=None, want=True):
        """mm_moe_forward: host arrays in and out through the synchronous
        host-pointer entry point.  Returns out, topk_idx, topk_w, probs (the
        last three preset to -1 / NaN so a dense layer shows them untouched)."""
        cfg = self._moe_cfg
        xn = np.ascontiguousarray(xn, np.float32)
        T = xn.shape[0]
        E, K, H = cfg.n_routed_experts, cfg.n_experts_per_tok, cfg.hidden_size
        o = np.zeros((T, H), np.float32) if out is None else \
            np.array(out, np.float32, copy=True, order="C")
        idx = np.full((T, K), -1, np.int32)
        w = np.full((T, K), np.nan, np.float32)
        p = np.full((T, E), np.nan, np.float32)
        q = (lambda a: a.ctypes.data) if want else (lambda a: None)
        _check(lib().mm_moe_forward(self.h, layer, T, xn.ctypes.data, o.ctypes.data, q(idx), q(w),
                                    q(p), flags))
        return o, idx, w, p

    def moe_forward_dev(self, layer, T, xn, out, logits=None, topk_idx=None, topk_w=None,
                        probs=None, flags=MM_FWD_BF16):
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        _check(lib().mm_moe_forward_dev(self.h, layer, T, p(xn), p(out), p(logits),
                                        p(topk_idx), p(topk_w), p(probs), flags))

    def moe_forward(self, layer, xn, logits=None, flags=MM_FWD_BF16):
        """Host arrays in and out: returns out, topk_idx, topk_w, probs."""
        cfg = self._moe_cfg
        xn = np.ascontiguousarray(xn, np.float32)
        T = xn.shape[0]
        E, K, H = cfg.n_routed_experts, cfg.n_experts_per_tok, cfg.hidden_size
        dx = self.alloc(xn.nbytes, keep=False).upload(xn)
        dout = self.alloc(T * H * 4, keep=False)
        didx = self.alloc(T * K * 4, keep=False)
        dw = self.alloc(T * K * 4, keep=False)
        dp = self.alloc(T * E * 4, keep=False)
        dl = None
        if logits is not None:
            dl = self.alloc(T * E * 4, keep=False).upload(np.ascontiguousarray(logits, np.float32))
        try:
            self.moe_forward_dev(layer, T, dx, dout, dl, didx, dw, dp, flags)
            return (dout.download(np.float32, (T, H)), didx.download(np.int32, (T, K)),
                    dw.download(np.float32, (T, K)), dp.download(np.float32, (T, E)))
        finally:
            for b in (dx, dout, didx, dw, dp, dl):
                if b is not None:
                    b.free()

    def router_logits_dev(self, layer, T, xn, logits, logit_bias=None):
        _check(lib().mm_moe_router_logits_dev(self.h, layer, T, xn.ptr,
                                              logit_bias.ptr if logit_bias is not None else None,
                                              logits.ptr))

    def router_logits(self, layer, xn, logit_bias=None):
        xn = np.ascontiguousarray(xn, np.float32)
        T = xn.shape[0]
        E = self._moe_cfg.n_routed_experts
        dx = self.to_device(xn)
        dl = self.empty((T, E), np.float32)
        db = self.to_device(np.ascontiguousarray(logit_bias, np.float32)) \
            if logit_bias is not None else None
        self.router_logits_dev(layer, T, dx, dl, db)
        out = dl.download()
        for b in [dx, dl] + ([db] if db is not None else []):
            b.free()
            self._bufs.remove(b)
        return out

    def moe_forward_i8_debug(self, layer, xn, logits=None, flags=MM_FWD_INT8):
        """int8 forward returning (out, idx, w, probs, intermediates dict)."""
        cfg = self._moe_cfg
        xn = np.ascontiguousarray(xn, np.float32)
        T = xn.shape[0]
        E, K, H = cfg.n_routed_experts, cfg.n_experts_per_tok, cfg.hidden_size
        I = cfg.moe_inter_size
        S = cfg.n_shared_experts * I
        R = T * K
        shapes = dict(qx=((T, H), np.int8), sx=((T,), np.float32),
                      acc_gu=((R, 2, I), np.int32), h=((R, I), np.float32),
                      qh=((R, I), np.int8), sh=((R,), np.float32), acc_d=((R, H), np.int32),
                      y=((R, H), np.float32), hs=((T, max(S, 1)), np.float32),
                      qhs=((T, max(S, 1)), np.int8), shs=((T,), np.float32),
                      ys=((T, H), np.float32))
        bufs = {k: self.empty(shp, dt) for k, (shp, dt) in shapes.items()}
        dbg = MoeI8Debug(*[bufs[n].ptr for n, _ in MoeI8Debug._fields_])
        dx = self.to_device(xn)
        dout = self.empty((T, H), np.float32)
        didx = self.empty((T, K), np.int32)
        dw = self.empty((T, K), np.float32)
        dp = self.empty((T, E), np.float32)
        dl = self.to_device(np.ascontiguousarray(logits, np.float32)) if logits is not None else None
        _check(lib().mm_moe_forward_i8_debug_dev(self.h, layer, T, dx.ptr, dout.ptr,
                                                 dl.ptr if dl else None, didx.ptr, dw.ptr,
                                                 dp.ptr, flags, C.byref(dbg)))
        res = {k: b.download() for k, b in bufs.items()}
        out = (dout.download(), didx.download(), dw.download(), dp.download(), res)
        for b in list(bufs.values()) + [dx, dout, didx, dw, dp] + ([dl] if dl else []):
            b.free()
            self._bufs.remove(b)
        return out

    # dense bf16 matmul ----------------------------------------------------------
    def matmul_dev(self, y, x, w, d_out, n_in, T, flags=0):
        _check(lib().mm_matmul_bf16_dev(self.h, y.ptr, x.ptr, w.ptr, d_out, n_in, T, flags))

    def matmul_hl(self, xhl, w, flags=0, y0=None):
        """mm_matmul_bf16_hl_dev: x given as bf16 hi/lo planes [2, T, n_in]."""
        xhl = np.ascontiguousarray(xhl, np.uint16)
        w = np.ascontiguousarray(w, np.uint16)
        T, (d_out, n_in) = xhl.shape[1], w.shape
        dx, dw = self.to_device(xhl), self.to_device(w)
        dy = self.to_device(np.ascontiguousarray(y0, np.float32)) if y0 is not None else \
            self.empty((T, d_out), np.float32)
        _check(lib().mm_matmul_bf16_hl_dev(self.h, dy.ptr, dx.ptr, dw.ptr, d_out, n_in, T, flags))
        y = dy.download()
        for b in (dx, dw, dy):
            b.free()
            self._bufs.remove(b)
        return y

    def matmul_host(self, x, w, flags=MM_MATMUL_W_HOST, y0=None):
        """mm_matmul_bf16: host x (and y), w a host bf16 array (kept by the
        context, MM_MATMUL_W_HOST) or a DevBuf."""
        dev = isinstance(w, DevBuf)
        wa = w if dev else np.ascontiguousarray(w, np.uint16)
        d_out, n_in = w.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, n_in)
        y = np.zeros((x.shape[0], d_out), np.float32) if y0 is None else \
            np.array(y0, np.float32, copy=True, order="C")
        _check(lib().mm_matmul_bf16(self.h, y.ctypes.data, x.ctypes.data,
                                    wa.ptr if dev else wa.ctypes.data, d_out, n_in, x.shape[0],
                                    flags))
        return y

    def host_weights_release(self):
        _check(lib().mm_host_weights_release(self.h))

    def matmul(self, x, w, flags=0, y0=None):
        """Mirror of the reference matmul (src/run.c:30) over the rows of x."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, np.shape(w)[1])
        w = np.ascontiguousarray(w, np.uint16)
        T, (d_out, n_in) = x.shape[0], w.shape
        dx, dw = self.to_device(x), self.to_device(w)
        dy = self.to_device(np.ascontiguousarray(y0, np.float32)) if y0 is not None else \
            self.empty((T, d_out), np.float32)
        self.matmul_dev(dy, dx, dw, d_out, n_in, T, flags)
        y = dy.download()
        for b in (dx, dw, dy):
            b.free()
            self._bufs.remove(b)
        return y

    # LM head ------------------------------------------------------------------
    def _tmp(self, bufs):
        for b in bufs:
            if b is not None:
                b.free()
                self._bufs.remove(b)

    def rmsnorm(self, x, w, eps):
        """Mirror of rmsnorm (src/run.c:22-27) over the rows of x."""
        w = np.ascontiguousarray(w, np.uint16)
        x = np.ascontiguousarray(x, np.float32).reshape(-1, w.size)
        dx, dw, dy = self.to_device(x), self.to_device(w), self.empty(x.shape, np.float32)
        _check(lib().mm_rmsnorm_dev(self.h, x.shape[0], dx.ptr, dw.ptr, w.size, float(eps), dy.ptr))
        y = dy.download()
        self._tmp((dx, dw, dy))
        return y

    def argmax(self, logits):
        """Mirror of sample (src/run.c:503-508) over the rows of logits."""
        lg = np.ascontiguousarray(logits, np.float32)
        rows = lg.reshape(-1, lg.shape[-1])
        dl, dt = self.to_device(rows), self.empty((rows.shape[0],), np.int32)
        _check(lib().mm_argmax_dev(self.h, rows.shape[0], dl.ptr, rows.shape[1], dt.ptr))
        t = dt.download()
        self._tmp((dl, dt))
        return t.reshape(lg.shape[:-1])

    def lm_head_dev(self, B, x, norm, eps, lm_head, vocab, hidden, logits, tokens):
        _check(lib().mm_lm_head_dev(self.h, B, x.ptr, norm.ptr, float(eps), lm_head.ptr, vocab,
                                    hidden, logits.ptr if logits is not None else None, tokens.ptr))

    def lm_head(self, x, norm, eps, lm_head, want_logits=True):
        """Final rmsnorm + lm_head matmul + greedy argmax for the rows of x
        (src/run.c:493-494, 503-508); returns (logits or None, tokens)."""
        lm_head = np.ascontiguousarray(lm_head, np.uint16)
        V, H = lm_head.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, H)
        B = x.shape[0]
        dx, dn, dw = self.to_device(x), self.to_device(np.ascontiguousarray(norm, np.uint16)), \
            self.to_device(lm_head)
        dl = self.empty((B, V), np.float32) if want_logits else None
        dt = self.empty((B,), np.int32)
        self.lm_head_dev(B, dx, dn, eps, dw, V, H, dl, dt)
        logits = dl.download() if dl is not None else None
        tokens = dt.download()
        self._tmp((dx, dn, dw, dl, dt))
        return logits, tokens

    # MLA absorbed decode -------------------------------------------------------
    def mla_init(self, NH, QKN=128, QKR=64, KVL=512, VHD=128, scale=None, n_layers=1):
        if scale is None:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(QKN + QKR)))
        cfg = MlaConfig(NH, QKN, QKR, KVL, VHD, scale)
        _check(lib().mm_mla_init(self.h, C.byref(cfg), n_layers))
        self._mla_cfg = cfg

    def mla_load_layer(self, layer, kv_b, flags=0):
        if flags & MM_LOAD_DEVICE_PTRS:
            _check(lib().mm_mla_load_layer(self.h, layer, kv_b.ptr, flags))
        else:
            kv_b = np.ascontiguousarray(kv_b, np.uint16)
            _check(lib().mm_mla_load_layer(self.h, layer, kv_b.ctypes.data, flags))

    def mla_absorbed_decode_dev(self, layer, B, q, cache, seq_stride, kv_len, ctx_out,
                                kv_lens=None, qabs=None, probs=None, clat=None):
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        _check(lib().mm_mla_absorbed_decode_dev(self.h, layer, B, q.ptr, cache.ptr, seq_stride,
                                                p(kv_lens), kv_len, ctx_out.ptr, p(qabs),
                                                p(probs), p(clat)))

    def mla_absorbed_decode(self, layer, q, cache, kv_len, kv_lens=None, want_probs=True):
        """Host arrays: q [B, NH, QKN+QKR] fp32, cache [B, L, KVL+QKR] bf16
        (uint16).  Returns ctx [B, NH*VHD], qabs, probs (None without
        want_probs), clat."""
        cfg = self._mla_cfg
        q = np.ascontiguousarray(q, np.float32)
        cache = np.ascontiguousarray(cache, np.uint16)
        B, L = cache.shape[0], cache.shape[1]
        NH, KVL, VHD = cfg.n_heads, cfg.kv_lora_rank, cfg.v_head_dim
        bufs = dict(q=self.to_device(q), cache=self.to_device(cache),
                    ctx=self.empty((B, NH * VHD), np.float32),
                    qabs=self.empty((B, NH, KVL), np.float32),
                    clat=self.empty((B, NH, KVL), np.float32))
        if want_probs:
            bufs["probs"] = self.empty((B, NH, kv_len), np.float32)
        if kv_lens is not None:
            bufs["lens"] = self.to_device(np.ascontiguousarray(kv_lens, np.int32))
        self.mla_absorbed_decode_dev(layer, B, bufs["q"], bufs["cache"], L, kv_len, bufs["ctx"],
                                     bufs.get("lens"), bufs["qabs"], bufs.get("probs"), bufs["clat"])
        out = tuple(bufs[k].download() if k in bufs else None for k in ("ctx", "qabs", "probs", "clat"))
        for b in bufs.values():
            b.free()
            self._bufs.remove(b)
        return out

    def mla_absorbed_decode_host(self, layer, q, cache, kv_len, kv_lens=None, want=True):
        """mm_mla_absorbed_decode: host q [B, NH, QKN+QKR] and the fp32 cache
        [B, L, KVL+QKR]; returns ctx, qabs, probs, clat (None without want)."""
        cfg = self._mla_cfg
        q = np.ascontiguousarray(q, np.float32)
        cache = np.ascontiguousarray(cache, np.float32)
        B, L = cache.shape[0], cache.shape[1]
        NH, KVL, VHD = cfg.n_heads, cfg.kv_lora_rank, cfg.v_head_dim
        ctx = np.empty((B, NH * VHD), np.float32)
        outs = [np.empty((B, NH, KVL), np.float32), np.empty((B, NH, kv_len), np.float32),
                np.empty((B, NH, KVL), np.float32)] if want else [None] * 3
        lens = np.ascontiguousarray(kv_lens, np.int32) if kv_lens is not None else None
        p = lambda a: None if a is None else a.ctypes.data  # noqa: E731
        _check(lib().mm_mla_absorbed_decode(self.h, layer, B, q.ctypes.data, cache.ctypes.data, L,
                                            p(lens), kv_len, ctx.ctypes.data, *[p(a) for a in outs]))
        return (ctx, *outs)

    # MLA decode front -----------------------------------------------------------
    def mla_front_init(self, H, inv_freq, q_lora=0, rms_eps=1e-6, mla_eps=1e-6, interleaved=0):
        inv = np.ascontiguousarray(inv_freq, np.float32)
        cfg = MlaFrontConfig(H, q_lora, rms_eps, mla_eps, interleaved,
                             inv.ctypes.data_as(C.POINTER(C.c_float)))
        _check(lib().mm_mla_front_init(self.h, C.byref(cfg)))
        self._front_cfg = (H, q_lora)

    def front_weights(self, w):
        """Upload a dict of host weights (FRONT_WEIGHTS names, or in_norm /
        kv_a for input_norm / kv_a_proj; None or absent for unused ones) and
        return (struct, buffers)."""
        alias = dict(input_norm="in_norm", kv_a_proj="kv_a")   # synth.attn_layer's names
        get = lambda k: w.get(k) if w.get(k) is not None else w.get(alias.get(k))  # noqa: E731
        bufs = {k: self.to_device(np.ascontiguousarray(get(k), np.uint16))
                for k in FRONT_WEIGHTS if get(k) is not None}
        return MlaFrontWeights(*[bufs[k].ptr if k in bufs else None for k in FRONT_WEIGHTS]), bufs

    def mla_front_dev(self, B, x, wstruct, pos, q, cache, seq_stride, kv_rows=None):
        _check(lib().mm_mla_front_dev(self.h, B, x.ptr, C.byref(wstruct), pos.ptr, q.ptr,
                                      cache.ptr, seq_stride,
                                      kv_rows.ptr if kv_rows is not None else None))

    def mla_front(self, x, w, pos, cache):
        """Host arrays: x [B, H] fp32, w a dict of bf16 weights, pos [B],
        cache [B, L, KVL+QKR] bf16 (uint16).  Returns (q [B, NH*(QKN+QKR)],
        kv_rows [B, KVL+QKR] fp32, the cache after the append)."""
        m = self._mla_cfg
        x = np.ascontiguousarray(x, np.float32)
        cache = np.ascontiguousarray(cache, np.uint16)
        B, L = cache.shape[0], cache.shape[1]
        QD = m.n_heads * (m.qk_nope_head_dim + m.qk_rope_head_dim)
        KVD = m.kv_lora_rank + m.qk_rope_head_dim
        ws, wb = self.front_weights(w)
        dx, dp, dc = self.to_device(x), self.to_device(np.ascontiguousarray(pos, np.int32)), \
            self.to_device(cache)
        dq, dk = self.empty((B, QD), np.float32), self.empty((B, KVD), np.float32)
        self.mla_front_dev(B, dx, ws, dp, dq, dc, L, dk)
        out = dq.download(), dk.download(), dc.download()
        self._tmp((dx, dp, dc, dq, dk, *wb.values()))
        return out

    def ffn_compute(self, layer, xn, flags=MM_FWD_BF16):
        """Mirror of the reference ffn_compute (src/run.c:116) for one token:
        returns out, topk_idx, topk_w and the router scores (what the
        reference leaves in s->moe_logits); the last three keep their preset
        -1 / NaN on a dense layer, which the reference does not route."""
        cfg = self._moe_cfg
        xn = np.ascontiguousarray(xn, np.float32)
        out = np.empty(cfg.hidden_size, np.float32)
        idx = np.full(cfg.n_experts_per_tok, -1, np.int32)
        w = np.full(cfg.n_experts_per_tok, np.nan, np.float32)
        p = np.full(cfg.n_routed_experts, np.nan, np.float32)
        _check(lib().mm_ffn_compute(self.h, layer, xn.ctypes.data, out.ctypes.data,
                                    idx.ctypes.data, w.ctypes.data, p.ctypes.data, flags))
        return out, idx, w, p
