"""mlamoe.engine -- the batched decode engine (mm_engine_*) from Python.

`Engine.from_host(ctx, cfg, model, inv_freq)` uploads a whole model given
as host arrays (mlamoe.synth.model's layout: DeepSeek-V2 tensor roles, bf16
as uint16), configures the context (MLA, decode front, MoE) and creates the
engine; `step` runs one decode step for B slots, `generate` the
continuous-batching greedy generation of the reference's inference()
(src/getp_run.hip:920-995).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import (FRONT_WEIGHTS, MM_FWD_BF16, MM_FWD_INT8, MM_LOAD_BF16, MM_LOAD_INT8, EngineConfig,
               EngineLayer, MlaFrontWeights, _check, lib)

_vp = C.c_void_p


class Engine:
    def __init__(self, ctx, handle, cfg, bufs):
        self.ctx, self.h, self.cfg, self._bufs = ctx, handle, cfg, bufs

    @classmethod
    def from_host(cls, ctx, c, m, inv_freq, max_batch, max_seq, int8=False, init_seq=0,
                  max_rows=0):
        """c: dict of Config fields (n_layers, first_dense, H, NH, QKN, QKR,
        KVL, VHD, dense_inter, E, n_shared, K, I, vocab, router_sigmoid,
        norm_topk, routed_scaling, rms_eps, and optionally q_lora,
        interleaved); m: synth.model(); init_seq: positions per slot the
        latent caches start with, max_rows: token rows per step (0: the
        library's defaults)."""
        L = c["n_layers"]
        ctx.mla_init(c["NH"], c["QKN"], c["QKR"], c["KVL"], c["VHD"], n_layers=L)
        ctx.mla_front_init(c["H"], inv_freq, c.get("q_lora", 0), c["rms_eps"], 1e-6,
                           c.get("interleaved", 0))
        if c["first_dense"] < L:
            ctx.moe_init(c["H"], c["E"], c["n_shared"], c["K"], c["I"], c["router_sigmoid"],
                         c["norm_topk"], c["routed_scaling"], n_layers=L)
        bufs = []

        def dev(a):
            if a is None:
                return None
            b = ctx.to_device(np.ascontiguousarray(a, np.uint16))
            bufs.append(b)
            return b.ptr
        layers = []
        for l, lw in enumerate(m["layers"]):
            ctx.mla_load_layer(l, lw["kv_b"])
            if l >= c["first_dense"]:
                ctx.moe_load_layer(l, lw, MM_LOAD_INT8 if int8 else MM_LOAD_BF16)
            alias = dict(input_norm="in_norm", kv_a_proj="kv_a")
            front = MlaFrontWeights(*[dev(lw.get(k) if lw.get(k) is not None else lw.get(alias.get(k)))
                                      for k in FRONT_WEIGHTS])
            layers.append(EngineLayer(front, dev(lw["o_proj"]), dev(lw["post_norm"]),
                                      dev(lw.get("dgate")), dev(lw.get("dup")), dev(lw.get("ddown"))))
        cfg = EngineConfig(L, c["first_dense"], c["H"], c.get("dense_inter", 8), c["vocab"],
                           c["rms_eps"], max_batch, max_seq, MM_FWD_INT8 if int8 else MM_FWD_BF16,
                           init_seq, max_rows)
        h = _vp()
        _check(lib().mm_engine_create(ctx.h, C.byref(cfg), C.byref(h)))
        eng = cls(ctx, h.value, cfg, bufs)
        for l, lw in enumerate(layers):
            _check(lib().mm_engine_set_layer(eng.h, l, C.byref(lw)))
        _check(lib().mm_engine_set_head(eng.h, dev(m["embed"]), dev(m["final_norm"]),
                                        dev(m["lm_head"])))
        return eng

    def close(self):
        if self.h:
            lib().mm_engine_destroy(self.h)
            self.h = None

    def capacity(self):
        """Positions per slot the latent caches hold now."""
        return int(lib().mm_engine_capacity(self.h))

    def reserve(self, positions):
        _check(lib().mm_engine_reserve(self.h, positions))

    def step(self, tokens, pos, want_logits=False):
        """One decode step; returns (next tokens [B], logits [B, vocab] or None)."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        B = tokens.size
        nxt = np.empty(B, np.int32)
        lg = self.ctx.empty((B, self.cfg.vocab_size), np.float32) if want_logits else None
        try:
            _check(lib().mm_engine_step(self.h, B, tokens.ctypes.data, pos.ctypes.data,
                                        nxt.ctypes.data, lg.ptr if lg is not None else None))
            return nxt, (lg.download() if lg is not None else None)
        finally:
            if lg is not None:
                self.ctx._tmp((lg,))

    def step_rows(self, slots, tokens, pos, want_rows, want_logits=False):
        """One step over token rows (slot, token, position): prompt chunks and
        decode rows together.  Returns (next tokens of want_rows, logits
        [len(want_rows), vocab] or None)."""
        slots = np.ascontiguousarray(slots, np.int32)
        tokens = np.ascontiguousarray(tokens, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        want = np.ascontiguousarray(want_rows, np.int32)
        nw = want.size
        nxt = np.empty(max(nw, 1), np.int32)
        lg = self.ctx.empty((max(nw, 1), self.cfg.vocab_size), np.float32) if want_logits else None
        try:
            _check(lib().mm_engine_step_rows(self.h, slots.size, slots.ctypes.data,
                                             tokens.ctypes.data, pos.ctypes.data, nw,
                                             want.ctypes.data if nw else None,
                                             nxt.ctypes.data if nw else None,
                                             lg.ptr if lg is not None else None))
            return nxt[:nw], (lg.download()[:nw] if lg is not None else None)
        finally:
            if lg is not None:
                self.ctx._tmp((lg,))

    def generate(self, prompts, max_steps, eos=-1):
        """Greedy continuous-batching generation; returns (list of token
        arrays, total generated)."""
        n = len(prompts)
        ps = [np.ascontiguousarray(p, np.int32) for p in prompts]
        outs = [np.zeros(max(max_steps, 1), np.int32) for _ in range(n)]
        pp = (_vp * max(n, 1))(*[p.ctypes.data for p in ps])
        op = (_vp * max(n, 1))(*[o.ctypes.data for o in outs])
        lens = np.ascontiguousarray([p.size for p in ps] or [0], np.int32)
        olens = np.zeros(max(n, 1), np.int32)
        total = lib().mm_engine_generate(self.h, n, pp, lens.ctypes.data, max_steps, eos, op,
                                         olens.ctypes.data)
        if total < 0:
            _check(int(total))
        return [outs[r][:olens[r]].copy() for r in range(n)], int(total)
