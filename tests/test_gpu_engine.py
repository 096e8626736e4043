"""GPU checks of the batched decode engine (mm_engine_*): whole decode steps
against the reference's forward_absorbed (tests/golden/engine.npz, pinned
bit for bit by the oracle's composition), and the continuous-batching
generation against the oracle token by token.

Bars: logits normwise <= 2e-3 of the reference's (the north-star bf16 bar;
this build's latent cache is bf16 where the reference's is fp32); a
generated token is the oracle's argmax for the same prefix, or within 2e-3
(normwise) of its maximum where the two differ by a near-tie.
"""
import ctypes

import numpy as np
import pytest

import mlamoe
from conftest import engine_case, max_abs_rel
from mlamoe.engine import Engine

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.mark.parametrize("name", ["dsv2", "glm"])
@pytest.mark.parametrize("int8", [False, True])
def test_engine_teacher_forced_logits(name, int8):
    """B = 1 (GEMV projections) and B = 6 slots (MFMA GEMMs) on the same
    token sequence at once, bf16 and int8 experts (measured 2.5e-4 and
    6.7e-4 of the reference for the DeepSeek-V2 flavour); the GLM flavour
    adds q-LoRA, split-half RoPE and the sigmoid router with bias."""
    c, m, g = engine_case(name)
    toks, ref = g["tokens"], g["logits"]
    print(f"engine teacher forced {name} int8={int8}", flush=True)
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, g["inv"], max_batch=6, max_seq=32, int8=int8)
        try:
            for B in (1, 6):
                errs = []
                for p, t in enumerate(toks):
                    nxt, lg = eng.step(np.full(B, t), np.full(B, p), want_logits=True)
                    for b in range(B):
                        errs.append(max_abs_rel(lg[b], ref[p]))
                        if not int8:
                            assert lg[b][nxt[b]] >= ref[p].max() - TOL * np.abs(ref[p]).max()
                print(f"B={B} worst normwise logits error {max(errs):.2e}", flush=True)
                assert max(errs) < TOL
        finally:
            eng.close()


@pytest.mark.parametrize("name", ["dsv2", "glm"])
@pytest.mark.parametrize("int8", [False, True])
def test_engine_distinct_slots(oracle, name, int8):
    """B = 6 slots (skinny MFMA projections, MoE at T = 6), each teacher
    forced on its own token sequence and starting one step after the slot
    before it, so rows hold different tokens, positions and cache lengths in
    every step: a row or cache mix-up changes some slot's logits.  Each
    slot's logits are checked against the oracle's forward_absorbed
    composition for its own sequence (with int8 experts, the oracle's int8
    expert scheme: the int8-vs-bf16 drift is quantisation, not parity, and
    reaches ~1e-2 on some of these rows)."""
    c, m, g = engine_case(name)
    inv = g["inv"]
    B, n = 6, 9
    rng = np.random.default_rng(77)
    seqs = [rng.integers(0, c["vocab"], n).astype(np.int32) for _ in range(B)]
    refs = [oracle.model_logits(c, m, s, inv, int8=int8) for s in seqs]
    print(f"engine distinct slots {name} int8={int8}", flush=True)
    errs = []
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, inv, max_batch=B, max_seq=16, int8=int8)
        try:
            for step in range(n + B - 1):
                # slot b runs position step - b; before its start it decodes
                # token 0 at position 0 (overwritten when it starts)
                p = np.array([max(step - b, 0) for b in range(B)], np.int32)
                live = [0 <= step - b < n for b in range(B)]
                t = np.array([seqs[b][p[b]] if live[b] else 0 for b in range(B)], np.int32)
                p = np.where([step - b >= n for b in range(B)], 0, p).astype(np.int32)
                _, lg = eng.step(t, p, want_logits=True)
                for b in range(B):
                    if live[b]:
                        errs.append(max_abs_rel(lg[b], refs[b][step - b]))
        finally:
            eng.close()
    print(f"worst normwise logits error {max(errs):.2e} over {len(errs)} rows", flush=True)
    assert len(errs) == B * n and max(errs) < TOL


def test_engine_cache_grows_on_demand():
    """An engine that starts with 4 positions per slot grows its latent
    caches as the steps pass them (doubling: 4 -> 8 -> 16), keeping every
    slot's earlier rows: its logits equal, bit for bit, those of an engine
    created with the whole capacity, and both match the reference's."""
    c, m, g = engine_case()
    toks, ref = g["tokens"], g["logits"]
    B = 6
    got = {}
    for init in (4, 32):
        with mlamoe.Context(0) as ctx:
            eng = Engine.from_host(ctx, c, m, g["inv"], max_batch=B, max_seq=32, init_seq=init)
            try:
                assert eng.capacity() == init
                caps, rows = [], []
                for p, t in enumerate(toks):
                    _, lg = eng.step(np.full(B, t), np.full(B, p), want_logits=True)
                    rows.append(lg)
                    caps.append(eng.capacity())
                got[init] = np.stack(rows)
                if init == 4:
                    assert caps[3] == 4 and caps[4] == 8 and caps[8] == 16, caps
                    with pytest.raises(mlamoe.MMError, match="max_seq"):
                        eng.reserve(33)
                    assert eng.capacity() == 16
            finally:
                eng.close()
    assert np.array_equal(got[4], got[32])
    for p in range(len(toks)):
        assert max_abs_rel(got[4][p][0], ref[p]) < TOL


def test_engine_generate_five_slots(oracle):
    """9 requests of mixed prompt lengths through 5 slots: steps of 5 rows
    take the MFMA projections with every slot at its own position; each
    generated token is the oracle's argmax for its prefix (near-ties within
    2e-3 accepted)."""
    c, m, g = engine_case()
    inv = g["inv"]
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, c["vocab"], n).astype(np.int32) for n in (4, 1, 8, 2, 6, 3, 5, 7, 2)]
    max_seq, max_steps = 14, 5
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, inv, max_batch=5, max_seq=max_seq)
        try:
            outs, total = eng.generate(prompts, max_steps)
        finally:
            eng.close()
    assert total == sum(len(o) for o in outs)
    for p, o in zip(prompts, outs):
        assert len(o) == min(max_steps, max_seq - len(p))
        seq = np.concatenate([p, o])
        lg = oracle.model_logits(c, m, seq[:-1], inv)
        for k, t in enumerate(o):
            row = lg[len(p) - 1 + k]
            assert t == row.argmax() or row[t] >= row.max() - TOL * np.abs(row).max()


def test_engine_generate_continuous_batching(oracle):
    """7 requests of different prompt lengths through 3 slots: every
    generated token checked against the oracle's logits for its prefix; the
    position budget (max_seq) and max_steps limits; eos stops a request."""
    c, m, g = engine_case()
    inv = g["inv"]
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, c["vocab"], n).astype(np.int32) for n in (3, 1, 7, 2, 5, 9, 4)]
    max_seq, max_steps = 14, 6
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, inv, max_batch=3, max_seq=max_seq)
        try:
            outs, total = eng.generate(prompts, max_steps)
            assert total == sum(len(o) for o in outs)
            for p, o in zip(prompts, outs):
                assert len(o) == min(max_steps, max_seq - len(p))
                seq = np.concatenate([p, o])
                lg = oracle.model_logits(c, m, seq[:-1], inv)
                for k, t in enumerate(o):
                    row = lg[len(p) - 1 + k]
                    assert t == row.argmax() or row[t] >= row.max() - TOL * np.abs(row).max()
            # eos: stop at the first sampled eos (not stored)
            eos = int(outs[0][2])
            outs2, _ = eng.generate(prompts[:1], max_steps, eos=eos)
            assert list(outs2[0]) == list(outs[0][:2])
            # an empty prompt generates nothing
            o, t = eng.generate([np.zeros(0, np.int32), prompts[1]], 0)
            assert t == 0 and len(o[0]) == 0 and len(o[1]) == 0
        finally:
            eng.close()


def test_engine_step_errors():
    """Out-of-range batch sizes and positions are rejected before any launch."""
    c, m, g = engine_case()
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, g["inv"], max_batch=2, max_seq=8)
        try:
            with pytest.raises(mlamoe.MMError, match="outside"):
                eng.step(np.zeros(3, np.int32), np.zeros(3, np.int32))
            with pytest.raises(mlamoe.MMError, match="pos"):
                eng.step(np.zeros(1, np.int32), np.full(1, 8, np.int32))
            nxt, _ = eng.step(np.zeros(2, np.int32), np.zeros(2, np.int32))   # still usable
            assert nxt.shape == (2,)
        finally:
            eng.close()


def test_engine_errors():
    L = mlamoe.lib()
    with mlamoe.Context(0) as ctx:
        cfg = mlamoe.EngineConfig(1, 1, 256, 64, 100, 1e-6, 2, 8, 0)
        h = ctypes.c_void_p()
        assert L.mm_engine_create(ctx.h, cfg, ctypes.byref(h)) != 0
        assert b"mm_mla_init" in L.mm_last_error()
