"""Batched prefill in the engine (mm_engine_step_rows): a prompt's tokens as
rows of one step, attended causally in the latent cache, and mixed with
other slots' decode rows; the reference's whole-prompt prefill is
forward_unabsorbed (src/run.c:189-370; on its GPU, gpu_forward_unabsorbed +
batched_gpu_ffn, src/getp_run.hip:394-460, 558-701).

Bars: logits at every prompt position within 2e-3 (normwise) of the
reference's forward_unabsorbed (tests/golden/prefill.npz, written by its own
dump) for bf16 experts, and of the oracle's int8-expert composition for int8
experts; prefills split into chunks, and steps mixing prefill with decode
rows, against the oracle per slot; generation with chunked prefill
checked token by token against the oracle's argmax (near-ties within 2e-3).
"""
import numpy as np
import pytest

import mlamoe
from conftest import engine_case, load_golden, max_abs_rel
from mlamoe.engine import Engine

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.mark.parametrize("name", ["dsv2", "glm"])
@pytest.mark.parametrize("int8", [False, True])
def test_prefill_whole_prompt(oracle, name, int8):
    """All 24 prompt tokens in one step, logits of every row."""
    c, m, _ = engine_case(name)
    g = load_golden("prefill.npz")
    toks, inv = g[f"{name}_tokens"], g[f"{name}_inv"]
    ref = oracle.model_logits(c, m, toks, inv, int8=True) if int8 else g[f"{name}_logits"]
    n = len(toks)
    print(f"prefill {name} int8={int8}: {n} rows in one step", flush=True)
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, inv, max_batch=2, max_seq=64, int8=int8)
        try:
            nxt, lg = eng.step_rows(np.zeros(n), toks, np.arange(n), np.arange(n), want_logits=True)
        finally:
            eng.close()
    errs = [max_abs_rel(lg[p], ref[p]) for p in range(n)]
    print(f"worst normwise logits error {max(errs):.2e}", flush=True)
    assert max(errs) < TOL
    for p in range(n):
        assert nxt[p] == lg[p].argmax()


@pytest.mark.parametrize("int8", [False, True])
def test_prefill_chunks_and_mixed_rows(oracle, int8):
    """Slot 0's 24-token prompt in chunks of 3, 9 and 12 rows; slot 1's
    prompt prefilled in the first step next to it, then decoded one row per
    step beside slot 0's chunks; slot 2 prefilled in the last step only
    (rows of three slots, different positions, in one step).  Every row's
    logits against the oracle for its own slot's sequence."""
    c, m, g = engine_case("dsv2")
    inv = g["inv"]
    rng = np.random.default_rng(31)
    s0 = rng.integers(0, c["vocab"], 24).astype(np.int32)
    s1 = rng.integers(0, c["vocab"], 6).astype(np.int32)
    s2 = rng.integers(0, c["vocab"], 5).astype(np.int32)
    refs = {s: oracle.model_logits(c, m, q, inv, int8=int8) for s, q in ((0, s0), (1, s1), (2, s2))}
    seqs = {0: s0, 1: s1, 2: s2}
    # (slot, first position, count) per step
    steps = [[(0, 0, 3), (1, 0, 4)], [(1, 4, 1), (0, 3, 9)], [(0, 12, 12), (1, 5, 1), (2, 0, 5)]]
    errs = []
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, inv, max_batch=3, max_seq=32, int8=int8)
        try:
            for st in steps:
                rows = [(s, p0 + i) for s, p0, k in st for i in range(k)]
                sl = [s for s, _ in rows]
                ps = [p for _, p in rows]
                tk = [seqs[s][p] for s, p in rows]
                print(f"step: {len(rows)} rows {st}", flush=True)
                _, lg = eng.step_rows(sl, tk, ps, np.arange(len(rows)), want_logits=True)
                for r, (s, p) in enumerate(rows):
                    errs.append(max_abs_rel(lg[r], refs[s][p]))
        finally:
            eng.close()
    print(f"worst normwise logits error {max(errs):.2e} over {len(errs)} rows", flush=True)
    assert max(errs) < TOL


def test_prefill_rejects_bad_rows():
    c, m, g = engine_case("dsv2")
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, g["inv"], max_batch=2, max_seq=16, max_rows=8)
        try:
            with pytest.raises(mlamoe.MMError, match="not above"):
                eng.step_rows([0, 0], [1, 2], [3, 3], [1])       # one cache row twice
            with pytest.raises(mlamoe.MMError, match="slot"):
                eng.step_rows([2], [1], [0], [0])                # slot past max_batch
            with pytest.raises(mlamoe.MMError, match="want_rows"):
                eng.step_rows([0, 1], [1, 2], [0, 0], [1, 0])    # not ascending
            with pytest.raises(mlamoe.MMError, match="outside"):
                eng.step_rows([0] * 9, list(range(9)), list(range(9)), [8])   # > max_rows
            nxt, _ = eng.step_rows([0, 1], [1, 2], [0, 0], [0, 1])           # still usable
            assert nxt.shape == (2,)
        finally:
            eng.close()


@pytest.mark.parametrize("max_rows", [8, 0])
def test_generate_with_chunked_prefill(oracle, max_rows):
    """7 requests through 3 slots with prompts up to 19 tokens: with 8 rows
    per step the longer prompts are prefilled over several steps beside the
    other slots' decode rows; with the default every prompt fits one step.
    Each generated token is the oracle's argmax for its prefix."""
    c, m, g = engine_case()
    inv = g["inv"]
    rng = np.random.default_rng(41)
    prompts = [rng.integers(0, c["vocab"], n).astype(np.int32) for n in (19, 1, 7, 12, 5, 9, 3)]
    max_seq, max_steps = 26, 6
    with mlamoe.Context(0) as ctx:
        eng = Engine.from_host(ctx, c, m, inv, max_batch=3, max_seq=max_seq, max_rows=max_rows)
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


def test_prefill_rows_in_attention_groups(monkeypatch):
    """120 prompt rows in one step (past the hi/lo operand rows: the
    attention's chunk partials sized per row, two 64-key chunks each), with
    the per-launch cap on the partials (MLAMOE_MLA_PART_MAX) set to 7 rows'
    worth: the front's RoPE / cache append for all rows, then the rows in
    groups of 7.  Logits bit-identical to the same step without the cap."""
    c, m, g = engine_case("dsv2")
    inv = g["inv"]
    toks = np.random.default_rng(77).integers(0, c["vocab"], 120).astype(np.int32)
    n = len(toks)
    out = []
    for cap in (None, 7 * 2 * (16 * 512 + 32) * 4):
        if cap:
            monkeypatch.setenv("MLAMOE_MLA_PART_MAX", str(cap))
        with mlamoe.Context(0) as ctx:
            eng = Engine.from_host(ctx, c, m, inv, max_batch=1, max_seq=128)
            try:
                _, lg = eng.step_rows(np.zeros(n), toks, np.arange(n), np.arange(n),
                                      want_logits=True)
            finally:
                eng.close()
        out.append(lg)
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))


@pytest.mark.parametrize("n", [42, 2048])
def test_prefill_row_groups_agree_with_rows(monkeypatch, n):
    """A step's rows attend in groups of 4 rows of one slot (the keys read
    once per group) unless MLAMOE_MLA_ROWS4=0; both forms give the same
    logits to rounding.  42 rows: 20 heads (two head groups, the second
    part empty), a last group of 2 rows, the context in chunks.  2048
    rows: 512 groups, each group's whole context in one block (no chunk
    partials, no merge), logits of a sample of rows up to the longest."""
    from mlamoe import synth
    c, _, _ = engine_case("dsv2")
    c = dict(c, NH=20 if n < 64 else 16, n_layers=2)
    m = synth.model(971, c["n_layers"], c["first_dense"], c["H"], c["NH"], c["QKN"], c["QKR"],
                    c["KVL"], c["VHD"], c["dense_inter"], c["E"], c["I"], c["n_shared"], c["vocab"])
    inv = np.array([1.0 / 10000.0 ** (2 * j / c["QKR"]) for j in range(c["QKR"] // 2)], np.float32)
    toks = np.random.default_rng(972).integers(0, c["vocab"], n).astype(np.int32)
    want = np.arange(n) if n < 64 else np.unique(np.r_[np.arange(0, n, 97), n - 5 + np.arange(5)])
    out = []
    for rows4 in ("1", "0"):
        monkeypatch.setenv("MLAMOE_MLA_ROWS4", rows4)
        print(f"row groups {rows4}: {n} rows, NH={c['NH']}", flush=True)
        with mlamoe.Context(0) as ctx:
            eng = Engine.from_host(ctx, c, m, inv, max_batch=2, max_seq=max(64, n),
                                   max_rows=n if n > 1024 else 0)
            try:
                _, lg = eng.step_rows(np.zeros(n), toks, np.arange(n), want, want_logits=True)
            finally:
                eng.close()
        out.append(lg)
    err = max(max_abs_rel(a, b) for a, b in zip(out[0], out[1]))
    print(f"worst normwise difference {err:.2e} over {len(want)} rows", flush=True)
    assert 0.0 < err < 1e-4    # the two forms sum a row's keys in different orders    # the two forms sum a row's keys in different orders
