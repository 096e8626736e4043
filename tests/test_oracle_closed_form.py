"""Closed-form and invariant checks of the CPU oracle, chosen so that a dropped
term, a transposed operand or a wrong index fails one of them.  These pin the
int8 pieces, which have no reference counterpart, and back up the golden
vectors for the reference-derived pieces."""
import numpy as np

from conftest import max_abs_rel
from mlamoe import synth


def _int_bf16(rng, shape, lim=127):
    """Integer-valued bf16 matrix (|v| <= 127 is exact in bf16)."""
    v = rng.integers(-lim, lim + 1, size=shape).astype(np.float32)
    return synth.bf16_from_f32(v), v


def test_matmul_integer_closed_form(oracle):
    # integer operands with partial sums < 2^24: fp32 accumulation is exact
    rng = np.random.default_rng(1)
    w, wf = _int_bf16(rng, (33, 512))
    x = rng.integers(-127, 128, size=512).astype(np.float32)
    exact = (wf.astype(np.int64) @ x.astype(np.int64))
    assert np.abs(exact).max() < 2 ** 24
    assert np.array_equal(oracle.matmul(x, w), exact.astype(np.float32))


def test_matmul_one_hot_and_transpose(oracle):
    rng = np.random.default_rng(2)
    x = synth.normal_f32(rng, (64,))
    w = np.zeros((5, 64), np.uint16)
    cols = [3, 0, 63, 17, 17]
    for d, c in enumerate(cols):
        w[d, c] = 0x3F80
    assert np.array_equal(oracle.matmul(x, w), x[cols])
    # non-square: row d of W is used for output d (a transposed operand fails)
    w2 = synth.normal_bf16(rng, (3, 64), 0.1)
    ref = synth.bf16_to_f32(w2).astype(np.float64) @ x.astype(np.float64)
    assert max_abs_rel(oracle.matmul(x, w2), ref) < 1e-6


def test_softmax_invariants(oracle):
    rng = np.random.default_rng(3)
    x = synth.normal_f32(rng, (64,), 2.0)
    p = oracle.softmax(x)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
    assert np.array_equal(np.argsort(-p, kind="stable"), np.argsort(-x, kind="stable"))
    e = np.exp(x.astype(np.float64) - x.max())
    assert max_abs_rel(p, e / e.sum()) < 1e-6
    m = x.copy()
    m[[1, 5]] = -np.inf
    pm = oracle.softmax(m)
    assert pm[1] == 0 and pm[5] == 0


def test_route_closed_forms(oracle):
    cfg = oracle.moe_cfg(8, 64, 0, 6, 8)
    # strictly ordered logits: top-6 are the six largest, in descending order
    rng = np.random.default_rng(4)
    lg = rng.permutation(64).astype(np.float32) * 0.1
    p, idx, w = oracle.route(cfg, lg)
    assert list(idx) == list(np.argsort(-lg)[:6])
    assert np.all(np.diff(w) <= 0) and np.array_equal(w, p[idx])
    # equal logits: lowest indices win, weights 1/64
    p, idx, w = oracle.route(cfg, np.zeros(64, np.float32))
    assert list(idx) == [0, 1, 2, 3, 4, 5] and np.all(w == np.float32(1 / 64))
    # sigmoid + bias + norm + scaling (GLM noaux_tc): select on score+bias,
    # weight = raw score normalised then scaled
    cfg2 = oracle.moe_cfg(8, 16, 0, 4, 8, 1, 1, 2.5)
    lg = synth.normal_f32(rng, (16,))
    bias = np.zeros(16, np.float32)
    bias[[2, 9]] = 10.0
    p, idx, w = oracle.route(cfg2, lg, bias)
    s = 1.0 / (1.0 + np.exp(-lg.astype(np.float64)))
    assert set(idx[:2]) == {2, 9}
    assert abs(float(w.astype(np.float64).sum()) - 2.5) < 1e-5
    assert max_abs_rel(w / 2.5, s[idx] / s[idx].sum()) < 1e-6


def test_swiglu_zero_up_gives_zero(oracle):
    rng = np.random.default_rng(5)
    H, I = 32, 16
    cfg = oracle.moe_cfg(H, 4, 0, 1, I)
    w = synth.moe_layer(5, H, 4, I, 0)
    w["eu"] = np.zeros_like(w["eu"])
    out, *_ = oracle.ffn_compute_rows(cfg, w, synth.normal_f32(rng, (2, H)))
    assert np.all(out == 0)


def test_combine_linearity(oracle):
    """out = sum_r w_r * expert_r(x) + shared(x): recompute each term with
    swiglu-by-matmul in float64 and check the weighted sum."""
    H, E, K, I, NS = 48, 6, 2, 20, 1
    w = synth.moe_layer(6, H, E, I, NS)
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    x = synth.activations(7, 1, H)
    out, idx, wt, _ = oracle.ffn_compute_rows(cfg, w, x)
    f = synth.bf16_to_f32
    xd = x[0].astype(np.float64)

    def mlp(g, u, d):
        a = f(g).astype(np.float64) @ xd
        b = f(u).astype(np.float64) @ xd
        return f(d).astype(np.float64) @ (a / (1 + np.exp(-a)) * b)
    ref = sum(float(wt[0, r]) * mlp(w["eg"][idx[0, r]], w["eu"][idx[0, r]], w["ed"][idx[0, r]])
              for r in range(K)) + mlp(w["sg"], w["su"], w["sd"])
    assert max_abs_rel(out[0], ref) < 1e-5


def test_quant_row_closed_form(oracle):
    rng = np.random.default_rng(8)
    x = synth.normal_f32(rng, (5, 300))
    q, s = oracle.quant_rows(x)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(s, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q) <= 127) and np.all(np.abs(q).max(axis=1) == 127)
    # round-to-nearest: dequantisation error at most half a step
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-6))
    # a zero row quantises to zeros with scale 0
    q0, s0 = oracle.quant_rows(np.zeros((1, 16), np.float32))
    assert s0[0] == 0 and np.all(q0 == 0)
    # exactly representable rows survive unchanged: x = k * 2^-3, max |k| = 127
    k = rng.integers(-127, 128, size=64)
    k[0] = 127
    q1, s1 = oracle.quant_rows((k * 0.125).astype(np.float32)[None])
    assert s1[0] == np.float32(0.125) and np.array_equal(q1[0], k)


def test_gemm_i8_exact(oracle):
    rng = np.random.default_rng(9)
    for M, N, K in ((1, 7, 64), (19, 33, 2048), (4, 2048, 1408)):
        a = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
        b = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
        c = oracle.gemm_i8(a, b)
        assert np.array_equal(c, a.astype(np.int64) @ b.astype(np.int64).T)
    # extreme operands: all -127 * -127 over K=2048 is the largest magnitude
    a = np.full((1, 2048), -127, np.int8)
    assert oracle.gemm_i8(a, a)[0, 0] == 2048 * 127 * 127
    # the reference matmul on integer-valued operands gives the same numbers
    a = rng.integers(-127, 128, size=(1, 512)).astype(np.int8)
    b = rng.integers(-127, 128, size=(9, 512)).astype(np.int8)
    wb = synth.bf16_from_f32(b.astype(np.float32))
    assert np.array_equal(oracle.matmul(a[0].astype(np.float32), wb),
                          oracle.gemm_i8(a, b)[0].astype(np.float32))


def test_ffn_i8_reduces_to_reference(oracle):
    """With operands that int8 represents exactly (x integer with max |x| = 127,
    weights k/128 with max |k| = 127 per row) the int8 gate/up stage equals the
    reference matmul bit for bit, the quantised hidden row equals quantising
    the reference SwiGLU hidden, and the final output matches the reference
    matmul on the dequantised operands."""
    H, E, K, I, NS, T = 64, 4, 2, 32, 1, 3
    rng = np.random.default_rng(10)
    S = NS * I

    def wmat(shape):
        k = rng.integers(-127, 128, size=shape)
        k[..., 0] = 127
        return synth.bf16_from_f32((k / 128.0).astype(np.float32))
    w = dict(moe_gate=synth.normal_bf16(rng, (E, H), 0.05), moe_gate_bias=None,
             eg=wmat((E, I, H)), eu=wmat((E, I, H)), ed=wmat((E, H, I)),
             sg=wmat((S, H)), su=wmat((S, H)), sd=wmat((H, S)))
    x = rng.integers(-127, 128, size=(T, H)).astype(np.float32)
    x[:, 0] = 127
    cfg = oracle.moe_cfg(H, E, NS, K, I)
    qw = oracle.quantize_moe_weights(w)
    assert np.all(qw["seg"] == np.float32(1 / 128))
    out, idx, wt, probs, d = oracle.ffn_i8(cfg, w, qw, x, debug=True)
    ro, ri, rw, rp = oracle.ffn_compute_rows(cfg, w, x)
    assert np.array_equal(idx, ri) and np.array_equal(wt, rw)
    assert np.array_equal(d["qx"], x.astype(np.int8)) and np.all(d["sx"] == 1.0)
    f = synth.bf16_to_f32
    for t in range(T):
        for r in range(K):
            e = idx[t, r]
            g = oracle.matmul(x[t], w["eg"][e])
            u = oracle.matmul(x[t], w["eu"][e])
            acc = d["acc_gu"][t, r]
            assert np.array_equal(acc[0].astype(np.float32) * np.float32(1 / 128), g)
            assert np.array_equal(acc[1].astype(np.float32) * np.float32(1 / 128), u)
            L = oracle.lib()
            h = np.array([L.or_silu(float(a)) for a in g], np.float32) * u
            qh, sh = oracle.quant_rows(h[None])
            assert np.array_equal(d["qh"][t, r], qh[0]) and d["sh"][t, r] == sh[0]
            assert np.array_equal(d["acc_d"][t, r],
                                  qh[0].astype(np.int64) @ qw["qed"][e].astype(np.int64).T)
            y = oracle.matmul(qh[0].astype(np.float32) * sh[0], w["ed"][e])
            yq = (d["acc_d"][t, r].astype(np.float32) * sh[0]) * qw["sed"][e]
            assert max_abs_rel(yq, y) < 1e-5
    # whole-layer drift against the bf16 reference stays small on this input
    assert max_abs_rel(out, ro) < 2e-2


def _absorbed_f64(q, kv_b, cache, NH, QKN, QKR, KVL, VHD, scale):
    """Unabsorbed MLA in float64 (per-head K/V materialised, the
    forward_unabsorbed formulation, run.c:248-287), which the absorbed chain
    equals algebraically."""
    f = synth.bf16_to_f32(kv_b).astype(np.float64).reshape(NH, QKN + VHD, KVL)
    ckv, kpe = cache[:, :KVL].astype(np.float64), cache[:, KVL:].astype(np.float64)
    out = []
    for h in range(NH):
        k_nope = ckv @ f[h, :QKN].T
        v = ckv @ f[h, QKN:].T
        s = (k_nope @ q[h, :QKN] + kpe @ q[h, QKN:]) * scale
        a = np.exp(s - s.max())
        a /= a.sum()
        out.append(a @ v)
    return np.concatenate(out)


def test_absorbed_equals_unabsorbed(oracle):
    NH, QKN, QKR, KVL, VHD, L = 3, 16, 8, 32, 12, 9
    rng = np.random.default_rng(12)
    kv_b = synth.normal_bf16(rng, (NH * (QKN + VHD), KVL), 0.1)
    q = synth.normal_f32(rng, (1, NH, QKN + QKR))
    cache = synth.normal_f32(rng, (1, L, KVL + QKR))
    scale = float(np.float32(1) / np.sqrt(np.float32(QKN + QKR)))
    ctx, *_ = oracle.absorbed_decode(q, kv_b, cache, L, NH, QKN, QKR, KVL, VHD)
    ref = _absorbed_f64(q[0].astype(np.float64), kv_b, cache[0], NH, QKN, QKR, KVL, VHD, scale)
    assert max_abs_rel(ctx[0], ref) < 1e-5


def test_absorbed_closed_forms(oracle):
    NH, QKN, QKR, KVL, VHD = 2, 8, 4, 16, 8
    rng = np.random.default_rng(13)
    kv_b = synth.normal_bf16(rng, (NH * (QKN + VHD), KVL), 0.1)
    cache = synth.normal_bf16(rng, (1, 8, KVL + QKR), 1.0)       # bf16 cache
    cf = synth.bf16_to_f32(cache)
    # kv_len == 1: softmax is exactly 1 and the latent context is row 0
    q = synth.normal_f32(rng, (1, NH, QKN + QKR))
    ctx, qabs, probs, clat = oracle.absorbed_decode(q, kv_b, cache, 1, NH, QKN, QKR, KVL, VHD)
    assert np.all(probs == 1.0)
    assert np.array_equal(clat[0], np.stack([cf[0, 0, :KVL]] * NH))
    # q == 0: uniform weights (kv_len = 8 is a power of two, so 1/8 is exact)
    z = np.zeros_like(q)
    ctx, qabs, probs, clat = oracle.absorbed_decode(z, kv_b, cache, 8, NH, QKN, QKR, KVL, VHD)
    assert np.all(qabs == 0) and np.all(probs == np.float32(0.125))
    assert max_abs_rel(clat[0, 0], cf[0, :, :KVL].astype(np.float64).mean(axis=0)) < 1e-6
    # fp32 and bf16 caches holding the same values agree exactly
    c2, *_ = oracle.absorbed_decode(q, kv_b, cf.astype(np.float32), 8, NH, QKN, QKR, KVL, VHD)
    c3, *_ = oracle.absorbed_decode(q, kv_b, cache, 8, NH, QKN, QKR, KVL, VHD)
    assert np.array_equal(c2, c3)


def test_rmsnorm_closed_form(oracle):
    # constant x = c with unit weights: ss = n c^2 exactly (small integers), so
    # y = c * (1 / sqrt(c^2 + eps)) with every fp32 step correctly rounded
    for c, n, eps in ((2.0, 64, 1e-6), (-3.0, 2048, 1e-5), (0.5, 8, 0.0)):
        x = np.full(n, c, np.float32)
        w = synth.bf16_from_f32(np.ones(n, np.float32))
        ss = np.float32(c * c * n)
        inv = np.float32(1.0) / np.sqrt(ss / np.float32(n) + np.float32(eps))
        assert np.array_equal(oracle.rmsnorm(x, w, eps), np.full(n, np.float32(c) * inv))
    # the weight multiplies last: w = 2^k scales the output exactly
    rng = np.random.default_rng(3)
    x = synth.normal_f32(rng, (256,))
    one = synth.bf16_from_f32(np.ones(256, np.float32))
    four = synth.bf16_from_f32(np.full(256, 4.0, np.float32))
    assert np.array_equal(oracle.rmsnorm(x, four, 1e-6), 4.0 * oracle.rmsnorm(x, one, 1e-6))
    # scale invariance up to eps: rmsnorm(k x) ~ rmsnorm(x)
    assert max_abs_rel(oracle.rmsnorm(8.0 * x, one, 0.0), oracle.rmsnorm(x, one, 0.0)) < 1e-6


def test_argmax_tie_and_nan_rules(oracle):
    rng = np.random.default_rng(4)
    v = synth.normal_f32(rng, (513,))
    assert oracle.argmax(v) == int(np.argmax(v))              # first maximum
    assert oracle.argmax(np.arange(10, dtype=np.float32)) == 9
    t = np.zeros(9, np.float32)
    t[[2, 6]] = 5.0
    assert oracle.argmax(t) == 2                               # lowest index on a tie
    n = v.copy()
    n[0] = np.nan
    assert oracle.argmax(n) == 0                               # NaN at 0 is never beaten
    m = v.copy()
    m[int(np.argmax(v))] = np.nan
    assert oracle.argmax(m) == int(np.nanargmax(m))            # other NaNs never win
    assert oracle.argmax(np.full(5, -np.inf, np.float32)) == 0


def test_rope_closed_forms(oracle):
    """RoPE (run.c:47-67): position 0 is the identity; each rotated pair keeps
    its length; rotating by -p undoes p; the split-half layout holds exactly
    the adjacent layout's values, evens first (a dropped sign, a swapped
    sin/cos or a wrong output index fails one of these)."""
    rng = np.random.default_rng(3)
    inv = oracle.rope_inv_freq(64, 10000.0)
    v = synth.normal_f32(rng, (5, 64))
    for il in (0, 1):
        assert np.array_equal(oracle.rope_apply(v, 0, inv, il), v if il == 0 else
                              np.concatenate([v[:, 0::2], v[:, 1::2]], axis=1))
    for pos in (1, 17, 3000):
        a = oracle.rope_apply(v, pos, inv, 0)
        n0 = np.hypot(v[:, 0::2], v[:, 1::2])
        assert np.allclose(np.hypot(a[:, 0::2], a[:, 1::2]), n0, rtol=1e-6, atol=0)
        assert np.allclose(oracle.rope_apply(a, -pos, inv, 0), v, rtol=0, atol=2e-6)
        b = oracle.rope_apply(v, pos, inv, 1)
        assert np.array_equal(b, np.concatenate([a[:, 0::2], a[:, 1::2]], axis=1))
        # pair j rotates by pos * inv[j]: compare with a float64 rotation
        ang = (np.float32(pos) * inv).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        e = v[:, 0::2].astype(np.float64) * c - v[:, 1::2] * s
        o = v[:, 0::2].astype(np.float64) * s + v[:, 1::2] * c
        assert np.allclose(a[:, 0::2], e, rtol=0, atol=1e-6)
        assert np.allclose(a[:, 1::2], o, rtol=0, atol=1e-6)


def test_rope_inv_freq_closed_forms(oracle):
    """YaRN blend (model_load.c:299-325): factor 1 is plain RoPE (1 / theta^(2j/d));
    below the correction range the table is the extrapolated frequency, above
    it the interpolated one (that / factor), strictly between them inside."""
    plain = oracle.rope_inv_freq(64, 10000.0, 1.0)
    j = np.arange(32)
    assert np.allclose(plain, 1.0 / 10000.0 ** (2.0 * j / 64), rtol=2e-7, atol=0)
    y = oracle.rope_inv_freq(64, 10000.0, 40.0, 32.0, 1.0, 4096.0)
    lo = np.floor(64 * np.log(4096 / (32 * 2 * np.pi)) / (2 * np.log(10000.0)))
    hi = np.ceil(64 * np.log(4096 / (1 * 2 * np.pi)) / (2 * np.log(10000.0)))
    assert 0 < lo < hi < 31
    assert np.array_equal(y[j <= lo], plain[j <= lo])
    assert np.array_equal(y[j >= hi], (plain / np.float32(40.0))[j >= hi])
    mid = (j > lo) & (j < hi)
    assert np.all(y[mid] < plain[mid]) and np.all(y[mid] > plain[mid] / 40.0)
