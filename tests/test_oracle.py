"""Pins the CPU oracle (oracle/ember_oracle.c) before anything is checked
against it.  CPU only.

What pins what:
* closed forms (tests/closed_forms.py)  <- central finite differences and
  textbook special cases (uniform attention, V = 1, one-hot scores);
* oracle attention fwd/bwd              <- golden fixtures from the closed
  forms, the reference's own CPU ops composed the way Ember composes
  attention today (oracle/_ref, when built), mask invariants;
* oracle matmul                         <- the reference's compiled
  operators_cpu.c matmul, bit for bit, on the reference's own test shapes.
Planted-mistake tests show each pin fails for a plausible bug.
"""

import math

import numpy as np
import pytest

import closed_forms
import oracle

TOL = dict(rtol=1e-5, atol=2e-6)


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


# ------------------------------------------------------------ closed forms


@pytest.mark.parametrize("causal", [False, True])
def test_closed_form_gradients_match_finite_differences(causal):
    q, k, v, d_o = (_rand((1, 1, 5, 3), s) for s in (1, 2, 3, 4))
    scale = 0.7
    fd = closed_forms.finite_difference_grads(q, k, v, d_o, causal, scale)
    cf = closed_forms.bwd(q, k, v, d_o, causal, scale)
    for a, b in zip(cf, fd):
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def test_closed_form_special_cases():
    S, D = 9, 4
    v = _rand((1, 1, S, D), 5)
    q = _rand((1, 1, S, D), 6)
    zeros = np.zeros_like(q)
    # K = 0: uniform attention.  Causal row i averages V[0..i]; LSE = ln(i+1).
    o, lse = closed_forms.fwd(q, zeros, v, True, 1.0)
    cum = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    np.testing.assert_allclose(o[0, 0], cum, rtol=1e-12)
    np.testing.assert_allclose(lse[0, 0], np.log(np.arange(1, S + 1)), rtol=1e-12)
    o, lse = closed_forms.fwd(q, zeros, v, False, 1.0)
    np.testing.assert_allclose(o[0, 0], np.broadcast_to(v[0, 0].astype(np.float64).mean(0), (S, D)), rtol=1e-12)
    np.testing.assert_allclose(lse[0, 0], np.full(S, math.log(S)), rtol=1e-12)
    # V = 1 => O = 1.
    o, _ = closed_forms.fwd(q, _rand((1, 1, S, D), 7), np.ones_like(v), False, 1.0)
    np.testing.assert_allclose(o, 1.0, rtol=1e-12)
    # One dominant score per row => O_i ~ v_j.
    k = np.zeros((1, 1, S, D), dtype=np.float32)
    qd = np.zeros_like(k)
    qd[0, 0, :, 0] = 1.0
    k[0, 0, 3, 0] = 100.0
    o, _ = closed_forms.fwd(qd, k, v, False, 1.0)
    np.testing.assert_allclose(o[0, 0], np.broadcast_to(v[0, 0, 3], (S, D)), atol=1e-30)


# ------------------------------------------------------------- golden pins


def test_golden_fixtures_cover_the_tile_edges(golden):
    seqs = {c["q"].shape[2] for c in golden.values()}
    assert {1, 2, 17, 33, 64, 65, 130} <= seqs
    assert {bool(c["causal"]) for c in golden.values()} == {False, True}


def test_oracle_forward_matches_golden(golden):
    for name, c in golden.items():
        o, lse = oracle.attention_fwd(c["q"], c["k"], c["v"], bool(c["causal"]), float(c["scale"]))
        np.testing.assert_allclose(o, c["o"], err_msg=name, **TOL)
        np.testing.assert_allclose(lse, c["lse"], err_msg=name, **TOL)


def test_oracle_backward_matches_golden(golden):
    for name, c in golden.items():
        causal, scale = bool(c["causal"]), float(c["scale"])
        o, lse = oracle.attention_fwd(c["q"], c["k"], c["v"], causal, scale)
        dq, dk, dv = oracle.attention_bwd(c["q"], c["k"], c["v"], o, lse, c["do"], causal, scale)
        for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            np.testing.assert_allclose(got, c[key], err_msg=f"{name}/{key}", rtol=1e-5, atol=1e-5)


def test_planted_mistakes_fail_the_golden_pin(golden):
    """A flipped mask, a wrong scale or a transposed operand must not pass."""
    c = golden["s65_d64_c"]
    q, k, v = c["q"], c["k"], c["v"]
    scale = float(c["scale"])
    for bad in (
        lambda: oracle.attention_fwd(q, k, v, False, scale),                    # mask dropped
        lambda: oracle.attention_fwd(q, k, v, True, scale * 1.01),              # scale off
        lambda: oracle.attention_fwd(k, q, v, True, scale),                     # q <-> k
        lambda: oracle.attention_fwd(q, k, v[:, :, ::-1].copy(), True, scale),  # v rows reversed
    ):
        o, _ = bad()
        assert not np.allclose(o, c["o"], **TOL)


# ------------------------------------- the reference's own ops, composed


needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


@needs_ref
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S,D", [(48, 16), (65, 32)])
def test_oracle_matches_reference_composed_ops(S, D, causal):
    q, k, v, d_o = (_rand((1, 1, S, D), s) for s in (21, 22, 23, 24))
    scale = oracle.default_scale(D)
    o_ref, dq_ref, dk_ref, dv_ref = oracle.ref_composed_attention_head(
        q[0, 0], k[0, 0], v[0, 0], d_o[0, 0], causal, scale, backward=True)
    o, lse = oracle.attention_fwd(q, k, v, causal, scale)
    np.testing.assert_allclose(o[0, 0], o_ref, rtol=1e-5, atol=1e-6)
    dq, dk, dv = oracle.attention_bwd(q, k, v, o, lse, d_o, causal, scale)
    np.testing.assert_allclose(dq[0, 0], dq_ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dk[0, 0], dk_ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dv[0, 0], dv_ref, rtol=1e-4, atol=1e-5)


@needs_ref
@pytest.mark.parametrize(
    "n,k,m", [(4, 5, 3), (1, 1, 1), (32, 128, 64), (64, 32, 128), (16, 50, 50), (33, 17, 65)]
)
def test_oracle_matmul_is_bitwise_the_reference(n, k, m):
    """Shapes from the reference's test_tensor.py:125-145 and test_linear.py:12-17."""
    a = _rand((n, k), 31)
    b = _rand((k, m), 32)
    ref = np.empty((n, m), dtype=np.float32)
    oracle.ref_lib().matmul(a, b, ref, n, m, k)
    assert np.array_equal(oracle.matmul(a, b), ref)
    assert np.array_equal(oracle.matmul(a, b, threads=True), ref)


@needs_ref
def test_oracle_batched_and_transpose_match_reference():
    a = _rand((3, 5, 6), 33)
    b = _rand((3, 6, 4), 34)
    ref = np.empty((3, 5, 4), dtype=np.float32)
    oracle.ref_lib().matmul_batched(a, b, ref, 3, 5, 4, 6)
    got = np.empty_like(ref)
    oracle.lib().oracle_matmul_batched(a, b, got, 3, 5, 4, 6)
    assert np.array_equal(got, ref)
    t_ref = np.empty((6, 5), dtype=np.float32)
    oracle.ref_lib().transpose(np.ascontiguousarray(a[0]), t_ref, 5, 6)
    t = np.empty_like(t_ref)
    oracle.lib().oracle_transpose(np.ascontiguousarray(a[0]), t, 5, 6)
    assert np.array_equal(t, t_ref)


def test_oracle_matmul_against_float64():
    a = _rand((40, 300), 35)
    b = _rand((300, 20), 36)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    # FP64 accumulation: one rounding of (nearly) the exact value.
    np.testing.assert_allclose(oracle.matmul(a, b), exact.astype(np.float32), rtol=2e-7, atol=1e-12)


# ------------------------------------------------------- mask invariants


def test_oracle_mask_invariants_are_bitwise():
    S, D = 40, 16
    q, k, v = (_rand((1, 1, S, D), s) for s in (41, 42, 43))
    o, lse = oracle.attention_fwd(q, k, v, True)
    i = 17
    k2, v2 = k.copy(), v.copy()
    k2[0, 0, i + 1:] += 3.0
    v2[0, 0, i + 1:] -= 5.0
    o2, lse2 = oracle.attention_fwd(q, k2, v2, True)
    assert np.array_equal(o[0, 0, : i + 1], o2[0, 0, : i + 1])
    assert np.array_equal(lse[0, 0, : i + 1], lse2[0, 0, : i + 1])
    assert np.array_equal(o[0, 0, 0], v[0, 0, 0])  # row 0 sees key 0 only
    assert lse[0, 0, 0] == np.float32(oracle.default_scale(D) * float(np.dot(
        q[0, 0, 0].astype(np.float64), k[0, 0, 0].astype(np.float64))))


def test_oracle_backward_invariants():
    S, D = 24, 8
    q, k, v, d_o = (_rand((1, 1, S, D), s) for s in (51, 52, 53, 54))
    o, lse = oracle.attention_fwd(q, k, v, True)
    dq, dk, dv = oracle.attention_bwd(q, k, v, o, lse, np.zeros_like(d_o), True)
    assert not dq.any() and not dk.any() and not dv.any()
    dq, dk, dv = oracle.attention_bwd(q, k, v, o, lse, d_o, True)
    # The last key is seen only by the last query, with weight P[S-1][S-1].
    s_last = oracle.default_scale(D) * np.dot(q[0, 0, -1].astype(np.float64), k[0, 0, -1])
    p = math.exp(s_last - float(lse[0, 0, -1]))
    np.testing.assert_allclose(dv[0, 0, -1], p * d_o[0, 0, -1].astype(np.float64), rtol=1e-6)


def test_oracle_strided_layout_matches_contiguous():
    B, H, S, D = 2, 3, 19, 8
    qkv = _rand((B, S, 3, H, D), 61)
    q = np.ascontiguousarray(qkv[:, :, 0].transpose(0, 2, 1, 3))
    k = np.ascontiguousarray(qkv[:, :, 1].transpose(0, 2, 1, 3))
    v = np.ascontiguousarray(qkv[:, :, 2].transpose(0, 2, 1, 3))
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, True)
    o = np.zeros((B, S, H, D), dtype=np.float32)
    lse = np.zeros((B, H, S), dtype=np.float32)
    flat = np.ascontiguousarray(qkv).reshape(-1)
    L = oracle.lib()
    scale = oracle.default_scale(D)
    in_st = (S * 3 * H * D, D, 3 * H * D)
    out_st = (S * H * D, D, H * D)
    rc = L.oracle_attention_fwd(flat, np.ascontiguousarray(flat[H * D:]),
                                np.ascontiguousarray(flat[2 * H * D:]), o.reshape(-1), lse,
                                B, H, S, D, scale, 1, *in_st, *out_st)
    assert rc == 0
    assert np.array_equal(o.transpose(0, 2, 1, 3), o_ref)
    assert np.array_equal(lse, lse_ref)


# ------------------------------------------------------------------- Adam


def _adam_state(n, seed):
    rng = np.random.default_rng(seed)
    p = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    m = (0.1 * rng.standard_normal(n)).astype(np.float32)
    v = np.abs(0.01 * rng.standard_normal(n)).astype(np.float32)
    return p, g, m, v


@needs_ref
@pytest.mark.parametrize("hp", [(1e-3, 0.9, 0.999, 1e-8), (0.01, 0.8, 0.99, 1e-6), (0.1, 0.5, 0.9, 1e-3)])
@pytest.mark.parametrize("t", [1, 2, 17])
def test_oracle_adam_is_bitwise_the_reference_composition(hp, t):
    """oracle_adam_step == adam.py's 14 element-wise ops run through the
    reference's own compiled operators_cpu.c, bit for bit."""
    lr, b1, b2, eps = hp
    p, g, m, v = _adam_state(1000, t)
    rp, rm, rv = oracle.ref_composed_adam_step(p, g, m, v, lr, b1, b2, eps, t)
    oracle.adam_step(p, g, m, v, lr, b1, b2, eps, t)
    assert np.array_equal(p, rp) and np.array_equal(m, rm) and np.array_equal(v, rv)


def test_oracle_adam_matches_the_textbook_formula():
    """The reference's own test formula (tests/optim/test_adam.py:9-20), float64."""
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-8
    p, g, m, v = _adam_state(500, 3)
    P, G, M, V = (x.astype(np.float64) for x in (p, g, m, v))
    for t in (1, 2, 3):
        M = b1 * M + (1 - b1) * G
        V = b2 * V + (1 - b2) * G * G
        P = P - lr * (M / (1 - b1 ** t)) / (np.sqrt(V / (1 - b2 ** t)) + eps)
        oracle.adam_step(p, g, m, v, lr, b1, b2, eps, t)
    # fp32 against float64: rtol as the reference's test, plus a small atol
    # for entries that cancel to near zero.
    np.testing.assert_allclose(p, P, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(m, M, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(v, V, rtol=1e-5, atol=1e-9)


def test_oracle_adam_planted_mistakes_fail():
    """Swapping the betas or dropping the bias correction must not pass."""
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-8
    base = _adam_state(200, 4)
    good = [x.copy() for x in base]
    oracle.adam_step(*good, lr, b1, b2, eps, 1)
    bad = [x.copy() for x in base]
    oracle.adam_step(*bad, lr, b2, b1, eps, 1)
    assert not np.allclose(bad[0], good[0], rtol=1e-6)
    bad = [x.copy() for x in base]
    oracle.adam_step(*bad, lr, b1, b2, eps, 1000)   # bias corrections ~1
    assert not np.allclose(bad[0], good[0], rtol=1e-6)


# ------------------------------------------------------------ AdamW, SGD


@needs_ref
@pytest.mark.parametrize("hp", [(1e-3, 0.9, 0.999, 1e-8, 0.01), (0.01, 0.8, 0.99, 1e-6, 0.1),
                                (0.1, 0.5, 0.9, 1e-3, 0.5), (0.01, 0.9, 0.999, 1e-8, 0.0)])
@pytest.mark.parametrize("t", [1, 2, 17])
def test_oracle_adamw_is_bitwise_the_reference_composition(hp, t):
    """oracle_adamw_step == adamw.py's element-wise ops (:45-56) run through
    the reference's own compiled operators_cpu.c, bit for bit."""
    lr, b1, b2, eps, wd = hp
    p, g, m, v = _adam_state(1000, t)
    rp, rm, rv = oracle.ref_composed_adamw_step(p, g, m, v, lr, b1, b2, eps, wd, t)
    oracle.adamw_step(p, g, m, v, lr, b1, b2, eps, wd, t)
    assert np.array_equal(p, rp) and np.array_equal(m, rm) and np.array_equal(v, rv)


def test_oracle_adamw_special_cases():
    """weight_decay = 0 is Adam bit for bit (p - p*0 == p); with g = m = v = 0
    the Adam term is exactly 0 and p becomes p - p*fp32(lr*wd), the
    reference's test_weight_decay_shrinks_params_without_grad in closed form."""
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-8
    base = _adam_state(300, 5)
    a, w = [x.copy() for x in base], [x.copy() for x in base]
    oracle.adam_step(*a, lr, b1, b2, eps, 3)
    oracle.adamw_step(*w, lr, b1, b2, eps, 0.0, 3)
    assert all(np.array_equal(x, y) for x, y in zip(a, w))
    p = base[0].copy()
    z = np.zeros_like(p)
    m, v = z.copy(), z.copy()
    oracle.adamw_step(p, z.copy(), m, v, 0.1, b1, b2, eps, 0.5, 1)
    p0 = base[0]
    assert np.array_equal(p, p0 - p0 * np.float32(0.1 * 0.5))
    assert np.all(np.abs(p) < np.abs(p0) + (p0 == 0))


def test_oracle_adamw_matches_the_textbook_formula():
    """The reference's own test formula (tests/optim/test_adamw.py:9-17),
    float64, three steps."""
    lr, b1, b2, eps, wd = 0.01, 0.9, 0.999, 1e-8, 0.1
    p, g, m, v = _adam_state(500, 6)
    P, G, M, V = (x.astype(np.float64) for x in (p, g, m, v))
    for t in (1, 2, 3):
        M = b1 * M + (1 - b1) * G
        V = b2 * V + (1 - b2) * G * G
        P = P - lr * wd * P
        P = P - lr * (M / (1 - b1 ** t)) / (np.sqrt(V / (1 - b2 ** t)) + eps)
        oracle.adamw_step(p, g, m, v, lr, b1, b2, eps, wd, t)
    np.testing.assert_allclose(p, P, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(m, M, rtol=1e-5, atol=1e-7)


@needs_ref
def test_oracle_adamw_planted_mistakes_fail():
    """Decay applied after the Adam step instead of before, or dropped, must
    not pass the bitwise comparison with the reference's composition."""
    lr, b1, b2, eps, wd = 0.1, 0.9, 0.999, 1e-8, 0.5
    base = _adam_state(400, 7)
    rp, _, _ = oracle.ref_composed_adamw_step(*base, lr, b1, b2, eps, wd, 1)
    adam = [x.copy() for x in base]
    oracle.adam_step(*adam, lr, b1, b2, eps, 1)                  # no decay
    assert not np.array_equal(adam[0], rp)
    late = adam[0] - adam[0] * np.float32(lr * wd)                # decay after the step
    assert not np.array_equal(late, rp)


@needs_ref
@pytest.mark.parametrize("lr,momentum", [(0.1, 0.0), (0.01, 0.9), (0.5, 0.99)])
def test_oracle_sgd_is_bitwise_the_reference_composition(lr, momentum):
    """oracle_sgd_step == sgd.py:33-35 run through the reference's compiled
    operators, over three steps."""
    p, g, _, v = _adam_state(1000, 8)
    rp, rv = p.copy(), v.copy()
    for _ in range(3):
        rp, rv = oracle.ref_composed_sgd_step(rp, g, rv, lr, momentum)
        oracle.sgd_step(p, g, v, lr, momentum)
        assert np.array_equal(p, rp) and np.array_equal(v, rv)


def test_oracle_sgd_closed_forms_and_planted_mistake():
    """momentum 0: p - g*lr exactly and v = g; the reference's test formula
    (tests/optim/test_sgd.py:9-12) in float64; swapping lr and momentum fails."""
    p, g, _, _ = _adam_state(400, 9)
    v = np.zeros_like(p)
    q = p.copy()
    oracle.sgd_step(q, g, v, 0.1, 0.0)
    assert np.array_equal(q, p - g * np.float32(0.1)) and np.array_equal(v, g)
    P, V = p.astype(np.float64), np.zeros(p.size)
    q, v = p.copy(), np.zeros_like(p)
    for _ in range(3):
        V = 0.9 * V + g
        P = P - 0.05 * V
        oracle.sgd_step(q, g, v, 0.05, 0.9)
    np.testing.assert_allclose(q, P, rtol=1e-5, atol=1e-6)
    bad, bv = p.copy(), np.zeros_like(p)
    for _ in range(3):
        oracle.sgd_step(bad, g, bv, 0.9, 0.05)
    assert not np.allclose(bad, P, rtol=1e-3)


# ------------------------------------------------------ LayerNorm and GELU


@needs_ref
def test_oracle_gelu_is_bitwise_the_reference_composition():
    x, dy = _rand((3000,), 71), _rand((3000,), 72)
    y_ref, dx_ref = oracle.ref_composed_gelu(x, dy)
    y = oracle.gelu_fwd(x)
    assert np.array_equal(y, y_ref)
    assert np.array_equal(oracle.gelu_bwd(dy, x, y), dx_ref)


def test_gelu_backward_formula_is_the_derivative():
    """Ember's backward formula (activations.py:65-66) equals d/dx of its
    forward, by central differences in float64."""
    x = np.linspace(-4, 4, 81)
    f = lambda z: 0.5 * z * (1 + np.tanh(0.8 * z))  # noqa: E731
    h = 1e-6
    fd = (f(x + h) - f(x - h)) / (2 * h)
    y = f(x)
    np.testing.assert_allclose((1 + np.tanh(0.8 * x)) * (0.5 + 0.8 * (x - y)), fd, rtol=1e-7, atol=1e-9)
    np.testing.assert_allclose(oracle.gelu_bwd(np.ones(81), x, oracle.gelu_fwd(x)), fd, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,d", [(1, 4), (7, 64), (33, 1024), (3, 4096)])
def test_oracle_layernorm_forward_closed_form(rows, d):
    x = _rand((rows, d), 73) * 3 + 1
    g, b = _rand((d,), 74), _rand((d,), 75)
    y, mean, rstd = oracle.layernorm_fwd(x, g, b, 1e-5)
    np.testing.assert_allclose(y, closed_forms.layernorm(x, g, b, 1e-5), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mean, x.astype(np.float64).mean(-1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(rstd, 1 / np.sqrt(x.astype(np.float64).var(-1) + 1e-5), rtol=1e-6)


def test_oracle_layernorm_backward_finite_differences():
    rows, d = 3, 8
    x, dy = _rand((rows, d), 76), _rand((rows, d), 77)
    g, b = _rand((d,), 78), _rand((d,), 79)
    _, mean, rstd = oracle.layernorm_fwd(x, g, b, 1e-5)
    dx, dg, db = oracle.layernorm_bwd(x, g, mean, rstd, dy)
    fx, fg, fb = closed_forms.layernorm_grads_fd(x, g, b, dy, 1e-5)
    np.testing.assert_allclose(dx, fx, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dg, fg, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(db, fb, rtol=1e-6, atol=1e-6)
    # planted mistake: the mean(g * xhat) term dropped
    xh = (x.astype(np.float64) - mean[:, None]) * rstd[:, None]
    gg = dy * g
    wrong = rstd[:, None] * (gg - gg.mean(-1, keepdims=True))
    assert not np.allclose(wrong, fx, rtol=1e-3, atol=1e-4)
    del xh


@needs_ref
def test_oracle_layernorm_matches_reference_composition():
    """LayerNorm written with the reference's own operators (sum_axis, broadcast
    sub / mul / div / add, sqrt), the way Ember would have to compose it."""
    R = oracle.ref_lib()
    rows, d = 16, 96
    x = _rand((rows, d), 80)
    g, b = _rand((d,), 81), _rand((d,), 82)
    s = np.empty((rows, 1), np.float32)
    R.sum_axis(x, s, rows, 1, d)
    mu = s / np.float32(d)
    shp, sa, sb = oracle._bcast((rows, d), (rows, 1))
    xc = np.empty((rows, d), np.float32)
    R.sub_broadcasted(x, np.ascontiguousarray(mu), xc, shp, sa, sb, 2)
    sq = np.empty_like(xc)
    R.mul_tensor(xc, xc, sq, rows * d)
    v = np.empty((rows, 1), np.float32)
    R.sum_axis(sq, v, rows, 1, d)
    den = np.empty_like(v)
    R.sqrt_tensor(np.ascontiguousarray(v / np.float32(d) + np.float32(1e-5)), den, rows)
    xh = np.empty_like(xc)
    R.truediv_broadcasted(xc, den, xh, shp, sa, sb, 2)
    shp2, sa2, sb2 = oracle._bcast((rows, d), (1, d))
    t = np.empty_like(xh)
    R.mul_broadcasted(xh, np.ascontiguousarray(g.reshape(1, d)), t, shp2, sa2, sb2, 2)
    y_ref = np.empty_like(t)
    R.add_broadcasted(t, np.ascontiguousarray(b.reshape(1, d)), y_ref, shp2, sa2, sb2, 2)
    y, _, _ = oracle.layernorm_fwd(x, g, b, 1e-5)
    np.testing.assert_allclose(y, y_ref, rtol=1e-5, atol=1e-5)


# -------------------------------------------- config 5's decoder block


@pytest.mark.parametrize("causal", [True, False])
def test_decoder_oracle_backward_finite_differences(causal):
    """oracle/decoder.py's backward equals central differences of
    f = <block(x), dy> for every input and parameter (float64)."""
    from oracle import decoder

    B, S, H, d, r = 2, 3, 2, 8, 2
    rng = np.random.default_rng(90)
    params = decoder.init_params(d, H, r, rng)
    x = rng.standard_normal((B * S, d))
    dy = rng.standard_normal((B * S, d))
    y, cache = decoder.forward(params, x, B, S, H, causal)
    dx, grads = decoder.backward(params, cache, dy, B, S, H)

    def f():
        return float((decoder.forward(params, x, B, S, H, causal)[0] * dy).sum())

    h = 1e-6
    for arr, g in [(x, dx)] + list(zip(params, grads)):
        fd = np.zeros_like(arr)
        for idx in np.ndindex(*arr.shape):
            old = arr[idx]
            arr[idx] = old + h
            fp = f()
            arr[idx] = old - h
            fm = f()
            arr[idx] = old
            fd[idx] = (fp - fm) / (2 * h)
        np.testing.assert_allclose(g, fd, rtol=1e-5, atol=1e-7)


def test_decoder_oracle_causal_rows_see_only_the_past():
    from oracle import decoder

    B, S, H, d = 1, 5, 2, 8
    rng = np.random.default_rng(91)
    params = decoder.init_params(d, H, 2, rng)
    x = rng.standard_normal((S, d))
    y, _ = decoder.forward(params, x, B, S, H, True)
    x2 = x.copy()
    x2[3:] += 1.0
    y2, _ = decoder.forward(params, x2, B, S, H, True)
    np.testing.assert_array_equal(y[:3], y2[:3])


# ---- axis reductions and softmax through the reference's CPU operators ----

@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("shape,axis", [((7, 33), 1), ((7, 33), 0), ((3, 5, 9), 1), ((1, 1000), 1)])
def test_ref_axis_reduce_is_a_sequential_float_fold(shape, axis):
    """sum_axis is a float32 fold in index order: it equals the last entry of
    a float32 running sum (np.add.accumulate is strictly sequential), and
    max_axis equals np.max exactly."""
    x = np.random.default_rng(5).standard_normal(shape).astype(np.float32) * 100
    run = np.add.accumulate(x, axis=axis, dtype=np.float32)
    last = np.take(run, [-1], axis=axis)
    np.testing.assert_array_equal(oracle.ref_axis_reduce(x, axis, "sum"), last)
    np.testing.assert_array_equal(oracle.ref_axis_reduce(x, axis, "max"), x.max(axis=axis, keepdims=True))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("shape,axis", [((5, 40), 1), ((5, 40), 0), ((3, 4, 6), 1)])
def test_ref_softmax_against_float64(shape, axis):
    x = np.random.default_rng(6).standard_normal(shape).astype(np.float32) * 4
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=axis, keepdims=True))
    np.testing.assert_allclose(oracle.ref_softmax(x, axis), e / e.sum(axis=axis, keepdims=True),
                               rtol=2e-6, atol=1e-9)
