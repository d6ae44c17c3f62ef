"""The Python boundary on the GPU: ember_amd.Tensor over the _core binding
over libember_amd.so, checked the way the reference's own suite checks
ember.Tensor (tests/tensor/test_tensor.py: numpy as the oracle,
rtol = atol = 1e-5 for element-wise work), plus attention through the
front-end and the nn layer against the CPU oracle (north-star tolerance
max-abs 2e-4 / rel 1e-3)."""

import operator

import numpy as np
import pytest

import ember_amd as em
import gpu_helpers as G
import oracle
from ember_amd import Tensor, _core

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-5)
ATT_TOL = dict(rtol=1e-3, atol=2e-4)
SHAPES = [(10,), (5, 5), (2, 5), (2, 3, 4)]


def rnd(shape, seed=0, positive=False):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    return np.abs(x) + 0.5 if positive else x


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op, np_op", [
    (operator.add, np.add), (operator.sub, np.subtract), (operator.mul, np.multiply),
    (operator.truediv, np.true_divide), (operator.gt, np.greater), (operator.lt, np.less),
    (operator.pow, np.power), (em.max, np.maximum), (em.min, np.minimum)])
def test_binary_same_shape(shape, op, np_op):
    G.say(f"front-end binary {getattr(op, '__name__', op)} {shape}")
    a, b = rnd(shape, 1, True), rnd(shape, 2, True)
    np.testing.assert_allclose(op(Tensor(a), Tensor(b)).to_np(), np_op(a, b).astype(np.float32),
                               **TOL)


@pytest.mark.parametrize("sa, sb", [((32, 10), (10,)), ((10, 1), (1, 5)), ((8, 1, 64), (1, 10, 1))])
@pytest.mark.parametrize("op", [operator.add, operator.sub, operator.mul, operator.truediv])
@pytest.mark.parametrize("reverse", [False, True])
def test_binary_broadcast(sa, sb, op, reverse):
    a, b = rnd(sa, 3, True), rnd(sb, 4, True)
    if reverse:
        a, b = b, a
    got = op(Tensor(a), Tensor(b))
    ref = op(a, b)
    assert got.shape == ref.shape
    np.testing.assert_allclose(got.to_np(), ref, **TOL)


@pytest.mark.parametrize("scalar", [0.0, 1.0, -5.5, 100])
@pytest.mark.parametrize("op", [operator.add, operator.sub, operator.mul, operator.truediv])
def test_scalar_both_sides(scalar, op):
    a = rnd((3, 7), 5, True)
    with np.errstate(divide="ignore"):   # x / 0 -> +-inf on both sides, as intended
        ref = op(a, np.float32(scalar))
    np.testing.assert_allclose(op(Tensor(a), scalar).to_np(), ref, **TOL)
    if op is operator.truediv and scalar == 0:
        return
    np.testing.assert_allclose(op(scalar, Tensor(a)).to_np(), op(np.float32(scalar), a), **TOL)


@pytest.mark.parametrize("fn, np_fn", [
    (operator.neg, np.negative), (em.exp, np.exp), (em.log, np.log), (em.sqrt, np.sqrt),
    (em.sin, np.sin), (em.cos, np.cos), (em.tan, np.tan), (em.tanh, np.tanh),
    (em.ctg, lambda x: 1 / np.tan(x)), (em.ctgh, lambda x: 1 / np.tanh(x))])
def test_unary(fn, np_fn):
    a = rnd((4, 6), 6, True)
    np.testing.assert_allclose(fn(Tensor(a)).to_np(), np_fn(a), rtol=1e-4, atol=1e-5)


def test_lists_and_transpose():
    t = Tensor([[1, 2, 3], [4, 5, 6]])
    assert t.shape == (2, 3) and t.dtype == "float32"
    assert em.T(t).to_list() == [[1.0, 4.0], [2.0, 5.0], [3.0, 6.0]]
    assert Tensor(2.5).to_list() == 2.5


@pytest.mark.parametrize("sa, sb", [((4, 5), (5, 3)), ((1, 1), (1, 1)), ((32, 128), (128, 64)),
                                    ((2, 3, 4), (2, 4, 5)), ((4, 2, 3, 6), (4, 2, 6, 2))])
def test_matmul(sa, sb):
    a, b = rnd(sa, 7), rnd(sb, 8)
    got = Tensor(a) @ Tensor(b)
    assert got.shape == (a @ b).shape
    np.testing.assert_allclose(got.to_np(), a @ b, **TOL)


@pytest.mark.parametrize("shape", SHAPES)
def test_reductions_and_softmax(shape):
    a = rnd(shape, 9)
    t = Tensor(a)
    assert abs(em.sum(t) - float(a.sum(dtype=np.float64))) < 1e-4 * max(1.0, a.size / 10)
    for axis in range(len(shape)):
        np.testing.assert_allclose(em.sum(t, axis=axis).to_np(), a.sum(axis), **TOL)
        np.testing.assert_allclose(em.amax(t, axis=axis, keepdims=True).to_np(),
                                   a.max(axis, keepdims=True), **TOL)
        e = np.exp(a - a.max(axis, keepdims=True))
        np.testing.assert_allclose(em.softmax(t, axis=axis).to_np(),
                                   e / e.sum(axis, keepdims=True), **TOL)


def test_inplace_adopts_buffer():
    a = rnd((3, 3), 10)
    t = Tensor(a)
    ident = id(t)
    t += 1.0
    t *= Tensor(a)
    assert id(t) == ident
    np.testing.assert_allclose(t.to_np(), (a + 1) * a, **TOL)


def test_random_seed_reproducible():
    em.random.seed(123)
    x = em.random.uniform(-1.0, 1.0, (100,)).to_np()
    em.random.seed(123)
    y = em.random.uniform(-1.0, 1.0, (100,)).to_np()
    assert np.array_equal(x, y) and x.min() >= -1 and x.max() <= 1
    assert np.array_equal(em.random.zeros((5,)).to_np(), np.zeros(5, np.float32))


# ------------------------------------------------------------------ attention


@pytest.mark.parametrize("shape", [(1, 4, 256, 64), (2, 3, 65, 128), (97, 32), (2, 130, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_front_end_matches_oracle(shape, causal):
    G.say(f"front-end attention {shape} causal={causal}")
    q, k, v, d_o = (rnd(shape, s) for s in (11, 12, 13, 14))
    full = (1,) * (4 - len(shape)) + shape
    o, lse = em.attention_forward(Tensor(q), Tensor(k), Tensor(v), causal)
    assert o.shape == shape and lse.shape == shape[:-1]
    o_ref, lse_ref = oracle.attention_fwd(q.reshape(full), k.reshape(full), v.reshape(full), causal)
    np.testing.assert_allclose(o.to_np().reshape(full), o_ref, **ATT_TOL)
    np.testing.assert_allclose(lse.to_np().reshape(full[:-1]), lse_ref, **ATT_TOL)
    grads = em.attention_backward(Tensor(q), Tensor(k), Tensor(v), o, lse, Tensor(d_o), causal)
    refs = oracle.attention_bwd(q.reshape(full), k.reshape(full), v.reshape(full), o_ref, lse_ref,
                                d_o.reshape(full), causal)
    for got, ref in zip(grads, refs):
        np.testing.assert_allclose(got.to_np().reshape(full), ref, **ATT_TOL)


def test_attention_layer_forward_backward():
    shape = (2, 2, 100, 64)
    q, k, v, g = (rnd(shape, s) for s in (21, 22, 23, 24))
    layer = em.nn.Attention(causal=True)
    o = layer((Tensor(q), Tensor(k), Tensor(v)))
    dq, dk, dv = layer.backward(Tensor(g))
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, True)
    np.testing.assert_allclose(o.to_np(), o_ref, **ATT_TOL)
    for got, ref in zip((dq, dk, dv), oracle.attention_bwd(q, k, v, o_ref, lse_ref, g, True)):
        np.testing.assert_allclose(got.to_np(), ref, **ATT_TOL)
    assert layer.parameters() == [] and layer.gradients() == []


@pytest.mark.parametrize("causal", [False, True])
def test_fused_attention_equals_ember_composition(causal):
    """Attention written with the front-end's own ops the way Ember composes it
    (q @ T(k) * scale + mask -> softmax -> @ v), run on the GPU, equals the
    fused kernel."""
    S, D = 96, 64
    q, k, v = (rnd((S, D), s) for s in (31, 32, 33))
    scale = G.scale_for(D)
    mask = np.where(np.tril(np.ones((S, S), bool)) | (not causal), 0.0, -np.inf).astype(np.float32)
    s = Tensor(q) @ em.T(Tensor(k)) * scale + Tensor(mask)
    composed = em.softmax(s, axis=-1) @ Tensor(v)
    fused = em.attention(Tensor(q), Tensor(k), Tensor(v), causal)
    np.testing.assert_allclose(fused.to_np(), composed.to_np(), **ATT_TOL)


def test_device_errors_become_exceptions():
    q = Tensor(rnd((1, 1, 8, 48), 40))        # head_dim 48 is not supported
    with pytest.raises(ValueError):
        em.attention(q, q, q)
    t = Tensor(rnd((4,), 41))
    with pytest.raises(ValueError):
        _core._matmul(t._core, t._core, 3, 3, 3)   # 4 elements are not 3 x 3
