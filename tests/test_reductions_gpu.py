"""Axis reductions, fused softmax and cross-entropy on the GPU.

sum_axis / max_axis keep the reference's arithmetic (a float fold in index
order per output, operators_gpu.cu:175-219 and operators_cpu.c:92-120), so
they are checked bitwise against the reference's own CPU operators built from
its sources (oracle/_ref).  softmax_axis fuses Ember's five-operator softmax
(tensor.py:430-437); it is checked against that composition run through the
reference's CPU operators, and against float64 NumPy at the reference's own
test tolerance (tests/tensor/test_tensor.py:53-57,208-219: rtol = atol =
1e-5)."""

import numpy as np
import pytest

import ember_amd as em
import gpu_helpers as G
import oracle
from ember_amd import Tensor, loss

pytestmark = pytest.mark.gpu

REF_SHAPES = [(10,), (5, 5), (2, 5), (2, 3, 4)]          # test_tensor.py SHAPES
BIG_SHAPES = [(8192, 1024), (3, 5000), (64, 3, 777), (1, 100000), (300, 63), (129, 65),
              (7, 1), (2048, 2049)]


def rnd(shape, seed=0, scale=3.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


@pytest.mark.parametrize("shape", REF_SHAPES + BIG_SHAPES)
def test_axis_reductions_bitwise_vs_reference(shape):
    G.say(f"sum/amax axis shape={shape}")
    x = rnd(shape, 1)
    t = Tensor(x)
    for axis in range(len(shape)):
        got_s = em.sum(t, axis=axis, keepdims=True).to_np()
        got_m = em.amax(t, axis=axis, keepdims=True).to_np()
        np.testing.assert_array_equal(got_s, oracle.ref_axis_reduce(x, axis, "sum"))
        np.testing.assert_array_equal(got_m, oracle.ref_axis_reduce(x, axis, "max"))


SOFTMAX_CASES = REF_SHAPES + [(4096, 1), (3, 64), (5, 65), (1000, 1024), (33, 2048), (9, 2049),
                              (16, 4096), (5, 10001), (2, 65536), (6, 300, 7), (4, 5, 6)]


@pytest.mark.parametrize("shape", SOFTMAX_CASES)
def test_softmax_matches_reference_composition(shape):
    G.say(f"softmax shape={shape}")
    x = rnd(shape, 2)
    t = Tensor(x)
    for axis in range(len(shape)):
        got = em.softmax(t, axis=axis).to_np()
        ref = oracle.ref_softmax(x, axis)
        # The composition's divisor is a sequential float sum of L terms,
        # itself off by up to (L-1) u relative (u = 2^-24); the fused
        # kernel's tree sum is within log2(L) u.
        L = shape[axis]
        np.testing.assert_allclose(got, ref, rtol=max(1e-5, 2.0 * L * 2.0 ** -24), atol=1e-7)
        x64 = x.astype(np.float64)
        e = np.exp(x64 - x64.max(axis=axis, keepdims=True))
        np.testing.assert_allclose(got, e / e.sum(axis=axis, keepdims=True), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(em.softmax(t).to_np().sum(-1), 1.0, rtol=1e-5)


def test_softmax_inf_and_extreme_rows():
    """A -inf entry gives probability 0; a dominant entry gives 1; large
    shifts do not overflow (the max is subtracted first)."""
    x = np.zeros((4, 3000), np.float32)
    x[0, 5] = -np.inf
    x[1, 17] = 200.0
    x[2] += 1e30
    x[3] = np.linspace(-80, 80, 3000, dtype=np.float32)
    got = em.softmax(Tensor(x)).to_np()
    assert got[0, 5] == 0.0 and np.isfinite(got).all()
    assert got[1, 17] == pytest.approx(1.0) and got[1, :17].max() < 1e-80 + 1e-38
    np.testing.assert_allclose(got[2], 1.0 / 3000, rtol=1e-5)
    np.testing.assert_allclose(got, oracle.ref_softmax(x, 1), rtol=1e-5, atol=1e-30)


def test_cross_entropy_forward_backward():
    """CrossEntropyLoss (losses.py:29-56) against float64 NumPy."""
    B, Cn = 257, 1000
    logits = rnd((B, Cn), 3)
    target = np.eye(Cn, dtype=np.float32)[np.random.default_rng(4).integers(0, Cn, B)]
    ce = loss.CrossEntropyLoss()
    value = ce(Tensor(logits), Tensor(target))
    grad = ce.backward().to_np()
    l64 = logits.astype(np.float64)
    lp = l64 - l64.max(-1, keepdims=True)
    lp -= np.log(np.exp(lp).sum(-1, keepdims=True))
    assert value == pytest.approx(-(target * lp).sum() / B, rel=1e-5)
    np.testing.assert_allclose(grad, (np.exp(lp) - target) / B, rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("shape", [(8192, 1024), (3, 7), (1000003,)])
def test_mse_fused_pass_is_bitwise_the_composed_operators(shape):
    """MSELoss with equal shapes runs one fused pass; its loss equals
    sum(diff * diff) / n and its gradient (2 / n) * diff of the composed
    operators (losses.py:19-26) bit for bit, and both match float64."""
    pred, target = rnd(shape, 21), rnd(shape, 22)
    mse = loss.MSELoss()
    value = mse(Tensor(pred), Tensor(target))
    grad = mse.backward().to_np()
    diff = Tensor(pred) - Tensor(target)
    n = int(np.prod(shape))
    assert value == em.sum(diff * diff) / n
    assert np.array_equal(grad, ((2.0 / n) * diff).to_np())
    d64 = pred.astype(np.float64) - target.astype(np.float64)
    assert value == pytest.approx((d64 * d64).sum() / n, rel=1e-6)
    # Broadcasting targets still compose the reference's operators.
    if len(shape) == 2:
        row = rnd((1, shape[1]), 23)
        value_b = loss.MSELoss()(Tensor(pred), Tensor(row))
        d = pred.astype(np.float64) - row
        assert value_b == pytest.approx((d * d).sum() / n, rel=1e-6)
