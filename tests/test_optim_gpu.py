"""Fused optimiser steps (adam_step, adamw_step, sgd_step) on the GPU.

Bit-exact against the CPU oracle, which is itself bit-exact against the
reference's own CPU operators composed as ember/optim/adam.py, adamw.py and
sgd.py compose them (tests/test_oracle.py).  The front-end optimisers are
also checked the way the reference's tests/optim/test_adam.py,
test_adamw.py and test_sgd.py check Ember's (numpy formulas)."""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from ember_amd import Tensor, capi, optim
from ember_amd.capi import DeviceArray

pytestmark = pytest.mark.gpu

HP = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8)


def _states(sizes, seed):
    rng = np.random.default_rng(seed)
    out = []
    for n in sizes:
        out.append([rng.standard_normal(n).astype(np.float32),
                    np.zeros(n, np.float32), np.zeros(n, np.float32)])
    return out


def test_multi_tensor_bitwise_over_steps():
    # 70 tensors: more than one launch (48 per launch), empty, tiny, ragged and
    # chunk-edge sizes.
    rng = np.random.default_rng(1)
    sizes = [0, 1, 3, 4095, 4096, 4097, 100003] + list(rng.integers(1, 20000, 63))
    G.say(f"adam_step {len(sizes)} tensors")
    host = _states(sizes, 2)
    dev = [[DeviceArray.from_numpy(x) if x.size else DeviceArray((0,)) for x in st] for st in host]
    for t in (1, 2, 3):
        grads = [rng.standard_normal(n).astype(np.float32) for n in sizes]
        dgrads = [DeviceArray.from_numpy(g) if g.size else DeviceArray((0,)) for g in grads]
        st = capi.adam_step([d[0] for d in dev], dgrads, [d[1] for d in dev], [d[2] for d in dev],
                            HP["lr"], HP["beta1"], HP["beta2"], HP["eps"], t)
        capi.check(st, "adam_step")
        for (p, m, v), g in zip(host, grads):
            oracle.adam_step(p, g, m, v, HP["lr"], HP["beta1"], HP["beta2"], HP["eps"], t)
    for (p, m, v), (dp, dm, dv) in zip(host, dev):
        if p.size == 0:
            continue
        assert np.array_equal(dp.numpy(), p)
        assert np.array_equal(dm.numpy(), m)
        assert np.array_equal(dv.numpy(), v)


def test_unaligned_tensors_take_the_scalar_path_and_stay_exact():
    n = 9000
    rng = np.random.default_rng(3)
    p, g, m, v = (rng.standard_normal(n + 1).astype(np.float32) for _ in range(4))
    v = np.abs(v)
    dp, dg, dm, dv = (DeviceArray.from_numpy(x) for x in (p, g, m, v))
    L = capi.lib()
    tab = lambda x: (capi._vp * 1)(x.ptr + 4)  # noqa: E731  (offset by one float)
    sizes = (capi._i64 * 1)(n)
    st = L.adam_step(tab(dp), tab(dg), tab(dm), tab(dv), sizes, 1, 0.01, 0.8, 0.99, 1e-6, 5)
    capi.check(st, "adam_step")
    P, M, V = p[1:].copy(), m[1:].copy(), v[1:].copy()
    oracle.adam_step(P, g[1:].copy(), M, V, 0.01, 0.8, 0.99, 1e-6, 5)
    assert np.array_equal(dp.numpy()[1:], P) and dp.numpy()[0] == p[0]
    assert np.array_equal(dm.numpy()[1:], M) and np.array_equal(dv.numpy()[1:], V)


def test_invalid_arguments_are_rejected():
    L = capi.lib()
    empty = (capi._vp * 1)(None)
    sizes = (capi._i64 * 1)(10)
    assert L.adam_step(empty, empty, empty, empty, sizes, 1, 0.1, 0.9, 0.9, 1e-8, 1) == 1
    assert L.adam_step(empty, empty, empty, empty, sizes, 0, 0.1, 0.9, 0.9, 1e-8, 0) == 1  # t < 1
    L.ember_get_last_error()


# ---------------------------------------------------- front-end (optim.Adam)


def _numpy_adam(param, grad, m, v, t, lr, b1, b2, eps):
    m = b1 * m + (1 - b1) * grad
    v = b2 * v + (1 - b2) * grad ** 2
    return param - lr * (m / (1 - b1 ** t)) / (np.sqrt(v / (1 - b2 ** t)) + eps), m, v


def test_adam_initialization():
    opt = optim.Adam([Tensor(np.random.randn(2, 3).astype(np.float32))], lr=0.1)
    assert len(opt.means) == len(opt.variances) == 1 and opt.t == 0
    assert not opt.means[0].to_np().any() and not opt.variances[0].to_np().any()


def test_adam_step_math_and_bitwise():
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-8
    p = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    g = np.array([[0.1, -0.1], [0.5, 0.0]], np.float32)
    tp = Tensor(p)
    opt = optim.Adam([tp], lr=lr, betas=(b1, b2), eps=eps)
    opt.apply([Tensor(g)])
    ep, em_, ev = _numpy_adam(p, g, 0, 0, 1, lr, b1, b2, eps)
    np.testing.assert_allclose(tp.to_np(), ep, rtol=1e-5)
    np.testing.assert_allclose(opt.means[0].to_np(), em_, rtol=1e-5)
    np.testing.assert_allclose(opt.variances[0].to_np(), ev, rtol=1e-5)
    P, M, V = p.reshape(-1).copy(), np.zeros(4, np.float32), np.zeros(4, np.float32)
    oracle.adam_step(P, g.reshape(-1).copy(), M, V, lr, b1, b2, eps, 1)
    assert np.array_equal(tp.to_np().reshape(-1), P) and opt.t == 1


def test_adam_multistep_convergence():
    lr = 0.1
    tp = Tensor(np.array([2.0], np.float32))
    opt = optim.Adam([tp], lr=lr)
    x, m, v = np.array([2.0], np.float32), 0.0, 0.0
    for t in range(1, 6):
        g = 2 * tp.to_np()
        opt.apply([Tensor(g)])
        x, m, v = _numpy_adam(x, 2 * x, m, v, t, lr, 0.9, 0.999, 1e-8)
        np.testing.assert_allclose(tp.to_np(), x, rtol=1e-5)
    assert 0.0 < tp.to_np()[0] < 2.0


def test_adam_rejects_wrong_gradients():
    opt = optim.Adam([Tensor(np.zeros(3, np.float32))])
    with pytest.raises(ValueError):
        opt.apply([])
    with pytest.raises(ValueError):
        opt.apply([Tensor(np.zeros(4, np.float32))])


# ------------------------------------------------------ AdamW and SGD kernels


def _ragged_sizes(seed):
    rng = np.random.default_rng(seed)
    return [0, 1, 3, 4095, 4096, 4097, 100003] + list(rng.integers(1, 20000, 55))


def test_adamw_multi_tensor_bitwise_over_steps():
    rng = np.random.default_rng(21)
    sizes = _ragged_sizes(22)
    G.say(f"adamw_step {len(sizes)} tensors")
    host = _states(sizes, 23)
    dev = [[DeviceArray.from_numpy(x) if x.size else DeviceArray((0,)) for x in st] for st in host]
    for t, wd in ((1, 0.01), (2, 0.5), (3, 0.0)):
        grads = [rng.standard_normal(n).astype(np.float32) for n in sizes]
        dgrads = [DeviceArray.from_numpy(g) if g.size else DeviceArray((0,)) for g in grads]
        st = capi.adamw_step([d[0] for d in dev], dgrads, [d[1] for d in dev], [d[2] for d in dev],
                             0.01, 0.9, 0.999, 1e-8, wd, t)
        capi.check(st, "adamw_step")
        for (p, m, v), g in zip(host, grads):
            oracle.adamw_step(p, g, m, v, 0.01, 0.9, 0.999, 1e-8, wd, t)
    for (p, m, v), (dp, dm, dv) in zip(host, dev):
        if p.size:
            assert np.array_equal(dp.numpy(), p)
            assert np.array_equal(dm.numpy(), m) and np.array_equal(dv.numpy(), v)


@pytest.mark.parametrize("momentum", [0.0, 0.9])
def test_sgd_multi_tensor_bitwise_over_steps(momentum):
    rng = np.random.default_rng(31)
    sizes = _ragged_sizes(32)
    G.say(f"sgd_step {len(sizes)} tensors momentum={momentum}")
    host = [[rng.standard_normal(n).astype(np.float32), np.zeros(n, np.float32)] for n in sizes]
    dev = [[DeviceArray.from_numpy(x) if x.size else DeviceArray((0,)) for x in st] for st in host]
    for _ in range(3):
        grads = [rng.standard_normal(n).astype(np.float32) for n in sizes]
        dgrads = [DeviceArray.from_numpy(g) if g.size else DeviceArray((0,)) for g in grads]
        capi.check(capi.sgd_step([d[0] for d in dev], dgrads, [d[1] for d in dev], 0.05, momentum),
                   "sgd_step")
        for (p, v), g in zip(host, grads):
            oracle.sgd_step(p, g, v, 0.05, momentum)
    for (p, v), (dp, dv) in zip(host, dev):
        if p.size:
            assert np.array_equal(dp.numpy(), p) and np.array_equal(dv.numpy(), v)


def test_adamw_and_sgd_unaligned_tensors_stay_exact():
    n = 9000
    rng = np.random.default_rng(33)
    p, g, m, v = (rng.standard_normal(n + 1).astype(np.float32) for _ in range(4))
    v = np.abs(v)
    dp, dg, dm, dv = (DeviceArray.from_numpy(x) for x in (p, g, m, v))
    L = capi.lib()
    tab = lambda x: (capi._vp * 1)(x.ptr + 4)  # noqa: E731  (offset by one float)
    sizes = (capi._i64 * 1)(n)
    capi.check(L.adamw_step(tab(dp), tab(dg), tab(dm), tab(dv), sizes, 1, 0.01, 0.8, 0.99, 1e-6, 0.2, 5),
               "adamw_step")
    P, M, V = p[1:].copy(), m[1:].copy(), v[1:].copy()
    oracle.adamw_step(P, g[1:].copy(), M, V, 0.01, 0.8, 0.99, 1e-6, 0.2, 5)
    assert np.array_equal(dp.numpy()[1:], P) and dp.numpy()[0] == p[0]
    assert np.array_equal(dm.numpy()[1:], M) and np.array_equal(dv.numpy()[1:], V)
    capi.check(L.sgd_step(tab(dp), tab(dg), tab(dm), sizes, 1, 0.03, 0.7), "sgd_step")
    oracle.sgd_step(P, g[1:].copy(), M, 0.03, 0.7)
    assert np.array_equal(dp.numpy()[1:], P) and np.array_equal(dm.numpy()[1:], M)
    assert dp.numpy()[0] == p[0]


def test_adamw_and_sgd_reject_invalid_arguments():
    L = capi.lib()
    empty = (capi._vp * 1)(None)
    sizes = (capi._i64 * 1)(10)
    assert L.adamw_step(empty, empty, empty, empty, sizes, 1, 0.1, 0.9, 0.9, 1e-8, 0.1, 1) == 1
    assert L.adamw_step(empty, empty, empty, empty, sizes, 0, 0.1, 0.9, 0.9, 1e-8, 0.1, 0) == 1
    assert L.sgd_step(empty, empty, empty, sizes, 1, 0.1, 0.9) == 1
    assert L.sgd_step(empty, empty, empty, sizes, -1, 0.1, 0.9) == 1
    L.ember_get_last_error()


# ------------------------------- front-end (optim.AdamW, optim.SGD), as the
# reference's tests/optim/test_adamw.py and test_sgd.py


def _numpy_adamw(p, g, m, v, t, lr, b1, b2, eps, wd):
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * (g ** 2)
    p = p - lr * wd * p
    return p - lr * (m / (1 - b1 ** t)) / (np.sqrt(v / (1 - b2 ** t)) + eps), m, v


def test_adamw_step_math_and_bitwise():
    lr, b1, b2, eps, wd = 0.01, 0.9, 0.999, 1e-8, 0.1
    p = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    g = np.array([[0.1, -0.1], [0.5, 0.0]], np.float32)
    tp = Tensor.from_np(p)
    opt = optim.AdamW([tp], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    x, m, v = p.copy(), np.zeros_like(p), np.zeros_like(p)
    P, M, V = p.reshape(-1).copy(), np.zeros(4, np.float32), np.zeros(4, np.float32)
    for t in (1, 2, 3):
        opt.apply([Tensor.from_np(g)])
        x, m, v = _numpy_adamw(x, g, m, v, t, lr, b1, b2, eps, wd)
        np.testing.assert_allclose(tp.to_np(), x, rtol=1e-4, atol=1e-6)
        oracle.adamw_step(P, g.reshape(-1).copy(), M, V, lr, b1, b2, eps, wd, t)
        assert np.array_equal(tp.to_np().reshape(-1), P) and opt.t == t


def test_adamw_weight_decay_shrinks_params_without_grad():
    tp = Tensor.from_np(np.full((3,), 2.0, np.float32))
    opt = optim.AdamW([tp], lr=0.1, weight_decay=0.5)
    opt.apply([Tensor.from_np(np.zeros((3,), np.float32))])
    assert np.all(tp.to_np() < 2.0)
    assert np.array_equal(tp.to_np(), np.full((3,), 2.0, np.float32) - np.float32(2.0) * np.float32(0.05))


@pytest.mark.parametrize("momentum", [0.0, 0.9])
def test_sgd_step_math(momentum):
    lr = 0.1
    p = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    g = np.array([[0.1, -0.2], [0.5, 0.0]], np.float32)
    tp = Tensor.from_np(p)
    opt = optim.SGD([tp], lr=lr, momentum=momentum)
    x, v = p.copy(), np.zeros_like(p)
    for _ in range(3):
        opt.apply([Tensor.from_np(g)])
        v = momentum * v + g
        x = x - lr * v
        np.testing.assert_allclose(tp.to_np(), x, rtol=1e-5, atol=1e-6)


def test_sgd_converges_and_rejects_wrong_gradients():
    tp = Tensor.from_np(np.array([5.0], np.float32))
    opt = optim.SGD([tp], lr=0.1)
    for _ in range(50):
        opt.apply([Tensor.from_np(2.0 * tp.to_np())])
    assert abs(tp.to_np()[0]) < 0.1
    with pytest.raises(ValueError):
        opt.apply([])
    with pytest.raises(ValueError):
        optim.AdamW([tp]).apply([Tensor.from_np(np.zeros(2, np.float32))])
