"""The drop-in, executed: the reference's own CPython bindings, unchanged,
calling this library on the GPU.

oracle/Makefile (target link-check) compiles the reference's
src/tensor/tensor_api.c and src/random/random_api.c where they lie and links
them as the extension modules ember._core._tensor and ember._core._em_random
against libember_amd.so instead of the reference's CPU/CUDA backend sources
(the build runs where the reference checkout exists; the built modules travel
to the GPU box with the rest of the tree).  Here they are imported and called
through their own Python API (_from_numpy, _matmul, _sum_axis, ..., _to_np),
so every device allocation, copy, launch and synchronisation below goes
through the reference's C code into this library:
  * matmul / matmul_batched: the oracle's FP64-accumulated result within the
    north-star tolerance and the order-free fp32 bound (as tests/
    test_matmul_gpu.py); the reference's shape errors raised by its own code;
  * transpose, element-wise add / mul / scalar ops and broadcasts: bitwise
    the reference's compiled CPU operators (the same IEEE operations);
    exp / tanh within 1e-5 (device and host math libraries differ in ulps);
  * sum_axis / max_axis: bitwise the reference's CPU fold; sum within fp32
    rounding of the float64 sum;
  * _uniform / _constant: values in range, the constant exact.
"""

import importlib.util
import os
import sys
import types

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from tolerance import assert_north_star

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LINK = os.path.join(ROOT, "oracle", "_ref", "link")


def _load(name, fname):
    spec = importlib.util.spec_from_file_location(name, os.path.join(LINK, fname))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def ref():
    if not (os.path.exists(os.path.join(LINK, "_tensor.so")) and oracle.ref_available()):
        pytest.skip("the reference's bindings are built from its checkout (oracle/Makefile link-check)")
    G.say("importing the reference's own bindings linked against libember_amd.so")
    # The reference's package layout, ember/_core/{_tensor,_em_random}.so:
    # _em_random finds the _Tensor type by importing ember._core._tensor.
    # Only the two compiled modules are loaded, under empty parent packages.
    saved = {k: sys.modules.get(k) for k in ("ember", "ember._core", "ember._core._tensor",
                                              "ember._core._em_random")}
    for name in ("ember", "ember._core"):
        pkg = types.ModuleType(name)
        pkg.__path__ = []
        sys.modules[name] = pkg
    try:
        yield _load("ember._core._tensor", "_tensor.so"), _load("ember._core._em_random", "_em_random.so")
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


def _u(shape, seed):
    return np.random.default_rng(seed).uniform(-1, 1, shape).astype(np.float32)


def _np(t, shape):
    return t._to_np().reshape(shape)


def test_matmul_through_reference_binding(ref):
    T, _ = ref
    n, k, m = 256, 192, 320
    a, b = _u((n, k), 1), _u((k, m), 2)
    G.say("reference _matmul 256x192 @ 192x320")
    c = _np(T._matmul(T._from_numpy(a), T._from_numpy(b), n, m, k), (n, m))
    exact = oracle.matmul(a, b)
    assert (np.abs(c.astype(np.float64) - exact) <= G.gemm_error_bound(a, b)).all()
    assert_north_star(c, exact)

    ab, bb = _u((3, 64, 96), 3), _u((3, 96, 80), 4)
    G.say("reference _matmul_batched 3 x (64x96 @ 96x80)")
    cb = _np(T._matmul_batched(T._from_numpy(ab), T._from_numpy(bb), 3, 64, 80, 96), (3, 64, 80))
    for i in range(3):
        assert_north_star(cb[i], oracle.matmul(ab[i], bb[i]), f"batch {i}")

    with pytest.raises(ValueError, match="Shape mismatch A"):
        T._matmul(T._from_numpy(a), T._from_numpy(b), n + 1, m, k)
    with pytest.raises(ValueError, match="Shape mismatch B"):
        T._matmul_batched(T._from_numpy(ab), T._from_numpy(bb), 3, 64, 81, 96)


def test_elementwise_and_broadcast_through_reference_binding(ref):
    T, _ = ref
    R = oracle.ref_lib()
    x, y = _u((4, 5, 3), 5), _u((4, 5, 3), 6) + 1.5
    tx, ty = T._from_numpy(x), T._from_numpy(y)
    n = x.size

    def cpu(name, *args):
        out = np.empty(n, np.float32)
        getattr(R, name)(*args, out, n)
        return out.reshape(x.shape)

    G.say("reference element-wise operators")
    assert np.array_equal(_np(T._add_tensor(tx, ty), x.shape), cpu("add_tensor", x, y))
    assert np.array_equal(_np(T._mul_tensor(tx, ty), x.shape), cpu("mul_tensor", x, y))
    assert np.array_equal(_np(T._truediv_tensor(tx, ty), x.shape), cpu("truediv_tensor", x, y))
    assert np.array_equal(_np(T._mul_scalar(tx, 0.37), x.shape), cpu("mul_scalar", x, np.float32(0.37)))
    assert np.array_equal(_np(T._add_scalar(tx, -2.5), x.shape), cpu("add_scalar", x, np.float32(-2.5)))
    np.testing.assert_allclose(_np(T._exponent(tx), x.shape), np.exp(x.astype(np.float64)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(T._tanh(tx), x.shape), np.tanh(x.astype(np.float64)), rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match="Size mismatch"):
        T._add_tensor(tx, T._from_numpy(x[:2]))

    # (4, 1, 3) + (1, 5, 3) -> (4, 5, 3): element strides with 0 on broadcast axes.
    p, q = _u((4, 1, 3), 7), _u((1, 5, 3), 8)
    shape, sp, sq = (4, 5, 3), (3, 0, 1), (0, 3, 1)
    G.say("reference _add_broadcasted / _truediv_broadcasted")
    for op in ("add", "truediv"):
        got = _np(getattr(T, f"_{op}_broadcasted")(T._from_numpy(p), T._from_numpy(q + 2.0), shape, sp, sq), shape)
        want = np.empty(60, np.float32)
        ints = lambda t: np.array(t, np.int32)  # noqa: E731
        getattr(R, f"{op}_broadcasted")(p, (q + 2.0).astype(np.float32), want, ints(shape), ints(sp), ints(sq), 3)
        assert np.array_equal(got, want.reshape(shape)), op


def test_transpose_and_reductions_through_reference_binding(ref):
    T, _ = ref
    a = _u((33, 70), 9)
    G.say("reference _transpose / _sum / _sum_axis / _max_axis")
    assert np.array_equal(_np(T._transpose(T._from_numpy(a), 33, 70), (70, 33)), a.T)
    x = _u((6, 257, 5), 10)
    tx = T._from_numpy(x)
    for axis in (0, 1, 2):
        shape = list(x.shape)
        shape[axis] = 1
        for kind in ("sum", "max"):
            got = _np(getattr(T, f"_{kind}_axis")(tx, x.shape, axis), tuple(shape))
            assert np.array_equal(got, oracle.ref_axis_reduce(x, axis, kind)), (kind, axis)
    total = T._sum(tx)
    exact = float(x.astype(np.float64).sum())
    assert abs(total - exact) <= 1e-5 * np.abs(x).sum()


def test_tensor_lifetime_and_random_through_reference_binding(ref):
    T, Rnd = ref
    G.say("reference _Tensor allocation, _uniform, _constant")
    for size in (1, 1000, 1 << 20):  # alloc_memory / free_memory through tp_init / tp_dealloc
        t = T._Tensor(size)
        assert t.size == size
        del t
    Rnd._seed(3)
    u = Rnd._uniform(-2.0, 3.0, (40, 25))._to_np()
    assert u.shape == (1000,) and (u >= -2.0).all() and (u <= 3.0).all() and u.std() > 1.0
    c = Rnd._constant(2.5, (7, 3))._to_np()
    assert np.array_equal(c, np.full(21, 2.5, np.float32))
