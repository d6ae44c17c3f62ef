"""The off-hot-path operators of the ABI (element-wise table, transpose,
reductions) against NumPy, in the style of the reference's
tests/tensor/test_tensor.py (rtol = atol = 1e-5)."""

import ctypes as C

import numpy as np
import pytest

from ember_amd import capi
from ember_amd.capi import DeviceArray

pytestmark = pytest.mark.gpu

BINARY = {
    "add": np.add, "sub": np.subtract, "mul": np.multiply, "truediv": np.true_divide,
    "max": np.maximum, "min": np.minimum,
    "gt": lambda x, y: (x > y).astype(np.float32), "lt": lambda x, y: (x < y).astype(np.float32),
    "pow": np.power,
}
SCALAR = dict(BINARY, rsub=lambda x, y: y - x, rtruediv=lambda x, y: y / x, rpow=lambda x, y: np.power(y, x))
UNARY = {
    "negate": np.negative, "exponent": np.exp, "log": np.log, "sqrt": np.sqrt, "sin": np.sin,
    "cos": np.cos, "tan": np.tan, "ctg": lambda x: 1 / np.tan(x), "sinh": np.sinh,
    "cosh": np.cosh, "tanh": np.tanh, "ctgh": lambda x: 1 / np.tanh(x),
}


def _pos(n, seed):
    return (np.abs(np.random.default_rng(seed).standard_normal(n)) + 0.5).astype(np.float32)


def _call(fn, inputs, out_shape, *tail, scalar=None):
    """fn(*input ptrs, [scalar], out ptr, *tail) with explicit C types."""
    ins = [DeviceArray.from_numpy(a) for a in inputs]
    out = DeviceArray(out_shape)
    args = [C.c_void_p(x.ptr) for x in ins]
    if scalar is not None:
        args.append(C.c_float(scalar))
    args.append(C.c_void_p(out.ptr))
    args.extend(C.c_int(t) for t in tail)
    fn(*args)
    capi.check()
    return out.numpy()


@pytest.mark.parametrize("name", list(BINARY))
def test_binary(name):
    x, y = _pos(1000, 1), _pos(1000, 2)
    got = _call(getattr(capi.lib(), f"{name}_tensor"), [x, y], (1000,), 1000)
    np.testing.assert_allclose(got, BINARY[name](x, y), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("name", list(SCALAR))
def test_scalar(name):
    x = _pos(777, 3)
    got = _call(getattr(capi.lib(), f"{name}_scalar"), [x], (777,), 777, scalar=1.5)
    np.testing.assert_allclose(got, SCALAR[name](x, np.float32(1.5)), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("name", list(UNARY))
def test_unary(name):
    x = _pos(513, 4)
    got = _call(getattr(capi.lib(), f"{name}_tensor"), [x], (513,), 513)
    np.testing.assert_allclose(got, UNARY[name](x), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("sa,sb", [((32, 10), (10,)), ((10, 1), (1, 5)), ((8, 1, 64), (1, 10, 1))])
@pytest.mark.parametrize("name", ["add", "sub", "mul", "truediv"])
def test_broadcast(name, sa, sb):
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(sa) + 3).astype(np.float32)
    b = (rng.standard_normal(sb) + 3).astype(np.float32)
    ref = BINARY[name](a, b)
    nd = ref.ndim
    sa_p = (1,) * (nd - a.ndim) + sa
    sb_p = (1,) * (nd - b.ndim) + sb

    def strides(shape):
        st, cur = [0] * len(shape), 1
        for i in range(len(shape) - 1, -1, -1):
            st[i] = 0 if shape[i] == 1 and ref.shape[i] != 1 else cur
            cur *= shape[i]
        return st

    arr = lambda v: (C.c_int * nd)(*v)  # noqa: E731
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    out = DeviceArray(ref.shape)
    getattr(capi.lib(), f"{name}_broadcasted")(
        C.c_void_p(da.ptr), C.c_void_p(db.ptr), C.c_void_p(out.ptr), arr(ref.shape),
        arr(strides(sa_p)), arr(strides(sb_p)), nd)
    capi.check()
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n,m", [(5, 5), (2, 5), (33, 70), (1024, 3)])
def test_transpose(n, m):
    a = np.random.default_rng(6).standard_normal((n, m)).astype(np.float32)
    da = DeviceArray.from_numpy(a)
    out = DeviceArray((m, n))
    capi.lib().transpose(da.ptr, out.ptr, n, m)
    capi.check()
    assert np.array_equal(out.numpy(), a.T)


@pytest.mark.parametrize("shape", [(10,), (5, 5), (2, 5), (2, 3, 4), (300, 1000)])
def test_reductions(shape):
    a = np.random.default_rng(7).standard_normal(shape).astype(np.float32)
    da = DeviceArray.from_numpy(a)
    L = capi.lib()
    assert abs(float(np.sum(a, dtype=np.float64)) - L.sum(da.ptr, a.size)) < 1e-5 * max(1, a.size / 100)
    for axis in range(a.ndim):
        outer = int(np.prod(shape[:axis]))
        inner = int(np.prod(shape[axis + 1:]))
        for fn, ref in ((L.sum_axis, np.sum), (L.max_axis, np.max)):
            out = DeviceArray((outer * inner,))
            fn(da.ptr, out.ptr, outer, inner, shape[axis])
            capi.check()
            np.testing.assert_allclose(out.numpy(), ref(a, axis=axis).reshape(-1), rtol=1e-5, atol=1e-4)
