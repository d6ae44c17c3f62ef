"""The Python boundary without a device: ember_amd._core exports every name
of the reference's ember._core (ember/_core/__init__.py:1-48) plus the
attention entry points, and the front-end's argument checks (the reference's
TypeError / ValueError contract, ember/tensor/tensor.py:163-197,231-252)
fire before any device call.  CPU only."""

import math

import numpy as np
import pytest

import ember_amd as em
from ember_amd import _core
from ember_amd.tensor import Tensor, broadcast

REFERENCE_CORE = {
    "_constant", "_seed", "_uniform", "_add_broadcasted", "_add_scalar", "_add_tensor", "_cos",
    "_cosh", "_ctg", "_ctgh", "_exponent", "_from_numpy", "_gt_scalar", "_gt_tensor", "_log",
    "_lt_scalar", "_lt_tensor", "_matmul", "_matmul_batched", "_max_axis", "_max_scalar",
    "_max_tensor", "_min_scalar", "_min_tensor", "_mul_broadcasted", "_mul_scalar",
    "_mul_tensor", "_negate", "_pow_scalar", "_pow_tensor", "_rpow_scalar", "_rsub_scalar",
    "_rtruediv_scalar", "_sin", "_sinh", "_sqrt", "_sub_broadcasted", "_sub_scalar",
    "_sub_tensor", "_sum", "_sum_axis", "_tan", "_tanh", "_Tensor", "_transpose",
    "_truediv_broadcasted", "_truediv_scalar", "_truediv_tensor",
}
REFERENCE_TOP = {"Tensor", "max", "min", "amax", "exp", "log", "sin", "cos", "tan", "ctg",
                 "sinh", "cosh", "tanh", "ctgh", "T", "sum", "softmax", "sqrt"}


def fake(shape):
    """Metadata-only Tensor (no device buffer) for checks that must fire first."""
    return Tensor._from_core(None, shape)


def test_core_exports_reference_names_and_attention():
    for name in REFERENCE_CORE | {"_attention_fwd", "_attention_bwd"}:
        assert callable(getattr(_core, name)), name
    assert set(_core.REFERENCE_NAMES) == REFERENCE_CORE


def test_front_end_exports_reference_names():
    for name in REFERENCE_TOP | {"attention", "attention_forward", "attention_backward"}:
        assert callable(getattr(em, name)), name
    assert em.nn.Attention and em.random.uniform


def test_tensor_type_interface():
    T_ = _core._Tensor
    for meth in ("_copy_from_list", "_to_list", "_to_np"):
        assert callable(getattr(T_, meth))
    assert "size" in dir(T_)


def test_binding_rejects_wrong_types_before_device_work():
    with pytest.raises(TypeError):
        _core._matmul(1, 2, 3, 4, 5)
    with pytest.raises(TypeError):
        _core._add_tensor([1.0], [2.0])
    with pytest.raises(TypeError):
        _core._from_numpy(np.zeros(3, dtype=np.float64))   # float32 only
    with pytest.raises(TypeError):
        _core._from_numpy(object())
    with pytest.raises(TypeError):
        _core._attention_fwd(None, None, None, 1, 1, 1, 64, 0.125, True)


@pytest.mark.parametrize(
    "sa, sb, out",
    [((32, 10), (10,), (32, 10)), ((10, 1), (1, 5), (10, 5)),
     ((8, 1, 64), (1, 10, 1), (8, 10, 64)), ((3,), (3,), (3,))],
)
def test_broadcast_matches_numpy(sa, sb, out):
    def st(shape):
        return tuple(int(s) // 4 for s in np.empty(shape, np.float32).strides)

    shape, stra, strb = broadcast(sa, st(sa), sb, st(sb))
    assert shape == out == np.broadcast_shapes(sa, sb)
    # Every output index maps to the element numpy would broadcast.
    a = np.arange(math.prod(sa)).reshape(sa)
    b = np.arange(math.prod(sb)).reshape(sb)
    ea, eb = np.broadcast_arrays(a, b)
    for idx in np.ndindex(*shape):
        assert a.reshape(-1)[sum(i * s for i, s in zip(idx, stra))] == ea[idx]
        assert b.reshape(-1)[sum(i * s for i, s in zip(idx, strb))] == eb[idx]


def test_broadcast_rejects_incompatible_shapes():
    with pytest.raises(ValueError):
        broadcast((4, 3), (3, 1), (4, 2), (2, 1))


@pytest.mark.parametrize(
    "a, b, exc",
    [((4, 5), (4, 3), ValueError),      # inner dimensions differ
     ((4, 5, 2), (2, 3), ValueError),   # rank mismatch, batch dims differ
     ((5,), (5, 2), ValueError),        # 1-D operand
     ((2, 4, 5), (3, 5, 6), ValueError)],  # batch dims differ
)
def test_matmul_shape_errors(a, b, exc):
    with pytest.raises(exc):
        fake(a) @ fake(b)


def test_matmul_type_error():
    with pytest.raises(TypeError):
        fake((4, 5)) @ np.zeros((5, 2), np.float32)


@pytest.mark.parametrize(
    "start, target, ok",
    [((2, 3), (3, 2), True), ((2, 3), (6,), True), ((2, 3), (-1,), True),
     ((2, 3), (2, -1), True), ((2, 3), (4, 4), False), ((2, 3), (-1, -1), False),
     ((2, 3), (4, -1), False)],
)
def test_reshape(start, target, ok):
    t = fake(start)
    if not ok:
        with pytest.raises(ValueError):
            t.reshape(target)
        return
    assert t.reshape(target).shape == np.empty(start).reshape(target).shape


def test_transpose_and_reductions_validate():
    with pytest.raises(ValueError):
        em.T(fake((2, 3, 4)))
    with pytest.raises(TypeError):
        em.T(np.zeros((2, 2)))
    with pytest.raises(ValueError):
        em.amax(fake((2, 3)), axis=2)
    with pytest.raises(TypeError):
        em.softmax([1.0, 2.0])


def test_list_construction_errors():
    with pytest.raises(ValueError):
        Tensor([[1.0, 2.0], [3.0]])          # ragged
    with pytest.raises(TypeError):
        Tensor([[True, False]])              # bool
    with pytest.raises(TypeError):
        Tensor("abc")


def test_attention_argument_errors():
    q = fake((2, 4, 16, 64))
    with pytest.raises(ValueError):
        em.attention(q, fake((2, 4, 16, 32)), q)
    with pytest.raises(ValueError):
        em.attention(fake((64,)), fake((64,)), fake((64,)))
    with pytest.raises(TypeError):
        em.attention(q, q, np.zeros((2, 4, 16, 64)))
    with pytest.raises(RuntimeError):
        em.nn.Attention(causal=True).backward(q)


@pytest.mark.parametrize("module", ["_tensor", "_em_random"])
def test_type_stubs_match_the_binding_modules(module):
    """ember_amd/_core/<module>.pyi declares exactly the functions the
    compiled module exports, with as many parameters as each parses."""
    import ast
    import importlib
    import inspect
    import os

    mod = importlib.import_module(f"ember_amd._core.{module}")
    path = os.path.join(os.path.dirname(mod.__file__), f"{module}.pyi")
    tree = ast.parse(open(path).read())
    stubbed = {n.name for n in tree.body if isinstance(n, ast.FunctionDef)}
    exported = {n for n, f in vars(mod).items() if inspect.isbuiltin(f)}
    assert stubbed == exported, (sorted(stubbed - exported), sorted(exported - stubbed))
    if module == "_tensor":
        cls = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "_Tensor")
        members = {n.name for n in cls.body if isinstance(n, ast.FunctionDef)} - {"__init__"}
        assert members <= set(dir(mod._Tensor)), sorted(members - set(dir(mod._Tensor)))


def _reference_classes(relpath):
    """{class name: (base names, {method: {arg: default}})} of a reference
    source file, read as text (nothing of it is imported or run)."""
    import ast
    import os

    tree = ast.parse(open(os.path.join("/root/reference", relpath)).read())
    out = {}
    for node in tree.body:
        if not isinstance(node, ast.ClassDef):
            continue
        methods = {}
        for f in node.body:
            if isinstance(f, ast.FunctionDef):
                args = f.args.args[len(f.args.args) - len(f.args.defaults):]
                methods[f.name] = {a.arg: ast.literal_eval(d) for a, d in zip(args, f.args.defaults)}
        out[node.name] = ([b.id for b in node.bases if isinstance(b, ast.Name)], methods)
    return out


@pytest.mark.skipif(not __import__("os").path.isdir("/root/reference/ember"),
                    reason="needs the reference checkout (read as text)")
@pytest.mark.parametrize("relpath,module", [
    ("ember/nn/activations.py", "nn"), ("ember/nn/layers.py", "nn"), ("ember/nn/base.py", "nn"),
    ("ember/optim/adam.py", "optim"), ("ember/optim/adamw.py", "optim"), ("ember/optim/sgd.py", "optim"),
    ("ember/loss/base.py", "loss"), ("ember/loss/losses.py", "loss"),
])
def test_nn_optim_loss_classes_mirror_the_reference(relpath, module):
    """Every class of the reference's nn / optim / loss modules exists here
    with the same base class, the same public methods and the same
    constructor defaults (no device work: nothing is instantiated)."""
    import inspect

    mod = getattr(em, module)
    for name, (bases, methods) in _reference_classes(relpath).items():
        cls = getattr(mod, name, None)
        assert cls is not None, f"{module}.{name} missing"
        for b in bases:
            if b != "ABC":
                assert issubclass(cls, getattr(mod, b)), (name, b)
        for meth, defaults in methods.items():
            if meth.startswith("_") and meth not in ("__init__", "__call__"):
                continue
            assert hasattr(cls, meth), f"{module}.{name}.{meth}"
            params = inspect.signature(getattr(cls, meth)).parameters
            for arg, value in defaults.items():
                assert arg in params and params[arg].default == value, (name, meth, arg)


def test_dropout_rejects_bad_probability():
    for p in (1.0, -0.1, 1.5):
        with pytest.raises(ValueError):
            em.nn.Dropout(p)
