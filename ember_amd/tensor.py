"""Tensor front-end over ``ember_amd._core`` (the MI355X backend).

Mirrors the reference's ``ember.Tensor`` (``ember/tensor/tensor.py``) for the
operations on the attention / matmul path: construction from numpy or nested
lists, element-wise arithmetic with scalars and NumPy-style broadcasting,
``@`` (2-D, or batched with equal leading dimensions, ``tensor.py:163-197``),
``T`` (2-D only, ``:376-384``), ``sum`` / ``amax`` / ``softmax``
(``:404-437``), the unary math functions, in-place operators that adopt the
result's buffer (``:205-222``).  Error types and messages follow the
reference: TypeError for non-Tensor operands, ValueError for shape problems.

Beyond the reference: ``attention`` (fused flash attention, forward) and
``attention_forward`` / ``attention_backward`` (O and logsumexp; gradients
recomputed from the logsumexp) on the HIP kernels.
"""

from __future__ import annotations

import builtins
import math
from typing import Any, Union

import numpy as np

from ember_amd import _core as C

Scalar = Union[int, float]


def contiguous_strides(shape: tuple[int, ...]) -> tuple[int, ...]:
    """Row-major strides in elements (``tensor_utils.py:85-94``)."""
    strides, step = [], 1
    for d in reversed(shape):
        strides.append(step)
        step *= d
    return tuple(reversed(strides))


def broadcast(shape_a, strides_a, shape_b, strides_b):
    """Output shape and per-operand strides of a NumPy-style broadcast: the
    shorter shape is padded with leading 1s, size-1 dimensions get stride 0
    (``tensor_utils.py:97-140``)."""
    nd = builtins.max(len(shape_a), len(shape_b))  # `max` below is the element-wise op
    sa = (1,) * (nd - len(shape_a)) + tuple(shape_a)
    sb = (1,) * (nd - len(shape_b)) + tuple(shape_b)
    ta = (0,) * (nd - len(strides_a)) + tuple(strides_a)
    tb = (0,) * (nd - len(strides_b)) + tuple(strides_b)
    out, oa, ob = [], [], []
    for da, xa, db, xb in zip(sa, ta, sb, tb):
        if da == db:
            out.append(da), oa.append(xa), ob.append(xb)
        elif da == 1:
            out.append(db), oa.append(0), ob.append(xb)
        elif db == 1:
            out.append(da), oa.append(xa), ob.append(0)
        else:
            raise ValueError(
                f"Operands could not be broadcast together with shapes {tuple(shape_a)} "
                f"and {tuple(shape_b)}")
    return tuple(out), tuple(oa), tuple(ob)


def _flatten(data: Any) -> tuple[tuple[int, ...], list[float]]:
    """Shape and flat values of a scalar or a rectangular nested list
    (``tensor_utils.py:4-82``: ragged input is a ValueError, bool and
    non-numbers a TypeError)."""
    if not isinstance(data, list):
        if isinstance(data, bool) or not isinstance(data, (int, float)):
            raise TypeError(f"Unsupported data type: {type(data)}")
        return (), [float(data)]
    shape = []
    node = data
    while isinstance(node, list):
        shape.append(len(node))
        if not node:
            break
        node = node[0]
    flat: list[float] = []

    def walk(node, depth):
        if depth < len(shape):
            if not isinstance(node, list):
                raise ValueError(f"Ragged sequence: expected a list at depth {depth}")
            if len(node) != shape[depth]:
                raise ValueError(f"Shape mismatch at depth {depth}: expected length "
                                 f"{shape[depth]}, got {len(node)}")
            for item in node:
                walk(item, depth + 1)
        else:
            if isinstance(node, list):
                raise ValueError("Ragged sequence: expected a scalar, got a list")
            if isinstance(node, bool) or not isinstance(node, (int, float)):
                raise TypeError(f"Unsupported item type: {type(node)}")
            flat.append(float(node))

    walk(data, 0)
    return tuple(shape), flat


class Tensor:
    """A float32 tensor in device memory (row-major, shape kept in Python)."""

    dtype = "float32"

    def __init__(self, data: Any):
        if isinstance(data, np.ndarray):
            self._core = C._from_numpy(np.ascontiguousarray(data, dtype=np.float32))
            self.shape = tuple(int(d) for d in data.shape)
        else:
            shape, flat = _flatten(data)
            self._core = C._Tensor(math.prod(shape))
            self._core._copy_from_list(flat)
            self.shape = shape
        self.strides = contiguous_strides(self.shape)

    @classmethod
    def _from_core(cls, core, shape: tuple[int, ...]) -> Tensor:
        t = cls.__new__(cls)
        t._core = core
        t.shape = tuple(shape)
        t.strides = contiguous_strides(t.shape)
        return t

    @classmethod
    def from_np(cls, array: np.ndarray) -> Tensor:
        return cls(np.asarray(array))

    # ---- conversion ----
    def to_np(self) -> np.ndarray:
        return self._core._to_np().reshape(self.shape)

    def to_list(self):
        return self._core._to_list(self.shape)

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    def reshape(self, new_shape: tuple[int, ...]) -> Tensor:
        """In-place metadata reshape; one dimension may be -1 (``tensor.py:231-252``)."""
        new_shape = tuple(new_shape)
        total = self.size
        if new_shape.count(-1) > 1:
            raise ValueError("Only one dimension can be -1 (inferred)")
        if -1 in new_shape:
            known = -math.prod(new_shape)
            if known == 0 or total % known:
                raise ValueError(f"Cannot reshape size {total} into {new_shape}")
            new_shape = tuple(total // known if d == -1 else d for d in new_shape)
        elif math.prod(new_shape) != total:
            raise ValueError(f"Cannot reshape size {total} into {new_shape}")
        self.shape = new_shape
        self.strides = contiguous_strides(new_shape)
        return self

    def __repr__(self) -> str:
        return f"Tensor({self.to_list()})"

    # ---- arithmetic ----
    def __add__(self, o):
        return _binary(self, o, "+", C._add_tensor, C._add_scalar, C._add_broadcasted)

    def __radd__(self, o):
        return self + o

    def __sub__(self, o):
        return _binary(self, o, "-", C._sub_tensor, C._sub_scalar, C._sub_broadcasted)

    def __rsub__(self, o):
        return _binary(self, o, "-", C._sub_tensor, C._rsub_scalar)

    def __mul__(self, o):
        return _binary(self, o, "*", C._mul_tensor, C._mul_scalar, C._mul_broadcasted)

    def __rmul__(self, o):
        return self * o

    def __truediv__(self, o):
        return _binary(self, o, "/", C._truediv_tensor, C._truediv_scalar, C._truediv_broadcasted)

    def __rtruediv__(self, o):
        return _binary(self, o, "/", C._truediv_tensor, C._rtruediv_scalar)

    def __gt__(self, o):
        return _binary(self, o, ">", C._gt_tensor, C._gt_scalar)

    def __lt__(self, o):
        return _binary(self, o, "<", C._lt_tensor, C._lt_scalar)

    def __pow__(self, o):
        return _binary(self, o, "**", C._pow_tensor, C._pow_scalar)

    def __rpow__(self, o):
        return _binary(self, o, "**", C._pow_tensor, C._rpow_scalar)

    def __neg__(self):
        return Tensor._from_core(C._negate(self._core), self.shape)

    def __matmul__(self, other: Tensor) -> Tensor:
        if not isinstance(other, Tensor):
            raise TypeError(
                f"Unsupported operand type(s) for @: Tensor and '{type(other).__name__}'")
        if len(self.shape) < 2 or len(other.shape) < 2:
            raise ValueError(
                f"matmul requires at least 2D operands, got {self.shape} and {other.shape}")
        if self.shape[-1] != other.shape[-2]:
            raise ValueError(f"Shape mismatch: {self.shape} cannot multiply {other.shape}")
        n, k, m = self.shape[-2], self.shape[-1], other.shape[-1]
        if len(self.shape) == 2 and len(other.shape) == 2:
            return Tensor._from_core(C._matmul(self._core, other._core, n, m, k), (n, m))
        if self.shape[:-2] != other.shape[:-2]:
            raise ValueError("Batch dimensions must match for batched matmul: "
                             f"{self.shape} vs {other.shape}")
        lead = self.shape[:-2]
        core = C._matmul_batched(self._core, other._core, math.prod(lead), n, m, k)
        return Tensor._from_core(core, (*lead, n, m))

    # In-place operators recompute and adopt the result's buffer, so the same
    # Tensor object is updated (optimizers rely on it).
    def _adopt(self, other: Tensor) -> Tensor:
        self._core, self.shape, self.strides = other._core, other.shape, other.strides
        return self

    def __iadd__(self, o):
        return self._adopt(self + o)

    def __isub__(self, o):
        return self._adopt(self - o)

    def __imul__(self, o):
        return self._adopt(self * o)

    def __itruediv__(self, o):
        return self._adopt(self / o)


def _binary(a: Tensor, b, sym: str, tensor_op, scalar_op, bcast_op=None) -> Tensor:
    if isinstance(b, (int, float)):
        return Tensor._from_core(scalar_op(a._core, float(b)), a.shape)
    if isinstance(b, Tensor):
        if a.shape == b.shape:
            return Tensor._from_core(tensor_op(a._core, b._core), a.shape)
        if bcast_op is not None:
            shape, sa, sb = broadcast(a.shape, a.strides, b.shape, b.strides)
            return Tensor._from_core(bcast_op(a._core, b._core, shape, sa, sb), shape)
        raise ValueError(f"Operands with shapes {a.shape} and {b.shape} do not match, and "
                         f"operation '{sym}' does not support broadcasting.")
    raise TypeError(f"Unsupported operand type(s) for {sym}: Tensor and '{type(b).__name__}'")


def _need_tensor(a, name: str) -> None:
    if not isinstance(a, Tensor):
        raise TypeError(
            f"Ember operator ember.{name} doesn't support '{type(a).__name__}', only Tensors")


def _unary(a: Tensor, name: str, op) -> Tensor:
    _need_tensor(a, name)
    return Tensor._from_core(op(a._core), a.shape)


def _pairwise(a, b, name: str, tensor_op, scalar_op) -> Tensor:
    if isinstance(a, Tensor):
        return _binary(a, b, name, tensor_op, scalar_op)
    if isinstance(b, Tensor):
        return _binary(b, a, name, tensor_op, scalar_op)
    raise TypeError(f"ember.{name} needs one Tensor object. Got {type(a).__name__} and "
                    f"{type(b).__name__}")


def max(a, b) -> Tensor:  # noqa: A001 - the reference's name
    return _pairwise(a, b, "max()", C._max_tensor, C._max_scalar)


def min(a, b) -> Tensor:  # noqa: A001
    return _pairwise(a, b, "min()", C._min_tensor, C._min_scalar)


def exp(a: Tensor) -> Tensor:
    return _unary(a, "exp()", C._exponent)


def log(a: Tensor) -> Tensor:
    return _unary(a, "log()", C._log)


def sqrt(a: Tensor) -> Tensor:
    return _unary(a, "sqrt()", C._sqrt)


def sin(a: Tensor) -> Tensor:
    return _unary(a, "sin()", C._sin)


def cos(a: Tensor) -> Tensor:
    return _unary(a, "cos()", C._cos)


def tan(a: Tensor) -> Tensor:
    return _unary(a, "tan()", C._tan)


def ctg(a: Tensor) -> Tensor:
    return _unary(a, "ctg()", C._ctg)


def sinh(a: Tensor) -> Tensor:
    return _unary(a, "sinh()", C._sinh)


def cosh(a: Tensor) -> Tensor:
    return _unary(a, "cosh()", C._cosh)


def tanh(a: Tensor) -> Tensor:
    return _unary(a, "tanh()", C._tanh)


def ctgh(a: Tensor) -> Tensor:
    return _unary(a, "ctgh()", C._ctgh)


def T(a: Tensor) -> Tensor:
    _need_tensor(a, "T()")
    if len(a.shape) != 2:
        raise ValueError(f"You can only transpose 2D matrices, not {len(a.shape)}D")
    return Tensor._from_core(C._transpose(a._core, *a.shape), (a.shape[1], a.shape[0]))


def _axis(a: Tensor, axis: int) -> int:
    nd = len(a.shape)
    ax = axis + nd if axis < 0 else axis
    if not 0 <= ax < nd:
        raise ValueError(f"Axis {axis} out of bound for {nd} dim Tensor")
    return ax


def _reduced(shape, axis: int, keepdims: bool):
    if keepdims:
        return tuple(1 if i == axis else d for i, d in enumerate(shape))
    return tuple(d for i, d in enumerate(shape) if i != axis)


def sum(a: Tensor, axis: int | None = None, keepdims: bool = False):  # noqa: A001
    """Sum of all elements (a float) or along ``axis`` (a Tensor)."""
    _need_tensor(a, "sum()")
    if axis is None:
        return C._sum(a._core)
    ax = _axis(a, axis)
    return Tensor._from_core(C._sum_axis(a._core, a.shape, ax), _reduced(a.shape, ax, keepdims))


def amax(a: Tensor, axis: int, keepdims: bool = False) -> Tensor:
    """Maximum along ``axis`` (a reduction, unlike the element-wise ``max``)."""
    _need_tensor(a, "amax()")
    ax = _axis(a, axis)
    return Tensor._from_core(C._max_axis(a._core, a.shape, ax), _reduced(a.shape, ax, keepdims))


def softmax(a: Tensor, axis: int = -1) -> Tensor:
    """Softmax along ``axis``: shift by the max, exp, divide by the sum
    (``tensor.py:430-437``), fused into one device launch."""
    _need_tensor(a, "softmax()")
    ax = _axis(a, axis)
    return Tensor._from_core(C._softmax(a._core, a.shape, ax), a.shape)


# ---------------------------------------------------------------- attention


def _attention_shape(q: Tensor, k: Tensor, v: Tensor) -> tuple[int, int, int, int]:
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need_tensor(t, f"attention() {name}")
    if len(q.shape) not in (2, 3, 4):
        raise ValueError(f"attention expects (S, D), (H, S, D) or (B, H, S, D), got {q.shape}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes differ: {q.shape}, {k.shape}, {v.shape}")
    shape = (1,) * (4 - len(q.shape)) + q.shape
    return tuple(int(x) for x in shape)  # type: ignore[return-value]


def _scale(D: int, scale: float | None) -> float:
    return float(np.float32(1.0 / math.sqrt(D))) if scale is None else float(scale)


def attention_forward(q: Tensor, k: Tensor, v: Tensor, causal: bool = False,
                      scale: float | None = None) -> tuple[Tensor, Tensor]:
    """Fused attention forward: (O, LSE) with O shaped like q and LSE like q
    without its last dimension (natural-log logsumexp of the scaled scores).
    Causal: key j is visible to query i iff j <= i."""
    B, H, S, D = _attention_shape(q, k, v)
    o, lse = C._attention_fwd(q._core, k._core, v._core, B, H, S, D, _scale(D, scale), causal)
    return Tensor._from_core(o, q.shape), Tensor._from_core(lse, q.shape[:-1])


def attention(q: Tensor, k: Tensor, v: Tensor, causal: bool = False,
              scale: float | None = None) -> Tensor:
    """softmax(q k^T * scale + mask) v in one fused kernel (scale defaults to
    1/sqrt(D))."""
    return attention_forward(q, k, v, causal, scale)[0]


def attention_backward(q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, d_o: Tensor,
                       causal: bool = False, scale: float | None = None):
    """Gradients (dQ, dK, dV) of <O, dO>, recomputing the attention matrix
    from the forward's O and LSE."""
    B, H, S, D = _attention_shape(q, k, v)
    if o.shape != q.shape or d_o.shape != q.shape or lse.shape != q.shape[:-1]:
        raise ValueError("o, d_o must be shaped like q and lse like q without its last dim")
    dq, dk, dv = C._attention_bwd(q._core, k._core, v._core, o._core, lse._core, d_o._core,
                                  B, H, S, D, _scale(D, scale), causal)
    return tuple(Tensor._from_core(g, q.shape) for g in (dq, dk, dv))


def synchronize() -> None:
    """Waits for all queued device work."""
    C._synchronize()


def empty_cache() -> None:
    """Returns the device allocator's cached (freed) blocks and the library's
    scratch buffers to HIP; the next allocations call hipMalloc again.  Call
    it when no other thread is inside the library."""
    C._empty_cache()


def memory_stats() -> dict:
    """Bytes the device allocator has handed out (``in_use``), holds freed for
    reuse (``cached``) and the peak of ``in_use``, on the current device."""
    return C._memory_stats()
