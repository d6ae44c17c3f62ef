"""CPU checkers for the attention / matmul hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, always as the checker and never as
the thing measured or shipped.  The product (``ember_amd``) never imports it.

Two libraries sit behind this module:

* ``liboracle.so`` -- this repository's C restatement (``ember_oracle.c``):
  Ember's FP64-accumulating ``matmul`` (reference ``src/tensor/
  operators_cpu.c:47-67``) and the build-defined attention forward/backward
  written in the same style.
* ``_ref/libember_ref.so`` -- the reference's own ``operators_cpu.c`` compiled
  in place by ``oracle/Makefile``.  ``ref_composed_attention_*`` below drive
  *those* functions in the order Ember's Python front-end would
  (``ember/tensor/tensor.py:163-197`` for ``@``, ``:376-384`` for ``T``,
  ``:430-437`` for ``softmax``; broadcast strides as in
  ``ember/tensor/tensor_utils.py:97-140``), which is "attention as Ember can
  express it today".  It is optional: absent when the reference checkout is.
"""

from __future__ import annotations

import ctypes as C
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_ORACLE_SO = os.path.join(_HERE, "liboracle.so")
_REF_SO = os.path.join(_HERE, "_ref", "libember_ref.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = C.c_int64

_lib = None
_ref = None


def build(reference_root: str = "/root/reference") -> None:
    """Compile liboracle.so, and _ref/ when the reference checkout exists."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)
    if os.path.isdir(os.path.join(reference_root, "src", "tensor")):
        subprocess.run(["make", "-s", "-B", "-C", _HERE, "ref", f"REF={reference_root}"], check=True)
        # The reference's own bindings linked against libember_amd.so (the
        # executed drop-in check of tests/test_reference_binding_gpu.py).
        if os.path.isdir(os.path.join(reference_root, "src", "random")):
            subprocess.run(["make", "-s", "-B", "-C", _HERE, "link-check", f"REF={reference_root}"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_ORACLE_SO):
            build()
        L = C.CDLL(_ORACLE_SO)
        L.oracle_matmul.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.oracle_matmul_mt.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.oracle_matmul_batched.argtypes = [_f32p, _f32p, _f32p] + [C.c_int] * 4
        L.oracle_transpose.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
        L.oracle_attention_fwd.argtypes = [_f32p] * 5 + [_i64] * 4 + [C.c_float, C.c_int] + [_i64] * 6
        L.oracle_attention_fwd.restype = C.c_int
        L.oracle_attention_bwd.argtypes = [_f32p] * 9 + [_i64] * 4 + [C.c_float, C.c_int] + [_i64] * 6
        L.oracle_attention_bwd.restype = C.c_int
        L.oracle_adam_step.argtypes = [_f32p] * 4 + [_i64] + [C.c_double] * 4 + [_i64]
        L.oracle_adamw_step.argtypes = [_f32p] * 4 + [_i64] + [C.c_double] * 5 + [_i64]
        L.oracle_sgd_step.argtypes = [_f32p] * 3 + [_i64] + [C.c_double] * 2
        L.oracle_layernorm_fwd.argtypes = [_f32p] * 6 + [_i64, _i64, C.c_float]
        L.oracle_layernorm_bwd.argtypes = [_f32p] * 8 + [_i64, _i64]
        L.oracle_gelu_fwd.argtypes = [_f32p, _f32p, _i64]
        L.oracle_gelu_bwd.argtypes = [_f32p] * 4 + [_i64]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(_REF_SO)


def ref_lib() -> C.CDLL:
    """The reference's operators_cpu.c, compiled in place (see Makefile)."""
    global _ref
    if _ref is None:
        if not os.path.exists(_REF_SO):
            raise FileNotFoundError(f"{_REF_SO} not built (needs the reference checkout)")
        L = C.CDLL(_REF_SO)
        L.matmul.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.matmul_batched.argtypes = [_f32p, _f32p, _f32p] + [C.c_int] * 4
        L.transpose.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
        for name in ("sum_axis", "max_axis"):
            getattr(L, name).argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int]
        for name in ("add_tensor", "sub_tensor", "mul_tensor", "truediv_tensor"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, C.c_int]
        for name in ("mul_scalar", "add_scalar", "truediv_scalar"):
            getattr(L, name).argtypes = [_f32p, C.c_float, _f32p, C.c_int]
        for name in ("exponent_tensor", "sqrt_tensor", "tanh_tensor"):
            getattr(L, name).argtypes = [_f32p, _f32p, C.c_int]
        for name in ("sub_broadcasted", "truediv_broadcasted", "mul_broadcasted", "add_broadcasted"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _i32p, _i32p, _i32p, C.c_int]
        _ref = L
    return _ref


def default_scale(d: int) -> float:
    """fp32(1/sqrt(D)), the softmax scale every config uses."""
    return float(np.float32(1.0 / math.sqrt(d)))


# ---------------------------------------------------------------- restatement


def matmul(a: np.ndarray, b: np.ndarray, threads: bool = False) -> np.ndarray:
    """Ember's CPU matmul semantics (FP64 accumulation, one cast per output)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    n, k = a.shape
    k2, m = b.shape
    assert k == k2
    out = np.empty((n, m), dtype=np.float32)
    (lib().oracle_matmul_mt if threads else lib().oracle_matmul)(a, b, out, n, m, k)
    return out


def _strides4(shape):
    B, H, S, D = shape
    return (H * S * D, S * D, D)


def attention_fwd(q, k, v, causal: bool, scale: float | None = None):
    """(B,H,S,D) contiguous fp32 -> (O (B,H,S,D), LSE (B,H,S))."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    B, H, S, D = q.shape
    scale = default_scale(D) if scale is None else scale
    o = np.empty_like(q)
    lse = np.empty((B, H, S), dtype=np.float32)
    st = _strides4(q.shape)
    rc = lib().oracle_attention_fwd(q, k, v, o, lse, B, H, S, D, scale, int(causal), *st, *st)
    assert rc == 0
    return o, lse


def attention_bwd(q, k, v, o, lse, d_o, causal: bool, scale: float | None = None):
    """Gradients (dQ, dK, dV) of <O, dO>, recomputing P from the given LSE."""
    q, k, v, o, d_o = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, o, d_o))
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    B, H, S, D = q.shape
    scale = default_scale(D) if scale is None else scale
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    st = _strides4(q.shape)
    rc = lib().oracle_attention_bwd(q, k, v, o, lse, d_o, dq, dk, dv, B, H, S, D, scale,
                                    int(causal), *st, *st)
    assert rc == 0
    return dq, dk, dv


# ------------------------------------------- the reference's own ops, composed


def _bcast(shape_a, shape_b):
    """Output shape and strides exactly as tensor_utils.calculate_broadcast."""
    def contig(shape):
        st, cur = [0] * len(shape), 1
        for i in range(len(shape) - 1, -1, -1):
            st[i] = cur
            cur *= shape[i]
        return st
    sa, sb = contig(shape_a), contig(shape_b)
    out, oa, ob = [], [], []
    for da, xa, db, xb in zip(shape_a, sa, shape_b, sb):
        if da == db:
            out.append(da); oa.append(xa); ob.append(xb)
        elif da == 1:
            out.append(db); oa.append(0); ob.append(xb)
        else:
            out.append(da); oa.append(xa); ob.append(0)
    return [np.asarray(x, dtype=np.int32) for x in (out, oa, ob)]


def _ref_softmax_rows(R, x: np.ndarray) -> np.ndarray:
    """em.softmax(x, axis=-1) on an (n, m) tensor: amax -> sub -> exp -> sum -> div."""
    n, m = x.shape
    mx = np.empty((n, 1), dtype=np.float32)
    R.max_axis(x, mx, n, 1, m)
    shp, sa, sb = _bcast((n, m), (n, 1))
    shifted = np.empty((n, m), dtype=np.float32)
    R.sub_broadcasted(x, mx, shifted, shp, sa, sb, 2)
    e = np.empty((n, m), dtype=np.float32)
    R.exponent_tensor(shifted, e, n * m)
    s = np.empty((n, 1), dtype=np.float32)
    R.sum_axis(e, s, n, 1, m)
    out = np.empty((n, m), dtype=np.float32)
    R.truediv_broadcasted(e, s, out, shp, sa, sb, 2)
    return out


def _as3(x: np.ndarray, axis: int):
    """(outer, L, inner) view of a C-contiguous float32 array around `axis`."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    outer = int(np.prod(x.shape[:axis], dtype=np.int64))
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    return x.reshape(outer, x.shape[axis], inner), outer, inner


def ref_axis_reduce(x: np.ndarray, axis: int, kind: str) -> np.ndarray:
    """The reference's sum_axis / max_axis (operators_cpu.c:92-120) over
    `axis` (keepdims shape)."""
    R = ref_lib()
    x3, outer, inner = _as3(x, axis)
    out = np.empty((outer, 1, inner), dtype=np.float32)
    getattr(R, kind + "_axis")(x3, out, outer, inner, x3.shape[1])
    shape = list(x.shape)
    shape[axis] = 1
    return out.reshape(shape)


def ref_softmax(x: np.ndarray, axis: int) -> np.ndarray:
    """em.softmax(x, axis) through the reference's own CPU operators:
    max_axis -> sub_broadcasted -> exponent_tensor -> sum_axis ->
    truediv_broadcasted (ember/tensor/tensor.py:430-437)."""
    R = ref_lib()
    x3, outer, inner = _as3(x, axis)
    L = x3.shape[1]
    mx = np.empty((outer, 1, inner), dtype=np.float32)
    R.max_axis(x3, mx, outer, inner, L)
    shp, sa, sb = _bcast(x3.shape, mx.shape)
    shifted = np.empty_like(x3)
    R.sub_broadcasted(x3, mx, shifted, shp, sa, sb, 3)
    e = np.empty_like(x3)
    R.exponent_tensor(shifted, e, x3.size)
    s = np.empty((outer, 1, inner), dtype=np.float32)
    R.sum_axis(e, s, outer, inner, L)
    out = np.empty_like(x3)
    R.truediv_broadcasted(e, s, out, shp, sa, sb, 3)
    return out.reshape(x.shape)


def _ref_mm(R, a, b):
    n, k = a.shape
    m = b.shape[1]
    out = np.empty((n, m), dtype=np.float32)
    R.matmul(np.ascontiguousarray(a), np.ascontiguousarray(b), out, n, m, k)
    return out


def _ref_T(R, a):
    n, m = a.shape
    out = np.empty((m, n), dtype=np.float32)
    R.transpose(np.ascontiguousarray(a), out, n, m)
    return out


def _mask(S: int, causal: bool) -> np.ndarray:
    if not causal:
        return np.zeros((S, S), dtype=np.float32)
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    return np.where(j <= i, 0.0, -np.inf).astype(np.float32)


def ref_composed_attention_head(qh, kh, vh, doh, causal: bool, scale: float, backward: bool):
    """One head through the reference's own CPU ops, the way Ember composes it.

    Forward: ``p = softmax(q @ T(k) * scale + mask); o = p @ v``.  Backward,
    written with the same ops: ``dV = T(p) @ dO``, ``dP = dO @ T(v)``,
    ``dS = p * (dP - rowsum(dO * o))``, ``dQ = (dS @ k) * scale``,
    ``dK = (T(dS) @ q) * scale``.  Returns (o, p) or (o, dq, dk, dv).
    """
    R = ref_lib()
    S, D = qh.shape
    qh, kh, vh = (np.ascontiguousarray(x, dtype=np.float32) for x in (qh, kh, vh))
    s = _ref_mm(R, qh, _ref_T(R, kh))
    s2 = np.empty_like(s)
    R.mul_scalar(s, np.float32(scale), s2, S * S)
    s3 = np.empty_like(s)
    R.add_tensor(s2, _mask(S, causal), s3, S * S)
    p = _ref_softmax_rows(R, s3)
    o = _ref_mm(R, p, vh)
    if not backward:
        return o, p
    doh = np.ascontiguousarray(doh, dtype=np.float32)
    dv = _ref_mm(R, _ref_T(R, p), doh)
    dp = _ref_mm(R, doh, _ref_T(R, vh))
    prod = np.empty_like(o)
    R.mul_tensor(doh, o, prod, S * D)
    delta = np.empty((S, 1), dtype=np.float32)
    R.sum_axis(prod, delta, S, 1, D)
    shp, sa, sb = _bcast((S, S), (S, 1))
    dpm = np.empty_like(dp)
    R.sub_broadcasted(dp, delta, dpm, shp, sa, sb, 2)
    ds = np.empty_like(dp)
    R.mul_tensor(p, dpm, ds, S * S)
    dq0 = _ref_mm(R, ds, kh)
    dq = np.empty_like(dq0)
    R.mul_scalar(dq0, np.float32(scale), dq, S * D)
    dk0 = _ref_mm(R, _ref_T(R, ds), qh)
    dk = np.empty_like(dk0)
    R.mul_scalar(dk0, np.float32(scale), dk, S * D)
    return o, dq, dk, dv


# ------------------------------------------------------------------ Adam


def adam_step(p, g, m, v, lr, beta1, beta2, eps, t):
    """In-place Adam step on float32 arrays p, m, v with gradient g, the way
    Ember's Adam.apply computes it (ember/optim/adam.py:24-45)."""
    for x in (p, g, m, v):
        assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().oracle_adam_step(p, g, m, v, p.size, lr, beta1, beta2, eps, t)


def ref_composed_adam_step(p, g, m, v, lr, beta1, beta2, eps, t):
    """Returns (p, m, v) after one step run through the reference's own CPU
    operators in adam.py's order; each Python scalar is rounded to float32
    as the binding's "f" conversion does."""
    R = ref_lib()
    n = p.size
    f32 = np.float32

    def new():
        return np.empty(n, dtype=np.float32)

    def scal(fn, a, x):
        out = new()
        getattr(R, fn)(a, f32(x), out, n)
        return out

    def ten(fn, a, b):
        out = new()
        getattr(R, fn)(a, b, out, n)
        return out

    p, g, m, v = (np.ascontiguousarray(x, dtype=np.float32).reshape(-1) for x in (p, g, m, v))
    m = scal("mul_scalar", m, beta1)                                      # m *= beta1
    m = ten("add_tensor", m, scal("mul_scalar", g, 1 - beta1))            # m += (1-b1)*g
    v = scal("mul_scalar", v, beta2)                                      # v *= beta2
    v = ten("add_tensor", v, scal("mul_scalar", ten("mul_tensor", g, g), 1 - beta2))
    m_hat = scal("truediv_scalar", m, 1 - beta1 ** t)
    v_hat = scal("truediv_scalar", v, 1 - beta2 ** t)
    num = scal("mul_scalar", m_hat, lr)                                   # lr * m_hat
    sq = new()
    R.sqrt_tensor(v_hat, sq, n)
    den = scal("add_scalar", sq, eps)                                     # sqrt(v_hat) + eps
    p = ten("sub_tensor", p, ten("truediv_tensor", num, den))             # p -= num / den
    return p, m, v


def adamw_step(p, g, m, v, lr, beta1, beta2, eps, weight_decay, t):
    """In-place AdamW step, as Ember's AdamW.apply computes it
    (ember/optim/adamw.py:33-56)."""
    for x in (p, g, m, v):
        assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().oracle_adamw_step(p, g, m, v, p.size, lr, beta1, beta2, eps, weight_decay, t)


def sgd_step(p, g, v, lr, momentum):
    """In-place SGD (momentum) step, as Ember's SGD.apply computes it
    (ember/optim/sgd.py:25-35)."""
    for x in (p, g, v):
        assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().oracle_sgd_step(p, g, v, p.size, lr, momentum)


def _ref_ops(n):
    """(scal, ten, sqrt) runners of the reference's own CPU operators on
    float32 vectors of n elements; scalars rounded to float32 as the
    binding's "f" conversion does."""
    R = ref_lib()
    f32 = np.float32

    def scal(fn, a, x):
        out = np.empty(n, dtype=np.float32)
        getattr(R, fn)(a, f32(x), out, n)
        return out

    def ten(fn, a, b):
        out = np.empty(n, dtype=np.float32)
        getattr(R, fn)(a, b, out, n)
        return out

    def sqrt(a):
        out = np.empty(n, dtype=np.float32)
        R.sqrt_tensor(a, out, n)
        return out

    return scal, ten, sqrt


def ref_composed_adamw_step(p, g, m, v, lr, beta1, beta2, eps, weight_decay, t):
    """(p, m, v) after one AdamW step run through the reference's CPU
    operators in adamw.py's order (:45-56)."""
    p, g, m, v = (np.ascontiguousarray(x, dtype=np.float32).reshape(-1) for x in (p, g, m, v))
    scal, ten, sqrt = _ref_ops(p.size)
    m = scal("mul_scalar", m, beta1)
    m = ten("add_tensor", m, scal("mul_scalar", g, 1 - beta1))
    v = scal("mul_scalar", v, beta2)
    v = ten("add_tensor", v, scal("mul_scalar", ten("mul_tensor", g, g), 1 - beta2))
    m_hat = scal("truediv_scalar", m, 1 - beta1 ** t)
    v_hat = scal("truediv_scalar", v, 1 - beta2 ** t)
    p = ten("sub_tensor", p, scal("mul_scalar", p, lr * weight_decay))   # p -= lr*wd*p
    num = scal("mul_scalar", m_hat, lr)
    den = scal("add_scalar", sqrt(v_hat), eps)
    p = ten("sub_tensor", p, ten("truediv_tensor", num, den))
    return p, m, v


def ref_composed_sgd_step(p, g, v, lr, momentum):
    """(p, v) after one SGD step run through the reference's CPU operators in
    sgd.py's order (:33-35)."""
    p, g, v = (np.ascontiguousarray(x, dtype=np.float32).reshape(-1) for x in (p, g, v))
    scal, ten, _ = _ref_ops(p.size)
    v = scal("mul_scalar", v, momentum)
    v = ten("add_tensor", v, g)
    p = ten("sub_tensor", p, scal("mul_scalar", v, lr))
    return p, v


# --------------------------------------------- LayerNorm, GELU (block pieces)


def _f32c(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def layernorm_fwd(x, gamma, beta, eps=1e-5):
    """(y, mean, rstd) of LayerNorm over the last axis, FP64 inside."""
    x, gamma, beta = _f32c(x), _f32c(gamma), _f32c(beta)
    d = x.shape[-1]
    rows = x.size // d
    y = np.empty_like(x)
    mean = np.empty(x.shape[:-1], np.float32)
    rstd = np.empty(x.shape[:-1], np.float32)
    lib().oracle_layernorm_fwd(x, gamma, beta, y, mean, rstd, rows, d, eps)
    return y, mean, rstd


def layernorm_bwd(x, gamma, mean, rstd, dy):
    """(dx, dgamma, dbeta) from the forward's mean / rstd, FP64 inside."""
    x, gamma, mean, rstd, dy = (_f32c(a) for a in (x, gamma, mean, rstd, dy))
    d = x.shape[-1]
    dx = np.empty_like(x)
    dg = np.empty(d, np.float32)
    db = np.empty(d, np.float32)
    lib().oracle_layernorm_bwd(x, gamma, mean, rstd, dy, dx, dg, db, x.size // d, d)
    return dx, dg, db


def gelu_fwd(x):
    x = _f32c(x)
    y = np.empty_like(x)
    lib().oracle_gelu_fwd(x, y, x.size)
    return y


def gelu_bwd(dy, x, y):
    dy, x, y = _f32c(dy), _f32c(x), _f32c(y)
    dx = np.empty_like(x)
    lib().oracle_gelu_bwd(dy, x, y, dx, x.size)
    return dx


def ref_composed_gelu(x, dy):
    """Ember's GELU forward and backward (ember/nn/activations.py:56-66) run
    through the reference's own compiled operators, in Python's evaluation
    order.  Returns (y, dx)."""
    R = ref_lib()
    x, dy = _f32c(x).reshape(-1), _f32c(dy).reshape(-1)
    n = x.size
    f32 = np.float32

    def new():
        return np.empty(n, np.float32)

    def scal(fn, a, v):
        out = new()
        getattr(R, fn)(a, f32(v), out, n)
        return out

    def ten(fn, a, b):
        out = new()
        getattr(R, fn)(a, b, out, n)
        return out

    def tanh(a):
        out = new()
        R.tanh_tensor(a, out, n)
        return out

    # y = 0.5 * x * (1 + em.tanh(0.8 * x))
    y = ten("mul_tensor", scal("mul_scalar", x, 0.5), scal("add_scalar", tanh(scal("mul_scalar", x, 0.8)), 1.0))
    # grad_y * ((1.0 + em.tanh(a * x)) * (0.5 + a * (x - y)))
    t = scal("add_scalar", tanh(scal("mul_scalar", x, 0.8)), 1.0)
    r = scal("add_scalar", scal("mul_scalar", ten("sub_tensor", x, y), 0.8), 0.5)
    dx = ten("mul_tensor", dy, ten("mul_tensor", t, r))
    return y, dx
