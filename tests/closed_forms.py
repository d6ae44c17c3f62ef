"""NumPy float64 closed forms of attention, written independently of the C
oracle so that they can pin it (and a finite-difference check pins them).

softmax(q k^T * scale + mask) v, its logsumexp, and the gradients of
<O, dO> w.r.t. q, k, v.  The causal mask keeps key j for query i iff j <= i.
"""

from __future__ import annotations

import numpy as np


def _scores(q, k, causal: bool, scale: float):
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    S = q.shape[-2]
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * float(scale)
    if causal:
        s = np.where(np.tril(np.ones((S, S), dtype=bool)), s, -np.inf)
    return s


def fwd(q, k, v, causal: bool, scale: float):
    s = _scores(q, k, causal, scale)
    mx = s.max(axis=-1, keepdims=True)
    e = np.exp(s - mx)
    l = e.sum(axis=-1, keepdims=True)
    o = np.matmul(e / l, np.asarray(v, dtype=np.float64))
    return o, (mx + np.log(l))[..., 0]


def bwd(q, k, v, d_o, causal: bool, scale: float):
    q, k, v, d_o = (np.asarray(x, dtype=np.float64) for x in (q, k, v, d_o))
    s = _scores(q, k, causal, scale)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    o = p @ v
    dv = np.swapaxes(p, -1, -2) @ d_o
    dp = d_o @ np.swapaxes(v, -1, -2)
    delta = (d_o * o).sum(axis=-1, keepdims=True)
    ds = p * (dp - delta)
    return scale * (ds @ k), scale * (np.swapaxes(ds, -1, -2) @ q), dv


def finite_difference_grads(q, k, v, d_o, causal: bool, scale: float, eps: float = 1e-6):
    """Central differences of f = <O(q, k, v), dO> in float64 (tiny shapes only)."""
    q, k, v, d_o = (np.array(x, dtype=np.float64) for x in (q, k, v, d_o))

    def f():
        return float((fwd(q, k, v, causal, scale)[0] * d_o).sum())

    grads = []
    for x in (q, k, v):
        g = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            old = x[idx]
            x[idx] = old + eps
            fp = f()
            x[idx] = old - eps
            fm = f()
            x[idx] = old
            g[idx] = (fp - fm) / (2 * eps)
        grads.append(g)
    return tuple(grads)


def layernorm(x, gamma, beta, eps):
    """float64 LayerNorm over the last axis (biased variance)."""
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * np.asarray(gamma, np.float64) + np.asarray(beta, np.float64)


def layernorm_grads_fd(x, gamma, beta, dy, eps, h=1e-6):
    """Central differences of f = <LayerNorm(x), dy> w.r.t. x, gamma, beta."""
    x, gamma, beta, dy = (np.array(a, np.float64) for a in (x, gamma, beta, dy))

    def f():
        return float((layernorm(x, gamma, beta, eps) * dy).sum())

    out = []
    for a in (x, gamma, beta):
        g = np.zeros_like(a)
        for idx in np.ndindex(*a.shape):
            old = a[idx]
            a[idx] = old + h
            fp = f()
            a[idx] = old - h
            fm = f()
            a[idx] = old
            g[idx] = (fp - fm) / (2 * h)
        out.append(g)
    return tuple(out)
