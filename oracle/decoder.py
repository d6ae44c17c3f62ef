"""float64 NumPy restatement of config 5's pre-LN decoder block, forward and
backward, as the checker of ``ember_amd.nn.DecoderBlock``.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Built from the same
definitions the C oracle pins: LayerNorm over the last axis (biased
variance), Ember's GELU 0.5*x*(1 + tanh(0.8x)) (ember/nn/activations.py:58)
and its backward (:65-66), Linear y = b + x @ w (ember/nn/layers.py:45-48)
and its backward (:50-56), causal softmax attention with scale 1/sqrt(D)
over heads of the packed (B, S, 3, H, D) projection.  The whole backward is
pinned by central finite differences in tests/test_oracle.py.

Block:  h = LN1(x);  x2 = x + Attn(h Wqkv + bqkv) Wo + bo
        y = x2 + GELU(LN2(x2) W1 + b1) W2 + b2
Parameter order: ln1.gamma, ln1.beta, Wqkv, bqkv, Wo, bo, ln2.gamma,
ln2.beta, W1, b1, W2, b2 (that of DecoderBlock.parameters()).
"""

from __future__ import annotations

import numpy as np

EPS = 1e-5
A = 0.8


def _ln(x, g, b):
    mu = x.mean(-1, keepdims=True)
    xc = x - mu
    rs = 1.0 / np.sqrt((xc * xc).mean(-1, keepdims=True) + EPS)
    xh = xc * rs
    return xh * g + b, (xh, rs)


def _ln_bwd(dy, g, cache):
    xh, rs = cache
    gg = dy * g
    dx = rs * (gg - gg.mean(-1, keepdims=True) - xh * (gg * xh).mean(-1, keepdims=True))
    return dx, (dy * xh).sum(0), dy.sum(0)


def _gelu(u):
    return 0.5 * u * (1.0 + np.tanh(A * u))


def _attn(qkv, B, S, H, causal):
    d3 = qkv.shape[1]
    D = d3 // (3 * H)
    t = qkv.reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)  # (3, B, H, S, D)
    q, k, v = t[0], t[1], t[2]
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(D)
    if causal:
        s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = p @ v                                                  # (B, H, S, D)
    return o.transpose(0, 2, 1, 3).reshape(B * S, H * D), (q, k, v, p, D)


def _attn_bwd(do, cache, B, S, H):
    q, k, v, p, D = cache
    do = do.reshape(B, S, H, D).transpose(0, 2, 1, 3)
    dv = p.transpose(0, 1, 3, 2) @ do
    dp = do @ v.transpose(0, 1, 3, 2)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    dq = ds @ k / np.sqrt(D)
    dk = ds.transpose(0, 1, 3, 2) @ q / np.sqrt(D)
    g = np.stack([dq, dk, dv])                                 # (3, B, H, S, D)
    return g.transpose(1, 3, 0, 2, 4).reshape(B * S, 3 * H * D)


def forward(params, x, B, S, H, causal=True):
    """Returns (y, cache) for x of shape (B*S, d), params in parameter order."""
    g1, be1, wqkv, bqkv, wo, bo, g2, be2, w1, b1, w2, b2 = (np.asarray(p, np.float64) for p in params)
    x = np.asarray(x, np.float64)
    h1, c1 = _ln(x, g1, be1)
    qkv = h1 @ wqkv + bqkv
    o, ca = _attn(qkv, B, S, H, causal)
    x2 = x + o @ wo + bo
    h2, c2 = _ln(x2, g2, be2)
    u = h2 @ w1 + b1
    a = _gelu(u)
    y = x2 + a @ w2 + b2
    return y, (x, h1, c1, qkv, o, ca, x2, h2, c2, u, a)


def backward(params, cache, dy, B, S, H):
    """Returns (dx, [grads in parameter order])."""
    g1, be1, wqkv, bqkv, wo, bo, g2, be2, w1, b1, w2, b2 = (np.asarray(p, np.float64) for p in params)
    x, h1, c1, qkv, o, ca, x2, h2, c2, u, a = cache
    dy = np.asarray(dy, np.float64)
    gw2, gb2 = a.T @ dy, dy.sum(0)
    da = dy @ w2.T
    t = np.tanh(A * u)
    du = da * ((1.0 + t) * (0.5 + A * (u - a)))
    gw1, gb1 = h2.T @ du, du.sum(0)
    dh2 = du @ w1.T
    dx2_ln, gg2, gbe2 = _ln_bwd(dh2, g2, c2)
    dx2 = dy + dx2_ln
    gwo, gbo = o.T @ dx2, dx2.sum(0)
    dqkv = _attn_bwd(dx2 @ wo.T, ca, B, S, H)
    gwqkv, gbqkv = h1.T @ dqkv, dqkv.sum(0)
    dx1_ln, gg1, gbe1 = _ln_bwd(dqkv @ wqkv.T, g1, c1)
    return dx2 + dx1_ln, [gg1, gbe1, gwqkv, gbqkv, gwo, gbo, gg2, gbe2, gw1, gb1, gw2, gb2]


def init_params(d, H, ratio, rng):
    """Random parameters (LayerNorm gains near 1) for tests."""
    def u(*s, a=0.3):
        return rng.uniform(-a, a, s)
    return [1 + u(d, a=0.1), u(d, a=0.1), u(d, 3 * d), u(3 * d, a=0.05), u(d, d), u(d, a=0.05),
            1 + u(d, a=0.1), u(d, a=0.1), u(d, ratio * d), u(ratio * d, a=0.05), u(ratio * d, d),
            u(d, a=0.05)]
