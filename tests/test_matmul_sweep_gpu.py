"""A fixed-seed sweep of gemm_ex calls against float64: within the north-star
tolerance (max-abs 2e-4 / rel 1e-3) and within the order-free fp32 bound.

Each case draws the batch, n, m, k (tile-aligned or ragged, so every kernel
choice is met: the general kernel, the LDS-DMA kernel with 128- or 256-row
tiles, two k-groups per workgroup, split-K), which operand is stored
transposed, and the epilogue (bias, residual, GELU with the pre-activation
kept).  out and pre are checked on sampled rows: the product within
gamma_k |A||B| of the float64 one, the epilogue within fp32 rounding of
Ember's operator order.
"""

import numpy as np
import pytest

import gpu_helpers as G
from tolerance import assert_north_star

pytestmark = pytest.mark.gpu


def _dim(rng, unit, top):
    if rng.integers(0, 3):  # two in three aligned
        return int(unit * rng.integers(1, top // unit + 1))
    return int(rng.integers(1, top + 1))


def _case(seed):
    rng = np.random.default_rng(20_000 + seed)
    batch = int(rng.choice([1, 1, 1, 2, 3]))
    n, m = _dim(rng, 128, 1536), _dim(rng, 256, 1536)
    k = _dim(rng, 16, 2048) if rng.integers(0, 4) else int(rng.choice([1024, 2048, 4096]))
    ta, tb = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    bias, residual, act = bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), int(rng.integers(0, 2))
    return batch, n, m, k, ta, tb, bias, residual, act


def _gelu(x):
    x = x.astype(np.float32)
    return (x * np.float32(0.5)) * (np.tanh(x * np.float32(0.8)) + np.float32(1.0))


@pytest.mark.parametrize("seed", range(40))
def test_random_gemm_ex(seed):
    batch, n, m, k, ta, tb, has_bias, has_res, act = _case(seed)
    rng = np.random.default_rng(seed)
    lead = (batch,) if batch > 1 else ()
    a = rng.uniform(-1, 1, lead + ((k, n) if ta else (n, k))).astype(np.float32)
    b = rng.uniform(-1, 1, lead + ((m, k) if tb else (k, m))).astype(np.float32)
    bias = rng.uniform(-1, 1, m).astype(np.float32) if has_bias else None
    res = rng.uniform(-1, 1, lead + (n, m)).astype(np.float32) if has_res else None
    got = G.gemm_ex(a, b, ta=ta, tb=tb, bias=bias, residual=res, act=act)
    out, pre = got if act else (got, None)
    a3 = a.reshape((batch,) + a.shape[-2:])
    b3 = b.reshape((batch,) + b.shape[-2:])
    out3 = out.reshape(batch, n, m)
    pre3 = pre.reshape(batch, n, m) if act else None
    res3 = res.reshape(batch, n, m) if has_res else None
    rows = np.unique(np.concatenate([[0, n - 1], rng.choice(n, min(n, 48), replace=False)]))
    u = 2.0 ** -24
    for z in range(batch):
        A = (a3[z].T if ta else a3[z])[rows].astype(np.float64)
        B = (b3[z].T if tb else b3[z]).astype(np.float64)
        exact = A @ B
        bound = G.gemm_error_bound(A.astype(np.float32), B.astype(np.float32))
        add = exact + (bias.astype(np.float64) if has_bias else 0.0)
        bound = bound + 2 * u * np.abs(add)
        if act:
            np.testing.assert_array_less(np.abs(pre3[z][rows] - add), bound + 1e-30)
            assert_north_star(pre3[z][rows], add)
            want = _gelu(pre3[z][rows])
            if has_res:
                want = want + res3[z][rows]
            np.testing.assert_allclose(out3[z][rows], want, rtol=1e-5, atol=1e-6)
        else:
            if has_res:
                add = add + res3[z][rows]
                bound = bound + 2 * u * np.abs(add)
            np.testing.assert_array_less(np.abs(out3[z][rows] - add), bound + 1e-30)
            assert_north_star(out3[z][rows], add)
