"""CPU check that the GEMM parity assertions discriminate.

The GPU GEMM tests assert the north-star tolerance (max-abs 2e-4 / rel 1e-3
against the FP64-accumulating oracle, Ember's operators_cpu.c:47-60) besides
the order-free bound gamma_k |A||B|.  Here, on config 4's 4096^3 operands
(U(-1,1), the seeds the GPU test uses), on sampled rows:
  * an fp32 product (numpy's float32 matmul, fp32 accumulation like the GPU
    kernel) passes both;
  * the same product with operands rounded to bfloat16 -- a plausible
    precision regression -- passes the order-free bound (which is why that
    bound alone was not enough) and fails the north-star assertion.
"""

import numpy as np
import pytest

import oracle
from tolerance import assert_north_star, gemm_error_bound, north_star_ratio, round_to_bf16


def _u(shape, seed):
    return np.random.default_rng(seed).uniform(-1, 1, shape).astype(np.float32)


@pytest.fixture(scope="module")
def config4_rows():
    n = k = m = 4096
    a, b = _u((n, k), 7), _u((k, m), 8)
    rows = np.random.default_rng(9).choice(n, 24, replace=False)
    exact = oracle.matmul(a[rows], b, threads=True)
    return a[rows], b, exact


def test_round_to_bf16_keeps_8_bits_of_mantissa():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 2 ** -7, 1.0 + 3 * 2 ** -9, -3.140625, 1e-30], np.float32)
    y = round_to_bf16(x)
    assert y[0] == 1.0 and y[1] == 1.0                 # tie -> even
    assert y[2] == np.float32(1.0 + 2 ** -7)           # representable
    assert y[3] == np.float32(1.0 + 2 ** -7)           # rounds up
    assert y[4] == np.float32(-3.140625)
    assert (y.view(np.uint32) & 0xFFFF == 0).all()


def test_fp32_gemm_passes_both_checks(config4_rows):
    a, b, exact = config4_rows
    got = a @ b                                         # float32 BLAS, fp32 accumulation
    assert (np.abs(got.astype(np.float64) - exact) <= gemm_error_bound(a, b)).all()
    assert_north_star(got, exact)
    assert north_star_ratio(got, exact) < 0.5


def test_bf16_operands_pass_the_loose_bound_but_fail_the_north_star(config4_rows):
    a, b, exact = config4_rows
    planted = (round_to_bf16(a).astype(np.float64) @ round_to_bf16(b).astype(np.float64)).astype(np.float32)
    err = np.abs(planted.astype(np.float64) - exact)
    assert (err <= gemm_error_bound(a, b)).all()        # the old check alone is blind to it
    assert north_star_ratio(planted, exact) > 10
    with pytest.raises(AssertionError):
        assert_north_star(planted, exact)
