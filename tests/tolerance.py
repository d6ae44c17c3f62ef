"""Parity tolerances shared by the GPU tests and the CPU tests that pin them.

NORTH_STAR is the project's stated bar for every fp32 result of the hot path
(attention O / LSE / dQ / dK / dV and the GEMM): max-abs 2e-4 / rel 1e-3
against the CPU oracle, i.e. |got - ref| <= 2e-4 + 1e-3 |ref| elementwise.
gemm_error_bound is a second, order-free bound for GEMMs: it holds for any
fp32 summation order but is loose (about 0.5 at k = 4096 on U(-1,1)
operands), so on its own it cannot tell an fp32 GEMM from one whose operands
were rounded to bf16; tests/test_gemm_tolerance.py shows both facts on the
CPU.  GPU GEMM tests assert both.
"""

from __future__ import annotations

import numpy as np

NORTH_STAR = dict(rtol=1e-3, atol=2e-4)


def assert_north_star(got, ref, err_msg: str = "") -> None:
    """|got - ref| <= 2e-4 + 1e-3 |ref| everywhere (ref: the CPU oracle)."""
    np.testing.assert_allclose(got, ref, err_msg=err_msg, **NORTH_STAR)


def north_star_ratio(got, ref) -> float:
    """max |got - ref| / (2e-4 + 1e-3 |ref|): below 1 passes."""
    got64, ref64 = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(got64 - ref64) / (NORTH_STAR["atol"] + NORTH_STAR["rtol"] * np.abs(ref64))))


def gemm_error_bound(a, b):
    """Rigorous bound on |fl(a@b) - a@b| for any fp32 summation order of
    length k: gamma_k * (|a| @ |b|), gamma_k = k u / (1 - k u), u = 2^-24,
    doubled for the final rounding and margin."""
    k = a.shape[-1]
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    return 2.0 * gamma * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))) + 1e-30


def round_to_bf16(x):
    """x rounded to the nearest bfloat16 (ties to even), returned as float32:
    the operand precision of a bf16 GEMM, used to plant a precision loss."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)
