"""Random and constant tensors (``ember/random/generators.py:5-23``): host
draws with the C library's rand(), one upload per tensor."""

from __future__ import annotations

from ember_amd import _core as C
from ember_amd.tensor import Tensor


def seed(value: int) -> None:
    """Seeds the generator ``uniform`` draws from."""
    C._seed(value)


def uniform(low: float, high: float, size: tuple[int, ...]) -> Tensor:
    return Tensor._from_core(C._uniform(low, high, tuple(size)), tuple(size))


def constant(value: float, size: tuple[int, ...]) -> Tensor:
    return Tensor._from_core(C._constant(value, tuple(size)), tuple(size))


def zeros(size: tuple[int, ...]) -> Tensor:
    return constant(0.0, size)


def ones(size: tuple[int, ...]) -> Tensor:
    return constant(1.0, size)


__all__ = ["seed", "uniform", "constant", "zeros", "ones"]
