"""Losses (``ember/loss/losses.py``)."""

from __future__ import annotations

import math

from ember_amd.tensor import Tensor, sum as _sum


class MSELoss:
    """Mean squared error over all elements (``losses.py:9-26``):
    forward returns mean((pred - target)^2), backward (2/n)*(pred - target)."""

    def __init__(self) -> None:
        self.diff: Tensor | None = None
        self.n = 0

    def forward(self, pred: Tensor, target: Tensor) -> float:
        self.diff = pred - target
        self.n = math.prod(pred.shape)
        return _sum(self.diff * self.diff) / self.n

    def __call__(self, pred: Tensor, target: Tensor) -> float:
        return self.forward(pred, target)

    def backward(self) -> Tensor:
        if self.diff is None:
            raise RuntimeError("forward() must run before backward()")
        return (2.0 / self.n) * self.diff


__all__ = ["MSELoss"]
