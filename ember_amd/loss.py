"""Losses (``ember/loss/losses.py``)."""

from __future__ import annotations

import math
from abc import ABC, abstractmethod

from ember_amd import _core as C
from ember_amd.tensor import Tensor, amax, exp, log, sum as _sum


class Loss(ABC):
    """Base class (``ember/loss/base.py:6-22``): ``forward`` returns the scalar
    loss and keeps what ``backward`` needs; ``backward`` returns the gradient
    with respect to ``pred``."""

    def __call__(self, pred: Tensor, target: Tensor) -> float:
        return self.forward(pred, target)

    @abstractmethod
    def forward(self, pred: Tensor, target: Tensor) -> float: ...

    @abstractmethod
    def backward(self) -> Tensor: ...


class MSELoss(Loss):
    """Mean squared error over all elements (``losses.py:9-26``):
    forward returns mean((pred - target)^2), backward (2/n)*(pred - target).

    Equal shapes take one fused pass (``_mse_loss``) that returns the same
    float sum as ``sum(diff * diff)`` and the gradient ``(2/n) * diff`` bit
    for bit; broadcasting shapes compose the operators as the reference."""

    def __init__(self) -> None:
        self.diff: Tensor | None = None
        self.grad: Tensor | None = None
        self.n = 0

    def forward(self, pred: Tensor, target: Tensor) -> float:
        self.n = math.prod(pred.shape)
        if isinstance(pred, Tensor) and isinstance(target, Tensor) and pred.shape == target.shape:
            total, g = C._mse_loss(pred._core, target._core, 2.0 / self.n if self.n else 0.0)
            self.diff, self.grad = None, Tensor._from_core(g, pred.shape)
            return total / self.n
        self.grad = None
        self.diff = pred - target
        return _sum(self.diff * self.diff) / self.n

    def backward(self) -> Tensor:
        if self.grad is not None:
            return self.grad
        if self.diff is None:
            raise RuntimeError("forward() must run before backward()")
        return (2.0 / self.n) * self.diff


class CrossEntropyLoss(Loss):
    """Softmax cross-entropy over (batch, classes) logits against one-hot (or
    probability) targets, averaged over the batch (``losses.py:29-56``):
    forward -sum(target * log_softmax(pred)) / batch with the log-sum-exp
    shift; backward (softmax(pred) - target) / batch."""

    def __init__(self) -> None:
        self.probs: Tensor | None = None
        self.target: Tensor | None = None
        self.n = 0

    def forward(self, pred: Tensor, target: Tensor) -> float:
        self.n = pred.shape[0]
        self.target = target
        shifted = pred - amax(pred, axis=-1, keepdims=True)
        log_probs = shifted - log(_sum(exp(shifted), axis=-1, keepdims=True))
        self.probs = exp(log_probs)
        return -_sum(target * log_probs) / self.n

    def backward(self) -> Tensor:
        if self.probs is None or self.target is None:
            raise RuntimeError("forward() must run before backward()")
        return (self.probs - self.target) / self.n


__all__ = ["Loss", "MSELoss", "CrossEntropyLoss"]
