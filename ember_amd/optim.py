"""Optimisers (``ember/optim``).

``Adam``, ``AdamW`` and ``SGD`` keep the reference's interfaces
(``ember/optim/adam.py:7-45``, ``adamw.py:7-56``, ``sgd.py:7-35``: the same
constructor arguments and defaults, ``parameters``, ``lr``, ``t``,
``means`` / ``variances`` or ``velocities``, ``apply(gradients)``) but run
one fused launch per step (per 48 parameters) instead of 3 to 15
element-wise operators per parameter.  Results are bit-identical to the
reference's update (``adam_step``, ``adamw_step``, ``sgd_step`` in
``include/ember_amd.h``).
"""

from __future__ import annotations

from ember_amd import _core as C
from ember_amd import random as _random
from ember_amd.tensor import Tensor


class Optimizer:
    parameters: list[Tensor]

    def apply(self, gradients: list[Tensor]) -> None:  # pragma: no cover - interface
        raise NotImplementedError


class Adam(Optimizer):
    def __init__(self, parameters: list[Tensor], lr: float = 0.001,
                 betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8):
        self.parameters = parameters
        self.lr = lr
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.t = 0
        self.means = [_random.zeros(p.shape) for p in parameters]
        self.variances = [_random.zeros(p.shape) for p in parameters]

    def apply(self, gradients: list[Tensor]) -> None:
        _check_gradients(self.parameters, gradients)
        self.t += 1
        C._adam_step([p._core for p in self.parameters], [g._core for g in gradients],
                     [m._core for m in self.means], [v._core for v in self.variances],
                     self.lr, self.beta1, self.beta2, self.eps, self.t)


class AdamW(Optimizer):
    """Adam with decoupled weight decay: ``p -= lr*wd*p`` before the Adam
    step (``ember/optim/adamw.py:7-56``)."""

    def __init__(self, parameters: list[Tensor], lr: float = 0.001,
                 betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.01):
        self.parameters = parameters
        self.lr = lr
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.weight_decay = weight_decay
        self.t = 0
        self.means = [_random.zeros(p.shape) for p in parameters]
        self.variances = [_random.zeros(p.shape) for p in parameters]

    def apply(self, gradients: list[Tensor]) -> None:
        _check_gradients(self.parameters, gradients)
        self.t += 1
        C._adamw_step([p._core for p in self.parameters], [g._core for g in gradients],
                      [m._core for m in self.means], [v._core for v in self.variances],
                      self.lr, self.beta1, self.beta2, self.eps, self.weight_decay, self.t)


class SGD(Optimizer):
    """Gradient descent with optional (Polyak) momentum: ``v = momentum*v + g``,
    ``p -= lr*v`` (``ember/optim/sgd.py:7-35``)."""

    def __init__(self, parameters: list[Tensor], lr: float = 0.01, momentum: float = 0.0):
        self.parameters = parameters
        self.lr = lr
        self.momentum = momentum
        self.velocities = [_random.zeros(p.shape) for p in parameters]

    def apply(self, gradients: list[Tensor]) -> None:
        _check_gradients(self.parameters, gradients)
        C._sgd_step([p._core for p in self.parameters], [g._core for g in gradients],
                    [v._core for v in self.velocities], self.lr, self.momentum)


def _check_gradients(parameters: list[Tensor], gradients: list[Tensor]) -> None:
    if len(gradients) != len(parameters):
        raise ValueError(f"Optimizer expected {len(parameters)} gradients, "
                         f"but got {len(gradients)}")
    for p, g in zip(parameters, gradients):
        if not isinstance(g, Tensor) or g.shape != p.shape:
            raise ValueError(f"gradient shape {getattr(g, 'shape', None)} does not match "
                             f"parameter shape {p.shape}")


__all__ = ["Optimizer", "Adam", "AdamW", "SGD"]
