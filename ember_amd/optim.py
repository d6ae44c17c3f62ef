"""Optimisers (``ember/optim``).

``Adam`` keeps the reference's interface (``ember/optim/adam.py:7-45``:
``parameters``, ``lr``, ``beta1``/``beta2``, ``eps``, ``t``, ``means``,
``variances``, ``apply(gradients)``) but runs one fused launch per step
(per 48 parameters) instead of 13 element-wise operators per parameter.
Results are bit-identical to the reference's update (see ``adam_step`` in
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
        if len(gradients) != len(self.parameters):
            raise ValueError(f"Optimizer expected {len(self.parameters)} gradients, "
                             f"but got {len(gradients)}")
        for p, g in zip(self.parameters, gradients):
            if not isinstance(g, Tensor) or g.shape != p.shape:
                raise ValueError(f"gradient shape {getattr(g, 'shape', None)} does not match "
                                 f"parameter shape {p.shape}")
        self.t += 1
        C._adam_step([p._core for p in self.parameters], [g._core for g in gradients],
                     [m._core for m in self.means], [v._core for v in self.variances],
                     self.lr, self.beta1, self.beta2, self.eps, self.t)


__all__ = ["Optimizer", "Adam"]
