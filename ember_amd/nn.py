"""Layers with manual backward, in the reference's ``ember.nn`` style.

``Layer`` has the interface of the reference's ABC (``ember/nn/base.py:7-35``):
``__call__(x, training)`` stores the input and output and calls ``forward``;
``backward(grad_y)`` returns the gradient with respect to the input and keeps
parameter gradients for ``gradients()``.

``Attention`` is the layer the reference lacks: fused scaled-dot-product
attention on the MI355X kernels.  Its input is the tuple ``(q, k, v)`` of
same-shaped Tensors ((S, D), (H, S, D) or (B, H, S, D)); ``backward`` returns
``(dq, dk, dv)``, recomputing the attention matrix from the forward's
logsumexp instead of storing it.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from itertools import chain

from ember_amd.tensor import Tensor, attention_backward, attention_forward


class Layer(ABC):
    x: object
    y: object

    def __call__(self, x, training: bool = True):
        self.x = x
        self._training = training
        self.y = self.forward(x, training)
        return self.y

    @abstractmethod
    def reset(self) -> None: ...

    @abstractmethod
    def parameters(self) -> list[Tensor]: ...

    @abstractmethod
    def gradients(self) -> list[Tensor | None]: ...

    @abstractmethod
    def forward(self, x, training: bool): ...

    @abstractmethod
    def backward(self, grad_y): ...


class Sequential(Layer):
    """Layers applied in order; backward runs them in reverse
    (``ember/nn/base.py:50-75``)."""

    def __init__(self, *layers: Layer):
        self.layers = layers
        self.x = self.y = None

    def reset(self) -> None:
        self.x = self.y = None
        for layer in self.layers:
            layer.reset()

    def forward(self, x, training: bool):
        for layer in self.layers:
            x = layer(x, training)
        return x

    def backward(self, grad_y):
        for layer in reversed(self.layers):
            grad_y = layer.backward(grad_y)
        return grad_y

    def parameters(self) -> list[Tensor]:
        return list(chain.from_iterable(layer.parameters() for layer in self.layers))

    def gradients(self) -> list[Tensor | None]:
        return list(chain.from_iterable(layer.gradients() for layer in self.layers))


class Attention(Layer):
    """softmax(q k^T * scale + mask) v; no parameters.  ``causal`` masks key
    j for query i unless j <= i; ``scale`` defaults to 1/sqrt(D)."""

    def __init__(self, causal: bool = False, scale: float | None = None):
        self.causal = causal
        self.scale = scale
        self.reset()

    def reset(self) -> None:
        self.x = self.y = None
        self.lse: Tensor | None = None

    def parameters(self) -> list[Tensor]:
        return []

    def gradients(self) -> list[Tensor | None]:
        return []

    def forward(self, x, training: bool) -> Tensor:
        q, k, v = x
        o, self.lse = attention_forward(q, k, v, self.causal, self.scale)
        return o

    def backward(self, grad_y: Tensor):
        if self.x is None or self.lse is None:
            raise RuntimeError("forward() must run before backward()")
        q, k, v = self.x
        return attention_backward(q, k, v, self.y, self.lse, grad_y, self.causal, self.scale)
