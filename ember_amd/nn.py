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

import math
from abc import ABC, abstractmethod
from itertools import chain

from ember_amd import _core as C
from ember_amd import random as _random
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


def _rows(x: Tensor) -> tuple[int, int]:
    if len(x.shape) != 2:
        raise ValueError(f"expected a 2-D (rows, features) Tensor, got {x.shape}")
    return x.shape


def linear(x: Tensor, w: Tensor, b: Tensor | None = None, residual: Tensor | None = None,
           gelu: bool = False) -> tuple[Tensor, Tensor | None]:
    """``act(x @ w + b) + residual`` in one GEMM with a fused epilogue; returns
    (y, pre) where pre = x @ w + b is kept only when ``gelu`` (its backward
    needs it)."""
    n, k = _rows(x)
    k2, m = _rows(w)
    if k != k2:
        raise ValueError(f"Shape mismatch: {x.shape} cannot multiply {w.shape}")
    y, pre = C._linear(x._core, w._core, None if b is None else b._core,
                       None if residual is None else residual._core, n, m, k, 1 if gelu else 0, gelu)
    return Tensor._from_core(y, (n, m)), (Tensor._from_core(pre, (n, m)) if pre is not None else None)


def weight_grad(x: Tensor, grad_y: Tensor) -> Tensor:
    """x^T @ grad_y (in x out) for x (rows, in), grad_y (rows, out), reading x
    transposed in place (Ember's ``em.T(x) @ grad_y``, ``layers.py:53``)."""
    rows, n = _rows(x)
    rows2, m = _rows(grad_y)
    if rows != rows2:
        raise ValueError(f"Shape mismatch: {x.shape} and {grad_y.shape}")
    return Tensor._from_core(C._gemm(x._core, grad_y._core, 1, n, m, rows, True, False, None, None),
                             (n, m))


def input_grad(grad_y: Tensor, w: Tensor, residual: Tensor | None = None) -> Tensor:
    """grad_y @ w^T (+ residual) for w (in, out), reading w transposed in place
    (Ember's ``grad_y @ em.T(self.w)``, ``layers.py:55``)."""
    rows, m_out = _rows(grad_y)
    n_in, m_out2 = _rows(w)
    if m_out != m_out2:
        raise ValueError(f"Shape mismatch: {grad_y.shape} and {w.shape}")
    return Tensor._from_core(
        C._gemm(grad_y._core, w._core, 1, rows, n_in, m_out, False, True, None,
                None if residual is None else residual._core), (rows, n_in))


def col_sum(x: Tensor) -> Tensor:
    """Column sums of a 2-D Tensor (a Linear layer's bias gradient)."""
    n, m = _rows(x)
    return Tensor._from_core(C._col_sum(x._core, n, m), (m,))


class Linear(Layer):
    """y = b + x @ w (``ember/nn/layers.py:9-56``), x of shape (rows, in).
    ``activation="gelu"`` fuses Ember's GELU into the GEMM epilogue.  Weights
    start U(+-1/sqrt(in)), biases 0, as the reference's ``reset``."""

    def __init__(self, in_features: int, out_features: int, activation: str | None = None):
        if activation not in (None, "gelu"):
            raise ValueError(f"unsupported activation {activation!r}")
        self.in_features = in_features
        self.out_features = out_features
        self.activation = activation
        self.reset()

    def reset(self) -> None:
        self.x = self.y = self.pre = None
        scale = 1.0 / math.sqrt(self.in_features)
        self.w = _random.uniform(-scale, scale, (self.in_features, self.out_features))
        self.b = _random.zeros((self.out_features,))
        self.grad_w = self.grad_b = None

    def parameters(self) -> list[Tensor]:
        return [self.w, self.b]

    def gradients(self) -> list[Tensor | None]:
        return [self.grad_w, self.grad_b]

    def forward(self, x: Tensor, training: bool = True, residual: Tensor | None = None) -> Tensor:
        self.x = x
        y, self.pre = linear(x, self.w, self.b, residual, self.activation == "gelu")
        return y

    def backward(self, grad_y: Tensor) -> Tensor:
        if self.x is None:
            raise RuntimeError("forward() must run before backward()")
        if self.activation == "gelu":
            # The GELU output is recomputed from the pre-activation in the
            # kernel (bit-identical to the forward's); the bias gradient is
            # summed in the same pass.
            n, m = _rows(grad_y)
            g_core, b_core = C._gelu_bwd_col_sum(grad_y._core, self.pre._core, n, m)
            grad_y = Tensor._from_core(g_core, grad_y.shape)
            self.grad_b = Tensor._from_core(b_core, (m,))
        else:
            self.grad_b = col_sum(grad_y)
        self.grad_w = weight_grad(self.x, grad_y)
        return input_grad(grad_y, self.w)


class Activation(Layer):
    """A parameter-free element-wise layer (``ember/nn/base.py:38-47``); its
    ``forward`` keeps x and y for ``backward``, so it may be called directly
    as well as through ``__call__``."""

    def __init__(self) -> None:
        self.reset()

    def reset(self) -> None:
        self.x = self.y = None

    def parameters(self) -> list[Tensor]:
        return []

    def gradients(self) -> list[Tensor | None]:
        return []

    def _need_forward(self) -> None:
        if self.y is None:
            raise RuntimeError("forward() must run before backward()")


class ReLU(Activation):
    """max(x, 0); backward grad * (y > 0) (``ember/nn/activations.py:7-19``)."""

    def forward(self, x: Tensor, training: bool = True) -> Tensor:
        from ember_amd.tensor import max as em_max
        self.x = x
        self.y = em_max(x, 0)
        return self.y

    def backward(self, grad_y: Tensor) -> Tensor:
        self._need_forward()
        return grad_y * (self.y > 0.0)


class Sigmoid(Activation):
    """1 / (1 + exp(-x)); backward grad * (y * (1 - y))
    (``ember/nn/activations.py:22-34``)."""

    def forward(self, x: Tensor, training: bool = True) -> Tensor:
        from ember_amd.tensor import exp
        self.x = x
        self.y = 1.0 / (1.0 + exp(-x))
        return self.y

    def backward(self, grad_y: Tensor) -> Tensor:
        self._need_forward()
        return grad_y * (self.y * (1.0 - self.y))


class Tanh(Activation):
    """tanh(x); backward grad * (1 - y*y) (``ember/nn/activations.py:37-49``)."""

    def forward(self, x: Tensor, training: bool = True) -> Tensor:
        from ember_amd.tensor import tanh
        self.x = x
        self.y = tanh(x)
        return self.y

    def backward(self, grad_y: Tensor) -> Tensor:
        self._need_forward()
        return grad_y * (1 - self.y * self.y)


class Dropout(Layer):
    """Inverted dropout (``ember/nn/layers.py:59-97``): in training, keep
    each element where a uniform(0, 1) draw exceeds p and scale the kept ones
    by 1/(1-p); identity otherwise.  The mask comes from the library's
    seeded generator (``ember_amd.random``)."""

    def __init__(self, p: float):
        if not 0 <= p < 1:
            raise ValueError("p must be between 0 and 1 (exclusive of 1)")
        self.p = p
        self.scale = 1.0 / (1.0 - p)
        self.reset()

    def reset(self) -> None:
        self.x = self.y = self.mask = None

    def parameters(self) -> list[Tensor]:
        return []

    def gradients(self) -> list[Tensor | None]:
        return []

    def forward(self, x: Tensor, training: bool = True) -> Tensor:
        self.x = x
        if training:
            self.mask = _random.uniform(0.0, 1.0, x.shape) > self.p
            self.y = x * self.mask * self.scale
        else:
            self.y = x
        return self.y

    def backward(self, grad_y: Tensor) -> Tensor:
        if self.mask is None:
            raise RuntimeError("forward(training=True) must run before backward()")
        return grad_y * self.mask * self.scale


class GELU(Activation):
    """Ember's GELU, 0.5*x*(1 + tanh(0.8x)) (``ember/nn/activations.py:51-66``):
    the forward composed from element-wise operators as the reference does,
    the backward one fused kernel."""

    def forward(self, x: Tensor, training: bool = True) -> Tensor:
        from ember_amd.tensor import tanh
        self.x = x
        self.y = 0.5 * x * (1 + tanh(0.8 * x))
        return self.y

    def backward(self, grad_y: Tensor) -> Tensor:
        if self.x is None or self.y is None:
            raise RuntimeError("forward() must run before backward()")
        return Tensor._from_core(C._gelu_bwd(grad_y._core, self.x._core, self.y._core), grad_y.shape)


class LayerNorm(Layer):
    """LayerNorm over the last dimension: (x - mean)/sqrt(var + eps)*gamma + beta
    (biased variance); gamma = 1, beta = 0 at reset."""

    def __init__(self, features: int, eps: float = 1e-5):
        self.features = features
        self.eps = eps
        self.reset()

    def reset(self) -> None:
        self.x = self.y = None
        self.gamma = _random.ones((self.features,))
        self.beta = _random.zeros((self.features,))
        self.grad_gamma = self.grad_beta = None
        self._stats = None

    def parameters(self) -> list[Tensor]:
        return [self.gamma, self.beta]

    def gradients(self) -> list[Tensor | None]:
        return [self.grad_gamma, self.grad_beta]

    def forward(self, x: Tensor, training: bool = True) -> Tensor:
        d = x.shape[-1]
        rows = x.size // d
        y, mean, rstd = C._layernorm_fwd(x._core, self.gamma._core, self.beta._core, rows, d, self.eps)
        self._stats = (mean, rstd)
        return Tensor._from_core(y, x.shape)

    def backward(self, grad_y: Tensor, residual: Tensor | None = None) -> Tensor:
        """Gradient with respect to x; ``residual`` (the gradient reaching x
        through a skip connection) is added in the same pass."""
        if self.x is None or self._stats is None:
            raise RuntimeError("forward() must run before backward()")
        d = self.x.shape[-1]
        dx, dg, db = C._layernorm_bwd(self.x._core, self.gamma._core, *self._stats, grad_y._core,
                                      self.x.size // d, d,
                                      None if residual is None else residual._core)
        self.grad_gamma = Tensor._from_core(dg, (d,))
        self.grad_beta = Tensor._from_core(db, (d,))
        return Tensor._from_core(dx, self.x.shape)


def _xavier(fan_in: int, fan_out: int) -> Tensor:
    a = math.sqrt(6.0 / (fan_in + fan_out))
    return _random.uniform(-a, a, (fan_in, fan_out))


class DecoderBlock(Layer):
    """One pre-LN transformer decoder block on (B*S, d) token rows:
        h = LN1(x);  x2 = x + Attention(h Wqkv + bqkv) Wo + bo
        y = x2 + GELU(LN2(x2) W1 + b1) W2 + b2
    with causal fused attention reading the packed QKV projection in place.
    Weights Xavier-uniform, biases 0, LayerNorm gamma 1 / beta 0.  ``forward``
    takes (x, B, S); ``backward`` returns dx and fills ``gradients()``."""

    def __init__(self, d_model: int, n_heads: int, mlp_ratio: int = 4, causal: bool = True):
        if d_model % n_heads:
            raise ValueError("d_model must be a multiple of n_heads")
        self.d, self.h, self.r, self.causal = d_model, n_heads, mlp_ratio, causal
        self.reset()

    def reset(self) -> None:
        d, r = self.d, self.r
        self.ln1 = LayerNorm(d)
        self.ln2 = LayerNorm(d)
        self.w_qkv, self.b_qkv = _xavier(d, 3 * d), _random.zeros((3 * d,))
        self.w_o, self.b_o = _xavier(d, d), _random.zeros((d,))
        self.w_1, self.b_1 = _xavier(d, r * d), _random.zeros((r * d,))
        self.w_2, self.b_2 = _xavier(r * d, d), _random.zeros((d,))
        self._grads: list[Tensor | None] = [None] * 12
        self.x = self.y = None
        self._saved = None

    def parameters(self) -> list[Tensor]:
        return [self.ln1.gamma, self.ln1.beta, self.w_qkv, self.b_qkv, self.w_o, self.b_o,
                self.ln2.gamma, self.ln2.beta, self.w_1, self.b_1, self.w_2, self.b_2]

    def gradients(self) -> list[Tensor | None]:
        return list(self._grads)

    def __call__(self, x: Tensor, B: int, S: int, training: bool = True) -> Tensor:
        self.x = x
        self.y = self.forward((x, B, S), training)
        return self.y

    def forward(self, xbs, training: bool = True) -> Tensor:
        x, B, S = xbs
        D = self.d // self.h
        scale = float(1.0 / math.sqrt(D))
        self.ln1.x = x
        h1 = self.ln1.forward(x)
        qkv, _ = linear(h1, self.w_qkv, self.b_qkv)
        o_core, lse = C._attention_fwd_packed(qkv._core, B, S, self.h, D, scale, self.causal)
        o = Tensor._from_core(o_core, (B * S, self.d))
        x2, _ = linear(o, self.w_o, self.b_o, residual=x)
        self.ln2.x = x2
        h2 = self.ln2.forward(x2)
        a, u = linear(h2, self.w_1, self.b_1, gelu=True)
        y, _ = linear(a, self.w_2, self.b_2, residual=x2)
        self._saved = (B, S, scale, h1, qkv, o, lse, x2, h2, a, u)
        return y

    def backward(self, grad_y: Tensor) -> Tensor:
        if self._saved is None:
            raise RuntimeError("forward() must run before backward()")
        B, S, scale, h1, qkv, o, lse, x2, h2, a, u = self._saved
        D = self.d // self.h
        # MLP: y = x2 + GELU(h2 W1 + b1) W2 + b2
        g_w2, g_b2 = weight_grad(a, grad_y), col_sum(grad_y)
        da = input_grad(grad_y, self.w_2)
        n, m = _rows(da)
        du_core, g_b1_core = C._gelu_bwd_col_sum(da._core, u._core, n, m)  # a recomputed from u
        du, g_b1 = Tensor._from_core(du_core, da.shape), Tensor._from_core(g_b1_core, (m,))
        g_w1 = weight_grad(h2, du)
        dx2 = self.ln2.backward(input_grad(du, self.w_1), residual=grad_y)
        # attention: x2 = x + O Wo + bo
        g_wo, g_bo = weight_grad(o, dx2), col_sum(dx2)
        d_o = input_grad(dx2, self.w_o)
        dqkv = Tensor._from_core(
            C._attention_bwd_packed(qkv._core, o._core, lse, d_o._core, B, S, self.h, D, scale,
                                    self.causal), qkv.shape)
        g_wqkv, g_bqkv = weight_grad(h1, dqkv), col_sum(dqkv)
        dx = self.ln1.backward(input_grad(dqkv, self.w_qkv), residual=dx2)
        self._grads = [self.ln1.grad_gamma, self.ln1.grad_beta, g_wqkv, g_bqkv, g_wo, g_bo,
                       self.ln2.grad_gamma, self.ln2.grad_beta, g_w1, g_b1, g_w2, g_b2]
        return dx
