"""The element-wise layers and Dropout of ember_amd.nn, checked as the
reference checks its own (tests/nn/test_activations.py, tests/nn/
test_dropout.py): numpy formulas at rtol 1e-4 for ReLU, Sigmoid, Tanh and
GELU (forward called directly, then backward), and inverted-dropout
scaling, identity at inference, and the mask reused by backward.  The layers
compose the library's element-wise GPU operators (GELU's backward is one
fused kernel)."""

import numpy as np
import pytest

import gpu_helpers as G
from ember_amd import Tensor, nn
from ember_amd import random as em_random

pytestmark = pytest.mark.gpu

SHAPES = [(64,), (32, 128), (8, 10, 64)]
CONFIGS = [
    ("ReLU", nn.ReLU, lambda x: np.maximum(x, 0), lambda x, _, g: g * (x > 0)),
    ("Sigmoid", nn.Sigmoid, lambda x: 1.0 / (1.0 + np.exp(-x)), lambda _, y, g: g * (y * (1.0 - y))),
    ("Tanh", nn.Tanh, np.tanh, lambda _, y, g: g * (1.0 - y ** 2)),
    ("GELU", nn.GELU, lambda x: 0.5 * x * (1.0 + np.tanh(0.8 * x, dtype=np.float32)),
     lambda x, y, g: g * ((1.0 + np.tanh(0.8 * x)) * (0.5 + 0.8 * (x - y)))),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("name,cls,ref_fwd,ref_bwd", CONFIGS)
def test_activation(shape, name, cls, ref_fwd, ref_bwd):
    G.say(f"activation {name} {shape}")
    rng = np.random.default_rng(42)
    x = rng.standard_normal(shape).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    layer = cls()
    assert layer.parameters() == [] and layer.gradients() == []
    y = layer.forward(Tensor.from_np(x), training=True)
    y_ref = ref_fwd(x)
    np.testing.assert_allclose(y.to_np(), y_ref, rtol=1e-4, err_msg=f"{name} forward")
    dx = layer.backward(Tensor.from_np(g))
    np.testing.assert_allclose(dx.to_np(), ref_bwd(x, y_ref, g), rtol=1e-4, atol=1e-7,
                               err_msg=f"{name} backward")
    # through __call__ as well, inside a Sequential
    seq = nn.Sequential(cls())
    np.testing.assert_array_equal(seq(Tensor.from_np(x)).to_np(), y.to_np())


def test_activation_backward_needs_forward():
    with pytest.raises(RuntimeError):
        nn.ReLU().backward(Tensor.from_np(np.ones(3, np.float32)))


@pytest.mark.parametrize("p", [0.2, 0.5, 0.8])
def test_dropout_training_inverted(p):
    em_random.seed(3)
    x = np.ones((100, 100), np.float32)
    layer = nn.Dropout(p=p)
    y = layer.forward(Tensor.from_np(x), training=True).to_np()
    mask = layer.mask.to_np()
    assert set(np.unique(mask)) <= {0.0, 1.0}
    np.testing.assert_allclose(y, x * mask * (1.0 / (1.0 - p)), rtol=1e-5)
    assert abs(np.mean(y) - 1.0) < 0.1
    assert abs(mask.mean() - (1 - p)) < 0.05


@pytest.mark.parametrize("p", [0.2, 0.5, 0.8])
def test_dropout_inference_identity(p):
    x = np.random.default_rng(4).standard_normal((10, 10)).astype(np.float32)
    layer = nn.Dropout(p=p)
    np.testing.assert_allclose(layer.forward(Tensor.from_np(x), training=False).to_np(), x)
    assert layer.mask is None


def test_dropout_backward_scaled_and_seeded():
    layer = nn.Dropout(p=0.5)
    em_random.seed(9)
    layer.forward(Tensor.from_np(np.ones((5, 5), np.float32)), training=True)
    mask = layer.mask.to_np()
    grad = layer.backward(Tensor.from_np(np.ones((5, 5), np.float32)))
    np.testing.assert_allclose(grad.to_np(), mask * 2.0)
    em_random.seed(9)
    again = nn.Dropout(p=0.5)
    again.forward(Tensor.from_np(np.ones((5, 5), np.float32)), training=True)
    assert np.array_equal(again.mask.to_np(), mask)
    with pytest.raises(ValueError):
        nn.Dropout(p=1.0)
