"""ember_amd: the MI355X (gfx950) backend of Ember's attention / matmul path.

``libember_amd.so`` is the C ABI (``include/ember_amd.h``); ``ember_amd._core``
binds it for Python; this package mirrors the reference's ``ember`` front-end
on top (``Tensor``, the element-wise and reduction functions, ``softmax``,
``T``) and adds ``attention``.  Names resolve lazily so that
``ember_amd.build`` can run before anything is built.
"""

from __future__ import annotations

import importlib

_TENSOR_NAMES = (
    "Tensor", "max", "min", "amax", "exp", "log", "sin", "cos", "tan", "ctg", "sinh", "cosh",
    "tanh", "ctgh", "T", "sum", "softmax", "sqrt", "attention", "attention_forward",
    "attention_backward", "synchronize", "empty_cache", "memory_stats",
)
_CAPI_NAMES = ("set_deterministic", "is_deterministic")
_SUBMODULES = ("nn", "optim", "loss", "random", "capi", "build")

__all__ = list(_TENSOR_NAMES) + list(_CAPI_NAMES) + ["nn", "optim", "loss", "random"]


def __getattr__(name: str):
    if name in _TENSOR_NAMES:
        return getattr(importlib.import_module("ember_amd.tensor"), name)
    if name in _CAPI_NAMES:
        return getattr(importlib.import_module("ember_amd.capi"), name)
    if name in _SUBMODULES:
        return importlib.import_module(f"ember_amd.{name}")
    raise AttributeError(f"module 'ember_amd' has no attribute {name!r}")
