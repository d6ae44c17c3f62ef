"""Native façade: every name of the reference's ``ember._core``
(``ember/_core/__init__.py:1-48``) plus the attention entry points, from the
CPython modules built over libember_amd.so.  Importing fails loudly when the
modules have not been built (``python -m ember_amd.build``); there is no CPU
fallback."""

from ._em_random import _constant, _seed, _uniform
from ._tensor import (
    _add_broadcasted,
    _add_scalar,
    _adam_step,
    _add_tensor,
    _attention_bwd,
    _attention_bwd_packed,
    _attention_fwd,
    _attention_fwd_packed,
    _col_sum,
    _cos,
    _cosh,
    _ctg,
    _ctgh,
    _exponent,
    _from_numpy,
    _gelu_bwd,
    _gt_scalar,
    _gt_tensor,
    _layernorm_bwd,
    _layernorm_fwd,
    _linear,
    _log,
    _lt_scalar,
    _lt_tensor,
    _matmul,
    _matmul_batched,
    _max_axis,
    _max_scalar,
    _max_tensor,
    _min_scalar,
    _min_tensor,
    _mul_broadcasted,
    _mul_scalar,
    _mul_tensor,
    _negate,
    _pow_scalar,
    _pow_tensor,
    _rpow_scalar,
    _rsub_scalar,
    _rtruediv_scalar,
    _sin,
    _sinh,
    _sqrt,
    _sub_broadcasted,
    _sub_scalar,
    _sub_tensor,
    _sum,
    _sum_axis,
    _synchronize,
    _tan,
    _tanh,
    _Tensor,
    _transpose,
    _truediv_broadcasted,
    _truediv_scalar,
    _truediv_tensor,
)

# The 45 names of the reference's ember._core (its _types aliases aside).
REFERENCE_NAMES = (
    "_constant", "_seed", "_uniform",
    "_add_broadcasted", "_add_scalar", "_add_tensor", "_cos", "_cosh", "_ctg", "_ctgh",
    "_exponent", "_from_numpy", "_gt_scalar", "_gt_tensor", "_log", "_lt_scalar", "_lt_tensor",
    "_matmul", "_matmul_batched", "_max_axis", "_max_scalar", "_max_tensor", "_min_scalar",
    "_min_tensor", "_mul_broadcasted", "_mul_scalar", "_mul_tensor", "_negate", "_pow_scalar",
    "_pow_tensor", "_rpow_scalar", "_rsub_scalar", "_rtruediv_scalar", "_sin", "_sinh", "_sqrt",
    "_sub_broadcasted", "_sub_scalar", "_sub_tensor", "_sum", "_sum_axis", "_tan", "_tanh",
    "_Tensor", "_transpose", "_truediv_broadcasted", "_truediv_scalar", "_truediv_tensor",
)

__all__ = list(REFERENCE_NAMES) + [
    "_attention_fwd", "_attention_bwd", "_attention_fwd_packed", "_attention_bwd_packed",
    "_adam_step", "_linear", "_gelu_bwd", "_col_sum", "_layernorm_fwd", "_layernorm_bwd",
    "_synchronize",
]
