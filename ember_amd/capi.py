"""ctypes view of libember_amd.so's C ABI (declared in include/ember_amd.h).

This is how tests and the benchmark drive the library exactly as a foreign
caller would: plain pointers and sizes, no torch types.  ``DeviceArray`` is
a small owner of one ``alloc_memory`` block.  Loading fails loudly when the
library has not been built; there is no CPU fallback.
"""

from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libember_amd.so")
HEADER = os.path.join(os.path.dirname(_PKG), "include", "ember_amd.h")
OPS_DEF = os.path.join(_PKG, "csrc", "operators.def")

_lib: C.CDLL | None = None
_vp = C.c_void_p
_i64 = C.c_int64


class EmberError(RuntimeError):
    pass


def exported_symbols() -> list[str]:
    """Every function name include/ember_amd.h declares (operators.def expanded)."""
    names: list[str] = []
    with open(OPS_DEF) as f:
        for kind, name in re.findall(r"^EMBER_(BINARY|SCALAR|BROADCAST|UNARY)_OP\((\w+),", f.read(), re.M):
            suffix = {"BINARY": "_tensor", "SCALAR": "_scalar", "BROADCAST": "_broadcasted",
                      "UNARY": "_tensor"}[kind]
            names.append(name + suffix)
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"#define EMBER_\w+_OP\(.*?(?<!\\)\n", "", text, flags=re.S)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s]*?[\s\*]+(\w+)\s*\(", text, re.M):
        if m.group(1) not in ("defined",):
            names.append(m.group(1))
    return sorted(set(names))


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise EmberError(f"{LIB_PATH} is not built; run `python -m ember_amd.build`")
    L = C.CDLL(LIB_PATH)
    L.ember_get_last_error.restype = C.c_int
    L.ember_error_string.restype = C.c_char_p
    L.ember_error_string.argtypes = [C.c_int]
    L.alloc_memory.restype = _vp
    L.alloc_memory.argtypes = [C.c_size_t]
    L.free_memory.argtypes = [_vp]
    L.copy_to_device.argtypes = [_vp, _vp, C.c_size_t]
    L.copy_from_device.argtypes = [_vp, _vp, C.c_size_t]
    L.sync_device.argtypes = []
    L.ember_empty_cache.argtypes = []
    L.ember_memory_stats.argtypes = [C.POINTER(C.c_size_t)] * 3
    L.matmul.argtypes = [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int]
    L.matmul_batched.argtypes = [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int]
    L.transpose.argtypes = [_vp, _vp, C.c_int, C.c_int]
    L.sum.restype = C.c_float
    L.sum.argtypes = [_vp, C.c_int]
    L.sum_axis.argtypes = [_vp, _vp, C.c_int, C.c_int, C.c_int]
    L.max_axis.argtypes = [_vp, _vp, C.c_int, C.c_int, C.c_int]
    L.attention_fwd.restype = C.c_int
    L.attention_fwd.argtypes = [_vp] * 5 + [_i64] * 4 + [C.c_float, C.c_int] + [_i64] * 6
    L.attention_bwd.restype = C.c_int
    L.attention_bwd.argtypes = [_vp] * 9 + [_i64] * 4 + [C.c_float, C.c_int] + [_i64] * 6
    L.attention_bwd_noalloc.restype = C.c_int
    L.attention_bwd_noalloc.argtypes = [_vp] * 9 + [_i64] * 4 + [C.c_float, C.c_int] + [_i64] * 6
    L.softmax_axis.restype = C.c_int
    L.softmax_axis.argtypes = [_vp, _vp, C.c_int, C.c_int, C.c_int]
    L.gemm_ex.restype = C.c_int
    L.gemm_ex.argtypes = [_vp] * 3 + [C.c_int] * 6 + [_vp] * 3 + [C.c_int]
    L.ember_set_deterministic.argtypes = [C.c_int]
    L.ember_set_deterministic.restype = None
    L.ember_get_deterministic.argtypes = []
    L.ember_get_deterministic.restype = C.c_int
    L.ember_deterministic_timeouts.argtypes = []
    L.ember_deterministic_timeouts.restype = C.c_int
    L.ember_launch_log_reset.argtypes = []
    L.ember_launch_log_reset.restype = None
    L.ember_launch_log.argtypes = []
    L.ember_launch_log.restype = C.c_char_p
    L.adam_step.restype = C.c_int
    L.adam_step.argtypes = [C.POINTER(_vp)] * 4 + [C.POINTER(_i64), C.c_int] + [C.c_double] * 4 + [_i64]
    L.adamw_step.restype = C.c_int
    L.adamw_step.argtypes = [C.POINTER(_vp)] * 4 + [C.POINTER(_i64), C.c_int] + [C.c_double] * 5 + [_i64]
    L.sgd_step.restype = C.c_int
    L.sgd_step.argtypes = [C.POINTER(_vp)] * 3 + [C.POINTER(_i64), C.c_int] + [C.c_double] * 2
    _lib = L
    return L


def set_deterministic(enabled: bool) -> None:
    """Process-wide switch for bitwise-reproducible results
    (ember_set_deterministic).  Off by default.  With it on, attention_bwd's
    dq at S > 128 (S > 64 at D = 32) is added in a fixed key-block order per
    dQ tile (a counter per 16 rows) instead of in the atomics' arrival
    order; every other operator is reproducible either way."""
    lib().ember_set_deterministic(1 if enabled else 0)


def deterministic_timeouts() -> int:
    """Deterministic-mode waits for a dQ tile's turn that gave up on the
    current device (ember_deterministic_timeouts); 0 means every
    deterministic dQ so far was added in its fixed order.  Synchronises."""
    n = lib().ember_deterministic_timeouts()
    if n < 0:
        check(what="ember_deterministic_timeouts")
    return n


def is_deterministic() -> bool:
    return bool(lib().ember_get_deterministic())


def launch_log_reset() -> None:
    """Clears this thread's log of launched kernels (ember_launch_log_reset)."""
    lib().ember_launch_log_reset()


def launch_log() -> list[str]:
    """Names of the kernels this thread launched since launch_log_reset()."""
    text = lib().ember_launch_log().decode()
    return text.split(",") if text else []


def check(status: int | None = None, what: str = "ember_amd") -> None:
    """Raise EmberError if `status` (or the sticky library status) is an error."""
    L = lib()
    sticky = L.ember_get_last_error()
    st = status if status else sticky
    if st:
        raise EmberError(f"{what}: {L.ember_error_string(st).decode()} (status {st})")


class DeviceArray:
    """One float32 device buffer from alloc_memory(), freed on close/GC."""

    def __init__(self, shape, fill: np.ndarray | None = None):
        self.shape = tuple(int(s) for s in shape)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = 4 * self.size
        self.ptr = lib().alloc_memory(max(self.nbytes, 4))
        if not self.ptr:
            raise MemoryError(f"alloc_memory({self.nbytes}) failed")
        if fill is not None:
            self.upload(fill)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> DeviceArray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        return cls(a.shape, a)

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=np.float32)
        assert a.size == self.size, (a.shape, self.shape)
        lib().copy_to_device(self.ptr, a.ctypes.data, self.nbytes)
        check(what="copy_to_device")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=np.float32)
        lib().sync_device()
        lib().copy_from_device(out.ctypes.data, self.ptr, self.nbytes)
        check(what="copy_from_device")
        return out

    def close(self) -> None:
        if self.ptr:
            lib().free_memory(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def contiguous_strides(B: int, H: int, S: int, D: int) -> tuple[int, int, int]:
    """(stride_b, stride_h, stride_s) of a dense (B, H, S, D) tensor."""
    return (H * S * D, S * D, D)


def adam_step(params, grads, means, variances, lr, beta1, beta2, eps, step) -> int:
    """adam_step over lists of DeviceArray (same lengths and sizes)."""
    n = len(params)
    table = lambda xs: (_vp * n)(*(x.ptr for x in xs))  # noqa: E731
    sizes = (_i64 * n)(*(x.size for x in params))
    return lib().adam_step(table(params), table(grads), table(means), table(variances), sizes, n,
                           lr, beta1, beta2, eps, step)


def adamw_step(params, grads, means, variances, lr, beta1, beta2, eps, weight_decay, step) -> int:
    """adamw_step over lists of DeviceArray (same lengths and sizes)."""
    n = len(params)
    table = lambda xs: (_vp * n)(*(x.ptr for x in xs))  # noqa: E731
    sizes = (_i64 * n)(*(x.size for x in params))
    return lib().adamw_step(table(params), table(grads), table(means), table(variances), sizes, n,
                            lr, beta1, beta2, eps, weight_decay, step)


def sgd_step(params, grads, velocities, lr, momentum) -> int:
    """sgd_step over lists of DeviceArray (same lengths and sizes)."""
    n = len(params)
    table = lambda xs: (_vp * n)(*(x.ptr for x in xs))  # noqa: E731
    sizes = (_i64 * n)(*(x.size for x in params))
    return lib().sgd_step(table(params), table(grads), table(velocities), sizes, n, lr, momentum)
