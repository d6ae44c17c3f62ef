"""Calls the HIP attention / matmul entry points through the C ABI
(ember_amd.capi -> libember_amd.so) on numpy inputs.  GPU tests only."""

from __future__ import annotations

import math
import sys

import numpy as np

from ember_amd import capi
from ember_amd.capi import DeviceArray
from tolerance import gemm_error_bound  # noqa: F401  (re-exported for the GPU tests)


def say(msg: str) -> None:
    """Names the case about to run on the GPU (flushed, for post-mortems)."""
    print(f"[gpu] {msg}", file=sys.stderr, flush=True)


def scale_for(D: int) -> float:
    return float(np.float32(1.0 / math.sqrt(D)))


SENTINEL = np.float32(12345.0)


def padded_strides(B, H, S, D, pad, hpad):
    """Strides (sb, sh, ss) of a (B, H, S + hpad, D + pad) buffer, and its size."""
    ss = D + pad
    sh = (S + hpad) * ss
    return (H * sh, sh, ss), B * H * sh


def upload_padded(x, strides, total):
    """x (B, H, S, D) into a padded device buffer whose padding is SENTINEL."""
    buf = np.full(total, SENTINEL, np.float32)
    view = np.lib.stride_tricks.as_strided(buf, shape=x.shape, strides=tuple(4 * s for s in strides) + (4,))
    view[...] = x
    return DeviceArray.from_numpy(buf)


def download_padded(dev, strides, shape):
    """The (B, H, S, D) view of a padded device buffer, and the whole buffer."""
    buf = dev.numpy()
    view = np.lib.stride_tricks.as_strided(buf, shape=shape, strides=tuple(4 * s for s in strides) + (4,))
    return np.array(view), buf


def attention_fwd(q, k, v, causal, scale=None, log=None):
    """O, LSE of the HIP forward.  If `log` is a list, the names of the
    kernels the call launched are appended to it."""
    B, H, S, D = q.shape
    scale = scale_for(D) if scale is None else scale
    say(f"attention_fwd B={B} H={H} S={S} D={D} causal={causal}")
    dq, dk, dv = (DeviceArray.from_numpy(x) for x in (q, k, v))
    o = DeviceArray((B, H, S, D))
    lse = DeviceArray((B, H, S))
    st = capi.contiguous_strides(B, H, S, D)
    capi.launch_log_reset()
    rc = capi.lib().attention_fwd(dq.ptr, dk.ptr, dv.ptr, o.ptr, lse.ptr, B, H, S, D, scale,
                                  int(causal), *st, *st)
    if log is not None:
        log.extend(capi.launch_log())
    capi.check(rc, "attention_fwd")
    return o.numpy(), lse.numpy()


def attention_bwd(q, k, v, o, lse, d_o, causal, scale=None, log=None):
    """dQ, dK, dV of the HIP backward.  If `log` is a list, the names of the
    kernels the call launched are appended to it."""
    B, H, S, D = q.shape
    scale = scale_for(D) if scale is None else scale
    say(f"attention_bwd B={B} H={H} S={S} D={D} causal={causal}")
    ins = [DeviceArray.from_numpy(x) for x in (q, k, v, o, lse, d_o)]
    outs = [DeviceArray((B, H, S, D)) for _ in range(3)]
    st = capi.contiguous_strides(B, H, S, D)
    capi.launch_log_reset()
    rc = capi.lib().attention_bwd(*(x.ptr for x in ins), *(x.ptr for x in outs), B, H, S, D,
                                  scale, int(causal), *st, *st)
    if log is not None:
        log.extend(capi.launch_log())
    capi.check(rc, "attention_bwd")
    return tuple(x.numpy() for x in outs)


def matmul(a, b):
    n, k = a.shape
    m = b.shape[1]
    say(f"matmul n={n} m={m} k={k}")
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    out = DeviceArray((n, m))
    capi.lib().matmul(da.ptr, db.ptr, out.ptr, n, m, k)
    capi.check(what="matmul")
    return out.numpy()


def matmul_batched(a, b):
    batch, n, k = a.shape
    m = b.shape[2]
    say(f"matmul_batched batch={batch} n={n} m={m} k={k}")
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    out = DeviceArray((batch, n, m))
    capi.lib().matmul_batched(da.ptr, db.ptr, out.ptr, batch, n, m, k)
    capi.check(what="matmul_batched")
    return out.numpy()


def gemm_ex(a, b, ta=False, tb=False, bias=None, residual=None, act=0):
    """gemm_ex on stored operands: a is (k, n) when ta else (n, k), b is (m, k)
    when tb else (k, m); leading batch dimensions allowed.  Returns out, and
    pre as well when act is set."""
    batch = a.shape[0] if a.ndim == 3 else 1
    n, k = (a.shape[-1], a.shape[-2]) if ta else (a.shape[-2], a.shape[-1])
    m = b.shape[-2] if tb else b.shape[-1]
    say(f"gemm_ex batch={batch} n={n} m={m} k={k} ta={ta} tb={tb} act={act} "
        f"bias={bias is not None} residual={residual is not None}")
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    dbias = DeviceArray.from_numpy(bias) if bias is not None else None
    dres = DeviceArray.from_numpy(residual) if residual is not None else None
    shape = (batch, n, m) if a.ndim == 3 else (n, m)
    out = DeviceArray(shape)
    pre = DeviceArray(shape) if act else None
    rc = capi.lib().gemm_ex(da.ptr, db.ptr, out.ptr, batch, n, m, k, int(ta), int(tb),
                            None if dbias is None else dbias.ptr,
                            None if dres is None else dres.ptr,
                            None if pre is None else pre.ptr, act)
    capi.check(rc, "gemm_ex")
    return (out.numpy(), pre.numpy()) if act else out.numpy()
