"""attention_bwd_noalloc (the backward with its row statistics in a fixed
device array inside the library) against attention_bwd on the same inputs,
through the C ABI: dK and dV bit for bit, dQ (summed with atomics in a
run-dependent order) within 1e-5, on consecutive calls of decreasing size;
the largest accepted size (2^21 padded rows) moves no device memory; a larger
call is rejected before any launch.  The medium call is also held to the
north-star tolerance against the CPU oracle.  In deterministic mode both
entry points give the same bits for dQ as well."""

import ctypes

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from ember_amd import capi
from ember_amd.capi import DeviceArray
from tolerance import assert_north_star

pytestmark = pytest.mark.gpu

MAX_ROWS = 1 << 21


def _free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


class _Case:
    """Inputs on the device, the forward's O and LSE, and output buffers for
    both entry points."""

    def __init__(self, B, H, S, D, causal, seed):
        self.shape, self.causal = (B, H, S, D), causal
        rng = np.random.default_rng(seed)
        self.host = [rng.standard_normal((B, H, S, D), dtype=np.float32) for _ in range(4)]
        self.dev = [DeviceArray.from_numpy(x) for x in self.host]
        self.o, self.lse = DeviceArray((B, H, S, D)), DeviceArray((B, H, S))
        self.st = capi.contiguous_strides(B, H, S, D)
        self.scale = G.scale_for(D)
        q, k, v, _ = self.dev
        G.say(f"no-alloc case B={B} H={H} S={S} D={D} causal={causal}: forward")
        capi.check(capi.lib().attention_fwd(q.ptr, k.ptr, v.ptr, self.o.ptr, self.lse.ptr, B, H, S, D,
                                            self.scale, int(causal), *self.st, *self.st), "attention_fwd")
        self.out = {name: [DeviceArray((B, H, S, D)) for _ in range(3)]
                    for name in ("attention_bwd", "attention_bwd_noalloc")}

    def run(self, name):
        q, k, v, d_o = self.dev
        G.say(f"{name} B,H,S,D={self.shape} causal={self.causal}")
        outs = self.out[name]
        return getattr(capi.lib(), name)(q.ptr, k.ptr, v.ptr, self.o.ptr, self.lse.ptr, d_o.ptr,
                                         *(x.ptr for x in outs), *self.shape, self.scale, int(self.causal),
                                         *self.st, *self.st)

    def compare(self):
        reg = [x.numpy() for x in self.out["attention_bwd"]]
        new = [x.numpy() for x in self.out["attention_bwd_noalloc"]]
        assert np.array_equal(new[1], reg[1]) and np.array_equal(new[2], reg[2])
        np.testing.assert_allclose(new[0], reg[0], rtol=1e-5, atol=1e-6)
        return new


def test_noalloc_matches_attention_bwd_on_consecutive_calls():
    # Loads the kernels and looks up the array's address (first call on the device).
    warm = _Case(1, 2, 200, 32, True, 1)
    capi.check(warm.run("attention_bwd_noalloc"), "attention_bwd_noalloc")
    capi.lib().sync_device()

    # 1) the largest accepted call: B*H*S_pad = 2^21 rows (16 MiB of statistics)
    big = _Case(64, 32, 1024, 32, True, 2)
    assert 64 * 32 * 1024 == MAX_ROWS
    capi.lib().sync_device()
    before = _free_device_bytes()
    capi.check(big.run("attention_bwd_noalloc"), "attention_bwd_noalloc")
    capi.lib().sync_device()
    after = _free_device_bytes()
    assert before - after < (4 << 20), f"device memory fell by {before - after} bytes"
    capi.check(big.run("attention_bwd"), "attention_bwd")
    big.compare()
    del big

    # 2) a smaller call right after (the array still holds the big call's rows)
    mid = _Case(1, 3, 300, 64, False, 3)
    capi.check(mid.run("attention_bwd_noalloc"), "attention_bwd_noalloc")
    capi.check(mid.run("attention_bwd"), "attention_bwd")
    dq, dk, dv = mid.compare()
    q, k, v, d_o = mid.host
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, False, mid.scale)
    refs = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, False, mid.scale)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), refs):
        assert_north_star(got, ref, name)

    # 3) S <= 32: kernels that need no statistics; dQ has no atomics there
    short = _Case(2, 5, 20, 128, True, 4)
    capi.check(short.run("attention_bwd_noalloc"), "attention_bwd_noalloc")
    capi.check(short.run("attention_bwd"), "attention_bwd")
    new = short.compare()
    assert np.array_equal(new[0], short.out["attention_bwd"][0].numpy())

    # 4) 64 < S <= 128 at D = 128: one workgroup per head, no statistics, no atomics
    mid128 = _Case(3, 4, 100, 128, True, 5)
    capi.check(mid128.run("attention_bwd_noalloc"), "attention_bwd_noalloc")
    capi.check(mid128.run("attention_bwd"), "attention_bwd")
    new = mid128.compare()
    assert np.array_equal(new[0], mid128.out["attention_bwd"][0].numpy())


def test_noalloc_deterministic_matches_attention_bwd():
    """Deterministic mode: the tile counters live in the same fixed array, and
    both entry points add every dQ tile in the same fixed order, so dQ, dK
    and dV are the same bits; two calls in a row, the second smaller."""
    capi.set_deterministic(True)
    try:
        for B, H, S, D, causal, seed in ((2, 8, 1024, 64, True, 6), (1, 3, 300, 128, False, 7)):
            case = _Case(B, H, S, D, causal, seed)
            capi.check(case.run("attention_bwd_noalloc"), "attention_bwd_noalloc")
            capi.check(case.run("attention_bwd"), "attention_bwd")
            reg = [x.numpy() for x in case.out["attention_bwd"]]
            new = [x.numpy() for x in case.out["attention_bwd_noalloc"]]
            for name, a, b in zip(("dq", "dk", "dv"), new, reg):
                assert np.array_equal(a, b), name
        assert capi.deterministic_timeouts() == 0
    finally:
        capi.set_deterministic(False)


def test_noalloc_rejects_more_rows_than_its_array():
    """B*H*S_pad = 2^21 + 32 rows: EMBER_ERR_INVALID_ARGUMENT, nothing launched
    (the small buffers below would not hold the problem)."""
    L = capi.lib()
    L.ember_get_last_error()
    buf = DeviceArray((64,))
    p = buf.ptr
    S = (MAX_ROWS // 64) + 32                 # H = 64 heads of S_pad = S
    st = capi.contiguous_strides(1, 64, S, 32)
    G.say("attention_bwd_noalloc over its row limit (rejected on the host)")
    rc = L.attention_bwd_noalloc(p, p, p, p, p, p, p, p, p, 1, 64, S, 32, 0.125, 1, *st, *st)
    assert rc == 1 and L.ember_get_last_error() == 1
