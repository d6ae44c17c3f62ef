"""The host generator behind ember_amd.random: the C library's rand()
sequence (glibc's additive feedback generator), reproduced privately so that
other users of rand() in the process (the GPU runtime) cannot shift it.
Checked against the C library itself; no GPU needed."""

import ctypes
import sys

import pytest

from ember_amd._core._em_random import _host_rand, _seed

libc = ctypes.CDLL("libc.so.6") if sys.platform.startswith("linux") else None


@pytest.mark.skipif(libc is None, reason="needs glibc")
@pytest.mark.parametrize("seed", [0, 1, 2, 42, 12345, 2**31 - 1, -5])
def test_sequence_is_the_c_library_rand(seed):
    _seed(seed)
    got = _host_rand(5000)
    libc.srand(ctypes.c_uint(seed & 0xFFFFFFFF))
    want = [libc.rand() for _ in range(5000)]
    assert got == want


def test_reseeding_restarts_the_sequence():
    _seed(7)
    a = _host_rand(100)
    _host_rand(12345)
    _seed(7)
    assert _host_rand(100) == a
    assert all(0 <= v <= 2**31 - 1 for v in a)
