"""ember_amd.random on the device: after _seed the tensors hold the C
library's rand() sequence whatever device allocations happen in between
(the GPU runtime itself advances the C library's rand() state, so the
generator is private), and a seeded model is bitwise reproducible whatever
stale data the device allocator's cached blocks hold."""

import ctypes

import numpy as np
import pytest

import gpu_helpers as G
from ember_amd import Tensor, nn
from ember_amd import random as erand

pytestmark = pytest.mark.gpu

SHAPES = [(256, 768), (256, 256), (256, 1024), (1024, 256)]


def _libc_uniform(seed, shapes, low, high):
    libc = ctypes.CDLL("libc.so.6")
    libc.srand(seed)
    out = []
    for s in shapes:
        r = np.array([libc.rand() for _ in range(s[0] * s[1])], np.float32)
        out.append(np.float32(low) + (r / np.float32(2147483647.0)) * np.float32(high - low))
    return out


def _poison_cache():
    junk = [Tensor(np.full(n, np.nan, np.float32)) for n in (1 << 16, 1 << 18, 1 << 20, 3 << 18)]
    del junk


@pytest.mark.parametrize("poison", [False, True])
def test_uniform_follows_the_rand_sequence_across_allocations(poison):
    G.say(f"uniform sequence poison={poison}")
    if poison:
        _poison_cache()
    erand.seed(3)
    got = [erand.uniform(-1.0, 1.0, s).to_np().ravel() for s in SHAPES]
    for g, w in zip(got, _libc_uniform(3, SHAPES, -1.0, 1.0)):
        np.testing.assert_array_equal(g, w)


def test_seeded_block_is_bitwise_reproducible_over_stale_memory():
    B, S, d, H = 2, 256, 256, 4
    G.say("seeded decoder block over stale memory")

    def run():
        erand.seed(0)
        block = nn.DecoderBlock(d, H, 4, True)
        x = Tensor(np.random.default_rng(6).standard_normal((B * S, d), dtype=np.float32))
        y = block(x, B, S)
        dx = block.backward(Tensor(np.ones((B * S, d), np.float32)))
        return y.to_np(), [p.to_np() for p in block.parameters()], block.gradients()[2].to_np()

    y1, p1, g1 = run()
    _poison_cache()
    y2, p2, g2 = run()
    for a, b in zip(p1, p2):
        np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(y1, y2)
    assert np.isfinite(g2).all()
    # dQ is accumulated with atomics (order not fixed): gradients agree to
    # rounding, not bitwise.
    np.testing.assert_allclose(g1, g2, rtol=1e-4, atol=1e-5)


# ---- the C-ABI entry points the reference's random binding links against
# (uniform / constant, src/random/distributions.h:8-9)


@pytest.mark.parametrize("size", [1, 7, 4096, 100_003])
def test_capi_uniform_draws_the_c_library_sequence(size):
    """uniform() draws from the C library's rand() (what the reference
    binding's _seed() seeds with srand), low + (r / RAND_MAX) * (high - low)
    in fp32, distributions_gpu.cu:11-24."""
    from ember_amd import capi
    from ember_amd.capi import DeviceArray

    G.say(f"capi uniform size={size}")
    L = capi.lib()
    libc = ctypes.CDLL("libc.so.6")
    out = DeviceArray((size,))
    L.uniform.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_int]
    libc.srand(11)
    L.uniform(-0.5, 2.0, out.ptr, size)
    capi.check(what="uniform")
    (want,) = _libc_uniform(11, [(1, size)], -0.5, 2.0)
    np.testing.assert_array_equal(out.numpy(), want)


@pytest.mark.parametrize("size,offset", [(1, 0), (5, 1), (4096, 0), (4099, 3), (1_000_001, 2)])
def test_capi_constant_fills_exactly_the_range(size, offset):
    """constant() sets out[0..size) and nothing else, at any alignment."""
    from ember_amd import capi
    from ember_amd.capi import DeviceArray

    G.say(f"capi constant size={size} offset={offset}")
    L = capi.lib()
    L.constant.argtypes = [ctypes.c_float, ctypes.c_void_p, ctypes.c_int]
    buf = DeviceArray.from_numpy(np.full(size + offset + 5, -7.0, np.float32))
    L.constant(np.float32(0.1), buf.ptr + 4 * offset, size)
    capi.check(what="constant")
    got = buf.numpy()
    assert (got[:offset] == -7.0).all() and (got[offset + size:] == -7.0).all()
    assert (got[offset:offset + size] == np.float32(0.1)).all()
    L.constant(np.float32(3.0), buf.ptr, 0)          # size 0: nothing written
    capi.check(what="constant")
    assert buf.numpy()[0] == got[0]
