"""Parity of the HIP fp32 MFMA GEMM (matmul / matmul_batched) with Ember's
CPU matmul (FP64 accumulation, oracle/ember_oracle.c, itself bitwise the
reference's operators_cpu.c).  Every product is held to the north-star
tolerance, max-abs 2e-4 / rel 1e-3 against that oracle, and to the rigorous
order-free fp32 bound gamma_k * |A||B| as a second check; bitwise where fp32
arithmetic is exact.  (The order-free bound alone is loose enough that a GEMM
on bf16-rounded operands passes it: tests/test_gemm_tolerance.py.)"""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from tolerance import assert_north_star

pytestmark = pytest.mark.gpu


def _u(shape, seed):
    return np.random.default_rng(seed).uniform(-1, 1, shape).astype(np.float32)


def _check(got, a, b, exact=None):
    exact = oracle.matmul(a, b, threads=True) if exact is None else exact
    bound = G.gemm_error_bound(a, b)
    err = np.abs(got.astype(np.float64) - exact.astype(np.float64))
    assert (err <= bound).all(), f"max err {err.max()} vs bound {bound.min()}"
    assert_north_star(got, exact)


@pytest.mark.parametrize(
    "shape_a, shape_b",
    [((4, 5), (5, 3)), ((1, 1), (1, 1))],  # reference test_tensor.py:125-145
)
def test_reference_matmul_cases(shape_a, shape_b):
    rng = np.random.default_rng(1)
    a = rng.standard_normal(shape_a).astype(np.float32)
    b = rng.standard_normal(shape_b).astype(np.float32)
    np.testing.assert_allclose(G.matmul(a, b), a @ b, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize(
    "shape_a, shape_b",
    [((2, 3, 4), (2, 4, 5)), ((4, 2, 3), (4, 3, 6)), ((6, 5, 6), (6, 6, 2))],  # test_tensor.py:165-176
)
def test_reference_batched_cases(shape_a, shape_b):
    rng = np.random.default_rng(2)
    a = rng.standard_normal(shape_a).astype(np.float32)
    b = rng.standard_normal(shape_b).astype(np.float32)
    np.testing.assert_allclose(G.matmul_batched(a, b), a @ b, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize(
    "n,k,m",
    [(32, 128, 64), (1, 10, 5), (64, 32, 128), (16, 50, 50),        # test_linear.py shapes
     (127, 33, 129), (128, 32, 128), (129, 1, 255), (257, 300, 3), (5, 4096, 7),
     (300, 64, 260), (1000, 500, 700),
     # tile-aligned shapes (n % 128, m % 256, k % 16 == 0) take the LDS-DMA kernel
     (128, 16, 256), (256, 48, 512), (384, 1024, 768), (1024, 16, 2048)],
)
def test_matmul_within_fp32_bound(n, k, m):
    a, b = _u((n, k), n), _u((k, m), m)
    _check(G.matmul(a, b), a, b)


@pytest.mark.parametrize("shape_a, shape_b", [((5, 130, 70), (5, 70, 90)),
                                              ((3, 128, 32), (3, 32, 256))])
def test_batched_matches_per_batch(shape_a, shape_b):
    a, b = _u(shape_a, 3), _u(shape_b, 4)
    got = G.matmul_batched(a, b)
    for i in range(shape_a[0]):
        _check(got[i], a[i], b[i])


def test_identity_and_integers_are_exact():
    a = _u((200, 136), 5)
    assert np.array_equal(G.matmul(a, np.eye(136, dtype=np.float32)), a)
    a = _u((256, 512), 6)   # tile-aligned: the LDS-DMA kernel
    assert np.array_equal(G.matmul(a, np.eye(512, dtype=np.float32)), a)
    rng = np.random.default_rng(6)
    ai = rng.integers(-8, 8, (150, 260)).astype(np.float32)
    bi = rng.integers(-8, 8, (260, 90)).astype(np.float32)
    assert np.array_equal(G.matmul(ai, bi), (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 4096), (16384, 1024, 3072)])
def test_config4_shapes_sampled(n, k, m):
    """Full product on the GPU; 96 rows (first, last, random) against the CPU path."""
    a, b = _u((n, k), 7), _u((k, m), 8)
    got = G.matmul(a, b)
    rows = np.unique(np.concatenate([[0, 1, n - 1], np.random.default_rng(9).integers(0, n, 93)]))
    exact = oracle.matmul(a[rows], b, threads=True)
    _check(got[rows], a[rows], b, exact)


def _stored(x, trans):
    """The operand as gemm_ex reads it: its transpose, contiguous, if trans."""
    return np.ascontiguousarray(np.swapaxes(x, -1, -2)) if trans else x


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize(
    "n,k,m",
    [(33, 17, 65), (100, 70, 90), (128, 16, 256), (256, 48, 512),      # unaligned / fast path
     (128, 4096, 256), (1024, 8192, 1024), (256, 2048, 768),           # split-K: few tiles, long k
     (384, 1040, 512), (1024, 1024, 3072)],                            # uneven split, no split
)
def test_gemm_ex_transposes_within_fp32_bound(n, k, m, ta, tb):
    a, b = _u((n, k), n + k), _u((k, m), m + 1)
    _check(G.gemm_ex(_stored(a, ta), _stored(b, tb), ta, tb), a, b)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)])
def test_gemm_ex_batched_split(ta, tb):
    a, b = _u((3, 128, 2048), 5), _u((3, 2048, 256), 6)
    got = G.gemm_ex(_stored(a, ta), _stored(b, tb), ta, tb)
    for i in range(3):
        _check(got[i], a[i], b[i])


@pytest.mark.parametrize("n,k,m,ta,tb,batch",
                         [(8192, 1024, 1024, False, False, 1), (8192, 4096, 1024, False, True, 1),
                          (1024, 512, 512, True, False, 1), (512, 96, 256, True, True, 2),
                          (256, 64, 768, False, False, 3)])
def test_gemm_two_k_groups(n, k, m, ta, tb, batch):
    """Outputs with no more 128 x 256 tiles than CUs and an even slab count
    take the kernel whose workgroup splits the k-slabs between two wave
    groups (even / odd slabs, summed through LDS): config 5's 8192 x 1024
    products, transposed operands, batches, and a 4-slab minimum."""
    a, b = _u((batch, n, k), n + k), _u((batch, k, m), m + 2)
    sa = np.stack([_stored(a[i], ta) for i in range(batch)])
    sb = np.stack([_stored(b[i], tb) for i in range(batch)])
    got = G.gemm_ex(sa if batch > 1 else sa[0], sb if batch > 1 else sb[0], ta, tb)
    got = got.reshape(batch, n, m)
    rows = np.random.default_rng(n).choice(n, min(n, 64), replace=False)
    for i in range(batch):
        _check(got[i][rows], a[i][rows], b[i])


@pytest.mark.parametrize("n,k,m", [(128, 4096, 256), (256, 64, 512), (70, 40, 30)])
def test_gemm_ex_epilogue_with_and_without_split(n, k, m):
    """bias + residual, and bias + GELU with pre, through the split-K reduction
    (first shape), the fused store (second) and the fallback kernel (third)."""
    a, b = _u((n, k), 7), _u((k, m), 8)
    bias, res = _u((m,), 9), _u((n, m), 10)
    exact = oracle.matmul(a, b, threads=True).astype(np.float64)
    bound = G.gemm_error_bound(a, b)
    got = G.gemm_ex(_stored(a, True), b, True, False, bias=bias, residual=res)
    ref = exact + bias + res
    assert (np.abs(got - ref) <= bound + 1e-6 * (1 + np.abs(ref))).all()
    assert_north_star(got, ref)
    y, pre = G.gemm_ex(a, _stored(b, True), False, True, bias=bias, act=1)
    assert (np.abs(pre - (exact + bias)) <= bound + 1e-6 * (1 + np.abs(exact))).all()
    assert_north_star(pre, exact + bias)
    np.testing.assert_allclose(y, oracle.gelu_fwd(pre), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n,k,m,tb", [(4096, 64, 4096, False), (4096, 48, 4096, True),
                                      (16384, 32, 3072, False)])
def test_gemm_256_row_tiles(n, k, m, tb):
    """Outputs whose 256 x 256 tiles fill whole waves of CUs take the 8-wave
    kernel (256-row tiles)."""
    a, b = _u((n, k), 11), _u((k, m), 12)
    _check(G.gemm_ex(a, _stored(b, tb), False, tb), a, b)


def test_gemm_256_row_tiles_epilogue():
    n, k, m = 4096, 32, 4096
    a, b = _u((n, k), 13), _u((k, m), 14)
    bias, res = _u((m,), 15), _u((n, m), 16)
    exact = oracle.matmul(a, b, threads=True).astype(np.float64)
    bound = G.gemm_error_bound(a, b)
    got = G.gemm_ex(a, b, bias=bias, residual=res)
    ref = exact + bias + res
    assert (np.abs(got - ref) <= bound + 1e-6 * (1 + np.abs(ref))).all()
    assert_north_star(got, ref)
    y, pre = G.gemm_ex(a, b, bias=bias, act=1)
    assert (np.abs(pre - (exact + bias)) <= bound + 1e-6 * (1 + np.abs(exact))).all()
    assert_north_star(pre, exact + bias)
    np.testing.assert_allclose(y, oracle.gelu_fwd(pre), rtol=1e-5, atol=1e-6)


def test_large_row_pitch_takes_the_checked_kernel():
    """k >= 2^22: the tile-aligned fast path addresses a tile's rows with
    32-bit byte offsets, so a row pitch this large must go to the generic
    (64-bit indexed) kernel.  a in {0, 1} and b = 1 make every output an
    integer below 2^24, exact in any fp32 summation order."""
    n, m, k = 128, 256, (1 << 22) + 16
    rng = np.random.default_rng(11)
    a = rng.integers(0, 2, size=(n, k), dtype=np.uint8).astype(np.float32)
    b = np.ones((k, m), dtype=np.float32)
    out = G.gemm_ex(a, b)
    del b
    rows = a.sum(axis=1, dtype=np.float64).astype(np.float32)
    assert np.array_equal(out, np.broadcast_to(rows[:, None], (n, m)))


@pytest.mark.parametrize("n,m", [(5, 7), (128, 256)])
def test_empty_inner_dimension_gives_empty_sums(n, m):
    """k = 0: every output is an empty sum, 0, as in the reference's loop
    (operators_cpu.c:47-60).  Through the C ABI, and through Tensor @, whose
    empty operands carry null device pointers; gemm_ex then applies its
    epilogue to the zeros."""
    from ember_amd import Tensor

    a = np.zeros((n, 0), np.float32)
    b = np.zeros((0, m), np.float32)
    out = G.matmul(a, b)
    assert out.shape == (n, m) and not out.any()
    t = Tensor(a) @ Tensor(b)
    assert t.shape == (n, m) and not t.to_np().any()
    bias = np.linspace(-2, 2, m).astype(np.float32)
    res = np.random.default_rng(3).standard_normal((n, m)).astype(np.float32)
    got, pre = G.gemm_ex(a, b, bias=bias, residual=res, act=1)
    full = np.ascontiguousarray(np.broadcast_to(bias, (n, m)))
    assert np.array_equal(pre, full)
    np.testing.assert_allclose(got, oracle.gelu_fwd(full) + res, rtol=1e-6, atol=1e-6)
