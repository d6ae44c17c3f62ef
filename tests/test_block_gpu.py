"""Config 5's transformer-block pieces on the GPU: LayerNorm, the GEMM
epilogue (bias / Ember's GELU / residual), GELU backward, column sums, and
the whole pre-LN decoder block forward + backward + Adam step, each against
the CPU oracle (oracle/ember_oracle.c, oracle/decoder.py)."""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from ember_amd import Tensor, _core, loss, nn, optim
from oracle import decoder
from tolerance import assert_north_star

pytestmark = pytest.mark.gpu


def rnd(shape, seed, scale=1.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


@pytest.mark.parametrize("rows,d", [(1, 64), (7, 1024), (1000, 1024), (33, 4096), (5, 100),
                                    (8192, 1024), (70000, 64)])
def test_layernorm_fwd_bwd(rows, d):
    G.say(f"layernorm rows={rows} d={d}")
    x = rnd((rows, d), 1, 2.0) + 0.5
    g, b, dy = rnd((d,), 2), rnd((d,), 3), rnd((rows, d), 4)
    y, mean, rstd = _core._layernorm_fwd(Tensor(x)._core, Tensor(g)._core, Tensor(b)._core, rows, d, 1e-5)
    y_ref, mean_ref, rstd_ref = oracle.layernorm_fwd(x, g, b, 1e-5)
    np.testing.assert_allclose(y._to_np().reshape(rows, d), y_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mean._to_np(), mean_ref.reshape(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rstd._to_np(), rstd_ref.reshape(-1), rtol=1e-5)
    dx, dg, db = _core._layernorm_bwd(Tensor(x)._core, Tensor(g)._core, mean, rstd, Tensor(dy)._core, rows, d)
    dx_ref, dg_ref, db_ref = oracle.layernorm_bwd(x, g, mean._to_np(), rstd._to_np(), dy)
    np.testing.assert_allclose(dx._to_np().reshape(rows, d), dx_ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dg._to_np(), dg_ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(db._to_np(), db_ref, rtol=1e-4, atol=1e-4)
    # the residual gradient is added to dx in the same pass
    res = rnd((rows, d), 5)
    dx2, dg2, db2 = _core._layernorm_bwd(Tensor(x)._core, Tensor(g)._core, mean, rstd, Tensor(dy)._core,
                                         rows, d, Tensor(res)._core)
    np.testing.assert_allclose(dx2._to_np().reshape(rows, d), dx_ref + res, rtol=1e-4, atol=1e-5)
    np.testing.assert_array_equal(dg2._to_np(), dg._to_np())


def test_layernorm_rejects_bad_widths():
    x = Tensor(rnd((2, 6), 5))
    g = Tensor(rnd((6,), 6))
    with pytest.raises(ValueError):
        _core._layernorm_fwd(x._core, g._core, g._core, 2, 6, 1e-5)   # 6 % 4 != 0


@pytest.mark.parametrize("n,k,m", [(128, 64, 256), (256, 1024, 512), (100, 70, 90), (33, 17, 65)])
@pytest.mark.parametrize("mode", ["bias", "bias_residual", "gelu"])
def test_linear_epilogue(n, k, m, mode):
    G.say(f"linear {mode} n={n} k={k} m={m}")
    x, w, b, r = rnd((n, k), 7), rnd((k, m), 8, 0.1), rnd((m,), 9), rnd((n, m), 10)
    gelu = mode == "gelu"
    res = Tensor(r) if mode == "bias_residual" else None
    y, pre = nn.linear(Tensor(x), Tensor(w), Tensor(b), res, gelu)
    acc = oracle.matmul(x, w, threads=True).astype(np.float64) + b
    bound = G.gemm_error_bound(x, w) + 1e-6
    if gelu:
        assert np.all(np.abs(pre.to_np() - acc) <= bound)
        np.testing.assert_allclose(y.to_np(), oracle.gelu_fwd(pre.to_np()), rtol=1e-5, atol=1e-6)
    else:
        ref = acc + (r if res is not None else 0)
        assert pre is None
        assert np.all(np.abs(y.to_np() - ref) <= bound + 1e-6 * np.abs(ref))


def test_gelu_bwd_and_col_sum():
    u = rnd((5000,), 11, 2.0)
    a = oracle.gelu_fwd(u)
    dy = rnd((5000,), 12)
    dx = _core._gelu_bwd(Tensor(dy)._core, Tensor(u)._core, Tensor(a)._core)._to_np()
    np.testing.assert_allclose(dx, oracle.gelu_bwd(dy, u, a), rtol=1e-5, atol=1e-6)
    for rows, cols in ((1, 7), (300, 1024), (8192, 3), (0, 5), (8192, 1024), (256, 64), (100000, 12),
                       (257, 4096)):
        x = rnd((rows, cols), 13)
        got = nn.col_sum(Tensor(x) if rows else Tensor._from_core(_core._Tensor(0), (0, cols)))
        np.testing.assert_allclose(got.to_np(), x.astype(np.float64).sum(0), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (300, 1024), (257, 12), (256, 64), (5, 7), (1, 4)])
def test_gelu_bwd_col_sum_is_bitwise_the_two_calls(rows, cols):
    """_gelu_bwd_col_sum (one pass, dx summed as it is written) gives the
    same bits as _gelu_bwd followed by _col_sum: one 256-row slice, several
    slices, and an unaligned width (the two entry points in turn)."""
    G.say(f"gelu_bwd_col_sum rows={rows} cols={cols}")
    u, dy = rnd((rows, cols), 17, 3.0), rnd((rows, cols), 18)
    tu, tdy = Tensor(u), Tensor(dy)
    dx, db = _core._gelu_bwd_col_sum(tdy._core, tu._core, rows, cols)
    dx_ref = _core._gelu_bwd(tdy._core, tu._core)
    db_ref = _core._col_sum(dx_ref, rows, cols)
    assert np.array_equal(dx._to_np(), dx_ref._to_np())
    assert np.array_equal(db._to_np(), db_ref._to_np())
    np.testing.assert_allclose(db._to_np(), dx_ref._to_np().reshape(rows, cols).astype(np.float64).sum(0),
                               rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("n", [4096 * 33, 5001])
def test_gelu_bwd_recomputed_output_is_bitwise_the_stored_one(n):
    """_gelu_bwd(dy, u) recomputes the GELU output from u: bit-identical to
    passing the output that the GEMM epilogue or the composed GELU layer
    stored (float4 path for n % 4 == 0, scalar path otherwise)."""
    u = rnd((n,), 15, 3.0)
    dy = rnd((n,), 16)
    tu, tdy = Tensor(u), Tensor(dy)
    y_layer = nn.GELU()(tu)                                   # composed element-wise operators
    got = _core._gelu_bwd(tdy._core, tu._core)._to_np()
    stored = _core._gelu_bwd(tdy._core, tu._core, y_layer._core)._to_np()
    assert np.array_equal(got, stored)
    np.testing.assert_allclose(got, oracle.gelu_bwd(dy, u, oracle.gelu_fwd(u)), rtol=1e-5, atol=1e-6)
    if n % 1024 == 0:   # through the GEMM epilogue: out = GELU(pre), pre = x @ I
        rows = n // 1024
        xm = u.reshape(rows, 1024)
        y_epi, pre = nn.linear(Tensor(xm), Tensor(np.eye(1024, dtype=np.float32)), None, None, True)
        assert np.array_equal(pre.to_np(), xm)
        got2 = _core._gelu_bwd(tdy._core, pre._core)._to_np()
        stored2 = _core._gelu_bwd(tdy._core, pre._core, y_epi._core)._to_np()
        assert np.array_equal(got2, stored2) and np.array_equal(got2, got)


def _gpu_block_params(block):
    return [p.to_np().astype(np.float64) for p in block.parameters()]


@pytest.mark.parametrize("causal", [True, False])
def test_decoder_block_matches_oracle(causal):
    B, S, H, d = 2, 40, 2, 64
    G.say(f"decoder block B={B} S={S} H={H} d={d} causal={causal}")
    block = nn.DecoderBlock(d, H, 4, causal)
    params = decoder.init_params(d, H, 4, np.random.default_rng(14))
    for dev, host in zip(block.parameters(), params):   # give the block known parameters
        dev._adopt(Tensor(host.astype(np.float32)))
    x, dy = rnd((B * S, d), 15), rnd((B * S, d), 16)
    y = block(Tensor(x), B, S)
    dx = block.backward(Tensor(dy))
    y_ref, cache = decoder.forward(params, x, B, S, H, causal)
    dx_ref, g_ref = decoder.backward(params, cache, dy, B, S, H)
    assert_north_star(y.to_np(), y_ref, "y")
    assert_north_star(dx.to_np(), dx_ref, "dx")
    for i, (got, ref) in enumerate(zip(block.gradients(), g_ref)):
        assert_north_star(got.to_np(), ref, f"grad {i}")


def test_decoder_training_step_reduces_the_loss():
    """Config 5's step at a reduced size: forward, MSE, backward, fused Adam;
    the loss falls over the first steps."""
    B, S, H, d = 2, 128, 4, 128
    em_rng = np.random.default_rng(17)
    block = nn.DecoderBlock(d, H, 4, True)
    opt = optim.Adam(block.parameters(), lr=1e-3)
    mse = loss.MSELoss()
    x = Tensor(em_rng.standard_normal((B * S, d)).astype(np.float32))
    target = Tensor(em_rng.standard_normal((B * S, d)).astype(np.float32))
    losses = []
    for _ in range(5):
        y = block(x, B, S)
        losses.append(mse(y, target))
        block.backward(mse.backward())
        opt.apply(block.gradients())
    assert all(np.isfinite(losses)) and losses[-1] < losses[0]
