"""Config 5 at its full size on the GPU: one pre-LN decoder-block training
step (d_model 1024, 16 heads of 64, S 1024, B 8, causal; Xavier weights and
N(0,1) token embeddings, all seeded) and the attention launch inside it.

* The attention launch: B8 H16 S1024 D64 causal, q / k / v read in place
  from the packed (B, S, 3, H, D) projection and O / dO in (B, S, H, D)
  (the strides the block uses), through the C ABI; three heads against the
  CPU oracle at the north-star tolerance, and the packed launch bitwise equal
  to the contiguous one for O, LSE, dK, dV.
* The step: forward, Ember's MSELoss, backward, one fused Adam step, against
  the float64 restatement of the block (oracle/decoder.py) over the whole
  batch: y at the north-star tolerance; dx and all 12 parameter gradients in
  units of (y - target), i.e. divided by the loss's gradient scale
  2/n = 2^-22 (an exact power of two); the loss value; the MSE gradient
  bitwise; and the post-Adam parameters bitwise against the oracle's Adam
  (Ember's op order, ember/optim/adam.py:33-45) applied to the GPU's
  gradients.
  Tolerance of the gradients: dx at the north star.  Each parameter
  gradient is a sum over all B*S = 8192 token rows, so its entries are about
  sqrt(8192) ~ 90 times the per-row terms, and an fp32 sum of 8192 such
  terms carries an absolute rounding error proportional to its partial sums,
  not to its (possibly tiny) final value.  Each parameter gradient is
  therefore held to the north-star tolerance in units of its own RMS (when
  that is above 1): |err| <= 2e-4 * max(1, rms(ref)) + 1e-3 |ref|.  The
  measured errors are printed (first run: worst |err| = 1.65 x the unscaled
  atol, in w_1's gradient, whose RMS is far above 1).
Reference pieces: ember/nn/layers.py:45-56 (Linear), ember/nn/activations.py
:56-66 (GELU), ember/loss/losses.py:19-26 (MSELoss), ember/optim/adam.py.
"""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from oracle import decoder
from tolerance import assert_north_star, north_star_ratio

pytestmark = pytest.mark.gpu

B, S, H, D = 8, 1024, 16, 64
DM = H * D


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_config5_attention_packed_launch():
    from ember_amd import capi
    from ember_amd.capi import DeviceArray

    qkv = _rand((B, S, 3, H, D), 501)
    d_o_bshd = _rand((B, S, H, D), 502)
    scale = G.scale_for(D)
    L = capi.lib()
    G.say(f"config-5 attention, packed strides B={B} H={H} S={S} D={D} causal")
    dqkv, ddo = DeviceArray.from_numpy(qkv), DeviceArray.from_numpy(d_o_bshd)
    o, lse = DeviceArray((B, S, H, D)), DeviceArray((B, H, S))
    grads = DeviceArray((B, S, 3, H, D))
    in_st, out_st = (S * 3 * DM, D, 3 * DM), (S * DM, D, DM)
    base, step = dqkv.ptr, DM * 4
    capi.check(L.attention_fwd(base, base + step, base + 2 * step, o.ptr, lse.ptr, B, H, S, D,
                               scale, 1, *in_st, *out_st), "attention_fwd")
    gb = grads.ptr
    capi.check(L.attention_bwd(base, base + step, base + 2 * step, o.ptr, lse.ptr, ddo.ptr,
                               gb, gb + step, gb + 2 * step, B, H, S, D, scale, 1, *in_st, *out_st),
               "attention_bwd")
    o_np = o.numpy().transpose(0, 2, 1, 3)               # (B, H, S, D)
    lse_np = lse.numpy()
    g = grads.numpy()
    dq, dk, dv = (g[:, :, i].transpose(0, 2, 1, 3) for i in range(3))
    q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    d_o = np.ascontiguousarray(d_o_bshd.transpose(0, 2, 1, 3))

    for b, h in ((0, 0), (3, 7), (7, 15)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        o_ref, lse_ref = oracle.attention_fwd(q[sl], k[sl], v[sl], True, scale)
        assert_north_star(o_np[sl], o_ref, f"O b={b} h={h}")
        assert_north_star(lse_np[sl], lse_ref, f"LSE b={b} h={h}")
        refs = oracle.attention_bwd(q[sl], k[sl], v[sl], o_ref, lse_ref, d_o[sl], True, scale)
        for name, got, ref in zip(("dQ", "dK", "dV"), (dq, dk, dv), refs):
            assert_north_star(got[sl], ref, f"{name} b={b} h={h}")

    # The same problem in contiguous (B, H, S, D) tensors: the kernels see
    # only the strides, so O, LSE, dK and dV must be identical bit for bit
    # (dQ is summed with atomics in a run-dependent order).
    o_c, lse_c = G.attention_fwd(q, k, v, True, scale)
    assert np.array_equal(o_c, o_np) and np.array_equal(lse_c, lse_np)
    dq_c, dk_c, dv_c = G.attention_bwd(q, k, v, o_c, lse_c, d_o, True, scale)
    assert np.array_equal(dk_c, dk) and np.array_equal(dv_c, dv)
    np.testing.assert_allclose(dq_c, dq, rtol=1e-5, atol=1e-6)


def test_config5_decoder_step_full_size():
    from ember_amd import Tensor, loss, nn, optim
    from ember_amd import random as em_random

    G.say(f"config-5 decoder step d={DM} H={H} S={S} B={B}: GPU forward/backward/Adam")
    em_random.seed(5)
    block = nn.DecoderBlock(DM, H, 4, causal=True)       # Xavier weights from the seeded generator
    params0 = [p.to_np().copy() for p in block.parameters()]
    x = _rand((B * S, DM), 503)
    target = _rand((B * S, DM), 504)
    y = block(Tensor(x), B, S)
    mse = loss.MSELoss()
    loss_val = mse(y, Tensor(target))
    dy = mse.backward()
    dx = block.backward(dy)
    grads = [g.to_np() for g in block.gradients()]
    opt = optim.Adam(block.parameters(), lr=1e-3)
    opt.apply(block.gradients())
    params1 = [p.to_np() for p in block.parameters()]
    y_np, dy_np, dx_np = y.to_np(), dy.to_np(), dx.to_np()

    n = y_np.size
    inv = float(n) / 2.0                                   # 2^22: exact rescaling
    diff = y_np.astype(np.float64) - target.astype(np.float64)
    np.testing.assert_allclose(loss_val, float((diff * diff).mean()), rtol=1e-5)
    assert np.array_equal(dy_np, (y_np - target) * np.float32(2.0 / n))

    G.say("config-5 decoder step: float64 oracle forward")
    y_ref, cache = decoder.forward(params0, x, B, S, H, True)
    assert_north_star(y_np, y_ref, "y")
    G.say("config-5 decoder step: float64 oracle backward")
    dx_ref, g_ref = decoder.backward(params0, cache, dy_np, B, S, H)
    names = ["ln1.gamma", "ln1.beta", "w_qkv", "b_qkv", "w_o", "b_o", "ln2.gamma", "ln2.beta",
             "w_1", "b_1", "w_2", "b_2"]
    rows = [("dx", dx_np * inv, dx_ref * inv, 1.0)]
    for name, got, ref in zip(names, grads, g_ref):
        ref_n = ref * inv
        rows.append((name, got * inv, ref_n, max(1.0, float(np.sqrt(np.mean(ref_n * ref_n))))))
    for name, got, ref, r in rows:
        err = float(np.max(np.abs(got.astype(np.float64) - ref)))
        G.say(f"config-5 {name}: rms(ref) {float(np.sqrt(np.mean(ref * ref))):.4g}, max|err| {err:.3g}, "
              f"unscaled ratio {north_star_ratio(got, ref):.3f}, ratio in rms units {north_star_ratio(got / r, ref / r):.4f}")
    for name, got, ref, r in rows:
        assert_north_star(got / r, ref / r, f"grad {name} (in units of max(1, rms) = {r:.4g})")

    G.say("config-5 decoder step: Adam against the oracle")
    for name, p0, g, p1 in zip(names, params0, grads, params1):
        p, m, v = p0.reshape(-1).copy(), np.zeros(p0.size, np.float32), np.zeros(p0.size, np.float32)
        oracle.adam_step(p, np.ascontiguousarray(g.reshape(-1)), m, v, 1e-3, 0.9, 0.999, 1e-8, 1)
        assert np.array_equal(p, p1.reshape(-1)), f"Adam {name}"
