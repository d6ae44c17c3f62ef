"""Deterministic mode (ember_set_deterministic) of attention_bwd on the GPU.

With the switch on, the kernels that add dQ with atomics (S > 128, S > 64
at D = 32) add each 16- or 32-row dQ tile's key-block contributions in a
fixed order, highest key block first (ordered dQ: a counter per tile, O(S)
scratch), instead of in arrival order.  Checked here, on contiguous and
padded layouts, causal or not, every head dim, S from 65 (one key block with
a tail) to 32768 (512 key blocks of 64):
* dQ is bitwise identical over repeated launches, with default-mode
  launches in between (the default mode's atomics vary the order);
* dK and dV are bitwise the default mode's (same kernels but for the order
  of the dQ adds), and dQ agrees with the default mode's to fp32 rounding;
* dQ, dK, dV agree with the CPU oracle at the north-star tolerance
  (max-abs 2e-4 / rel 1e-3), or with float64 on sampled rows where the
  oracle cannot reach, and padding stays untouched;
* no wait for a tile's turn gave up (ember_deterministic_timeouts() == 0),
  so every order above was the fixed one;
* the Python front end (ember_amd.set_deterministic + attention_backward)
  takes the same path.
S <= 64, and S <= 128 at D = 64 and 128 (attn_bwd_s128), have no atomics in
either mode; one such case each checks that the switch leaves them bitwise
alone.  S <= 128 at D = 32 takes the atomic kernel and is among the cases.
"""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from ember_amd import capi
from ember_amd.capi import DeviceArray

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-3, atol=2e-4)


@pytest.fixture
def deterministic():
    capi.set_deterministic(True)
    try:
        yield
    finally:
        capi.set_deterministic(False)


class _Problem:
    """One attention problem resident on the device in padded layouts."""

    def __init__(self, B, H, S, D, causal, pads, hpads, seed):
        rng = np.random.default_rng(seed)
        self.shape = (B, H, S, D)
        self.causal = causal
        self.q, self.k, self.v, self.d_o = (rng.standard_normal(self.shape).astype(np.float32)
                                            for _ in range(4))
        self.in_st, self.in_tot = G.padded_strides(B, H, S, D, pads[0], hpads[0])
        self.out_st, self.out_tot = G.padded_strides(B, H, S, D, pads[1], hpads[1])
        self.scale = G.scale_for(D)
        self.dev = [G.upload_padded(x, self.in_st, self.in_tot) for x in (self.q, self.k, self.v)]
        self.ddo = G.upload_padded(self.d_o, self.out_st, self.out_tot)
        self.o = G.upload_padded(np.zeros_like(self.q), self.out_st, self.out_tot)
        self.lse = DeviceArray((B, H, S))
        L = capi.lib()
        capi.check(L.attention_fwd(*(x.ptr for x in self.dev), self.o.ptr, self.lse.ptr, B, H, S, D,
                                   self.scale, int(causal), *self.in_st, *self.out_st), "attention_fwd")

    def backward(self):
        """(dq, dk, dv) as (B, H, S, D) arrays, and the padded buffers."""
        B, H, S, D = self.shape
        grads = [G.upload_padded(np.zeros_like(self.q), self.in_st, self.in_tot) for _ in range(3)]
        L = capi.lib()
        capi.check(L.attention_bwd(*(x.ptr for x in self.dev), self.o.ptr, self.lse.ptr, self.ddo.ptr,
                                   *(g.ptr for g in grads), B, H, S, D, self.scale, int(self.causal),
                                   *self.in_st, *self.out_st), "attention_bwd")
        out = [G.download_padded(g, self.in_st, self.shape) for g in grads]
        return [o[0] for o in out], [o[1] for o in out]


CASES = [
    # B, H, S, D, causal, pads, hpads
    (1, 2, 4096, 128, True, [0, 0], [0, 0]),     # config 3's slice: 32 key blocks
    (2, 3, 300, 64, False, [4, 12], [1, 0]),
    (1, 4, 200, 32, True, [0, 32], [3, 1]),
    (2, 2, 129, 128, False, [12, 4], [0, 3]),
    (3, 5, 1000, 64, True, [0, 0], [0, 0]),
    (1, 1, 65, 32, False, [0, 0], [0, 0]),
    (3, 3, 100, 128, True, [4, 0], [0, 1]),      # S <= 128 at D = 128: attn_bwd_s128, no atomics
    (2, 16, 1024, 64, True, [0, 0], [0, 0]),     # config 5's shape per head, 32 heads
]


@pytest.mark.parametrize("B,H,S,D,causal,pads,hpads", CASES)
def test_deterministic_dq_is_reproducible_and_exact(B, H, S, D, causal, pads, hpads, deterministic):
    G.say(f"deterministic bwd B={B} H={H} S={S} D={D} causal={causal} pads={pads} hpads={hpads}")
    p = _Problem(B, H, S, D, causal, pads, hpads, seed=S + D + B * H)
    (dq1, dk1, dv1), bufs = p.backward()
    capi.set_deterministic(False)
    (dq_a, dk_a, dv_a), _ = p.backward()                # atomic dQ, in between
    (dq_b, _, _), _ = p.backward()
    capi.set_deterministic(True)
    (dq2, dk2, dv2), _ = p.backward()

    assert np.array_equal(dq1, dq2)
    assert np.array_equal(dk1, dk2) and np.array_equal(dv1, dv2)
    assert np.array_equal(dk1, dk_a) and np.array_equal(dv1, dv_a)
    np.testing.assert_allclose(dq1, dq_a, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dq_b, dq_a, rtol=1e-5, atol=1e-6)
    for name, buf in zip(("dq", "dk", "dv"), bufs):
        assert np.count_nonzero(buf == G.SENTINEL) == p.in_tot - B * H * S * D, name

    assert capi.deterministic_timeouts() == 0

    # The oracle on at most 4 heads (config 3's slice is 2).
    nh = min(H, 4)
    sl = (slice(0, 1), slice(0, nh))
    o_ref, lse_ref = oracle.attention_fwd(p.q[sl], p.k[sl], p.v[sl], causal, p.scale)
    refs = oracle.attention_bwd(p.q[sl], p.k[sl], p.v[sl], o_ref, lse_ref, p.d_o[sl], causal, p.scale)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq1, dk1, dv1), refs):
        np.testing.assert_allclose(got[sl], ref, err_msg=name, **TOL)


@pytest.mark.parametrize("B,H,S,D,causal", [(4, 8, 48, 64, True), (2, 6, 112, 128, True),
                                             (3, 5, 128, 64, False)])
def test_deterministic_switch_leaves_short_sequences_alone(B, H, S, D, causal, deterministic):
    """S <= 64, and S <= 128 at D = 64 or 128: the same kernels in both
    modes (no atomics there)."""
    p = _Problem(B, H, S, D, causal, [4, 0], [1, 0], seed=7 + S)
    (dq1, dk1, dv1), _ = p.backward()
    capi.set_deterministic(False)
    (dq0, dk0, dv0), _ = p.backward()
    for a, b in ((dq1, dq0), (dk1, dk0), (dv1, dv0)):
        assert np.array_equal(a, b)


def test_front_end_deterministic_backward():
    import ember_amd as em
    from ember_amd import Tensor

    rng = np.random.default_rng(11)
    q, k, v, d_o = (rng.standard_normal((2, 4, 384, 64)).astype(np.float32) for _ in range(4))
    tq, tk, tv, tdo = (Tensor(x) for x in (q, k, v, d_o))
    o, lse = em.attention_forward(tq, tk, tv, causal=True)
    assert em.is_deterministic() is False
    em.set_deterministic(True)
    try:
        assert em.is_deterministic() is True
        first = [g.to_np() for g in em.attention_backward(tq, tk, tv, o, lse, tdo, causal=True)]
        again = [g.to_np() for g in em.attention_backward(tq, tk, tv, o, lse, tdo, causal=True)]
    finally:
        em.set_deterministic(False)
    for a, b in zip(first, again):
        assert np.array_equal(a, b)
    o_ref, lse_ref = oracle.attention_fwd(q[:1, :2], k[:1, :2], v[:1, :2], True)
    refs = oracle.attention_bwd(q[:1, :2], k[:1, :2], v[:1, :2], o_ref, lse_ref, d_o[:1, :2], True)
    for got, ref in zip(first, refs):
        np.testing.assert_allclose(got[:1, :2], ref, **TOL)


@pytest.mark.parametrize("S,D,causal", [(32768, 64, True), (16384, 128, True), (8192, 64, False)])
def test_deterministic_long_sequence(S, D, causal, deterministic):
    """B=1 H=2 at up to S = 32768: O(S) scratch (the tile counters), so long
    sequences run in deterministic mode as in the default mode.  dQ is
    bitwise repeatable, dK and dV are bitwise the default mode's, and dQ
    rows, dK and dV keys at tile edges and random positions agree with
    float64 evaluations of the closed-form gradients from the given O and
    LSE (P = exp(scale q.k - LSE), Delta = dO.O)."""
    rng = np.random.default_rng(S + D)
    q, k, v, d_o = (rng.standard_normal((1, 2, S, D), dtype=np.float32) for _ in range(4))
    scale = G.scale_for(D)
    o, lse = G.attention_fwd(q, k, v, causal)
    dq1, dk1, dv1 = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    dq2, dk2, dv2 = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    assert capi.deterministic_timeouts() == 0
    assert np.array_equal(dq1, dq2) and np.array_equal(dk1, dk2) and np.array_equal(dv1, dv2)
    capi.set_deterministic(False)
    _, dk0, dv0 = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    capi.set_deterministic(True)
    assert np.array_equal(dk1, dk0) and np.array_equal(dv1, dv0)
    picks = sorted({0, 1, 15, 16, 63, 64, 127, 128, S // 2, S - 65, S - 17, S - 1}
                   | set(rng.choice(S, 8, replace=False).tolist()))
    for h in range(2):
        q64, k64, v64, g64 = (x[0, h].astype(np.float64) for x in (q, k, v, d_o))
        lse64 = lse[0, h].astype(np.float64)
        delta = (g64 * o[0, h].astype(np.float64)).sum(axis=1)
        for i in picks:
            nk = i + 1 if causal else S
            p = np.exp(scale * (k64[:nk] @ q64[i]) - lse64[i])
            ds = p * (v64[:nk] @ g64[i] - delta[i])
            np.testing.assert_allclose(dq1[0, h, i], scale * (ds @ k64[:nk]), err_msg=f"dQ {h}/{i}", **TOL)
        for j in picks:
            i0 = j if causal else 0
            p = np.exp(scale * (q64[i0:] @ k64[j]) - lse64[i0:])
            ds = p * (g64[i0:] @ v64[j] - delta[i0:])
            np.testing.assert_allclose(dv1[0, h, j], p @ g64[i0:], err_msg=f"dV {h}/{j}", **TOL)
            np.testing.assert_allclose(dk1[0, h, j], scale * (ds @ q64[i0:]), err_msg=f"dK {h}/{j}", **TOL)
