"""Bit-exact causal masking on every attention kernel the library dispatches.

The causal predicate (key j visible to query i iff j <= i) is integer work,
so its contract is bitwise, not within a tolerance.  Each kernel is reached
by a launch shape chosen for it, and the launch log (ember_launch_log) shows
that the intended kernel ran.  Per launch, every head h gets a cutoff c_h at
a tile edge (multiples of 16, 32, 64, 128 and +-1) or inside a tile, and:

forward (O, LSE):
  * K and V rows > c_h replaced by fresh values leave O and LSE rows <= c_h
    bitwise unchanged (a key past the diagonal that leaked into a row's max,
    sum or O would move it);
  * row 0 sees key 0 only, so O_0 == V_0 in every head (to two ulp: its
    weight is exp2 of the score's rounding error), and the cutoff-0 case
    above shows bitwise that no later key reaches it;
backward (dQ, dK, dV, with O and LSE passed in unchanged):
  * Q, dO, O and LSE rows < c_h replaced leave dK and dV rows >= c_h
    bitwise unchanged (query i < j must contribute exactly zero to key j);
  * K and V rows > c_h replaced leave dQ rows <= c_h bitwise unchanged
    (key j > i must contribute exactly zero to query i), and dK, dV rows
    <= c_h as well (with O and LSE fixed, key j's gradient reads only row j
    of K and V).  Kernels whose dQ is added with atomics run this check in
    deterministic mode, whose per-row sum order is fixed; a launch that runs
    only with atomic dQ (key-block pairs) holds dQ to the reordering of a
    sum (1e-5) instead.
Two tilings (forward): the same head through a split-key kernel (in a
small launch) and through attn_fwd_kernel (single or paired query blocks), attn_fwd_head or
attn_fwd_wave_pair (among 65 heads) agrees within the north-star tolerance and with the CPU oracle, and
both pass the cutoff check above.  Every launch's first and last head are also held to the oracle
at the north-star tolerance.

The slot these kernels fill is the reference's src/tensor/operators.h:20-27;
the composed form they replace adds the mask before softmax
(ember/tensor/tensor.py:430-437).
"""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from ember_amd import capi

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-3, atol=2e-4)

_EDGES = (0, 1, 15, 16, 17, 31, 32, 33, 47, 63, 64, 65, 95, 96, 97, 111, 127, 128, 129,
          191, 255, 256, 257, 383, 511, 512, 513, 767, 1023)


def _cutoff_rounds(nheads, S, seed, max_rounds=32):
    """Cutoffs per head for successive launches, so that every tile edge
    below S - 1 (and S - 2) is some head's cutoff in some launch; heads past
    the edges take random rows."""
    edges = [c for c in _EDGES if c < S - 1] + [S - 2]
    rng = np.random.default_rng(seed)
    rounds = min(max_rounds, -(-len(edges) // nheads))
    out = []
    for r in range(rounds):
        idx = [r * nheads + h for h in range(nheads)]
        out.append(np.array([edges[i] if i < len(edges) else int(rng.integers(0, S - 1)) for i in idx]))
    return out


def _rand(shape, rng):
    return rng.standard_normal(shape, dtype=np.float32)


def _replace_after(x, cut, rng):
    """x (B, H, S, D) with rows > cut[h] of head h (flattened B*H) replaced."""
    B, H, S, D = x.shape
    y = x.reshape(B * H, S, D).copy()
    for h, c in enumerate(cut):
        y[h, c + 1:] = _rand((S - c - 1, D), rng)
    return y.reshape(x.shape)


def _replace_before(x, cut, rng, scale=1.0, add=False):
    """x (B, H, S[, D]) with rows < cut[h] of head h replaced (or, add=True,
    shifted) by `scale` times fresh values."""
    B, H, S = x.shape[:3]
    y = x.reshape((B * H, S) + x.shape[3:]).copy()
    for h, c in enumerate(cut):
        fresh = scale * _rand((c,) + x.shape[3:], rng)
        y[h, :c] = y[h, :c] + fresh if add else fresh
    return y.reshape(x.shape)


def _rows_equal(a, b, cut, upto):
    """Heads' rows <= cut (upto) or >= cut (not upto) of a and b are bitwise equal."""
    B, H, S = a.shape[:3]
    a = a.reshape((B * H, S) + a.shape[3:])
    b = b.reshape((B * H, S) + b.shape[3:])
    for h, c in enumerate(cut):
        rows = slice(0, c + 1) if upto else slice(c, S)
        if not np.array_equal(a[h, rows], b[h, rows]):
            bad = np.nonzero(np.any((a[h, rows] != b[h, rows]).reshape(a[h, rows].shape[0], -1), axis=1))[0]
            return f"head {h} cutoff {c}: rows {(bad + rows.start)[:8].tolist()} differ"
    return None


def _oracle_heads(q, k, v, o, lse, heads):
    B, H = q.shape[:2]
    for f in heads:
        b, h = divmod(f, H)
        sl = (slice(b, b + 1), slice(h, h + 1))
        o_ref, lse_ref = oracle.attention_fwd(q[sl], k[sl], v[sl], True)
        np.testing.assert_allclose(o[sl], o_ref, err_msg=f"O head {f}", **TOL)
        np.testing.assert_allclose(lse[sl], lse_ref, err_msg=f"LSE head {f}", **TOL)


# (kernel, B, H, S, D): each shape reaches the named forward kernel.
FWD_CASES = [
    ("attn_fwd_split16", 1, 1, 300, 128),      # <= 256 16-query workgroups, 4 waves
    ("attn_fwd_split16", 1, 4, 128, 64),
    ("attn_fwd_split16", 1, 3, 100, 64),
    ("attn_fwd_split16_w8", 1, 2, 300, 64),    # 8 waves (D = 64, S > 128)
    ("attn_fwd_split16_w8", 1, 4, 1024, 64),
    ("attn_fwd_split16_w8", 1, 4, 256, 64),    # config 1's shape
    ("attn_fwd_split16_w8", 1, 1, 4096, 64),   # 32 tiles per wave
    ("attn_fwd_split", 1, 5, 1024, 64),        # <= 64 one-head 128-query blocks, > 256 of 16
    ("attn_fwd_split", 1, 3, 2048, 128),
    ("attn_fwd_split", 1, 2, 129, 32),         # D = 32
    ("attn_fwd_kernel", 1, 65, 129, 128),      # 128-query workgroups
    ("attn_fwd_kernel", 1, 65, 300, 64),
    ("attn_fwd_kernel", 1, 130, 1024, 128),    # block pairs would exceed one round: single blocks
    ("attn_fwd_kernel", 1, 200, 1024, 64),
    ("attn_fwd_kernel", 1, 65, 200, 32),
    ("attn_fwd_kernel_pairs", 1, 33, 1024, 128),  # blocks nqb - 1 - p and p per workgroup
    ("attn_fwd_kernel_pairs", 1, 40, 1024, 64),
    ("attn_fwd_kernel_pairs", 1, 40, 640, 64),    # odd nqb: the middle block alone
    ("attn_fwd_kernel_pairs", 1, 30, 600, 32),
    ("attn_fwd_head", 1, 65, 128, 64),         # persistent whole-head workgroups, D = 64
    ("attn_fwd_head", 1, 300, 80, 64),         # more heads than CUs: each workgroup walks several
    ("attn_fwd_head", 1, 70, 113, 64),
    ("attn_fwd_head", 1, 65, 97, 64),
    ("attn_fwd_wave_pair", 1, 65, 80, 128),    # one wave per pair of query blocks
    ("attn_fwd_wave_pair", 1, 65, 128, 128),
    ("attn_fwd_wave_pair", 1, 70, 113, 128),
    ("attn_fwd_wave", 1, 65, 64, 128),         # one wave per query block, S <= 64
    ("attn_fwd_wave", 1, 65, 40, 64),
    ("attn_fwd_wave", 1, 9, 17, 128),
    ("attn_fwd_packed_hp4", 1, 65, 32, 32),    # 4 heads per workgroup, S <= 32
    ("attn_fwd_packed_hp4", 1, 7, 20, 32),
    ("attn_fwd_packed_hp2", 1, 65, 64, 32),    # 2 heads per workgroup, S <= 64
    ("attn_fwd_packed_hp2", 1, 9, 50, 32),
]


def _forward_cutoff_check(q, k, v, rounds, kernel, seed):
    log = []
    o, lse = G.attention_fwd(q, k, v, True, log=log)
    assert log == [kernel], log
    # Row 0 sees key 0 only: O_0 = V_0 * p / l with p = l = exp2 of the
    # rounding error of the scaled score (1 to within an ulp), so O_0 is V_0
    # to within two ulp; that no key after 0 reaches row 0 is the bitwise
    # statement, checked by the cutoff-0 case below.
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], rtol=2.5e-7, atol=0, err_msg=f"{kernel}: O_0")
    rng = np.random.default_rng(seed)
    for cut in rounds:
        k2, v2 = _replace_after(k, cut, rng), _replace_after(v, cut, rng)
        o2, lse2 = G.attention_fwd(q, k2, v2, True)
        err = _rows_equal(o, o2, cut, True) or _rows_equal(lse, lse2, cut, True)
        assert err is None, f"{kernel}: {err}"
    return o, lse


@pytest.mark.parametrize("kernel,B,H,S,D", FWD_CASES)
def test_forward_mask_is_bit_exact(kernel, B, H, S, D):
    rng = np.random.default_rng(S * 131 + D + H)
    q, k, v = (_rand((B, H, S, D), rng) for _ in range(3))
    G.say(f"forward mask {kernel} B={B} H={H} S={S} D={D}")
    o, lse = _forward_cutoff_check(q, k, v, _cutoff_rounds(B * H, S, S + D), kernel, S + 7)
    _oracle_heads(q, k, v, o, lse, (0, B * H - 1))


@pytest.mark.parametrize("S,D,H1,alone,other", [
    (300, 128, 1, "attn_fwd_split16", "attn_fwd_kernel"),
    (1024, 64, 5, "attn_fwd_split", "attn_fwd_kernel_pairs"),
    (1024, 64, 1, "attn_fwd_split16_w8", "attn_fwd_kernel_pairs"),
    (128, 64, 1, "attn_fwd_split16", "attn_fwd_head"),
    (96, 128, 1, "attn_fwd_split16", "attn_fwd_wave_pair"),
    (100, 128, 1, "attn_fwd_split16", "attn_fwd_wave_pair"),
    (2048, 128, 3, "attn_fwd_split", "attn_fwd_kernel"),
])
def test_two_tilings_same_mask(S, D, H1, alone, other):
    """One head through a split-key kernel (16 or 32 queries per workgroup,
    four waves over interleaved 32-key tiles; as head 0 of H1) and through a
    second kernel (128-query blocks over 64-key tiles, whole heads staged in
    LDS with 16-query chunks, or one wave per pair of 32-query blocks) as
    head 7 of 65: both pass the cutoff check with the same
    cutoffs for that head, and agree with the oracle and with each other
    within the north-star tolerance."""
    rng = np.random.default_rng(S + D)
    q1, k1, v1 = (_rand((1, H1, S, D), rng) for _ in range(3))
    qs, ks, vs = (_rand((1, 65, S, D), rng) for _ in range(3))
    for big, one in ((qs, q1), (ks, k1), (vs, v1)):
        big[0, 7] = one[0, 0]
    one_rounds = _cutoff_rounds(H1, S, S)
    many_rounds = []
    for r, cut1 in enumerate(one_rounds):
        cut = _cutoff_rounds(65, S, S + r)[0]
        cut[7] = cut1[0]
        many_rounds.append(cut)
    G.say(f"two tilings S={S} D={D}: {alone}")
    o1, lse1 = _forward_cutoff_check(q1, k1, v1, one_rounds, alone, S)
    G.say(f"two tilings S={S} D={D}: {other}")
    o65, lse65 = _forward_cutoff_check(qs, ks, vs, many_rounds, other, S + 1)
    np.testing.assert_allclose(o65[0, 7], o1[0, 0], **TOL)
    np.testing.assert_allclose(lse65[0, 7], lse1[0, 0], **TOL)
    o_ref, lse_ref = oracle.attention_fwd(q1[:, :1], k1[:, :1], v1[:, :1], True)
    np.testing.assert_allclose(o1[:, :1], o_ref, **TOL)
    np.testing.assert_allclose(lse1[:, :1], lse_ref, **TOL)
    np.testing.assert_allclose(o65[:, 7:8], o_ref, **TOL)
    np.testing.assert_allclose(lse65[:, 7:8], lse_ref, **TOL)


# (kernel, B, H, S, D, deterministic dQ needed): each shape reaches the named
# backward kernel.
BWD_CASES = [
    ("attn_bwd_lds16_r32", 1, 8, 32, 128, False),       # S <= 32, D = 128: persistent, two per CU
    ("attn_bwd_lds16_r32", 1, 600, 17, 128, False),     # > 512 heads: a second pass
    ("attn_bwd_short_lds64p", 1, 300, 64, 128, False),  # persistent, > 256 heads
    ("attn_bwd_short_lds64p", 1, 5, 50, 128, False),
    ("attn_bwd_lds16_r32", 1, 8, 32, 64, False),        # S <= 32, D <= 64
    ("attn_bwd_lds16_r32", 1, 8, 25, 32, False),
    ("attn_bwd_lds16_r32", 1, 1000, 25, 64, False),   # persistent (S < 32 at D = 64), > 768 heads
    ("attn_bwd_lds16_r64", 1, 300, 64, 64, False),      # persistent at D = 64
    ("attn_bwd_lds16_r64", 1, 6, 48, 32, False),
    ("attn_bwd_s128", 1, 400, 72, 128, False),          # persistent, odd chunk count
    ("attn_bwd_s128", 1, 300, 100, 128, False),
    ("attn_bwd_s128", 1, 9, 128, 128, False),
    ("attn_bwd_s128", 1, 9, 128, 64, False),
    ("attn_bwd_s128", 1, 300, 112, 64, False),
    ("attn_bwd_kernel", 1, 4, 300, 128, True),          # key blocks of 128, dQ atomics
    ("attn_bwd_kernel", 1, 2, 1024, 128, True),
    ("attn_bwd_kernel", 1, 4, 129, 32, True),
    ("attn_bwd_kernel", 1, 3, 300, 32, True),
    ("attn_bwd_w16", 1, 4, 300, 64, True),              # key blocks of 64, dQ atomics
    ("attn_bwd_w16", 1, 2, 1024, 64, True),
    ("attn_bwd_w16", 1, 5, 129, 64, True),
]


@pytest.fixture
def restore_mode():
    yield
    capi.set_deterministic(False)


@pytest.mark.parametrize("kernel,B,H,S,D,det", BWD_CASES)
def test_backward_mask_is_bit_exact(kernel, B, H, S, D, det, restore_mode):
    rng = np.random.default_rng(S * 17 + D + H)
    q, k, v, d_o = (_rand((B, H, S, D), rng) for _ in range(4))
    o, lse = G.attention_fwd(q, k, v, True)
    capi.set_deterministic(det)
    G.say(f"backward mask {kernel} B={B} H={H} S={S} D={D} deterministic={det}")
    log = []
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, True, log=log)
    assert kernel in log, log

    for cut in _cutoff_rounds(B * H, S, S * 3 + D):
        # Queries before the cutoff must not reach keys at or after it.
        q2, d_o2, o2 = (_replace_before(x, cut, rng) for x in (q, d_o, o))
        lse2 = _replace_before(lse, cut, rng, scale=0.25, add=True)
        _, dk2, dv2 = G.attention_bwd(q2, k, v, o2, lse2, d_o2, True)
        err = _rows_equal(dk, dk2, cut, False) or _rows_equal(dv, dv2, cut, False)
        assert err is None, f"{kernel} dK/dV: {err}"

        # Keys after the cutoff must not reach queries at or before it.
        k3, v3 = _replace_after(k, cut, rng), _replace_after(v, cut, rng)
        dq3, dk3, dv3 = G.attention_bwd(q, k3, v3, o, lse, d_o, True)
        err = (_rows_equal(dq, dq3, cut, True) or _rows_equal(dk, dk3, cut, True)
               or _rows_equal(dv, dv3, cut, True))
        assert err is None, f"{kernel} dQ: {err}"

    for f in (0, B * H - 1):
        b, h = divmod(f, H)
        sl = (slice(b, b + 1), slice(h, h + 1))
        refs = oracle.attention_bwd(q[sl], k[sl], v[sl], o[sl], lse[sl], d_o[sl], True)
        for name, got, ref in zip(("dQ", "dK", "dV"), (dq, dk, dv), refs):
            np.testing.assert_allclose(got[sl], ref, err_msg=f"{name} head {f}", **TOL)


# (kernel, B, H, S, D): launches that run only with atomic dQ (the ordered
# dQ of deterministic mode follows single key blocks).
BWD_ATOMIC_CASES = [
    ("attn_bwd_w16_pairs", 1, 6, 1024, 64),   # key blocks p and nkb - 1 - p per workgroup
    ("attn_bwd_w16_pairs", 1, 5, 1030, 64),   # odd nkb: the middle block alone
]


@pytest.mark.parametrize("kernel,B,H,S,D", BWD_ATOMIC_CASES)
def test_backward_mask_atomic_dq(kernel, B, H, S, D, restore_mode):
    """As test_backward_mask_is_bit_exact, with dQ added by atomics in
    whatever order the hardware runs them: dK and dV bitwise, dQ rows at or
    before the cutoff equal to within the reordering of a sum (1e-5; one
    leaked key would move a row by about P * |dP - delta| * |K| * scale,
    about 1e-4 here)."""
    rng = np.random.default_rng(S * 19 + D + H)
    q, k, v, d_o = (_rand((B, H, S, D), rng) for _ in range(4))
    o, lse = G.attention_fwd(q, k, v, True)
    capi.set_deterministic(False)
    G.say(f"backward mask (atomic dQ) {kernel} B={B} H={H} S={S} D={D}")
    log = []
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, True, log=log)
    assert kernel in log, log
    for cut in _cutoff_rounds(B * H, S, S * 3 + D):
        q2, d_o2, o2 = (_replace_before(x, cut, rng) for x in (q, d_o, o))
        lse2 = _replace_before(lse, cut, rng, scale=0.25, add=True)
        _, dk2, dv2 = G.attention_bwd(q2, k, v, o2, lse2, d_o2, True)
        err = _rows_equal(dk, dk2, cut, False) or _rows_equal(dv, dv2, cut, False)
        assert err is None, f"{kernel} dK/dV: {err}"
        k3, v3 = _replace_after(k, cut, rng), _replace_after(v, cut, rng)
        dq3, dk3, dv3 = G.attention_bwd(q, k3, v3, o, lse, d_o, True)
        err = _rows_equal(dk, dk3, cut, True) or _rows_equal(dv, dv3, cut, True)
        assert err is None, f"{kernel} dK/dV (keys replaced): {err}"
        a, b3 = dq.reshape(B * H, S, D), dq3.reshape(B * H, S, D)
        for h, c in enumerate(cut):
            np.testing.assert_allclose(b3[h, :c + 1], a[h, :c + 1], rtol=1e-5, atol=1e-5,
                                       err_msg=f"{kernel} dQ head {h} cutoff {c}")
    for f in (0, B * H - 1):
        b, h = divmod(f, H)
        sl = (slice(b, b + 1), slice(h, h + 1))
        refs = oracle.attention_bwd(q[sl], k[sl], v[sl], o[sl], lse[sl], d_o[sl], True)
        for name, got, ref in zip(("dQ", "dK", "dV"), (dq, dk, dv), refs):
            np.testing.assert_allclose(got[sl], ref, err_msg=f"{name} head {f}", **TOL)
