"""Parity of the HIP flash-attention forward/backward with the CPU oracle.

Tolerance (from the project's north star): max-abs 2e-4 / rel 1e-3 in
fp32 for O, LSE, dQ, dK, dV; mask handling and tile boundaries are checked
bitwise through invariants that any leak across the mask would break.
All calls go through the C ABI (libember_amd.so).
"""

import ctypes

import numpy as np
import pytest

import gpu_helpers as G
import oracle

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-3, atol=2e-4)


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def _inputs(B, H, S, D, seed=0):
    return tuple(_rand((B, H, S, D), seed + i) for i in range(4))


# ------------------------------------------------------------ golden fixtures


def _gpu_cases(golden):
    return [n for n, c in golden.items() if c["q"].shape[-1] in (32, 64, 128)]


def test_forward_matches_golden(golden):
    for name in _gpu_cases(golden):
        c = golden[name]
        o, lse = G.attention_fwd(c["q"], c["k"], c["v"], bool(c["causal"]), float(c["scale"]))
        np.testing.assert_allclose(o, c["o"], err_msg=name, **TOL)
        np.testing.assert_allclose(lse, c["lse"], err_msg=name, **TOL)


def test_backward_matches_golden(golden):
    for name in _gpu_cases(golden):
        c = golden[name]
        causal, scale = bool(c["causal"]), float(c["scale"])
        o, lse = G.attention_fwd(c["q"], c["k"], c["v"], causal, scale)
        dq, dk, dv = G.attention_bwd(c["q"], c["k"], c["v"], o, lse, c["do"], causal, scale)
        for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            np.testing.assert_allclose(got, c[key], err_msg=f"{name}/{key}", **TOL)


# ------------------------------------------------------------ edges and sizes


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("S", [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 257])
@pytest.mark.parametrize("causal", [False, True])
def test_fwd_bwd_edges_match_oracle(S, D, causal):
    q, k, v, d_o = _inputs(1, 2, S, D, seed=S * 7 + D)
    o, lse = G.attention_fwd(q, k, v, causal)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, causal)
    np.testing.assert_allclose(o, o_ref, **TOL)
    np.testing.assert_allclose(lse, lse_ref, **TOL)
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    dq_r, dk_r, dv_r = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, causal)
    np.testing.assert_allclose(dq, dq_r, **TOL)
    np.testing.assert_allclose(dk, dk_r, **TOL)
    np.testing.assert_allclose(dv, dv_r, **TOL)


@pytest.mark.parametrize("B,H,S,D,causal", [(3, 3, 20, 64, True), (3, 3, 50, 128, False),
                                           (1, 5, 32, 32, True), (2, 3, 64, 128, True),
                                           (5, 1, 7, 128, False), (2, 7, 33, 64, False)])
def test_short_sequences_pack_heads(B, H, S, D, causal):
    """S <= 64 packs 2 or 4 heads into a workgroup; head counts that do not
    fill the last workgroup must neither leak nor write past the last head."""
    q, k, v, d_o = _inputs(B, H, S, D, seed=S + D + B * H)
    o, lse = G.attention_fwd(q, k, v, causal)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, causal, G.scale_for(D))
    np.testing.assert_allclose(o, o_ref, **TOL)
    np.testing.assert_allclose(lse, lse_ref, **TOL)
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    refs = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, causal, G.scale_for(D))
    for got, ref in zip((dq, dk, dv), refs):
        np.testing.assert_allclose(got, ref, **TOL)


@pytest.mark.parametrize("B,H,S,D,causal", [(4, 20, 257, 64, True), (2, 40, 129, 128, False),
                                           (4, 17, 200, 32, True), (3, 30, 300, 128, True)])
def test_full_width_launches_with_ragged_length(B, H, S, D, causal):
    """Enough heads that the forward takes its one-head-per-workgroup path
    (small launches split the keys across waves instead, covered by the
    edge cases above), with S not a multiple of the 128-query block."""
    q, k, v, d_o = _inputs(B, H, S, D, seed=S + H)
    o, lse = G.attention_fwd(q, k, v, causal)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, causal)
    np.testing.assert_allclose(o, o_ref, **TOL)
    np.testing.assert_allclose(lse, lse_ref, **TOL)


def test_config1_forward_full():
    """B=1 H=4 S=256 D=64 non-causal: full O against the CPU path."""
    q, k, v, _ = _inputs(1, 4, 256, 64, seed=100)
    o, lse = G.attention_fwd(q, k, v, False)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, False)
    np.testing.assert_allclose(o, o_ref, **TOL)
    np.testing.assert_allclose(lse, lse_ref, **TOL)


def test_config2_causal_forward_slices():
    """B=8 H=16 S=2048 D=64 causal, whole problem on the GPU, three heads checked."""
    q, k, v, _ = _inputs(8, 16, 2048, 64, seed=200)
    o, lse = G.attention_fwd(q, k, v, True)
    for b, h in ((0, 0), (0, 15), (7, 3)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        o_ref, lse_ref = oracle.attention_fwd(q[sl], k[sl], v[sl], True)
        np.testing.assert_allclose(o[sl], o_ref, err_msg=f"b={b} h={h}", **TOL)
        np.testing.assert_allclose(lse[sl], lse_ref, err_msg=f"b={b} h={h}", **TOL)


def test_config3_causal_fwd_bwd_slice():
    """B=4 H=32 S=4096 D=128 causal fwd+bwd on the GPU; B=1 H=2 slice vs CPU."""
    q, k, v, d_o = _inputs(4, 32, 4096, 128, seed=300)
    o, lse = G.attention_fwd(q, k, v, True)
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, True)
    sl = (slice(0, 1), slice(0, 2))
    o_ref, lse_ref = oracle.attention_fwd(q[sl], k[sl], v[sl], True)
    np.testing.assert_allclose(o[sl], o_ref, **TOL)
    np.testing.assert_allclose(lse[sl], lse_ref, **TOL)
    dq_r, dk_r, dv_r = oracle.attention_bwd(q[sl], k[sl], v[sl], o_ref, lse_ref, d_o[sl], True)
    np.testing.assert_allclose(dq[sl], dq_r, **TOL)
    np.testing.assert_allclose(dk[sl], dk_r, **TOL)
    np.testing.assert_allclose(dv[sl], dv_r, **TOL)
    # Size-independent properties over all 128 heads:
    #   sum_j dV_j = sum_i dO_i          (rows of P sum to 1)
    #   sum_j dK_j = 0                   (sum_j dS_ij = sum_j P_ij dP_ij - delta_i = 0)
    assert np.isfinite(dq).all() and np.isfinite(dk).all() and np.isfinite(dv).all()
    sum_dv = dv.astype(np.float64).sum(axis=2)
    sum_do = d_o.astype(np.float64).sum(axis=2)
    np.testing.assert_allclose(sum_dv, sum_do, rtol=1e-4, atol=1e-3)
    sum_dk = np.abs(dk.astype(np.float64).sum(axis=2))
    assert (sum_dk <= 1e-3 * np.abs(dk.astype(np.float64)).sum(axis=2) + 1e-4).all()


# ------------------------------------------------------- bitwise invariants


@pytest.mark.parametrize("S,D", [(300, 64), (300, 128), (64, 128), (40, 64)])
def test_causal_mask_does_not_leak(S, D):
    """Changing keys/values after row i leaves O and LSE of rows <= i bitwise unchanged."""
    q, k, v, _ = _inputs(1, 1, S, D, seed=400 + D)
    o, lse = G.attention_fwd(q, k, v, True)
    for i in (x for x in (0, 31, 32, 63, 64, 127, 128, 200) if x < S - 1):
        k2, v2 = k.copy(), v.copy()
        k2[0, 0, i + 1:] = _rand((S - i - 1, D), i)
        v2[0, 0, i + 1:] = _rand((S - i - 1, D), i + 1)
        o2, lse2 = G.attention_fwd(q, k2, v2, True)
        assert np.array_equal(o[0, 0, : i + 1], o2[0, 0, : i + 1]), i
        assert np.array_equal(lse[0, 0, : i + 1], lse2[0, 0, : i + 1]), i
    assert np.array_equal(o[0, 0, 0], v[0, 0, 0])  # row 0 attends key 0 only


def test_keys_past_the_end_do_not_leak():
    """Non-causal S=65: rows are identical whether or not the buffer has junk after S."""
    S, D = 65, 64
    q, k, v, _ = _inputs(1, 1, S, D, seed=500)
    o, lse = G.attention_fwd(q, k, v, False)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, False)
    np.testing.assert_allclose(o, o_ref, **TOL)
    np.testing.assert_allclose(lse, lse_ref, **TOL)


def test_forward_is_deterministic():
    q, k, v, _ = _inputs(2, 3, 200, 128, seed=600)
    a = G.attention_fwd(q, k, v, True)
    b = G.attention_fwd(q, k, v, True)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_backward_zero_upstream_gradient_is_exactly_zero():
    q, k, v, _ = _inputs(1, 2, 150, 64, seed=700)
    o, lse = G.attention_fwd(q, k, v, True)
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, np.zeros_like(q), True)
    assert not dq.any() and not dk.any() and not dv.any()


def test_backward_last_key_sees_only_last_query():
    S, D = 129, 64
    q, k, v, d_o = _inputs(1, 1, S, D, seed=800)
    o, lse = G.attention_fwd(q, k, v, True)
    _, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, True)
    s = G.scale_for(D) * float(np.dot(q[0, 0, -1].astype(np.float64), k[0, 0, -1]))
    p = np.exp(s - float(lse[0, 0, -1]))
    np.testing.assert_allclose(dv[0, 0, -1], p * d_o[0, 0, -1], **TOL)


# ------------------------------------------------------------ strided layout


@pytest.mark.parametrize("S,D", [(160, 64), (48, 128), (300, 128)])
def test_packed_qkv_layout(S, D):
    """q, k, v read from one (B, S, 3, H, D) buffer; o / dO in (B, S, H, D)
    (S = 48, D = 128 takes the one-wave-per-query-block forward)."""
    from ember_amd import capi
    from ember_amd.capi import DeviceArray

    B, H = 2, 4
    qkv = _rand((B, S, 3, H, D), 900)
    d_o_bshd = _rand((B, S, H, D), 901)
    q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    d_o = np.ascontiguousarray(d_o_bshd.transpose(0, 2, 1, 3))
    o_ref, lse_ref = G.attention_fwd(q, k, v, True)
    dq_ref, dk_ref, dv_ref = G.attention_bwd(q, k, v, o_ref, lse_ref, d_o, True)

    G.say("packed qkv layout")
    L = capi.lib()
    dqkv = DeviceArray.from_numpy(qkv)
    ddo = DeviceArray.from_numpy(d_o_bshd)
    o = DeviceArray((B, S, H, D))
    lse = DeviceArray((B, H, S))
    grads = DeviceArray((B, S, 3, H, D))
    in_st = (S * 3 * H * D, D, 3 * H * D)
    out_st = (S * H * D, D, H * D)
    base, step = dqkv.ptr, H * D * 4
    st = L.attention_fwd(base, base + step, base + 2 * step, o.ptr, lse.ptr, B, H, S, D,
                         G.scale_for(D), 1, *in_st, *out_st)
    capi.check(st, "attention_fwd")
    gb = grads.ptr
    st = L.attention_bwd(base, base + step, base + 2 * step, o.ptr, lse.ptr, ddo.ptr,
                         gb, gb + step, gb + 2 * step, B, H, S, D, G.scale_for(D), 1,
                         *in_st, *out_st)
    capi.check(st, "attention_bwd")
    o_np = o.numpy().transpose(0, 2, 1, 3)
    g = grads.numpy()
    assert np.array_equal(o_np, o_ref)
    assert np.array_equal(lse.numpy(), lse_ref)
    assert np.array_equal(g[:, :, 1].transpose(0, 2, 1, 3), dk_ref)
    assert np.array_equal(g[:, :, 2].transpose(0, 2, 1, 3), dv_ref)
    np.testing.assert_allclose(g[:, :, 0].transpose(0, 2, 1, 3), dq_ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("S", [96, 160])
def test_row_stride_at_the_guard_edge(S):
    """Row stride 2^24 - 4 floats, the largest the entry points accept (rows
    64 MiB apart): the forward's HBM->LDS copies address a 64-key tile's
    rows with 32-bit byte offsets up to 4 * 63 * (2^24 - 4), past 2^31.
    65 heads of S = 96 make the forward take its one-head-per-workgroup
    kernel and the backward attn_bwd_s128; at S = 160 the backward takes
    attn_bwd_w16, whose dQ rows past 127 sit more than 2^31 floats from the
    head's first.  q / k / v of a head sit side by side in each row.  A
    stride of 2^24 is rejected with EMBER_ERR_INVALID_ARGUMENT before any
    launch."""
    from ember_amd import capi
    from ember_amd.capi import DeviceArray

    B, H, D = 1, 65, 64
    ss = (1 << 24) - 4
    width = 3 * H * D
    rows = _rand((S, H, 3, D), 950)
    d_o = _rand((B, H, S, D), 951)
    q, k, v = (np.ascontiguousarray(rows[:, :, i].transpose(1, 0, 2))[None] for i in range(3))
    scale = G.scale_for(D)
    L = capi.lib()
    G.say(f"row stride {ss} floats: B={B} H={H} S={S} D={D} causal (two {S * ss * 4 / 2**30:.1f} GiB buffers)")
    buf, gbuf = DeviceArray((S * ss,)), DeviceArray((S * ss,))
    for r in range(S):
        L.copy_to_device(buf.ptr + 4 * r * ss, np.ascontiguousarray(rows[r]).ctypes.data, 4 * width)
    capi.check(what="copy_to_device")
    o, lse = DeviceArray((B, H, S, D)), DeviceArray((B, H, S))
    ddo = DeviceArray.from_numpy(d_o)
    in_st, out_st = (S * ss, 3 * D, ss), capi.contiguous_strides(B, H, S, D)
    base, gb = buf.ptr, gbuf.ptr
    capi.check(L.attention_fwd(base, base + 4 * D, base + 8 * D, o.ptr, lse.ptr, B, H, S, D, scale, 1,
                               *in_st, *out_st), "attention_fwd")
    capi.check(L.attention_bwd(base, base + 4 * D, base + 8 * D, o.ptr, lse.ptr, ddo.ptr,
                               gb, gb + 4 * D, gb + 8 * D, B, H, S, D, scale, 1, *in_st, *out_st),
               "attention_bwd")
    o_np, lse_np = o.numpy(), lse.numpy()
    g = np.empty((S, width), np.float32)
    for r in range(S):
        L.copy_from_device(g[r].ctypes.data, gb + 4 * r * ss, 4 * width)
    capi.check(what="copy_from_device")
    g = g.reshape(S, H, 3, D)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, True, scale)
    np.testing.assert_allclose(o_np, o_ref, **TOL)
    np.testing.assert_allclose(lse_np, lse_ref, **TOL)
    refs = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, True, scale)
    for i, (name, ref) in enumerate(zip(("dq", "dk", "dv"), refs)):
        np.testing.assert_allclose(g[:, :, i].transpose(1, 0, 2)[None], ref, err_msg=name, **TOL)
    del buf, gbuf

    too_far = (S * (1 << 24), 3 * D, 1 << 24)
    st = L.attention_fwd(o.ptr, o.ptr, o.ptr, o.ptr, lse.ptr, B, H, S, D, scale, 1, *too_far, *out_st)
    assert st == 1 and L.ember_get_last_error() == 1   # EMBER_ERR_INVALID_ARGUMENT
    st = L.attention_bwd(o.ptr, o.ptr, o.ptr, o.ptr, lse.ptr, ddo.ptr, o.ptr, o.ptr, o.ptr, B, H, S, D,
                         scale, 1, *too_far, *out_st)
    assert st == 1 and L.ember_get_last_error() == 1


@pytest.mark.parametrize("S,D,kernel", [(50, 64, "attn_bwd_lds16_r64"), (50, 128, "attn_bwd_short_lds64p")])
def test_short_backward_row_stride_at_the_guard_edge(S, D, kernel):
    """Row stride 2^24 - 4 floats at S <= 64, where the backward runs a
    persistent LDS-staged kernel whose stores are branch-free and bounded:
    a store for a row past S (rows 50..63 of the 64-row tile) takes an
    offset past the store descriptor's range, and at this stride the range
    is 4 * (49 * (2^24 - 4) + D) bytes, past 2^31.  One head; q / k / v side
    by side in each row, the gradients in a buffer of the same layout filled
    with SENTINEL first: every gradient matches the oracle and the padding
    of every row (the 256 floats after its data) is untouched."""
    from ember_amd import capi
    from ember_amd.capi import DeviceArray

    B, H = 1, 1
    ss = (1 << 24) - 4
    width = 3 * H * D
    rows = _rand((S, H, 3, D), 960 + D)
    d_o = _rand((B, H, S, D), 961 + D)
    q, k, v = (np.ascontiguousarray(rows[:, :, i].transpose(1, 0, 2))[None] for i in range(3))
    scale = G.scale_for(D)
    L = capi.lib()
    L.constant.argtypes = [ctypes.c_float, ctypes.c_void_p, ctypes.c_int]
    G.say(f"short backward, row stride {ss} floats: S={S} D={D} (two {S * ss * 4 / 2**30:.1f} GiB buffers)")
    buf, gbuf = DeviceArray((S * ss,)), DeviceArray((S * ss,))
    L.constant(G.SENTINEL, gbuf.ptr, S * ss)
    for r in range(S):
        L.copy_to_device(buf.ptr + 4 * r * ss, np.ascontiguousarray(rows[r]).ctypes.data, 4 * width)
    capi.check(what="copy_to_device")
    o, lse = DeviceArray((B, H, S, D)), DeviceArray((B, H, S))
    ddo = DeviceArray.from_numpy(d_o)
    in_st, out_st = (S * ss, 3 * D, ss), capi.contiguous_strides(B, H, S, D)
    base, gb = buf.ptr, gbuf.ptr
    capi.check(L.attention_fwd(base, base + 4 * D, base + 8 * D, o.ptr, lse.ptr, B, H, S, D, scale, 1,
                               *in_st, *out_st), "attention_fwd")
    capi.launch_log_reset()
    capi.check(L.attention_bwd(base, base + 4 * D, base + 8 * D, o.ptr, lse.ptr, ddo.ptr,
                               gb, gb + 4 * D, gb + 8 * D, B, H, S, D, scale, 1, *in_st, *out_st),
               "attention_bwd")
    assert kernel in capi.launch_log()
    span = width + 256
    g = np.empty((S, span), np.float32)
    for r in range(S):
        L.copy_from_device(g[r].ctypes.data, gb + 4 * r * ss, 4 * span)
    capi.check(what="copy_from_device")
    assert np.all(g[:, width:] == G.SENTINEL)
    g = g[:, :width].reshape(S, H, 3, D)
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, True, scale)
    refs = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, True, scale)
    for i, (name, ref) in enumerate(zip(("dq", "dk", "dv"), refs)):
        np.testing.assert_allclose(g[:, :, i].transpose(1, 0, 2)[None], ref, err_msg=name, **TOL)
    del buf, gbuf


# ------------------------------------------------------------ long sequences


def _f64_reference(q, k, v, d_o, causal, scale, chunk=1024):
    """float64 O and LSE of every row of one head, streamed over row chunks
    (the S x S scores of a chunk at a time), and Delta = rowsum(dO * O)."""
    S, D = q.shape
    q64, k64, v64 = (x.astype(np.float64) for x in (q, k, v))
    o = np.empty((S, D))
    lse = np.empty(S)
    for r0 in range(0, S, chunk):
        r1 = min(S, r0 + chunk)
        nk = r1 if causal else S
        s = (q64[r0:r1] @ k64[:nk].T) * scale
        if causal:
            s[np.arange(r1 - r0)[:, None] + r0 < np.arange(nk)[None, :]] = -np.inf
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        l = p.sum(axis=1, keepdims=True)
        o[r0:r1] = (p @ v64[:nk]) / l
        lse[r0:r1] = (m + np.log(l))[:, 0]
    delta = (d_o.astype(np.float64) * o).sum(axis=1)
    return o, lse, delta


@pytest.mark.parametrize("S,D,causal", [(16384, 128, True), (8192, 64, False)])
def test_long_sequence_against_float64(S, D, causal):
    """The longest loops (S/32 query blocks per key block): O and LSE of every
    row, dQ of sampled rows and dK, dV of sampled keys against a float64
    NumPy evaluation of the same formulas (closed-form gradients)."""
    q, k, v, d_o = _inputs(1, 1, S, D, seed=1100 + D)
    scale = G.scale_for(D)
    o, lse = G.attention_fwd(q, k, v, causal)
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    q0, k0, v0, g0 = q[0, 0], k[0, 0], v[0, 0], d_o[0, 0]
    o_r, lse_r, delta = _f64_reference(q0, k0, v0, g0, causal, scale)
    np.testing.assert_allclose(o[0, 0], o_r, **TOL)
    np.testing.assert_allclose(lse[0, 0], lse_r, **TOL)
    q64, k64, v64, g64 = (x.astype(np.float64) for x in (q0, k0, v0, g0))
    picks = sorted({0, 1, 31, 32, 127, 128, S // 2, S - 129, S - 33, S - 1}
                   | set(np.random.default_rng(S).choice(S, 16, replace=False).tolist()))
    for i in picks:  # dQ_i = scale sum_j P_ij (dO_i . V_j - Delta_i) K_j
        nk = i + 1 if causal else S
        p = np.exp(scale * (k64[:nk] @ q64[i]) - lse_r[i])
        ds = p * (v64[:nk] @ g64[i] - delta[i])
        np.testing.assert_allclose(dq[0, 0, i], scale * (ds @ k64[:nk]), err_msg=f"dQ row {i}", **TOL)
    for j in picks:  # dV_j = sum_i P_ij dO_i, dK_j = scale sum_i dS_ij Q_i
        i0 = j if causal else 0
        p = np.exp(scale * (q64[i0:] @ k64[j]) - lse_r[i0:])
        ds = p * (g64[i0:] @ v64[j] - delta[i0:])
        np.testing.assert_allclose(dv[0, 0, j], p @ g64[i0:], err_msg=f"dV row {j}", **TOL)
        np.testing.assert_allclose(dk[0, 0, j], scale * (ds @ q64[i0:]), err_msg=f"dK row {j}", **TOL)


def _check_against_oracle(q, k, v, d_o, causal, scale, grad_atol):
    o, lse = G.attention_fwd(q, k, v, causal, scale)
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, causal, scale)
    np.testing.assert_allclose(o, o_ref, **TOL)
    np.testing.assert_allclose(lse, lse_ref, rtol=1e-5, atol=2e-4)
    grads = G.attention_bwd(q, k, v, o, lse, d_o, causal, scale)
    refs = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, causal, scale)
    for name, got, ref in zip(("dq", "dk", "dv"), grads, refs):
        assert np.isfinite(got).all(), name
        G.say(f"  {name}: max |err| {float(np.max(np.abs(got - ref))):.3g} (atol {grad_atol:.3g})")
        np.testing.assert_allclose(got, ref, rtol=1e-3, atol=grad_atol, err_msg=f"{name} scale={scale}")
    return lse


@pytest.mark.parametrize("S,D,causal", [(1024, 128, True), (513, 128, False), (300, 64, True), (64, 64, True),
                                         (200, 32, False)])
def test_running_max_climbs_along_the_keys(S, D, causal):
    """Key j carries a component (32 j / S) u along a direction u that every
    query shares, so each row's maximum score climbs by ~32 (natural log
    units) over the keys: the running maximum, which the forward raises
    lazily (only when a score exceeds it by more than 2^8 in base 2, i.e.
    5.5), is raised five or more times along a full row, and a wrong rescale
    of O or of the running sum would show at once.  Scores stay within
    ~+-40, so the north-star tolerance applies unchanged."""
    q, k, v, d_o = _inputs(1, 2, S, D, seed=1400 + S + D)
    u = np.ones(D, np.float32) / np.sqrt(D)
    q = (q + 4.0 * u).astype(np.float32)                    # q . u ~ 4
    k = (k + (8.0 * np.arange(S) / S)[:, None].astype(np.float32) * u * np.sqrt(D)).astype(np.float32)
    G.say(f"climbing max S={S} D={D} causal={causal}")
    _check_against_oracle(q, k, v, d_o, causal, G.scale_for(D), 2e-4)


@pytest.mark.parametrize("S,D,causal", [(1024, 128, True), (513, 128, False), (200, 32, False)])
def test_peaked_scores_and_zero_scale(S, D, causal):
    """Scale 1 with q, k ~ N(0, 4): scores with a standard deviation of
    sigma = 4 sqrt(D) (up to ~+-200), softmax rows close to one-hot.  O and
    LSE are held to the north-star tolerance.  The gradients' absolute
    tolerance is the north star's times sigma: the backward recomputes each
    score in fp32, with an absolute rounding of order |s| D 2^-24 that
    perturbs P relatively by as much, and dK, dQ sum such terms against
    Q, K of magnitude 2 (measured: 0.9e-3 to 1.6e-3 worst absolute error
    in dQ and dK at D = 128, against 2e-4 sigma = 9e-3; 1e-5 to 5e-5 in the
    climbing-maximum test above, at ordinary score magnitudes).  Then
    scale 0: every visible key gets exactly the same weight
    (LSE = ln(count)), at the north star."""
    q, k, v, d_o = _inputs(1, 2, S, D, seed=1500 + S + D)
    q, k = 2.0 * q, 2.0 * k
    sigma = 4.0 * np.sqrt(D)
    G.say(f"peaked scores S={S} D={D} causal={causal}")
    _check_against_oracle(q, k, v, d_o, causal, 1.0, 2e-4 * sigma)
    G.say(f"zero scale S={S} D={D} causal={causal}")
    lse = _check_against_oracle(q, k, v, d_o, causal, 0.0, 2e-4)
    n = np.arange(1, S + 1) if causal else np.full(S, S)
    np.testing.assert_allclose(lse[0, 0], np.log(n), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("B,H,S,D,causal", [
    (64, 64, 128, 128, True),    # 16-key-chunk workgroup kernel, 4096 heads
    (32, 64, 130, 64, False),    # two key blocks, atomic dQ, 2048 heads
    (128, 64, 64, 128, True),    # persistent S <= 64 kernel, 8192 heads
    (256, 64, 32, 64, False),    # one-head LDS workgroups, 16384 heads
])
def test_many_heads_sampled(B, H, S, D, causal):
    """The bench's short-sequence scale (2^19-2^20 query rows, thousands of
    heads): every output finite, and the first, a middle and the last head
    against the oracle."""
    rng = np.random.default_rng(1600 + S + D)
    q, k, v, d_o = (rng.standard_normal((B, H, S, D), dtype=np.float32) for _ in range(4))
    o, lse = G.attention_fwd(q, k, v, causal)
    grads = G.attention_bwd(q, k, v, o, lse, d_o, causal)
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    assert all(np.isfinite(g).all() for g in grads)
    for b, h in ((0, 0), (B // 2, H // 3), (B - 1, H - 1)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        o_ref, lse_ref = oracle.attention_fwd(q[sl], k[sl], v[sl], causal)
        np.testing.assert_allclose(o[sl], o_ref, err_msg=f"O b={b} h={h}", **TOL)
        np.testing.assert_allclose(lse[sl], lse_ref, err_msg=f"LSE b={b} h={h}", **TOL)
        refs = oracle.attention_bwd(q[sl], k[sl], v[sl], o_ref, lse_ref, d_o[sl], causal)
        for name, got, ref in zip(("dQ", "dK", "dV"), grads, refs):
            np.testing.assert_allclose(got[sl], ref, err_msg=f"{name} b={b} h={h}", **TOL)


@pytest.mark.parametrize("S,D", [(131072, 64), (65536, 128)])
def test_very_long_sequence_sampled_rows(S, D):
    """One causal head of 64k-128k rows, beyond the oracle's reach: O and
    LSE of sampled rows against float64 (each an O(S D) sum), and the
    backward's contract on sampled rows and keys in float64 from the given O
    and LSE (P = exp(scale q.k - LSE), Delta = dO.O): dQ rows, dK and dV
    keys.  The row, block and statistic offsets here exceed 2^22 elements
    per tensor, the largest index products of any test."""
    q, k, v, d_o = _inputs(1, 1, S, D, seed=1300 + D)
    scale = G.scale_for(D)
    o, lse = G.attention_fwd(q, k, v, True)
    dq, dk, dv = G.attention_bwd(q, k, v, o, lse, d_o, True)
    q64, k64, v64, g64 = (x[0, 0].astype(np.float64) for x in (q, k, v, d_o))
    o64, lse64 = o[0, 0].astype(np.float64), lse[0, 0].astype(np.float64)
    delta = (g64 * o64).sum(axis=1)
    picks = sorted({0, 1, 127, 128, S // 2 - 1, S // 2, S - 129, S - 2, S - 1}
                   | set(np.random.default_rng(S + D).choice(S, 8, replace=False).tolist()))
    for i in picks:
        sc = scale * (k64[:i + 1] @ q64[i])
        m = sc.max()
        w = np.exp(sc - m)
        ref_lse = m + np.log(w.sum())
        np.testing.assert_allclose(lse[0, 0, i], ref_lse, err_msg=f"LSE row {i}", **TOL)
        np.testing.assert_allclose(o[0, 0, i], (w @ v64[:i + 1]) / w.sum(), err_msg=f"O row {i}", **TOL)
        p = np.exp(sc - lse64[i])
        ds = p * (v64[:i + 1] @ g64[i] - delta[i])
        np.testing.assert_allclose(dq[0, 0, i], scale * (ds @ k64[:i + 1]), err_msg=f"dQ row {i}", **TOL)
    for j in picks:
        p = np.exp(scale * (q64[j:] @ k64[j]) - lse64[j:])
        ds = p * (g64[j:] @ v64[j] - delta[j:])
        np.testing.assert_allclose(dv[0, 0, j], p @ g64[j:], err_msg=f"dV row {j}", **TOL)
        np.testing.assert_allclose(dk[0, 0, j], scale * (ds @ q64[j:]), err_msg=f"dK row {j}", **TOL)


@pytest.mark.parametrize("D,causal", [(128, True), (64, False)])
def test_known_answers_at_full_length(D, causal):
    """Closed forms at S = 4096 on the HIP kernels themselves: K = 0 makes
    every score equal, so row i averages V[0..i] (causal) or all of V, with
    LSE = ln(i+1) or ln(S); V = 1 gives O = 1; and (non-causal) permuting
    keys together with values leaves O and LSE unchanged."""
    S = 4096
    q, k, v, _ = _inputs(1, 2, S, D, seed=1200 + D)
    o, lse = G.attention_fwd(q, np.zeros_like(k), v, causal)
    v64 = v.astype(np.float64)
    if causal:
        mean = np.cumsum(v64, axis=2) / np.arange(1, S + 1)[None, None, :, None]
        ln_n = np.log(np.arange(1, S + 1, dtype=np.float64))
    else:
        mean = np.broadcast_to(v64.mean(axis=2, keepdims=True), v64.shape)
        ln_n = np.full(S, np.log(S))
    np.testing.assert_allclose(o, mean, **TOL)
    np.testing.assert_allclose(lse, np.broadcast_to(ln_n, lse.shape), rtol=1e-6, atol=1e-6)
    o1, _ = G.attention_fwd(q, k, np.ones_like(v), causal)
    np.testing.assert_allclose(o1, 1.0, rtol=0, atol=1e-5)
    if not causal:
        perm = np.random.default_rng(D).permutation(S)
        o2, lse2 = G.attention_fwd(q, k[:, :, perm], v[:, :, perm], causal)
        o3, lse3 = G.attention_fwd(q, k, v, causal)
        np.testing.assert_allclose(o2, o3, **TOL)
        np.testing.assert_allclose(lse2, lse3, **TOL)
