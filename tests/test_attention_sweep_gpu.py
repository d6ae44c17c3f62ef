"""A fixed-seed sweep of attention shapes and layouts against the CPU oracle.

Each case draws B, H, S, D, the mask and a layout: rows padded past D and
heads padded past S (strides that are not those of a contiguous tensor),
separately for the q/k/v/dq/dk/dv and the o/dO triples, so the kernels'
stride arithmetic and tile tails meet shapes no hand-written case lists.
The first sweep keeps B, H <= 3, so its launches with S > 64 are small
(ceil(S/128) * B * H <= 64 workgroups) and take the split-key forward; at
S <= 64 they take the packed and wave forwards and the short backwards.  The
second sweep draws enough heads that ceil(S/128) * B * H > 64, which sends
the forward to the one-head-per-workgroup kernel (attn_fwd_kernel) on the
same kind of padded strides.  The third keeps S <= 64 (the backward's
LDS-staged one-workgroup-per-head kernels) with 20-640 heads, so that
several workgroups share each CU.  Tolerance as everywhere: max-abs 2e-4 /
rel 1e-3; padding must stay untouched.
"""

import numpy as np
import pytest

import gpu_helpers as G
import oracle
from ember_amd import capi
from ember_amd.capi import DeviceArray

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-3, atol=2e-4)
SENTINEL = G.SENTINEL
_strided, _download = G.padded_strides, G.download_padded


def _case(seed):
    rng = np.random.default_rng(10_000 + seed)
    B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    S = int(rng.choice([1, 2, 5, 31, 32, 33, 64, 65, 100, 127, 128, 129, 200, 256, 300, 513, 700]))
    D = int(rng.choice([32, 64, 128]))
    causal = bool(rng.integers(0, 2))
    pads = [int(rng.choice([0, 4, 12, 32])) for _ in range(2)]  # row padding (floats) per triple
    hpads = [int(rng.choice([0, 1, 3])) for _ in range(2)]       # extra rows per head per triple
    return B, H, S, D, causal, pads, hpads


def _short_case(seed):
    """S <= 64 (the LDS-staged one-workgroup-per-head backward kernels) with
    enough heads that several workgroups share each CU."""
    rng = np.random.default_rng(40_000 + seed)
    B, H = int(rng.integers(1, 9)), int(rng.integers(20, 80))
    S = int(rng.choice([1, 3, 16, 17, 31, 32, 33, 40, 47, 63, 64]))
    D = int(rng.choice([32, 64, 128]))
    causal = bool(rng.integers(0, 2))
    pads = [int(rng.choice([0, 4, 12, 32])) for _ in range(2)]
    hpads = [int(rng.choice([0, 1, 3])) for _ in range(2)]
    return B, H, S, D, causal, pads, hpads


def _wide_case(seed):
    """S > 64 with more than 64 regular (128-query) workgroups."""
    rng = np.random.default_rng(30_000 + seed)
    B = int(rng.integers(1, 4))
    S = int(rng.choice([65, 100, 129, 200, 255, 300, 513, 700]))
    nqb = -(-S // 128)
    H = -(-65 // (nqb * B)) + int(rng.integers(0, 6))
    D = int(rng.choice([32, 64, 128]))
    causal = bool(rng.integers(0, 2))
    pads = [int(rng.choice([0, 4, 12, 32])) for _ in range(2)]
    hpads = [int(rng.choice([0, 1, 3])) for _ in range(2)]
    assert nqb * B * H > 64
    return B, H, S, D, causal, pads, hpads


@pytest.mark.parametrize("seed", range(64))
def test_random_shape_and_layout(seed):
    _run(seed, *_case(seed))


@pytest.mark.parametrize("seed", range(12))
def test_random_wide_launch_and_layout(seed):
    _run(100 + seed, *_wide_case(seed))


@pytest.mark.parametrize("seed", range(16))
def test_random_short_sequence_many_heads(seed):
    _run(200 + seed, *_short_case(seed))


@pytest.mark.parametrize("B,H,S,D,causal,pads,hpads", [
    (4, 250, 20, 64, True, [4, 0], [1, 2]),     # D = 64, S < 32: persistent 32-row workgroups, 1000 heads
    (2, 400, 32, 64, False, [0, 12], [0, 1]),   # non-causal S = 32: the same, 800 heads
    (1, 257, 32, 128, False, [0, 0], [0, 0]),
    (3, 171, 9, 128, True, [4, 12], [1, 0]),
    (5, 206, 32, 128, True, [0, 32], [3, 1]),
    (8, 128, 32, 128, False, [12, 4], [0, 3]),
    (16, 160, 31, 128, False, [0, 0], [0, 0]),
    (1, 257, 64, 128, True, [0, 0], [0, 0]),
    (3, 171, 48, 128, False, [4, 12], [1, 0]),
    (10, 256, 64, 128, False, [0, 4], [0, 1]),
    (1, 300, 64, 64, True, [0, 0], [0, 0]),
    (5, 206, 33, 64, False, [12, 4], [3, 0]),
    (16, 160, 64, 64, True, [4, 0], [0, 2]),
])
def test_short_backward_walks_many_heads(B, H, S, D, causal, pads, hpads):
    """S <= 64 with hundreds to thousands of heads (257 to 2560, ragged S),
    padded strides on both triples: at S <= 32 the workgroups that share a
    CU must not disturb each other's LDS tiles; at 32 < S <= 64 with D = 64
    or 128 one persistent workgroup per CU walks several heads, each
    prefetched during the previous one (a ragged last pass included), as do
    three 32-row workgroups per CU at D = 64 for S < 32 and non-causally,
    and two per CU at D = 128 for S <= 32."""
    _run(300 + B + H + S + D, B, H, S, D, causal, pads, hpads)


@pytest.mark.parametrize("B,H,S,D,causal,pads,hpads", [
    (2, 150, 128, 128, True, [0, 0], [0, 0]),
    (3, 101, 128, 128, False, [4, 12], [1, 0]),
    (1, 300, 113, 128, True, [0, 32], [3, 1]),
    (4, 64, 65, 128, True, [12, 4], [0, 3]),
    (2, 140, 96, 128, False, [0, 0], [0, 2]),
    (2, 300, 128, 64, True, [0, 0], [0, 0]),
    (5, 61, 127, 64, False, [4, 0], [1, 0]),
    (1, 513, 80, 64, True, [32, 12], [0, 1]),
    (3, 97, 65, 64, False, [0, 4], [3, 3]),
    (2, 128, 100, 64, True, [12, 12], [1, 1]),
    (2, 200, 72, 128, True, [0, 4], [1, 0]),
    (3, 120, 100, 128, False, [12, 0], [0, 3]),
    (1, 517, 80, 128, True, [4, 4], [2, 1]),
])
def test_s128_backward_many_heads(B, H, S, D, causal, pads, hpads):
    """64 < S <= 128 at D = 64 and 128 (attn_bwd_s128: 16-key chunks dealt
    out over the waves, the row statistics formed in the kernel, dQ stored
    directly) with 256 to 600 heads, ragged S (one to eight 16-row chunks,
    partial last chunks) and padded strides on both triples.  At D = 128 one
    workgroup per CU walks the heads; with more heads than CUs and an odd
    chunk count (S = 72, 80, 100: 5 or 7 chunks) a workgroup starts its
    second head on the other LDS set and dS half, with the previous head's
    dQ, dK and dV stores still deferred."""
    _run(500 + B + H + S + D, B, H, S, D, causal, pads, hpads)


@pytest.mark.parametrize("B,H,S,D,causal,pads,hpads", [
    (2, 12, 1024, 64, True, [4, 12], [1, 0]),   # 8 query blocks: pairs; backward key-block pairs too
    (1, 33, 640, 128, True, [12, 4], [0, 3]),   # 5 query blocks: the middle one alone
    (3, 10, 600, 32, True, [32, 0], [1, 1]),
])
def test_paired_query_blocks(B, H, S, D, causal, pads, hpads):
    """Causal launches of 128-query workgroups whose block pairs fit one
    round of resident workgroups (attn_fwd_kernel_pairs: query blocks
    nqb - 1 - p and p per workgroup, the second's first K tile copied during
    the first's last tile), with padded strides on both triples."""
    _run(900 + B + H + S + D, B, H, S, D, causal, pads, hpads)


@pytest.mark.parametrize("B,H,S,D,causal,pads,hpads", [
    (2, 60, 200, 64, True, [0, 0], [0, 0]),
    (1, 40, 321, 64, False, [4, 12], [1, 0]),
    (3, 30, 257, 64, True, [0, 32], [3, 1]),
    (1, 12, 700, 64, True, [12, 4], [0, 3]),
    (2, 20, 513, 64, False, [0, 0], [0, 2]),
    (1, 8, 1000, 64, True, [32, 12], [1, 1]),
    (1, 3, 1025, 64, True, [4, 4], [1, 1]),     # 17 key blocks: pairs, the middle one alone
    (4, 24, 129, 64, True, [4, 0], [0, 1]),
])
def test_w16_backward_many_heads(B, H, S, D, causal, pads, hpads):
    """S > 128 at D = 64 (attn_bwd_w16: 64 keys per workgroup in 16-key
    chunks, four workgroups per CU, one dS buffer and two barriers per step)
    with up to 480 workgroups, ragged S (partial last 16-row chunks and
    64-key blocks with keys past S), both masks and padded strides on both
    triples; causal S = 1000 and 1025 (16 and 17 key blocks) take the key
    blocks in pairs per workgroup."""
    _run(700 + B + H + S + D, B, H, S, D, causal, pads, hpads)


def _run(seed, B, H, S, D, causal, pads, hpads):
    G.say(f"sweep seed={seed} B={B} H={H} S={S} D={D} causal={causal} pads={pads} hpads={hpads}")
    rng = np.random.default_rng(seed)
    q, k, v, d_o = (rng.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(4))
    in_st, in_tot = _strided(B, H, S, D, pads[0], hpads[0])
    out_st, out_tot = _strided(B, H, S, D, pads[1], hpads[1])
    L = capi.lib()
    scale = G.scale_for(D)
    dq_, dk_, dv_ = (G.upload_padded(x, in_st, in_tot) for x in (q, k, v))
    ddo = G.upload_padded(d_o, out_st, out_tot)
    o = G.upload_padded(np.zeros_like(q), out_st, out_tot)
    lse = DeviceArray((B, H, S))
    capi.check(L.attention_fwd(dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, lse.ptr, B, H, S, D, scale, int(causal),
                               *in_st, *out_st), "attention_fwd")
    o_np, o_buf = _download(o, out_st, (B, H, S, D))
    lse_np = lse.numpy()
    o_ref, lse_ref = oracle.attention_fwd(q, k, v, causal)
    np.testing.assert_allclose(o_np, o_ref, **TOL)
    np.testing.assert_allclose(lse_np, lse_ref, **TOL)
    assert np.count_nonzero(o_buf == SENTINEL) == out_tot - B * H * S * D  # padding untouched

    grads = [G.upload_padded(np.zeros_like(q), in_st, in_tot) for _ in range(3)]
    capi.check(L.attention_bwd(dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, lse.ptr, ddo.ptr,
                               *(g.ptr for g in grads), B, H, S, D, scale, int(causal),
                               *in_st, *out_st), "attention_bwd")
    refs = oracle.attention_bwd(q, k, v, o_ref, lse_ref, d_o, causal)
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        got, buf = _download(g, in_st, (B, H, S, D))
        np.testing.assert_allclose(got, r, err_msg=name, **TOL)
        assert np.count_nonzero(buf == SENTINEL) == in_tot - B * H * S * D, name
