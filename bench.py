"""Benchmark: fused causal attention forward+backward, fp32, on one MI355X.

Workload (the configuration the headline metric is quoted on):
B=4, H=32, S=4096, D=128, causal, Q/K/V/dO ~ N(0,1) seeded, scale 1/sqrt(D).
One step = attention_fwd + attention_bwd through the C ABI of
libember_amd.so on inputs already resident in HBM.

Throughput uses the FlashAttention-2 flop convention: fwd 4*B*H*S^2*D,
bwd 2.5x fwd, both halved for causal -> 7*B*H*S^2*D per step (1.924e12).
Timing: W warm-up steps, then K steps between two device synchronisations;
per-entry-point durations come from HIP events recorded on the null stream,
which is the stream every kernel of the library is launched on.  The other
configurations (`secondary`) run each measured call untimed for 150 ms first,
so that the engine clock has come back up after the host-side set-up.

The CPU baseline runs Ember's own CPU operators (the reference's
operators_cpu.c, compiled in place under oracle/_ref) composed the way Ember
expresses attention today, on a bounded sample of the timed workload itself:
heads 0..15 of batch 0 (S=4096, D=128), one per host thread, fwd+bwd.  It
falls back to this repository's C restatement (oracle/ember_oracle.c) when
_ref is absent.  The same leg times the reference on samples of configs 1, 2
and 4, and compares every CPU result with the GPU's output for the same
inputs (`parity_vs_gpu`: max error and max error / (2e-4 + 1e-3 |ref|)).
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from ember_amd import capi  # noqa: E402
from ember_amd.capi import DeviceArray  # noqa: E402

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak (AMD spec)
PEAK_HBM_GBS = 8000.0
METRIC = "attention fwd+bwd TFLOP/s at S=4096 D=128 fp32, % of MFMA fp32 peak, 1 GPU"
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "attn_bwd_c3_traffic.json")


class HipEvents:
    """hipEvent timing on the null stream via libamdhip64 (plumbing only)."""

    def __init__(self):
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        self.hip = C.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = C.c_void_p()
            assert self.hip.hipEventCreate(C.byref(e)) == 0
            evs.append(e)
        return evs

    def record(self, e):
        assert self.hip.hipEventRecord(e, None) == 0

    def elapsed_ms(self, a, b):
        assert self.hip.hipEventSynchronize(b) == 0
        t = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(t), a, b) == 0
        return float(t.value)


def attention_flops(B, H, S, D, causal=True):
    fwd = 4.0 * B * H * S * S * D * (0.5 if causal else 1.0)
    return fwd, 2.5 * fwd


def _run_threads(fn, items):
    """Wall seconds of fn(item) for every item, one host thread each (the
    C calls release the GIL)."""
    ts = [threading.Thread(target=fn, args=(it,)) for it in items]
    t0 = time.perf_counter()
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    return time.perf_counter() - t0


ATOL, RTOL = 2e-4, 1e-3  # the parity tolerance for O, dQ, dK, dV (and the GEMM)


def _parity(pairs):
    """max |gpu - ref| and max |gpu - ref| / (ATOL + RTOL |ref|) over (gpu, ref) pairs."""
    err = ratio = 0.0
    for g, r in pairs:
        d = np.abs(g.astype(np.float64) - r.astype(np.float64))
        err = max(err, float(d.max()))
        ratio = max(ratio, float((d / (ATOL + RTOL * np.abs(r.astype(np.float64)))).max()))
    return {"max_abs_err": err, "max_err_over_tol": ratio, "within_tolerance": ratio <= 1.0}


def cpu_other_configs(threads, keep):
    """The reference's CPU operators on bounded samples of configs 1, 2 and 4,
    on the very inputs the GPU ran in `secondary`, timed (reported beside the
    GPU figures, not targets) and compared with the GPU outputs: config 1 in
    full (its 4 heads, one per thread), `threads` heads of config 2 (causal
    forward, one per thread), and `threads` blocks of 8 rows of config 4's
    4096^3 product (the reference's FP64-accumulating matmul, one block per
    thread)."""
    import oracle

    if not oracle.ref_available() or keep is None:
        return None
    R = oracle.ref_lib()
    out = {}

    def attn_fwd(tag, q, k, v, o_gpu, causal, heads, sample):
        S, D = q.shape[2:]
        scale = oracle.default_scale(D)
        res = {}

        def one(bh):
            b, h = bh
            res[bh] = oracle.ref_composed_attention_head(q[b, h], k[b, h], v[b, h], None, causal, scale,
                                                         backward=False)[0]

        wall = _run_threads(one, heads)
        fwd, _ = attention_flops(1, len(heads), S, D, causal)
        out[tag] = {"value": fwd / wall / 1e12, "unit": "TFLOP/s", "cores": len(heads), "wall_s": wall,
                    "sample": sample,
                    "parity_vs_gpu": _parity([(o_gpu[b, h], res[(b, h)]) for (b, h) in heads])}

    q, k, v, o = keep["config1_fwd"]
    attn_fwd("config1_fwd", q, k, v, o, False, [(0, h) for h in range(4)],
             "config 1 in full: B1 H4 S256 D64 non-causal fwd, one head per thread")
    q, k, v, o = keep["config2_causal_fwd"]
    B, H = q.shape[:2]
    heads = [(i % B, (7 * i) % H) for i in range(threads)]
    attn_fwd("config2_causal_fwd", q, k, v, o, True, heads,
             f"{threads} of config 2's {B * H} heads (S2048 D64 causal fwd), one per thread")

    a, b, c = keep["config4_gemm_4096"]
    n, kk = a.shape
    m = b.shape[1]
    blocks = [tuple(range(i * (n // threads), i * (n // threads) + 8)) for i in range(threads)]
    res = {}

    def mm(rs):
        blk = np.ascontiguousarray(a[list(rs)])
        r = np.empty((len(rs), m), dtype=np.float32)
        R.matmul(blk, b, r, len(rs), m, kk)
        res[rs] = r

    wall = _run_threads(mm, blocks)
    out["config4_gemm_4096"] = {
        "value": 2.0 * 8 * threads * m * kk / wall / 1e12, "unit": "TFLOP/s", "cores": threads, "wall_s": wall,
        "sample": f"{threads} blocks of 8 rows of the 4096^3 product with operators_cpu.c's matmul, one per thread",
        "parity_vs_gpu": _parity([(c[list(rs)], res[rs]) for rs in blocks])}
    return out


def host_info(threads):
    """Where the CPU baseline ran: the host's CPU model and logical CPU count,
    the CPUs this process may use, and the worker threads actually used."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = None
    cores = os.cpu_count()
    if cores is not None and threads >= min(cores, allowed or cores):
        cap = (f"all {min(cores, allowed or cores)} host CPUs this process may use, one worker thread each; "
               "the reference's CPU ops are single-threaded C, one head (or row block) per thread")
    else:
        cap = (f"{threads} of {cores} host CPUs: threads = min(16, os.cpu_count()), because a GPU box allots "
               "16 host CPUs to its one GPU's jobs; the reference's CPU ops are single-threaded C, one head "
               "(or row block) per thread")
    return {"cpu_model": model, "host_cores": cores, "affinity_cores": allowed, "threads": threads,
            "thread_cap": cap}


def cpu_baseline(S, D, threads, inputs, outputs):
    """Times Ember's CPU path on `threads` heads of the timed workload (batch
    0, heads 0..threads-1, one per thread), fwd+bwd, and compares its
    O, dQ, dK, dV with the GPU's for the same heads."""
    import oracle

    q, k, v, d_o = inputs
    heads = list(range(threads))
    scale = oracle.default_scale(D)
    kind = "reference" if oracle.ref_available() else "port"
    res = {}

    def run(h):
        if kind == "reference":
            res[h] = oracle.ref_composed_attention_head(q[0, h], k[0, h], v[0, h], d_o[0, h], True, scale,
                                                        backward=True)
        else:
            sl = (slice(0, 1), slice(h, h + 1))
            o, lse = oracle.attention_fwd(q[sl], k[sl], v[sl], True, scale)
            dq, dk, dv = oracle.attention_bwd(q[sl], k[sl], v[sl], o, lse, d_o[sl], True, scale)
            res[h] = (o[0, 0], dq[0, 0], dk[0, 0], dv[0, 0])

    wall = _run_threads(run, heads)
    fwd, bwd = attention_flops(1, threads, S, D)
    what = ("the reference's operators_cpu.c ops composed as Ember would (matmul, transpose, "
            "mul_scalar, add_tensor mask, softmax via max_axis/sub/exp/sum_axis/div; "
            "backward with the same ops)") if kind == "reference" else \
        "oracle/ember_oracle.c FP64 restatement"
    return {
        "value": (fwd + bwd) / wall / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": kind,
        "sample": f"{threads} head(s) of the timed workload (batch 0, heads 0..{threads - 1}; S={S} D={D} "
                  f"causal fwd+bwd), one per thread, {wall:.1f} s wall; {what}; flops counted as on the GPU "
                  f"(causal half)",
        "wall_s": wall,
        "parity_vs_gpu": _parity([(g[0, h], r) for h in heads for g, r in zip(outputs, res[h])]),
    }


def _timed(ev, fn, reps, settle_s=0.15):
    """Average ms of fn() over reps back-to-back launches: one HIP event on
    the null stream before the first and one after the last.

    fn() first runs back to back for settle_s seconds: after the host-side
    set-up between measurements the GPU sits idle and its engine clock drops,
    and it takes some tens of milliseconds of load to come back up (one
    warm-up launch before ten 1 ms GEMMs measured 126 against 147 TFLOP/s
    after 50).  An event recorded between every two launches would add its
    own cost to each (a 64-element negate_tensor: 6.4 us per call timed that
    way, 2.6-3.0 us back to back), which matters only for microsecond
    launches such as config 1's forward."""
    L = capi.lib()
    t0 = time.perf_counter()
    fn()
    L.sync_device()
    while time.perf_counter() - t0 < settle_s:
        for _ in range(4):
            fn()
        L.sync_device()
    marks = ev.create(2)
    ev.record(marks[0])
    for _ in range(reps):
        fn()
    ev.record(marks[1])
    return ev.elapsed_ms(marks[0], marks[1]) / reps


def short_s_study(L, ev, copy_probe_mb, reps=5):
    """Attention where it is HBM-bound: the forward at S = 32, 64, 128 and
    D = 64, 128, causal, 2^20 query rows per tensor (the shapes `secondary`
    reports), achieved bandwidth over the algorithmic bytes 16*B*H*S*D +
    4*B*H*S; then the backward at the same shapes.  With copy_probe_mb, one
    negate_tensor pass over that many MiB follows (known bytes for scaling
    the traffic counters)."""
    out = {}
    rng = np.random.default_rng(7)
    for S, D in ((32, 64), (32, 128), (64, 64), (64, 128), (128, 64), (128, 128)):
        B, H = (1 << 20) // S // 64, 64
        n = B * H * S * D
        q, k, v = (DeviceArray((n,), rng.standard_normal(n, dtype=np.float32)) for _ in range(3))
        o, lse = DeviceArray((n,)), DeviceArray((B * H * S,))
        st = capi.contiguous_strides(B, H, S, D)
        sc = float(np.float32(1.0 / math.sqrt(D)))
        ms = _timed(ev, lambda: L.attention_fwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, B, H, S, D, sc, 1,
                                                *st, *st), reps)
        capi.check(what=f"short-S forward S={S}")
        byts = 16 * n + 4 * B * H * S
        out[f"short_s{S}_d{D}_fwd"] = {"shape": f"B{B} H{H} S{S} D{D} causal=True", "fwd_ms": round(ms, 4),
                                  "algorithmic_bytes": byts, "fwd_hbm_gbs": round(byts / ms / 1e6, 1),
                                  "frac_of_hbm_peak": round(byts / ms / 1e6 / PEAK_HBM_GBS, 4)}
        del q, k, v, o, lse
    # The backward in the same regime: algorithmic bytes 32*B*H*S*D + 8*B*H*S
    # (read q, k, v, o, dO, lse; write dq, dk, dv).  S <= 64: LDS-staged
    # workgroups (one per head at S <= 32, persistent with a register
    # prefetch of the next head at S = 64); S = 128: attn_bwd_s128 (one
    # workgroup per head, 16-key chunks dealt out evenly over the waves).
    for S, D in ((32, 64), (32, 128), (64, 64), (64, 128), (128, 64), (128, 128)):
        B, H = (1 << 20) // S // 64, 64
        n = B * H * S * D
        q, k, v, g = (DeviceArray((n,), rng.standard_normal(n, dtype=np.float32)) for _ in range(4))
        o, lse = DeviceArray((n,)), DeviceArray((B * H * S,))
        dq, dk, dv = DeviceArray((n,)), DeviceArray((n,)), DeviceArray((n,))
        st = capi.contiguous_strides(B, H, S, D)
        sc = float(np.float32(1.0 / math.sqrt(D)))
        capi.check(L.attention_fwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, B, H, S, D, sc, 1, *st, *st),
                   "short-S forward")
        ms = _timed(ev, lambda: L.attention_bwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, g.ptr, dq.ptr, dk.ptr,
                                                dv.ptr, B, H, S, D, sc, 1, *st, *st), reps)
        capi.check(what=f"short-S backward S={S} D={D}")
        byts = 32 * n + 8 * B * H * S
        out[f"short_s{S}_d{D}_bwd"] = {"shape": f"B{B} H{H} S{S} D{D} causal=True", "bwd_ms": round(ms, 4),
                                       "algorithmic_bytes": byts, "bwd_hbm_gbs": round(byts / ms / 1e6, 1),
                                       "frac_of_hbm_peak": round(byts / ms / 1e6 / PEAK_HBM_GBS, 4)}
        del q, k, v, g, o, lse, dq, dk, dv
    if copy_probe_mb > 0:
        n = copy_probe_mb * (1 << 20) // 4
        src, dst = DeviceArray((n,)), DeviceArray((n,))
        L.negate_tensor.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        L.negate_tensor(src.ptr, dst.ptr, n)
        L.sync_device()
        capi.check(what="copy probe")
        out["copy_probe_bytes"] = {"read": 4 * n, "write": 4 * n}
    return out


def decoder_step(B, S, d, H, steps, settle_s=0.15):
    """Times config 5's training step after one step and settle_s seconds of
    untimed ones; flops: 3 x the forward GEMMs (2*B*S*d*d*(3 + 1 + 4 + 4))
    plus causal attention fwd+bwd."""
    from ember_amd import Tensor, loss, nn, optim, random as erand

    erand.seed(0)
    block = nn.DecoderBlock(d, H, 4, True)
    opt = optim.Adam(block.parameters(), lr=1e-3)
    mse = loss.MSELoss()
    rng = np.random.default_rng(6)
    x = Tensor(rng.standard_normal((B * S, d), dtype=np.float32))
    target = Tensor(rng.standard_normal((B * S, d), dtype=np.float32))

    def step():
        y = block(x, B, S)
        value = mse(y, target)
        block.backward(mse.backward())
        opt.apply(block.gradients())
        return value

    first = step()
    L = capi.lib()
    L.sync_device()
    settle = 0  # untimed steps until the engine clock is back up (see _timed)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < settle_s:
        step()
        L.sync_device()
        settle += 1
    t0 = time.perf_counter()
    for _ in range(steps):
        last = step()
    L.sync_device()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    gemm = 3 * 2.0 * B * S * d * d * 12
    fwd, bwd = attention_flops(B, H, S, d // H, True)
    flops = gemm + fwd + bwd
    return {"shape": f"B{B} S{S} d{d} H{H} mlp4x causal", "ms_per_step": round(ms, 3),
            "tflops": round(flops / ms / 1e9, 2), "flops_per_step": flops,
            "untimed_steps": 1 + settle,
            "loss_first": round(float(first), 5), "loss_last": round(float(last), 5)}


def secondary(L, ev):
    """The other benchmark configurations, measured the same way (reported beside the
    headline, not part of `value`): attention fwd at configs 1 and 2, the
    attention part of config 5 (fwd+bwd), the config-4 GEMM shapes, and
    attention at short S where it is HBM-bound (achieved GB/s)."""
    out, keep = {}, {}
    rng = np.random.default_rng(5)

    def attn(tag, B, H, S, D, causal, bwd, reps, kept=False, det=False):
        n = B * H * S * D
        hosts = [rng.standard_normal(n, dtype=np.float32) for _ in range(3)]
        q, k, v = (DeviceArray((n,), h) for h in hosts)
        g = DeviceArray((n,), hosts[0]) if bwd else None
        o, lse = DeviceArray((n,)), DeviceArray((B * H * S,))
        dq, dk, dv = (DeviceArray((n,)) for _ in range(3)) if bwd else (None, None, None)
        st = capi.contiguous_strides(B, H, S, D)
        sc = float(np.float32(1.0 / math.sqrt(D)))
        f = lambda: L.attention_fwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, B, H, S, D, sc,
                                    int(causal), *st, *st)  # noqa: E731
        fwd_fl, bwd_fl = attention_flops(B, H, S, D, causal)
        fwd_ms = _timed(ev, f, reps)
        rec = {"shape": f"B{B} H{H} S{S} D{D} causal={causal}", "fwd_ms": round(fwd_ms, 4),
               "fwd_tflops": round(fwd_fl / fwd_ms / 1e9, 2)}
        if fwd_ms < 0.1:  # microsecond launches: four decimals of a millisecond hide them
            rec["fwd_us"] = round(fwd_ms * 1e3, 2)
        if bwd:
            b = lambda: L.attention_bwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, g.ptr, dq.ptr,  # noqa: E731
                                        dk.ptr, dv.ptr, B, H, S, D, sc, int(causal), *st, *st)
            bwd_ms = _timed(ev, b, reps)
            rec.update(bwd_ms=round(bwd_ms, 4), bwd_tflops=round(bwd_fl / bwd_ms / 1e9, 2),
                       fwd_bwd_tflops=round((fwd_fl + bwd_fl) / (fwd_ms + bwd_ms) / 1e9, 2),
                       bwd_hbm_gbs=round((32 * n + 8 * B * H * S) / bwd_ms / 1e6, 1))
            if det:  # the same backward with ember_set_deterministic(1)
                L.ember_set_deterministic(1)
                try:
                    det_ms = _timed(ev, b, reps)
                finally:
                    L.ember_set_deterministic(0)
                rec.update(bwd_deterministic_ms=round(det_ms, 4),
                           bwd_deterministic_tflops=round(bwd_fl / det_ms / 1e9, 2),
                           deterministic_time_ratio=round(det_ms / bwd_ms, 3))
        fwd_bytes = 16 * B * H * S * D + 4 * B * H * S
        rec["fwd_hbm_gbs"] = round(fwd_bytes / fwd_ms / 1e6, 1)
        capi.check(what=tag)
        out[tag] = rec
        if kept:  # inputs and output, for the CPU leg's comparison
            keep[tag] = tuple(x.reshape(B, H, S, D) for x in hosts + [o.numpy()])

    attn("config1_fwd", 1, 4, 256, 64, False, False, 50, kept=True)
    attn("config2_causal_fwd", 8, 16, 2048, 64, True, False, 20, kept=True)
    attn("config5_attention_fwd_bwd", 8, 16, 1024, 64, True, True, 20, det=True)
    # Config 3's backward once more in deterministic mode (dq added in a
    # fixed order per tile, a counter per 16 rows).
    attn("config3_deterministic_bwd", 4, 32, 4096, 128, True, True, 5, det=True)
    L.ember_empty_cache()
    for S in (32, 64, 128):  # 2^20 query rows of D=128 per tensor (512 MiB)
        attn(f"short_s{S}_fwd", (1 << 20) // S // 64, 64, S, 128, True, False, 20)
    # The backward where it is HBM-bound (AI = S/8 causal): S = 32 and 64
    # (one LDS-staged workgroup per head) and S = 128 (attn_bwd_s128, at the
    # ridge point: one workgroup per head, 16-key chunks dealt out evenly).
    for S in (32, 64, 128):
        for D in (64, 128):
            attn(f"short_s{S}_d{D}_fwd_bwd", (1 << 20) // S // 64, 64, S, D, True, True, 20)

    # Fused Adam over config 5's parameters (pre-LN decoder block, d=1024,
    # MLP 4x): LN gains/biases, QKV, out-proj, MLP weights and biases.
    d = 1024
    shapes = [d, d, 3 * d * d, 3 * d, d * d, d, d, d, 4 * d * d, 4 * d, 4 * d * d, d]
    tens = [[DeviceArray((n,), rng.standard_normal(n).astype(np.float32)) for _ in range(4)]
            for n in shapes]
    nparam = sum(shapes)
    t_box = [0]
    # Pointer tables built once, so that the host keeps ahead of the GPU and
    # the events time the kernel, not Python (building them per call takes
    # about as long as the ~60 us launch).
    nt = len(shapes)
    tables = [(C.c_void_p * nt)(*(x[j].ptr for x in tens)) for j in range(4)]
    sizes = (C.c_int64 * nt)(*shapes)

    def adam():
        t_box[0] += 1
        return L.adam_step(*tables, sizes, nt, 1e-3, 0.9, 0.999, 1e-8, t_box[0])

    ms = _timed(ev, adam, 20)
    capi.check(what="adam_step")
    out["config5_fused_adam"] = {"params": nparam, "tensors": len(shapes), "ms": round(ms, 4),
                                 "hbm_gbs": round(28.0 * nparam / ms / 1e6, 1),
                                 "frac_of_hbm_peak": round(28.0 * nparam / ms / 1e6 / PEAK_HBM_GBS, 4)}
    del tens

    # Softmax over rows (an (8192, 1024) score block) fused in one launch,
    # against Ember's five-operator composition on the same device, and the
    # row sums that keep the reference's sequential order.
    rows, cols = 8192, 1024
    x = DeviceArray((rows * cols,), rng.standard_normal(rows * cols).astype(np.float32))
    y = DeviceArray((rows * cols,))
    r = DeviceArray((rows,))
    ms = _timed(ev, lambda: L.softmax_axis(x.ptr, y.ptr, rows, 1, cols), 20)
    from ember_amd import Tensor, softmax as em_softmax, amax as em_amax, exp as em_exp, sum as em_sum
    xt = Tensor(np.random.default_rng(1).standard_normal((rows, cols), dtype=np.float32))

    def composed():
        e = em_exp(xt - em_amax(xt, axis=1, keepdims=True))
        return e / em_sum(e, axis=1, keepdims=True)

    composed()
    t0 = time.perf_counter()
    for _ in range(5):
        composed()
    L.sync_device()
    comp_ms = (time.perf_counter() - t0) * 1e3 / 5
    em_softmax(xt)
    L.sync_device()
    t0 = time.perf_counter()
    for _ in range(5):
        em_softmax(xt)
    L.sync_device()
    fused_py_ms = (time.perf_counter() - t0) * 1e3 / 5
    sum_ms = _timed(ev, lambda: L.sum_axis(x.ptr, r.ptr, rows, 1, cols), 20)
    out["softmax_rows_8192x1024"] = {
        "fused_kernel_ms": round(ms, 4), "hbm_gbs": round(8.0 * rows * cols / ms / 1e6, 1),
        "fused_python_ms": round(fused_py_ms, 4), "composed_five_ops_python_ms": round(comp_ms, 4),
        "sum_axis_ms": round(sum_ms, 4), "sum_axis_hbm_gbs": round(4.0 * rows * cols / sum_ms / 1e6, 1)}
    capi.check(what="softmax")
    del x, y, r, xt

    # Config 5: one decoder-block training step (forward, MSE loss, backward,
    # fused Adam) at d=1024, 16 heads of 64, S=1024, B=8, causal, through the
    # Python front-end.  Wall-clock per step (the loss is read back each step,
    # as Ember's MSELoss returns a float).
    out["config5_decoder_step"] = decoder_step(8, 1024, 1024, 16, steps=5)

    for tag, (n, k, m) in {"config4_gemm_4096": (4096, 4096, 4096),
                           "config4_gemm_16384x1024x3072": (16384, 1024, 3072)}.items():
        a_h = rng.uniform(-1, 1, n * k).astype(np.float32)
        b_h = rng.uniform(-1, 1, k * m).astype(np.float32)
        a, b = DeviceArray((n * k,), a_h), DeviceArray((k * m,), b_h)
        c = DeviceArray((n * m,))
        ms = _timed(ev, lambda: L.matmul(a.ptr, b.ptr, c.ptr, n, m, k), 10)
        capi.check(what=tag)
        if tag == "config4_gemm_4096":
            keep[tag] = (a_h.reshape(n, k), b_h.reshape(k, m), c.numpy().reshape(n, m))
        out[tag] = {"shape": f"n={n} k={k} m={m}", "ms": round(ms, 4),
                    "tflops": round(2.0 * n * m * k / ms / 1e9, 2),
                    "frac_of_fp32_mfma_peak": round(2.0 * n * m * k / ms / 1e9 / PEAK_FP32_MFMA_TFLOPS, 4)}
    return out, keep


def vendor_gemm_ab(reps=6):
    """This library's matmul against the vendor's fp32 GEMM (torch.matmul on
    ROCm: hipBLASLt) on the config-4 and config-5 shapes, alternating the two
    in one process with the same inputs, so both see the same clock state
    (the engine clock drops while the GPU idles between measurements and needs
    tens of milliseconds of load to come back up, so short figures taken at
    different moments are not comparable).  The vendor library is measured,
    never used by the product."""
    import torch

    L = capi.lib()
    out = {}
    for n, k, m in ((4096, 4096, 4096), (16384, 1024, 3072), (8192, 1024, 3072), (8192, 4096, 1024)):
        rng = np.random.default_rng(7)
        a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
        da, db, dc = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b), DeviceArray((n, m))
        ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        fns = {"ember_amd": lambda: L.matmul(da.ptr, db.ptr, dc.ptr, n, m, k),
               "vendor": lambda: torch.matmul(ta, tb)}
        ms = {name: [] for name in fns}
        for rep in range(reps):
            order = list(fns) if rep % 2 == 0 else list(fns)[::-1]
            for name in order:
                for _ in range(3):
                    fns[name]()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(10):
                    fns[name]()
                e1.record()
                torch.cuda.synchronize()
                ms[name].append(e0.elapsed_time(e1) / 10)
        capi.check(what="matmul")
        fl = 2.0 * n * m * k
        out[f"{n}x{k}x{m}"] = {name: {"median_tflops": round(fl / float(np.median(v)) / 1e9, 1),
                                      "min_tflops": round(fl / max(v) / 1e9, 1),
                                      "max_tflops": round(fl / min(v) / 1e9, 1)} for name, v in ms.items()}
        del da, db, dc, ta, tb
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=4)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--seq", type=int, default=4096)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--non-causal", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other configs (1, 2, 4, 5-attention, short S)")
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="host threads (= heads) for the CPU baseline; 0 skips it")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="after the timed steps, run one plain copy-like kernel "
                         "(negate_tensor: reads and writes N MiB) so rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE can be scaled against known bytes")
    ap.add_argument("--short-s-study", action="store_true",
                    help="only run the short-sequence forwards (S = 32, 64, 128; D = 128, causal; "
                         "the HBM-bound regime) and the copy probe if asked, and print their records "
                         "(for the rocprofv3 traffic counters)")
    ap.add_argument("--decoder-steps", type=int, default=0,
                    help="only run config 5's decoder-block training step this many "
                         "times and print its record (for profiling)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only compare this library's matmul with the vendor fp32 GEMM "
                         "(torch.matmul), alternating in one process, and print the record")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on exactly one GPU (no multi-GPU path); "
              "use --gpus 1", file=sys.stderr)
        return 2
    if args.vendor_gemm:
        print(json.dumps({"gemm_vs_vendor": vendor_gemm_ab()}), flush=True)
        return 0
    if args.decoder_steps > 0:
        print(json.dumps({"config5_decoder_step": decoder_step(8, 1024, 1024, 16, args.decoder_steps)}),
              flush=True)
        return 0
    if args.short_s_study:
        print(json.dumps(short_s_study(capi.lib(), HipEvents(), args.copy_probe_mb)), flush=True)
        return 0

    B, H, S, D = args.batch, args.heads, args.seq, args.head_dim
    causal = not args.non_causal
    scale = float(np.float32(1.0 / math.sqrt(D)))
    L = capi.lib()

    rng = np.random.default_rng(0)
    host = [rng.standard_normal((B, H, S, D), dtype=np.float32) for _ in range(4)]
    q, k, v, d_o = (DeviceArray.from_numpy(x) for x in host)
    o = DeviceArray((B, H, S, D))
    lse = DeviceArray((B, H, S))
    dq, dk, dv = (DeviceArray((B, H, S, D)) for _ in range(3))
    st = capi.contiguous_strides(B, H, S, D)

    def fwd():
        return L.attention_fwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, B, H, S, D, scale,
                               int(causal), *st, *st)

    def bwd():
        return L.attention_bwd(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, d_o.ptr, dq.ptr, dk.ptr,
                               dv.ptr, B, H, S, D, scale, int(causal), *st, *st)

    ev = HipEvents()
    for _ in range(args.warmup):
        capi.check(fwd(), "attention_fwd")
        capi.check(bwd(), "attention_bwd")
    L.sync_device()
    capi.check(what="warmup")

    K = args.steps
    marks = ev.create(2 * K + 1)
    L.sync_device()
    t0 = time.perf_counter()
    ev.record(marks[0])
    for i in range(K):
        fwd()
        ev.record(marks[2 * i + 1])
        bwd()
        ev.record(marks[2 * i + 2])
    L.sync_device()
    wall = time.perf_counter() - t0
    capi.check(what="timed steps")

    fwd_ms = [ev.elapsed_ms(marks[2 * i], marks[2 * i + 1]) for i in range(K)]
    bwd_ms = [ev.elapsed_ms(marks[2 * i + 1], marks[2 * i + 2]) for i in range(K)]
    total_ms = ev.elapsed_ms(marks[0], marks[2 * K])
    ms_per_step = total_ms / K

    out_ok = all(np.isfinite(x.numpy()).all() for x in (o, dq))
    fwd_fl, bwd_fl = attention_flops(B, H, S, D, causal)
    value = (fwd_fl + bwd_fl) / (ms_per_step * 1e-3) / 1e12
    bwd_avg = sum(bwd_ms) / K
    fwd_avg = sum(fwd_ms) / K
    achieved = bwd_fl / (bwd_avg * 1e-3) / 1e12

    traffic = None
    if os.path.exists(PROFILE_TRAFFIC):
        with open(PROFILE_TRAFFIC) as f:
            prof = json.load(f)
        if prof.get("workload") == f"B{B} H{H} S{S} D{D} causal={causal}":
            traffic = prof.get("hbm_bytes_per_launch")

    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"causal attention fwd+bwd B={B} H={H} S={S} D={D} fp32"
            if causal else f"attention fwd+bwd B={B} H={H} S={S} D={D} fp32",
            "batch": B, "heads": H, "seq_len": S, "head_dim": D, "causal": causal,
            "flops_per_step": fwd_fl + bwd_fl,
        },
        "frac_of_fp32_mfma_peak": round(value / PEAK_FP32_MFMA_TFLOPS, 4),
        "fwd_ms": round(fwd_avg, 4),
        "bwd_ms": round(bwd_avg, 4),
        "fwd_tflops": round(fwd_fl / (fwd_avg * 1e-3) / 1e12, 3),
        "wall_s_timed": round(wall, 4),
        "outputs_finite": bool(out_ok),
        "roofline": {
            "kernel": "attention_bwd (attn_bwd_pre + attn_bwd_kernel)",
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic,
        },
    }
    if args.copy_probe_mb > 0:
        n = args.copy_probe_mb * (1 << 20) // 4
        src, dst = DeviceArray((n,)), DeviceArray((n,))
        L.negate_tensor.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        L.negate_tensor(src.ptr, dst.ptr, n)
        L.sync_device()
        capi.check(what="copy probe")
        result["copy_probe_bytes"] = {"read": 4 * n, "write": 4 * n}

    keep = None
    if not args.no_secondary:
        result["secondary"], keep = secondary(L, ev)

    threads = args.cpu_threads
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    if threads > 0:
        cpu_heads = min(threads, H)
        gpu_out = [x.numpy()[:1, :cpu_heads] for x in (o, dq, dk, dv)]
        result["cpu_baseline"] = cpu_baseline(S, D, cpu_heads, [x[:1, :cpu_heads] for x in host], gpu_out)
        result["cpu_baseline"].update(host_info(cpu_heads))
        others = cpu_other_configs(threads, keep)
        if others is not None:
            result["cpu_baseline"]["other_configs"] = others
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
