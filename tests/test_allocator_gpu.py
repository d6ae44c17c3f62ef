"""The device allocator behind alloc_memory / free_memory: freed blocks are
cached and reused without a device synchronisation, and reuse is ordered by
the null stream.  The ordering test frees a tensor while a GEMM that reads it
is still queued, refills the reused block from the host, and checks that the
GEMM saw the old contents."""

import os
import subprocess
import sys

import numpy as np
import pytest

import ember_amd as em
import gpu_helpers as G
from ember_amd import Tensor

pytestmark = pytest.mark.gpu


def test_freed_block_is_reused_and_counted():
    G.say("allocator reuse")
    em.synchronize()
    em.empty_cache()
    base = em.memory_stats()
    assert base["cached"] == 0
    t = Tensor(np.ones(3 << 20, np.float32))           # 12 MiB -> 12 MiB block
    ptr = t._core.data_ptr
    s = em.memory_stats()
    assert s["in_use"] - base["in_use"] == 12 << 20
    del t
    s = em.memory_stats()
    assert s["in_use"] == base["in_use"] and s["cached"] == 12 << 20
    u = Tensor(np.full(3 << 20, 2.0, np.float32))       # same size class: same block
    assert u._core.data_ptr == ptr
    assert em.memory_stats()["cached"] == 0
    np.testing.assert_array_equal(u.to_np()[:5], 2.0)
    del u
    em.empty_cache()
    assert em.memory_stats()["cached"] == 0


def test_reuse_is_ordered_after_queued_readers():
    G.say("allocator ordering")
    n = 4096
    rng = np.random.default_rng(0)
    a_host = rng.standard_normal((n, n), dtype=np.float32)
    b_host = np.eye(n, dtype=np.float32)
    b = Tensor(b_host)
    outs = []
    for rep in range(3):
        a = Tensor(a_host + rep)
        ptr = a._core.data_ptr
        outs.append(a @ b)          # queued; reads a for ~1 ms
        del a                        # back to the cache while the GEMM may still run
        c = Tensor(np.full((n, n), -7.0, np.float32))   # reuses a's block, overwritten
        assert c._core.data_ptr == ptr
        del c
    for rep, out in enumerate(outs):
        np.testing.assert_array_equal(out.to_np(), a_host + rep)


def test_cache_can_be_turned_off():
    G.say("allocator EMBER_AMD_NO_CACHE=1 (child process)")
    code = (
        "import numpy as np, ember_amd as em\n"
        "t = em.Tensor(np.ones(1000, np.float32)); del t\n"
        "s = em.memory_stats(); assert s['cached'] == 0 and s['in_use'] == 0, s\n"
        "print('ok')\n"
    )
    env = dict(os.environ, EMBER_AMD_NO_CACHE="1")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env["PYTHONPATH"] = root + os.pathsep + env.get("PYTHONPATH", "")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr
