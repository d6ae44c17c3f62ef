"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message before any device work, and the help text names the flags
the driver and the profiles use."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode != 0
    assert "exactly one GPU" in (r.stdout + r.stderr)


def test_help_lists_the_driver_and_profile_flags():
    r = _bench("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--short-s-study", "--copy-probe-mb", "--decoder-steps",
                 "--vendor-gemm", "--no-secondary", "--cpu-threads"):
        assert flag in r.stdout, flag
