"""Builds libember_amd.so (HIP, gfx950) and the CPython binding modules in-tree.

Usage: ``python -m ember_amd.build`` (or ``__graft_entry__.build()``).
Every call recompiles everything; objects go to ``ember_amd/_build/``.

HIP flags:
* ``--offload-arch=gfx950`` only: the kernels are written for CDNA4.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: keep the compiler
  from forming packed fp32 VALU ops (results from some of their forms have
  been unreliable on these machines); the host pass warns that it does not
  know the feature, which is harmless.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libember_amd.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# (source, extra hipcc flags).  -amdgpu-mfma-vgpr-form=1 keeps MFMA
# accumulators in VGPRs; attention_bwd.hip explains which instantiations use
# which form and why.
HIP_SOURCES = [
    ("runtime.hip", []),
    ("elementwise.hip", []),
    ("gemm.hip", []),
    ("attention_fwd.hip", []),
    ("attention_bwd.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]),
    ("attention_bwd_c128.hip", []),
    ("attention_bwd_s128.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]),
    ("attention_bwd_w16.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]),
    ("optim.hip", []),
    ("layernorm.hip", []),
    ("block_ops.hip", []),
    ("softmax.hip", []),
    ("distributions.hip", []),
]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]

# CPython extension modules: (module path relative to the package, sources).
EXTENSIONS = [
    ("_core/_tensor", ["tensor_api.c"]),
    ("_core/_em_random", ["random_api.c"]),
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in r.stdout.splitlines()
        if "packed-fp32-ops" not in ln and "is not a recognized feature" not in ln
    )
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")
    if out.strip() and os.environ.get("EMBER_BUILD_VERBOSE"):
        sys.stderr.write(out + "\n")


def _compile_hip(src: str, flags: list[str], extra: list[str]) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    _run([HIPCC, *HIP_FLAGS, *flags, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_library(extra_flags: list[str] | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    extra = list(extra_flags or [])
    sources = [(s, f) for s, f in HIP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda sf: _compile_hip(sf[0], sf[1], extra), sources))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_extensions() -> list[str]:
    inc_py = sysconfig.get_paths()["include"]
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    built = []
    for mod, srcs in EXTENSIONS:
        srcs = [os.path.join(CSRC, s) for s in srcs]
        if not all(os.path.exists(s) for s in srcs):
            continue
        out = os.path.join(PKG, mod + suffix)
        os.makedirs(os.path.dirname(out), exist_ok=True)
        rel = os.path.relpath(PKG, os.path.dirname(out))
        _run([
            "gcc", "-O2", "-std=gnu11", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
            "-Wno-missing-field-initializers",
            "-I", inc_py, "-I", os.path.join(ROOT, "include"), "-I", CSRC,
            *srcs, "-o", out + ".tmp",
            "-L", PKG, "-lember_amd", f"-Wl,-rpath,$ORIGIN/{rel}",
        ])
        os.replace(out + ".tmp", out)
        built.append(out)
    return built


def build_all() -> None:
    build_library()
    build_extensions()


if __name__ == "__main__":
    build_all()
    print(LIB)
