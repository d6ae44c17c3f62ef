"""The C-ABI library loads and exports every symbol include/ember_amd.h
declares; argument validation rejects bad calls before any device work; and,
where the reference checkout exists, the reference's own CPython bindings
link against the library with nothing left undefined.
CPU only: no call here reaches the HIP runtime."""

import ctypes as C
import os
import re
import subprocess

import pytest

from ember_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"

# The reference's backend ABI (src/core/memory.h:10-14, src/tensor/operators.h:10-27).
REFERENCE_SYMBOLS = {
    "alloc_memory", "free_memory", "copy_to_device", "copy_from_device", "sync_device",
    "matmul", "matmul_batched", "transpose", "sum", "sum_axis_product", "sum_axis", "max_axis",
    "add_tensor", "sub_tensor", "mul_tensor", "truediv_tensor", "max_tensor", "min_tensor",
    "gt_tensor", "lt_tensor", "pow_tensor",
    "add_scalar", "sub_scalar", "rsub_scalar", "mul_scalar", "truediv_scalar",
    "rtruediv_scalar", "max_scalar", "min_scalar", "gt_scalar", "lt_scalar", "pow_scalar",
    "rpow_scalar",
    "add_broadcasted", "sub_broadcasted", "mul_broadcasted", "truediv_broadcasted",
    "negate_tensor", "exponent_tensor", "log_tensor", "sqrt_tensor", "sin_tensor", "cos_tensor",
    "tan_tensor", "ctg_tensor", "sinh_tensor", "cosh_tensor", "tanh_tensor", "ctgh_tensor",
    "uniform", "constant",   # src/random/distributions.h:8-9
}


def test_library_loads():
    assert capi.lib() is not None


def test_header_declares_reference_abi_and_attention():
    names = set(capi.exported_symbols())
    assert REFERENCE_SYMBOLS <= names
    assert {"attention_fwd", "attention_bwd"} <= names


def test_every_declared_symbol_is_exported():
    L = capi.lib()
    missing = [n for n in capi.exported_symbols() if not hasattr(L, n)]
    assert missing == []


def test_error_strings():
    L = capi.lib()
    assert L.ember_error_string(0) == b"success"
    assert L.ember_error_string(2) == b"unsupported configuration"
    assert L.ember_get_last_error() == 0


def _fwd_call(D=64, B=1, H=1, S=8, ptr=16, strides=(512, 512, 64)):
    L = capi.lib()
    p = C.c_void_p(ptr)
    return L.attention_fwd(p, p, p, p, p, B, H, S, D, 0.125, 1, *strides, *strides)


@pytest.mark.parametrize("D", [0, 8, 48, 96, 256])
def test_attention_rejects_unsupported_head_dims(D):
    st = _fwd_call(D=D)
    assert st in (1, 2)
    assert capi.lib().ember_get_last_error() == st


def test_attention_rejects_bad_layouts():
    L = capi.lib()
    assert _fwd_call(ptr=0) == 1                       # null pointer
    assert _fwd_call(ptr=18) == 1                      # not 16-byte aligned
    assert _fwd_call(strides=(512, 512, 66)) == 1      # stride not a multiple of 4
    assert _fwd_call(B=-1) == 1
    # More than 2^33 elements per tensor (B*H*S*D = 2^34): rejected before any
    # device work, so that no launch's grid can pass 2^32 work-items.
    assert _fwd_call(B=1, H=1 << 10, S=1 << 17, D=128) == 1
    # Factors whose product would overflow int64 are rejected one by one.
    assert _fwd_call(B=1 << 40, H=1 << 40) == 1
    assert _fwd_call(B=1 << 62, H=4) == 1
    assert _fwd_call(B=3, H=(1 << 62) + 1) == 1
    L.ember_get_last_error()
    assert _fwd_call(S=0) == 0                         # empty: nothing to do


def test_deterministic_switch_and_noalloc_limit():
    """ember_set_deterministic is host state (no device call); with it on,
    attention_bwd_noalloc still checks its row limit (B*H*S_pad <= 2^21)
    before any device work, and still accepts the empty problem."""
    L = capi.lib()
    assert capi.is_deterministic() is False
    p = C.c_void_p(16)
    st = (128 * 64, 128 * 64, 64)
    try:
        capi.set_deterministic(True)
        assert L.ember_get_deterministic() == 1
        # 2^15 heads of S = 200 (S_pad 224): 7.3 M rows > 2^21.
        assert L.attention_bwd_noalloc(*[p] * 9, 1, 1 << 15, 200, 64, 0.125, 1, *st, *st) == 1
        assert L.ember_get_last_error() == 1
        assert L.attention_bwd_noalloc(*[p] * 9, 1, 1, 0, 64, 0.125, 1, *st, *st) == 0
    finally:
        capi.set_deterministic(False)
    assert L.ember_get_deterministic() == 0


def test_capi_raises_on_sticky_error():
    _fwd_call(D=48)
    with pytest.raises(capi.EmberError):
        capi.check()


def _nm(path, *flags):
    out = subprocess.run(["nm", *flags, path], check=True, capture_output=True, text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.strip()}


def _reference_backend_abi():
    """Function names the reference's backend headers declare
    (src/core/memory.h, src/tensor/operators.h with operators.def expanded,
    src/random/distributions.h), read through the C preprocessor."""
    src = '#include "memory.h"\n#include "operators.h"\n#include "distributions.h"\n'
    pre = subprocess.run(["gcc", "-E", "-P", "-x", "c", "-", "-I", f"{REF}/src/core", "-I", f"{REF}/src/tensor",
                          "-I", f"{REF}/src/random"], input=src, check=True, capture_output=True,
                         text=True).stdout
    return set(re.findall(r"\b(\w+)\s*\([^()]*\)\s*;", pre))


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src", "random")),
                    reason="needs the reference checkout (its bindings are compiled, never copied)")
def test_reference_bindings_link_against_the_library():
    """The drop-in claim, checked by the linker: the reference's
    src/tensor/tensor_api.c and src/random/random_api.c, compiled where they
    lie (oracle/Makefile, target link-check), link as extension modules
    against libember_amd.so with -Wl,--no-undefined and no backend source of
    the reference; every backend function they call is exported here, and so
    is every function the backend headers declare."""
    subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"), "link-check", f"REF={REF}"],
                   check=True)
    link = os.path.join(ROOT, "oracle", "_ref", "link")
    exports = _nm(capi.LIB_PATH, "-D", "--defined-only")
    abi = _reference_backend_abi()
    assert REFERENCE_SYMBOLS == abi
    assert abi <= exports, sorted(abi - exports)
    for obj, must in (("tensor_api.o", {"matmul", "matmul_batched", "sum_axis", "alloc_memory"}),
                      ("random_api.o", {"uniform", "constant", "alloc_memory"})):
        used = _nm(os.path.join(link, obj), "-u") & abi
        assert must <= used, obj
        assert used <= exports, (obj, sorted(used - exports))
    for mod in ("_tensor.so", "_em_random.so"):
        dyn = subprocess.run(["readelf", "-d", os.path.join(link, mod)], check=True, capture_output=True,
                             text=True).stdout
        assert "[libember_amd.so]" in dyn, mod


def test_mask_tests_reach_every_attention_kernel():
    """tests/test_mask_bitwise_gpu.py names a launch shape for every attention
    kernel the sources launch (the names passed to launch_ok, which the
    launch log records), so a kernel added later without a bitwise mask
    check fails here."""
    import test_mask_bitwise_gpu as M

    names = set()
    csrc = os.path.join(ROOT, "ember_amd", "csrc")
    for f in os.listdir(csrc):
        if f.startswith("attention"):
            with open(os.path.join(csrc, f)) as fh:
                for line in fh:
                    if "launch_ok(" in line:
                        names.update(re.findall(r'"(attn_\w+)"', line))
    helpers = {"attn_bwd_pre", "attn_bwd_dq_reduce"}   # row statistics and the slab sum: no mask
    assert names - helpers == ({c[0] for c in M.FWD_CASES} | {c[0] for c in M.BWD_CASES}
                                | {c[0] for c in M.BWD_ATOMIC_CASES})
    assert len(names) >= 13


def test_launch_log_starts_empty_and_resets():
    capi.launch_log_reset()
    assert capi.launch_log() == []
