"""Writes tests/golden/attention_golden.npz: seeded inputs and float64
closed-form outputs for attention forward/backward on small shapes.

The reference (pawel002/ember) has no attention and commits no golden
vectors for this path, so these fixtures are generated here from NumPy
float64 closed forms (tests/closed_forms.py), themselves checked against
central finite differences in tests/test_oracle.py.  Shapes cover S in
{1, 2, 17, 33, 64, 65, 130} (tile edges +-1 for the 32/64/128 tilings),
D in {8, 32, 64, 128}, causal and not.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import closed_forms  # noqa: E402

# name: (B, H, S, D, causal, seed)
CASES = {
    "s1_d8_nc": (1, 1, 1, 8, False, 11),
    "s2_d8_c": (1, 1, 2, 8, True, 12),
    "s17_d8_c": (1, 2, 17, 8, True, 13),
    "s17_d32_nc": (1, 1, 17, 32, False, 14),
    "s33_d128_c": (1, 1, 33, 128, True, 15),
    "s64_d64_c": (1, 1, 64, 64, True, 16),
    "s65_d64_c": (1, 1, 65, 64, True, 17),
    "s65_d64_nc": (1, 1, 65, 64, False, 18),
    "s130_d32_c": (1, 1, 130, 32, True, 19),
}


def make_case(B, H, S, D, causal, seed):
    rng = np.random.default_rng(seed)
    q, k, v, d_o = (rng.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(4))
    scale = float(np.float32(1.0 / math.sqrt(D)))
    o, lse = closed_forms.fwd(q, k, v, causal, scale)
    dq, dk, dv = closed_forms.bwd(q, k, v, d_o, causal, scale)
    f32 = np.float32
    # Expected values are the float64 results rounded once to float32.
    return dict(q=q, k=k, v=v, do=d_o, o=o.astype(f32), lse=lse.astype(f32), dq=dq.astype(f32),
                dk=dk.astype(f32), dv=dv.astype(f32), causal=np.array(causal),
                scale=np.array(scale, dtype=f32))


def main() -> None:
    out = {}
    for name, args in CASES.items():
        for key, val in make_case(*args).items():
            out[f"{name}/{key}"] = val
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
