"""Writes tests/golden/reference_cases.npz: the oracle's outputs on the closed-form
inputs of the reference's quantized-linear tests (src/npu.rs:1172-1188 and
src/npu/narrow_projection.rs:26-45), after the oracle has been pinned by
tests/test_oracle.py.  The GPU parity tests compare against these arrays.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402
from tests import refcases  # noqa: E402


def main():
    out = {}
    for bits in (4, 8):
        codes, scales, inp = refcases.padding_case(bits)
        q, s, acc, y = oracle.linear(inp, codes, scales)
        out[f"pad_w{bits}_q"] = q
        out[f"pad_w{bits}_s"] = s
        out[f"pad_w{bits}_acc"] = acc
        out[f"pad_w{bits}_out"] = y
        if bits == 4:
            out["pad_w4_swiglu"] = oracle.swiglu(y)
    for n in (32, 64):
        codes, scales, inp = refcases.narrow_case(n, 7)
        q, s, acc, y = oracle.linear(inp, codes, scales)
        out[f"narrow_n{n}_acc"] = acc
        out[f"narrow_n{n}_out"] = y
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_cases.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
