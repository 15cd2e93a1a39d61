"""Closed-form inputs of the reference's own quantized-linear tests, regenerated bit for bit.

- quantized_linear_padding_and_swiglu, src/npu.rs:1161-1224 (inputs at 1172-1188):
  K = N = 256, bits 4 and 8, rows {1,2,3,5,9,17,32,33,65,127,128,129,191,192,193,255,256},
  compared at rel tol 2e-5 (plain) and 3e-5 (SwiGLU, rows >= 32 on W4).
- narrow_w8_gdn_gates_match_integer_oracle, src/npu/narrow_projection.rs:3-68 (inputs at 26-45):
  W8, K = 2560, N in {32, 64}, rows {1,2,3,5,7}, rel tol 2e-6.
The Rust expressions are evaluated with the same integer and f32 operations.
"""
import numpy as np

PADDING_ROWS = [1, 2, 3, 5, 9, 17, 32, 33, 65, 127, 128, 129, 191, 192, 193, 255, 256]
NARROW_ROWS = [1, 2, 3, 5, 7]


def padding_case(bits: int):
    """(codes [K,N] int8, scales f32 [N], input f32 [256, 256]) of src/npu.rs:1172-1188."""
    i = np.arange(256 * 256, dtype=np.int64)
    mod, off = (16, 8) if bits == 4 else (255, 127)
    codes = (((i * 13 + i // 256 * 7) % mod) - off).astype(np.int8).reshape(256, 256)
    n = np.arange(256, dtype=np.int64)
    scales = np.float32(0.002) + (n % 11).astype(np.float32) * np.float32(0.0001)
    inp = ((i * 17 + i // 256 * 3) % 127).astype(np.float32) / np.float32(63.0) - np.float32(1.0)
    return codes, scales.astype(np.float32), inp.astype(np.float32).reshape(256, 256)


def narrow_case(n: int, rows: int, k: int = 2560):
    """(codes [K,N] int8, scales f32 [N], input f32 [rows, K]) of narrow_projection.rs:26-45."""
    i = np.arange(k * n, dtype=np.int64)
    codes = (((i * 13 + i // n * 7) % 255) - 127).astype(np.int8).reshape(k, n)
    j = np.arange(n, dtype=np.int64)
    scales = np.float32(0.001) + (j % 11).astype(np.float32) * np.float32(0.0001)
    r = np.arange(rows * k, dtype=np.int64)
    inp = ((r * 17 + r // k * 3) % 127).astype(np.float32) / np.float32(63.0) - np.float32(1.0)
    return codes, scales.astype(np.float32), inp.astype(np.float32).reshape(rows, k)


def compare(actual, expected, tol):
    """src/npu.rs:1125-1130: |a - e| <= tol * max(|e|, 1), and a finite."""
    a = np.asarray(actual, dtype=np.float32)
    e = np.asarray(expected, dtype=np.float32)
    assert np.all(np.isfinite(a))
    bad = np.abs(a - e) > tol * np.maximum(np.abs(e), 1.0)
    assert not bad.any(), f"{bad.sum()} elements off, first at {np.argwhere(bad)[0]}: " \
                          f"{a[tuple(np.argwhere(bad)[0])]} vs {e[tuple(np.argwhere(bad)[0])]}"
