"""The device code's short rounding sequence for finite rows (quant_finite in
csrc/qlin_internal.hpp): round half away from zero, as Rust's f32::round used by the
reference quantizer (src/npu.rs:1109), is computed as (x + copysign(0.5 - 2^-25, x))
truncated toward zero.  Checked here in IEEE single precision (numpy float32) against
floor(|x| + 0.5) in double precision: exhaustively over every float in [2^-2, 2^3) and
both signs, and on random floats over the whole range |x| < 256 that quantization
produces (|x * (1/s)| <= 127 plus a few ulp)."""
import numpy as np


def fast_round(x: np.ndarray) -> np.ndarray:
    half = np.float32(0.49999997)
    assert half == np.nextafter(np.float32(0.5), np.float32(0))
    return np.trunc((x + np.copysign(half, x)).astype(np.float32))


def ref_round(x: np.ndarray) -> np.ndarray:
    a = np.abs(x.astype(np.float64))
    return (np.floor(a + 0.5) * np.sign(x)).astype(np.float32)


def test_exhaustive_ties_region():
    m = np.arange(1 << 23, dtype=np.uint32)
    for e in range(125, 130):  # biased exponents: [0.25, 8)
        x = ((np.uint32(e) << np.uint32(23)) | m).view(np.float32)
        for sgn in (1.0, -1.0):
            v = (x * np.float32(sgn)).astype(np.float32)
            assert np.array_equal(fast_round(v), ref_round(v)), e


def test_random_full_range():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 0x43800000, size=4_000_000, dtype=np.uint32)  # |x| < 256, subnormals included
    x = bits.view(np.float32)
    x = np.concatenate([x, -x, np.float32([0.5, 1.5, 2.5, 126.5, 127.5, 0.49999997, 1.4999999])])
    assert np.array_equal(fast_round(x), ref_round(x))
