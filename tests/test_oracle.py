"""Pins the CPU oracle before anything is checked against it.

Each check reaches the answer by a route independent of the C code: hand-computed
known answers, exact rational arithmetic, plain integer sums in numpy int64, the
native library's digit-split identity, float64 references, and numpy's IEEE fp16
conversion.  The reference's own tests carry no numeric golden outputs (they
compare against an in-file oracle at a tolerance), so their closed-form inputs are
re-derived here and the oracle is held to their tolerances as well.
"""
from fractions import Fraction
import math

import numpy as np
import pytest

from tests import refcases

F32_MIN = np.float32(np.finfo(np.float32).tiny)


# ---------------------------------------------------------------- quantization


def quantize_independent(A, rne=False):
    """numpy route: f32 division/multiply (IEEE), rounding decided in float64 exactly."""
    A = np.asarray(A, np.float32)
    absmax = np.max(np.abs(np.nan_to_num(A, nan=0.0)), axis=1)
    s = np.where(absmax == 0, np.float32(1), np.maximum(absmax / np.float32(127), F32_MIN)).astype(np.float32)
    inv = (np.float32(1) / s).astype(np.float32)
    v = (A * inv[:, None]).astype(np.float32).astype(np.float64)
    if rne:
        r = np.round(v)  # numpy rounds half to even
    else:
        r = np.sign(v) * np.floor(np.abs(v) + 0.5)  # exact in float64
    r = np.nan_to_num(r, nan=0.0)
    return np.clip(r, -127, 127).astype(np.int8), s


def test_quantize_known_answers(oracle):
    # absmax = 127 -> s = 1 exactly, so q = round(x); ties pick the rounding mode
    row = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, 3.4999998, -0.0]], np.float32)
    q, s, bad = oracle.quantize(row, oracle.ROUND_AWAY)
    assert s[0] == 1.0 and bad == 0
    assert q[0].tolist() == [127, 3, -3, 1, -1, 2, -2, 127, 3, 0]
    q, s, _ = oracle.quantize(row, oracle.ROUND_EVEN)
    assert q[0].tolist() == [127, 2, -2, 0, 0, 2, -2, 126, 3, 0]


def test_quantize_special_rows(oracle):
    tiny = np.float32(1e-40)  # denormal: absmax/127 is below FLT_MIN -> floor
    A = np.array([[0, 0, 0, 0], [tiny, -tiny, 0, 0], [-3, 1, 0, 2]], np.float32)
    q, s, bad = oracle.quantize(A)
    assert s[0] == 1.0 and q[0].tolist() == [0, 0, 0, 0]  # src/npu.rs:1102-1103
    assert s[1] == F32_MIN
    assert s[2] == np.float32(3) / np.float32(127)
    assert q[2, 0] == -127 and bad == 0
    # the extreme element always maps to +-127
    rng = np.random.default_rng(1)
    A = rng.standard_normal((64, 333)).astype(np.float32)
    q, s, _ = oracle.quantize(A)
    idx = np.argmax(np.abs(A), axis=1)
    assert np.all(np.abs(q[np.arange(64), idx]) == 127)


def test_quantize_nonfinite_rows_flagged(oracle):
    A = np.array([[1.0, np.nan, 2.0], [np.inf, 1.0, 0.0], [1.0, 2.0, 3.0]], np.float32)
    q, s, bad = oracle.quantize(A)
    assert bad == 2
    assert q[0, 1] == 0 and q[0, 2] == 127  # NaN ignored by max, maps to 0
    assert q[1].tolist() == [0, 0, 0]     # s = inf, 1/s = 0


@pytest.mark.parametrize("rne", [False, True])
def test_quantize_matches_independent_route(oracle, rne):
    rng = np.random.default_rng(7)
    A = (rng.standard_normal((40, 1000)) * rng.choice([1e-3, 1, 50], size=(40, 1))).astype(np.float32)
    A[:, ::97] *= 20
    A[3] = 0
    # plant exact ties: x * (1/s) == k + 0.5 with s = 1
    A[5, :] = 0
    A[5, 0] = 127
    A[5, 1:20] = np.arange(19, dtype=np.float32) + np.float32(0.5)
    A = np.asarray(A.astype(np.float16), np.float32)  # activations arrive as fp16
    q, s, _ = oracle.quantize(A, oracle.ROUND_EVEN if rne else oracle.ROUND_AWAY)
    q2, s2 = quantize_independent(A, rne)
    assert np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    assert np.array_equal(q, q2)


# ---------------------------------------------------------------- integer GEMM


def test_gemm_three_routes_agree(oracle):
    rng = np.random.default_rng(3)
    for bits, (M, K, N) in [(4, (5, 96, 40)), (8, (3, 257, 17)), (8, (1, 2560, 64))]:
        lo, hi = (-8, 7) if bits == 4 else (-127, 127)
        codes = rng.integers(lo, hi + 1, size=(K, N)).astype(np.int8)
        q = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
        expect = q.astype(np.int64) @ codes.astype(np.int64)
        acc_kn = oracle.gemm_i32_kn(q, codes)
        acc_nk = oracle.gemm_i32_nk(q, np.ascontiguousarray(codes.T))
        acc_ds = oracle.gemm_i32_digit_split(q, codes)
        assert np.array_equal(acc_kn, expect)
        assert np.array_equal(acc_nk, expect)
        assert np.array_equal(acc_ds, expect)


def test_gemm_extreme_magnitude(oracle):
    # largest |acc| of the Qwen3-4B shapes: K = 9728, q = 127, codes = -127
    K = 9728
    q = np.full((1, K), 127, np.int8)
    codes = np.full((K, 2), -127, np.int8)
    acc = oracle.gemm_i32_kn(q, codes)
    assert acc[0, 0] == -127 * 127 * K


# ---------------------------------------------------------------- dequant / SwiGLU


def test_dequant_order(oracle):
    rng = np.random.default_rng(5)
    acc = rng.integers(-2 ** 27, 2 ** 27, size=(4, 33)).astype(np.int32)
    s = rng.uniform(1e-3, 1, 4).astype(np.float32)
    sc = rng.uniform(1e-3, 0.1, 33).astype(np.float32)
    out = oracle.dequant(acc, s, sc)
    # (float(acc) * s) * scale, each product rounded once (numpy f32 ops)
    expect = (acc.astype(np.float32) * s[:, None]).astype(np.float32) * sc[None, :]
    assert np.array_equal(out.view(np.uint32), expect.astype(np.float32).view(np.uint32))
    other = acc.astype(np.float32) * (s[:, None] * sc[None, :]).astype(np.float32)
    assert not np.array_equal(out, other)  # the grouping is observable, so it is pinned


def test_swiglu_against_float64(oracle):
    rng = np.random.default_rng(9)
    out = (rng.standard_normal((3, 2 * 513)) * 30).astype(np.float32)
    out[0, :4] = [-100, 100, 0, -0.0]
    mid = oracle.swiglu(out)
    g = out[:, :513].astype(np.float64)
    u = out[:, 513:].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert np.allclose(mid, ref, rtol=1e-6, atol=1e-30)
    assert mid[0, 0] == 0.0 or abs(mid[0, 0]) < 1e-30


def test_residual_add_roundings(oracle):
    """hidden + projected * m as two f32 roundings in the reference's order
    (src/model/dense.rs:486-489): known answers that a fused multiply-add, a dropped
    multiplier or a wrong rounding would each fail."""
    h = np.array([[1.0, 1.0, 3.0]], np.float32)
    p = np.array([[2.0**-24, 2.0**-24 + 2.0**-47, 1.0]], np.float32)
    out = oracle.residual_add(h, p, 1.0)
    assert out[0, 0] == 1.0  # 1 + 2^-24 is a tie: to even
    assert out[0, 1] == np.float32(1 + 2.0**-23)
    assert out[0, 2] == 4.0
    # (1 + 2^-23)^2 = 1 + 2^-22 + 2^-46 rounds to 1 + 2^-22 before the add, so the sum is
    # exactly 0; one rounding (an FMA) would leave 2^-46
    m = float(np.float32(1 + 2.0**-23))
    out = oracle.residual_add(np.array([[-(1 + 2.0**-22)]], np.float32), np.array([[m]], np.float32), m)
    assert out[0, 0] == 0.0
    rng = np.random.default_rng(11)
    hid = rng.standard_normal((4, 64)).astype(np.float32)
    pr = rng.standard_normal((4, 64)).astype(np.float32)
    assert np.array_equal(oracle.residual_add(hid, pr, 0.0), hid)  # multiplier 0: hidden unchanged
    assert np.array_equal(oracle.residual_add(np.zeros_like(pr), pr, 1.0), pr)
    # the input arrays are not modified
    h0 = hid.copy()
    oracle.residual_add(hid, pr, 0.5)
    assert np.array_equal(hid, h0)


# ---------------------------------------------------------------- RMSNorm


def f32_round(fr: Fraction) -> np.float32:
    """Correct rounding (half to even) of an exact rational to binary32."""
    if fr == 0:
        return np.float32(0.0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ue = max(e - 23, -149)
    scaled = a / Fraction(2) ** ue
    n = math.floor(scaled)
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(n * Fraction(2) ** ue))


def neon16_scale_exact(x: np.ndarray, eps: float) -> np.float32:
    """cpu.rs:11-41,47-66 with exact-rational FMAs (each vfmaq lane rounds once)."""
    K = x.size
    acc = [np.float32(0)] * 16
    i = 0
    while i + 16 <= K:
        for j in range(16):
            v = Fraction(float(x[i + j]))
            acc[j] = f32_round(v * v + Fraction(float(acc[j])))
        i += 16
    t = [np.float32(np.float32(acc[j] + acc[4 + j]) + np.float32(acc[8 + j] + acc[12 + j])) for j in range(4)]
    s = np.float32(np.float32(t[0] + t[1]) + np.float32(t[2] + t[3]))
    for v in x[i:]:
        s = np.float32(s + np.float32(v * v))
    return np.float32(np.float32(1.0) / np.sqrt(np.float32(s / np.float32(K)) + np.float32(eps)))


@pytest.mark.parametrize("K", [2560, 100, 16, 7])
def test_rmsnorm_neon16_order(oracle, K):
    rng = np.random.default_rng(K)
    x = (rng.standard_normal((2, K)) * np.array([[1.0], [300.0]])).astype(np.float32)
    w = rng.uniform(0.8, 1.2, K).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-6, "neon16")
    for r in range(2):
        sc = neon16_scale_exact(x[r], 1e-6)
        expect = (x[r] * sc).astype(np.float32) * w
        assert np.array_equal(y[r].view(np.uint32), expect.astype(np.float32).view(np.uint32))


def test_rmsnorm_formula_float64(oracle):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 2560)).astype(np.float32)
    w = rng.uniform(0.8, 1.2, 2560).astype(np.float32)
    for order in ("neon16", "seq"):
        y = oracle.rmsnorm(x, w, 1e-6, order)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-6) * w
        assert np.allclose(y, ref, rtol=3e-6, atol=0)  # src/model/cpu.rs:397-420 tolerance


def test_rmsnorm_sequential_order(oracle):
    x = np.array([[16777216.0] + [1.0] * 31], np.float32)  # 2^24 absorbs +1 sequentially
    w = np.ones(32, np.float32)
    seq = oracle.rmsnorm(x, w, 1e-6, "seq")
    s = np.float32(0)
    for v in x[0]:
        s = np.float32(s + np.float32(v * v))
    sc = np.float32(np.float32(1) / np.sqrt(np.float32(s / np.float32(32)) + np.float32(1e-6)))
    assert np.array_equal(seq[0], (x[0] * sc).astype(np.float32))


# ---------------------------------------------------------------- fp16


def test_f16_conversion_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    special = np.array([0.0, -0.0, 65504, 65519.996, 65520, -65520, 5.96e-8, 2.98e-8, 2.99e-8,
                        6.1e-5, 6.09e-5, np.inf, -np.inf, 1.0, 1.00048828125, 1.000732421875], np.float32)
    x = np.concatenate([x, special])
    ours = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7C00) == 0x7C00) and np.all(ours[nan] & 0x3FF)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = oracle.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(back[ok].view(np.uint32), ref[ok].view(np.uint32))


# ---------------------------------------------------------------- checkpoint decode


def test_compressed_unpack(oracle):
    # one word 0x76543210 holds fields 0..7 LSB-first; value = field - 8
    codes = oracle.unpack_compressed(np.array([[0x76543210]], np.uint32), 1, 8, 4)
    assert codes[:, 0].tolist() == [-8, -7, -6, -5, -4, -3, -2, -1]
    rng = np.random.default_rng(2)
    for bits, N, K in [(4, 5, 37), (8, 3, 13)]:
        lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
        c = rng.integers(lo, hi + 1, size=(N, K))
        factor = 32 // bits
        cols = -(-K // factor)
        words = np.zeros((N, cols), np.uint64)
        for k in range(K):
            words[:, k // factor] |= ((c[:, k] - lo).astype(np.uint64) << np.uint64((k % factor) * bits))
        out = oracle.unpack_compressed(words.astype(np.uint32), N, K, bits)
        assert np.array_equal(out, c.T.astype(np.int8))


# ---------------------------------------------------------------- reference test inputs


@pytest.mark.parametrize("bits", [4, 8])
def test_reference_padding_case(oracle, bits):
    codes, scales, inp = refcases.padding_case(bits)
    q, s, acc, out = oracle.linear(inp, codes, scales)
    # float64 route of the same math: the reference compares at 2e-5
    expect = (q.astype(np.float64) @ codes.astype(np.float64)) * s[:, None].astype(np.float64) * scales
    refcases.compare(out, expect.astype(np.float32), 2e-5)
    if bits == 4:
        mid = oracle.swiglu(out)
        g, u = out[:, :128].astype(np.float64), out[:, 128:].astype(np.float64)
        refcases.compare(mid, (g / (1 + np.exp(-g)) * u).astype(np.float32), 3e-5)


@pytest.mark.parametrize("n", [32, 64])
def test_reference_narrow_case(oracle, n):
    codes, scales, inp = refcases.narrow_case(n, 7)
    q, s, acc, out = oracle.linear(inp, codes, scales)
    # narrow_projection.rs:49-57 uses scale.recip() and no zero-row guard: identical here
    absmax = np.max(np.abs(inp), axis=1)
    sc = (absmax / np.float32(127)).astype(np.float32)
    assert np.array_equal(s, sc)
    expect = (acc.astype(np.float32) * sc[:, None]).astype(np.float32) * scales
    refcases.compare(out, expect, 2e-6)


def test_golden_fixtures(oracle):
    """The committed fixtures (written by tests/golden/make_golden.py) still reproduce."""
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "reference_cases.npz")
    data = np.load(path)
    for bits in (4, 8):
        codes, scales, inp = refcases.padding_case(bits)
        q, s, acc, out = oracle.linear(inp, codes, scales)
        assert np.array_equal(q, data[f"pad_w{bits}_q"])
        assert np.array_equal(s.view(np.uint32), data[f"pad_w{bits}_s"].view(np.uint32))
        assert np.array_equal(acc, data[f"pad_w{bits}_acc"])
        assert np.array_equal(out.view(np.uint32), data[f"pad_w{bits}_out"].view(np.uint32))
    for n in (32, 64):
        codes, scales, inp = refcases.narrow_case(n, 7)
        q, s, acc, out = oracle.linear(inp, codes, scales)
        assert np.array_equal(acc, data[f"narrow_n{n}_acc"])
        assert np.array_equal(out.view(np.uint32), data[f"narrow_n{n}_out"].view(np.uint32))


# ---------------------------------------------------------------- whole linear (the timed CPU baseline)


def linear_f16_independent(A_bits, w_nk, scales, gamma=None, eps=1e-6, rne=False):
    """oracle_linear_f16 by routes that share no code with it: numpy fp16 -> f32, the
    exact-rational NEON-order RMSNorm scale, numpy quantization with exact rounding,
    an int64 matmul, numpy f32 dequant; returns the f32 result before SwiGLU / fp16."""
    x = A_bits.view(np.float16).astype(np.float32)
    if gamma is not None:
        rows = []
        for r in range(x.shape[0]):
            sc = neon16_scale_exact(x[r], eps)
            rows.append((x[r] * sc).astype(np.float32) * gamma)
        x = np.stack(rows).astype(np.float32)
    q, s = quantize_independent(x, rne)
    acc = q.astype(np.int64) @ w_nk.astype(np.int64).T
    assert np.abs(acc).max() < 2 ** 31
    return (acc.astype(np.float32) * s[:, None]).astype(np.float32) * scales[None, :]


@pytest.mark.parametrize("bits,M,K,N,use_gamma,swiglu,rne,threads", [
    (4, 3, 2560, 128, False, False, False, 1),
    (8, 2, 2560, 96, True, False, False, 4),
    (4, 5, 333, 64, True, True, False, 3),
    (8, 4, 512, 200, False, True, True, 2),
    (4, 1, 16, 2, True, False, True, 1),
])
def test_linear_f16_matches_independent_route(oracle, bits, M, K, N, use_gamma, swiglu, rne, threads):
    """oracle_linear_f16 (src/npu.rs:1097-1121, 1202-1208; src/model/cpu.rs:11-66): bit-exact
    against the independent route for the plain output, and for SwiGLU bit-exact against the
    pinned oracle_swiglu of that route plus 1e-6 of float64 x*sigmoid(x)*u."""
    rng = np.random.default_rng(1000 + M * K + N)
    lo, hi = (-8, 7) if bits == 4 else (-127, 127)
    w_nk = rng.integers(lo, hi + 1, size=(N, K)).astype(np.int8)
    sc = rng.uniform(0.01, 0.1, N).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, max(1, K // 100), replace=False)] *= 20
    if K >= 8:
        x[0, :4] = [127.0, 2.5, -2.5, 0.5]  # ties when s lands on 1
    A = x.astype(np.float16).view(np.uint16)
    gamma = rng.uniform(0.8, 1.2, K).astype(np.float16).astype(np.float32) if use_gamma else None
    got = oracle.linear_f16(A, w_nk, sc, swiglu=swiglu, gamma=gamma, eps=1e-6,
                            round_mode=oracle.ROUND_EVEN if rne else oracle.ROUND_AWAY, threads=threads)
    y = linear_f16_independent(A, w_nk, sc, gamma, 1e-6, rne)
    if not swiglu:
        assert np.array_equal(got, y.astype(np.float16).view(np.uint16))
        return
    mid = oracle.swiglu(y)
    assert np.array_equal(got, mid.astype(np.float16).view(np.uint16))
    g, u = y[:, :N // 2].astype(np.float64), y[:, N // 2:].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert np.allclose(mid, ref, rtol=1e-6, atol=1e-30)


def test_linear_f16_catches_planted_mistakes(oracle):
    """The route above tells apart the mistakes a restatement could make: swapped gate and
    up halves, a dropped RMSNorm weight, and the other rounding mode on exact ties (the
    dequant grouping is pinned at f32 by test_dequant_order)."""
    rng = np.random.default_rng(77)
    M, K, N = 2, 256, 64
    w_nk = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    sc = rng.uniform(0.01, 0.1, N).astype(np.float32)
    A = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    gamma = rng.uniform(0.8, 1.2, K).astype(np.float32)
    y = linear_f16_independent(A, w_nk, sc, gamma)
    got = oracle.linear_f16(A, w_nk, sc, swiglu=True, gamma=gamma)
    swapped = oracle.swiglu(np.concatenate([y[:, N // 2:], y[:, :N // 2]], axis=1))
    assert not np.array_equal(got, swapped.astype(np.float16).view(np.uint16))
    no_gamma = oracle.swiglu(linear_f16_independent(A, w_nk, sc, None))
    assert not np.array_equal(got, no_gamma.astype(np.float16).view(np.uint16))
    # absmax 127 -> s = 1: every x = j + 0.5 is a tie that the two modes round apart
    x = np.zeros((1, K), np.float32)
    x[0, 0] = 127
    x[0, 1:] = (np.arange(K - 1) % 50) + 0.5
    At = x.astype(np.float16).view(np.uint16)
    away = oracle.linear_f16(At, w_nk, sc)
    assert np.array_equal(away, linear_f16_independent(At, w_nk, sc).astype(np.float16).view(np.uint16))
    even = linear_f16_independent(At, w_nk, sc, rne=True).astype(np.float16).view(np.uint16)
    assert not np.array_equal(away, even)
