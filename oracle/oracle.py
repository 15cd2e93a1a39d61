"""ctypes wrapper over oracle/liboracle.so, the CPU oracle of the quantized linear path.

TEST INFRASTRUCTURE ONLY.  Imported by the test suite, the smoke check and the CPU
baseline leg of bench.py, always as the checker.  The product path never imports it.

Each function mirrors one C entry point of qlin_oracle.h; see that header for the
reference file:line each one restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

ROUND_AWAY = 0
ROUND_EVEN = 1


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        C = ctypes.c_int
        F = ctypes.c_float
        sig = {
            "oracle_row_scale": (F, [P, I]),
            "oracle_quantize": (I, [P, I, I, I, C, P, I, P]),
            "oracle_gemm_i32_kn": (None, [P, I, I, I, P, I, P]),
            "oracle_gemm_i32_nk": (None, [P, I, I, I, P, I, P, C]),
            "oracle_gemm_i32_digit_split": (None, [P, I, I, I, P, I, P]),
            "oracle_dequant": (None, [P, I, I, P, P, P]),
            "oracle_swiglu": (None, [P, I, I, P]),
            "oracle_residual_add": (None, [P, P, I, I, F]),
            "oracle_rmsnorm_neon16": (None, [P, I, I, I, P, F, P]),
            "oracle_rmsnorm_seq": (None, [P, I, I, I, P, F, P]),
            "oracle_f32_to_f16_array": (None, [P, I, P]),
            "oracle_f16_to_f32_array": (None, [P, I, P]),
            "oracle_linear_f16": (None, [P, I, I, P, F, P, P, I, C, C, P, C]),
            "oracle_unpack_compressed": (None, [P, I, I, C, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def row_scale(a) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return float(lib().oracle_row_scale(_p(a), a.size))


def quantize(A, round_mode=ROUND_AWAY):
    """A f32 [M,K] -> (q i8 [M,K], s f32 [M], rows_with_nonfinite)."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    M, K = A.shape
    q = np.zeros((M, K), np.int8)
    s = np.zeros(M, np.float32)
    bad = lib().oracle_quantize(_p(A), M, K, K, round_mode, _p(q), K, _p(s))
    return q, s, int(bad)


def gemm_i32_kn(q, codes_kn):
    q = np.ascontiguousarray(q, dtype=np.int8)
    codes_kn = np.ascontiguousarray(codes_kn, dtype=np.int8)
    M, K = q.shape
    K2, N = codes_kn.shape
    assert K == K2
    acc = np.zeros((M, N), np.int32)
    lib().oracle_gemm_i32_kn(_p(q), K, M, K, _p(codes_kn), N, _p(acc))
    return acc


def gemm_i32_nk(q, w_nk, threads=0):
    q = np.ascontiguousarray(q, dtype=np.int8)
    w_nk = np.ascontiguousarray(w_nk, dtype=np.int8)
    M, K = q.shape
    N, K2 = w_nk.shape
    assert K == K2
    acc = np.zeros((M, N), np.int32)
    lib().oracle_gemm_i32_nk(_p(q), K, M, K, _p(w_nk), N, _p(acc), threads)
    return acc


def gemm_i32_digit_split(q, codes_kn):
    q = np.ascontiguousarray(q, dtype=np.int8)
    codes_kn = np.ascontiguousarray(codes_kn, dtype=np.int8)
    M, K = q.shape
    N = codes_kn.shape[1]
    acc = np.zeros((M, N), np.int32)
    lib().oracle_gemm_i32_digit_split(_p(q), K, M, K, _p(codes_kn), N, _p(acc))
    return acc


def dequant(acc, s, scales):
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    s = np.ascontiguousarray(s, dtype=np.float32)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    M, N = acc.shape
    out = np.zeros((M, N), np.float32)
    lib().oracle_dequant(_p(acc), M, N, _p(s), _p(scales), _p(out))
    return out


def residual_add(hidden, projected, multiplier=1.0):
    """hidden + projected * multiplier (f32, the decoder's residual update); returns a new array."""
    h = np.array(hidden, dtype=np.float32, copy=True, order="C")
    pr = np.ascontiguousarray(projected, dtype=np.float32)
    M, N = h.shape
    lib().oracle_residual_add(_p(h), _p(pr), M, N, multiplier)
    return h


def swiglu(out):
    out = np.ascontiguousarray(out, dtype=np.float32)
    M, N = out.shape
    mid = np.zeros((M, N // 2), np.float32)
    lib().oracle_swiglu(_p(out), M, N, _p(mid))
    return mid


def rmsnorm(x, w, eps, order="neon16"):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = x.shape
    y = np.zeros((M, K), np.float32)
    fn = lib().oracle_rmsnorm_neon16 if order == "neon16" else lib().oracle_rmsnorm_seq
    fn(_p(x), M, K, K, _p(w), eps, _p(y))
    return y


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), x.size, _p(out))
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.zeros(h.shape, np.float32)
    lib().oracle_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


def linear(A_f32, codes_kn, scales, round_mode=ROUND_AWAY):
    """Reference linear (src/npu.rs:1097-1121): returns (q, s, acc, out_f32)."""
    q, s, _ = quantize(A_f32, round_mode)
    acc = gemm_i32_kn(q, codes_kn)
    return q, s, acc, dequant(acc, s, scales)


def linear_f16(A_f16, w_nk, scales, swiglu=False, gamma=None, eps=1e-6,
               round_mode=ROUND_AWAY, threads=0):
    """Threaded whole-linear over fp16 bits in / fp16 bits out (the timed CPU baseline)."""
    A = np.ascontiguousarray(A_f16).view(np.uint16)
    w_nk = np.ascontiguousarray(w_nk, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    M, K = A.shape
    N = w_nk.shape[0]
    out = np.zeros((M, N // 2 if swiglu else N), np.uint16)
    g = None
    if gamma is not None:
        g = np.ascontiguousarray(gamma, dtype=np.float32)
    lib().oracle_linear_f16(_p(A), M, K, _p(g) if g is not None else None, eps, _p(w_nk),
                            _p(scales), N, int(bool(swiglu)), round_mode, _p(out), threads)
    return out


def unpack_compressed(packed_u32, N, K, bits):
    packed_u32 = np.ascontiguousarray(packed_u32, dtype=np.uint32)
    codes = np.zeros((K, N), np.int8)
    lib().oracle_unpack_compressed(_p(packed_u32), N, K, bits, _p(codes))
    return codes
