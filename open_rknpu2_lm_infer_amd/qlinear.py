"""Device-tensor front end of the C ABI (include/qlinear.h) for torch callers.

torch supplies device memory and streams; every computation is a libqlinear.so
kernel launched on torch's current stream.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import (QLIN_F16, QLIN_F32, QLIN_NO_FUSED_QUANT, QLIN_NORM_SEQUENTIAL,  # noqa: F401
                   QLIN_PATH_GEMM, QLIN_PATH_GEMV, QLIN_PATH_GEMV_FUSED, QLIN_RESIDUAL, QLIN_ROUND_HALF_EVEN,
                   QLIN_SWIGLU, check)

_DT = {torch.float32: QLIN_F32, torch.float16: QLIN_F16}


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


class Weights:
    """Device-resident W4/W8 codes + per-channel scales (qlin_weights)."""

    def __init__(self, handle: ctypes.c_void_p):
        self.handle = handle
        info = _lib.WeightInfo()
        check(_lib.load().qlin_weights_query(handle, ctypes.byref(info)), "qlin_weights_query")
        self.bits, self.K, self.N = info.bits, info.K, info.N
        self.K_padded, self.N_padded = info.K_padded, info.N_padded
        self.device_bytes = info.device_bytes

    @classmethod
    def from_codes_kn(cls, bits: int, codes_kn: np.ndarray, scales: np.ndarray) -> "Weights":
        """Reference QuantMatrix layout: int8 [K, N] K-major + f32 [N]."""
        codes_kn = np.ascontiguousarray(codes_kn, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        K, N = codes_kn.shape
        cfg = _lib.WeightConfig(bits, K, N)
        h = ctypes.c_void_p()
        check(_lib.load().qlin_weights_create(ctypes.byref(cfg), codes_kn.ctypes.data_as(ctypes.c_void_p),
                                              scales.ctypes.data_as(ctypes.c_void_p), ctypes.byref(h)),
              "qlin_weights_create")
        return cls(h)

    @classmethod
    def from_packed_device(cls, bits: int, K: int, N: int, packed: torch.Tensor,
                           scales: torch.Tensor) -> "Weights":
        """Packed codes on the GPU: uint8 [N, K/2] (W4, low nibble = even k) or int8 [N, K] (W8) + f32 [N]."""
        assert packed.is_cuda and scales.is_cuda and packed.is_contiguous() and scales.is_contiguous()
        cfg = _lib.WeightConfig(bits, K, N)
        h = ctypes.c_void_p()
        check(_lib.load().qlin_weights_create_packed_device(ctypes.byref(cfg), _ptr(packed), _ptr(scales),
                                                            _stream(), ctypes.byref(h)),
              "qlin_weights_create_packed_device")
        return cls(h)

    def close(self):
        if self.handle:
            _lib.load().qlin_weights_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Workspace:
    """Scratch for runs of up to max_rows rows over weights up to max_k x max_n."""

    def __init__(self, max_rows: int, max_k: int, max_n: int):
        self.handle = ctypes.c_void_p()
        check(_lib.load().qlin_workspace_create(max_rows, max_k, max_n, ctypes.byref(self.handle)),
              "qlin_workspace_create")
        self.max_rows, self.max_k, self.max_n = max_rows, max_k, max_n

    def status(self, clear: bool = True) -> int:
        return _lib.load().qlin_workspace_status(self.handle, int(clear))

    def close(self):
        if self.handle:
            _lib.load().qlin_workspace_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _DeviceArray:
    """__cuda_array_interface__ view of library-owned device memory."""

    def __init__(self, ptr: int, shape, strides, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "strides": tuple(strides), "typestr": typestr,
                                         "data": (ptr, False), "version": 2}


class Chain:
    """Decode chain (qlin_chain): several linears in one persistent launch, 1..4 rows of
    fp16 activations.  stages: dicts with weights (Weights), flags, gamma (device f32
    [K] or None), eps, input (-1 = chain input, j = output of stage j; default: the
    previous stage), offset (first column read) and, for a residual stage, residual
    (-1 = chain input, j = output of stage j), residual_offset and residual_scale
    (QLIN_RESIDUAL is added to the flags when residual is given)."""

    def __init__(self, stages: list, max_rows: int = 1):
        arr = (_lib.ChainStage * len(stages))()
        self._keep = []
        for i, st in enumerate(stages):
            g = st.get("gamma")
            res = st.get("residual")
            flags = st.get("flags", 0) | (QLIN_RESIDUAL if res is not None else 0)
            arr[i] = _lib.ChainStage(st["weights"].handle, flags, g.data_ptr() if g is not None else None,
                                     st.get("eps", 1e-6), st.get("input", -1 if i == 0 else i - 1), st.get("offset", 0),
                                     res if res is not None else 0, st.get("residual_offset", 0),
                                     st.get("residual_scale", 1.0))
            self._keep.append(st["weights"])
            if g is not None:
                self._keep.append(g)
        self.handle = ctypes.c_void_p()
        check(_lib.load().qlin_chain_create(arr, len(stages), max_rows, ctypes.byref(self.handle)),
              "qlin_chain_create")
        self.cols = [st["weights"].N // 2 if st.get("flags", 0) & QLIN_SWIGLU else st["weights"].N for st in stages]
        self.max_rows = max_rows

    def run(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        M = x.shape[0]
        if out is None:
            out = torch.empty((M, self.cols[-1]), dtype=torch.float16, device=x.device)
        assert x.dtype == torch.float16 and out.dtype == torch.float16 and x.stride(1) == 1 and out.stride(1) == 1
        check(_lib.load().qlin_chain_run(self.handle, M, _ptr(x), x.stride(0), _ptr(out), out.stride(0), _stream()),
              "qlin_chain_run")
        return out

    def stage_output(self, stage: int, rows: int) -> torch.Tensor:
        """Copy of stage `stage`'s output from the last run (not the last stage)."""
        ptr, ld = ctypes.c_void_p(), ctypes.c_int64()
        check(_lib.load().qlin_chain_stage_output(self.handle, stage, ctypes.byref(ptr), ctypes.byref(ld)),
              "qlin_chain_stage_output")
        view = torch.as_tensor(_DeviceArray(ptr.value, (rows, self.cols[stage]), (2 * ld.value, 2), "<f2"),
                               device=torch.device("cuda", torch.cuda.current_device()))
        return view.clone()

    def status(self, clear: bool = True) -> int:
        return _lib.load().qlin_chain_status(self.handle, int(clear))

    def set_wait_limit(self, polls: int) -> None:
        check(_lib.load().qlin_chain_set_wait_limit(self.handle, polls), "qlin_chain_set_wait_limit")

    def close(self):
        if self.handle:
            _lib.load().qlin_chain_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BoundRun:
    """One qlin_run call with every argument bound once (handles, device pointers, strides,
    stream): calling it makes a single C-ABI call, the way a native engine's decode loop calls
    the library, so eager launch timings measure the library rather than Python."""

    def __init__(self, ws: Workspace, w: Weights, A: torch.Tensor, out: torch.Tensor, flags: int = 0,
                 stream: torch.cuda.Stream | None = None):
        assert A.stride(1) == 1 and out.stride(1) == 1
        self._fn = _lib.load().qlin_run
        st = (stream or torch.cuda.current_stream()).cuda_stream
        self._args = (ws.handle, w.handle, A.shape[0], A.data_ptr(), _DT[A.dtype], A.stride(0), out.data_ptr(),
                      _DT[out.dtype], out.stride(0), flags, st)

    def __call__(self) -> None:
        rc = self._fn(*self._args)
        if rc:
            check(rc, "qlin_run")


def tune(ws: Workspace, w: Weights, rows: int, flags: int = 0, reps: int = 20) -> None:
    """Time the kernel variants of (w, rows, flags) and record the fastest (qlin_tune)."""
    check(_lib.load().qlin_tune(ws.handle, w.handle, rows, flags, reps, _stream()), "qlin_tune")


def tune_count() -> int:
    return _lib.load().qlin_tune_count()


def tune_clear() -> None:
    _lib.load().qlin_tune_clear()


def tune_save(path: str) -> None:
    check(_lib.load().qlin_tune_save(path.encode()), "qlin_tune_save")


def tune_load(path: str) -> int:
    n = _lib.load().qlin_tune_load(path.encode())
    check(min(n, 0), "qlin_tune_load")
    return n


def run(ws: Workspace, w: Weights, A: torch.Tensor, out: torch.Tensor | None = None,
        out_dtype=torch.float16, flags: int = 0, gamma: torch.Tensor | None = None,
        eps: float = 1e-6, residual: torch.Tensor | None = None, residual_scale: float = 1.0) -> torch.Tensor:
    """out[M, N] (or [M, N/2] with QLIN_SWIGLU) = quantized linear of A[M, K] (device).
    With residual R [M, N]: out = R + linear * residual_scale (qlin_run_residual; out may be R)."""
    M = A.shape[0]
    ncols = w.N // 2 if flags & QLIN_SWIGLU else w.N
    if out is None:
        out = torch.empty((M, ncols), dtype=out_dtype, device=A.device)
    assert A.stride(1) == 1 and out.stride(1) == 1
    L = _lib.load()
    if residual is not None:
        assert gamma is None and residual.stride(1) == 1
        rc = L.qlin_run_residual(ws.handle, w.handle, M, _ptr(A), _DT[A.dtype], A.stride(0), _ptr(residual),
                                 _DT[residual.dtype], residual.stride(0), residual_scale, _ptr(out), _DT[out.dtype],
                                 out.stride(0), flags, _stream())
        check(rc, "qlin_run_residual")
        return out
    if gamma is None:
        rc = L.qlin_run(ws.handle, w.handle, M, _ptr(A), _DT[A.dtype], A.stride(0), _ptr(out), _DT[out.dtype],
                        out.stride(0), flags, _stream())
    else:
        rc = L.qlin_run_rmsnorm(ws.handle, w.handle, M, _ptr(A), _DT[A.dtype], A.stride(0), _ptr(gamma), eps,
                                _ptr(out), _DT[out.dtype], out.stride(0), flags, _stream())
    check(rc, "qlin_run")
    return out


def swiglu(X: torch.Tensor, out: torch.Tensor | None = None, out_dtype=torch.float16) -> torch.Tensor:
    """Y[m, j] = SiLU(X[m, j]) * X[m, F + j] on the unfused [M, 2F] layout (qlin_swiglu)."""
    M, F2 = X.shape
    F = F2 // 2
    if out is None:
        out = torch.empty((M, F), dtype=out_dtype, device=X.device)
    assert X.stride(1) == 1 and out.stride(1) == 1
    check(_lib.load().qlin_swiglu(M, F, _ptr(X), _DT[X.dtype], X.stride(0), _ptr(out), _DT[out.dtype],
                                  out.stride(0), _stream()), "qlin_swiglu")
    return out


def plan(ws: Workspace, w: Weights, A: torch.Tensor, flags: int = 0, gamma: torch.Tensor | None = None) -> dict:
    """The launches qlin_run / qlin_run_rmsnorm would make for these arguments (qlin_run_plan)."""
    out = _lib.Plan()
    check(_lib.load().qlin_run_plan(ws.handle, w.handle, A.shape[0], _ptr(A), A.stride(0),
                                    _ptr(gamma) if gamma is not None else None, flags, ctypes.byref(out)),
          "qlin_run_plan")
    return {f: getattr(out, f) for f, _ in _lib.Plan._fields_ if f != "reserved"}


def quantize(A: torch.Tensor, ldq: int | None = None, gamma: torch.Tensor | None = None, eps: float = 1e-6,
             flags: int = 0, err: torch.Tensor | None = None):
    """Per-token quantization alone: returns (q int8 [M, ldq], s f32 [M])."""
    M, K = A.shape
    ldq = ldq or K
    q = torch.empty((M, ldq), dtype=torch.int8, device=A.device)
    s = torch.empty((M,), dtype=torch.float32, device=A.device)
    check(_lib.load().qlin_quantize(M, K, _ptr(A), _DT[A.dtype], A.stride(0),
                                    _ptr(gamma) if gamma is not None else None, eps, _ptr(q), ldq, _ptr(s),
                                    _ptr(err) if err is not None else None, flags, _stream()),
          "qlin_quantize")
    return q, s


def gemm_i32(ws: Workspace, w: Weights, q: torch.Tensor) -> torch.Tensor:
    M = q.shape[0]
    acc = torch.empty((M, w.N), dtype=torch.int32, device=q.device)
    check(_lib.load().qlin_gemm_i32(ws.handle, w.handle, M, _ptr(q), q.stride(0), _ptr(acc), acc.stride(0),
                                    _stream()), "qlin_gemm_i32")
    return acc


def run_quantized(ws: Workspace, w: Weights, q: torch.Tensor, s: torch.Tensor, out_dtype=torch.float16,
                  flags: int = 0) -> torch.Tensor:
    M = q.shape[0]
    ncols = w.N // 2 if flags & QLIN_SWIGLU else w.N
    out = torch.empty((M, ncols), dtype=out_dtype, device=q.device)
    check(_lib.load().qlin_run_quantized(ws.handle, w.handle, M, _ptr(q), q.stride(0), _ptr(s), _ptr(out),
                                         _DT[out_dtype], out.stride(0), flags, _stream()), "qlin_run_quantized")
    return out


def run_host_f32(ws: Workspace, w: Weights, A: np.ndarray, swiglu: bool = False) -> np.ndarray:
    """The synchronous host-buffer entry (drop-in for rk_npu_w4a8_run_f32 / _run_swiglu_f32)."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    M = A.shape[0]
    out = np.zeros((M, w.N // 2 if swiglu else w.N), np.float32)
    fn = _lib.load().qlin_run_swiglu_f32 if swiglu else _lib.load().qlin_run_f32
    rc = fn(ws.handle, w.handle, M, A.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p))
    check(rc, "qlin_run_f32")
    return out


def pack_w4_nk(codes_nk: np.ndarray) -> np.ndarray:
    """[N, K] codes in [-8, 7] -> [N, K/2] bytes, low nibble = even k (the packing the
    weight-creation entry points take; the library reorders nibbles for its kernels)."""
    c = np.ascontiguousarray(codes_nk, dtype=np.int8).astype(np.uint8) & 0xF
    return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)
