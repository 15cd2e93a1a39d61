"""ctypes binding of libqlinear.so (include/qlinear.h).

The library is the product: every compute call here goes to the HIP kernels, and
loading fails loudly when the library has not been built.  torch is imported
before the library is opened so both bind the same HIP runtime (libamdhip64.so.7
is matched by SONAME once torch has loaded it).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqlinear.so")

QLIN_OK = 0
QLIN_ERR_PARAM = -1
QLIN_ERR_NOMEM = -2
QLIN_ERR_DEVICE = -3
QLIN_ERR_NONFINITE = -4
QLIN_ERR_UNSUPPORTED = -5
QLIN_ERR_NODEVICE = -6

QLIN_F32 = 0
QLIN_F16 = 1

QLIN_ROUND_HALF_EVEN = 0x1
QLIN_NORM_SEQUENTIAL = 0x2
QLIN_SWIGLU = 0x4
QLIN_NO_FUSED_QUANT = 0x8
QLIN_RESIDUAL = 0x10

QLIN_PATH_GEMV_FUSED = 0
QLIN_PATH_GEMV = 1
QLIN_PATH_GEMM = 2

QLIN_PACK_QUANTIZED = 0
QLIN_INT_QUANTIZED = 1

# Every function declared in include/qlinear.h: name -> (restype, argtypes)
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_F = ctypes.c_float
SIGNATURES = {
    "qlin_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "qlin_device_query": (ctypes.c_int, [_I32, _P]),
    "qlin_weights_create": (ctypes.c_int, [_P, _P, _P, _P]),
    "qlin_weights_create_packed": (ctypes.c_int, [_P, _P, _P, _P]),
    "qlin_weights_create_packed_device": (ctypes.c_int, [_P, _P, _P, _P, _P]),
    "qlin_weights_free": (None, [_P]),
    "qlin_weights_query": (ctypes.c_int, [_P, _P]),
    "qlin_workspace_create": (ctypes.c_int, [_I32, _I32, _I32, _P]),
    "qlin_workspace_free": (None, [_P]),
    "qlin_workspace_query": (ctypes.c_int, [_P, _P]),
    "qlin_workspace_status": (ctypes.c_int, [_P, _I32]),
    "qlin_run_f32": (ctypes.c_int, [_P, _P, _I32, _P, _P]),
    "qlin_run_swiglu_f32": (ctypes.c_int, [_P, _P, _I32, _P, _P]),
    "qlin_run": (ctypes.c_int, [_P, _P, _I32, _P, _I32, _I64, _P, _I32, _I64, _U32, _P]),
    "qlin_run_rmsnorm": (ctypes.c_int, [_P, _P, _I32, _P, _I32, _I64, _P, _F, _P, _I32, _I64, _U32, _P]),
    "qlin_run_residual": (ctypes.c_int, [_P, _P, _I32, _P, _I32, _I64, _P, _I32, _I64, _F, _P, _I32, _I64, _U32,
                                         _P]),
    "qlin_quantize": (ctypes.c_int, [_I32, _I32, _P, _I32, _I64, _P, _F, _P, _I64, _P, _P, _U32, _P]),
    "qlin_gemm_i32": (ctypes.c_int, [_P, _P, _I32, _P, _I64, _P, _I64, _P]),
    "qlin_run_quantized": (ctypes.c_int, [_P, _P, _I32, _P, _I64, _P, _P, _I32, _I64, _U32, _P]),
    "qlin_weights_create_compressed": (ctypes.c_int, [_P, _I32, _I32, _P, _P, _P, _P]),
    "qlin_tune": (ctypes.c_int, [_P, _P, _I32, _U32, _I32, _P]),
    "qlin_tune_count": (ctypes.c_int, []),
    "qlin_tune_clear": (None, []),
    "qlin_tune_save": (ctypes.c_int, [ctypes.c_char_p]),
    "qlin_tune_load": (ctypes.c_int, [ctypes.c_char_p]),
    "qlin_chain_create": (ctypes.c_int, [_P, _I32, _I32, _P]),
    "qlin_chain_free": (None, [_P]),
    "qlin_chain_run": (ctypes.c_int, [_P, _I32, _P, _I64, _P, _I64, _P]),
    "qlin_chain_stage_output": (ctypes.c_int, [_P, _I32, _P, _P]),
    "qlin_chain_status": (ctypes.c_int, [_P, _I32]),
    "qlin_chain_set_wait_limit": (ctypes.c_int, [_P, _I32]),
    "qlin_run_noalloc": (ctypes.c_int, [_P, _I32, _P, _I32, _I64, _P, _F, _P, _I32, _I64, _U32, _P, _P]),
    "qlin_swiglu": (ctypes.c_int, [_I32, _I32, _P, _I32, _I64, _P, _I32, _I64, _P]),
    "qlin_run_plan": (ctypes.c_int, [_P, _P, _I32, _P, _I64, _P, _U32, _P]),
}


class WeightConfig(ctypes.Structure):
    _fields_ = [("bits", _I32), ("K", _I32), ("N", _I32)]


class WeightInfo(ctypes.Structure):
    _fields_ = [("bits", _I32), ("K", _I32), ("N", _I32), ("K_padded", _I32), ("N_padded", _I32),
                ("device", _I32), ("device_bytes", ctypes.c_uint64)]


class WorkspaceInfo(ctypes.Structure):
    _fields_ = [("max_rows", _I32), ("reserved", _I32), ("device_bytes", ctypes.c_uint64),
                ("pinned_host_bytes", ctypes.c_uint64)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("device", _I32), ("cu_count", _I32), ("arch", _I32), ("reserved", _I32),
                ("sclk_khz", _I64), ("mclk_khz", _I64), ("bus_width_bits", _I64), ("hbm_bytes", _I64)]


class Plan(ctypes.Structure):
    _fields_ = [("path", _I32), ("launches", _I32), ("waves", _I32), ("item_width", _I32), ("items", _I32),
                ("grid", _I32), ("splits", _I32), ("tile_m", _I32), ("tile_n", _I32), ("reserved", _I32 * 3)]


class ChainStage(ctypes.Structure):
    _fields_ = [("weights", _P), ("flags", _U32), ("gamma", _P), ("eps", _F), ("input", _I32),
                ("input_offset", _I32), ("residual", _I32), ("residual_offset", _I32),
                ("residual_multiplier", _F)]


class QlinError(RuntimeError):
    def __init__(self, rc: int, what: str):
        self.rc = rc
        super().__init__(f"{what}: {strerror(rc)} ({rc})")


_lib = None


def load():
    """Open libqlinear.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    try:
        import torch  # noqa: F401  (binds the process to torch's HIP runtime first)
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m open_rknpu2_lm_infer_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def strerror(rc: int) -> str:
    return load().qlin_strerror(rc).decode()


def check(rc: int, what: str) -> None:
    if rc != QLIN_OK:
        raise QlinError(rc, what)


def device_info(device: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    check(load().qlin_device_query(device, ctypes.byref(info)), "qlin_device_query")
    return info
