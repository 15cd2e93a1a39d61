"""C ABI checks that need no GPU: the library loads, exports every entry point the
header declares, and rejects invalid arguments before touching the device."""
import ctypes
import os
import re

import numpy as np
import pytest

from open_rknpu2_lm_infer_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names += re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(qlin_\w+)\s*\(", text, re.M)
    return names


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 18
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_strerror_names_every_code():
    for rc in (0, -1, -2, -3, -4, -5, -6):
        assert _lib.strerror(rc) != "unknown error"
    assert _lib.strerror(-99) == "unknown error"


def _create(bits, K, N, codes, scales):
    cfg = _lib.WeightConfig(bits, K, N)
    h = ctypes.c_void_p()
    rc = _lib.load().qlin_weights_create(ctypes.byref(cfg),
                                         codes.ctypes.data_as(ctypes.c_void_p) if codes is not None else None,
                                         scales.ctypes.data_as(ctypes.c_void_p) if scales is not None else None,
                                         ctypes.byref(h))
    return rc, h


@pytest.mark.parametrize("bits,K,N", [(3, 8, 8), (16, 8, 8), (4, 0, 8), (8, 8, -1), (8, 1 << 20, 8)])
def test_weights_create_rejects_bad_geometry(bits, K, N):
    codes = np.zeros((max(K, 1), max(N, 1)), np.int8)
    scales = np.ones(max(N, 1), np.float32)
    rc, h = _create(bits, K, N, codes, scales)
    assert rc == _lib.QLIN_ERR_PARAM and not h.value


def test_weights_create_rejects_bad_codes_and_scales():
    codes = np.zeros((8, 4), np.int8)
    scales = np.ones(4, np.float32)
    bad = codes.copy()
    bad[3, 1] = 8  # outside W4 [-8, 7]
    assert _create(4, 8, 4, bad, scales)[0] == _lib.QLIN_ERR_PARAM
    bad[3, 1] = -128  # outside W8 [-127, 127]
    assert _create(8, 8, 4, bad, scales)[0] == _lib.QLIN_ERR_PARAM
    for s in (0.0, -1.0, np.nan, np.inf):
        sc = scales.copy()
        sc[2] = s
        assert _create(8, 8, 4, codes, sc)[0] == _lib.QLIN_ERR_PARAM
    assert _create(8, 8, 4, None, scales)[0] == _lib.QLIN_ERR_PARAM
    assert _create(8, 8, 4, codes, None)[0] == _lib.QLIN_ERR_PARAM


def test_null_handles_rejected():
    L = _lib.load()
    assert L.qlin_run_f32(None, None, 1, None, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_run(None, None, 1, None, 0, 1, None, 0, 1, 0, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_weights_query(None, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_workspace_query(None, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_workspace_status(None, 0) == _lib.QLIN_ERR_PARAM
    h = ctypes.c_void_p()
    assert L.qlin_workspace_create(0, 8, 8, ctypes.byref(h)) == _lib.QLIN_ERR_PARAM
    assert L.qlin_workspace_create(4, 8, 0, ctypes.byref(h)) == _lib.QLIN_ERR_PARAM
    assert L.qlin_quantize(0, 8, None, 0, 8, None, 0.0, None, 8, None, None, 0, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_swiglu(0, 8, None, 0, 16, None, 0, 8, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_swiglu(1, 8, None, 0, 16, None, 0, 8, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_run_plan(None, None, 1, None, 8, None, 0, None) == _lib.QLIN_ERR_PARAM
    assert L.qlin_chain_set_wait_limit(None, 0) == _lib.QLIN_ERR_PARAM
    L.qlin_weights_free(None)
    L.qlin_workspace_free(None)


def test_structs_match_header_sizes():
    assert ctypes.sizeof(_lib.WeightConfig) == 12
    assert ctypes.sizeof(_lib.WeightInfo) == 32
    assert ctypes.sizeof(_lib.WorkspaceInfo) == 24
    assert ctypes.sizeof(_lib.DeviceInfo) == 48
    assert ctypes.sizeof(_lib.ChainStage) == 48
    assert ctypes.sizeof(_lib.Plan) == 48


def test_static_archive_links_and_runs():
    """libqlinear.a carries every declared entry point, and a C program linked against it
    whole (the way the reference's build.rs links its native library, build.rs:13-67)
    runs its argument checks without a GPU."""
    import subprocess
    here = os.path.join(ROOT, "open_rknpu2_lm_infer_amd")
    syms = subprocess.run(["nm", "-g", "--defined-only", os.path.join(here, "libqlinear.a")], check=True,
                          capture_output=True, text=True).stdout
    defined = set(re.findall(r"\bT (qlin_\w+)", syms))
    assert set(declared_functions()) <= defined, set(declared_functions()) - defined
    exe = os.path.join(ROOT, "tests", "cpp", "_build", "static_link_test")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "static link ok" in r.stdout, (r.returncode, r.stdout, r.stderr)
