"""Runs the native port of the reference's board tests (tests/cpp/npu_backend_test.cpp)
against the C++ npu::Backend / npu::Linear mirror."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "npu_backend_test")


def _run(mode, timeout):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built: run python -m open_rknpu2_lm_infer_amd.build")
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert f"PASS {mode} tests" in r.stdout


def test_npu_mirror_host_logic():
    _run("cpu", 60)


@pytest.mark.gpu
def test_npu_mirror_reference_board_tests():
    _run("gpu", 110)
