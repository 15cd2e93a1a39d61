"""The static archive on the GPU: a C program linked against libqlinear.a whole, the way
the reference's build.rs links its native library (build.rs:13-67), creates W4 weights,
runs the M=1 decode GEMV and the M=64 prefill GEMM through qlin_run_f32 (host buffers)
and one qlin_run_noalloc (device buffers, the static scratch array), and checks each bit
for bit against the CPU oracle compiled into it (tests/cpp/static_link_test.c)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.gpu


def test_static_archive_runs_kernels():
    exe = os.path.join(ROOT, "tests", "cpp", "_build", "static_link_test")
    assert os.path.exists(exe), "build first: python -m open_rknpu2_lm_infer_amd.build"
    print("[static] static_link_test gpu", flush=True)
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "static link gpu ok" in r.stdout, (r.returncode, r.stdout, r.stderr)
