"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer: every function
runs on small and edge-case inputs (tests/cpp/oracle_sanitize.c, built by
`make -C oracle sanitize`) without an out-of-bounds access, an overflowing float-to-int
conversion, a float division by zero or other undefined behaviour.  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("make") is None, reason="needs gcc and make")
def test_oracle_clean_under_sanitizers():
    build = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True,
                           text=True, timeout=300)
    assert build.returncode == 0, build.stdout + build.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1", OMP_NUM_THREADS="2")
    run = subprocess.run([os.path.join(ROOT, "tests", "cpp", "_build", "oracle_sanitize")], capture_output=True,
                         text=True, timeout=300, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "oracle sanitize ok" in run.stdout
