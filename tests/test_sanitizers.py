"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the host code that executes on
the CPU: the oracle (every entry point the tests use, edge cases included) and the
library's checkpoint readers (fixtures, every truncation of them and 400 random
single-byte corruptions each).  Built with gcc / g++ by tests/sanitize/Makefile."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None, reason="needs gcc and g++")
def test_host_code_under_asan_ubsan():
    r = subprocess.run(["make", "-s", "-C", HERE, "run"], capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "oracle sanitizer run: ok" in out and "checkpoint reader sanitizer run: ok" in out
