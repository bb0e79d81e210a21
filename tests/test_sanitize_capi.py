"""The C-ABI's host-side validation under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU: tests/sanitize/capi_validation.cpp
calls every entry point with arguments it must reject (and the workspace
queries with valid, invalid and overflowing shapes) against a sanitized
host-only build of the library; any memory error, undefined behaviour, leak
or wrong return code fails the run."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(not Path("/opt/rocm/bin/hipcc").exists(), reason="needs hipcc")
def test_capi_validation_under_asan_ubsan():
    sys.path.insert(0, str(HERE / "sanitize"))
    try:
        import build as san_build
    finally:
        sys.path.pop(0)
    exe = san_build.build()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "0 failures" in r.stdout
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
