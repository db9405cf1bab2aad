"""Host sanitizer run (CPU): the library's host side (desc validation, size
queries, pair and static-scratch entry points, conv validation) and the C oracle,
built with AddressSanitizer + UndefinedBehaviorSanitizer by tests/sanitize/Makefile
and exercised by tests/sanitize/abi_check.cpp.  No GPU work is launched: every
library call there is refused by validation first."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")
BIN = os.path.join(HERE, "_build", "abi_check")


def test_host_code_is_clean_under_asan_and_ubsan():
    if shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc / make not available: the sanitizer build needs the ROCm toolchain")
    # incremental: rebuilds only when the library, the oracle or the harness changed
    build = subprocess.run(["make", "-C", HERE], capture_output=True, text=True)
    assert build.returncode == 0, build.stdout[-2000:] + build.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([BIN], capture_output=True, text=True, env=env, timeout=600)
    out = run.stdout + run.stderr
    assert run.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert "all checks passed" in out
