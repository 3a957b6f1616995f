"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

tests/native/sanitize.mk builds librocketnpu with each -fsanitize= applied to the host pass
(device code unchanged) and links tests/native/shim_check.cpp, which drives every path that
needs no GPU: planners, rejections, the log channel, hardware profiles, the serialised-weight
reader on intact and corrupted blobs, the fp64 FFN / attention host references against the
oracle (built into the same binary with the same sanitizers), and handle-table calls from
several threads. Any sanitizer report fails the run.
"""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_host_code_under_asan_and_ubsan():
    if not os.path.exists("/opt/rocm/bin/hipcc") or not shutil.which("make"):
        pytest.skip("needs hipcc and make")
    import torch
    if torch.cuda.is_available():
        pytest.skip("the sanitizer driver targets machines without a GPU")
    jobs = str(min(8, os.cpu_count() or 4))
    b = subprocess.run(["make", "-f", os.path.join(REPO, "tests", "native", "sanitize.mk"), "-j", jobs],
                       capture_output=True, text=True, timeout=900)
    assert b.returncode == 0, b.stdout[-3000:] + b.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([os.path.join(REPO, "_build_asan", "shim_check"), os.path.join(REPO, "tests", "golden")],
                       capture_output=True, text=True, timeout=600, env=env, cwd=REPO)
    report = r.stderr[-4000:]
    assert r.returncode == 0, report
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, report
    assert "all checks passed" in r.stdout
