"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/sanitize/Makefile builds, into _build/asan, sanitized copies of the f64
oracle (C), of librhizome_gdr.so's host side (the C ABI's validation and
dispatch; GPU code is not instrumented) and of the host layer with its C++
test programs, then runs those programs and the CPU test suites of the ABI,
its fuzzing, the oracle, the planner and the adjoint against the sanitized
libraries.  Any memory error or undefined behaviour aborts the run.

CPU only: the sanitized library is never loaded where a GPU is visible.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _gpu_visible() -> bool:
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.mark.skipif(_gpu_visible(), reason="CPU-only: the sanitized build is exercised without a GPU")
@pytest.mark.skipif(not shutil.which("make") or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs make and hipcc")
def test_host_code_under_asan_and_ubsan():
    res = subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "tests", "sanitize"), "check"],
                         capture_output=True, text=True, timeout=1500)
    tail = (res.stdout + res.stderr)[-4000:]
    assert res.returncode == 0, tail
    assert "OK: 0 failed" in res.stdout and " passed" in res.stdout, tail
    assert "ERROR: AddressSanitizer" not in res.stderr and "runtime error" not in res.stderr, tail
