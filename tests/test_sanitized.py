"""The CPU suite again under AddressSanitizer + UndefinedBehaviorSanitizer
(tests/run_sanitized.sh): the oracle and the product library's host code --
the C-ABI validation, kernel choice and launch glue, the C++ ops::attention
mirror -- built with the sanitizers, every CPU test run against them, and a
planted out-of-bounds call into the sanitized oracle that must be caught.
CPU only; the sanitized libraries never reach a GPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpu_suite_under_asan_and_ubsan():
    if not shutil.which("/opt/rocm/llvm/bin/clang") or not shutil.which("hipcc"):
        pytest.skip("ROCm clang / hipcc not available")
    env = dict(os.environ)
    env.pop("LD_PRELOAD", None)
    res = subprocess.run(["bash", os.path.join(ROOT, "tests", "run_sanitized.sh"), "-k", "not under_asan"],
                         capture_output=True, text=True, timeout=1200, env=env)
    tail = (res.stdout + res.stderr)[-3000:]
    assert res.returncode == 0, tail
    assert "planted overflow caught" in res.stdout, tail
    assert " passed" in res.stdout and " failed" not in res.stdout, tail
