"""The planners under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/native/plan_check.cpp drives ssl_plan_build, ssl_prefill_plan_build and
ssl_debug_set with thousands of random and corrupted structures and checks
every table; here it is compiled with csrc/plan.cpp by the host compiler (the
planners use no HIP) with both sanitizers on and run. Any out-of-bounds
access, leak, overflow or failed check fails the test.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_planners_are_clean_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "plan_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I", str(ROOT / "include"),
           str(ROOT / "s-salaad_amd" / "csrc" / "plan.cpp"),
           str(ROOT / "tests" / "native" / "plan_check.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                              "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert res.returncode == 0, res.stderr[-4000:]
    assert "all checks passed" in res.stdout
