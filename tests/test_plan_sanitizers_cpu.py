"""The host layout planners (csrc/plan.cpp) under AddressSanitizer with
UndefinedBehaviorSanitizer, and under ThreadSanitizer.

Each build compiles plan.cpp with g++ together with tests/sanitize/plan_driver.cpp
(host code only, no GPU), then runs the driver: panel (plain and pair), band
and row-block plans of several graphs on one and on 16 threads must agree, and
out-of-range columns must be rejected.  Any sanitizer report fails the run.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "neurosim-gpu_amd" / "csrc"
DRIVER = ROOT / "tests" / "sanitize" / "plan_driver.cpp"


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
@pytest.mark.parametrize("sanitizer", ["address,undefined", "thread"])
def test_planners_under_sanitizers(tmp_path, sanitizer):
    exe = tmp_path / "plan_driver"
    build = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-pthread",
             f"-fsanitize={sanitizer}", "-fno-sanitize-recover=all", "-D_GLIBCXX_ASSERTIONS",
             f"-I{ROOT / 'include'}", f"-I{CSRC}", str(CSRC / "plan.cpp"), str(DRIVER),
             "-o", str(exe)]
    subprocess.run(build, check=True, capture_output=True, timeout=300)
    env = {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
           "TSAN_OPTIONS": "halt_on_error=1", "PATH": "/usr/bin:/bin"}
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    assert run.returncode == 0, run.stderr[-4000:]
    assert run.stdout.strip() == "ok"
    assert "Sanitizer" not in run.stderr, run.stderr[-4000:]
