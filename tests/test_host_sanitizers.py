"""CPU: the library's host-side argument checks and launch planning
(``trinix_amd/csrc/host_plan.cpp``: forward/backward validation, the tile
choice, the split-KV decode plan) built with AddressSanitizer and
UndefinedBehaviorSanitizer, every report fatal, and driven through the C
ABI's status-code cases plus a seeded fuzz over int64 extremes
(``tests/sanitize/host_plan_check.cpp``)."""
import shutil
import subprocess
from pathlib import Path

import pytest

from trinix_amd.build import CSRC_DIR, INCLUDE_DIR

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_plan_under_asan_ubsan(tmp_path):
    exe = tmp_path / "host_plan_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", str(CSRC_DIR / "host_plan.cpp"),
           str(HERE / "sanitize" / "host_plan_check.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("ok"), res.stdout
    assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr
