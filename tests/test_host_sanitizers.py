"""CPU: the library's host-side argument checks and launch planning
(``trinix_amd/csrc/host_plan.cpp``: forward/backward validation, the tile
choice, the launch plans, the split-KV decode plan) built with
AddressSanitizer and UndefinedBehaviorSanitizer, every report fatal, and
driven through the C ABI's status-code cases plus a seeded fuzz over int64
extremes (``tests/sanitize/host_plan_check.cpp``).  The same driver runs the
bounds model of the kernels' memory accesses (``tests/sanitize/
bounds_model.h``) over the kernels' own index maps
(``trinix_amd/csrc/index_map.h``); a second test plants mistakes in a copy
of those index maps and requires the model to report each one."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from trinix_amd.build import CSRC_DIR, INCLUDE_DIR

HERE = Path(__file__).resolve().parent
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]


def _build(tmp_path, name, extra_inc=(), sanitize=True):
    exe = tmp_path / name
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", *(SANITIZE if sanitize else []),
           *[f"-I{d}" for d in extra_inc], f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", str(CSRC_DIR / "host_plan.cpp"),
           str(HERE / "sanitize" / "host_plan_check.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_plan_under_asan_ubsan(tmp_path):
    exe = _build(tmp_path, "host_plan_check")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("ok"), res.stdout
    assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr
    m = re.search(r"bounds model: (\d+) argument sets, (\d+) checks, (\d+) failures", res.stdout)
    assert m and int(m.group(1)) > 1000 and int(m.group(2)) > 10 ** 8 and m.group(3) == "0", res.stdout


# Mistakes planted in a copy of index_map.h: each must make the bounds model
# report failures (an off-by-one tile count, a lane offset one unit off, a
# row block map that skips a block, a query range that drops a tile, a
# decode chunk past the keys, an unpadded dropout keep map).
PLANTED = [
    ("tr.t_hi = hi > lo ? (int)((hi + BN - 1) / BN) : tr.t_lo;", "tr.t_hi = hi > lo ? (int)(hi / BN) : tr.t_lo;"),
    ("return row * (uint32_t)ss * 2u + unit * 16u;", "return row * (uint32_t)ss * 2u + unit * 16u + 16u;"),
    ("const int mblk = causal ? (num_mblk - 1 - mi) : mi;", "const int mblk = causal ? (num_mblk - 1 - mi) : (mi ? mi - 1 : 0);"),
    ("qt_hi = i_hi > i_lo ? (i_hi + BQ - 1) / BQ : qt_lo;", "qt_hi = i_hi > i_lo ? (i_hi + BQ - 1) / BQ - (kb0 > 0) : qt_lo;"),
    ("c1 = imin(khi, c0 + chunk);", "c1 = imin(khi + 64, c0 + chunk);"),
    # a keep map without the padding to whole 128-key groups
    ("return 4 * ((Sk + 127) / 128);", "return (Sk + 31) / 32;"),
]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
@pytest.mark.parametrize("k", range(len(PLANTED)))
def test_bounds_model_reports_planted_index_mistakes(tmp_path, k):
    old, new = PLANTED[k]
    src = (CSRC_DIR / "index_map.h").read_text()
    assert src.count(old) == 1, old
    mut = tmp_path / "mut"
    mut.mkdir()
    (mut / "index_map.h").write_text(src.replace(old, new))
    exe = _build(tmp_path, "planted", extra_inc=[mut], sanitize=False)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    m = re.search(r"bounds model: (\d+) argument sets, (\d+) checks, (\d+) failures", res.stdout)
    assert m and int(m.group(3)) > 0, res.stdout[-2000:]
    assert res.returncode != 0
