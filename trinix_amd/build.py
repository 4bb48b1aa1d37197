"""Builds ``libtrinix_attn.so`` (the gfx950 HIP kernels + C ABI) in-tree.

``python -m trinix_amd.build`` compiles every ``csrc/*.hip`` file with hipcc
for gfx950 into ``trinix_amd/lib/libtrinix_attn.so``.  The library is loaded
by ``trinix_amd._native`` through ctypes; nothing is compiled at import time.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "lib"
LIB_NAME = "libtrinix_attn.so"
LIB_PATH = LIB_DIR / LIB_NAME

ARCH = "gfx950"

# Packed-FP32 VALU ops are switched off for all device code: hipcc -O3 would
# otherwise form v_pk_{add,mul,fma}_f32 from scalar float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the gfx950 HIP library cannot be built")
    return found


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def _compile_flags() -> list[str]:
    return [*HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}"]


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip to an object (in parallel), then link the
    shared library; returns the path of the built ``.so``."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = LIB_DIR / "_obj"
    obj_dir.mkdir(exist_ok=True)
    hipcc = hipcc_path()
    cflags = [f for f in _compile_flags() if f != "-shared"]
    srcs = sources()
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    jobs = jobs or max(1, min(len(srcs), os.cpu_count() or 1, 8))
    pending = list(zip(srcs, objs))
    running = []
    errors = []
    while pending or running:
        while pending and len(running) < jobs:
            src, obj = pending.pop(0)
            cmd = [hipcc, *cflags, "-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            running.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        src, proc = running.pop(0)
        _, err = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"{src.name}:\n{err[-6000:]}")
        elif verbose:
            lines = [l for l in err.splitlines() if "packed-fp32-ops" not in l]
            if lines:
                print("\n".join(lines[-40:]), file=sys.stderr)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    tmp = LIB_DIR / (LIB_NAME + f".tmp{os.getpid()}")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        if tmp.exists():
            tmp.unlink()
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
