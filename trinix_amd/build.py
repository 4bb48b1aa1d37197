"""Builds ``libtrinix_attn.so`` (the gfx950 HIP kernels + C ABI) in-tree.

``python -m trinix_amd.build`` compiles every ``csrc/*.hip`` file with hipcc
for gfx950 into ``trinix_amd/lib/libtrinix_attn.so``.  The library is loaded
by ``trinix_amd._native`` through ctypes; nothing is compiled at import time.

Every compile also reports each kernel's register use
(``-Rpass-analysis=kernel-resource-usage``) and keeps its gfx950 assembly
(``-save-temps=obj``, next to the objects).  The build fails if any kernel
spills to memory (scratch, VGPR spills) or holds a register spilled into an
accumulation register (the assembly's "Spill" / "Reload" annotations): a
spilling build once mis-restored an operand saved into an AGPR and produced
wrong scores.  SGPR spills go to lanes of a VGPR (no memory) and are only
reported.  The per-kernel table is written to ``lib/resource_usage.txt``.
"""
from __future__ import annotations

import os
import re
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
RESOURCE_REPORT = LIB_DIR / "resource_usage.txt"

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


def host_sources() -> list[Path]:
    """Plain C++ host code (argument checks, launch planning), compiled by g++."""
    return sorted(CSRC_DIR.glob("*.cpp"))


def _compile_flags() -> list[str]:
    return [*HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}"]


_REMARK = re.compile(r"remark: .*?(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]|"
                     r"SGPRs Spill|VGPRs Spill): (\S+)")


def parse_resource_remarks(text: str) -> dict:
    """{kernel symbol: {field: value}} from -Rpass-analysis=kernel-resource-usage output."""
    out, cur = {}, None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key.split(" [")[0]] = int(val)
    return out


def asm_spill_annotations(asm_path: Path) -> dict:
    """{kernel symbol: count} of spill / reload annotations in a gfx950 .s file."""
    counts, cur = {}, None
    if not asm_path.exists():
        return counts
    for line in asm_path.read_text().splitlines():
        m = re.match(r"([A-Za-z_][\w$]*):", line)
        if m:
            cur = m.group(1)
            continue
        if cur and re.search(r";.*(Spill|Reload)", line):
            counts[cur] = counts.get(cur, 0) + 1
    return counts


def check_resources(per_source: dict, report: Path = RESOURCE_REPORT) -> list[str]:
    """Writes the per-kernel table to ``report``; returns the list of violations."""
    rows, bad = [], []
    for src, (usage, spills) in sorted(per_source.items()):
        for name, u in sorted(usage.items()):
            asm = spills.get(name, 0)
            rows.append(f"{src}\t{name}\tVGPRs={u.get('VGPRs', -1)}\tAGPRs={u.get('AGPRs', -1)}\t"
                        f"occupancy={u.get('Occupancy', -1)}\tscratch={u.get('ScratchSize', -1)}\t"
                        f"vgpr_spill={u.get('VGPRs Spill', -1)}\tsgpr_spill={u.get('SGPRs Spill', -1)}\t"
                        f"asm_spill_annotations={asm}")
            if u.get("ScratchSize", 0) or u.get("VGPRs Spill", 0) or asm:
                bad.append(f"{src}: {name}: scratch {u.get('ScratchSize')} B/lane, VGPR spills "
                           f"{u.get('VGPRs Spill')}, spill annotations {asm}")
    report.write_text("# per-kernel resource usage of the last build (hipcc kernel-resource-usage remarks)\n"
                      + "\n".join(rows) + "\n")
    return bad


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip to an object (in parallel), then link the
    shared library; returns the path of the built ``.so``."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = LIB_DIR / "_obj"
    obj_dir.mkdir(exist_ok=True)
    hipcc = hipcc_path()
    cflags = [f for f in _compile_flags() if f != "-shared"]
    cflags += ["-Rpass-analysis=kernel-resource-usage", "-save-temps=obj"]
    srcs = sources()
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    host_objs = [obj_dir / (s.stem + ".host.o") for s in host_sources()]
    for src, obj in zip(host_sources(), host_objs):
        cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", "-c", str(src),
               "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"g++ failed on {src.name}:\n{res.stderr[-6000:]}")
    jobs = jobs or max(1, min(len(srcs), os.cpu_count() or 1, 8))
    pending = list(zip(srcs, objs))
    running = []
    errors = []
    per_source = {}
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
            continue
        asm = obj_dir / f"{src.stem}-hip-amdgcn-amd-amdhsa-{ARCH}.s"
        per_source[src.name] = (parse_resource_remarks(err), asm_spill_annotations(asm))
        if verbose:
            lines = [l for l in err.splitlines() if "packed-fp32-ops" not in l and "remark:" not in l
                     and "-Rpass-analysis" not in l and not l.lstrip().startswith(("|", "^"))]
            if lines:
                print("\n".join(lines[-40:]), file=sys.stderr)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    bad = check_resources(per_source)
    if bad:
        raise RuntimeError("kernels spill registers to memory or to accumulation registers:\n" + "\n".join(bad))
    tmp = LIB_DIR / (LIB_NAME + f".tmp{os.getpid()}")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), *map(str, host_objs), "-o", str(tmp)]
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
