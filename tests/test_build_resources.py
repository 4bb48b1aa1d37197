"""CPU checks of the build's register guard.

``trinix_amd.build`` compiles every kernel with hipcc's kernel-resource-usage
remarks and keeps the gfx950 assembly, and fails if a kernel spills to
scratch memory, spills VGPRs, or carries a spill / reload annotation (a
register parked in an accumulation register: a spilling build of the D=256
mask kernel once mis-restored such a register and computed wrong scores).
These tests pin the parsers on planted inputs and check the table the last
build wrote for the shipped library.
"""
import os
import re
from pathlib import Path

import pytest

from trinix_amd import build as B


REMARKS = """\
x.hip:46:0: remark: Function Name: _Zkernel_a [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     VGPRs: 203 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     SGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark: Function Name: _Zkernel_b [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:46:0: remark:     VGPRs Spill: 2 [-Rpass-analysis=kernel-resource-usage]
"""

ASM = """\
_Zkernel_a:                             ; @_Zkernel_a
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
\tv_accvgpr_write_b32 a3, v7            ;  Reload Reuse
\ts_endpgm
.Lfunc_end0:
_Zkernel_c:                             ; @_Zkernel_c
\tv_add_f32_e32 v1, v2, v3
\ts_endpgm
"""


def test_remark_and_asm_parsers_flag_planted_spills(tmp_path):
    usage = B.parse_resource_remarks(REMARKS)
    assert usage["_Zkernel_a"] == {"VGPRs": 203, "AGPRs": 0, "ScratchSize": 0, "Occupancy": 2, "SGPRs Spill": 3,
                                   "VGPRs Spill": 0}
    assert usage["_Zkernel_b"]["ScratchSize"] == 12 and usage["_Zkernel_b"]["VGPRs Spill"] == 2
    asm = tmp_path / "k.s"
    asm.write_text(ASM)
    spills = B.asm_spill_annotations(asm)
    assert spills == {"_Zkernel_a": 1}
    bad = B.check_resources({"x.hip": (usage, spills)}, tmp_path / "report.txt")
    # kernel_a: a parked register in the assembly; kernel_b: scratch and VGPR spills
    assert len(bad) == 2 and any("_Zkernel_a" in b for b in bad) and any("_Zkernel_b" in b for b in bad)
    clean = {"_Zkernel_c": dict(usage["_Zkernel_a"])}
    assert B.check_resources({"y.hip": (clean, {})}, tmp_path / "report2.txt") == []


def _report_rows():
    srcs = B.sources() + list(B.CSRC_DIR.glob("*.h")) + [B.INCLUDE_DIR / "trinix_attn.h"]
    newest = max(os.path.getmtime(p) for p in srcs)
    if not B.RESOURCE_REPORT.exists() or os.path.getmtime(B.RESOURCE_REPORT) < newest:
        B.build()  # raises if any kernel spills
    rows = []
    for line in B.RESOURCE_REPORT.read_text().splitlines():
        if line.startswith("#") or not line.strip():
            continue
        src, name, *fields = line.split("\t")
        rows.append((src, name, dict(f.split("=") for f in fields)))
    return rows


def test_shipped_kernels_do_not_spill():
    rows = _report_rows()
    names = " ".join(name for _, name, _ in rows)
    for family in ("attn_fwd_mfma16", "attn_fwd_f32", "attn_bwd_dkdv", "attn_bwd_dq", "bwd_dkdv_generic",
                   "bwd_dq_generic", "attn_decode16", "attn_decode_combine", "rope16_kernel", "qk_norm_kernel",
                   "blockmap_kernel", "alibi_bias_kernel"):
        assert family in names, family
    # every (dtype, head_dim, feature) instantiation of the forward is there
    assert len([n for _, n, _ in rows if "attn_fwd_mfma16" in n]) >= 2 * 3 * 8
    for src, name, f in rows:
        assert f["scratch"] == "0" and f["vgpr_spill"] == "0" and f["asm_spill_annotations"] == "0", (src, name, f)
