"""The HIP path against the committed fixtures of tests/golden/ (float64
closed-form answers of small problems covering every feature of the path,
and BASELINE config 1's checksums), at the north star's parity bars."""
import os

import numpy as np
import pytest
import torch

from test_golden import HERE, NAMES, fixture, kwargs, parity
import trinix_amd as tx

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("name", NAMES)
def test_hip_path_matches_fixture(name):
    case, q, k, v, mask, slopes, expected = fixture(name)
    print(f"golden case {name} {tuple(q.shape)} {tuple(k.shape)} {case[8]}", flush=True)
    kw = kwargs(case, None if slopes is None else slopes.to(DEV))
    out = tx.triton_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), attn_mask=None if mask is None else mask.to(DEV),
                              **kw)
    parity(out.float().cpu().numpy(), expected, case[8], name)


def test_hip_path_matches_c1_checksums():
    from trinix_amd.workloads import WORKLOADS, make_inputs

    z = np.load(os.path.join(HERE, "c1_checksums.npz"))
    w = WORKLOADS["c1"]
    inp = make_inputs(w, device=DEV)
    out = tx.triton_attn_func(inp.q, inp.k, inp.v, causal=w.causal).double().cpu().numpy().reshape(-1)
    scale = np.abs(z["sample_value"]).max()
    assert np.abs(out[z["sample_index"]] - z["sample_value"]).max() <= 1e-5 * scale
    assert abs(out.sum() - float(z["out_sum"])) <= 1e-5 * float(z["out_abs_sum"])
