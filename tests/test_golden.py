"""The committed fixtures (tests/golden/, written by make_golden.py): the
generator reproduces their inputs bit for bit, the float64 closed form
reproduces their answers, the oracle (restated eager path) meets the parity
bar against them, and BASELINE config 1's checksums hold.  The GPU side is
tests/test_golden_gpu.py."""
import importlib.util
import os

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_maker():
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


MG = load_maker()
NAMES = [c[0] for c in MG.CASES]


def fixture(name):
    """(case tuple, q, k, v, mask, slopes, expected) from cases.npz."""
    z = np.load(os.path.join(HERE, "cases.npz"))
    case = next(c for c in MG.CASES if c[0] == name)
    dtype = case[8]

    def tensor(a):
        t = torch.from_numpy(a)
        return t.view(dtype) if dtype in (torch.bfloat16, torch.float16) else t

    q, k, v = (tensor(z[f"{name}/{n}"]) for n in "qkv")
    mask = torch.from_numpy(z[f"{name}/mask"]) if f"{name}/mask" in z.files else None
    slopes = torch.from_numpy(z[f"{name}/alibi"]) if f"{name}/alibi" in z.files else None
    return case, q, k, v, mask, slopes, z[f"{name}/expected"]


def kwargs(case, slopes):
    opts = case[9]
    return dict(causal=opts.get("causal", False), window_size=opts.get("window_size"),
                softmax_scale=opts.get("softmax_scale"), alibi_slopes=slopes)


def parity(out: np.ndarray, ref: np.ndarray, dtype, what: str):
    """The north star's bars: bf16/fp16 max abs <= 2e-2 and mean abs <= 2e-3;
    fp32 max abs <= 1e-5 of the largest reference element."""
    d = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    if dtype == torch.float32:
        assert d.max() <= 1e-5 * np.abs(ref).max(), (what, d.max())
    else:
        assert d.max() <= 2e-2 and d.mean() <= 2e-3, (what, d.max(), d.mean())


@pytest.mark.parametrize("name", NAMES)
def test_fixture_inputs_and_closed_form_reproduce(name):
    case, q, k, v, mask, slopes, expected = fixture(name)
    _, seed, B, Sq, Sk, H, Hkv, D, dtype, opts = case
    q2, k2, v2, mask2, slopes2 = MG.case_inputs(seed, B, Sq, Sk, H, Hkv, D, dtype, opts)
    for a, b in ((q, q2), (k, k2), (v, v2)):
        assert torch.equal(a.view(torch.int16) if a.dtype != torch.float32 else a,
                           b.view(torch.int16) if b.dtype != torch.float32 else b)
    assert (mask is None) == (mask2 is None) and (mask is None or torch.equal(mask, mask2))
    cf = orc.closed_form(q, k, v, attn_mask=mask, **kwargs(case, slopes))
    assert np.allclose(cf.astype(np.float32), expected, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_meets_the_bar_on_fixtures(name):
    case, q, k, v, mask, slopes, expected = fixture(name)
    out = orc.functional_attention(q, k, v, attn_mask=mask, **kwargs(case, slopes))
    parity(out.float().numpy(), expected, case[8], name)


def test_c1_checksums():
    from trinix_amd.workloads import WORKLOADS, make_inputs

    z = np.load(os.path.join(HERE, "c1_checksums.npz"))
    w = WORKLOADS["c1"]
    inp = make_inputs(w)
    sums = np.array([t.double().sum().item() for t in (inp.q, inp.k, inp.v)])
    assert np.array_equal(sums, z["input_sums"])
    out = orc.closed_form(inp.q, inp.k, inp.v, causal=w.causal).reshape(-1)
    assert np.allclose(out[z["sample_index"]], z["sample_value"], rtol=1e-12, atol=1e-12)
    assert abs(out.sum() - z["out_sum"]) <= 1e-9 * max(1.0, abs(float(z["out_abs_sum"])))
