"""Seeded random configurations through ``triton_attn_func`` against the
oracle: a sweep across the paths the dispatcher picks (prefill kernel,
split-KV decode kernel, head-dim padding, fp32 kernel) and the features
they combine (GQA/MQA, causal, windows, ALiBi, masks of every dtype,
scale, lse).  Each case is fixed by its seed, so a failure names a
reproducible configuration.  Bar as in the other parity tests.
"""
import random

import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func
from test_attn_gpu import assert_parity_or_more_accurate, oracle_on, rand

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_case(seed):
    r = random.Random(seed)
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    D = r.choice([32, 64, 64, 80, 128, 128, 192, 256])
    Hkv = r.choice([1, 2, 3])
    H = Hkv * r.choice([1, 2, 4])
    B = r.choice([1, 2])
    Sq = r.choice([1, 2, 5, 16, r.randint(17, 300)])
    Sk = Sq if r.random() < 0.5 else r.choice([1, 63, 64, 65, r.randint(2, 700)])
    kw = {}
    if r.random() < 0.4:
        kw["causal"] = True
    if r.random() < 0.3:
        kw["window_size"] = (r.randint(0, 80), r.randint(0, 80))
    if r.random() < 0.3:
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    if r.random() < 0.3:
        g = torch.Generator().manual_seed(seed)
        kind = r.choice(["f32", "bool", "bf16"])
        m = torch.randn(Sq, Sk, generator=g)
        m[torch.rand(Sq, Sk, generator=g) < 0.2] = float("-inf")
        m[:, 0] = 0.0
        if kind == "bool":
            m = torch.rand(Sq, Sk, generator=g) < 0.7
            m[:, 0] = True
        elif kind == "bf16":
            m = m.to(torch.bfloat16)
        kw["attn_mask"] = m
    if r.random() < 0.2:
        kw["softmax_scale"] = r.uniform(0.02, 0.3)
    return dict(B=B, Sq=Sq, Sk=Sk, H=H, Hkv=Hkv, D=D, dtype=dtype, kw=kw)


SEEDS = list(range(40))


@pytest.mark.parametrize("seed", SEEDS)
def test_random_config(seed):
    c = make_case(seed)
    print(f"seed {seed}: {dict((k, v) for k, v in c.items() if k != 'kw')} {sorted(c['kw'])}", flush=True)
    B, Sq, Sk, H, Hkv, D, dtype, kw = c["B"], c["Sq"], c["Sk"], c["H"], c["Hkv"], c["D"], c["dtype"], c["kw"]
    q, k, v = rand((B, Sq, H, D), dtype, 3 * seed), rand((B, Sk, Hkv, D), dtype, 3 * seed + 1), \
        rand((B, Sk, Hkv, D), dtype, 3 * seed + 2)
    dev_kw = {a: (b.to(DEV) if torch.is_tensor(b) else b) for a, b in kw.items()}
    out, lse = triton_attn_func(q, k, v, return_lse=True, **dev_kw)
    ref_kw = dict(kw)
    if "attn_mask" in ref_kw:
        m = ref_kw["attn_mask"]
        ref_kw["attn_mask"] = (m.to(torch.uint8) if m.dtype == torch.bool else m).float()
    ref = oracle_on(q, k, v, **ref_kw)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), **ref_kw)
    assert_parity_or_more_accurate(out, ref, x64, dtype, f"seed {seed}")
    # log-sum-exp against the fp64 scores (rows with no allowed key: -inf)
    scale = ref_kw.get("softmax_scale", D ** -0.5)
    bias = orc._bias64(Sq, Sk, H, B, ref_kw.get("attn_mask"), ref_kw.get("causal", False),
                       ref_kw.get("window_size"), ref_kw.get("alibi_slopes"))
    qd = q.cpu().double()
    kd = k.cpu().double().repeat_interleave(H // Hkv, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", qd, kd) * scale + torch.from_numpy(bias)
    lse64 = torch.logsumexp(s, dim=-1)
    got = lse.cpu().double()
    fin = torch.isfinite(lse64)
    assert torch.equal(torch.isneginf(got), ~fin), f"seed {seed}: lse -inf pattern"
    tol = 5e-3 if dtype != torch.float32 else 1e-4
    assert torch.allclose(got[fin], lse64[fin], atol=tol, rtol=1e-4), f"seed {seed}: lse"
