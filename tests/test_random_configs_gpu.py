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


def make_shape_case(seed):
    """Larger random shapes (up to 1300 rows / 1400 keys) with the tile shape
    forced at random among those built for the call: the 256-row, 128-key
    workgroups at head_dim 128 without a mask, the key splits at head_dim 64
    (small-grid and per-item), or the planner's choice; a third of the cases
    also run the backward."""
    r = random.Random(10_000 + seed)
    dtype = r.choice([torch.bfloat16, torch.float16])
    D = r.choice([64, 64, 128, 128, 96, 256])
    Hkv = r.choice([1, 2, 4])
    H = Hkv * r.choice([1, 2, 4])
    B = r.choice([1, 2])
    Sq = r.choice([r.randint(17, 600), r.randint(600, 1300), 256, 512, 129])
    Sk = Sq if r.random() < 0.6 else r.randint(1, 1400)
    kw = {}
    if r.random() < 0.5:
        kw["causal"] = True
    if r.random() < 0.3:
        kw["window_size"] = (r.randint(0, 300), r.randint(0, 300))
    if r.random() < 0.3:
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    if r.random() < 0.25:
        g = torch.Generator().manual_seed(seed)
        m = torch.randn(Sq, Sk, generator=g)
        m[torch.rand(Sq, Sk, generator=g) < 0.2] = float("-inf")
        m[:, 0] = 0.0
        kw["attn_mask"] = m
    if r.random() < 0.15:
        kw["softmax_scale"] = r.uniform(0.02, 0.3)
    cfg = None
    if D == 128 and "attn_mask" not in kw and r.random() < 0.5:
        cfg = "8,2,128,1"
    elif D == 64 and r.random() < 0.6:
        cfg = r.choice(["4,2,64,2", "4,2,64,0", "4,2,64,1"])
    grad = r.random() < 0.3 and D in (64, 128)
    return dict(B=B, Sq=Sq, Sk=Sk, H=H, Hkv=Hkv, D=D, dtype=dtype, kw=kw, cfg=cfg, grad=grad)


# 112, 301, 311, 332: windows that leave rows with no allowed key, with grad
@pytest.mark.parametrize("seed", list(range(40)) + [112, 301, 311, 332])
def test_random_shape_and_tile_config(seed, monkeypatch):
    """Output against the oracle (and, with ``grad``, q/k/v gradients against
    fp64 autograd of the oracle at the backward bar) for make_shape_case.
    Rows with no allowed key give NaN in the forward as in eager; eager
    autograd then turns the whole (batch, head)'s gradients into NaN, while
    the HIP backward gives such rows zero gradient: there the gradients must
    be finite and the rows' dq zero, and the other (batch, head) slices
    meet the bar."""
    c = make_shape_case(seed)
    print(f"seed {seed}: {dict((k, v) for k, v in c.items() if k != 'kw')} {sorted(c['kw'])}", flush=True)
    B, Sq, Sk, H, Hkv, D, dtype, kw = c["B"], c["Sq"], c["Sk"], c["H"], c["Hkv"], c["D"], c["dtype"], c["kw"]
    if c["cfg"]:
        monkeypatch.setenv("TRINIX_ATTN_CFG", c["cfg"])
    q, k, v = rand((B, Sq, H, D), dtype, 3 * seed), rand((B, Sk, Hkv, D), dtype, 3 * seed + 1), \
        rand((B, Sk, Hkv, D), dtype, 3 * seed + 2)
    dev_kw = {a: (b.to(DEV) if torch.is_tensor(b) else b) for a, b in kw.items()}
    ts = [t.detach().clone().requires_grad_(c["grad"]) for t in (q, k, v)]
    out = triton_attn_func(*ts, **dev_kw)
    ref = oracle_on(q, k, v, **kw)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), **kw)
    assert_parity_or_more_accurate(out.detach(), ref, x64, dtype, f"seed {seed}")
    if not c["grad"]:
        return
    do = rand((B, Sq, H, D), dtype, 7 * seed)
    out.backward(do)
    hip = [t.grad.cpu().double() for t in ts]

    def eager(dt):
        xs = [t.detach().cpu().to(dt).clone().requires_grad_(True) for t in (q, k, v)]
        orc.functional_attention(*xs, **kw).backward(do.cpu().to(dt))
        return [x.grad.double() for x in xs]

    truth, eag = eager(torch.float64), eager(dtype)
    dead = torch.isnan(torch.as_tensor(x64)).any(-1)  # (B, Sq, H): rows with no allowed key
    assert all(torch.isfinite(h).all() for h in hip), f"seed {seed}: non-finite gradient"
    assert int(torch.count_nonzero(hip[0][dead])) == 0, f"seed {seed}: dq of rows with no allowed key"
    bad_bh = dead.any(1)  # (B, H) slices whose eager gradients are NaN
    G = H // Hkv
    for b in range(B):
        for h in range(H):
            if bad_bh[b, h]:
                continue
            hk = h // G
            kv_ok = not bool(bad_bh[b, hk * G:(hk + 1) * G].any())
            pairs = [(hip[0][b, :, h], eag[0][b, :, h], truth[0][b, :, h])]
            if kv_ok:
                pairs += [(hip[i][b, :, hk], eag[i][b, :, hk], truth[i][b, :, hk]) for i in (1, 2)]
            for hh, e, t in pairs:
                sc = t.abs().max().item()
                eh, ee = (hh - t).abs().max().item(), (e - t).abs().max().item()
                assert eh <= 2 * ee + 2e-3 * sc, (f"seed {seed} b{b} h{h}", eh, ee, sc)
