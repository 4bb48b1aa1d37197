"""GPU parity tests: the HIP attention path (through the C ABI) against the
CPU oracle (a restatement of the reference eager path) on identical seeded
inputs.

Tolerances (stated by the north star): bf16/fp16 outputs max abs <= 2e-2
and mean abs <= 2e-3; fp32 outputs ||out - ref||_inf / ||ref||_inf <= 1e-5.
The BASELINE workloads are checked at full size on every (batch, head) and
every query row (C4 in row bands with the keys their window can see), plus
size-independent properties (GQA == repeated KV bit for bit, stride-0 MQA ==
materialised KV).
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func
from trinix_amd import _native
from trinix_amd.kernels import TritonAttentionKernel, rope_apply
from trinix_amd.workloads import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


def assert_parity(out, ref, dtype, what=""):
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert out.shape == ref.shape, (what, out.shape, ref.shape)
    nan_o, nan_r = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_o, nan_r), f"{what}: NaN pattern differs ({int(nan_o.sum())} vs {int(nan_r.sum())})"
    ok = ~nan_r
    if not ok.any():
        return
    d = (out - ref)[ok].abs()
    if dtype == torch.float32:
        rel = (d.max() / ref[ok].abs().max().clamp_min(1e-30)).item()
        assert rel <= 1e-5, f"{what}: fp32 rel err {rel:.3g} > 1e-5"
    else:
        mx, mean = d.max().item(), d.mean().item()
        assert mx <= 2e-2 and mean <= 2e-3, f"{what}: max abs {mx:.4g} (<=2e-2), mean abs {mean:.4g} (<=2e-3)"


def assert_parity_or_more_accurate(out, ref, x64, dtype, what=""):
    """Parity with the eager oracle.  Where the oracle's own rounding of the
    biased scores to the input dtype (reference base.py:392 adds the fp32
    mask/ALiBi bias in place into bf16/fp16 scores) already costs more than
    half of the max-abs budget against the fp64 closed form, the kernel, which
    adds biases in fp32, must instead meet the budget against the fp64 closed
    form and be at least as accurate as the oracle."""
    x64 = torch.as_tensor(x64).float()
    ok = ~torch.isnan(x64)
    o_err = (ref.float().cpu() - x64)[ok].abs().max().item()
    if dtype != torch.float32 and o_err > 1e-2:
        assert_parity(out, x64, dtype, what + " (vs fp64)")
        k_err = (out.float().cpu() - x64)[ok].abs().max().item()
        assert k_err <= o_err, f"{what}: kernel err {k_err:.4g} > oracle err {o_err:.4g} vs fp64"
    else:
        assert_parity(out, ref, dtype, what)


def rand(shape, dtype, seed, device=DEV):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(device)


def oracle_on(q, k, v, **kw):
    return orc.functional_attention(q.cpu(), k.cpu(), v.cpu(), **kw)


def assert_parity_full(out, ref, dtype, what, q, k, v, row0=0, **kw):
    """Parity of a full-size output with the oracle, element by element.

    The mean abs error must meet the bar against the oracle.  An element
    further than the max-abs bar from the oracle passes only where the
    oracle's own bf16/fp16 arithmetic is more than half the bar away from
    the fp64 closed form (evaluated for those rows) and the kernel is within
    the bar of it: at |out| >= 2 one bf16 ulp is 0.0156, so two independent
    roundings can differ by more than 2e-2 while both are close to the
    truth.  ``q, k, v`` and ``kw`` are the oracle's inputs (CPU, all rows);
    ``out`` / ``ref`` row r is query position ``row0 + r``."""
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert out.shape == ref.shape, (what, out.shape, ref.shape)
    nan_o, nan_r = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_o, nan_r), f"{what}: NaN pattern differs"
    ok = ~nan_r
    d = (out - ref).abs().masked_fill(~ok, 0.0)
    mean = d[ok].mean().item()
    assert mean <= 2e-3, f"{what}: mean abs {mean:.4g} (<=2e-3)"
    bad = (d > 2e-2).nonzero().tolist()
    # the adjudication below is for isolated roundings, not a second bar: at
    # most one element in 10^7 (C3 had 1 of 268M) may need it
    limit = max(8, out.numel() // 10 ** 7)
    print(f"{what}: {len(bad)} element(s) beyond 2e-2 of the oracle (limit {limit})", flush=True)
    assert len(bad) <= limit, f"{what}: {len(bad)} elements beyond 2e-2 of the oracle (limit {limit})"
    rows = {}
    for b, i, h, _ in bad:
        rows.setdefault((b, h), set()).add(i)
    for (b, h), rs in rows.items():
        rs = sorted(rs)
        pos = [row0 + i for i in rs]
        sub_kw = dict(kw)
        if sub_kw.get("alibi_slopes") is not None:
            sub_kw["alibi_slopes"] = sub_kw["alibi_slopes"].reshape(-1, q.shape[2])[:, h:h + 1].reshape(-1)
        hk = h // (q.shape[2] // k.shape[2])
        x = torch.from_numpy(orc.closed_form(q[b:b + 1, pos][:, :, h:h + 1], k[b:b + 1, :, hk:hk + 1],
                                             v[b:b + 1, :, hk:hk + 1], row_pos=pos, **sub_kw))[0, :, 0]
        for r, i in enumerate(rs):
            for c in (d[b, i, h] > 2e-2).nonzero().flatten().tolist():
                o_err = abs(ref[b, i, h, c].item() - x[r, c].item())
                k_err = abs(out[b, i, h, c].item() - x[r, c].item())
                assert o_err > 1e-2 and k_err <= 2e-2, \
                    f"{what}: b{b} i{row0 + i} h{h} d{c}: kernel {out[b, i, h, c].item():.5f} oracle {ref[b, i, h, c].item():.5f} " \
                    f"fp64 {x[r, c].item():.5f}"


# ---------------------------------------------------------------------------
# BASELINE workloads
# ---------------------------------------------------------------------------
def test_library_loaded_and_device():
    assert TritonAttentionKernel.is_available()
    assert _native.library_loaded()


def test_c1_fp32_mha():
    w = WORKLOADS["c1"]
    inp = make_inputs(w)
    out = triton_attn_func(inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV))
    ref = orc.functional_attention(inp.q, inp.k, inp.v)
    assert out.dtype == torch.float32 and out.shape == inp.q.shape
    assert_parity(out, ref, torch.float32, "c1")


def test_c2_bf16_causal_mha():
    w = WORKLOADS["c2"]
    inp = make_inputs(w)
    out = triton_attn_func(inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV), causal=True)
    ref = orc.functional_attention(inp.q, inp.k, inp.v, causal=True)
    assert_parity(out, ref, torch.bfloat16, "c2")


def test_c3_gqa_rope_causal_every_head_every_row():
    """C3 at full size against the oracle on every (batch, head) and every
    query row (a row or work item the kernel never wrote would hold
    leftover memory and fail)."""
    w = WORKLOADS["c3"]
    inp = make_inputs(w)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    out = triton_attn_func(q, k, v, causal=True, rotary_cos=inp.cos.to(DEV), rotary_sin=inp.sin.to(DEV)).cpu()
    qr = orc.apply_rope(inp.q, inp.cos, inp.sin)
    kr = orc.apply_rope(inp.k, inp.cos, inp.sin)
    ref = orc.functional_attention(qr, kr, inp.v, causal=True, head_chunk=4)
    assert_parity_full(out, ref, torch.bfloat16, "c3 all heads, all rows", qr, kr, inp.v, causal=True)
    for r0 in (0, 4096, 8064):  # first, middle and last row block, reported on their own
        assert_parity_full(out[:, r0:r0 + 128], ref[:, r0:r0 + 128], torch.bfloat16, f"c3 rows {r0}..{r0 + 127}",
                           qr, kr, inp.v, row0=r0, causal=True)


def test_c4_sliding_window_every_head_every_row():
    """C4 at full size against the oracle on every (batch, head) and every
    query row, in 512-row bands whose key range [r0 - 4096, r0 + 512) holds
    every key the causal window (4096, 0) lets them see."""
    w = WORKLOADS["c4"]
    inp = make_inputs(w)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    out = triton_attn_func(q, k, v, causal=True, window_size=w.window, rotary_cos=inp.cos.to(DEV),
                           rotary_sin=inp.sin.to(DEV)).cpu()
    qr = orc.apply_rope(inp.q, inp.cos, inp.sin)
    kr = orc.apply_rope(inp.k, inp.cos, inp.sin)
    S, wl = w.seqlen, w.window[0]
    band = 512
    for r0 in range(0, S, band):
        keys = (max(0, r0 - wl), r0 + band)
        ref = orc.functional_attention(qr, kr, inp.v, causal=True, window_size=w.window, rows=(r0, r0 + band),
                                       keys=keys, head_chunk=8)
        assert_parity_full(out[:, r0:r0 + band], ref, torch.bfloat16, f"c4 rows {r0}..{r0 + band - 1}",
                           qr, kr, inp.v, row0=r0, causal=True, window_size=w.window)


@pytest.mark.parametrize("name", ["c5a", "c5b"])
def test_c5_alibi_block_mask_every_head_every_row(name):
    """C5a (MHA) / C5b (MQA, stride-0 KV) at full size against the oracle
    on every (batch, head) and every row."""
    w = WORKLOADS[name]
    inp = make_inputs(w)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    if w.nheads_kv == 1:
        # MQA as the reference layer feeds it: one KV head expanded (stride 0)
        k = k.expand(-1, -1, w.nheads, -1)
        v = v.expand(-1, -1, w.nheads, -1)
        assert k.stride(2) == 0
    out = triton_attn_func(q, k, v, attn_mask=inp.mask.to(DEV), alibi_slopes=inp.alibi.to(DEV)).cpu()
    ref = orc.functional_attention(inp.q, inp.k, inp.v, attn_mask=inp.mask, alibi_slopes=inp.alibi, head_chunk=8)
    assert_parity_full(out, ref, torch.float16, name + " all heads, all rows", inp.q, inp.k, inp.v,
                       attn_mask=inp.mask, alibi_slopes=inp.alibi)


def test_gqa_equals_repeated_kv_bitwise():
    """C3-sized: GQA kernel on 8 KV heads == kernel on KV repeated to 32 heads."""
    w = WORKLOADS["c3"]
    inp = make_inputs(w)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    out_g = triton_attn_func(q, k, v, causal=True)
    kr = torch.repeat_interleave(k, 4, dim=2)
    vr = torch.repeat_interleave(v, 4, dim=2)
    out_r = triton_attn_func(q, kr, vr, causal=True)
    assert torch.equal(out_g, out_r)


LONG_CASES = [
    # (S, H, Hkv, D, dtype, causal, window): one sequence, S query rows and keys
    (65536, 2, 1, 128, torch.bfloat16, True, None),        # 1024 key tiles in the last rows' chain
    (131072, 1, 1, 64, torch.float16, True, (8192, 0)),    # 2^17 rows, a window of 8192 keys
    (98304, 4, 4, 128, torch.bfloat16, False, (1000, 300)),  # two-sided window, K/V rows of 1 KiB
]


@pytest.mark.parametrize("case", LONG_CASES, ids=[f"S{c[0]}-D{c[3]}" for c in LONG_CASES])
def test_long_context_row_bands(case):
    """Sequences of 64K-128K positions: output and lse against the oracle on
    the first, a middle and the last 64-row band (their key ranges hold
    every key the causal / window band lets them see), so the 64-bit tile
    base addresses, the longest causal chains and the window arithmetic are
    exercised at lengths no BASELINE workload reaches."""
    S, H, Hkv, D, dtype, causal, window = case
    q, k, v = rand((1, S, H, D), dtype, 131), rand((1, S, Hkv, D), dtype, 132), rand((1, S, Hkv, D), dtype, 133)
    out, lse = TritonAttentionKernel.apply(q, k, v, causal=causal, window_size=window, return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    band = 64
    for r0 in (0, S // 2 - 37, S - band):
        lo = 0 if window is None else max(0, r0 - window[0])
        hi = r0 + band if causal else (S if window is None else min(S, r0 + band + window[1]))
        ref = orc.functional_attention(qc, kc, vc, causal=causal, window_size=window, rows=(r0, r0 + band),
                                       keys=(lo, hi), head_chunk=H)
        assert_parity(out[:, r0:r0 + band], ref, dtype, f"S={S} rows {r0}..{r0 + band - 1}")
        # lse of the band in fp64 from the same rows and keys
        qs = qc[0, r0:r0 + band].double().transpose(0, 1)                      # (H, band, D)
        ks = kc[0, lo:hi].double().repeat_interleave(H // Hkv, dim=1).transpose(0, 1)  # (H, keys, D)
        s = qs @ ks.transpose(1, 2) * D ** -0.5
        i = torch.arange(r0, r0 + band)[:, None]
        j = torch.arange(lo, hi)[None, :]
        allowed = torch.ones_like(s[0], dtype=torch.bool)
        if causal:
            allowed &= j <= i
        if window is not None:
            allowed &= (j - i >= -window[0]) & (j - i <= window[1])
        s = s.masked_fill(~allowed, float("-inf"))
        ref_lse = torch.logsumexp(s, dim=-1)
        d = (lse[0, :, r0:r0 + band].double() - ref_lse).abs().max().item()
        assert d <= 2e-2, f"S={S} rows {r0}..: lse err {d:.3g}"


def test_mqa_stride0_equals_materialised_bitwise():
    w = WORKLOADS["c5b"]
    inp = make_inputs(w)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    m, sl = inp.mask.to(DEV), inp.alibi.to(DEV)
    a = triton_attn_func(q, k, v, attn_mask=m, alibi_slopes=sl)
    b = triton_attn_func(q, k.expand(-1, -1, w.nheads, -1), v.expand(-1, -1, w.nheads, -1), attn_mask=m,
                         alibi_slopes=sl)
    c = triton_attn_func(q, k.expand(-1, -1, w.nheads, -1).contiguous(), v.expand(-1, -1, w.nheads, -1).contiguous(),
                         attn_mask=m, alibi_slopes=sl)
    assert torch.equal(a, b) and torch.equal(a, c)


def test_blockmap_is_exact_and_skipping_matches_full_read():
    w = WORKLOADS["c5a"]
    inp = make_inputs(w)
    m4 = TritonAttentionKernel._prepare_mask(inp.mask.to(DEV), w.batch, w.nheads, w.seqlen)
    bmap, _ = TritonAttentionKernel.mask_blockmap(m4)
    mc = inp.mask.view(w.seqlen // 32, 32, w.seqlen // 64, 64).permute(0, 2, 1, 3).reshape(w.seqlen // 32, w.seqlen // 64, -1)
    want = torch.ones(mc.shape[:2], dtype=torch.uint8)
    want[(mc == 0).all(-1)] = 0
    want[torch.isneginf(mc).all(-1)] = 2
    assert torch.equal(bmap.cpu()[0, 0], want)
    q, k, v = inp.q.to(DEV), inp.k.to(DEV), inp.v.to(DEV)
    a = TritonAttentionKernel.apply(q, k, v, attn_mask=inp.mask.to(DEV), use_blockmap=True)
    b = TritonAttentionKernel.apply(q, k, v, attn_mask=inp.mask.to(DEV), use_blockmap=False)
    # At head_dim 64 the all-zero blocks run the plain softmax (the scale folded
    # into the exp's FMA) and the per-element read the generic one (scale, add,
    # subtract): equal up to the last bit of the fp16 output.
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    d = (a.float() - b.float()).abs()
    assert d.max().item() <= 4e-3 and d.mean().item() <= 1e-5, (d.max().item(), d.mean().item())
    # At head_dim 128 both run one softmax body: skipping is bit-exact.
    q2, k2, v2 = (torch.cat([t, t], dim=-1)[:1, :1024].contiguous() for t in (q, k, v))
    m2 = inp.mask[:1024, :1024].to(DEV)
    a2 = TritonAttentionKernel.apply(q2, k2, v2, attn_mask=m2, use_blockmap=True)
    b2 = TritonAttentionKernel.apply(q2, k2, v2, attn_mask=m2, use_blockmap=False)
    assert torch.equal(a2, b2)


@pytest.mark.parametrize("causal", [False, True])
def test_blockmap_longer_than_64_columns(causal):
    """Sk = 5000 keys = 79 block-map columns: the kernel fetches the codes of
    one 32-row block 64 columns at a time, so a second fetch is exercised;
    checked against the oracle on a row subset and against the per-element
    mask read on the full problem."""
    B, S, H, D = 1, 5000, 2, 64
    q, k, v = rand((B, S, H, D), torch.float16, 81), rand((B, S, H, D), torch.float16, 82), rand((B, S, H, D), torch.float16, 83)
    nb = -(-S // 64)
    g = torch.Generator().manual_seed(84)
    grid = torch.rand((nb, nb), generator=g) < 0.3
    grid[:, 0] = False  # every row keeps its first block (allowed under causal)
    full = grid.repeat_interleave(64, 0).repeat_interleave(64, 1)[:S, :S]
    m = torch.zeros((S, S))
    m[full] = float("-inf")
    md = m.to(DEV)
    a = TritonAttentionKernel.apply(q, k, v, attn_mask=md, causal=causal, use_blockmap=True)
    b = TritonAttentionKernel.apply(q, k, v, attn_mask=md, causal=causal, use_blockmap=False)
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    assert (a.float() - b.float()).abs().max().item() <= 4e-3
    # Rows r0.. against the oracle; those rows see key tiles past column 64.
    # The oracle runs on the row slice alone, so the causal bound j <= i of
    # the full problem is written into the mask.
    r0 = 4096
    mr = m[r0:].clone()
    if causal:
        mr[torch.arange(S)[None, :] > torch.arange(r0, S)[:, None]] = float("-inf")
    ref = orc.functional_attention(q.cpu()[:, r0:], k.cpu(), v.cpu(), attn_mask=mr)
    assert_parity(a[:, r0:], ref, torch.float16, f"long block map causal={causal}")


@pytest.mark.parametrize("dtype,D", [(torch.float16, 64), (torch.bfloat16, 128)])
@pytest.mark.parametrize("scale", [None, 0.0, -0.07, 0.5])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("bias", ["alibi", "none", "mask"])
def test_scales_and_biases(dtype, D, scale, causal, bias):
    """Scores stay in the raw domain with the scale folded into the exp's FMA
    (c > 0): a negative scale negates the q operand, a zero scale zeroes it;
    ALiBi rides in the score accumulator as bias / c and the mask is added as
    mask * log2e / c.  Output and log-sum-exp against fp64."""
    B, S, H = 1, 300, 4
    q, k, v = rand((B, S, H, D), dtype, 91), rand((B, S, H, D), dtype, 92), rand((B, S, H, D), dtype, 93)
    kw = dict(causal=causal, softmax_scale=scale)
    slopes = orc.alibi_slopes(H)
    m = None
    if bias == "alibi":
        kw["alibi_slopes"] = slopes
    if bias == "mask":
        g = torch.Generator().manual_seed(94)
        m = torch.randn((S, S), generator=g) * 3
        m[torch.rand((S, S), generator=g) < 0.2] = float("-inf")
        m[:, 0] = 0
        kw["attn_mask"] = m
    out, lse = triton_attn_func(q, k, v, return_lse=True, **{a: (b.to(DEV) if torch.is_tensor(b) else b) for a, b in kw.items()})
    ref = oracle_on(q, k, v, **kw)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), **kw)
    assert_parity_or_more_accurate(out, ref, x64, dtype, f"{bias} scale={scale} causal={causal}")
    sc = D ** -0.5 if scale is None else scale
    s = torch.einsum("bihd,bjhd->bhij", q.cpu().double(), k.cpu().double()) * sc
    if bias == "alibi":
        ij = (torch.arange(S)[:, None] - torch.arange(S)[None, :]).abs().double()
        s = s - slopes.double()[None, :, None, None] * ij
    if bias == "mask":
        s = s + m.double()
    if causal:
        s.masked_fill_(torch.triu(torch.ones(S, S), 1).bool(), float("-inf"))
    want = torch.logsumexp(s, dim=-1)
    # the row sum adds P rounded to the input dtype (as the PV product uses
    # it): at most one rounding of relative size 2^-8 (bf16) / 2^-11 (fp16)
    atol = 8e-3 if dtype == torch.bfloat16 else 2e-3
    assert torch.allclose(lse.cpu().double(), want, atol=atol, rtol=1e-4)


# ---------------------------------------------------------------------------
# edge cases against the oracle (small shapes)
# ---------------------------------------------------------------------------
CASES = [
    # (B, Sq, Sk, H, Hkv, D, causal, window)
    (1, 1, 1, 1, 1, 64, False, None),
    (2, 100, 100, 3, 3, 64, True, None),
    (1, 257, 257, 2, 1, 128, True, None),
    (1, 130, 130, 4, 2, 128, False, (16, 4)),
    (2, 200, 200, 2, 2, 64, True, (0, 0)),
    (1, 300, 300, 2, 2, 64, True, (37, 0)),
    (1, 70, 190, 2, 2, 64, False, None),
    (1, 190, 70, 2, 2, 128, True, None),
    (1, 1, 300, 4, 1, 128, False, None),
    (1, 96, 96, 2, 2, 32, True, None),
    (1, 96, 96, 2, 2, 80, False, None),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", CASES)
def test_edge_shapes(case, dtype):
    B, Sq, Sk, H, Hkv, D, causal, window = case
    q = rand((B, Sq, H, D), dtype, 11)
    k = rand((B, Sk, Hkv, D), dtype, 12)
    v = rand((B, Sk, Hkv, D), dtype, 13)
    out = triton_attn_func(q, k, v, causal=causal, window_size=window)
    ref = oracle_on(q, k, v, causal=causal, window_size=window)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), causal=causal, window_size=window)
    assert_parity_or_more_accurate(out, ref, x64, dtype, str(case))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mask_kind", ["2d", "3d", "4d_h1", "4d", "bool2d", "bf16_2d"])
def test_masks_and_alibi(mask_kind, dtype):
    B, S, H, D = 2, 160, 4, 64
    q, k, v = rand((B, S, H, D), dtype, 21), rand((B, S, H, D), dtype, 22), rand((B, S, H, D), dtype, 23)
    g = torch.Generator().manual_seed(24)
    if mask_kind == "2d":
        m = torch.randn((S, S), generator=g)
        m[torch.rand((S, S), generator=g) < 0.2] = float("-inf")
    elif mask_kind == "3d":
        m = torch.randn((B, S, S), generator=g)
    elif mask_kind == "4d_h1":
        m = torch.randn((B, 1, S, S), generator=g)
    elif mask_kind == "4d":
        m = torch.randn((B, H, S, S), generator=g)
    elif mask_kind == "bool2d":
        m = torch.rand((S, S), generator=g) < 0.5
    else:
        m = torch.randn((S, S), generator=g).to(torch.bfloat16)
    slopes = orc.alibi_slopes(H)
    if m.dtype != torch.bool:
        m[..., :, 0] = 0  # every row keeps key 0 (allowed under causal)
    out = triton_attn_func(q, k, v, attn_mask=m.to(DEV), alibi_slopes=slopes.to(DEV), causal=True)
    mref = m.to(torch.uint8) if m.dtype == torch.bool else m
    ref = oracle_on(q, k, v, attn_mask=mref.float(), alibi_slopes=slopes, causal=True)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), attn_mask=mref.float(), alibi_slopes=slopes, causal=True)
    assert_parity_or_more_accurate(out, ref, x64, dtype, mask_kind)


def test_leading_tiles_fully_masked_are_exact():
    """Rows whose first key tiles are all -inf (the reference Triton kernel
    returns NaN there) match the eager path."""
    B, S, H, D = 1, 512, 2, 64
    q, k, v = rand((B, S, H, D), torch.bfloat16, 31), rand((B, S, H, D), torch.bfloat16, 32), rand((B, S, H, D), torch.bfloat16, 33)
    m = torch.zeros(S, S)
    m[:, :200] = float("-inf")
    out = triton_attn_func(q, k, v, attn_mask=m.to(DEV))
    ref = oracle_on(q, k, v, attn_mask=m)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), attn_mask=m)
    assert_parity_or_more_accurate(out, ref, x64, torch.bfloat16, "leading masked")
    out2 = triton_attn_func(q, k, v, causal=True, window_size=(64, 0))
    ref2 = oracle_on(q, k, v, causal=True, window_size=(64, 0))
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), causal=True, window_size=(64, 0))
    assert_parity_or_more_accurate(out2, ref2, x64, torch.bfloat16, "window")


def test_fully_masked_rows_give_nan_like_eager():
    B, S, H, D = 1, 96, 1, 64
    q, k, v = rand((B, S, H, D), torch.float16, 41), rand((B, S, H, D), torch.float16, 42), rand((B, S, H, D), torch.float16, 43)
    m = torch.zeros(S, S)
    m[5] = float("-inf")
    m[70] = float("-inf")
    out = triton_attn_func(q, k, v, attn_mask=m.to(DEV))
    ref = oracle_on(q, k, v, attn_mask=m)
    assert torch.isnan(ref[0, 5]).all() and torch.isnan(ref[0, 70]).all()
    assert_parity(out, ref, torch.float16, "nan rows")


@pytest.mark.parametrize("D,dtype", [(64, torch.float16), (128, torch.bfloat16)])
def test_window_bounds_beyond_the_sequence_are_exact(D, dtype):
    """Window bounds of any size select the keys they name: (2^40, 0) with
    causal is causal, (5, 2^62) is (5, Sk), and a bound of -2^40 (no key
    within reach) gives the NaN rows of an empty softmax, in the forward and
    the backward.  (Bounds are clamped to +-2^30 ahead of the kernels'
    32-bit index arithmetic; |j - i| < 2^30 for every accepted shape.)"""
    B, S, H, HKV = 1, 200, 4, 2
    q, k, v = rand((B, S, H, D), dtype, 61), rand((B, S, HKV, D), dtype, 62), rand((B, S, HKV, D), dtype, 63)
    big = 1 << 40
    assert torch.equal(triton_attn_func(q, k, v, causal=True, window_size=(big, 0)),
                       triton_attn_func(q, k, v, causal=True))
    assert torch.equal(triton_attn_func(q, k, v, window_size=(5, 1 << 62)),
                       triton_attn_func(q, k, v, window_size=(5, S)))
    assert torch.equal(triton_attn_func(q, k, v, window_size=(S, 1 << 62)),
                       triton_attn_func(q, k, v, window_size=(1 << 62, S)))
    out = triton_attn_func(q, k, v, window_size=(-big, big))  # needs j - i >= 2^40: no key
    assert torch.isnan(out).all()
    # the backward takes the same band: gradients equal those of the small bounds
    grads = []
    for ws in ((big, 3), (S, 3)):
        ts = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
        triton_attn_func(*ts, causal=True, window_size=ws).backward(torch.ones_like(q))
        grads.append([t.grad for t in ts])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_single_open_column_returns_that_value_row():
    B, S, H, D = 1, 128, 2, 128
    q, k, v = rand((B, S, H, D), torch.bfloat16, 51), rand((B, S, H, D), torch.bfloat16, 52), rand((B, S, H, D), torch.bfloat16, 53)
    m = torch.full((S, S), float("-inf"))
    m[:, 77] = 0
    out = triton_attn_func(q, k, v, attn_mask=m.to(DEV))
    assert torch.equal(out.cpu(), v[:, 77:78].expand(-1, S, -1, -1).cpu())


def test_noncontiguous_qkv_from_packed_projection():
    B, S, H, D = 2, 150, 4, 64
    qkv = rand((B, S, 3, H, D), torch.bfloat16, 61)
    q, k, v = qkv.unbind(dim=2)
    assert not q.is_contiguous()
    out = triton_attn_func(q, k, v, causal=True)
    ref = oracle_on(q.contiguous(), k.contiguous(), v.contiguous(), causal=True)
    assert_parity(out, ref, torch.bfloat16, "packed qkv")


def test_lse_output():
    B, S, H, D = 1, 200, 2, 64
    q, k, v = rand((B, S, H, D), torch.float32, 71), rand((B, S, H, D), torch.float32, 72), rand((B, S, H, D), torch.float32, 73)
    out, lse = triton_attn_func(q, k, v, causal=True, return_lse=True)
    s = torch.einsum("bihd,bjhd->bhij", q.cpu().double(), k.cpu().double()) * D ** -0.5
    s.masked_fill_(torch.triu(torch.ones(S, S), 1).bool(), float("-inf"))
    ref = torch.logsumexp(s, dim=-1)
    assert torch.allclose(lse.cpu().double(), ref, atol=1e-4, rtol=1e-5)


LSE16_CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, kwargs): short causal rows (few keys, so
    # the rounding of P is not averaged out), long rows, ALiBi with a window,
    # head_dim 256, and a split-KV decode call (which sums fp32 P)
    (1, 200, 200, 4, 2, 64, torch.bfloat16, dict(causal=True)),
    (2, 130, 700, 2, 2, 128, torch.float16, dict()),
    (1, 256, 256, 4, 4, 128, torch.bfloat16, dict(alibi_slopes=orc.alibi_slopes(4), window_size=(40, 10))),
    (1, 96, 96, 2, 1, 256, torch.float16, dict(causal=True, softmax_scale=0.3)),
    (2, 4, 3000, 8, 2, 128, torch.bfloat16, dict()),
]


@pytest.mark.parametrize("case", range(len(LSE16_CASES)))
def test_lse_output_16bit_within_one_unit_roundoff(case):
    """bf16/fp16 lse against the fp64 log-sum-exp of the same rounded inputs:
    within the dtype's unit roundoff (the 16-bit kernels sum P as rounded for
    the P @ V product) plus fp32 slack.  A log2 lse, a missing log of the row
    sum or a dropped bias is off by far more."""
    B, Sq, Sk, H, Hkv, D, dtype, kw = LSE16_CASES[case]
    q, k, v = rand((B, Sq, H, D), dtype, 90 + case), rand((B, Sk, Hkv, D), dtype, 95 + case), rand((B, Sk, Hkv, D), dtype, 99)
    dkw = {key: (val.to(DEV) if torch.is_tensor(val) else val) for key, val in kw.items()}
    _, lse = triton_attn_func(q, k, v, return_lse=True, **dkw)
    assert lse.shape == (B, H, Sq) and lse.dtype == torch.float32
    q64 = q.cpu().double()
    k64 = k.cpu().double().repeat_interleave(H // Hkv, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", q64, k64) * kw.get("softmax_scale", D ** -0.5)
    s = s + torch.from_numpy(orc._bias64(Sq, Sk, H, B, None, kw.get("causal", False), kw.get("window_size"),
                                         kw.get("alibi_slopes")))
    ref = torch.logsumexp(s, dim=-1)
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = (lse.cpu().double() - ref).abs().max().item()
    assert err <= u + 2e-5 * (1 + ref.abs().max().item()), (err, u)


@pytest.mark.parametrize("dtype,masked", [(torch.bfloat16, False), (torch.float16, True)])
def test_outputs_merged_by_lse_equal_one_call(dtype, masked):
    """Attention over keys [0, Sk) from the calls over [0, c) and [c, Sk)
    merged by their lse (what a chunked-prefill or ring caller does): as
    close to the fp64 closed form as the single call, and its lse the
    log-add-exp of the two."""
    B, Sq, Sk, H, D, c = 1, 160, 384, 4, 128, 150
    q, k, v = rand((B, Sq, H, D), dtype, 111), rand((B, Sk, H, D), dtype, 112), rand((B, Sk, H, D), dtype, 113)
    mask = None
    if masked:
        g = torch.Generator().manual_seed(114)
        mask = (torch.randn(Sq, Sk, generator=g) * 0.5).masked_fill(torch.rand(Sq, Sk, generator=g) < 0.1, float("-inf"))
        mask[:, 0] = mask[:, c] = 0.0
    part = lambda a, b: None if mask is None else mask[:, a:b].to(DEV)
    o, l = triton_attn_func(q, k, v, attn_mask=part(0, Sk), return_lse=True)
    o1, l1 = triton_attn_func(q, k[:, :c], v[:, :c], attn_mask=part(0, c), return_lse=True)
    o2, l2 = triton_attn_func(q, k[:, c:], v[:, c:], attn_mask=part(c, Sk), return_lse=True)
    l12 = torch.logaddexp(l1.double(), l2.double())
    w1 = torch.exp(l1.double() - l12).transpose(1, 2)[..., None]
    w2 = torch.exp(l2.double() - l12).transpose(1, 2)[..., None]
    merged = (w1 * o1.double() + w2 * o2.double()).cpu()
    x64 = torch.from_numpy(orc.closed_form(q.cpu(), k.cpu(), v.cpu(), attn_mask=mask))
    err_one = (o.cpu().double() - x64).abs().max().item()
    err_merged = (merged - x64).abs().max().item()
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    assert err_merged <= 2 * err_one + u * x64.abs().max().item(), (err_merged, err_one)
    assert (l12 - l.double()).abs().max().item() <= 2 * u + 1e-4


def test_runs_on_side_stream():
    B, S, H, D = 1, 256, 2, 128
    q, k, v = rand((B, S, H, D), torch.bfloat16, 81), rand((B, S, H, D), torch.bfloat16, 82), rand((B, S, H, D), torch.bfloat16, 83)
    ref = triton_attn_func(q, k, v, causal=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = triton_attn_func(q, k, v, causal=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


# ---------------------------------------------------------------------------
# RoPE (standalone kernel, bit-exact with the eager rounding sequence)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128, 6])
def test_rope_bit_exact(dtype, D):
    B, S, H = 2, 77, 3
    x = rand((B, S, H, D), dtype, 91)
    cos, sin = orc.rope_tables(S, D, 10000.0, dtype)
    out = rope_apply(x, cos.to(DEV), sin.to(DEV))
    ref = orc.apply_rope(x.cpu(), cos, sin)
    assert torch.equal(out.cpu(), ref)
    pos = torch.randint(0, S, (B, S), generator=torch.Generator().manual_seed(92))
    out2 = rope_apply(x, cos.to(DEV), sin.to(DEV), position_ids=pos.to(DEV))
    ref2 = orc.apply_rope(x.cpu(), cos, sin, position_ids=pos)
    assert torch.equal(out2.cpu(), ref2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_rope_matches_prerotated(dtype):
    B, S, H, Hkv, D = 1, 300, 4, 2, 128
    q, k, v = rand((B, S, H, D), dtype, 95), rand((B, S, Hkv, D), dtype, 96), rand((B, S, Hkv, D), dtype, 97)
    cos, sin = orc.rope_tables(S, D, 500000.0, dtype)
    fused = triton_attn_func(q, k, v, causal=True, rotary_cos=cos.to(DEV), rotary_sin=sin.to(DEV))
    qr = orc.apply_rope(q.cpu(), cos, sin).to(DEV)
    kr = orc.apply_rope(k.cpu(), cos, sin).to(DEV)
    pre = triton_attn_func(qr, kr, v, causal=True)
    assert torch.equal(fused, pre)


# ---------------------------------------------------------------------------
# dropout: exact against the oracle's Philox stream
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dropout_matches_philox_oracle(dtype):
    B, S, H, D, p = 1, 128, 2, 64, 0.3
    q, k, v = rand((B, S, H, D), dtype, 101), rand((B, S, H, D), dtype, 102), rand((B, S, H, D), dtype, 103)
    torch.manual_seed(1234)
    out = triton_attn_func(q, k, v, dropout_p=p, causal=True)
    torch.manual_seed(1234)
    seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    keep = torch.from_numpy(orc.dropout_keep(B, H, S, S, p, seed)).double()
    s = torch.einsum("bihd,bjhd->bhij", q.cpu().double(), k.cpu().double()) * D ** -0.5
    s.masked_fill_(torch.triu(torch.ones(S, S), 1).bool(), float("-inf"))
    P = torch.softmax(s, dim=-1) * keep / (1 - p)
    ref = torch.einsum("bhij,bjhd->bihd", P, v.cpu().double())
    tol = 1e-5 if dtype == torch.float32 else 3e-2
    assert (out.cpu().double() - ref).abs().max().item() <= tol
    frac = keep.mean().item()
    assert abs(frac - (1 - p)) < 0.02


KS_CASES = [
    # (B, Sq, Sk, H, Hkv, D, causal, window, features)
    (2, 1024, 1024, 3, 3, 64, True, None, ""),
    (1, 700, 700, 4, 2, 64, True, (200, 0), "alibi"),
    (2, 333, 333, 2, 1, 64, False, None, "mask"),
    (1, 257, 400, 2, 2, 64, False, (50, 70), "alibi,mask"),
    (1, 190, 190, 2, 2, 64, True, None, "lse"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", KS_CASES, ids=[str(c) for c in KS_CASES])
def test_key_split_configs(case, dtype, monkeypatch):
    """Head_dim 64 small grids split each 32-row group's keys between two
    wavefronts (ks = 2) and merge the halves through LDS; both tile configs
    are forced through TRINIX_ATTN_CFG and checked against the oracle, and
    against each other."""
    B, Sq, Sk, H, Hkv, D, causal, window, feats = case
    q, k, v = rand((B, Sq, H, D), dtype, 101), rand((B, Sk, Hkv, D), dtype, 102), rand((B, Sk, Hkv, D), dtype, 103)
    kw = dict(causal=causal, window_size=window)
    if "alibi" in feats:
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    if "mask" in feats:
        g = torch.Generator().manual_seed(104)
        m = torch.randn((Sq, Sk), generator=g)
        m[torch.rand((Sq, Sk), generator=g) < 0.2] = float("-inf")
        nb = -(-Sk // 64)
        blk = (torch.rand((-(-Sq // 64), nb), generator=g) < 0.3).repeat_interleave(64, 0).repeat_interleave(64, 1)
        m[blk[:Sq, :Sk]] = float("-inf")
        m[:, 0] = 0
        if window is not None:  # every row keeps its diagonal key, inside any window
            m[torch.arange(Sq), torch.arange(Sq).clamp(max=Sk - 1)] = 0
        kw["attn_mask"] = m
    outs = {}
    for ks in (1, 2):
        monkeypatch.setenv("TRINIX_ATTN_CFG", f"4,2,64,{ks}")
        dkw = {a: (b.to(DEV) if torch.is_tensor(b) else b) for a, b in kw.items()}
        out, lse = triton_attn_func(q, k, v, return_lse=True, **dkw)
        outs[ks] = (out, lse)
    monkeypatch.delenv("TRINIX_ATTN_CFG")
    ref = oracle_on(q, k, v, **kw)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), **kw)
    for ks in (1, 2):
        assert_parity_or_more_accurate(outs[ks][0], ref, x64, dtype, f"{case} ks={ks}")
    d = (outs[1][0].float() - outs[2][0].float()).abs()
    ok = ~torch.isnan(outs[1][0].float())
    assert torch.equal(torch.isnan(outs[1][0]), torch.isnan(outs[2][0]))
    assert d[ok].max().item() <= 2e-2
    l1, l2 = outs[1][1], outs[2][1]
    fin = torch.isfinite(l1)
    assert torch.equal(fin, torch.isfinite(l2))
    assert (l1[fin] - l2[fin]).abs().max().item() <= 1e-2


WIDE_CASES = [
    # (B, Sq, Sk, H, Hkv, causal, window, features), head_dim 128
    (1, 300, 300, 4, 2, True, None, ""),
    (2, 200, 333, 4, 4, False, None, "alibi"),
    (1, 520, 520, 2, 1, True, (100, 0), ""),
    (1, 64, 700, 2, 2, False, (50, 60), ""),
    (1, 257, 257, 4, 4, True, None, "rope,qn"),
    (1, 1000, 1000, 2, 2, True, None, "alibi,qn"),
    (1, 130, 600, 2, 1, True, None, "rope"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", WIDE_CASES, ids=[str(c) for c in WIDE_CASES])
def test_wide_tile_config(case, dtype, monkeypatch):
    """Head_dim 128 without a mask or dropout runs 256-row workgroups with
    128-key tiles once the grid is large (C3, C4).  Forced here through
    TRINIX_ATTN_CFG on small problems (partial tiles, Sq != Sk, windows,
    GQA/MQA, ALiBi, fused RoPE and q RMSNorm): output and lse against the
    oracle, and against the 128-row, 64-key shape."""
    B, Sq, Sk, H, Hkv, causal, window, feats = case
    D = 128
    q, k, v = rand((B, Sq, H, D), dtype, 111), rand((B, Sk, Hkv, D), dtype, 112), rand((B, Sk, Hkv, D), dtype, 113)
    kw = dict(causal=causal, window_size=window)
    if "alibi" in feats:
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    dkw = {a: (b.to(DEV) if torch.is_tensor(b) else b) for a, b in kw.items()}
    qr, kr, eps = q.cpu(), k.cpu(), 1e-5
    if "rope" in feats:
        cos, sin = orc.rope_tables(max(Sq, Sk), D, 10000.0, dtype)
        dkw.update(rotary_cos=cos.to(DEV), rotary_sin=sin.to(DEV))
        qr, kr = orc.apply_rope(qr, cos, sin), orc.apply_rope(kr, cos, sin)
    if "qn" in feats:
        w = (1.0 + 0.3 * torch.randn(D, generator=torch.Generator().manual_seed(114))).to(dtype)
        dkw.update(q_norm_weight=w.to(DEV), q_norm_eps=eps)
        qr = orc.qk_rms_norm(qr, w, eps)
    outs = {}
    for cfg in ("4,2,64,1", "8,2,128,1"):
        monkeypatch.setenv("TRINIX_ATTN_CFG", cfg)
        outs[cfg] = TritonAttentionKernel.apply(q, k, v, return_lse=True, **dkw)
    monkeypatch.delenv("TRINIX_ATTN_CFG")
    ref = oracle_on(qr, kr, v, **kw)
    x64 = orc.closed_form(qr, kr, v.cpu(), **kw)
    for cfg, (out, _) in outs.items():
        assert_parity_or_more_accurate(out, ref, x64, dtype, f"{case} {cfg}")
    (o1, l1), (o2, l2) = outs.values()
    ok = ~torch.isnan(o1.float())
    assert torch.equal(torch.isnan(o1), torch.isnan(o2))
    assert (o1.float() - o2.float()).abs()[ok].max().item() <= 2e-2
    fin = torch.isfinite(l1)
    assert torch.equal(fin, torch.isfinite(l2))
    assert (l1[fin] - l2[fin]).abs().max().item() <= 1e-2


SPLIT_CASES = [
    # (B, Sq, Sk, H, Hkv, features), head_dim 64, causal
    (2, 1024, 1024, 12, 12, ""),   # blocks 4..7 split into 64-row halves, 0..3 whole
    (1, 700, 700, 6, 3, "alibi"),
    (1, 1000, 1200, 4, 2, ""),     # Sq != Sk
    (1, 300, 300, 4, 4, ""),       # the last block partial
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", SPLIT_CASES, ids=[str(c) for c in SPLIT_CASES])
def test_split_rows_config(case, dtype, monkeypatch):
    """The per-item key split at head_dim 64 (C2's default: the longest
    causal row blocks run as two 64-row items with two wavefronts per 32-row
    group, the others whole), forced through TRINIX_ATTN_CFG: output and lse
    against the oracle and against the unsplit shape."""
    B, Sq, Sk, H, Hkv, feats = case
    D = 64
    q, k, v = rand((B, Sq, H, D), dtype, 121), rand((B, Sk, Hkv, D), dtype, 122), rand((B, Sk, Hkv, D), dtype, 123)
    kw = dict(causal=True)
    if "alibi" in feats:
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    dkw = {a: (b.to(DEV) if torch.is_tensor(b) else b) for a, b in kw.items()}
    outs = {}
    for cfg in ("4,2,64,1", "4,2,64,0"):
        monkeypatch.setenv("TRINIX_ATTN_CFG", cfg)
        outs[cfg] = TritonAttentionKernel.apply(q, k, v, return_lse=True, **dkw)
    monkeypatch.delenv("TRINIX_ATTN_CFG")
    ref = oracle_on(q, k, v, **kw)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), **kw)
    for cfg, (out, _) in outs.items():
        assert_parity_or_more_accurate(out, ref, x64, dtype, f"{case} {cfg}")
    (o1, l1), (o2, l2) = outs.values()
    assert (o1.float() - o2.float()).abs().max().item() <= 2e-2
    assert (l1 - l2).abs().max().item() <= 1e-2


def test_wide_tile_config_chosen_for_large_grids(monkeypatch):
    """The planner's choice: 256-row, 128-key workgroups at head_dim 128 for
    C3-sized grids without a mask or dropout; the 128-row shape for small
    causal grids, with a mask, and at head_dim 64 (checked through the
    forced-config error: a shape that is not built for a call is rejected)."""
    from trinix_amd.kernels import tile_config

    cfg = tile_config(128, torch.bfloat16)
    assert (cfg["block_m"], cfg["block_n"], cfg["waves"]) == (256, 128, 8)
    q = rand((1, 64, 2, 128), torch.bfloat16, 5)
    m = torch.zeros(64, 64, device=DEV)
    monkeypatch.setenv("TRINIX_ATTN_CFG", "8,2,128,1")
    with pytest.raises((ValueError, RuntimeError)):
        TritonAttentionKernel.apply(q, q, q, attn_mask=m)  # no mask kernels at this shape
    q64 = rand((1, 64, 2, 64), torch.bfloat16, 6)
    with pytest.raises((ValueError, RuntimeError)):
        TritonAttentionKernel.apply(q64, q64, q64)
