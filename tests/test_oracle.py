"""Pins the CPU oracle before it is trusted as the parity reference.

The reference ships no golden vectors, so each oracle function is checked
against something independent of its own formula: an fp64 closed form
(einsum), brute-force Python loops, special cases whose answer the
mathematics fixes, and published known-answer vectors (Philox).
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd.kernels.attention_kernel import allowed_pairs
from trinix_amd import workloads as wl


def r(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


FEATURES = [
    dict(),
    dict(causal=True),
    dict(window_size=(3, 1)),
    dict(causal=True, window_size=(2, 0)),
    dict(alibi=True),
    dict(mask=True),
    dict(causal=True, alibi=True, mask=True),
]


def _features(f, B, S, H, seed):
    kw = {}
    if f.get("causal"):
        kw["causal"] = True
    if "window_size" in f:
        kw["window_size"] = f["window_size"]
    if f.get("alibi"):
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    if f.get("mask"):
        m = r((B, S, S), seed)
        m[:, :, 0] = 0
        m[:, 1:, 1][r((B, S - 1), seed + 1) > 0.5] = float("-inf")
        kw["attn_mask"] = m
    return kw


@pytest.mark.parametrize("f", FEATURES)
@pytest.mark.parametrize("hkv", [4, 2, 1])
def test_eager_fp32_matches_fp64_closed_form(f, hkv):
    B, S, H, D = 2, 37, 4, 16
    q, k, v = r((B, S, H, D), 1), r((B, S, hkv, D), 2), r((B, S, hkv, D), 3)
    kw = _features(f, B, S, H, 4)
    out = orc.functional_attention(q, k, v, **kw)
    ref = orc.closed_form(q, k, v, **kw)
    assert np.allclose(out.double().numpy(), ref, atol=2e-6, rtol=1e-5, equal_nan=True)


@pytest.mark.parametrize("f", FEATURES)
def test_closed_form_matches_brute_force(f):
    B, S, H, D = 1, 6, 2, 3
    q, k, v = r((B, S, H, D), 5, torch.float64), r((B, S, 1, D), 6, torch.float64), r((B, S, 1, D), 7, torch.float64)
    kw = _features(f, B, S, H, 8)
    cf = orc.closed_form(q, k, v, **kw)
    bf = np.array(orc.brute_force(q, k, v, **kw))
    assert np.allclose(cf, bf, atol=1e-12, equal_nan=True)


def test_special_cases():
    B, S, H, D = 1, 9, 2, 8
    q, k, v = r((B, S, H, D), 10), r((B, S, H, D), 11), r((B, S, H, D), 12)
    # one key -> output is that value row
    o = orc.functional_attention(q[:, :1], k[:, :1], v[:, :1])
    assert torch.equal(o, v[:, :1])
    # causal row 0 sees only key 0
    o = orc.functional_attention(q, k, v, causal=True)
    assert torch.equal(o[:, 0], v[:, 0])
    # window (0, 0): each row sees only itself
    o = orc.functional_attention(q, k, v, window_size=(0, 0))
    assert torch.allclose(o, v, atol=0, rtol=0)
    # identical keys -> uniform weights -> mean of values
    ke = k[:, :1].expand(B, S, H, D).contiguous()
    o = orc.functional_attention(q, ke, v)
    assert torch.allclose(o, v.mean(dim=1, keepdim=True).expand_as(o), atol=1e-6)
    # zero scale -> prefix means under causal
    o = orc.functional_attention(q, k, v, softmax_scale=0.0, causal=True)
    pref = v.cumsum(dim=1) / torch.arange(1, S + 1).view(1, S, 1, 1)
    assert torch.allclose(o, pref, atol=1e-6)
    # a single open column c -> v[c] for every row
    m = torch.full((S, S), float("-inf"))
    m[:, 4] = 0
    o = orc.functional_attention(q, k, v, attn_mask=m)
    assert torch.equal(o, v[:, 4:5].expand_as(o))
    # zero ALiBi slopes == no ALiBi
    a = orc.functional_attention(q, k, v, alibi_slopes=torch.zeros(H))
    b = orc.functional_attention(q, k, v)
    assert torch.equal(a, b)
    # a row with no allowed key is NaN, as the eager softmax gives
    m = torch.zeros(S, S)
    m[3] = float("-inf")
    o = orc.functional_attention(q, k, v, attn_mask=m)
    assert torch.isnan(o[:, 3]).all() and not torch.isnan(o[:, 2]).any()


def test_gqa_tiling_is_head_div_group():
    B, S, H, D = 1, 5, 6, 4
    q, k, v = r((B, S, H, D), 20), r((B, S, 2, D), 21), r((B, S, 2, D), 22)
    a = orc.functional_attention(q, k, v)
    b = orc.functional_attention(q, torch.repeat_interleave(k, 3, dim=2), torch.repeat_interleave(v, 3, dim=2))
    assert torch.equal(a, b)
    t = orc.tile_kv_heads(k, 3)
    for h in range(H):
        assert torch.equal(t[:, :, h], k[:, :, h // 3])


def test_alibi_slopes_closed_form():
    for n in (1, 2, 4, 8, 16, 32):
        sl = orc.alibi_slopes(n)
        want = torch.tensor([2.0 ** (-8.0 * (i + 1) / n) for i in range(n)])
        assert torch.allclose(sl, want, rtol=1e-6)
    # non power of two: 8 slopes of n=8, then every other slope of n=16
    sl12 = orc.alibi_slopes(12).tolist()
    want12 = [2.0 ** -(i + 1) for i in range(8)] + [2.0 ** -(0.5 * (2 * i + 1)) for i in range(4)]
    assert np.allclose(sl12, want12, rtol=1e-6)
    assert torch.equal(orc.alibi_slopes(12), wl.alibi_slopes(12))
    b = orc.alibi_bias(3, 4, torch.tensor([0.5]))
    assert torch.equal(b[0], torch.tensor([[0, -0.5, -1, -1.5], [-0.5, 0, -0.5, -1], [-1, -0.5, 0, -0.5]]))


def test_rope_tables_and_rotation():
    S, D = 50, 16
    cos, sin = orc.rope_tables(S, D, 10000.0, torch.float32)
    assert torch.equal(cos[0], torch.ones(D)) and torch.equal(sin[0], torch.zeros(D))
    inv = 1.0 / 10000.0 ** (np.arange(0, D, 2) / D)
    ang = np.arange(S)[:, None] * inv[None, :]
    assert np.allclose(cos[:, : D // 2].numpy(), np.cos(ang), atol=2e-6 * S)
    assert np.allclose(sin[:, D // 2:].numpy(), np.sin(ang), atol=2e-6 * S)
    # rotation by angle a of each pair (x_d, x_{d+D/2}), in fp64
    x = r((1, S, 1, D), 30, torch.float64)
    c64, s64 = torch.from_numpy(np.cos(np.concatenate([ang, ang], 1))), torch.from_numpy(np.sin(np.concatenate([ang, ang], 1)))
    y = orc.apply_rope(x, c64, s64)
    x1, x2 = x[..., : D // 2], x[..., D // 2:]
    a = torch.from_numpy(ang)[None, :, None, :]
    assert torch.allclose(y[..., : D // 2], x1 * torch.cos(a) - x2 * torch.sin(a), atol=1e-12)
    assert torch.allclose(y[..., D // 2:], x2 * torch.cos(a) + x1 * torch.sin(a), atol=1e-12)
    # relative-position property: <rope(q, m), rope(k, n)> depends on m - n only
    qv, kv = r((1, 1, 1, D), 31, torch.float64), r((1, 1, 1, D), 32, torch.float64)
    qs, ks = qv.expand(1, S, 1, D), kv.expand(1, S, 1, D)
    qr, kr = orc.apply_rope(qs, c64, s64), orc.apply_rope(ks, c64, s64)
    dots = torch.einsum("bihd,bjhd->ij", qr, kr)
    for off in (0, 3, -7):
        dg = torch.diagonal(dots, offset=off)
        assert torch.allclose(dg, dg[0].expand_as(dg), atol=1e-9)
    assert torch.equal(orc.rope_tables(S, D, 500000.0, torch.bfloat16)[0], wl.rope_tables(S, D, 500000.0, torch.bfloat16)[0])


def test_rope_dtype_rounding_is_elementwise_eager():
    """The bf16 RoPE is x*cos + rot(x)*sin with one rounding per op."""
    S, D = 33, 8
    cos, sin = orc.rope_tables(S, D, 10000.0, torch.bfloat16)
    x = r((2, S, 3, D), 33, torch.bfloat16)
    y = orc.apply_rope(x, cos, sin)
    c, s = cos[None, :, None], sin[None, :, None]
    x1, x2 = x[..., : D // 2].float(), x[..., D // 2:].float()
    c1, s1 = c[..., : D // 2].float(), s[..., : D // 2].float()
    bf = lambda t: t.to(torch.bfloat16).float()
    lo = bf(bf(x1 * c1) - bf(x2 * s1))
    hi = bf(bf(x2 * c1) + bf(x1 * s1))
    assert torch.equal(y.float(), torch.cat([lo, hi], -1))


def test_philox_known_answers():
    """Random123 known-answer vectors for philox4x32-10."""
    kat = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in kat:
        got = orc.philox4x32_10(np.array(ctr, dtype=np.uint32), key)
        assert tuple(int(x) for x in got) == want


def test_dropout_keep_statistics():
    keep = orc.dropout_keep(2, 3, 64, 100, 0.25, seed=77)
    assert keep.shape == (2, 3, 64, 100)
    assert abs(keep.mean() - 0.75) < 0.01
    assert not np.array_equal(keep[0, 0], keep[0, 1])
    assert np.array_equal(keep, orc.dropout_keep(2, 3, 64, 100, 0.25, seed=77))


def test_dropout_keep_field_mapping():
    """Key j of row i takes 16-bit field j % 8 of the four Philox words of
    counter (j // 8, i, b*H + h, offset_lo): at p = 0.5 the keep test
    (field >= 2^15) is the field's top bit, so the mask must equal bit
    16*(j % 2) + 15 of word (j % 8) // 2, read off single scalar calls; at
    p = 1 - 2^-16 only fields equal to 0xFFFF are kept."""
    B, H, Sq, Sk, seed, off = 1, 2, 5, 21, 0x1234_5678_9ABC, (7 << 32) | 3
    keep = orc.dropout_keep(B, H, Sq, Sk, 0.5, seed, off)
    key = ((seed & 0xFFFFFFFF) ^ (off >> 32), seed >> 32)
    for h in range(H):
        for i in range(Sq):
            for j in range(Sk):
                w = orc.philox4x32_10(np.array([j // 8, i, h, off & 0xFFFFFFFF], dtype=np.uint32), key)
                bit = (int(w[(j % 8) // 2]) >> (16 * (j % 2) + 15)) & 1
                assert bool(keep[0, h, i, j]) == bool(bit), (h, i, j)
    keep_hi = orc.dropout_keep(B, H, Sq, Sk, 1.0 - 2.0 ** -16, seed, off)
    w = orc.philox4x32_10(np.array([[[0, i, h, off & 0xFFFFFFFF] for i in range(Sq)] for h in range(H)],
                                   dtype=np.uint32), key)
    fields = np.stack([w & 0xFFFF, w >> 16], axis=-1).reshape(H, Sq, 8)
    assert np.array_equal(keep_hi[0, :, :, :8], fields == 0xFFFF)


def test_dropout_in_eager_restatement_pinned():
    """Dropout with a given keep mask (base.py:395): against the fp64
    closed form, and two cases the mathematics fixes: a mask keeping
    everything scales the no-dropout output by 1/(1-p), a mask keeping
    nothing gives zeros; a row keeping one key c gives P[c] v[c] / (1-p)."""
    g = torch.Generator().manual_seed(9)
    B, S, H, D, p = 2, 12, 3, 8, 0.4
    q, k, v = (torch.randn(B, S, H, D, generator=g) for _ in range(3))
    keep = torch.from_numpy(orc.dropout_keep(B, H, S, S, p, seed=5))
    out = orc.functional_attention(q, k, v, causal=True, keep=keep, dropout_p=p)
    ref = orc.closed_form(q, k, v, causal=True, keep=keep.numpy(), dropout_p=p)
    assert np.allclose(out.double().numpy(), ref, rtol=1e-5, atol=1e-6)
    plain = orc.functional_attention(q, k, v, causal=True)
    ones = torch.ones(B, H, S, S, dtype=torch.bool)
    got = orc.functional_attention(q, k, v, causal=True, keep=ones, dropout_p=p)
    assert torch.allclose(got, plain / (1 - p), rtol=1e-6, atol=1e-6)
    assert torch.equal(orc.functional_attention(q, k, v, keep=~ones, dropout_p=p), torch.zeros(B, S, H, D))
    one = torch.zeros(B, H, S, S, dtype=torch.bool)
    one[..., 3] = True
    got = orc.functional_attention(q, k, v, keep=one, dropout_p=p)
    s = torch.einsum("bihd,bjhd->bhij", q.double(), k.double()) * D ** -0.5
    pc = torch.softmax(s, -1)[..., 3]  # (B, H, Sq)
    want = pc.permute(0, 2, 1)[..., None] * v.double()[:, 3][:, None] / (1 - p)
    assert torch.allclose(got.double(), want, rtol=1e-5, atol=1e-6)


def test_allowed_pairs_and_flops():
    for Sq, Sk, causal, win in [(7, 7, True, None), (9, 5, True, None), (10, 10, False, (2, 1)),
                                (12, 12, True, (3, 0)), (6, 9, False, None), (8, 8, True, (0, 0))]:
        i = np.arange(Sq)[:, None]
        j = np.arange(Sk)[None, :]
        ok = np.ones((Sq, Sk), bool)
        if causal:
            ok &= j <= i
        if win is not None:
            ok &= (j - i >= -win[0]) & (j - i <= win[1])
        assert allowed_pairs(Sq, Sk, causal, win) == int(ok.sum())
    c3 = wl.WORKLOADS["c3"]
    assert wl.flops(c3) == 4 * 128 * 32 * (8192 * 8193 // 2)
    c4 = wl.WORKLOADS["c4"]
    assert wl.flops(c4) == 4 * 128 * 2 * 32 * 58_734_592
    assert abs(wl.flops(c3) - 5.498e11) / 5.498e11 < 1e-3


def test_c5_block_mask_properties():
    m = wl.block_mask(2048, 5)
    blocks = torch.isneginf(m).view(32, 64, 32, 64).permute(0, 2, 1, 3).reshape(32, 32, -1)
    full = blocks.all(-1)
    assert torch.equal(full, blocks.any(-1))  # blocks are all -inf or all 0
    assert 0.05 < full.float().mean().item() < 0.15
    assert (~full).any(dim=1).all()  # every block-row keeps an open block


def test_qk_rms_norm_pinned():
    """The qk RMSNorm restatement against an fp64 per-row loop, the closed
    form of a constant row, and scale invariance (eps = 0)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 4, 16, generator=g)
    w = torch.randn(16, generator=g)
    y = orc.qk_rms_norm(x, w, 1e-6)
    xd, wd = x.double().numpy(), w.double().numpy()
    for idx in np.ndindex(2, 3, 4):
        row = xd[idx]
        want = wd * row / math.sqrt(sum(v * v for v in row) / 16 + 1e-6)
        assert np.allclose(y[idx].double().numpy(), want, rtol=2e-6, atol=1e-7)
    c = torch.full((1, 1, 1, 16), -3.0)
    assert torch.allclose(orc.qk_rms_norm(c, w, 0.0), -w, rtol=1e-6)
    assert torch.allclose(orc.qk_rms_norm(7.5 * x, w, 0.0), orc.qk_rms_norm(x, w, 0.0), rtol=1e-5, atol=1e-6)
    yb = orc.qk_rms_norm(x.bfloat16(), w.bfloat16(), 1e-6)
    assert yb.dtype == torch.bfloat16
    assert (yb.float() - y).abs().max() <= 2 ** -6 * y.abs().max()


def test_qk_layer_norm_pinned():
    """The qk LayerNorm restatement against an fp64 per-row loop (biased
    variance), its bf16 evaluation within the rounding of its fp32 one, and
    the gradients of its autograd (the reference's backward) against an
    fp64 finite difference."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 3, 4, 32, generator=g)
    w, b = torch.randn(32, generator=g), torch.randn(32, generator=g)
    y = orc.qk_layer_norm(x, w, b, 1e-5)
    xd, wd, bd = x.double().numpy(), w.double().numpy(), b.double().numpy()
    for idx in np.ndindex(2, 3, 4):
        row = xd[idx]
        mu = sum(row) / 32
        var = sum((v - mu) ** 2 for v in row) / 32
        want = (row - mu) / math.sqrt(var + 1e-5) * wd + bd
        assert np.allclose(y[idx].double().numpy(), want, rtol=1e-5, atol=1e-5)
    yb = orc.qk_layer_norm(x.bfloat16(), w, b, 1e-5)
    assert yb.dtype == torch.bfloat16
    assert (yb.float() - y).abs().max() <= 2 ** -6 * y.abs().max() + 2 ** -6
    # d/dx of sum(c * y) by central differences in fp64
    xx = x[0, 0, :1].double().requires_grad_(True)
    c = torch.randn(1, 32, generator=g).double()
    (orc.qk_layer_norm(xx, w.double(), b.double(), 1e-5) * c).sum().backward()
    h = 1e-6
    for j in (0, 7, 31):
        e = torch.zeros_like(xx)
        e[0, j] = h
        with torch.no_grad():
            fd = ((orc.qk_layer_norm(xx + e, w.double(), b.double(), 1e-5) * c).sum()
                  - (orc.qk_layer_norm(xx - e, w.double(), b.double(), 1e-5) * c).sum()) / (2 * h)
        assert abs(fd.item() - xx.grad[0, j].item()) <= 1e-6 * max(1.0, abs(fd.item()))


def test_row_and_key_bands_equal_full_evaluation():
    """A row band (and a key range covering the band) gives the rows of the
    full evaluation: causal, window, ALiBi and a user mask at absolute
    positions.  Pins the band evaluation the full-size GPU parity tests use."""
    g = torch.Generator().manual_seed(21)
    B, S, H, Hkv, D = 2, 96, 4, 2, 16
    q, k, v = (torch.randn(B, S, h, D, generator=g).bfloat16() for h in (H, Hkv, Hkv))
    m = torch.randn(S, S, generator=g)
    sl = orc.alibi_slopes(H)
    for kw, rows, keys in [
        (dict(causal=True), (32, 64), None),
        (dict(causal=True), (0, 16), (0, 16)),
        (dict(causal=True, window_size=(20, 0)), (40, 72), (20, 72)),
        (dict(window_size=(5, 9)), (50, 60), (45, 69)),
        (dict(attn_mask=m, alibi_slopes=sl), (10, 30), None),
        (dict(causal=True, alibi_slopes=sl, attn_mask=m), (70, 96), (0, 96)),
    ]:
        full = orc.functional_attention(q, k, v, **kw)
        band = orc.functional_attention(q, k, v, rows=rows, keys=keys, **kw)
        want = full[:, rows[0]:rows[1]]
        assert band.shape == want.shape
        assert (band.float() - want.float()).abs().max().item() <= 2 ** -7 * want.float().abs().max().item(), kw
    with pytest.raises(AssertionError):
        orc.functional_attention(q, k, v, causal=True, window_size=(20, 0), rows=(40, 72), keys=(30, 72))


def test_closed_form_row_positions():
    """closed_form on a subset of rows with their absolute positions equals
    those rows of the full evaluation (causal, window, ALiBi, mask)."""
    g = torch.Generator().manual_seed(23)
    B, S, H, D = 1, 40, 2, 8
    q, k, v = (torch.randn(B, S, H, D, generator=g) for _ in range(3))
    m = torch.randn(S, S, generator=g)
    for kw in (dict(causal=True), dict(window_size=(4, 2)), dict(alibi_slopes=orc.alibi_slopes(H), attn_mask=m)):
        full = orc.closed_form(q, k, v, **kw)
        pos = [3, 17, 39]
        part = orc.closed_form(q[:, pos], k, v, row_pos=pos, **kw)
        assert np.allclose(part, full[:, pos], rtol=1e-12, atol=1e-12)
