"""GPU tests of the attention backward (``trinix_attn_bwd`` through
``triton_attn_func`` / the layers).  The reference's Triton attention has no
backward; the gradients to match are those of its eager path, i.e. torch
autograd through the oracle (``oracle/attention_oracle.py``, the restated
``base.py:347-400``).

Bar (the usual one for fused attention): with fp64 autograd of the oracle as
the truth, the HIP gradients in bf16/fp16 must be within twice the error of
the oracle's own bf16/fp16 autograd, plus 2e-3 of the gradient's scale."""
import pytest
import torch

import trinix_amd as tx
from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, Sq, Sk, H, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, H, D, generator=g)
    k = torch.randn(B, Sk, Hkv, D, generator=g)
    v = torch.randn(B, Sk, Hkv, D, generator=g)
    do = torch.randn(B, Sq, H, D, generator=g)
    return q, k, v, do


def _eager_grads(q, k, v, do, dtype, **kw):
    ts = [t.detach().to(dtype).clone().requires_grad_(True) for t in (q, k, v)]
    out = orc.functional_attention(*ts, **kw)
    out.backward(do.to(dtype))
    return out.detach().double(), [t.grad.double() for t in ts]


def _hip_grads(q, k, v, do, dtype, **kw):
    ts = [t.detach().to(DEV, dtype).clone().requires_grad_(True) for t in (q, k, v)]
    kw = {key: (val.to(DEV) if torch.is_tensor(val) else val) for key, val in kw.items()}
    out = triton_attn_func(*ts, **kw)
    out.backward(do.to(DEV, dtype))
    return out.detach().cpu().double(), [t.grad.cpu().double() for t in ts]


def _check(hip, eager, truth):
    for name, h, e, t in zip("qkv", hip, eager, truth):
        scale = t.abs().max().item()
        err_h = (h - t).abs().max().item()
        err_e = (e - t).abs().max().item()
        assert err_h <= 2 * err_e + 2e-3 * scale, (name, err_h, err_e, scale)


CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, kwargs)
    (2, 160, 160, 4, 4, 64, torch.bfloat16, dict()),
    (1, 200, 200, 4, 2, 128, torch.bfloat16, dict(causal=True)),
    (1, 256, 256, 4, 1, 128, torch.float16, dict(causal=True, window_size=(70, 0))),
    (2, 96, 150, 2, 2, 64, torch.bfloat16, dict(softmax_scale=0.2)),
    (1, 130, 130, 4, 2, 64, torch.float16, dict(window_size=(20, 33))),
    (2, 128, 128, 4, 4, 64, torch.float16, dict(alibi_slopes=orc.alibi_slopes(4))),
    # the dK/dV kernel pipelines (q-head, 64-query tile) items over two
    # stages: one item (the second stage runs alone on the last step), two
    # items, and a key block past Sk with a single query tile
    (1, 17, 17, 1, 1, 128, torch.float16, dict(causal=True)),
    (1, 40, 70, 2, 1, 64, torch.bfloat16, dict()),
    (2, 64, 200, 3, 1, 128, torch.bfloat16, dict(window_size=(0, 90))),
    # top-left causal with Sq != Sk: keys past Sq - 1 get no gradient (Sq < Sk);
    # rows past Sk - 1 see every key (Sq > Sk)
    (1, 100, 180, 2, 1, 128, torch.bfloat16, dict(causal=True)),
    (1, 180, 100, 2, 2, 64, torch.float16, dict(causal=True)),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_backward_matches_eager_autograd(case):
    B, Sq, Sk, H, Hkv, D, dtype, kw = CASES[case]
    q, k, v, do = _inputs(B, Sq, Sk, H, Hkv, D, seed=100 + case)
    _, truth = _eager_grads(q, k, v, do, torch.float64, **kw)
    _, eager = _eager_grads(q, k, v, do, dtype, **kw)
    out, hip = _hip_grads(q, k, v, do, dtype, **kw)
    _check(hip, eager, truth)


def test_backward_with_block_mask_and_alibi():
    B, S, H, D = 2, 192, 4, 64
    q, k, v, do = _inputs(B, S, S, H, H, D, seed=7)
    m = torch.zeros(S, S)
    g = torch.Generator().manual_seed(3)
    blocks = torch.rand(S // 64, S // 64, generator=g) < 0.3
    blocks.fill_diagonal_(False)  # every row keeps its diagonal block
    m = torch.where(blocks.repeat_interleave(64, 0).repeat_interleave(64, 1), float("-inf"), 0.0)
    m[5, 7] = -2.5  # one finite non-zero entry: a per-element block
    kw = dict(attn_mask=m, alibi_slopes=orc.alibi_slopes(H))
    _, truth = _eager_grads(q, k, v, do, torch.float64, **kw)
    _, eager = _eager_grads(q, k, v, do, torch.float16, **kw)
    _, hip = _hip_grads(q, k, v, do, torch.float16, **kw)
    _check(hip, eager, truth)


def test_backward_mask_view_with_a_wide_row_stride():
    """A mask that is a column slice of a wider buffer (row stride 4099
    elements, rows not 16-byte aligned): the dK/dV kernel addresses each
    32-row sub-tile from its first row, the dQ kernel each row, both from
    the view's strides, and must read what the contiguous mask holds."""
    B, S, H, D = 1, 200, 4, 128
    q, k, v, do = _inputs(B, S, S, H, H, D, seed=19)
    g = torch.Generator().manual_seed(8)
    wide = torch.randn(S, 4099, generator=g) * 0.5
    blocks = torch.rand(-(-S // 32), -(-S // 32), generator=g) < 0.2
    blocks[:, 0] = False
    wide[:, :S].masked_fill_(blocks.repeat_interleave(32, 0).repeat_interleave(32, 1)[:S, :S], float("-inf"))
    m = wide[:, :S].contiguous()
    m_dev = wide.to(DEV)[:, :S]  # sliced on the device: .to() of the CPU view would make it contiguous
    assert m_dev.stride() == (4099, 1)
    kw = dict(causal=True)
    _, truth = _eager_grads(q, k, v, do, torch.float64, attn_mask=m, **kw)
    _, eager = _eager_grads(q, k, v, do, torch.bfloat16, attn_mask=m, **kw)
    _, hip = _hip_grads(q, k, v, do, torch.bfloat16, attn_mask=m_dev, **kw)
    _check(hip, eager, truth)


def test_backward_fused_rope_and_lse_output():
    B, S, H, Hkv, D = 1, 144, 4, 2, 128
    q, k, v, do = _inputs(B, S, S, H, Hkv, D, seed=11)
    dtype = torch.bfloat16

    def eager(dt):
        cos, sin = orc.rope_tables(S, D, 500000.0, dt)
        ts = [t.to(dt).requires_grad_(True) for t in (q, k, v)]
        out = orc.functional_attention(orc.apply_rope(ts[0], cos, sin), orc.apply_rope(ts[1], cos, sin), ts[2],
                                       causal=True)
        out.backward(do.to(dt))
        return [t.grad.double() for t in ts]

    truth, ref = eager(torch.float64), eager(dtype)
    cos, sin = orc.rope_tables(S, D, 500000.0, dtype)
    ts = [t.to(DEV, dtype).requires_grad_(True) for t in (q, k, v)]
    out, lse = triton_attn_func(*ts, causal=True, rotary_cos=cos.to(DEV), rotary_sin=sin.to(DEV), return_lse=True)
    assert not lse.requires_grad and lse.shape == (B, H, S)
    out.backward(do.to(DEV, dtype))
    _check([t.grad.cpu().double() for t in ts], ref, truth)


def test_backward_mqa_expanded_kv_sums_over_heads():
    B, S, H, D = 1, 100, 4, 64
    q, k, v, do = _inputs(B, S, S, H, 1, D, seed=5)
    qd = q.to(DEV, torch.bfloat16).requires_grad_(True)
    kd = k.to(DEV, torch.bfloat16).requires_grad_(True)
    vd = v.to(DEV, torch.bfloat16).requires_grad_(True)
    out = triton_attn_func(qd, kd.expand(-1, -1, H, -1), vd.expand(-1, -1, H, -1), causal=True)
    out.backward(do.to(DEV, torch.bfloat16))
    _, truth = _eager_grads(q, k, v, do, torch.float64, causal=True)
    _, eager = _eager_grads(q, k, v, do, torch.bfloat16, causal=True)
    _check([t.grad.cpu().double() for t in (qd, kd, vd)], eager, truth)


def test_backward_is_deterministic():
    q, k, v, do = _inputs(1, 300, 300, 8, 2, 128, seed=9)
    res = []
    for _ in range(2):
        ts = [t.to(DEV, torch.bfloat16).requires_grad_(True) for t in (q, k, v)]
        triton_attn_func(*ts, causal=True).backward(do.to(DEV, torch.bfloat16))
        res.append([t.grad.clone() for t in ts])
    for a, b in zip(*res):
        assert torch.equal(a, b)


WIDE_DQ_CASES = [
    # (B, Sq, Sk, H, Hkv, dtype, kwargs), head_dim 128
    (1, 300, 300, 4, 2, torch.bfloat16, dict(causal=True)),
    (2, 130, 250, 2, 2, torch.float16, dict(window_size=(60, 20), alibi_slopes=orc.alibi_slopes(2))),
    (1, 200, 200, 4, 1, torch.bfloat16, dict(causal=True, dropout_p=0.2)),
]


@pytest.mark.parametrize("case", range(len(WIDE_DQ_CASES)))
def test_wide_dq_shape(case, monkeypatch):
    """The dQ kernel's 256-row, 128-key shape (taken on large grids at head_dim
    128 without a mask), forced through TRINIX_BWD_DQ_WIDE: bitwise the
    gradients of the 128-row shape (the same per-row order of key tiles),
    and within the bar against fp64 autograd."""
    B, Sq, Sk, H, Hkv, dtype, kw = WIDE_DQ_CASES[case]
    q, k, v, do = _inputs(B, Sq, Sk, H, Hkv, 128, seed=700 + case)
    grads = {}
    for wide in ("0", "1"):
        monkeypatch.setenv("TRINIX_BWD_DQ_WIDE", wide)
        torch.manual_seed(99)  # the same dropout seed in both runs
        grads[wide] = _hip_grads(q, k, v, do, dtype, **kw)[1]
    for a, b in zip(grads["0"], grads["1"]):
        assert torch.equal(a, b)
    if "dropout_p" not in kw:
        _, truth = _eager_grads(q, k, v, do, torch.float64, **kw)
        _, eager = _eager_grads(q, k, v, do, dtype, **kw)
        _check(grads["1"], eager, truth)


def test_dropout_backward_is_deterministic_and_follows_the_seed():
    """The same dropout seed gives bitwise the same gradients; another seed
    gives other ones."""
    q, k, v, do = _inputs(1, 200, 200, 4, 2, 128, seed=19)
    res = []
    for seed in (77, 77, 78):
        ts = [t.to(DEV, torch.bfloat16).requires_grad_(True) for t in (q, k, v)]
        torch.manual_seed(seed)
        triton_attn_func(*ts, dropout_p=0.2, causal=True).backward(do.to(DEV, torch.bfloat16))
        res.append([t.grad.clone() for t in ts])
    for a, b, c in zip(*res):
        assert torch.equal(a, b)
        assert not torch.equal(a, c)


def test_layer_training_step_gradients():
    torch.manual_seed(21)
    E, H, HKV, S = 256, 4, 2, 96
    hip = tx.FastGroupedQueryAttention(E, H, HKV, causal=True, position_method="rope", rope_base=10000.0,
                                       kernel_type="flash")
    ref64 = tx.FastGroupedQueryAttention(E, H, HKV, causal=True, position_method="rope", rope_base=10000.0,
                                         kernel_type="pytorch").double()
    ref16 = tx.FastGroupedQueryAttention(E, H, HKV, causal=True, position_method="rope", rope_base=10000.0,
                                         kernel_type="pytorch").to(torch.bfloat16)
    ref64.load_state_dict(hip.state_dict())
    ref16.load_state_dict(hip.state_dict())
    hip = hip.to(DEV, torch.bfloat16)
    x = torch.randn(2, S, E)
    gy = torch.randn(2, S, E)
    grads = []
    for layer, dev, dt in ((hip, DEV, torch.bfloat16), (ref64, "cpu", torch.float64), (ref16, "cpu", torch.bfloat16)):
        xi = x.to(dev, dt).requires_grad_(True)
        y, _ = layer(xi)
        y.backward(gy.to(dev, dt))
        grads.append([xi.grad.cpu().double()] + [layer.get_parameter(n).grad.cpu().double()
                                                 for n in ("q_proj.weight", "k_proj.weight", "v_proj.weight")])
    h, t, e = grads
    for gh, gt, ge in zip(h, t, e):
        scale = gt.abs().max().item()
        assert (gh - gt).abs().max().item() <= 2 * (ge - gt).abs().max().item() + 2e-3 * scale


# ---------------------------------------------------------------------------
# the generic backward: fp32, head_dim 256 and dropout
# ---------------------------------------------------------------------------
def _check32(hip, eager, truth):
    """fp32: within twice the eager fp32 error plus 1e-5 of the scale (the
    north star's fp32 tolerance is 1e-5 relative)."""
    for name, h, e, t in zip("qkv", hip, eager, truth):
        scale = t.abs().max().item()
        err_h = (h - t).abs().max().item()
        err_e = (e - t).abs().max().item()
        assert err_h <= 2 * err_e + 1e-5 * scale, (name, err_h, err_e, scale)


GEN_CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, kwargs)
    (2, 100, 100, 4, 4, 64, torch.float32, dict()),
    (1, 150, 150, 4, 2, 128, torch.float32, dict(causal=True)),
    (1, 96, 130, 2, 1, 256, torch.float32, dict(window_size=(40, 10))),
    (2, 64, 64, 4, 4, 64, torch.float32, dict(alibi_slopes=orc.alibi_slopes(4), softmax_scale=0.3)),
    (1, 200, 200, 4, 2, 256, torch.bfloat16, dict(causal=True)),
    (2, 77, 77, 2, 2, 256, torch.float16, dict(alibi_slopes=orc.alibi_slopes(2))),
    (1, 65, 190, 4, 1, 256, torch.bfloat16, dict(window_size=(0, 100))),
    (1, 120, 120, 2, 2, 192, torch.bfloat16, dict(causal=True)),  # padded to 256
]


@pytest.mark.parametrize("case", range(len(GEN_CASES)))
def test_generic_backward_fp32_and_d256(case):
    B, Sq, Sk, H, Hkv, D, dtype, kw = GEN_CASES[case]
    print(f"generic backward case {GEN_CASES[case][:7]}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hkv, D, seed=300 + case)
    _, truth = _eager_grads(q, k, v, do, torch.float64, **kw)
    _, eager = _eager_grads(q, k, v, do, dtype, **kw)
    _, hip = _hip_grads(q, k, v, do, dtype, **kw)
    (_check32 if dtype == torch.float32 else _check)(hip, eager, truth)


def test_generic_backward_with_mask():
    B, S, H, D = 1, 130, 2, 256
    q, k, v, do = _inputs(B, S, S, H, H, D, seed=17)
    g = torch.Generator().manual_seed(4)
    m = torch.where(torch.rand(S, S, generator=g) < 0.1, float("-inf"), torch.randn(S, S, generator=g) * 0.5)
    m.fill_diagonal_(0.0)
    for dtype in (torch.float32, torch.bfloat16):
        _, truth = _eager_grads(q, k, v, do, torch.float64, attn_mask=m, causal=True)
        _, eager = _eager_grads(q, k, v, do, dtype, attn_mask=m, causal=True)
        _, hip = _hip_grads(q, k, v, do, dtype, attn_mask=m, causal=True)
        (_check32 if dtype == torch.float32 else _check)(hip, eager, truth)


def _dropout_grads(q, k, v, do, dtype, keep, p, dev, **kw):
    ts = [t.detach().to(dev, dtype).clone().requires_grad_(True) for t in (q, k, v)]
    kw = {key: (val.to(dev) if torch.is_tensor(val) else val) for key, val in kw.items()}
    if dev == "cpu":
        out = orc.functional_attention(*ts, keep=keep, dropout_p=p, **kw)
    else:
        torch.manual_seed(4321)  # the kernel's dropout seed comes from torch's CPU generator
        out = triton_attn_func(*ts, dropout_p=p, **kw)
    out.backward(do.to(dev, dtype))
    return out.detach().cpu().double(), [t.grad.cpu().double() for t in ts]


def _drop_mask(Sq, Sk, seed):
    """Additive float mask: -inf on ~20% of 32x32 blocks (never the first key
    block), N(0, 0.5) elsewhere."""
    g = torch.Generator().manual_seed(seed)
    blocks = torch.rand(-(-Sq // 32), -(-Sk // 32), generator=g) < 0.2
    blocks[:, 0] = False
    inf = blocks.repeat_interleave(32, 0).repeat_interleave(32, 1)[:Sq, :Sk]
    return torch.where(inf, float("-inf"), torch.randn(Sq, Sk, generator=g) * 0.5)


DROP_CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, p, kwargs): bf16/fp16 at head_dim 64/128
    # run the MFMA pipeline (dK/dV regenerates the keep bits of a key's rows
    # per quad of lanes, dQ those of a row's keys), fp32 and 256 the generic
    # kernels
    (1, 160, 160, 4, 2, 64, torch.bfloat16, 0.1, dict(causal=True)),
    (2, 96, 96, 2, 2, 128, torch.float16, 0.3, dict()),
    (1, 128, 128, 4, 1, 128, torch.bfloat16, 0.2, dict(alibi_slopes=orc.alibi_slopes(4), causal=True)),
    (1, 100, 100, 2, 2, 64, torch.float32, 0.25, dict(window_size=(30, 0))),
    (1, 90, 90, 2, 2, 256, torch.bfloat16, 0.1, dict(causal=True)),
    (1, 130, 200, 4, 2, 128, torch.bfloat16, 0.15, dict(window_size=(50, 20))),
    (2, 100, 100, 4, 4, 64, torch.float16, 0.5, dict(alibi_slopes=orc.alibi_slopes(4),
                                                     attn_mask=_drop_mask(100, 100, 31))),
    (1, 150, 150, 2, 1, 128, torch.bfloat16, 0.1, dict(attn_mask=_drop_mask(150, 150, 32), causal=True)),
    (1, 17, 17, 1, 1, 128, torch.float16, 0.1, dict(causal=True)),
    (1, 40, 70, 2, 1, 64, torch.bfloat16, 0.05, dict(softmax_scale=0.2)),
    # ALiBi + mask + dropout at head_dim 128: the dQ variant whose lanes make
    # their own Philox calls (no lane-pair exchange; every register in use)
    (1, 140, 140, 4, 2, 128, torch.float16, 0.2, dict(alibi_slopes=orc.alibi_slopes(4),
                                                      attn_mask=_drop_mask(140, 140, 33), causal=True)),
    (2, 70, 90, 2, 2, 128, torch.bfloat16, 0.35, dict(alibi_slopes=orc.alibi_slopes(2),
                                                      attn_mask=_drop_mask(70, 90, 34))),
]


@pytest.mark.parametrize("keep_map", ["1", "0"])
@pytest.mark.parametrize("case", range(len(DROP_CASES)))
def test_dropout_backward_matches_eager_with_philox_keep(case, keep_map, monkeypatch):
    """Forward and gradients with dropout against eager autograd of the
    oracle using the kernel's keep mask (the Philox stream the oracle
    restates), so the backward must use exactly the forward's mask: read
    from the forward's keep map (bf16/fp16 at head_dim 64/128), or
    regenerated (TRINIX_DROPOUT_KEEP_MAP=0, and the generic kernels)."""
    monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", keep_map)
    B, Sq, Sk, H, Hkv, D, dtype, p, kw = DROP_CASES[case]
    print(f"dropout backward case {DROP_CASES[case][:8]} keep map {keep_map}", flush=True)
    q, k, v, do = _inputs(B, Sq, Sk, H, Hkv, D, seed=500 + case)
    torch.manual_seed(4321)
    seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    keep = torch.from_numpy(orc.dropout_keep(B, H, Sq, Sk, p, seed))
    out64, truth = _dropout_grads(q, k, v, do, torch.float64, keep, p, "cpu", **kw)
    oute, eager = _dropout_grads(q, k, v, do, dtype, keep, p, "cpu", **kw)
    outh, hip = _dropout_grads(q, k, v, do, dtype, keep, p, DEV, **kw)
    # the output, like the gradients, within twice the eager error (in the
    # same dtype, same keep mask) against fp64, plus a small part of its
    # scale: at p = 0.5 the kept weights double, so one bf16 ulp of an
    # output near 2 is already 0.0156 and an absolute 2e-2 bar would be
    # about one rounding wide
    scale = out64.abs().max().item()
    err_h, err_e = (outh - out64).abs().max().item(), (oute - out64).abs().max().item()
    small = 1e-5 if dtype == torch.float32 else 2e-3
    print(f"  out: hip {err_h:.3e}, eager {err_e:.3e}, scale {scale:.3f}", flush=True)
    assert err_h <= 2 * err_e + small * scale, (err_h, err_e, scale)
    (_check32 if dtype == torch.float32 else _check)(hip, eager, truth)


def _layer_step_grads(make, x, gy, dtype, dropout_keep=None):
    """Input and q/k/v/o projection gradients of one training step of the
    HIP layer and of the eager ('pytorch') layer in fp64 and in ``dtype``,
    all from the same weights.  With ``dropout_keep`` = (keep, p) the eager
    layers drop with that mask instead of a random one."""
    hip = make("flash")
    refs = [make("pytorch").double(), make("pytorch").to(dtype)]
    for r in refs:
        r.load_state_dict(hip.state_dict())
        if dropout_keep is not None:
            keep, p = dropout_keep

            def fwd_attn(q, k, v, attn_mask=None, _r=r):
                return orc.functional_attention(q, k, v, attn_mask, causal=_r.causal, keep=keep, dropout_p=p)

            r.forward_attention = fwd_attn
    hip = hip.to(DEV, dtype)
    out = []
    for layer, dev, dt in ((hip, DEV, dtype), (refs[0], "cpu", torch.float64), (refs[1], "cpu", dtype)):
        layer.train()
        xi = x.to(dev, dt).requires_grad_(True)
        if dev == DEV:
            torch.manual_seed(777)
        y = layer(xi)
        y = y[0] if isinstance(y, tuple) else y
        y.backward(gy.to(dev, dt))
        out.append([xi.grad.cpu().double()] + [layer.get_parameter(n).grad.cpu().double()
                                                for n in ("q_proj.weight", "k_proj.weight", "v_proj.weight",
                                                          "o_proj.weight")])
    return out


def _check_layer(grads, add):
    h, t, e = grads
    for name, gh, gt, ge in zip(("x", "q_proj", "k_proj", "v_proj", "o_proj"), h, t, e):
        scale = gt.abs().max().item()
        err_h, err_e = (gh - gt).abs().max().item(), (ge - gt).abs().max().item()
        assert err_h <= 2 * err_e + add * scale, (name, err_h, err_e, scale)


def test_layer_training_step_with_dropout():
    """A bf16 GQA layer in training mode with dropout 0.1: the HIP step's
    gradients match eager autograd through the same dropout mask."""
    import warnings

    E, H, HKV, S, p = 256, 4, 2, 96, 0.1
    torch.manual_seed(31)

    def make(kt):
        return tx.FastGroupedQueryAttention(E, H, HKV, dropout=p, causal=True, position_method="rope",
                                            kernel_type=kt)

    torch.manual_seed(777)
    seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    keep = torch.from_numpy(orc.dropout_keep(2, H, S, S, p, seed))
    x, gy = torch.randn(2, S, E), torch.randn(2, S, E)
    torch.manual_seed(31)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        grads = _layer_step_grads(make, x, gy, torch.bfloat16, (keep, p))
    _check_layer(grads, 2e-3)


def test_layer_training_step_fp32():
    import warnings

    E, H, S = 256, 4, 80
    torch.manual_seed(32)

    def make(kt):
        return tx.FastMultiHeadAttention(E, H, causal=True, position_method="alibi", kernel_type=kt)

    x, gy = torch.randn(2, S, E), torch.randn(2, S, E)
    torch.manual_seed(32)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        grads = _layer_step_grads(make, x, gy, torch.float32)
    _check_layer(grads, 1e-5)


def test_layer_training_step_head_dim_256():
    import warnings

    E, H, HKV, S = 512, 2, 1, 112
    torch.manual_seed(33)

    def make(kt):
        return tx.FastGroupedQueryAttention(E, H, HKV, causal=True, position_method="rope", kernel_type=kt)

    x, gy = torch.randn(1, S, E), torch.randn(1, S, E)
    torch.manual_seed(33)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        grads = _layer_step_grads(make, x, gy, torch.bfloat16)
    _check_layer(grads, 2e-3)


def test_dropout_under_capture_needs_the_device_generator(monkeypatch):
    """A call with dropout under capture reads the device's dropout generator,
    which only a call outside a capture can create (its seed is copied to
    the device): without one the call raises before launching anything.
    The capture state is faked, so no graph is captured."""
    import trinix_amd.kernels.attention_kernel as ak

    q = torch.randn(1, 64, 2, 64, device=DEV, dtype=torch.bfloat16)
    monkeypatch.setattr(ak, "_DROPOUT_GENERATORS", {})
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="dropout generator"):
        triton_attn_func(q, q, q, dropout_p=0.1)
    triton_attn_func(q, q, q, dropout_p=0.0)  # without dropout the call proceeds


@pytest.mark.parametrize("wl", ["c3", "c2"])
def test_backward_full_size_against_fp32_eager(wl):
    """BASELINE configs 3 and 2 at full size (C3: the 256-row dQ shape and
    the dK/dV pipeline over every KV head; C2: head_dim 64): gradients of the
    bf16 kernels against fp32 eager autograd on the GPU over the same bf16
    inputs (a plain PyTorch fp32 reference; score matrices materialised,
    operands made contiguous).  Measured: max |error| 0.3-0.5% of max |grad|,
    mean |error| 0.23-0.28% of mean |grad| (the bf16 rounding of the
    gradients); the bar is twice that."""
    from trinix_amd.workloads import WORKLOADS, make_inputs

    w = WORKLOADS[wl]
    print(f"full-size backward {wl}", flush=True)
    inp = make_inputs(w, device=DEV)
    do = torch.randn(inp.q.shape, device=DEV, generator=torch.Generator(device=DEV).manual_seed(7)).to(inp.q.dtype)
    ts = [t.detach().clone().requires_grad_(True) for t in (inp.q, inp.k, inp.v)]
    triton_attn_func(*ts, causal=True).backward(do)
    hip = [t.grad.float() for t in ts]
    q, k, v = (t.detach().float().requires_grad_(True) for t in (inp.q, inp.k, inp.v))
    G, S = w.nheads // w.nheads_kv, w.seqlen
    ke = k.repeat_interleave(G, dim=2).transpose(1, 2).contiguous()
    ve = v.repeat_interleave(G, dim=2).transpose(1, 2).contiguous()
    s = torch.matmul(q.transpose(1, 2), ke.transpose(-1, -2).contiguous()) * w.head_dim ** -0.5
    s = s.masked_fill(torch.triu(torch.ones(S, S, device=DEV, dtype=torch.bool), 1), float("-inf"))
    torch.matmul(torch.softmax(s, dim=-1), ve).transpose(1, 2).backward(do.float())
    for name, h, t in zip("qkv", hip, (q.grad, k.grad, v.grad)):
        d = (h - t).abs()
        assert d.max().item() <= 1e-2 * t.abs().max().item(), (name, d.max().item(), t.abs().max().item())
        assert d.mean().item() <= 6e-3 * t.abs().mean().item(), (name, d.mean().item(), t.abs().mean().item())


LONG_BWD_CASES = [
    # (S, H, Hkv, D, dtype, window, r0): dO nonzero on rows r0..r0+63 only
    (32768, 2, 1, 128, torch.bfloat16, None, 32768 - 64),      # the longest causal chain (512 key tiles)
    (65536, 1, 1, 64, torch.float16, (4096, 0), 40000),        # a causal window inside a 64K sequence
]


@pytest.mark.parametrize("case", LONG_BWD_CASES, ids=[f"S{c[0]}-D{c[3]}" for c in LONG_BWD_CASES])
def test_backward_long_context_one_row_band(case):
    """Gradients of a 32K / 64K-position causal call whose dO is zero outside
    one 64-row band: dQ is then zero outside the band (dP = dO V^T = 0 and
    delta = rowsum(dO O) = 0 there), and dK / dV are the band's contribution
    alone, so the whole of every gradient has an exact reference from the
    band's rows: fp64 and bf16/fp16 autograd of the oracle on those rows
    (the usual bar)."""
    S, H, Hkv, D, dtype, window, r0 = case
    print(f"long backward S={S} D={D}", flush=True)
    q, k, v, _ = _inputs(1, S, S, H, Hkv, D, seed=140)
    do = torch.zeros(1, S, H, D)
    do[:, r0:r0 + 64] = torch.randn(1, 64, H, D, generator=torch.Generator().manual_seed(141))
    kw = dict(causal=True, window_size=window)
    lo = 0 if window is None else max(0, r0 - window[0])
    band = dict(kw, rows=(r0, r0 + 64), keys=(lo, r0 + 64), head_chunk=H)

    def band_grads(dt):
        ts = [t.detach().to(dt).clone().requires_grad_(True) for t in (q, k, v)]
        orc.functional_attention(*ts, **band).backward(do[:, r0:r0 + 64].to(dt))
        return [t.grad.double() for t in ts]

    truth, eager = band_grads(torch.float64), band_grads(dtype)
    _, hip = _hip_grads(q, k, v, do, dtype, **kw)
    for t in (hip[0][:, :r0], hip[0][:, r0 + 64:], hip[1][:, r0 + 64:], hip[2][:, r0 + 64:], hip[2][:, :lo]):
        assert int(torch.count_nonzero(t)) == 0  # outside the band's rows / keys: exactly zero
    _check(hip, eager, truth)


DEAD_ROW_CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, kwargs): some query rows see no key
    (1, 60, 40, 2, 1, 64, torch.bfloat16, dict(window_size=(5, 0))),          # rows >= 45: window past the keys
    (2, 96, 96, 4, 2, 128, torch.float16, dict(alibi_slopes=orc.alibi_slopes(4), dead_mask=(7, 50, 51))),
    (1, 80, 80, 2, 2, 64, torch.float32, dict(dead_mask=(0, 79), causal=True)),  # generic kernels (fp32)
    (1, 70, 70, 2, 1, 256, torch.bfloat16, dict(window_size=(3, 3), dead_mask=(33,))),  # generic (D=256)
]


def _dead_row_inputs(case):
    B, Sq, Sk, H, Hkv, D, dtype, kw = case
    kw = dict(kw)
    dead_rows = kw.pop("dead_mask", None)
    if dead_rows is not None:
        g = torch.Generator().manual_seed(151)
        m = torch.randn(Sq, Sk, generator=g) * 0.5
        m[list(dead_rows), :] = float("-inf")
        kw["attn_mask"] = m
    return B, Sq, Sk, H, Hkv, D, dtype, kw


@pytest.mark.parametrize("case", range(len(DEAD_ROW_CASES)))
def test_backward_rows_without_allowed_keys(case):
    """Rows with no allowed key (a window past the keys, a mask row of -inf)
    give NaN outputs, as eager does; eager autograd then makes the whole
    (batch, head)'s gradients NaN, the HIP backward gives those rows zero
    gradient.  Checked: every gradient finite, dq of those rows exactly 0,
    and all gradients equal (backward bar) to autograd of the same scores
    with those rows made visible and their dO set to 0, in fp64 and in the
    input dtype."""
    B, Sq, Sk, H, Hkv, D, dtype, kw = _dead_row_inputs(DEAD_ROW_CASES[case])
    q, k, v, do = _inputs(B, Sq, Sk, H, Hkv, D, seed=150 + case)
    out, hip = _hip_grads(q, k, v, do, dtype, **kw)
    bias = torch.from_numpy(orc._bias64(Sq, Sk, H, B, kw.get("attn_mask"), kw.get("causal", False),
                                        kw.get("window_size"), kw.get("alibi_slopes")))
    dead = torch.isinf(bias).all(-1)  # (B, H, Sq)
    assert dead.any()
    assert torch.isnan(out.permute(0, 2, 1, 3)[dead]).all()
    assert all(torch.isfinite(h).all() for h in hip)
    assert int(torch.count_nonzero(hip[0].permute(0, 2, 1, 3)[dead])) == 0
    live_bias = bias.masked_fill(dead[..., None], 0.0)  # dead rows made visible ...
    do_live = do.permute(0, 2, 1, 3).masked_fill(dead[..., None], 0.0).permute(0, 2, 1, 3)  # ... with dO = 0

    def grads(dt):
        xs = [t.detach().to(dt).clone().requires_grad_(True) for t in (q, k, v)]
        G = H // Hkv
        kk = xs[1].repeat_interleave(G, dim=2).transpose(1, 2)
        vv = xs[2].repeat_interleave(G, dim=2).transpose(1, 2)
        s = torch.matmul(xs[0].transpose(1, 2), kk.transpose(-1, -2)) * D ** -0.5 + live_bias.to(dt)
        o = torch.matmul(torch.softmax(s.double(), dim=-1).to(dt), vv).transpose(1, 2)
        o.backward(do_live.to(dt))
        return [x.grad.double() for x in xs]

    _check(hip, grads(dtype), grads(torch.float64))
