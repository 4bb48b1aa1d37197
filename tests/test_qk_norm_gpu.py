"""GPU tests of the fused qk-norm (``trinix_qk_norm`` / ``trinix_qk_layernorm``:
RoPE + RMSNorm or LayerNorm over head_dim, and ``trinix_qk_norm_bwd``)
against the oracle's restatement of the reference's eager path
(``orc.apply_rope`` then ``orc.qk_rms_norm`` / ``orc.qk_layer_norm``,
trinix/layers/norm/rmsnorm.py:62-75, layernorm.py:83-88), its autograd on the
CPU for the backward, and of the layers that use them.

Bar: the fp32 reductions are ordered differently from torch's, so a
normalisation factor can differ by an ulp of fp32 and an output element by
an ulp or two of the dtype.  Forward: at least 99% of the elements
bit-identical to the oracle and every element within 2 ulps of it.
Backward, RMSNorm: the gradient is a difference of two terms (the direct
one and the one through the row statistics), which cancel near zero; there
an fp32 rounding difference is large relative to the element, so the bar
adds 1e-3 of the tensor's largest element to the 2 ulps, and 98%
bit-identical.  dweight sums the rows in fp32 in another order: 2 ulps of
the dtype plus 1e-3 of the largest element.
Backward, LayerNorm: torch's CPU layer_norm backward rounds its
intermediate products differently from the fp32 formula (dx is about 70%
bit-identical, within an ulp or two), and the reference's path is torch's
GPU kernel anyway; so the bar is the one of the attention backward: the
error against the fp64 gradient at most twice the eager bf16/fp16 error plus
1e-3 of the largest element.
"""
import pytest
import torch

from oracle import attention_oracle as orc
import trinix_amd as tx
from trinix_amd.kernels import qk_layernorm, qk_rmsnorm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ulp(t: torch.Tensor) -> torch.Tensor:
    mant = 7 if t.dtype == torch.bfloat16 else 10
    a = t.float().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - mant)


def assert_ulps(out, ref, what):
    out, ref = out.cpu(), ref.cpu()
    assert out.dtype == ref.dtype and out.shape == ref.shape, what
    same = (out == ref).float().mean().item()
    d = (out.float() - ref.float()).abs()
    assert same >= 0.99, f"{what}: only {same:.4f} bit-identical"
    assert (d <= 2 * ulp(ref)).all(), f"{what}: max diff {d.max().item():.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [16, 64, 128, 256])
@pytest.mark.parametrize("rope", [False, True])
def test_qk_norm_matches_oracle(D, dtype, rope):
    g = torch.Generator().manual_seed(D + (1 if rope else 0))
    B, S, H = 2, 37, 5
    x = (3 * torch.randn(B, S, H, D, generator=g)).to(dtype)
    w = (1 + 0.3 * torch.randn(D, generator=g)).to(dtype)
    cos = sin = None
    xr = x
    if rope:
        cos, sin = orc.rope_tables(S, D, 10000.0, dtype)
        xr = orc.apply_rope(x, cos, sin)
    ref = orc.qk_rms_norm(xr, w, 1e-6)
    out = qk_rmsnorm(x.to(DEV), w.to(DEV), 1e-6, None if cos is None else cos.to(DEV),
                     None if sin is None else sin.to(DEV))
    assert_ulps(out, ref, f"D={D} {dtype} rope={rope}")


def test_qk_norm_position_ids_and_strided_input():
    dtype, D = torch.bfloat16, 128
    g = torch.Generator().manual_seed(9)
    B, S, H = 3, 20, 4
    x_bhsd = torch.randn(B, H, S, D, generator=g).to(dtype)
    x = x_bhsd.transpose(1, 2)  # a (B, S, H, D) view with head-major strides
    w = torch.randn(D, generator=g).to(dtype)
    pos = torch.randint(0, 100, (B, S), generator=g)
    cos, sin = orc.rope_tables(128, D, 500000.0, dtype)
    ref = orc.qk_rms_norm(orc.apply_rope(x, cos, sin, pos), w, 1e-5)
    xd = x_bhsd.to(DEV).transpose(1, 2)
    assert not xd.is_contiguous()
    out = qk_rmsnorm(xd, w.to(DEV), 1e-5, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_ulps(out, ref, "position_ids, strided")


def test_gqa_layer_with_qk_norm_uses_fused_kernel_in_inference():
    torch.manual_seed(12)
    E, H, HKV, S = 1024, 8, 2, 160
    kw = dict(causal=True, position_method="rope", rope_base=500000.0, qk_norm=True)
    hip = tx.FastGroupedQueryAttention(E, H, HKV, kernel_type="flash", **kw)
    with torch.no_grad():
        hip.q_norm.weight.uniform_(0.5, 1.5)
        hip.k_norm.weight.uniform_(0.5, 1.5)
    eager = tx.FastGroupedQueryAttention(E, H, HKV, kernel_type="pytorch", **kw)
    eager.load_state_dict(hip.state_dict())
    hip, eager = hip.to(DEV, torch.bfloat16), eager.to(DEV, torch.bfloat16)
    x = torch.randn(2, S, E, device=DEV).to(torch.bfloat16)
    D = E // H
    with torch.no_grad():
        probe_q = torch.empty(1, 1, H, D, device=DEV, dtype=torch.bfloat16)
        probe_k = torch.empty(1, 1, HKV, D, device=DEV, dtype=torch.bfloat16)
        assert hip._fused_qk_norm_applies(probe_q, probe_k)
        o1, (k1, v1) = hip(x, use_cache=True)
        o2, (k2, v2) = eager(x, use_cache=True)
    assert torch.equal(v1, v2)
    assert_ulps(k1.contiguous(), k2.contiguous(), "normalised k cache")
    d = (o1.float() - o2.float()).abs()
    scale = max(1.0, o2.float().abs().max().item())
    assert d.max().item() <= 2e-2 * scale and d.mean().item() <= 2e-3 * scale, d.max().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [16, 64, 128, 256])
@pytest.mark.parametrize("rope", [False, True])
def test_qk_layernorm_matches_oracle(D, dtype, rope):
    g = torch.Generator().manual_seed(100 + D + (1 if rope else 0))
    B, S, H = 2, 37, 5
    x = (3 * torch.randn(B, S, H, D, generator=g) + 0.5).to(dtype)
    w = (1 + 0.3 * torch.randn(D, generator=g)).to(dtype)
    b = (0.2 * torch.randn(D, generator=g)).to(dtype)
    cos = sin = None
    xr = x
    if rope:
        cos, sin = orc.rope_tables(S, D, 10000.0, dtype)
        xr = orc.apply_rope(x, cos, sin)
    ref = orc.qk_layer_norm(xr, w, b, 1e-5)
    out = qk_layernorm(x.to(DEV), w.to(DEV), b.to(DEV), 1e-5, None if cos is None else cos.to(DEV),
                       None if sin is None else sin.to(DEV))
    assert_ulps(out, ref, f"layernorm D={D} {dtype} rope={rope}")


def assert_grad(out, ref, what, frac=0.98):
    out, ref = out.detach().cpu(), ref.detach().cpu()
    assert out.dtype == ref.dtype and out.shape == ref.shape, what
    d = (out.float() - ref.float()).abs()
    bar = 2 * ulp(ref) + 1e-3 * ref.float().abs().max()
    same = (out == ref).float().mean().item()
    assert (d <= bar).all(), f"{what}: max diff {d.max().item():.3g} (largest element {ref.float().abs().max():.3g})"
    assert same >= frac, f"{what}: only {same:.4f} bit-identical"


def _norm_case(norm, D, dtype, rope, positions, seed):
    g = torch.Generator().manual_seed(seed)
    B, S, H = 2, 45, 3
    x = (2 * torch.randn(B, S, H, D, generator=g) + 0.3).to(dtype)
    w = (1 + 0.3 * torch.randn(D, generator=g)).to(dtype)
    b = (0.2 * torch.randn(D, generator=g)).to(dtype) if norm == "layer" else None
    dout = torch.randn(B, S, H, D, generator=g).to(dtype)
    cos = sin = pos = None
    if rope:
        cos, sin = orc.rope_tables(64, D, 10000.0, dtype)
        if positions:
            pos = torch.randint(0, 64, (B, S), generator=g)
    return x, w, b, dout, cos, sin, pos


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("rope", ["none", "rope", "rope+positions"])
def test_qk_norm_backward_matches_eager_autograd(norm, dtype, D, rope):
    """dx, dweight (and dbias) of the fused kernels against autograd through
    the oracle's eager RoPE and norm on the CPU (the reference's backward)."""
    x, w, b, dout, cos, sin, pos = _norm_case(norm, D, dtype, rope != "none", rope == "rope+positions",
                                              seed=D + 7 * len(rope) + (1 if norm == "layer" else 0))
    eps = 1e-6 if norm == "rms" else 1e-5

    def eager(dt):
        leaves = [t.detach().to(dt).clone().requires_grad_(True) for t in (x, w) + ((b,) if b is not None else ())]
        c, s_ = (None, None) if cos is None else (cos.to(dt), sin.to(dt))
        xr = orc.apply_rope(leaves[0], c, s_, pos) if c is not None else leaves[0]
        y = orc.qk_rms_norm(xr, leaves[1], eps) if norm == "rms" else orc.qk_layer_norm(xr, leaves[1], leaves[2], eps)
        y.backward(dout.to(dt))
        return y, leaves

    ref, leaves = eager(dtype)
    dev = [t.detach().to(DEV).requires_grad_(True) for t in (x, w) + ((b,) if b is not None else ())]
    tabs = [None if t is None else t.to(DEV) for t in (cos, sin, pos)]
    if norm == "rms":
        out = qk_rmsnorm(dev[0], dev[1], eps, *tabs)
    else:
        out = qk_layernorm(dev[0], dev[1], dev[2], eps, *tabs)
    out.backward(dout.to(DEV))
    what = f"{norm} D={D} {dtype} {rope}"
    assert_ulps(out.detach(), ref.detach(), what + " forward")
    if norm == "rms":
        assert_grad(dev[0].grad, leaves[0].grad, what + " dx")
        assert_grad(dev[1].grad, leaves[1].grad, what + " dweight", frac=0.0)
    else:
        _, truth = eager(torch.float64)
        for name, h, e, t in zip(("dx", "dweight", "dbias"), dev, leaves, truth):
            t64 = t.grad
            err_h = (h.grad.cpu().double() - t64).abs().max().item()
            err_e = (e.grad.double() - t64).abs().max().item()
            scale = t64.abs().max().item()
            assert err_h <= 2 * err_e + 1e-3 * scale, (what, name, err_h, err_e, scale)


def test_qk_norm_backward_strided_input_and_gradient():
    """A head-major (B, S, H, D) view as input and a non-contiguous output
    gradient: the same gradients as contiguous copies."""
    x, w, _, dout, cos, sin, _ = _norm_case("rms", 128, torch.bfloat16, True, False, seed=77)
    xd = x.permute(0, 2, 1, 3).contiguous().to(DEV).permute(0, 2, 1, 3).requires_grad_(True)
    assert not xd.is_contiguous()
    wd = w.to(DEV).requires_grad_(True)
    out = qk_rmsnorm(xd, wd, 1e-6, cos.to(DEV), sin.to(DEV))
    g = dout.to(DEV).permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    out.backward(g)
    xc = x.to(DEV).requires_grad_(True)
    wc = w.to(DEV).requires_grad_(True)
    qk_rmsnorm(xc, wc, 1e-6, cos.to(DEV), sin.to(DEV)).backward(dout.to(DEV))
    assert torch.equal(xd.grad, xc.grad) and torch.equal(wd.grad, wc.grad)


@pytest.mark.parametrize("norm_type", ["rmsnorm", "layernorm"])
def test_qk_norm_layer_training_uses_fused_kernels(norm_type, monkeypatch):
    """A GQA layer training step with qk_norm: the fused kernels (forward and
    backward) replace the eager norm modules, and the gradients of x, the
    projections and the norm parameters are within twice the bf16 eager
    layer's error (against fp64) plus 2e-3 of the largest element."""
    from trinix_amd.layers.attention import base as lb

    torch.manual_seed(13 + len(norm_type))
    E, H, HKV, S = 512, 4, 2, 64
    kw = dict(causal=True, position_method="rope", rope_base=10000.0, qk_norm=True, qk_norm_type=norm_type)
    hip = tx.FastGroupedQueryAttention(E, H, HKV, kernel_type="flash", **kw)
    with torch.no_grad():
        hip.q_norm.weight.uniform_(0.5, 1.5)
        hip.k_norm.weight.uniform_(0.5, 1.5)
        if norm_type == "layernorm":
            hip.q_norm.bias.uniform_(-0.2, 0.2)
            hip.k_norm.bias.uniform_(-0.2, 0.2)
    ref64 = tx.FastGroupedQueryAttention(E, H, HKV, kernel_type="pytorch", **kw).double()
    ref16 = tx.FastGroupedQueryAttention(E, H, HKV, kernel_type="pytorch", **kw).to(torch.bfloat16)
    ref64.load_state_dict(hip.state_dict())
    ref16.load_state_dict(hip.state_dict())
    hip = hip.to(DEV, torch.bfloat16)
    names = ["q_proj.weight", "k_proj.weight", "v_proj.weight", "q_norm.weight", "k_norm.weight"]
    if norm_type == "layernorm":
        names += ["q_norm.bias", "k_norm.bias"]
    x = torch.randn(2, S, E)
    gy = torch.randn(2, S, E)
    grads, outs = [], []
    from trinix_amd.kernels import attention_kernel as ak

    fused_q_calls = []
    apply = ak._HipAttnQNormFunction.apply
    monkeypatch.setattr(ak._HipAttnQNormFunction, "apply",
                        staticmethod(lambda *a: fused_q_calls.append(1) or apply(*a)))
    for layer, dev, dt in ((ref64, "cpu", torch.float64), (ref16, "cpu", torch.bfloat16), (hip, DEV, torch.bfloat16)):
        if layer is hip:  # the eager norm modules must not run on the fused path
            def refuse(self, x):
                raise AssertionError("eager qk-norm module called")
            monkeypatch.setattr(lb._QKRMSNorm, "forward", refuse)
            monkeypatch.setattr(lb._QKLayerNorm, "forward", refuse)
        xi = x.to(dev, dt).requires_grad_(True)
        y, _ = layer(xi)
        y.backward(gy.to(dev, dt))
        outs.append(y.detach().cpu().double())
        grads.append([xi.grad.cpu().double()] + [layer.get_parameter(n).grad.cpu().double() for n in names])
    t, e, h = grads
    if norm_type == "rmsnorm":  # q's norm ran in the attention prologue, k's in the fused kernel
        assert fused_q_calls, "the training step did not take the fused q-norm attention"
    assert (outs[2] - outs[0]).abs().max() <= 2 * (outs[1] - outs[0]).abs().max() + 2e-3 * outs[0].abs().max()
    for name, gh, gt, ge in zip(["x"] + names, h, t, e):
        scale = gt.abs().max().item()
        err_h, err_e = (gh - gt).abs().max().item(), (ge - gt).abs().max().item()
        assert err_h <= 2 * err_e + 2e-3 * scale, (name, err_h, err_e, scale)


def _rope_tables(q, S):
    emb = tx.FastRoPEPositionEmbedding(q.shape[-1], max_position_embeddings=S, base=500000.0).to(DEV)
    return emb(q, S)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("Sq", [150, 8])
@pytest.mark.parametrize("alibi", [False, True])
def test_q_norm_fused_into_attention_is_bitwise_the_two_kernel_path(D, dtype, rope, Sq, alibi, monkeypatch):
    """q's RoPE + RMSNorm in the attention kernel's prologue gives the
    output of qk_rmsnorm followed by the attention kernel, bit for bit (the
    prologue repeats qk_rmsnorm's rounding and its sum-of-squares order),
    with and without ALiBi (both are built with the fused norm)."""
    from trinix_amd.kernels import TritonAttentionKernel, rope_apply
    from trinix_amd.kernels import attention_kernel as ak

    monkeypatch.setattr(ak, "SPLITKV_ENABLED", False)  # short q: the same prefill kernel on both sides
    if D == 64:  # small D=64 grids take the key split, which the fused norm is not built with
        monkeypatch.setenv("TRINIX_ATTN_CFG", "4,2,64,1")
    g = torch.Generator().manual_seed(D + Sq + (7 if rope else 0))
    B, Sk, H, HKV = 2, 150, 4, 2
    q = (torch.randn(B, Sq, H, D, generator=g) * 3).to(DEV, dtype)
    k = torch.randn(B, Sk, HKV, D, generator=g).to(DEV, dtype)
    v = torch.randn(B, Sk, HKV, D, generator=g).to(DEV, dtype)
    w = (torch.rand(D, generator=g) + 0.5).to(DEV, dtype)
    eps = 1e-5
    kw = {}
    cos = sin = None
    if rope:
        cos, sin = _rope_tables(q, max(Sq, Sk))
        k = rope_apply(k, cos, sin)
        kw = dict(rotary_cos=cos, rotary_sin=sin, rotary_k=False)
    if alibi:
        kw["alibi_slopes"] = orc.alibi_slopes(H).to(DEV, torch.float32)
    ref = TritonAttentionKernel.apply(qk_rmsnorm(q, w, eps, cos, sin), k, v, causal=True,
                                      alibi_slopes=kw.get("alibi_slopes"))
    out = TritonAttentionKernel.apply(q, k, v, causal=True, q_norm_weight=w, q_norm_eps=eps, **kw)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("D,dtype", [(64, torch.float16), (128, torch.bfloat16)])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("alibi", [False, True])
def test_q_norm_fused_training_is_bitwise_the_two_kernel_path(D, dtype, rope, alibi, monkeypatch):
    """Gradients through q's RoPE + RMSNorm fused into the attention
    prologue: the kernel writes the normalised q it attends with, the
    attention backward runs on it and the qk-norm backward takes the
    gradient to the raw q and the norm weight.  Output and every gradient
    (q, k, v, weight) equal those of qk_rmsnorm, the RoPE of k and the
    attention as separate differentiable steps, bit for bit."""
    from trinix_amd.kernels.attention_kernel import attention
    from trinix_amd.kernels.rope_kernel import rotate

    if D == 64:  # the fused norm is built without the key split: the same kernel on both sides
        monkeypatch.setenv("TRINIX_ATTN_CFG", "4,2,64,1")
    g = torch.Generator().manual_seed(D + (3 if rope else 0) + (5 if alibi else 0))
    B, S, H, HKV = 2, 170, 4, 2
    q0 = (torch.randn(B, S, H, D, generator=g) * 2).to(DEV, dtype)
    k0 = torch.randn(B, S, HKV, D, generator=g).to(DEV, dtype)
    v0 = torch.randn(B, S, HKV, D, generator=g).to(DEV, dtype)
    w0 = (torch.rand(D, generator=g) + 0.5).to(DEV, dtype)
    do = torch.randn(B, S, H, D, generator=g).to(DEV, dtype)
    eps = 1e-5
    cos = sin = None
    if rope:
        cos, sin = _rope_tables(q0, S)
    slopes = orc.alibi_slopes(H).to(DEV, torch.float32) if alibi else None
    res = []
    for fused in (True, False):
        q, k, v, w = (t.clone().requires_grad_(True) for t in (q0, k0, v0, w0))
        if fused:
            out = attention(q, k, v, causal=True, alibi_slopes=slopes, rotary_cos=cos, rotary_sin=sin,
                            q_norm_weight=w, q_norm_eps=eps)
        else:
            qn = qk_rmsnorm(q, w, eps, cos, sin)
            kr = rotate(k, cos, sin) if rope else k
            out = attention(qn, kr, v, causal=True, alibi_slopes=slopes)
        out.backward(do)
        res.append([out.detach()] + [t.grad for t in (q, k, v, w)])
    for name, a, b in zip(("out", "dq", "dk", "dv", "dweight"), *res):
        assert torch.equal(a, b), name


def test_q_norm_fused_argument_errors():
    from trinix_amd.kernels import TritonAttentionKernel
    from trinix_amd.kernels.attention_kernel import attention

    q = torch.randn(1, 32, 2, 128, device=DEV, dtype=torch.bfloat16)
    w = torch.ones(128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        TritonAttentionKernel.apply(q.float(), q.float(), q.float(), q_norm_weight=w.float())
    with pytest.raises(ValueError):
        TritonAttentionKernel.apply(q, q, q, q_norm_weight=w[:64])
    q96 = torch.randn(1, 32, 2, 96, device=DEV, dtype=torch.bfloat16)  # padded to 128: no fused norm
    with pytest.raises(ValueError):
        TritonAttentionKernel.apply(q96, q96, q96, q_norm_weight=torch.ones(96, device=DEV, dtype=torch.bfloat16))
    qg = q.clone().requires_grad_(True)
    with pytest.raises(ValueError):  # differentiable too, but not with a mask or dropout
        attention(qg, q, q, attn_mask=torch.zeros(32, 32, device=DEV), q_norm_weight=w)
    with pytest.raises(ValueError):
        attention(qg, q, q, dropout_p=0.1, q_norm_weight=w)
    with pytest.raises(ValueError):  # built without the mask and dropout kernels
        TritonAttentionKernel.apply(q, q, q, attn_mask=torch.zeros(32, 32, device=DEV), q_norm_weight=w)
    with pytest.raises(ValueError):
        TritonAttentionKernel.apply(q, q, q, dropout_p=0.1, q_norm_weight=w)
    # ALiBi is built with the fused norm: same output as the two-kernel path
    slopes = torch.tensor([0.25, 0.0625], device=DEV)
    ref = TritonAttentionKernel.apply(qk_rmsnorm(q, w, 1e-6), q, q, causal=True, alibi_slopes=slopes)
    out = TritonAttentionKernel.apply(q, q, q, causal=True, alibi_slopes=slopes, q_norm_weight=w, q_norm_eps=1e-6)
    assert torch.equal(out, ref)
