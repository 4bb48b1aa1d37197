"""GPU tests of the fused qk-norm (``trinix_qk_norm``: RoPE + RMSNorm over
head_dim) against the oracle's restatement of the reference's eager path
(``orc.apply_rope`` then ``orc.qk_rms_norm``, trinix/layers/norm/rmsnorm.py:
62-75), and of the layers that use it.

Bar: the fp32 sum of squares is ordered differently from torch's reduction,
so the normalisation factor can differ by an ulp of fp32 and an output
element by an ulp or two of the dtype.  At least 99% of the elements must be
bit-identical to the oracle and every element within 2 ulps of it.
"""
import pytest
import torch

from oracle import attention_oracle as orc
import trinix_amd as tx
from trinix_amd.kernels import qk_rmsnorm

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


def test_qk_norm_layer_training_keeps_eager_gradients():
    torch.manual_seed(13)
    E, H, HKV, S = 512, 4, 2, 64
    layer = tx.FastGroupedQueryAttention(E, H, HKV, kernel_type="flash", position_method="rope", qk_norm=True,
                                         causal=True).to(DEV, torch.bfloat16)
    x = torch.randn(1, S, E, device=DEV).to(torch.bfloat16).requires_grad_(True)
    q = torch.empty(1, 1, H, E // H, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    assert not layer._fused_qk_norm_applies(q, q)
    out, _ = layer(x)
    out.float().sum().backward()
    assert layer.q_norm.weight.grad is not None and layer.k_norm.weight.grad is not None
    assert torch.isfinite(x.grad).all()


def _rope_tables(q, S):
    emb = tx.FastRoPEPositionEmbedding(q.shape[-1], max_position_embeddings=S, base=500000.0).to(DEV)
    return emb(q, S)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("Sq", [150, 8])
def test_q_norm_fused_into_attention_is_bitwise_the_two_kernel_path(D, dtype, rope, Sq, monkeypatch):
    """q's RoPE + RMSNorm in the attention kernel's prologue gives the
    output of qk_rmsnorm followed by the attention kernel, bit for bit (the
    prologue repeats qk_rmsnorm's rounding and its sum-of-squares order)."""
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
    ref = TritonAttentionKernel.apply(qk_rmsnorm(q, w, eps, cos, sin), k, v, causal=True)
    out = TritonAttentionKernel.apply(q, k, v, causal=True, q_norm_weight=w, q_norm_eps=eps, **kw)
    assert torch.equal(out, ref)


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
    with pytest.raises(ValueError):
        attention(qg, q, q, q_norm_weight=w)
    with pytest.raises(ValueError):  # built without the mask and dropout kernels
        TritonAttentionKernel.apply(q, q, q, attn_mask=torch.zeros(32, 32, device=DEV), q_norm_weight=w)
    with pytest.raises(ValueError):
        TritonAttentionKernel.apply(q, q, q, dropout_p=0.1, q_norm_weight=w)
    # ALiBi is built with the fused norm: same output as the two-kernel path
    slopes = torch.tensor([0.25, 0.0625], device=DEV)
    ref = TritonAttentionKernel.apply(qk_rmsnorm(q, w, 1e-6), q, q, causal=True, alibi_slopes=slopes)
    out = TritonAttentionKernel.apply(q, q, q, causal=True, alibi_slopes=slopes, q_norm_weight=w, q_norm_eps=1e-6)
    assert torch.equal(out, ref)
