"""Layer API tests (CPU): constructor/forward conventions of the reference
layers, parameter names (state_dict compatibility), and the eager
(kernel_type='pytorch') path against the oracle composition of projections,
RoPE / ALiBi / window and the restated eager attention."""
import pytest
import torch

import trinix_amd as tx
from oracle import attention_oracle as orc


def _proj(layer, name, x):
    lin = getattr(layer, name)
    return torch.nn.functional.linear(x, lin.weight, lin.bias)


def oracle_layer(layer, x, hkv, causal=False, rope=None, alibi=False, window=None, mask=None):
    """Reference semantics of the layer forward, built from oracle pieces."""
    B, S, _ = x.shape
    H, D = layer.num_heads, layer.head_dim
    if hasattr(layer, "qkv_proj"):
        qkv = _proj(layer, "qkv_proj", x).view(B, S, 3, H, D)
        q, k, v = qkv.unbind(2)
    else:
        q = _proj(layer, "q_proj", x).view(B, S, H, D)
        k = _proj(layer, "k_proj", x).view(B, S, hkv, D)
        v = _proj(layer, "v_proj", x).view(B, S, hkv, D)
    if rope is not None:
        cos, sin = orc.rope_tables(S, D, rope, x.dtype)
        q, k = orc.apply_rope(q, cos, sin), orc.apply_rope(k, cos, sin)
    out = orc.functional_attention(q, k, v, attn_mask=mask, softmax_scale=D ** -0.5, causal=causal,
                                   window_size=window, alibi_slopes=orc.alibi_slopes(H) if alibi else None)
    return torch.nn.functional.linear(out.reshape(B, S, H * D), layer.o_proj.weight, layer.o_proj.bias)


@pytest.mark.parametrize("kind", ["mha", "gqa", "mqa", "mhsa"])
@pytest.mark.parametrize("feat", ["plain", "causal_rope", "alibi", "window"])
def test_eager_layer_matches_oracle(kind, feat):
    torch.manual_seed(0)
    E, H = 128, 4
    kw = dict(kernel_type="pytorch")
    if feat == "causal_rope":
        kw.update(causal=True, position_method="rope", rope_base=500000.0)
    elif feat == "alibi":
        kw.update(position_method="alibi")
    elif feat == "window":
        kw.update(causal=True, use_sliding_window=True, sliding_window_size=5)
    if kind == "mha":
        layer, hkv = tx.FastMultiHeadAttention(E, H, **kw), H
    elif kind == "gqa":
        layer, hkv = tx.FastGroupedQueryAttention(E, H, 2, **kw), 2
    elif kind == "mqa":
        layer, hkv = tx.FastMultiQueryAttention(E, H, **kw), 1
    else:
        layer, hkv = tx.FastMultiHeadSelfAttention(E, H, **kw), H
    x = torch.randn(2, 23, E)
    out = layer(x)
    if isinstance(out, tuple):
        out = out[0]
    ref = oracle_layer(layer, x, hkv, causal=kw.get("causal", False),
                       rope=kw.get("rope_base") if feat == "causal_rope" else None,
                       alibi=feat == "alibi", window=(5, 0) if feat == "window" else None)
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)
    assert torch.isfinite(out).all()  # the reference's window mask is NaN here (0 * -inf)


def test_return_conventions_and_caches():
    x = torch.randn(1, 9, 64)
    mha = tx.FastMultiHeadAttention(64, 4, kernel_type="pytorch")
    assert isinstance(mha(x), torch.Tensor)
    o, (k, v) = mha(x, use_cache=True)
    assert k.shape == (1, 4, 9, 16) and v.shape == (1, 4, 9, 16)
    gqa = tx.FastGroupedQueryAttention(64, 4, 2, kernel_type="pytorch")
    o, pkv = gqa(x)
    assert pkv is None
    o, (k, v) = gqa(x, use_cache=True)
    assert k.shape == (1, 2, 9, 16)
    mqa = tx.FastMultiQueryAttention(64, 4, kernel_type="pytorch")
    assert isinstance(mqa(x), torch.Tensor)
    o, (k, v) = mqa(x, use_cache=True)
    assert k.shape == (1, 1, 9, 16)
    # a cache is consumed by the next call
    o2, (k2, v2) = mqa(x[:, :1], past_key_value=(k, v), use_cache=True)
    assert k2.shape == (1, 1, 10, 16)


def test_state_dict_names_match_reference():
    assert set(tx.FastMultiHeadAttention(64, 4).state_dict()) == {
        f"{p}_proj.{w}" for p in "qkvo" for w in ("weight", "bias")}
    assert set(tx.FastMultiHeadSelfAttention(64, 4, bias=False).state_dict()) == {"qkv_proj.weight", "o_proj.weight"}
    sd = tx.FastGroupedQueryAttention(64, 4, 2, qk_norm=True).state_dict()
    assert {"q_norm.weight", "k_norm.weight"} <= set(sd)
    assert tx.FastGroupedQueryAttention(64, 4, 2).k_proj.weight.shape == (32, 64)
    assert tx.FastMultiQueryAttention(64, 4).k_proj.weight.shape == (16, 64)
    # non-persistent buffers stay out of the state dict, as in the reference
    assert "position_embedding.inv_freq" not in tx.FastMultiHeadAttention(64, 4, position_method="rope").state_dict()


def test_constructor_errors_match_reference():
    with pytest.raises(AssertionError):
        tx.FastMultiHeadAttention(65, 4)
    with pytest.raises(AssertionError):
        tx.FastGroupedQueryAttention(64, 4, 3)
    with pytest.raises(AssertionError):
        tx.FastMultiHeadAttention(64, 4, position_method="bogus")
    with pytest.raises(TypeError):
        tx.FastMultiHeadAttention(64, 4, position_method=3)
    with pytest.raises(ValueError):
        tx.FastMultiHeadAttention(64, 4, qk_norm=True, qk_norm_type="batchnorm")


def test_default_kernel_type_is_kept_and_cpu_tensors_run_eager():
    layer = tx.FastMultiHeadAttention(64, 4)
    assert layer.kernel_type == "flash"
    out = layer(torch.randn(1, 5, 64))  # CPU input: eager path, as the reference layer on CPU
    assert out.shape == (1, 5, 64)


def test_rope_embedding_tables_and_alibi_module():
    rope = tx.FastRoPEPositionEmbedding(16, base=10000.0)
    cos, sin = rope(torch.zeros(1, 7, 2, 16, dtype=torch.bfloat16), 7)
    c2, s2 = orc.rope_tables(7, 16, 10000.0, torch.bfloat16)
    assert torch.equal(cos, c2) and torch.equal(sin, s2)
    alibi = tx.FastALiBiPositionEmbedding(8)
    assert torch.equal(alibi.slopes, orc.alibi_slopes(8))
    b = alibi(5, batch_size=2)
    assert b.shape == (2, 8, 5, 5)
    assert torch.equal(b[0], orc.alibi_bias(5, 5, orc.alibi_slopes(8)))


def test_custom_position_module_calling_conventions():
    """User position modules are called as the reference layers call them
    (base.py:239-285): the full argument list, else (q, k), else no
    arguments; results are (q, k, bias), (q, k) or a bias."""
    import torch.nn as nn

    E, H, S = 32, 2, 6
    bias = torch.randn(S, S)

    class Full(nn.Module):
        def forward(self, q, k, sq, sk, bs, pos):
            return q * 2, k, bias

    class QKOnly(nn.Module):
        def forward(self, q, k):
            return q * 3, k * 0.5

    class NoArgs(nn.Module):
        def forward(self):
            return bias

    torch.manual_seed(0)
    x = torch.randn(1, S, E)
    plain = tx.FastMultiHeadAttention(E, H, kernel_type="pytorch")
    for mod, qs, ks, b in ((Full(), 2.0, 1.0, bias), (QKOnly(), 3.0, 0.5, None), (NoArgs(), 1.0, 1.0, bias)):
        layer = tx.FastMultiHeadAttention(E, H, kernel_type="pytorch", position_method=mod)
        layer.load_state_dict(plain.state_dict(), strict=False)
        q = layer.q_proj(x).view(1, S, H, -1) * qs
        k = layer.k_proj(x).view(1, S, H, -1) * ks
        v = layer.v_proj(x).view(1, S, H, -1)
        w = torch.einsum("bihd,bjhd->bhij", q, k) * layer.scale
        if b is not None:
            w = w + b
        ref = layer.o_proj(torch.einsum("bhij,bjhd->bihd", w.softmax(-1), v).reshape(1, S, E))
        assert torch.allclose(layer(x), ref, atol=1e-5, rtol=1e-5), type(mod).__name__
