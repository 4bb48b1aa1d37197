"""GPU tests of the layers on the HIP path (kernel_type 'flash' / 'triton'):
the same layer weights give the reference semantics (oracle composition on
the CPU) in fp32, and match the eager path in bf16 within the stated
tolerance; caches hold the rotated keys."""
import pytest
import torch

import trinix_amd as tx
from oracle import attention_oracle as orc

from test_layers import oracle_layer

pytestmark = pytest.mark.gpu


def _make(kind, E, H, **kw):
    if kind == "mha":
        return tx.FastMultiHeadAttention(E, H, **kw), H
    if kind == "gqa":
        return tx.FastGroupedQueryAttention(E, H, 2, **kw), 2
    if kind == "mqa":
        return tx.FastMultiQueryAttention(E, H, **kw), 1
    return tx.FastMultiHeadSelfAttention(E, H, **kw), H


@pytest.mark.parametrize("kernel_type", ["flash", "triton"])
@pytest.mark.parametrize("kind", ["mha", "gqa", "mqa", "mhsa"])
@pytest.mark.parametrize("feat", ["plain", "causal_rope", "alibi", "window"])
def test_hip_layer_fp32_matches_oracle(kind, feat, kernel_type):
    torch.manual_seed(1)
    E, H = 256, 4  # head_dim 64
    kw = dict(kernel_type=kernel_type)
    if feat == "causal_rope":
        kw.update(causal=True, position_method="rope", rope_base=10000.0)
    elif feat == "alibi":
        kw.update(position_method="alibi")
    elif feat == "window":
        kw.update(causal=True, use_sliding_window=True, sliding_window_size=17)
    layer, hkv = _make(kind, E, H, **kw)
    x = torch.randn(2, 150, E)
    ref = oracle_layer(layer, x, hkv, causal=kw.get("causal", False),
                       rope=10000.0 if feat == "causal_rope" else None, alibi=feat == "alibi",
                       window=(17, 0) if feat == "window" else None)
    out = layer.cuda()(x.cuda())
    if isinstance(out, tuple):
        out = out[0]
    rel = ((out.cpu() - ref).abs().max() / ref.abs().max()).item()
    # the north star's fp32 bar; the layer's projections run as fp32 GEMMs on
    # the GPU and on the host (measured 0.5-1.2e-6 across these cases)
    assert rel <= 1e-5, rel


def test_hip_gqa_bf16_llama_block_matches_eager_and_cache():
    torch.manual_seed(2)
    E, H, HKV = 1024, 8, 2  # head_dim 128
    hip = tx.FastGroupedQueryAttention(E, H, HKV, causal=True, position_method="rope", rope_base=500000.0,
                                       kernel_type="flash").cuda().to(torch.bfloat16)
    eager = tx.FastGroupedQueryAttention(E, H, HKV, causal=True, position_method="rope", rope_base=500000.0,
                                         kernel_type="pytorch").cuda().to(torch.bfloat16)
    eager.load_state_dict(hip.state_dict())
    x = torch.randn(2, 300, E, device="cuda").to(torch.bfloat16)
    o1, (k1, v1) = hip(x, use_cache=True)
    o2, (k2, v2) = eager(x, use_cache=True)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)  # rotated keys bit-identical (RoPE kernel)
    d = (o1.float() - o2.float()).abs()
    scale = o2.float().abs().max().item()
    assert d.max().item() <= 2e-2 * max(1.0, scale) and d.mean().item() <= 2e-3 * max(1.0, scale)


def test_hip_layer_attention_mask_and_zero_attn():
    torch.manual_seed(3)
    E, H, S = 256, 4, 96
    layer = tx.FastMultiHeadAttention(E, H, kernel_type="flash", add_zero_attn=True)
    x = torch.randn(1, S, E)
    m = torch.zeros(1, H, S, S)
    m[..., :, 40:] = float("-inf")
    out = layer.cuda()(x.cuda(), attention_mask=m.cuda())
    eager = tx.FastMultiHeadAttention(E, H, kernel_type="pytorch", add_zero_attn=True)
    eager.load_state_dict(layer.state_dict())
    ref = eager(x, attention_mask=m)
    assert torch.allclose(out.cpu(), ref, atol=1e-4, rtol=1e-4)


def test_functional_forward_attention_gqa_unrepeated():
    torch.manual_seed(4)
    layer = tx.FastGroupedQueryAttention(256, 4, 2, kernel_type="flash", causal=True)
    q = torch.randn(1, 64, 4, 64, device="cuda")
    k = torch.randn(1, 64, 2, 64, device="cuda")
    v = torch.randn(1, 64, 2, 64, device="cuda")
    a = layer.forward_attention(q, k, v)
    b = layer.forward_attention(q, layer._tile_kv_heads(k.transpose(1, 2), 2).transpose(1, 2),
                                layer._tile_kv_heads(v.transpose(1, 2), 2).transpose(1, 2))
    assert torch.equal(a, b)
    ref = orc.functional_attention(q.cpu(), k.cpu(), v.cpu(), causal=True)
    assert ((a.cpu() - ref).abs().max() / ref.abs().max()).item() <= 1e-5


def _layer_case(seed):
    import random

    r = random.Random(70_000 + seed)
    kind = r.choice(["mha", "gqa", "mqa", "mhsa"])
    D, H = r.choice([64, 128]), r.choice([2, 4])
    dtype = r.choice([torch.float32, torch.bfloat16])
    kw = dict(causal=r.random() < 0.6)
    pm = r.choice(["none", "rope", "alibi"])
    kw["position_method"] = pm
    if pm == "rope":
        kw["rope_base"] = r.choice([10000.0, 500000.0])
    if r.random() < 0.3 and kw["causal"]:
        kw.update(use_sliding_window=True, sliding_window_size=r.randint(4, 60))
    if r.random() < 0.4 and kind != "mhsa":
        kw.update(qk_norm=True, qk_norm_type=r.choice(["rmsnorm", "layernorm"]))
    return kind, D * H, H, dtype, kw, r.choice([1, 2]), r.randint(2, 200), r.random() < 0.5, r.random() < 0.5


@pytest.mark.parametrize("seed", list(range(30)))
def test_random_layer_flash_matches_pytorch_backend(seed):
    """Seeded random layer configurations (class, head_dim, heads, dtype,
    causal, RoPE / ALiBi, sliding window, qk-norm type): the HIP path
    (kernel_type='flash') against the layer's own eager backend
    (kernel_type='pytorch', the restated reference path) with the same
    weights.  Forward output, and either the gradients of the input and of
    every parameter (training) or three cached decode steps after a prefill
    (inference).  Bars: 1e-4 (fp32) / 3e-2 (bf16) of max(1, |out|) for
    outputs; 2e-4 / 5e-2 of the largest gradient for gradients (the key
    bias's own gradient is 0 up to rounding)."""
    kind, E, H, dtype, kw, B, S, train, decode = _layer_case(seed)
    print(f"seed {seed}: {kind} E{E} H{H} {dtype} B{B} S{S} train={train} {kw}", flush=True)
    torch.manual_seed(seed)
    hip = _make(kind, E, H, kernel_type="flash", **kw)[0].cuda().to(dtype)
    ref = _make(kind, E, H, kernel_type="pytorch", **kw)[0].cuda().to(dtype)
    ref.load_state_dict(hip.state_dict())
    x = torch.randn(B, S, E, device="cuda", dtype=dtype)
    tol, gtol = (1e-4, 2e-4) if dtype == torch.float32 else (3e-2, 5e-2)
    res = []
    for m in (hip, ref):
        xx = x.detach().clone().requires_grad_(train)
        o = m(xx)
        o = o[0] if isinstance(o, tuple) else o
        grads = None
        if train:
            o.float().square().mean().backward()
            grads = [xx.grad.float()] + [p.grad.float() for p in m.parameters() if p.grad is not None]
        res.append((o.detach().float(), grads))
    (oh, gh), (orf, gr) = res
    assert (oh - orf).abs().max().item() <= tol * max(1.0, orf.abs().max().item())
    if train:
        assert len(gh) == len(gr)
        assert (gh[0] - gr[0]).abs().max().item() <= gtol * gr[0].abs().max().item()
        pscale = max(t.abs().max().item() for t in gr[1:])
        for a, b in zip(gh[1:], gr[1:]):
            assert (a - b).abs().max().item() <= gtol * pscale
    elif decode and kind != "mhsa" and S > 4:
        steps = []
        with torch.no_grad():
            for m in (hip, ref):
                _, cache = m(x[:, :-3], use_cache=True)[:2]
                outs = []
                for t in range(3):
                    o1, cache = m(x[:, S - 3 + t:S - 2 + t], past_key_value=cache, use_cache=True)[:2]
                    outs.append(o1.float())
                steps.append(torch.cat(outs, 1))
        assert (steps[0] - steps[1]).abs().max().item() <= tol * max(1.0, steps[1].abs().max().item())
