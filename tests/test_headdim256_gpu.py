"""GPU parity tests at head_dim 256 (and head dims padded up to it).

The reference pads head_dim to the next power of two
(``trinix/kernels/utils.py:107``, ``BLOCK_DMODEL = next_power_of_2``), so
D = 256 models run on its Triton path.  Here the forward kernels are built
for D = 256 (one wavefront per SIMD, 128 KiB of LDS per workgroup); D in
(128, 256) is zero-padded to 256.  Same oracle and bar as the other parity
tests.  D = 256 is differentiable through the generic backward kernels
(gradients tested in test_attn_bwd_gpu.py).
"""
import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func
from test_attn_gpu import assert_parity, assert_parity_or_more_accurate, oracle_on, rand

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # (B, Sq, Sk, Hq, Hkv, D, causal, window)
    (1, 300, 300, 4, 2, 256, True, None),
    (2, 130, 130, 2, 2, 256, False, None),
    (1, 200, 333, 4, 1, 256, False, (40, 17)),
    (1, 257, 257, 2, 2, 192, True, None),
    (1, 3, 900, 4, 2, 256, False, None),  # decode-shaped: prefill kernel (split-KV is built for D <= 128)
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_head_dim_256_shapes(case, dtype):
    B, Sq, Sk, Hq, Hkv, D, causal, window = case
    print(f"d256 case {case} {dtype}", flush=True)
    q, k, v = rand((B, Sq, Hq, D), dtype, 201), rand((B, Sk, Hkv, D), dtype, 202), rand((B, Sk, Hkv, D), dtype, 203)
    out = triton_attn_func(q, k, v, causal=causal, window_size=window)
    ref = oracle_on(q, k, v, causal=causal, window_size=window)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), causal=causal, window_size=window)
    assert_parity_or_more_accurate(out, ref, x64, dtype, str(case))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_head_dim_256_alibi_mask_rope_lse(dtype):
    B, S, H, D = 2, 192, 4, 256
    q, k, v = rand((B, S, H, D), dtype, 211), rand((B, S, H, D), dtype, 212), rand((B, S, H, D), dtype, 213)
    g = torch.Generator().manual_seed(214)
    m = torch.randn(S, S, generator=g)
    m[torch.rand(S, S, generator=g) < 0.2] = float("-inf")
    m[:, 0] = 0
    slopes = orc.alibi_slopes(H)
    out = triton_attn_func(q, k, v, attn_mask=m.to(DEV), alibi_slopes=slopes.to(DEV), causal=True)
    ref = oracle_on(q, k, v, attn_mask=m, alibi_slopes=slopes, causal=True)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), attn_mask=m, alibi_slopes=slopes, causal=True)
    assert_parity_or_more_accurate(out, ref, x64, dtype, "alibi+mask")
    cos, sin = orc.rope_tables(S, D, 10000.0, dtype)
    out, lse = triton_attn_func(q, k, v, causal=True, rotary_cos=cos.to(DEV), rotary_sin=sin.to(DEV),
                                return_lse=True)
    qr, kr = orc.apply_rope(q.cpu(), cos, sin), orc.apply_rope(k.cpu(), cos, sin)
    assert_parity(out, orc.functional_attention(qr, kr, v.cpu(), causal=True), dtype, "fused rope")
    s = torch.einsum("bihd,bjhd->bhij", qr.double(), kr.double()) * D ** -0.5
    s.masked_fill_(torch.triu(torch.ones(S, S), 1).bool(), float("-inf"))
    assert torch.allclose(lse.cpu().double(), torch.logsumexp(s, dim=-1), atol=2e-3, rtol=1e-4)


def test_head_dim_256_with_grad_is_differentiable():
    q, k, v = (rand((1, 64, 2, 256), torch.bfloat16, 221 + i).requires_grad_(True) for i in range(3))
    out = triton_attn_func(q, k, v, causal=True)
    assert out.grad_fn is not None
    assert_parity(out.detach(), oracle_on(q.detach(), k.detach(), v.detach(), causal=True), torch.bfloat16,
                  "d256 grad")
