"""ALiBi bias on MI355X through ``libtrinix_attn.so``.

Drop-in for ``TritonALiBiKernel`` / ``TritonALiBiFunction`` (reference
``trinix/kernels/alibi_kernel.py:8-160``): ``bias[b, h, i, j] =
-slopes[h] * |i - j|`` of shape (batch, heads, seq, seq) in ``slopes.dtype``.
The kernel computes in fp32 (the reference's ``-slope * distance`` with fp32
distances) and writes one (heads, seq, seq) tensor; for batch > 1 the result
is that tensor expanded over the batch (same values, one copy in memory).
"""
from __future__ import annotations

import torch

from .. import _native as nat
from .attention_kernel import current_stream_ptr


def alibi_bias(slopes: torch.Tensor, batch_size: int, num_heads: int, seq_len: int) -> torch.Tensor:
    """(batch, heads, seq, seq) ALiBi bias computed by the HIP kernel."""
    if not slopes.is_cuda:
        raise ValueError("alibi_bias requires a GPU slopes tensor")
    if slopes.numel() < num_heads or num_heads <= 0 or seq_len <= 0 or batch_size <= 0:
        raise ValueError("alibi_bias: need num_heads slopes and positive sizes")
    s32 = slopes.reshape(-1)[:num_heads].to(torch.float32)
    out = torch.empty((num_heads, seq_len, seq_len), dtype=torch.float32, device=slopes.device)
    lib = nat.load_library()
    rc = lib.trinix_alibi_bias(s32.data_ptr(), s32.stride(0), num_heads, seq_len, out.data_ptr(), out.stride(0),
                               out.stride(1), current_stream_ptr(slopes.device))
    nat.check(rc, "trinix_alibi_bias")
    if slopes.dtype != torch.float32:
        out = out.to(slopes.dtype)
    return out.unsqueeze(0).expand(batch_size, -1, -1, -1)


class TritonALiBiFunction(torch.autograd.Function):
    """ALiBi bias as an autograd node: no input receives a gradient
    (reference ``alibi_kernel.py:93-124``)."""

    @staticmethod
    def forward(ctx, slopes, batch_size, num_heads, seq_len):
        return alibi_bias(slopes, batch_size, num_heads, seq_len)

    @staticmethod
    def backward(ctx, grad_output):
        return None, None, None, None


class TritonALiBiKernel:
    """ALiBi bias producer (name kept from the reference for drop-in use)."""

    @staticmethod
    def apply(slopes: torch.Tensor, batch_size: int, num_heads: int, seq_len: int) -> torch.Tensor:
        return TritonALiBiFunction.apply(slopes, batch_size, num_heads, seq_len)

    @staticmethod
    def is_available() -> bool:
        from .attention_kernel import TritonAttentionKernel

        return TritonAttentionKernel.is_available()
