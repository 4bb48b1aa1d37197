"""qk-norm (RMSNorm over head_dim) fused with RoPE, through ``libtrinix_attn.so``.

The attention layers normalise q and k over head_dim after RoPE when built
with ``qk_norm=True`` (reference ``trinix/layers/attention/base.py:163-176``,
``grouped_query_attention.py:171-177``).  For head_dim <= 2048 the
reference's ``FastRMSNorm`` always takes its PyTorch path
(``trinix/layers/norm/rmsnorm.py:62-75``):
``weight * (x.float() * rsqrt(mean(x.float()**2) + eps)).to(x.dtype)``.
``qk_rmsnorm`` computes RoPE (optional) and that norm in one pass per tensor,
with the eager order of roundings; only the fp32 sum of squares is ordered
differently, so an element can differ from eager by one ulp of the dtype.
There is no backward: the layers use it where no gradient is needed.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _native as nat
from .attention_kernel import _DTYPE_CODE, current_stream_ptr
from .rope_kernel import _table, check_positions

QK_NORM_HEAD_DIMS = (16, 32, 64, 128, 256)


def qk_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when ``trinix_qk_norm`` covers (x, weight): GPU bf16/fp16 x of
    head_dim in QK_NORM_HEAD_DIMS, weight of the same dtype and length."""
    return (x.is_cuda and x.dim() == 4 and x.dtype in (torch.bfloat16, torch.float16)
            and weight.dtype == x.dtype and x.shape[-1] in QK_NORM_HEAD_DIMS
            and weight.numel() == x.shape[-1])


def qk_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, cos: Optional[torch.Tensor] = None,
               sin: Optional[torch.Tensor] = None, position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm over the last dim of a (B, S, H, D) tensor, after RoPE when
    cos/sin are given (row of the tables = position_ids[b, s] or s).
    Returns a new contiguous (B, S, H, D) tensor."""
    if not qk_norm_supported(x, weight):
        raise ValueError(f"qk_rmsnorm: unsupported input {tuple(x.shape)} {x.dtype} / weight {weight.dtype}")
    B, S, H, D = x.shape
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any(st % 8 for st in x.stride()[:3]):
        x = x.contiguous()
    w = weight.detach()
    if not w.is_contiguous() or w.data_ptr() % 16:
        w = w.contiguous()
    c = s = pos = None
    if cos is not None or sin is not None:
        if cos is None or sin is None:
            raise ValueError("cos and sin must be given together")
        c, s = _table(cos, x), _table(sin, x)
        if c.stride(0) != s.stride(0):
            c, s = c.contiguous(), s.contiguous()
        if c.shape[-1] < D // 2:
            raise ValueError("cos/sin tables narrower than head_dim/2")
        if position_ids is not None:
            pos = position_ids.to(device=x.device, dtype=torch.int64).expand(B, S).contiguous()
            check_positions(pos, c.shape[0])
        elif c.shape[0] < S:
            raise ValueError("cos/sin tables shorter than the sequence")
    out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    rc = nat.load_library().trinix_qk_norm(
        x.data_ptr(), (ctypes.c_int64 * 4)(*x.stride()), out.data_ptr(), (ctypes.c_int64 * 4)(*out.stride()),
        B, S, H, D, _DTYPE_CODE[x.dtype], w.data_ptr(), float(eps),
        c.data_ptr() if c is not None else None, s.data_ptr() if s is not None else None,
        c.stride(0) if c is not None else 0, c.shape[0] if c is not None else 0,
        pos.data_ptr() if pos is not None else None,
        current_stream_ptr(x.device))
    nat.check(rc, "trinix_qk_norm")
    return out
