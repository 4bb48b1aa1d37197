"""Rotary position embedding on MI355X through ``libtrinix_attn.so``.

Drop-in for ``TritonRoPEKernel`` (reference
``trinix/kernels/rope_kernel.py:180-222``) and the eager
``_apply_rope_pytorch`` / ``_apply_rope_with_position_ids``
(``trinix/layers/embeddings/rope.py:111-134``): ``x*cos + rotate_half(x)*sin``
with ``rotate_half(x) = cat(-x2, x1)``, every product and the sum rounded to
the tensor dtype exactly as eager PyTorch rounds them, so results are
bit-identical to the eager path.  Unlike the reference Triton kernel, strides
of ``x`` are honoured (its dim stride must be 1).
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from .. import _native as nat
from .attention_kernel import _DTYPE_CODE, current_stream_ptr


def _table(t: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """cos/sin table as 2-D (rows, >= D/2) in x's dtype/device, unit dim stride."""
    if t.dim() > 2:
        t = t.reshape(-1, t.shape[-1])
    t = t.to(device=x.device, dtype=x.dtype)
    if t.stride(-1) != 1 or t.data_ptr() % 16 or t.stride(0) % 8:
        t = t.contiguous()
    return t


def check_positions(pos: torch.Tensor, rows: int) -> None:
    """Reject position ids outside the cos/sin tables (reference: indexing
    ``cos[position_ids]`` raises).  Reading them needs a device-to-host copy,
    which a stream under graph capture does not allow: there the check is
    skipped and the kernels clamp ids into [0, rows) instead."""
    if torch.cuda.is_current_stream_capturing():
        return
    if int(pos.min()) < 0 or int(pos.max()) >= rows:
        raise ValueError("position_ids out of range of the cos/sin tables")


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               position_ids: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RoPE on one (B, S, H, D) tensor; row of cos/sin = position_ids[b, s] or s."""
    if not x.is_cuda:
        raise ValueError("rope_apply requires GPU tensors")
    if x.dim() != 4:
        raise ValueError(f"Expected (batch, seq, heads, head_dim), got {tuple(x.shape)}")
    if x.dtype not in _DTYPE_CODE:
        raise ValueError(f"Unsupported dtype {x.dtype}")
    B, S, H, D = x.shape
    if D % 2:
        raise ValueError("RoPE needs an even head_dim")
    if x.stride(-1) != 1:
        x = x.contiguous()
    c = _table(cos, x)
    s = _table(sin, x)
    if c.stride(0) != s.stride(0):
        c, s = c.contiguous(), s.contiguous()
    if c.shape[-1] < D // 2:
        raise ValueError("cos/sin tables narrower than head_dim/2")
    pos = None
    if position_ids is not None:
        pos = position_ids.to(device=x.device, dtype=torch.int64).expand(B, S).contiguous()
        check_positions(pos, c.shape[0])
    elif c.shape[0] < S:
        raise ValueError("cos/sin tables shorter than the sequence")
    if out is None:
        out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    xs = (ctypes.c_int64 * 4)(*x.stride())
    os_ = (ctypes.c_int64 * 4)(*out.stride())
    lib = nat.load_library()
    rc = lib.trinix_rope_apply(x.data_ptr(), xs, out.data_ptr(), os_, B, S, H, D, _DTYPE_CODE[x.dtype],
                               c.data_ptr(), s.data_ptr(), c.stride(0), c.shape[0],
                               pos.data_ptr() if pos is not None else None,
                               current_stream_ptr(x.device))
    nat.check(rc, "trinix_rope_apply")
    return out


def rope_template(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """The arguments ``rope_apply(x, cos, sin)`` passes to
    ``trinix_rope_apply`` apart from its data pointers: (x strides, out
    strides, B, S, H, D, table row stride, table rows, in_place), where
    in_place says that x and the tables are read as given (no copy, no
    conversion), which a cached launch needs."""
    B, S, H, D = x.shape
    c, s = _table(cos, x), _table(sin, x)
    in_place = (x.stride(-1) == 1 and c is cos and s is sin and c.stride(0) == s.stride(0) and c.dim() == 2
                and c.shape[-1] >= D // 2 and c.shape[0] >= S)
    out_stride = (S * H * D, H * D, D, 1)
    return ((ctypes.c_int64 * 4)(*x.stride()), (ctypes.c_int64 * 4)(*out_stride), B, S, H, D, c.stride(0),
            c.shape[0], in_place)


class _RoPEFunction(torch.autograd.Function):
    """RoPE of one tensor; the backward is the rotation by -theta."""

    @staticmethod
    def forward(ctx, x, cos, sin, position_ids):
        ctx.save_for_backward(cos, sin)
        ctx.position_ids = position_ids
        return rope_apply(x, cos, sin, position_ids)

    @staticmethod
    def backward(ctx, grad):
        cos, sin = ctx.saved_tensors
        return rope_apply(grad, cos, -sin, ctx.position_ids), None, None, None


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
           position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``rope_apply`` that records the inverse rotation for autograd when x
    requires a gradient."""
    if torch.is_grad_enabled() and x.requires_grad:
        return _RoPEFunction.apply(x, cos, sin, position_ids)
    return rope_apply(x, cos, sin, position_ids)


class TritonRoPEKernel:
    """RoPE on q and k (name kept from the reference for drop-in use)."""

    @staticmethod
    def is_available() -> bool:
        from .attention_kernel import TritonAttentionKernel

        return TritonAttentionKernel.is_available()

    @staticmethod
    def apply(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
              position_ids: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        return TritonRoPEFunction.apply(q, k, cos, sin, position_ids)


class TritonRoPEFunction(torch.autograd.Function):
    """RoPE on q and k with the reference's backward (``rope_kernel.py:134-177``):
    the gradient of a rotation by +theta is the rotation by -theta, i.e. the
    same kernel with sin negated.  cos/sin receive no gradient."""

    @staticmethod
    def forward(ctx, q, k, cos, sin, position_ids=None):
        ctx.save_for_backward(cos, sin)
        ctx.position_ids = position_ids
        return rope_apply(q, cos, sin, position_ids), rope_apply(k, cos, sin, position_ids)

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        cos, sin = ctx.saved_tensors
        neg = -sin
        gq = rope_apply(grad_q, cos, neg, ctx.position_ids) if grad_q is not None else None
        gk = rope_apply(grad_k, cos, neg, ctx.position_ids) if grad_k is not None else None
        return gq, gk, None, None, None
