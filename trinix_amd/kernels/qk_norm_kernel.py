"""qk-norm (RMSNorm or LayerNorm over head_dim) fused with RoPE, forward and
backward, through ``libtrinix_attn.so``.

The attention layers normalise q and k over head_dim after RoPE when built
with ``qk_norm=True`` (reference ``trinix/layers/attention/base.py:163-176``,
``grouped_query_attention.py:171-177``).  For these head dims the
reference's norm modules take their PyTorch paths:
- ``FastRMSNorm`` (``trinix/layers/norm/rmsnorm.py:62-75``):
  ``weight * (x.float() * rsqrt(mean(x.float()**2) + eps)).to(x.dtype)``;
- ``FastLayerNorm`` (``trinix/layers/norm/layernorm.py:83-88``):
  ``F.layer_norm(x, (D,), weight.to(x.dtype), bias.to(x.dtype), eps)``.
``qk_rmsnorm`` / ``qk_layernorm`` compute RoPE (optional) and the norm in one
pass per tensor, with the eager order of roundings; only the fp32 reductions
are ordered differently, so an element can differ from eager by one ulp of
the dtype.  When a gradient is needed they run as an autograd Function whose
backward (``trinix_qk_norm_bwd``) gives the gradients eager autograd gives
through the RoPE and the norm: dx, dweight and (LayerNorm) dbias.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from .. import _native as nat
from .attention_kernel import _DTYPE_CODE, current_stream_ptr
from .rope_kernel import _table, check_positions

QK_NORM_HEAD_DIMS = (16, 32, 64, 128, 256)
NORM_RMS, NORM_LAYER = nat.TRINIX_NORM_RMS, nat.TRINIX_NORM_LAYER
# at most this many workgroups (rows of dweight partial sums) in a backward
_MAX_PARTIAL_ROWS = 1024


def qk_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when the fused kernels cover (x, weight): GPU bf16/fp16 x of
    head_dim in QK_NORM_HEAD_DIMS, weight of the same dtype and length."""
    return (x.is_cuda and x.dim() == 4 and x.dtype in (torch.bfloat16, torch.float16)
            and weight.dtype == x.dtype and x.shape[-1] in QK_NORM_HEAD_DIMS
            and weight.numel() == x.shape[-1])


def _rows_ok(t: torch.Tensor) -> bool:
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(st % 8 == 0 for st in t.stride()[:3])


def _param(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def _tables(x: torch.Tensor, cos, sin, position_ids):
    """(cos, sin, positions) as the kernels read them, or Nones."""
    if cos is None and sin is None:
        return None, None, None
    if cos is None or sin is None:
        raise ValueError("cos and sin must be given together")
    B, S, _, D = x.shape
    c, s = _table(cos, x), _table(sin, x)
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
    return c, s, pos


def _strides(t: torch.Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


def _table_args(c, s, pos):
    return (c.data_ptr() if c is not None else None, s.data_ptr() if s is not None else None,
            c.stride(0) if c is not None else 0, c.shape[0] if c is not None else 0,
            pos.data_ptr() if pos is not None else None)


def _forward(x, w, b, eps, c, s, pos, norm: int) -> torch.Tensor:
    B, S, H, D = x.shape
    out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    lib = nat.load_library()
    if norm == NORM_RMS:
        rc = lib.trinix_qk_norm(x.data_ptr(), _strides(x), out.data_ptr(), _strides(out), B, S, H, D,
                                _DTYPE_CODE[x.dtype], w.data_ptr(), float(eps), *_table_args(c, s, pos),
                                current_stream_ptr(x.device))
        nat.check(rc, "trinix_qk_norm")
    else:
        rc = lib.trinix_qk_layernorm(x.data_ptr(), _strides(x), out.data_ptr(), _strides(out), B, S, H, D,
                                     _DTYPE_CODE[x.dtype], w.data_ptr(), b.data_ptr(), float(eps),
                                     *_table_args(c, s, pos), current_stream_ptr(x.device))
        nat.check(rc, "trinix_qk_layernorm")
    return out


def partial_rows(rows: int, head_dim: int) -> int:
    """Workgroups (rows of dweight partial sums) of a backward over ``rows``
    rows: one per 256/(head_dim/16) rows, at most 1024."""
    per = 256 // (head_dim // 16)
    return max(1, min(_MAX_PARTIAL_ROWS, -(-rows // per)))


def _backward(x, dout, w, eps, c, s, pos, norm: int) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """(dx, dweight, dbias) in x's dtype; dbias is None for RMSNorm."""
    B, S, H, D = x.shape
    if not _rows_ok(dout):
        dout = dout.contiguous()
    dx = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    nblk = partial_rows(B * S * H, D)
    dw_part = torch.empty((nblk, D), dtype=torch.float32, device=x.device)
    db_part = torch.empty((nblk, D), dtype=torch.float32, device=x.device) if norm == NORM_LAYER else None
    rc = nat.load_library().trinix_qk_norm_bwd(
        x.data_ptr(), _strides(x), dout.data_ptr(), _strides(dout), dx.data_ptr(), _strides(dx), B, S, H, D,
        _DTYPE_CODE[x.dtype], norm, w.data_ptr(), float(eps), *_table_args(c, s, pos), dw_part.data_ptr(),
        db_part.data_ptr() if db_part is not None else None, nblk, current_stream_ptr(x.device))
    nat.check(rc, "trinix_qk_norm_bwd")
    # fp32 column sums of the partial rows (a fixed order), rounded to the
    # weight's dtype like eager autograd's reduction of the per-row products
    dw = dw_part.sum(0).to(x.dtype)
    db = db_part.sum(0).to(x.dtype) if db_part is not None else None
    return dx, dw, db


class _QKNormFunction(torch.autograd.Function):
    """RoPE (optional) + RMSNorm / LayerNorm over head_dim with the backward
    of eager autograd through both (reference ``rope.py:111-118`` then
    ``rmsnorm.py:62-75`` / ``layernorm.py:83-88``)."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps, cos, sin, position_ids, norm):
        xc = x if _rows_ok(x) else x.contiguous()
        w = _param(weight)
        b = _param(bias) if bias is not None else None
        c, s, pos = _tables(xc, cos, sin, position_ids)
        out = _forward(xc, w, b, eps, c, s, pos, norm)
        ctx.save_for_backward(xc, w, c, s, pos)
        ctx.eps, ctx.norm, ctx.has_bias = eps, norm, bias is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        xc, w, c, s, pos = ctx.saved_tensors
        dx, dw, db = _backward(xc, dout, w, ctx.eps, c, s, pos, ctx.norm)
        return (dx if ctx.needs_input_grad[0] else None, dw if ctx.needs_input_grad[1] else None,
                db if ctx.has_bias and ctx.needs_input_grad[2] else None, None, None, None, None, None)


def _needs_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def _check(name: str, x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> None:
    if not qk_norm_supported(x, weight) or (bias is not None and (bias.dtype != x.dtype
                                                                   or bias.numel() != x.shape[-1])):
        raise ValueError(f"{name}: unsupported input {tuple(x.shape)} {x.dtype} / weight {weight.dtype}")


def qk_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, cos: Optional[torch.Tensor] = None,
               sin: Optional[torch.Tensor] = None, position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm over the last dim of a (B, S, H, D) tensor, after RoPE when
    cos/sin are given (row of the tables = position_ids[b, s] or s).
    Returns a new contiguous (B, S, H, D) tensor; differentiable in x and
    weight."""
    _check("qk_rmsnorm", x, weight)
    if _needs_grad(x, weight):
        return _QKNormFunction.apply(x, weight, None, eps, cos, sin, position_ids, NORM_RMS)
    xc = x if _rows_ok(x) else x.contiguous()
    return _forward(xc, _param(weight), None, eps, *_tables(xc, cos, sin, position_ids), NORM_RMS)


def qk_layernorm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float,
                 cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                 position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """LayerNorm (weight and bias in x's dtype) over the last dim of a
    (B, S, H, D) tensor, after RoPE when cos/sin are given.  Returns a new
    contiguous (B, S, H, D) tensor; differentiable in x, weight and bias."""
    _check("qk_layernorm", x, weight, bias)
    if _needs_grad(x, weight, bias):
        return _QKNormFunction.apply(x, weight, bias, eps, cos, sin, position_ids, NORM_LAYER)
    xc = x if _rows_ok(x) else x.contiguous()
    return _forward(xc, _param(weight), _param(bias), eps, *_tables(xc, cos, sin, position_ids), NORM_LAYER)
