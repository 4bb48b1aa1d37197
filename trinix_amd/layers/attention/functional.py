"""Public functional attention API (reference
``trinix/layers/attention/functional.py:8-140``), computed by the gfx950 HIP
kernels in ``libtrinix_attn.so``.
"""
from typing import Optional, Tuple

import torch

from ...kernels.attention_kernel import TritonAttentionKernel, attention


def triton_attn_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    attn_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
    window_size: Optional[Tuple[int, int]] = None,
    alibi_slopes: Optional[torch.Tensor] = None,
    *,
    rotary_cos: Optional[torch.Tensor] = None,
    rotary_sin: Optional[torch.Tensor] = None,
    return_lse: bool = False,
) -> torch.Tensor:
    """Scaled dot-product attention on the GPU.

    Args (same order and meaning as the reference):
        q: (batch, seq_len_q, num_heads, head_dim) GPU tensor (fp32/fp16/bf16).
        k, v: (batch, seq_len_k, num_kv_heads, head_dim); ``num_kv_heads``
            divides ``num_heads`` (equal to it in the reference).  Query head
            ``h`` reads KV head ``h // (num_heads // num_kv_heads)``.
        attn_mask: additive mask, 2-D (Sq, Sk), 3-D (B, Sq, Sk) or 4-D
            (B, 1|H, Sq, Sk); ``-inf`` removes a key.
        dropout_p: dropout probability on the attention weights.
        softmax_scale: defaults to ``head_dim ** -0.5``.
        causal: key j allowed only for j <= i (top-left aligned).
        window_size: (left, right): keys with -left <= j - i <= right.
        alibi_slopes: (H,), (1, H) or (B, H); adds ``-slope * |i - j|``.
    Keyword-only extensions:
        rotary_cos / rotary_sin: RoPE tables (rows = positions, in q.dtype,
            as ``FastRoPEPositionEmbedding.forward`` returns them); q is
            rotated inside the attention kernel, k by a pre-pass.
        return_lse: also return the fp32 (B, H, Sq) log-sum-exp.

    Returns:
        (batch, seq_len_q, num_heads, head_dim) tensor of q.dtype,
        differentiable through the HIP backward (dropout included; the
        reference's output is detached).

    Raises:
        ValueError: non-GPU tensors, inconsistent shapes, or a zero-sized
            batch, sequence or head dimension (``TRINIX_ERR_BAD_SHAPE``).
        RuntimeError: the HIP kernel library or a gfx950 GPU is unavailable.
    """
    if not q.is_cuda:
        raise ValueError("triton_attn_func only supports CUDA tensors")

    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError(
            f"Expected 4D tensors (batch, seqlen, nheads, headdim), "
            f"got q: {q.shape}, k: {k.shape}, v: {v.shape}"
        )

    batch, seqlen_q, nheads, headdim = q.shape
    _, seqlen_k, nheads_k, _ = k.shape

    if nheads_k <= 0 or nheads % nheads_k != 0 or k.shape != (batch, seqlen_k, nheads_k, headdim):
        raise ValueError(f"k shape {k.shape} doesn't match expected shape")

    if v.shape != (batch, seqlen_k, nheads_k, headdim):
        raise ValueError(f"v shape {v.shape} doesn't match expected shape")

    if not TritonAttentionKernel.is_available():
        raise RuntimeError(
            "HIP attention kernel not available. "
            "Build it with `python -m trinix_amd.build` and run on an MI355X (gfx950)."
        )

    if softmax_scale is None:
        softmax_scale = headdim**-0.5

    return attention(
        q,
        k,
        v,
        attn_mask=attn_mask,
        causal=causal,
        scale=softmax_scale,
        dropout_p=dropout_p,
        window_size=window_size,
        alibi_slopes=alibi_slopes,
        rotary_cos=rotary_cos,
        rotary_sin=rotary_sin,
        return_lse=return_lse,
    )
