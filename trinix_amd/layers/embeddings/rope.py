"""Rotary position embedding (reference ``trinix/layers/embeddings/rope.py``).

``forward`` returns the (cos, sin) tables exactly as the reference computes
them (``rope.py:61,69-79``: fp32 ``inv_freq``, ``cat(freqs, freqs)``, cast to
the input dtype), cached per (length, dtype, device) instead of recomputed on
every call.  ``apply_rotary_pos_emb`` runs the gfx950 RoPE kernel for GPU
tensors (bit-identical to the eager rounding of ``rope.py:111-134``) and the
eager formula for CPU tensors, as the reference's PyTorch path does.
"""
from typing import Optional, Tuple

import torch
import torch.nn as nn

from ...kernels.rope_kernel import rotate


class FastRoPEPositionEmbedding(nn.Module):
    def __init__(self, dim: int, max_position_embeddings: int = 2048, base: float = 10000.0,
                 use_triton: bool = True):
        super().__init__()
        self.dim = dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base
        self.use_triton = use_triton
        inv_freq = 1.0 / base ** (torch.arange(0, dim, 2).float() / dim)
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        self._cache = {}

    def _rotate_half(self, x: torch.Tensor) -> torch.Tensor:
        x1 = x[..., : x.shape[-1] // 2]
        x2 = x[..., x.shape[-1] // 2:]
        return torch.cat((-x2, x1), dim=-1)

    def forward(self, x: torch.Tensor, seq_len: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if seq_len is None:
            seq_len = x.shape[-2]
        key = (seq_len, x.dtype, x.device, self.inv_freq.device)
        hit = self._cache.get(key)
        if hit is not None:
            return hit
        t = torch.arange(seq_len, device=x.device, dtype=self.inv_freq.dtype)
        freqs = torch.outer(t, self.inv_freq.to(x.device))
        emb = torch.cat((freqs, freqs), dim=-1)
        out = (emb.cos().to(x.dtype), emb.sin().to(x.dtype))
        if len(self._cache) > 8:
            self._cache.clear()
        self._cache[key] = out
        return out

    def apply_rotary_pos_emb(self, q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                             position_ids: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if q.is_cuda:
            return rotate(q, cos, sin, position_ids), rotate(k, cos, sin, position_ids)
        if position_ids is not None:
            c = cos[position_ids].unsqueeze(2)
            s = sin[position_ids].unsqueeze(2)
        else:
            c = cos[: q.shape[1]].unsqueeze(0).unsqueeze(2)
            s = sin[: q.shape[1]].unsqueeze(0).unsqueeze(2)
        return q * c + self._rotate_half(q) * s, k * c + self._rotate_half(k) * s
