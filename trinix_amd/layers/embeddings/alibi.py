"""ALiBi position bias (reference ``trinix/layers/embeddings/alibi.py``).

Slopes follow ``_get_slopes`` (``alibi.py:47-63``).  ``forward`` returns the
``-slope * |i - j|`` bias of shape (B, H, S, S) for API compatibility
(``alibi.py:65-90``): from the HIP kernel when the slopes live on the GPU and
``use_triton`` is set (the reference's Triton branch), else in eager torch.
The attention layers never call it: they pass ``slopes`` to the attention
kernel, which adds the bias per element.
"""
import math

import torch
import torch.nn as nn


class FastALiBiPositionEmbedding(nn.Module):
    def __init__(self, num_heads: int, max_seq_len: int = 2048, use_triton: bool = True):
        super().__init__()
        self.num_heads = num_heads
        self.max_seq_len = max_seq_len
        self.use_triton = use_triton
        self.register_buffer("slopes", self._get_slopes(num_heads), persistent=False)

    def _get_slopes(self, num_heads: int) -> torch.Tensor:
        def pow2(n):
            start = 2 ** (-(2 ** (-(math.log2(n) - 3))))
            return [start * start**i for i in range(n)]

        if math.log2(num_heads).is_integer():
            slopes = pow2(num_heads)
        else:
            c = 2 ** math.floor(math.log2(num_heads))
            slopes = pow2(c) + pow2(2 * c)[0::2][: num_heads - c]
        return torch.tensor(slopes, dtype=torch.float32)

    def forward(self, seq_len: int, batch_size: int = 1) -> torch.Tensor:
        if self.use_triton and self.slopes.is_cuda:
            from ...kernels.alibi_kernel import TritonALiBiKernel

            if TritonALiBiKernel.is_available():
                return TritonALiBiKernel.apply(self.slopes, batch_size, self.num_heads, seq_len)
        return self._compute_alibi_pytorch(seq_len, batch_size)

    def _compute_alibi_pytorch(self, seq_len: int, batch_size: int) -> torch.Tensor:
        pos = torch.arange(seq_len, device=self.slopes.device)
        dist = (pos.unsqueeze(0) - pos.unsqueeze(1)).abs()
        bias = -(dist.unsqueeze(0) * self.slopes.unsqueeze(1).unsqueeze(2))
        return bias.unsqueeze(0).expand(batch_size, -1, -1, -1)
