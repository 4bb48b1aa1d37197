"""FastMultiHeadAttention (reference
``trinix/layers/attention/multihead_attention.py:10-209``): same constructor,
forward signature, parameter names and return convention (a tuple only when
``use_cache``)."""
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn

from .base import FastBaseAttention


class FastMultiHeadAttention(FastBaseAttention):
    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = True,
                 kernel_type: str = "flash", causal: bool = False, head_dim: Optional[int] = None,
                 position_method: Union[str, nn.Module] = "none", max_seq_len: int = 2048,
                 rope_base: float = 10000.0, use_sliding_window: bool = False,
                 sliding_window_size: Optional[int] = None, qk_norm: bool = False, qk_norm_type: str = "rmsnorm",
                 use_triton_norm: bool = True, use_triton_embeddings: bool = True, kdim: Optional[int] = None,
                 vdim: Optional[int] = None, add_zero_attn: bool = False, batch_first: bool = True):
        base_embed = num_heads * head_dim if head_dim is not None else embed_dim
        super().__init__(base_embed, num_heads, dropout, bias, kernel_type, causal, position_method, max_seq_len,
                         rope_base, use_sliding_window, sliding_window_size, qk_norm, qk_norm_type,
                         use_triton_norm, use_triton_embeddings, add_zero_attn)
        if head_dim is not None:
            self.head_dim = head_dim
        self.kdim = kdim if kdim is not None else embed_dim
        self.vdim = vdim if vdim is not None else embed_dim
        self.batch_first = batch_first
        self.q_proj = nn.Linear(embed_dim, num_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(self.kdim, num_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(self.vdim, num_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(num_heads * self.head_dim, embed_dim, bias=bias)
        self._init_weights()

    def _init_weights(self):
        for proj in [self.q_proj, self.k_proj, self.v_proj, self.o_proj]:
            nn.init.xavier_uniform_(proj.weight)
            if proj.bias is not None:
                nn.init.constant_(proj.bias, 0.0)

    def forward(self, query: torch.Tensor, key: Optional[torch.Tensor] = None, value: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None,
                position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                position_ids: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, use_cache: bool = False,
                **kwargs):
        if not self.batch_first:
            query = query.transpose(0, 1)
            if key is not None:
                key = key.transpose(0, 1)
            if value is not None:
                value = value.transpose(0, 1)
        if key is None:
            key = query
        if value is None:
            value = key
        bs, seq_len_q, _ = query.shape
        seq_len_k = key.shape[1]
        q = self.q_proj(query).view(bs, seq_len_q, self.num_heads, self.head_dim)
        k = self.k_proj(key).view(bs, seq_len_k, self.num_heads, self.head_dim)
        v = self.v_proj(value).view(bs, seq_len_k, self.num_heads, self.head_dim)
        out, k_cache, v_cache = self._attend(q, k, v, attention_mask, position_ids, past_key_value, True)
        out = self.o_proj(out.reshape(bs, seq_len_q, -1))
        if not self.batch_first:
            out = out.transpose(0, 1)
        if use_cache:
            return out, (k_cache, v_cache)
        return out
