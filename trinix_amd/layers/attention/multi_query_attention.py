"""FastMultiQueryAttention (reference
``trinix/layers/attention/multi_query_attention.py:10-195``): one KV head
shared by all query heads, passed to the HIP kernel as one head (the
reference ``expand``s it with stride 0, :173-174).  Returns a tuple only when
``use_cache`` (:192-195)."""
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn

from .base import FastBaseAttention


class FastMultiQueryAttention(FastBaseAttention):
    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = True,
                 kernel_type: str = "flash", causal: bool = False, head_dim: Optional[int] = None,
                 position_method: Union[str, nn.Module] = "none", max_seq_len: int = 2048,
                 rope_base: float = 10000.0, use_sliding_window: bool = False,
                 sliding_window_size: Optional[int] = None, qk_norm: bool = False, qk_norm_type: str = "rmsnorm",
                 use_triton_norm: bool = True, use_triton_embeddings: bool = True):
        base_embed = num_heads * head_dim if head_dim is not None else embed_dim
        super().__init__(base_embed, num_heads, dropout, bias, kernel_type, causal, position_method, max_seq_len,
                         rope_base, use_sliding_window, sliding_window_size, qk_norm, qk_norm_type,
                         use_triton_norm, use_triton_embeddings, False)
        if head_dim is not None:
            self.head_dim = head_dim
        self.q_proj = nn.Linear(embed_dim, num_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(embed_dim, self.head_dim, bias=bias)
        self.v_proj = nn.Linear(embed_dim, self.head_dim, bias=bias)
        self.o_proj = nn.Linear(num_heads * self.head_dim, embed_dim, bias=bias)
        self._init_weights()

    def _init_weights(self):
        for proj in [self.q_proj, self.k_proj, self.v_proj, self.o_proj]:
            nn.init.xavier_uniform_(proj.weight)
            if proj.bias is not None:
                nn.init.constant_(proj.bias, 0.0)

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                position_ids: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, use_cache: bool = False,
                **kwargs):
        bs, seq_len_q, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(bs, seq_len_q, self.num_heads, self.head_dim)
        k = self.k_proj(hidden_states).view(bs, seq_len_q, 1, self.head_dim)
        v = self.v_proj(hidden_states).view(bs, seq_len_q, 1, self.head_dim)
        out, k_cache, v_cache = self._attend(q, k, v, attention_mask, position_ids, past_key_value, False)
        out = self.o_proj(out.reshape(bs, seq_len_q, -1))
        if use_cache:
            return out, (k_cache, v_cache)
        return out
