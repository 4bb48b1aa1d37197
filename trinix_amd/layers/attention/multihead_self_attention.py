"""FastMultiHeadSelfAttention (reference
``trinix/layers/attention/multihead_self_attention.py``): fused QKV
projection; q/k/v are strided views of one (B, S, 3, H, D) tensor and reach
the HIP kernel without copies."""
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn

from .base import FastBaseAttention


class FastMultiHeadSelfAttention(FastBaseAttention):
    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = True,
                 kernel_type: str = "flash", causal: bool = False, head_dim: Optional[int] = None,
                 position_method: Union[str, nn.Module] = "none", max_seq_len: int = 2048,
                 rope_base: float = 10000.0, use_sliding_window: bool = False,
                 sliding_window_size: Optional[int] = None, qk_norm: bool = False, qk_norm_type: str = "rmsnorm",
                 use_triton_norm: bool = True, use_triton_embeddings: bool = True, add_zero_attn: bool = False,
                 batch_first: bool = True):
        base_embed = num_heads * head_dim if head_dim is not None else embed_dim
        super().__init__(base_embed, num_heads, dropout, bias, kernel_type, causal, position_method, max_seq_len,
                         rope_base, use_sliding_window, sliding_window_size, qk_norm, qk_norm_type,
                         use_triton_norm, use_triton_embeddings, add_zero_attn)
        if head_dim is not None:
            self.head_dim = head_dim
        self.batch_first = batch_first
        self.qkv_proj = nn.Linear(embed_dim, 3 * num_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(num_heads * self.head_dim, embed_dim, bias=bias)
        self._init_weights()

    def _init_weights(self):
        nn.init.xavier_uniform_(self.qkv_proj.weight)
        nn.init.xavier_uniform_(self.o_proj.weight)
        if self.qkv_proj.bias is not None:
            nn.init.constant_(self.qkv_proj.bias, 0.0)
        if self.o_proj.bias is not None:
            nn.init.constant_(self.o_proj.bias, 0.0)

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                position_ids: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, use_cache: bool = False,
                **kwargs):
        if not self.batch_first:
            hidden_states = hidden_states.transpose(0, 1)
        bs, seq_len, _ = hidden_states.shape
        qkv = self.qkv_proj(hidden_states).view(bs, seq_len, 3, self.num_heads, self.head_dim)
        q, k, v = qkv.unbind(dim=2)
        out, k_cache, v_cache = self._attend(q, k, v, attention_mask, position_ids, past_key_value, True)
        out = self.o_proj(out.reshape(bs, seq_len, -1))
        if not self.batch_first:
            out = out.transpose(0, 1)
        if use_cache:
            return out, (k_cache, v_cache)
        return out
