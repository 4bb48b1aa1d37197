from .base import FastBaseAttention
from .functional import triton_attn_func
from .grouped_query_attention import FastGroupedQueryAttention
from .multi_query_attention import FastMultiQueryAttention
from .multihead_attention import FastMultiHeadAttention
from .multihead_self_attention import FastMultiHeadSelfAttention

__all__ = [
    "FastBaseAttention",
    "FastGroupedQueryAttention",
    "FastMultiHeadAttention",
    "FastMultiHeadSelfAttention",
    "FastMultiQueryAttention",
    "triton_attn_func",
]
