from .attention import (
    FastBaseAttention,
    FastGroupedQueryAttention,
    FastMultiHeadAttention,
    FastMultiHeadSelfAttention,
    FastMultiQueryAttention,
    triton_attn_func,
)
from .embeddings import FastALiBiPositionEmbedding, FastRoPEPositionEmbedding
