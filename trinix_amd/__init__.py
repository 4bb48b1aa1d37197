"""trinix_amd: MI355X (gfx950) attention forward for the trinix API.

The public names of the reference's attention path are kept
(``trinix/__init__.py:25-31``, ``trinix/layers/attention/__init__.py``);
their GPU work runs in hand-written HIP kernels (``libtrinix_attn.so``).
"""
from .version import __version__
from .kernels import TritonAttentionKernel, TritonRoPEKernel, calculate_attention_block_sizes
from .layers.attention import (
    FastBaseAttention,
    FastGroupedQueryAttention,
    FastMultiHeadAttention,
    FastMultiHeadSelfAttention,
    FastMultiQueryAttention,
    triton_attn_func,
)
from .layers.embeddings import FastALiBiPositionEmbedding, FastRoPEPositionEmbedding

__all__ = [
    "__version__",
    "TritonAttentionKernel",
    "TritonRoPEKernel",
    "calculate_attention_block_sizes",
    "triton_attn_func",
    "FastBaseAttention",
    "FastGroupedQueryAttention",
    "FastMultiHeadAttention",
    "FastMultiHeadSelfAttention",
    "FastMultiQueryAttention",
    "FastRoPEPositionEmbedding",
    "FastALiBiPositionEmbedding",
]
