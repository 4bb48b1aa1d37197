"""trinix_amd: MI355X (gfx950) attention forward for the trinix API.

The public names of the reference's attention path are kept
(``trinix/__init__.py:25-31``, ``trinix/layers/attention/__init__.py``);
their GPU work runs in hand-written HIP kernels (``libtrinix_attn.so``).
"""
from .version import __version__
from .kernels import TritonAttentionKernel, TritonRoPEKernel, calculate_attention_block_sizes
from .layers.attention.functional import triton_attn_func

__all__ = [
    "__version__",
    "TritonAttentionKernel",
    "TritonRoPEKernel",
    "calculate_attention_block_sizes",
    "triton_attn_func",
]
