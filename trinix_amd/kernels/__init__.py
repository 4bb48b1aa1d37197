"""HIP kernel wrappers (gfx950); class names kept from the reference registry
``trinix/kernels/__init__.py:14`` for drop-in use."""
from .alibi_kernel import TritonALiBiKernel, alibi_bias
from .attention_kernel import TritonAttentionKernel, attention_flops, allowed_pairs
from .qk_norm_kernel import qk_layernorm, qk_norm_supported, qk_rmsnorm
from .rope_kernel import TritonRoPEKernel, rope_apply
from .utils import calculate_attention_block_sizes, get_cuda_compute_capability, tile_config

__all__ = [
    "TritonALiBiKernel",
    "alibi_bias",
    "TritonAttentionKernel",
    "TritonRoPEKernel",
    "rope_apply",
    "qk_rmsnorm",
    "qk_layernorm",
    "qk_norm_supported",
    "attention_flops",
    "allowed_pairs",
    "calculate_attention_block_sizes",
    "get_cuda_compute_capability",
    "tile_config",
]
