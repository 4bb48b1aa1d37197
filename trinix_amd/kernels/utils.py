"""Device queries and the gfx950 attention tile table.

Replaces ``calculate_attention_block_sizes`` / ``get_cuda_compute_capability``
/ ``get_gpu_shared_memory_limit`` (reference ``trinix/kernels/utils.py:5-15,
60-153``): tile shapes come from the library's fixed gfx950 table
(``trinix_attn_tile_config``), not from a shared-memory estimate.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _native as nat


def get_cuda_compute_capability() -> int:
    """``major*10 + minor`` of the current device (95 on MI355X / gfx950)."""
    if not torch.cuda.is_available():
        return 0
    major, minor = torch.cuda.get_device_capability()
    return major * 10 + minor


def get_gpu_shared_memory_limit() -> int:
    """LDS bytes per workgroup available on gfx950."""
    return 160 * 1024


def tile_config(head_dim: int, dtype: torch.dtype = torch.bfloat16) -> dict:
    from .attention_kernel import _DTYPE_CODE, kernel_head_dim

    d = kernel_head_dim(head_dim)
    if d is None:
        raise ValueError(f"head_dim {head_dim} is not supported")
    cfg = nat.TileCfg()
    nat.check(nat.load_library().trinix_attn_tile_config(d, _DTYPE_CODE[dtype], cfg), "trinix_attn_tile_config")
    return {k: getattr(cfg, k) for k, _ in nat.TileCfg._fields_}


def calculate_attention_block_sizes(head_dim: int, seq_len: int = None,
                                    dtype: torch.dtype = torch.bfloat16) -> Tuple[int, int, int]:
    """(BLOCK_M, BLOCK_N, BLOCK_DMODEL) the library launches for ``head_dim``."""
    cfg = tile_config(head_dim, dtype)
    return cfg["block_m"], cfg["block_n"], cfg["block_d"]
