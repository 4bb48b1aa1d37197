from .functional import triton_attn_func

__all__ = ["triton_attn_func"]
