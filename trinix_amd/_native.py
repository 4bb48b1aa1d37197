"""ctypes binding of ``libtrinix_attn.so`` (declared in ``include/trinix_attn.h``).

Only plain pointers, sizes and strides cross the boundary.  torch tensors are
turned into ``data_ptr()`` / ``stride()`` here, and the current torch stream
is passed as the HIP stream.  Status codes map to the exception types the
reference raises at its Python layer (``ValueError`` for bad inputs,
``RuntimeError`` for an unavailable or failing kernel).

There is no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_float, c_int32, c_int64, c_uint64, c_void_p, c_char_p

from .build import LIB_PATH

TRINIX_OK = 0
TRINIX_ERR_NULL_POINTER = 1
TRINIX_ERR_BAD_DTYPE = 2
TRINIX_ERR_BAD_HEAD_DIM = 3
TRINIX_ERR_BAD_SHAPE = 4
TRINIX_ERR_BAD_STRIDE = 5
TRINIX_ERR_BAD_ARGUMENT = 6
TRINIX_ERR_NO_DEVICE = 7
TRINIX_ERR_LAUNCH = 8
TRINIX_ERR_SCRATCH_TOO_SMALL = 9

SPLITKV_SCRATCH_BYTES = 32 << 20

TRINIX_F32 = 0
TRINIX_F16 = 1
TRINIX_BF16 = 2
TRINIX_U8 = 3

TRINIX_NORM_RMS = 0
TRINIX_NORM_LAYER = 1

BLOCKMAP_ROWS = 32
BLOCKMAP_COLS = 64

ABI_VERSION = 6

Int64x4 = c_int64 * 4
Int64x2 = c_int64 * 2


class AttnFwdArgs(ctypes.Structure):
    """Mirror of ``trinix_attn_fwd_args`` (field order and types identical)."""

    _fields_ = [
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("out", c_void_p),
        ("lse", c_void_p),
        ("q_stride", Int64x4),
        ("k_stride", Int64x4),
        ("v_stride", Int64x4),
        ("out_stride", Int64x4),
        ("batch", c_int64),
        ("seqlen_q", c_int64),
        ("seqlen_k", c_int64),
        ("nheads_q", c_int64),
        ("nheads_kv", c_int64),
        ("head_dim", c_int64),
        ("dtype", c_int32),
        ("softmax_scale", c_float),
        ("causal", c_int32),
        ("has_window", c_int32),
        ("window_left", c_int64),
        ("window_right", c_int64),
        ("alibi_slopes", c_void_p),
        ("alibi_stride", Int64x2),
        ("mask", c_void_p),
        ("mask_dtype", c_int32),
        ("mask_stride", Int64x4),
        ("mask_blockmap", c_void_p),
        ("blockmap_stride", Int64x2),
        ("dropout_p", c_float),
        ("dropout_seed", c_uint64),
        ("dropout_offset", c_uint64),
        ("rope_cos", c_void_p),
        ("rope_sin", c_void_p),
        ("rope_stride", c_int64),
        ("q_norm_weight", c_void_p),
        ("q_norm_eps", c_float),
        ("dropout_state", c_void_p),
        ("q_norm_out", c_void_p),
        ("dropout_keep_map", c_void_p),
    ]


class AttnBwdArgs(ctypes.Structure):
    """Mirror of ``trinix_attn_bwd_args`` (field order and types identical)."""

    _fields_ = [
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("out", c_void_p),
        ("dout", c_void_p),
        ("lse", c_void_p),
        ("delta", c_void_p),
        ("dq", c_void_p),
        ("dk", c_void_p),
        ("dv", c_void_p),
        ("q_stride", Int64x4),
        ("k_stride", Int64x4),
        ("v_stride", Int64x4),
        ("out_stride", Int64x4),
        ("dout_stride", Int64x4),
        ("dq_stride", Int64x4),
        ("dk_stride", Int64x4),
        ("dv_stride", Int64x4),
        ("batch", c_int64),
        ("seqlen_q", c_int64),
        ("seqlen_k", c_int64),
        ("nheads_q", c_int64),
        ("nheads_kv", c_int64),
        ("head_dim", c_int64),
        ("dtype", c_int32),
        ("softmax_scale", c_float),
        ("causal", c_int32),
        ("has_window", c_int32),
        ("window_left", c_int64),
        ("window_right", c_int64),
        ("alibi_slopes", c_void_p),
        ("alibi_stride", Int64x2),
        ("mask", c_void_p),
        ("mask_dtype", c_int32),
        ("mask_stride", Int64x4),
        ("mask_blockmap", c_void_p),
        ("blockmap_stride", Int64x2),
        ("dropout_p", c_float),
        ("dropout_seed", c_uint64),
        ("dropout_offset", c_uint64),
        ("dropout_state", c_void_p),
        ("dropout_keep_map", c_void_p),
    ]


class TileCfg(ctypes.Structure):
    """Mirror of ``trinix_tile_cfg``."""

    _fields_ = [
        ("block_m", c_int32),
        ("block_n", c_int32),
        ("block_d", c_int32),
        ("waves", c_int32),
        ("lds_bytes", c_int32),
    ]


# Every exported symbol with its (restype, argtypes).
SIGNATURES = {
    "trinix_attn_fwd": (c_int32, [POINTER(AttnFwdArgs), c_void_p]),
    "trinix_attn_mask_blockmap": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_int64, c_int64, POINTER(c_int64), c_void_p, c_void_p],
    ),
    "trinix_rope_apply": (
        c_int32,
        [c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64), c_int64, c_int64, c_int64, c_int64,
         c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "trinix_attn_fwd_splitkv_plan": (c_int32, [POINTER(AttnFwdArgs), POINTER(c_int32), POINTER(c_int64)]),
    "trinix_attn_fwd_splitkv": (c_int32, [POINTER(AttnFwdArgs), c_void_p, c_int64, c_void_p]),
    "trinix_attn_fwd_splitkv_noalloc": (c_int32, [POINTER(AttnFwdArgs), c_void_p]),
    "trinix_attn_bwd": (c_int32, [POINTER(AttnBwdArgs), c_void_p]),
    "trinix_qk_norm": (
        c_int32,
        [c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64), c_int64, c_int64, c_int64, c_int64, c_int32,
         c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "trinix_qk_layernorm": (
        c_int32,
        [c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64), c_int64, c_int64, c_int64, c_int64, c_int32,
         c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "trinix_qk_norm_bwd": (
        c_int32,
        [c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64), c_int64, c_int64,
         c_int64, c_int64, c_int32, c_int32, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
         c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "trinix_alibi_bias": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p]),
    "trinix_attn_tile_config": (c_int32, [c_int64, c_int32, POINTER(TileCfg)]),
    "trinix_dropout_state_advance": (c_int32, [c_void_p, c_void_p, c_uint64, c_void_p]),
    "trinix_dropout_keep_map_bytes": (c_int32, [c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "trinix_attn_is_available": (c_int32, []),
    "trinix_status_string": (c_char_p, [c_int32]),
    "trinix_abi_version": (c_int32, []),
}

_lib = None
_lock = threading.Lock()


def load_library() -> ctypes.CDLL:
    """Load the built library (once).  Raises ``RuntimeError`` if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m trinix_amd.build` "
                "(the gfx950 HIP library is required, there is no fallback)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.trinix_abi_version() != ABI_VERSION:
            raise RuntimeError("libtrinix_attn.so ABI version mismatch; rebuild it")
        _lib = lib
    return _lib


def library_loaded() -> bool:
    return _lib is not None


def status_string(code: int) -> str:
    return load_library().trinix_status_string(code).decode()


def check(code: int, what: str) -> None:
    """Raise the reference's exception type for a non-zero status."""
    if code == TRINIX_OK:
        return
    msg = f"{what}: {status_string(code)} (status {code})"
    if code in (TRINIX_ERR_NO_DEVICE, TRINIX_ERR_LAUNCH):
        raise RuntimeError(msg)
    raise ValueError(msg)


def int64x4(vals) -> Int64x4:
    return Int64x4(*[int(x) for x in vals])


def int64x2(vals) -> Int64x2:
    return Int64x2(*[int(x) for x in vals])
