"""Attention forward on MI355X through ``libtrinix_attn.so``.

Host side of the drop-in for ``TritonAttentionKernel``
(reference ``trinix/kernels/attention_kernel.py:437-664``): same class name,
same ``is_available()`` / ``apply(...)`` signature, argument meaning and
output (a new ``(B, Sq, H, D)`` tensor of ``q.dtype``).  Differences, all of
them inputs the reference rejected or mishandled:

* ``k``/``v`` may carry fewer heads than ``q`` (GQA/MQA, ``H % Hkv == 0``);
  the kernel maps query head ``h`` to KV head ``h // (H // Hkv)`` without
  copying (stride-0 ``expand``-ed KV also works without a copy);
* ``Sq != Sk`` is accepted (causal stays top-left aligned, ``j <= i``, as in
  the eager path ``trinix/layers/attention/base.py:375-379``);
* the mask is never materialised to ``(B, H, S, S)``
  (``attention_kernel.py:479-495``): it is read through broadcast strides and
  classified once per call into 32x64 blocks;
* rows whose first key tiles are fully masked are exact (the reference
  kernel returns NaN there); rows with no allowed key at all give NaN, as
  the eager softmax does;
* optional fused RoPE (``rotary_cos`` / ``rotary_sin``) and log-sum-exp
  output.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Tuple

import torch

from .. import _native as nat

_DTYPE_CODE = {
    torch.float32: nat.TRINIX_F32,
    torch.float16: nat.TRINIX_F16,
    torch.bfloat16: nat.TRINIX_BF16,
}
_MASK_DTYPE_CODE = {
    torch.float32: nat.TRINIX_F32,
    torch.float16: nat.TRINIX_F16,
    torch.bfloat16: nat.TRINIX_BF16,
    torch.uint8: nat.TRINIX_U8,
}
KERNEL_HEAD_DIMS = (64, 128, 256)
# The backward kernels are built for the same widths (bf16/fp16 at 64 and
# 128 run the MFMA pipeline, dropout included; fp32 and 256 the generic
# kernels).
BACKWARD_HEAD_DIMS = (64, 128, 256)


# Calls with at most this many query rows (bf16/fp16, no dropout) go to the
# split-KV decode kernel when its plan applies; SPLITKV_ENABLED = False
# forces the prefill kernel (tests compare the two).
SPLITKV_MAX_SQ = 16
SPLITKV_ENABLED = True


def kernel_head_dim(head_dim: int) -> Optional[int]:
    """Head dim the kernels run at: inputs are zero-padded up to it."""
    for d in KERNEL_HEAD_DIMS:
        if head_dim <= d:
            return d
    return None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_ptr(device: torch.device) -> int:
    # the raw handle without building a torch.cuda.Stream object (about 2 us
    # per call less, which shows at small shapes); the public route where
    # this torch build lacks the raw accessor
    if _raw_stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(index)


def _kernel_ready(t: torch.Tensor) -> bool:
    """True if ``t`` (4-D BSHD) meets the kernel's load constraints as is."""
    if t.stride(-1) != 1:
        return False
    if t.element_size() == 2:
        if t.data_ptr() % 16:
            return False
        return all(s % 8 == 0 for s in t.stride()[:3])
    return t.data_ptr() % 4 == 0


def _prepare_operand(t: torch.Tensor, d_kernel: int) -> torch.Tensor:
    d = t.shape[-1]
    if d != d_kernel:
        t = torch.nn.functional.pad(t, (0, d_kernel - d))
    if not _kernel_ready(t):
        t = t.contiguous()
        if not _kernel_ready(t):  # contiguous already, but its start is not 16-byte aligned
            t = t.clone()
    return t


class TritonAttentionKernel:
    """MI355X attention forward (name kept from the reference for drop-in use).

    Methods:
        is_available(): True if the HIP library loads and a gfx950 GPU is
            visible to torch.
        apply(q, k, v, attn_mask=None, causal=False, scale=None,
              dropout_p=0.0, window_size=None, alibi_slopes=None):
            attention forward; see the module docstring.
    """

    _available = False  # set once a check has passed; every call re-checks until then

    @staticmethod
    def is_available() -> bool:
        if TritonAttentionKernel._available:
            return True
        try:
            lib = nat.load_library()
        except (RuntimeError, OSError):
            return False
        if not torch.cuda.is_available():
            return False
        ok = bool(lib.trinix_attn_is_available())
        TritonAttentionKernel._available = ok
        return ok

    @staticmethod
    def _prepare_mask(attn_mask: torch.Tensor, batch_size: int, num_heads: int,
                      seq_len_q: int, seq_len_k: Optional[int] = None) -> torch.Tensor:
        """Broadcast view of the mask as (B, H, Sq, Sk), no copy.

        Accepts 2-D (Sq, Sk), 3-D (B, Sq, Sk) and 4-D (B, 1 or H, Sq, Sk)
        masks like the reference (``attention_kernel.py:479-495``); a size-1
        batch dimension also broadcasts.
        """
        if seq_len_k is None:
            seq_len_k = seq_len_q
        if attn_mask.dim() == 2:
            m = attn_mask[None, None]
        elif attn_mask.dim() == 3:
            m = attn_mask[:, None]
        elif attn_mask.dim() == 4:
            m = attn_mask
        else:
            raise ValueError(f"Unsupported mask shape: {attn_mask.shape}")
        target = (batch_size, num_heads, seq_len_q, seq_len_k)
        for have, want in zip(m.shape, target):
            if have != want and have != 1:
                raise ValueError(
                    f"Mask shape {tuple(attn_mask.shape)} doesn't match expected shape {target}"
                )
        return m.expand(*target)

    @staticmethod
    def mask_blockmap(mask4: torch.Tensor, stream: Optional[int] = None) -> Tuple[torch.Tensor, Tuple[int, int]]:
        """Per-32x64-block classification of a (B, H, Sq, Sk) mask view.

        Returns the uint8 map and its (batch, head) strides; broadcast
        dimensions of the mask are broadcast in the map too.
        """
        B, H, Sq, Sk = mask4.shape
        mb = B if mask4.stride(0) != 0 else 1
        mh = H if mask4.stride(1) != 0 else 1
        rows = -(-Sq // nat.BLOCKMAP_ROWS)
        cols = -(-Sk // nat.BLOCKMAP_COLS)
        bmap = torch.empty((mb, mh, rows, cols), dtype=torch.uint8, device=mask4.device)
        code = _MASK_DTYPE_CODE[mask4.dtype]
        strides = (ctypes.c_int64 * 4)(*mask4.stride())
        lib = nat.load_library()
        if stream is None:
            stream = current_stream_ptr(mask4.device)
        rc = lib.trinix_attn_mask_blockmap(mask4.data_ptr(), code, mb, mh, Sq, Sk, strides,
                                           bmap.data_ptr(), stream)
        nat.check(rc, "trinix_attn_mask_blockmap")
        bm_sb = mh * rows * cols if mb > 1 else 0
        bm_sh = rows * cols if mh > 1 else 0
        return bmap, (bm_sb, bm_sh)

    @staticmethod
    def apply(
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        attn_mask: torch.Tensor = None,
        causal: bool = False,
        scale: float = None,
        dropout_p: float = 0.0,
        window_size: tuple = None,
        alibi_slopes: torch.Tensor = None,
        *,
        rotary_cos: Optional[torch.Tensor] = None,
        rotary_sin: Optional[torch.Tensor] = None,
        rotary_k: bool = True,
        return_lse: bool = False,
        use_blockmap: bool = True,
        q_norm_weight: Optional[torch.Tensor] = None,
        q_norm_eps: float = 1e-6,
    ):
        """Attention forward (reference ``attention_kernel.py:497-664``); the
        output carries no autograd history, as in the reference.

        Extensions (keyword-only): ``rotary_cos``/``rotary_sin`` (rows of the
        reference RoPE tables in ``q.dtype``, indexed by position) apply RoPE
        to q inside the kernel and to k by a pre-pass (``rotary_k=False``
        leaves k as given); ``return_lse`` also returns the (B, H, Sq) fp32
        log-sum-exp; ``q_norm_weight``/``q_norm_eps`` apply the layers' q
        RMSNorm over head_dim (after the fused RoPE) in the kernel's q
        prologue, bitwise as ``qk_rmsnorm`` would (bf16/fp16, head_dim 64,
        128 or 256).  ``attention()`` is the differentiable entry point.
        """
        out, lse, _ = _forward(q, k, v, attn_mask, causal, scale, dropout_p, window_size, alibi_slopes,
                               rotary_cos, rotary_sin, rotary_k, return_lse, use_blockmap,
                               q_norm_weight=q_norm_weight, q_norm_eps=q_norm_eps)
        if return_lse:
            return out, lse
        return out


# Per device: the dropout generator {seed, offset} (two int64 in device
# memory) that calls captured in a HIP graph draw from.  Created by the
# first call with dropout outside a capture, seeded from torch's initial
# seed (torch.manual_seed makes it reproducible; no draw from torch's
# generator, so the eager calls' seeds are unchanged), offsets from 2^32 up
# so that its streams never repeat an eager call's (offset 0).
_DROPOUT_GENERATORS: dict = {}


def dropout_generator(device: torch.device) -> torch.Tensor:
    gen = _DROPOUT_GENERATORS.get(device)
    if gen is None:
        seed = (torch.initial_seed() * 0x9E3779B97F4A7C15 + 0x632BE59BD9B4E019) % (1 << 63)
        gen = torch.tensor([seed, 1 << 32], dtype=torch.int64, device=device)
        _DROPOUT_GENERATORS[device] = gen
    return gen


# Dropout keep map: a forward with dropout that keeps state for a backward
# writes its keep decisions (one bit per (row, key)) so that the backward
# reads them instead of regenerating them from Philox (about 0.3 ms of the
# backward at B=1, S=8192, 32 heads, D=128).  The map takes
# 128*B*H*2*ceil(Sq/64)*4*ceil(Sk/128) bytes (1/8 byte per (row, key); the
# eager path keeps a mask of one element per (row, key)): 268 MB at that
# shape.  Calls whose map would exceed 1/32 of the device's memory regenerate
# instead; TRINIX_DROPOUT_KEEP_MAP=0 / 1 forces either way.
_KEEP_MAP_LIMIT: dict = {}


def _keep_map_bytes(device: torch.device, B: int, H: int, Sq: int, Sk: int) -> int:
    mode = os.environ.get("TRINIX_DROPOUT_KEEP_MAP", "")
    if mode == "0":
        return 0
    n = ctypes.c_int64(0)
    nat.check(nat.load_library().trinix_dropout_keep_map_bytes(B, H, Sq, Sk, ctypes.byref(n)),
              "trinix_dropout_keep_map_bytes")
    if mode != "1":
        lim = _KEEP_MAP_LIMIT.get(device)
        if lim is None:
            lim = torch.cuda.get_device_properties(device).total_memory // 32
            _KEEP_MAP_LIMIT[device] = lim
        if n.value > lim:
            return 0
    return n.value


# ---------------------------------------------------------------------------
# Launch cache.  A call without mask, ALiBi, dropout, q-norm or lse output
# whose operands the kernels read in place is described, apart from its data
# pointers, by its tensors' shapes, strides, dtypes and devices and its
# scalar arguments.  The first such call goes through the full path below
# (checks, operand preparation, the argument struct) and leaves a template
# of its launch here; later calls of the same layout copy the template, set
# the pointers and launch.  A call that would not pass every check never
# leaves a template, so the errors of the full path are unchanged.
# ---------------------------------------------------------------------------
class _Launch:
    __slots__ = ("args", "out_shape", "dtype", "device", "align", "rope", "split")

    def __init__(self, args, out_shape, dtype, device, align, rope, split):
        self.args = args            # AttnFwdArgs with null data pointers
        self.out_shape = out_shape
        self.dtype = dtype
        self.device = device
        self.align = align          # byte alignment the operand pointers need
        self.rope = rope            # k pre-pass: (k_stride, out_stride, B, S, H, D, cs_stride, rows) or None
        self.split = split          # split-KV workspace bytes, or None for trinix_attn_fwd


_LAUNCHES: dict = {}
_MAX_LAUNCHES = 256


def _launch_key(q, k, v, causal, scale, window_size, rotary_cos, rotary_sin, rotary_k):
    """Everything a cached launch depends on except the data pointers, or
    None when an argument is not hashable."""
    try:
        rk = None
        if rotary_cos is not None:
            if rotary_sin is None:
                return None
            rk = (rotary_cos.shape, rotary_cos.stride(), rotary_cos.dtype, rotary_cos.device, rotary_sin.shape,
                  rotary_sin.stride(), rotary_sin.dtype, rotary_sin.device, bool(rotary_k))
        key = (q.shape, q.stride(), q.dtype, q.device, k.shape, k.stride(), k.dtype, k.device, v.shape, v.stride(),
               v.dtype, v.device, bool(causal), scale, None if window_size is None else tuple(window_size), rk,
               SPLITKV_ENABLED)
        hash(key)
        return key
    except (TypeError, AttributeError):
        return None


def _launch_cached(key, q, k, v, rotary_cos, rotary_sin):
    """The output of a call whose layout has a cached launch, or None."""
    ent = _LAUNCHES.get(key)
    if ent is None:
        return None
    qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
    if ent.rope is not None:
        cp, sp = rotary_cos.data_ptr(), rotary_sin.data_ptr()
        if (qp | kp | vp | cp | sp) % ent.align:
            return None
    elif (qp | kp | vp) % ent.align:
        return None
    lib = nat.load_library()
    stream = current_stream_ptr(ent.device)
    a = nat.AttnFwdArgs.from_buffer_copy(ent.args)
    if ent.rope is not None:
        ks, os_, B, S, H, D, cs_stride, rows = ent.rope
        kr = torch.empty((B, S, H, D), dtype=ent.dtype, device=ent.device)
        nat.check(lib.trinix_rope_apply(kp, ks, kr.data_ptr(), os_, B, S, H, D, a.dtype, cp, sp, cs_stride, rows,
                                        None, stream), "trinix_rope_apply")
        kp = kr.data_ptr()
        a.rope_cos, a.rope_sin = cp, sp
    out = torch.empty(ent.out_shape, dtype=ent.dtype, device=ent.device)
    a.q, a.k, a.v, a.out = qp, kp, vp, out.data_ptr()
    if ent.split is None:
        nat.check(lib.trinix_attn_fwd(ctypes.byref(a), stream), "trinix_attn_fwd")
    else:
        ws = torch.empty(ent.split, dtype=torch.uint8, device=ent.device) if ent.split else None
        nat.check(lib.trinix_attn_fwd_splitkv(ctypes.byref(a), None if ws is None else ws.data_ptr(), ent.split,
                                              stream), "trinix_attn_fwd_splitkv")
    return out


# Training launches.  A differentiable call (the forward keeps state for the
# backward) without mask, ALiBi, q-norm or fused rotary tables, whose
# operands the kernels read in place, is cached the same way: the forward's
# argument template (its lse written) and, once the first backward of the
# layout has run, the backward's template.  Dropout calls draw their seed
# (and keep map) per call as on the full path.
class _TrainLaunch:
    __slots__ = ("fwd", "bwd", "out_shape", "lse_shape", "dtype", "device", "align", "km_bytes", "do_stride",
                 "dk_shape")

    def __init__(self, fwd, out_shape, lse_shape, dtype, device, align, km_bytes, dk_shape):
        self.fwd = fwd                # AttnFwdArgs with null data pointers and seed
        self.bwd = None               # AttnBwdArgs template after the first backward, or None
        self.out_shape = out_shape
        self.lse_shape = lse_shape
        self.dtype = dtype
        self.device = device
        self.align = align
        self.km_bytes = km_bytes      # dropout keep map bytes (0: none)
        self.do_stride = None         # dout strides the backward template was built for
        self.dk_shape = dk_shape      # shape of k (and of dk, dv)


_TRAIN_LAUNCHES: dict = {}


def _train_key(q, k, v, causal, scale, dropout_p, window_size, return_lse):
    key = _launch_key(q, k, v, causal, scale, window_size, None, None, False)
    if key is None:
        return None
    return key, float(dropout_p), bool(return_lse), os.environ.get("TRINIX_DROPOUT_KEEP_MAP", "")


def _train_cached(tkey, q, k, v):
    """(out, lse, state) of a differentiable call whose layout has a cached
    training launch, or None."""
    ent = _TRAIN_LAUNCHES.get(tkey)
    if ent is None:
        return None
    qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
    if (qp | kp | vp) % ent.align:
        return None
    a = nat.AttnFwdArgs.from_buffer_copy(ent.fwd)
    keep_map = None
    if a.dropout_p > 0.0:
        if torch.cuda.is_current_stream_capturing():
            return None  # the device-side dropout state of the full path
        a.dropout_seed = int(torch.randint(0, 2 ** 62, (1,)).item())
        if ent.km_bytes:
            keep_map = torch.empty(ent.km_bytes, dtype=torch.uint8, device=ent.device)
            a.dropout_keep_map = keep_map.data_ptr()
    out = torch.empty(ent.out_shape, dtype=ent.dtype, device=ent.device)
    lse = torch.empty(ent.lse_shape, dtype=torch.float32, device=ent.device)
    a.q, a.k, a.v, a.out, a.lse = qp, kp, vp, out.data_ptr(), lse.data_ptr()
    nat.check(nat.load_library().trinix_attn_fwd(ctypes.byref(a), current_stream_ptr(ent.device)), "trinix_attn_fwd")
    D = ent.out_shape[-1]
    state = dict(q=q, k=k, v=v, out=out, lse=lse, D=D, d_kernel=D, args=a, launch=ent,
                 dropout=(float(a.dropout_p), int(a.dropout_seed), 0), dropout_state=None, keep_map=keep_map)
    return out, lse, state


def _forward(q, k, v, attn_mask, causal, scale, dropout_p, window_size, alibi_slopes, rotary_cos, rotary_sin,
             rotary_k, return_lse, use_blockmap, keep_state=False, q_norm_weight=None, q_norm_eps=1e-6,
             q_norm_out=None):
    """Launch ``trinix_attn_fwd``; returns (out, lse or None, state).  With
    ``keep_state`` the prepared operands (padded, strided as the kernel reads
    them), the lse and the mask / slope tensors are kept for the backward."""
    key = None
    if (attn_mask is None and alibi_slopes is None and not dropout_p and q_norm_weight is None and not return_lse
            and not keep_state):
        key = _launch_key(q, k, v, causal, scale, window_size, rotary_cos, rotary_sin, rotary_k)
        if key is not None:
            out = _launch_cached(key, q, k, v, rotary_cos, rotary_sin)
            if out is not None:
                return out, None, None
    tkey = None
    if (keep_state and attn_mask is None and alibi_slopes is None and q_norm_weight is None and rotary_cos is None
            and rotary_sin is None):
        tkey = _train_key(q, k, v, causal, scale, dropout_p, window_size, return_lse)
        if tkey is not None:
            res = _train_cached(tkey, q, k, v)
            if res is not None:
                return res
    q_in, k_in, v_in, cos_in, sin_in = q, k, v, rotary_cos, rotary_sin
    rope_tpl = None
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("TritonAttentionKernel requires GPU tensors")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"Expected 4D tensors, got q: {q.shape}, k: {k.shape}, v: {v.shape}")
    if q.dtype not in _DTYPE_CODE:
        raise ValueError(f"Unsupported dtype {q.dtype}; use float32, float16 or bfloat16")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    B, Sq, H, D = q.shape
    Bk, Sk, Hkv, Dk = k.shape
    if Bk != B or Dk != D or tuple(v.shape) != (B, Sk, Hkv, D):
        raise ValueError(f"k/v shapes {tuple(k.shape)}, {tuple(v.shape)} don't match q {tuple(q.shape)}")
    if Hkv <= 0 or H % Hkv != 0:
        raise ValueError(f"num_heads ({H}) must be a multiple of the KV heads ({Hkv})")
    d_kernel = kernel_head_dim(D)
    if d_kernel is None:
        raise ValueError(f"head_dim {D} > {KERNEL_HEAD_DIMS[-1]} is not supported")
    if not (0.0 <= dropout_p < 1.0):
        raise ValueError(f"dropout_p must be in [0, 1), got {dropout_p}")
    if q_norm_weight is not None:
        if q.dtype == torch.float32:
            raise ValueError("the fused q RMSNorm runs in bf16/fp16")
        if d_kernel != D:
            raise ValueError(f"the fused q RMSNorm needs head_dim in {KERNEL_HEAD_DIMS}, got {D}")
        if tuple(q_norm_weight.shape) != (D,):
            raise ValueError(f"q_norm_weight must have shape ({D},), got {tuple(q_norm_weight.shape)}")
        if attn_mask is not None or dropout_p > 0.0:
            raise ValueError("the fused q RMSNorm runs without a mask or dropout")
    if scale is None:
        scale = D ** -0.5
    device = q.device
    stream = current_stream_ptr(device)
    lib = nat.load_library()

    if rotary_cos is not None or rotary_sin is not None:
        if rotary_cos is None or rotary_sin is None:
            raise ValueError("rotary_cos and rotary_sin must be given together")
        if D % 2:
            raise ValueError("RoPE needs an even head_dim")
        if rotary_cos.shape[0] < max(Sq, Sk) or rotary_cos.shape[-1] < D // 2:
            raise ValueError("rotary tables are smaller than (seq_len, head_dim/2)")
        if rotary_k:
            from .rope_kernel import rope_apply, rope_template
            rope_tpl = rope_template(k, rotary_cos, rotary_sin) if key is not None else None
            k = rope_apply(k, rotary_cos, rotary_sin)
        if d_kernel != D:
            # RoPE pairs (d, d + D/2) of the unpadded head dim: rotate q
            # here, then pad, rather than fusing at the padded width.
            from .rope_kernel import rope_apply
            q = rope_apply(q, rotary_cos, rotary_sin)
            rotary_cos = rotary_sin = None

    # Decode-shaped calls (few query rows, long KV) take the split-KV kernel;
    # it has no fused RoPE, so q is rotated here first.
    split_kv = (SPLITKV_ENABLED and Sq <= SPLITKV_MAX_SQ and q.dtype != torch.float32 and dropout_p == 0.0
                and d_kernel <= 128 and q_norm_weight is None)
    if split_kv and rotary_cos is not None:
        from .rope_kernel import rope_apply
        q = rope_apply(q, rotary_cos, rotary_sin)
        rotary_cos = rotary_sin = None

    qk = _prepare_operand(q, d_kernel)
    kk = _prepare_operand(k, d_kernel)
    vk = _prepare_operand(v, d_kernel)
    out = torch.empty((B, Sq, H, d_kernel), dtype=q.dtype, device=device)

    args = nat.AttnFwdArgs()
    args.q, args.k, args.v, args.out = qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr()
    lse = None
    if return_lse or keep_state:
        lse = torch.empty((B, H, Sq), dtype=torch.float32, device=device)
        args.lse = lse.data_ptr()
    args.q_stride = nat.int64x4(qk.stride())
    args.k_stride = nat.int64x4(kk.stride())
    args.v_stride = nat.int64x4(vk.stride())
    args.out_stride = nat.int64x4(out.stride())
    args.batch, args.seqlen_q, args.seqlen_k = B, Sq, Sk
    args.nheads_q, args.nheads_kv, args.head_dim = H, Hkv, d_kernel
    args.dtype = _DTYPE_CODE[q.dtype]
    args.softmax_scale = float(scale)
    args.causal = 1 if causal else 0
    if window_size is not None:
        wl, wr = window_size
        args.has_window = 1
        args.window_left, args.window_right = int(wl), int(wr)

    keep = [qk, kk, vk]  # hold references until the launch returns
    if alibi_slopes is not None:
        sl = alibi_slopes
        if sl.dim() == 1:
            sl = sl.unsqueeze(0)
        if sl.dim() != 2 or sl.shape[-1] != H or sl.shape[0] not in (1, B):
            raise ValueError(f"alibi_slopes shape {tuple(alibi_slopes.shape)} must be (H,), (1, H) or (B, H)")
        sl = sl.to(device=device, dtype=torch.float32).contiguous()
        keep.append(sl)
        args.alibi_slopes = sl.data_ptr()
        args.alibi_stride = nat.int64x2((H if sl.shape[0] > 1 else 0, 1))

    if attn_mask is not None:
        m = attn_mask
        if m.device != device:
            m = m.to(device)
        if m.dtype == torch.bool:
            m = m.view(torch.uint8)
        elif m.dtype not in _MASK_DTYPE_CODE:
            m = m.to(torch.float32)
        m4 = TritonAttentionKernel._prepare_mask(m, B, H, Sq, Sk)
        keep.append(m4)
        args.mask = m4.data_ptr()
        args.mask_dtype = _MASK_DTYPE_CODE[m4.dtype]
        args.mask_stride = nat.int64x4(m4.stride())
        if use_blockmap and not split_kv:
            bmap, bst = TritonAttentionKernel.mask_blockmap(m4, stream)
            keep.append(bmap)
            args.mask_blockmap = bmap.data_ptr()
            args.blockmap_stride = nat.int64x2(bst)

    drop_state = keep_map = None
    if dropout_p > 0.0:
        args.dropout_p = float(dropout_p)
        if torch.cuda.is_current_stream_capturing():
            # A seed passed as a kernel argument would be frozen into the
            # graph.  Instead a kernel of the graph copies the device's
            # generator {seed, offset} to this call's own state and advances
            # the generator, and the kernels of this call (forward and
            # backward) read that state: every replay draws a new mask.
            gen = _DROPOUT_GENERATORS.get(device)
            if gen is None:
                raise RuntimeError(
                    "attention dropout under HIP graph capture reads the device's dropout generator, which one "
                    "call with dropout_p > 0 outside the capture creates (the warm-up before capturing)")
            drop_state = torch.empty(2, dtype=torch.int64, device=device)
            nat.check(lib.trinix_dropout_state_advance(gen.data_ptr(), drop_state.data_ptr(), 1, stream),
                      "trinix_dropout_state_advance")
            args.dropout_state = drop_state.data_ptr()
            keep.append(drop_state)
        else:
            dropout_generator(device)
            # Seed from torch's CPU generator: no device->host sync.
            args.dropout_seed = int(torch.randint(0, 2 ** 62, (1,)).item())
            args.dropout_offset = 0
        if keep_state and q.dtype != torch.float32 and d_kernel in (64, 128):
            km_bytes = _keep_map_bytes(device, B, H, Sq, Sk)
            if km_bytes:
                keep_map = torch.empty(km_bytes, dtype=torch.uint8, device=device)
                args.dropout_keep_map = keep_map.data_ptr()
                keep.append(keep_map)

    if rotary_cos is not None:
        cos = rotary_cos.to(device=device, dtype=q.dtype)
        sin = rotary_sin.to(device=device, dtype=q.dtype)
        if cos.stride(-1) != 1 or cos.stride(0) % 8 or cos.data_ptr() % 16:
            cos = cos.contiguous()
        if sin.stride(-1) != 1 or sin.stride(0) != cos.stride(0) or sin.data_ptr() % 16:
            sin = sin.contiguous()
            if sin.stride(0) != cos.stride(0):
                cos = cos.contiguous()
        keep += [cos, sin]
        args.rope_cos, args.rope_sin, args.rope_stride = cos.data_ptr(), sin.data_ptr(), cos.stride(0)

    if q_norm_weight is not None:
        qw = q_norm_weight.detach().to(device=device, dtype=q.dtype)
        if not qw.is_contiguous() or qw.data_ptr() % 16:
            qw = qw.contiguous()
        keep.append(qw)
        args.q_norm_weight, args.q_norm_eps = qw.data_ptr(), float(q_norm_eps)
        if q_norm_out is not None:
            if (q_norm_out.shape != q.shape or q_norm_out.dtype != q.dtype or not q_norm_out.is_contiguous()
                    or q_norm_out.data_ptr() % 16):
                raise ValueError("q_norm_out must be a contiguous, 16-byte aligned tensor shaped and typed like q")
            args.q_norm_out = q_norm_out.data_ptr()

    launched = False
    split_bytes = None
    if split_kv:
        ns, wsb = ctypes.c_int32(0), ctypes.c_int64(0)
        rc = lib.trinix_attn_fwd_splitkv_plan(ctypes.byref(args), ctypes.byref(ns), ctypes.byref(wsb))
        nat.check(rc, "trinix_attn_fwd_splitkv_plan")
        if ns.value > 0:
            ws = torch.empty(wsb.value, dtype=torch.uint8, device=device) if wsb.value else None
            rc = lib.trinix_attn_fwd_splitkv(ctypes.byref(args), None if ws is None else ws.data_ptr(), wsb.value,
                                             stream)
            nat.check(rc, "trinix_attn_fwd_splitkv")
            launched = True
            split_bytes = wsb.value
    if not launched:
        rc = lib.trinix_attn_fwd(ctypes.byref(args), stream)
        nat.check(rc, "trinix_attn_fwd")
    if key is not None and d_kernel == D:
        # the operands went to the kernel as given (no copy, no padding, q
        # not rotated ahead, tables used in place): remember the launch
        in_place = qk is q_in and vk is v_in and (kk is k_in if rope_tpl is None else True)
        if rotary_cos is not None or cos_in is not None:
            in_place = (in_place and rotary_cos is cos_in and args.rope_cos == cos_in.data_ptr()
                        and args.rope_sin == sin_in.data_ptr() and
                        (not rotary_k or (rope_tpl is not None and rope_tpl[-1])))
        if in_place:
            tpl = nat.AttnFwdArgs.from_buffer_copy(args)
            tpl.q = tpl.k = tpl.v = tpl.out = tpl.rope_cos = tpl.rope_sin = None
            if len(_LAUNCHES) >= _MAX_LAUNCHES:
                _LAUNCHES.clear()
            _LAUNCHES[key] = _Launch(tpl, tuple(out.shape), q.dtype, device, 16 if q.element_size() == 2 else 4,
                                     rope_tpl[:-1] if rope_tpl is not None else None, split_bytes)
    state = None
    if keep_state:
        ent = None
        if (tkey is not None and d_kernel == D and qk is q_in and kk is k_in and vk is v_in and drop_state is None
                and q.dtype != torch.float32 and not launched):
            tpl = nat.AttnFwdArgs.from_buffer_copy(args)
            tpl.q = tpl.k = tpl.v = tpl.out = tpl.lse = tpl.dropout_keep_map = None
            tpl.dropout_seed = 0
            if len(_TRAIN_LAUNCHES) >= _MAX_LAUNCHES:
                _TRAIN_LAUNCHES.clear()
            ent = _TrainLaunch(tpl, tuple(out.shape), tuple(lse.shape), q.dtype, device, 16,
                               keep_map.numel() if keep_map is not None else 0, tuple(kk.shape))
            _TRAIN_LAUNCHES[tkey] = ent
        state = dict(q=qk, k=kk, v=vk, out=out, lse=lse, D=D, d_kernel=d_kernel, keep=keep, args=args, launch=ent,
                     dropout=(float(args.dropout_p), int(args.dropout_seed), int(args.dropout_offset)),
                     dropout_state=drop_state, keep_map=keep_map)
    if d_kernel != D:
        out = out[..., :D].contiguous()
    return out, lse, state


def _backward(state, dout):
    """Launch ``trinix_attn_bwd`` for a forward run with ``keep_state``;
    returns (dq, dk, dv) at the caller's head_dim, in the input dtype."""
    ent = state.get("launch")
    if ent is not None and ent.bwd is not None:
        res = _backward_cached(state, ent, dout)
        if res is not None:
            return res
    qk, kk, vk, out, lse = state["q"], state["k"], state["v"], state["out"], state["lse"]
    fa = state["args"]
    D, dkrn = state["D"], state["d_kernel"]
    B, Sq, H, _ = qk.shape
    Sk, Hkv = kk.shape[1], kk.shape[2]
    do = _prepare_operand(dout.to(qk.dtype), dkrn)
    dq = torch.empty((B, Sq, H, dkrn), dtype=qk.dtype, device=qk.device)
    dk = torch.empty((B, Sk, Hkv, dkrn), dtype=qk.dtype, device=qk.device)
    dv = torch.empty((B, Sk, Hkv, dkrn), dtype=qk.dtype, device=qk.device)
    delta = torch.empty((B, H, Sq), dtype=torch.float32, device=qk.device)
    a = nat.AttnBwdArgs()
    a.q, a.k, a.v, a.out, a.dout = qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr(), do.data_ptr()
    a.lse, a.delta = lse.data_ptr(), delta.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    for name, t in (("q", qk), ("k", kk), ("v", vk), ("out", out), ("dout", do), ("dq", dq), ("dk", dk),
                    ("dv", dv)):
        setattr(a, name + "_stride", nat.int64x4(t.stride()))
    a.batch, a.seqlen_q, a.seqlen_k, a.nheads_q, a.nheads_kv, a.head_dim = B, Sq, Sk, H, Hkv, dkrn
    a.dtype = _DTYPE_CODE[qk.dtype]
    a.softmax_scale = fa.softmax_scale
    a.causal, a.has_window = fa.causal, fa.has_window
    a.window_left, a.window_right = fa.window_left, fa.window_right
    a.alibi_slopes, a.alibi_stride = fa.alibi_slopes, fa.alibi_stride
    a.mask, a.mask_dtype, a.mask_stride = fa.mask, fa.mask_dtype, fa.mask_stride
    a.mask_blockmap, a.blockmap_stride = fa.mask_blockmap, fa.blockmap_stride
    a.dropout_p, a.dropout_seed, a.dropout_offset = state["dropout"]
    if state["dropout_state"] is not None:
        a.dropout_state = state["dropout_state"].data_ptr()
    if state["keep_map"] is not None:
        a.dropout_keep_map = state["keep_map"].data_ptr()
    rc = nat.load_library().trinix_attn_bwd(ctypes.byref(a), current_stream_ptr(qk.device))
    nat.check(rc, "trinix_attn_bwd")
    if ent is not None and ent.bwd is None and do is dout and state["dropout_state"] is None:
        tpl = nat.AttnBwdArgs.from_buffer_copy(a)
        tpl.q = tpl.k = tpl.v = tpl.out = tpl.dout = tpl.lse = tpl.delta = tpl.dq = tpl.dk = tpl.dv = None
        tpl.dropout_keep_map = None
        tpl.dropout_seed = 0
        ent.do_stride = tuple(do.stride())
        ent.bwd = tpl
    if dkrn != D:
        dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
    return dq, dk, dv


def _backward_cached(state, ent, dout):
    """(dq, dk, dv) through the layout's backward template, or None when
    dout is not laid out as the template's."""
    if dout.dtype != ent.dtype or dout.stride() != ent.do_stride or dout.data_ptr() % ent.align:
        return None
    dev = ent.device
    a = nat.AttnBwdArgs.from_buffer_copy(ent.bwd)
    dq = torch.empty(ent.out_shape, dtype=ent.dtype, device=dev)
    dk = torch.empty(ent.dk_shape, dtype=ent.dtype, device=dev)
    dv = torch.empty(ent.dk_shape, dtype=ent.dtype, device=dev)
    delta = torch.empty(ent.lse_shape, dtype=torch.float32, device=dev)
    a.q, a.k, a.v = state["q"].data_ptr(), state["k"].data_ptr(), state["v"].data_ptr()
    a.out, a.dout, a.lse, a.delta = state["out"].data_ptr(), dout.data_ptr(), state["lse"].data_ptr(), delta.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    if a.dropout_p > 0.0:
        a.dropout_seed = state["dropout"][1]
        if state["keep_map"] is not None:
            a.dropout_keep_map = state["keep_map"].data_ptr()
    nat.check(nat.load_library().trinix_attn_bwd(ctypes.byref(a), current_stream_ptr(dev)), "trinix_attn_bwd")
    return dq, dk, dv


def _save_output(ctx, state, out, *tensors):
    """Keep the forward's state on ctx.  The returned output, when the state
    holds that very tensor, is saved through autograd instead
    (save_for_backward, after ``tensors``): a reference to it from the node
    that produced it would form a cycle (output -> node -> state -> output),
    so a forward whose output is dropped without a backward would hold its
    buffers (output, lse, dropout keep map) until Python's cycle collector
    runs."""
    if state["out"] is out:
        state["out"] = None
        ctx.save_for_backward(*tensors, out)
    else:
        ctx.save_for_backward(*tensors)
    ctx.state = state


def _saved_state(ctx, n_before=0):
    state = ctx.state
    if state["out"] is None:
        state["out"] = ctx.saved_tensors[n_before]
    return state


class _HipAttnFunction(torch.autograd.Function):
    """Differentiable attention: ``trinix_attn_fwd`` forward (keeping the
    log-sum-exp) and ``trinix_attn_bwd`` backward.  RoPE of q (and of k when
    ``rotary_k``) is applied here before the forward, and the gradients are
    rotated back (the RoPE kernel with -sin) in the backward."""

    @staticmethod
    def forward(ctx, q, k, v, attn_mask, causal, scale, dropout_p, window_size, alibi_slopes, rotary_cos, rotary_sin,
                rotary_k, return_lse):
        from .rope_kernel import rope_apply

        ctx.rope = None
        if rotary_cos is not None:
            q = rope_apply(q, rotary_cos, rotary_sin)
            if rotary_k:
                k = rope_apply(k, rotary_cos, rotary_sin)
            ctx.rope = (rotary_cos, rotary_sin, rotary_k)
        out, lse, state = _forward(q, k, v, attn_mask, causal, scale, dropout_p, window_size, alibi_slopes, None,
                                   None, True, True, True, keep_state=True)
        _save_output(ctx, state, out)
        if return_lse:
            ctx.mark_non_differentiable(lse)
            return out, lse
        return out

    @staticmethod
    def backward(ctx, dout, *unused):
        dq, dk, dv = _backward(_saved_state(ctx), dout.contiguous())
        ctx.state = None
        if ctx.rope is not None:
            from .rope_kernel import rope_apply

            cos, sin, rot_k = ctx.rope
            neg = -sin
            dq = rope_apply(dq, cos, neg)
            if rot_k:
                dk = rope_apply(dk, cos, neg)
        return dq, dk, dv, None, None, None, None, None, None, None, None, None, None


class _HipAttnQNormFunction(torch.autograd.Function):
    """Attention whose q is RoPE-rotated and RMS-normalised in the kernel's
    prologue (the layers' q_norm, reference grouped_query_attention.py:
    171-177), with gradients: the forward kernel also writes the normalised
    q, the attention backward runs on it, and trinix_qk_norm_bwd takes its
    gradient back through the norm and the RoPE to the raw q and the norm
    weight.  k is rotated here (rotary_k) and its gradient rotated back."""

    @staticmethod
    def forward(ctx, q, k, v, weight, eps, causal, scale, window_size, alibi_slopes, rotary_cos, rotary_sin,
                rotary_k):
        from .qk_norm_kernel import _param, _rows_ok, _tables
        from .rope_kernel import rope_apply

        qc = q if _rows_ok(q) else q.contiguous()
        w = _param(weight)
        if rotary_cos is not None and rotary_k:
            k = rope_apply(k, rotary_cos, rotary_sin)
        qn = torch.empty(qc.shape, dtype=qc.dtype, device=qc.device)
        out, _, state = _forward(qc, k, v, None, causal, scale, 0.0, window_size, alibi_slopes, rotary_cos,
                                 rotary_sin, False, True, True, keep_state=True, q_norm_weight=w, q_norm_eps=eps,
                                 q_norm_out=qn)
        state["q"] = qn  # the backward's q: the one attended with
        c, s, _ = _tables(qc, rotary_cos, rotary_sin, None)
        _save_output(ctx, state, out, qc, w, c, s)
        ctx.eps = float(eps)
        ctx.rope_k = (rotary_cos, rotary_sin) if rotary_cos is not None and rotary_k else None
        return out

    @staticmethod
    def backward(ctx, dout):
        from .qk_norm_kernel import NORM_RMS
        from .qk_norm_kernel import _backward as qk_norm_backward
        from .rope_kernel import rope_apply

        qc, w, c, s = ctx.saved_tensors[:4]
        dqn, dk, dv = _backward(_saved_state(ctx, 4), dout.contiguous())
        ctx.state = None
        dq, dw, _ = qk_norm_backward(qc, dqn, w, ctx.eps, c, s, None, NORM_RMS)
        if ctx.rope_k is not None:
            cos, sin = ctx.rope_k
            dk = rope_apply(dk, cos, -sin)
        return dq, dk, dv, dw, None, None, None, None, None, None, None, None


def backward_supported(q: torch.Tensor) -> bool:
    """True if ``trinix_attn_bwd`` covers attention on ``q`` (every dtype the
    forward takes, dropout included, at a kernel head_dim)."""
    return q.dtype in _DTYPE_CODE and kernel_head_dim(q.shape[-1]) in BACKWARD_HEAD_DIMS


def attention(q, k, v, attn_mask=None, causal=False, scale=None, dropout_p=0.0, window_size=None, alibi_slopes=None,
              *, rotary_cos=None, rotary_sin=None, rotary_k=True, return_lse=False, q_norm_weight=None,
              q_norm_eps=1e-6):
    """Attention with gradients when q, k or v require them; otherwise
    ``TritonAttentionKernel.apply``.

    The reference's Triton attention has no backward (its output is detached,
    ``attention_kernel.py:497-517``).  Here it is differentiable through
    ``trinix_attn_bwd`` for fp32, bf16 and fp16, with dropout (the backward
    regenerates the forward's keep mask), head_dim up to 256.  A call the
    backward does not cover while gradients are required raises instead of
    returning a detached output.
    """
    needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
    if q_norm_weight is not None and (needs_grad or (torch.is_grad_enabled() and q_norm_weight.requires_grad)):
        # differentiable through the fused q RoPE + RMSNorm (bf16/fp16, no
        # mask or dropout: the fused norm's own limits, checked by _forward)
        if attn_mask is not None or dropout_p > 0.0:
            raise ValueError("the fused q RMSNorm runs without a mask or dropout")
        if not backward_supported(q):
            raise ValueError(f"no HIP attention backward for dtype {q.dtype}, head_dim {q.shape[-1]}")
        if return_lse:
            raise ValueError("return_lse is not available with a differentiable fused q RMSNorm")
        if scale is None:
            scale = q.shape[-1] ** -0.5
        return _HipAttnQNormFunction.apply(q, k, v, q_norm_weight, q_norm_eps, causal, scale, window_size,
                                           alibi_slopes, rotary_cos, rotary_sin, rotary_k)
    if needs_grad:
        if not backward_supported(q):
            raise ValueError(f"no HIP attention backward for dtype {q.dtype}, head_dim {q.shape[-1]}")
        if scale is None:
            scale = q.shape[-1] ** -0.5
        return _HipAttnFunction.apply(q, k, v, attn_mask, causal, scale, dropout_p, window_size, alibi_slopes,
                                      rotary_cos, rotary_sin, rotary_k, return_lse)
    return TritonAttentionKernel.apply(q, k, v, attn_mask=attn_mask, causal=causal, scale=scale, dropout_p=dropout_p,
                                       window_size=window_size, alibi_slopes=alibi_slopes, rotary_cos=rotary_cos,
                                       rotary_sin=rotary_sin, rotary_k=rotary_k, return_lse=return_lse,
                                       q_norm_weight=q_norm_weight, q_norm_eps=q_norm_eps)


def attention_flops(batch: int, nheads: int, seqlen_q: int, seqlen_k: int, head_dim: int,
                    causal: bool = False, window_size: Optional[Tuple[int, int]] = None) -> int:
    """Algorithmic FLOP = 4 * D * (allowed (i, j) pairs), summed over (b, h).

    Masked-out pairs are not counted.  Pairs follow the kernel's predicate:
    j < Sk, j <= i if causal, -wl <= j - i <= wr with a window.
    """
    return 4 * head_dim * batch * nheads * allowed_pairs(seqlen_q, seqlen_k, causal, window_size)


def allowed_pairs(seqlen_q: int, seqlen_k: int, causal: bool = False,
                  window_size: Optional[Tuple[int, int]] = None) -> int:
    """Number of (i, j) with 0 <= i < Sq, 0 <= j < Sk allowed by causal/window."""
    lo_off = -math.inf
    hi_off = math.inf
    if window_size is not None:
        lo_off, hi_off = -window_size[0], window_size[1]
    if causal:
        hi_off = min(hi_off, 0)
    if lo_off == -math.inf and hi_off == math.inf:
        return seqlen_q * seqlen_k
    # per row i: j in [max(0, i + lo_off), min(Sk - 1, i + hi_off)]
    import numpy as np

    i = np.arange(seqlen_q, dtype=np.int64)
    lo = np.zeros_like(i) if lo_off == -math.inf else np.maximum(0, i + int(lo_off))
    hi = np.full_like(i, seqlen_k - 1) if hi_off == math.inf else np.minimum(seqlen_k - 1, i + int(hi_off))
    return int(np.clip(hi - lo + 1, 0, None).sum())
