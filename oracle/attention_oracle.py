"""CPU oracle for the attention-forward hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``trinix_amd``) imports
this module.  It is imported solely by ``tests/``, by
``__graft_entry__.smoke()`` as the checker, and by ``bench.py``'s
``cpu_baseline`` leg (timed as the CPU baseline, ``kind: "port"``).

It restates, on the CPU with torch ops in the input dtype, the reference
path the north star names as the parity target, the eager
``kernel_type='pytorch'`` backend:

* ``eager_attention``  <- ``FastBaseAttention._apply_pytorch_attention``
  (trinix/layers/attention/base.py:347-400): bmm -> *scale -> causal
  masked_fill(triu(.,1)) -> += mask -> softmax -> bmm, all in q.dtype.
* ``tile_kv_heads``    <- ``FastGroupedQueryAttention._tile_kv_heads``
  (trinix/layers/attention/grouped_query_attention.py:140-145); MQA's stride-0
  ``expand`` (multi_query_attention.py:173-174) is the same mapping.
* ``rope_tables`` / ``apply_rope`` <- ``FastRoPEPositionEmbedding``
  (trinix/layers/embeddings/rope.py:61, 64-79, 111-118).
* ``alibi_slopes`` / ``alibi_bias`` <- ``FastALiBiPositionEmbedding``
  (trinix/layers/embeddings/alibi.py:47-63, 79-90).
* ``window_bias``      <- ``FastBaseAttention._apply_sliding_window_mask``
  (base.py:222-237) with the intended semantics: the reference builds the
  additive mask as ``(1 - w) * -inf``, which is NaN on allowed positions
  (0 * -inf); here allowed -> 0, disallowed -> -inf, for the functional
  window ``-wl <= j - i <= wr`` (trinix/kernels/attention_kernel.py:132-135).
* ``qk_rms_norm``      <- ``FastRMSNorm._pytorch_forward``
  (trinix/layers/norm/rmsnorm.py:62-75), the qk-norm over head_dim the
  layers build at base.py:163-176 and apply after RoPE
  (grouped_query_attention.py:171-177); head_dim <= 2048 always takes this
  path in the reference.
* ``qk_layer_norm``    <- ``FastLayerNorm._pytorch_forward``
  (trinix/layers/norm/layernorm.py:83-88), the qk-norm of
  ``qk_norm_type='layernorm'`` (base.py:167-169): ``F.layer_norm`` with the
  weight and bias cast to the input dtype; head_dim <= 4096 always takes this
  path.  Both norms are differentiable torch ops: their autograd is the
  reference's backward.
* ``functional_attention`` composes them the way the layers feed the eager
  path: window mask + user mask + ALiBi bias summed in fp32
  (base.py:309-319) and added into the q.dtype scores (base.py:392).

Pinning (tests/test_oracle.py): an fp64 closed form (``closed_form``),
brute-force Python loops on tiny shapes (``brute_force``), and special cases
the mathematics fixes (S=1, equal keys, causal row 0, window (0,0), one open
column, zero scale, zero ALiBi slope, RoPE relative-position invariance,
ALiBi slope closed form).  The reference ships no golden vectors; the
build's own fixtures (tests/golden/: inputs and float64 closed-form answers)
are checked against this module in tests/test_golden.py.

``philox4x32_10`` restates the published Philox4x32-10 generator (Salmon et
al., SC'11) for the kernel's dropout stream; it is pinned to the Random123
known-answer vectors.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "eager_attention",
    "tile_kv_heads",
    "rope_tables",
    "apply_rope",
    "qk_layer_norm",
    "alibi_slopes",
    "alibi_bias",
    "window_bias",
    "functional_attention",
    "closed_form",
    "brute_force",
    "philox4x32_10",
    "dropout_keep",
]


# --------------------------------------------------------------------------
# eager path (base.py:347-400)
# --------------------------------------------------------------------------
def eager_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    attn_mask: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                    causal: bool = False, keep: Optional[torch.Tensor] = None,
                    dropout_p: float = 0.0) -> torch.Tensor:
    """``_apply_pytorch_attention``.  q (B,Sq,H,D), k/v (B,Sk,H,D) with H
    equal (tile KV first); mask broadcastable to (B,H,Sq,Sk).  Dropout
    (base.py:395, ``F.dropout`` after the softmax) uses the given keep mask
    (B,H,Sq,Sk) instead of a random draw: w * keep / (1 - dropout_p).
    Returns (B,Sq,H,D) in q.dtype."""
    B, S, H, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = D ** (-0.5)
    qh = q.transpose(1, 2).contiguous().view(B * H, S, D)
    kh = k.transpose(1, 2).contiguous().view(B * H, Sk, D)
    vh = v.transpose(1, 2).contiguous().view(B * H, Sk, D)
    w = torch.bmm(qh, kh.transpose(-2, -1)) * scale
    if causal:
        cm = torch.triu(torch.ones(S, Sk), diagonal=1).bool()
        w.masked_fill_(cm, float("-inf"))
    if attn_mask is not None:
        m = attn_mask
        if m.dim() == 2:
            m = m[None, None]
        elif m.dim() == 3:
            m = m[:, None]
        m = m.expand(B, H, S, Sk).reshape(B * H, S, Sk)
        w += m
    w = F.softmax(w, dim=-1)
    if keep is not None:
        w = w * keep.reshape(B * H, S, Sk).to(w.dtype) * (1.0 / (1.0 - dropout_p))
    out = torch.bmm(w, vh)
    return out.reshape(B, H, S, D).transpose(1, 2)


def tile_kv_heads(x_bshd: torch.Tensor, factor: int) -> torch.Tensor:
    """(B,S,Hkv,D) -> (B,S,Hkv*factor,D); head h reads KV head h // factor."""
    if factor == 1:
        return x_bshd
    b, s, h, d = x_bshd.shape
    return x_bshd[:, :, :, None, :].expand(b, s, h, factor, d).reshape(b, s, h * factor, d)


# --------------------------------------------------------------------------
# position encodings
# --------------------------------------------------------------------------
def rope_tables(seqlen: int, dim: int, base: float, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    inv_freq = 1.0 / base ** (torch.arange(0, dim, 2).float() / dim)
    t = torch.arange(seqlen, dtype=inv_freq.dtype)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x (B,S,H,D); cos/sin (>=S, D) in x.dtype."""
    if position_ids is None:
        c = cos[: x.shape[1]].unsqueeze(0).unsqueeze(2)
        s = sin[: x.shape[1]].unsqueeze(0).unsqueeze(2)
    else:
        c = cos[position_ids].unsqueeze(2)
        s = sin[position_ids].unsqueeze(2)
    return x * c + _rotate_half(x) * s


def qk_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * (x.float() * rsqrt(mean(x.float()**2, -1) + eps)).to(x.dtype),
    in the reference's op order (rmsnorm.py:70-75)."""
    dt = x.dtype
    h = x.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(dt)


def qk_layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float) -> torch.Tensor:
    """F.layer_norm over the last dim with weight and bias cast to x.dtype
    (layernorm.py:83-88)."""
    return F.layer_norm(x, (x.shape[-1],), weight.to(x.dtype), bias.to(x.dtype), eps)


def alibi_slopes(num_heads: int) -> torch.Tensor:
    def pow2(n):
        start = 2 ** (-(2 ** (-(math.log2(n) - 3))))
        ratio = start
        return [start * ratio ** i for i in range(n)]

    if math.log2(num_heads).is_integer():
        sl = pow2(num_heads)
    else:
        c = 2 ** math.floor(math.log2(num_heads))
        sl = pow2(c)
        sl.extend(pow2(2 * c)[0::2][: num_heads - c])
    return torch.tensor(sl, dtype=torch.float32)


def alibi_bias(seqlen_q: int, seqlen_k: int, slopes: torch.Tensor, row0: int = 0, key0: int = 0) -> torch.Tensor:
    """(H, Sq, Sk) fp32 bias ``-slope * |i - j|`` (alibi.py:79-90) for query
    positions row0.. and key positions key0..."""
    pos = (torch.arange(seqlen_k) + key0).unsqueeze(0) - (torch.arange(seqlen_q) + row0).unsqueeze(1)
    pos = pos.abs()
    return -(pos.unsqueeze(0) * slopes.float().view(-1, 1, 1))


def window_bias(seqlen_q: int, seqlen_k: int, wl: int, wr: int, row0: int = 0, key0: int = 0,
                causal: bool = False) -> torch.Tensor:
    """(Sq, Sk) fp32: 0 where -wl <= j - i <= wr (and j <= i if causal),
    else -inf, for query positions row0.. and key positions key0..."""
    d = (torch.arange(seqlen_k) + key0).unsqueeze(0) - (torch.arange(seqlen_q) + row0).unsqueeze(1)
    ok = (d >= -wl) & (d <= wr)
    if causal:
        ok &= d <= 0
    m = torch.zeros(seqlen_q, seqlen_k)
    m[~ok] = float("-inf")
    return m


# --------------------------------------------------------------------------
# the functional semantics, evaluated through the eager path
# --------------------------------------------------------------------------
def functional_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         attn_mask: Optional[torch.Tensor] = None, softmax_scale: Optional[float] = None,
                         causal: bool = False, window_size: Optional[Tuple[int, int]] = None,
                         alibi_slopes: Optional[torch.Tensor] = None,
                         heads: Optional[Sequence[int]] = None, batches: Optional[Sequence[int]] = None,
                         head_chunk: int = 1, keep: Optional[torch.Tensor] = None,
                         dropout_p: float = 0.0, rows: Optional[Tuple[int, int]] = None,
                         keys: Optional[Tuple[int, int]] = None) -> torch.Tensor:
    """What ``triton_attn_func`` computes, on the CPU through ``eager_attention``.

    GQA/MQA KV is tiled (grouped_query_attention.py:140-145).  Window, user
    mask and ALiBi bias are summed in fp32 into one additive mask, as the
    layers do (base.py:222-237, 309-319), then added to the q.dtype scores.
    ``heads`` / ``batches`` restrict the evaluation to a subset (heads are
    independent); results are (len(batches), Sq, len(heads), D).  The work is
    chunked over (b, head_chunk heads) to bound the S^2 score memory.
    ``keep`` (B,H,Sq,Sk) bool with ``dropout_p``: dropout with that mask
    (``dropout_keep`` gives the kernel's).

    ``rows`` = (r0, r1) evaluates query rows r0..r1-1 only (a row band: rows
    are independent), ``keys`` = (k0, k1) restricts the keys to k0..k1-1,
    which must hold every key the causal / window band lets those rows see
    (checked).  With either, causal and window masks are folded into the
    additive mask at the absolute positions (0 / -inf added to the scores,
    the same values masked_fill gives).
    """
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if softmax_scale is None:
        softmax_scale = D ** (-0.5)
    heads = list(range(H)) if heads is None else list(heads)
    batches = list(range(B)) if batches is None else list(batches)
    factor = H // Hkv
    r0, k0 = 0, 0
    if rows is not None or keys is not None:
        r0, r1 = rows if rows is not None else (0, Sq)
        k0, k1 = keys if keys is not None else (0, Sk)
        lo, hi = -math.inf, math.inf
        if window_size is not None:
            lo, hi = -window_size[0], window_size[1]
        if causal:
            hi = min(hi, 0)
        # keys rows r0..r1-1 may see: [max(0, r0 + lo), min(Sk - 1, r1 - 1 + hi)]
        need_lo = 0 if lo == -math.inf else max(0, r0 + lo)
        need_hi = Sk - 1 if hi == math.inf else min(Sk - 1, r1 - 1 + hi)
        assert k0 <= need_lo and k1 - 1 >= need_hi, "key range does not cover the rows' band"
        q = q[:, r0:r1]
        k = k[:, k0:k1]
        v = v[:, k0:k1]
        if attn_mask is not None and attn_mask.shape[-2] != 1:
            attn_mask = attn_mask[..., r0:r1, :]
        if attn_mask is not None and attn_mask.shape[-1] != 1:
            attn_mask = attn_mask[..., k0:k1]
        if keep is not None:
            keep = keep[:, :, r0:r1, k0:k1]
        wl, wr = (window_size if window_size is not None else (Sk + Sq, Sk + Sq))
        Sq, Sk = r1 - r0, k1 - k0
        window_size = (int(wl), int(wr))
    base = None
    if window_size is not None:
        base = window_bias(Sq, Sk, int(window_size[0]), int(window_size[1]), r0, k0,
                           causal=causal and (r0, k0) != (0, 0))
    causal_in_eager = causal and (r0, k0) == (0, 0)
    user = None
    if attn_mask is not None:
        user = attn_mask.float()
        if user.dim() == 2:
            user = user[None, None]
        elif user.dim() == 3:
            user = user[:, None]
    slopes = None
    if alibi_slopes is not None:
        slopes = alibi_slopes.float().reshape(-1, H)
    outs = []
    for b in batches:
        row = []
        for h0 in range(0, len(heads), head_chunk):
            hs = heads[h0:h0 + head_chunk]
            qs = q[b:b + 1, :, hs]
            ks = torch.stack([k[b, :, h // factor] for h in hs], dim=1).unsqueeze(0)
            vs = torch.stack([v[b, :, h // factor] for h in hs], dim=1).unsqueeze(0)
            m = None
            if base is not None:
                m = base[None, None].expand(1, len(hs), Sq, Sk)
            if user is not None:
                ub = user[b if user.shape[0] > 1 else 0]
                ub = torch.stack([ub[h if ub.shape[0] > 1 else 0] for h in hs])[None]
                m = ub if m is None else m + ub
            if slopes is not None:
                sb = slopes[b if slopes.shape[0] > 1 else 0]
                ab = alibi_bias(Sq, Sk, sb[hs], r0, k0)[None]
                m = ab if m is None else m + ab
            kp = None if keep is None else keep[b:b + 1, hs]
            row.append(eager_attention(qs, ks, vs, m, softmax_scale, causal_in_eager, kp, dropout_p))
        outs.append(torch.cat(row, dim=2))
    return torch.cat(outs, dim=0)


# --------------------------------------------------------------------------
# fp64 closed form and brute force (pins for the restatement above)
# --------------------------------------------------------------------------
def _bias64(Sq, Sk, H, B, attn_mask, causal, window_size, alibi_slopes, row_pos=None):
    bias = np.zeros((B, H, Sq, Sk), dtype=np.float64)
    i = (np.arange(Sq) if row_pos is None else np.asarray(row_pos))[:, None]
    j = np.arange(Sk)[None, :]
    allowed = np.ones((Sq, Sk), dtype=bool)
    if causal:
        allowed &= j <= i
    if window_size is not None:
        allowed &= (j - i >= -window_size[0]) & (j - i <= window_size[1])
    if alibi_slopes is not None:
        sl = alibi_slopes.double().reshape(-1, H).numpy()
        bias += -sl[:, :, None, None] * np.abs(i - j)[None, None].astype(np.float64)
    if attn_mask is not None:
        m = attn_mask.double()
        if m.dim() == 2:
            m = m[None, None]
        elif m.dim() == 3:
            m = m[:, None]
        if row_pos is not None and m.shape[-2] != 1:
            m = m[..., list(row_pos), :]
        bias = bias + np.broadcast_to(m.numpy(), (B, H, Sq, Sk))
    bias = np.where(allowed[None, None], bias, -np.inf)
    return bias


def closed_form(q, k, v, attn_mask=None, softmax_scale=None, causal=False, window_size=None,
                alibi_slopes=None, keep=None, dropout_p=0.0, row_pos=None) -> np.ndarray:
    """float64 ``softmax(q k^T * scale + bias) v`` from the same (rounded)
    inputs; GQA by ``h // (H/Hkv)``; with ``keep`` (B,H,Sq,Sk) the
    probabilities are multiplied by keep / (1 - dropout_p).  ``row_pos``
    gives the absolute positions of q's rows (q holds only those rows; the
    mask is indexed by them).  Returns (B,Sq,H,D) float64."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if softmax_scale is None:
        softmax_scale = D ** (-0.5)
    qd = q.double().numpy()
    kd = np.repeat(k.double().numpy(), H // Hkv, axis=2)
    vd = np.repeat(v.double().numpy(), H // Hkv, axis=2)
    s = np.einsum("bihd,bjhd->bhij", qd, kd) * softmax_scale
    s = s + _bias64(Sq, Sk, H, B, attn_mask, causal, window_size, alibi_slopes, row_pos)
    with np.errstate(invalid="ignore"):
        mx = s.max(axis=-1, keepdims=True)
        p = np.exp(s - mx)
        p = p / p.sum(axis=-1, keepdims=True)
    if keep is not None:
        p = p * np.asarray(keep, dtype=np.float64) / (1.0 - dropout_p)
    return np.einsum("bhij,bjhd->bihd", p, vd)


def brute_force(q, k, v, attn_mask=None, softmax_scale=None, causal=False, window_size=None,
                alibi_slopes=None) -> list:
    """Pure-Python loops (tiny shapes only): nested lists [b][i][h][d]."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if softmax_scale is None:
        softmax_scale = D ** (-0.5)
    Q, K, V = q.double().tolist(), k.double().tolist(), v.double().tolist()
    M = None
    if attn_mask is not None:
        M = attn_mask.double()
        while M.dim() < 4:
            M = M.unsqueeze(0) if M.dim() == 2 else M.unsqueeze(1)
        M = M.expand(B, H, Sq, Sk).tolist()
    SL = None if alibi_slopes is None else alibi_slopes.double().reshape(-1, H).tolist()
    out = [[[[0.0] * D for _ in range(H)] for _ in range(Sq)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            for i in range(Sq):
                scores = []
                for j in range(Sk):
                    ok = True
                    if causal and j > i:
                        ok = False
                    if window_size is not None and not (-window_size[0] <= j - i <= window_size[1]):
                        ok = False
                    if not ok:
                        scores.append(-math.inf)
                        continue
                    s = sum(Q[b][i][h][d] * K[b][j][hk][d] for d in range(D)) * softmax_scale
                    if SL is not None:
                        s += -SL[b if len(SL) > 1 else 0][h] * abs(i - j)
                    if M is not None:
                        s += M[b][h][i][j]
                    scores.append(s)
                mx = max(scores)
                if mx == -math.inf:
                    for d in range(D):
                        out[b][i][h][d] = math.nan
                    continue
                e = [math.exp(s - mx) if s != -math.inf else 0.0 for s in scores]
                tot = sum(e)
                for d in range(D):
                    out[b][i][h][d] = sum(e[j] * V[b][j][hk][d] for j in range(Sk)) / tot
    return out


# --------------------------------------------------------------------------
# Philox4x32-10 and the kernel's dropout stream
# --------------------------------------------------------------------------
_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint64(0x9E3779B9), np.uint64(0xBB67AE85)
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: Tuple[int, int]) -> np.ndarray:
    """ctr: (..., 4) uint32 counters; key: (k0, k1).  Returns (..., 4) uint32."""
    c = [np.asarray(ctr[..., t], dtype=np.uint64) for t in range(4)]
    k0, k1 = np.uint64(key[0]), np.uint64(key[1])
    for _ in range(10):
        p0 = _M0 * c[0]
        p1 = _M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & _MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & _MASK32
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + _W0) & _MASK32
        k1 = (k1 + _W1) & _MASK32
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def dropout_keep(batch: int, nheads: int, seqlen_q: int, seqlen_k: int, p: float, seed: int,
                 offset: int = 0) -> np.ndarray:
    """Keep mask (B,H,Sq,Sk) of the kernel's dropout: for key j of row i of
    (b, h), the Philox call with counter (j >> 3, i, b*H + h, offset_lo) and
    key (seed_lo ^ offset_hi, seed_hi) gives four words; key j takes 16-bit
    field j & 7 of them (word (j & 7) >> 1, the low half for even j) and is
    dropped iff that field < floor(p * 2^16) (kernels: csrc/common.h
    keep_field, dropout_pair in attn_params.h, keep_bits_of_key in
    attn_bwd16.h)."""
    thresh = min(int(p * 65536.0), 65535)
    ngrp = -(-seqlen_k // 8)
    bh = np.arange(batch * nheads, dtype=np.uint32)[:, None, None]
    ii = np.arange(seqlen_q, dtype=np.uint32)[None, :, None]
    gg = np.arange(ngrp, dtype=np.uint32)[None, None, :]
    shape = (batch * nheads, seqlen_q, ngrp)
    ctr = np.stack([np.broadcast_to(gg, shape), np.broadcast_to(ii, shape), np.broadcast_to(bh, shape),
                    np.full(shape, offset & 0xFFFFFFFF, dtype=np.uint32)], axis=-1)
    key = ((seed & 0xFFFFFFFF) ^ ((offset >> 32) & 0xFFFFFFFF), (seed >> 32) & 0xFFFFFFFF)
    words = philox4x32_10(ctr, key)  # (BH, Sq, ngrp, 4)
    fields = np.stack([words & np.uint32(0xFFFF), words >> np.uint32(16)], axis=-1)  # field k = word k>>1, half k&1
    fields = fields.reshape(batch * nheads, seqlen_q, ngrp * 8)[:, :, :seqlen_k]
    return (fields >= np.uint32(thresh)).reshape(batch, nheads, seqlen_q, seqlen_k)
