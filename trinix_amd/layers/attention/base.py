"""FastBaseAttention: backend dispatch, position encodings and masks
(reference ``trinix/layers/attention/base.py``), with the GPU attention on
the gfx950 HIP kernels.

Behaviour kept from the reference: constructor kwargs and defaults
(``base.py:106-123``), ``scale = head_dim ** -0.5``, the eager
``kernel_type='pytorch'`` backend (``base.py:347-400``), ``add_zero_attn``,
mask / bias merging, and the ValueError/TypeError/AssertionError behaviour of
the constructor.

Decisions where the reference is defective (kept in one place here):
* ``'flash'`` (the default) and ``'triton'`` run the HIP kernel with every
  feature; there is no silent fallback to the eager path: a HIP failure
  raises (reference: catch-all fallback, ``base.py:435-439``; ``'flash'``
  with a mask falls back, ``base.py:448-452``).
* the sliding window is ``i - w <= j <= i`` (the eager mask's intent,
  ``base.py:227-231``) without the ``0 * -inf = NaN`` of ``base.py:232``;
  on the HIP path it is the kernel's window ``(w, 0)``, not the reference
  Triton path's symmetric ``(w, w)`` (``base.py:419-421``).
* ALiBi is applied once, as per-head slopes inside the kernel (the reference
  Triton path adds it twice: merged into the mask and as slopes,
  ``base.py:309-319,415-417``); the eager path adds the materialised bias.
* GQA/MQA key/value heads reach the kernel un-repeated (no copy).
"""
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from ...kernels.attention_kernel import TritonAttentionKernel, attention


class _QKRMSNorm(nn.Module):
    """Eager RMSNorm over head_dim (reference FastRMSNorm's PyTorch path)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dt = x.dtype
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * h.to(dt)


class _QKLayerNorm(nn.Module):
    """Eager LayerNorm over head_dim (reference FastLayerNorm's PyTorch path)."""

    def __init__(self, hidden_size: int, eps: float = 1e-5):
        super().__init__()
        self.normalized_shape = (hidden_size,)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.bias = nn.Parameter(torch.zeros(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.layer_norm(x, self.normalized_shape, self.weight.to(x.dtype), self.bias.to(x.dtype), self.eps)


class FastBaseAttention(nn.Module):
    """Base attention layer; see the module docstring.

    Args (reference ``base.py:106-123``): embed_dim, num_heads, dropout=0.0,
    bias=True, kernel_type='flash' ('flash' | 'triton' -> HIP kernel,
    'pytorch' -> eager), causal=False, position_method='none' ('rope' |
    'alibi' | 'none' | nn.Module), max_seq_len=2048, rope_base=10000.0,
    use_sliding_window=False, sliding_window_size=None, qk_norm=False,
    qk_norm_type='rmsnorm', use_triton_norm=True, use_triton_embeddings=True,
    add_zero_attn=False.

    ``fuse_q_norm_in_attention`` (class attribute, default True): with the
    fused qk RMSNorm in inference, q's RoPE and norm run in the attention
    kernel's prologue (bitwise the same q) instead of their own pass.
    """

    fuse_q_norm_in_attention = True

    def __init__(
        self,
        embed_dim: int,
        num_heads: int,
        dropout: float = 0.0,
        bias: bool = True,
        kernel_type: str = "flash",
        causal: bool = False,
        position_method: Union[str, nn.Module] = "none",
        max_seq_len: int = 2048,
        rope_base: float = 10000.0,
        use_sliding_window: bool = False,
        sliding_window_size: Optional[int] = None,
        qk_norm: bool = False,
        qk_norm_type: str = "rmsnorm",
        use_triton_norm: bool = True,
        use_triton_embeddings: bool = True,
        add_zero_attn: bool = False,
    ):
        super().__init__()
        assert embed_dim % num_heads == 0, f"embed_dim ({embed_dim}) must be divisible by num_heads ({num_heads})"
        assert num_heads > 0, f"num_heads must be positive, got {num_heads}"
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.dropout = dropout
        self.causal = causal
        self.kernel_type = kernel_type
        self.use_sliding_window = use_sliding_window
        self.sliding_window_size = sliding_window_size
        self.qk_norm = qk_norm
        self.qk_norm_type = qk_norm_type
        self.add_zero_attn = add_zero_attn
        self.max_seq_len = max_seq_len
        self.scale = self.head_dim ** (-0.5)

        self._validate_position_method(position_method)
        self.position_method = position_method if isinstance(position_method, str) else "custom"
        self._setup_position_embedding(position_method, max_seq_len, rope_base, use_triton_embeddings)

        if qk_norm:
            if qk_norm_type == "rmsnorm":
                self.q_norm, self.k_norm = _QKRMSNorm(self.head_dim), _QKRMSNorm(self.head_dim)
            elif qk_norm_type == "layernorm":
                self.q_norm, self.k_norm = _QKLayerNorm(self.head_dim), _QKLayerNorm(self.head_dim)
            else:
                raise ValueError(f"Invalid qk_norm_type: {qk_norm_type}. Use 'rmsnorm' or 'layernorm'")
        else:
            self.q_norm = None
            self.k_norm = None

    # -- configuration -------------------------------------------------------
    def _validate_position_method(self, position_method):
        if isinstance(position_method, str):
            assert position_method in ["rope", "alibi", "none"] or position_method.startswith("custom"), (
                f"Invalid position_method: {position_method}. Use 'rope', 'alibi', 'none', or provide a custom nn.Module."
            )
        elif not isinstance(position_method, nn.Module):
            raise TypeError(f"position_method must be a string or nn.Module, got {type(position_method)}")

    def _setup_position_embedding(self, position_method, max_seq_len, rope_base, use_triton_embeddings):
        from ..embeddings import FastALiBiPositionEmbedding, FastRoPEPositionEmbedding

        if isinstance(position_method, nn.Module):
            self.position_embedding = position_method
        elif position_method == "rope":
            self.position_embedding = FastRoPEPositionEmbedding(
                dim=self.head_dim, max_position_embeddings=max_seq_len, base=rope_base,
                use_triton=use_triton_embeddings)
        elif position_method == "alibi":
            self.position_embedding = FastALiBiPositionEmbedding(
                num_heads=self.num_heads, max_seq_len=max_seq_len, use_triton=use_triton_embeddings)
        else:
            self.position_embedding = None

    def _uses_kernel(self, t: torch.Tensor) -> bool:
        return self.kernel_type in ("flash", "triton") and t.is_cuda

    # -- masks and position encodings ---------------------------------------
    def _window_size(self) -> Optional[Tuple[int, int]]:
        if self.use_sliding_window and self.sliding_window_size is not None:
            return (int(self.sliding_window_size), 0)
        return None

    def _apply_sliding_window_mask(self, attention_mask, seq_len, device, seq_len_q=None):
        """Additive (Sq, Sk) window mask for the eager path: 0 where
        i - w <= j <= i, -inf elsewhere (reference base.py:222-237 intent)."""
        if not self.use_sliding_window or self.sliding_window_size is None:
            return attention_mask
        sq = seq_len if seq_len_q is None else seq_len_q
        d = torch.arange(seq_len, device=device).unsqueeze(0) - torch.arange(sq, device=device).unsqueeze(1)
        ok = (d >= -self.sliding_window_size) & (d <= 0)
        window_mask = torch.zeros(sq, seq_len, device=device).masked_fill(~ok, float("-inf"))
        return window_mask if attention_mask is None else attention_mask + window_mask

    def _apply_position_embedding(self, q, k, seq_len_q, seq_len_k=None, batch_size=None, position_ids=None):
        """Returns (q, k, position_bias); reference base.py:239-285.  ALiBi
        returns no bias here: the slopes are applied inside the attention
        (kernel) or materialised by the eager path."""
        if seq_len_k is None:
            seq_len_k = seq_len_q
        if batch_size is None:
            batch_size = q.shape[0]
        position_bias = None
        max_seq_len = max(seq_len_q, seq_len_k)
        if self.position_method == "rope" and self.position_embedding is not None:
            cos, sin = self.position_embedding(q, max_seq_len)
            q, k = self.position_embedding.apply_rotary_pos_emb(q, k, cos, sin, position_ids)
        elif self.position_method == "custom" and self.position_embedding is not None:
            q, k, position_bias = self._custom_position(q, k, seq_len_q, seq_len_k, batch_size, position_ids)
        return q, k, position_bias

    def _custom_position(self, q, k, seq_len_q, seq_len_k, batch_size, position_ids):
        """A user position module, called with the calling convention user
        modules are written against (reference base.py:239-285): the full
        argument list first; if that signature does not fit (TypeError), just
        (q, k); if that fails as well, no arguments (a module that returns a
        precomputed bias).  With the full list a 3-tuple is (q, k, bias) and
        a 2-tuple (q, k); with (q, k) any tuple is (q, k); any other result is
        the additive bias."""
        emb = self.position_embedding
        full_args = (q, k, seq_len_q, seq_len_k, batch_size, position_ids)
        try:
            out = emb(*full_args)
        except TypeError:
            out = None
        else:
            if isinstance(out, tuple) and len(out) in (2, 3):
                return (*out, None) if len(out) == 2 else out
            return q, k, out
        try:
            out = emb(q, k)
        except Exception:
            return q, k, emb()
        if isinstance(out, tuple):
            q2, k2 = out
            return q2, k2, None
        return q, k, out

    def _alibi_slopes(self) -> Optional[torch.Tensor]:
        if self.position_method == "alibi" and self.position_embedding is not None:
            return self.position_embedding.slopes
        return None

    def _add_zero_attention(self, k, v, attention_mask):
        """Appends one all-zero key/value (k, v in (B, H, S, D)); reference base.py:287-307."""
        if not self.add_zero_attn:
            return k, v, attention_mask
        bs, nh, _, hd = k.shape
        k = torch.cat([k, torch.zeros(bs, nh, 1, hd, dtype=k.dtype, device=k.device)], dim=2)
        v = torch.cat([v, torch.zeros(bs, v.shape[1], 1, hd, dtype=v.dtype, device=v.device)], dim=2)
        if attention_mask is not None:
            m = attention_mask
            while m.dim() < 4:
                m = m.unsqueeze(0)
            m = m.expand(bs, -1, -1, -1) if m.shape[0] == 1 else m
            zero = torch.zeros(*m.shape[:3], 1, dtype=m.dtype, device=m.device)
            attention_mask = torch.cat([m, zero], dim=-1)
        return k, v, attention_mask

    def _merge_position_bias(self, attention_mask, position_bias):
        if position_bias is not None:
            attention_mask = position_bias if attention_mask is None else attention_mask + position_bias
        return attention_mask

    # -- backends -------------------------------------------------------------
    def _apply_pytorch_attention(self, q, k, v, attn_mask=None):
        """Eager backend (reference base.py:347-400): bmm -> *scale -> causal
        masked_fill -> += mask -> softmax -> dropout -> bmm, in q.dtype.  KV
        with fewer heads than q is tiled first (grouped_query_attention.py:140-145)."""
        batch_size, seq_len, num_heads, head_dim = q.shape
        seq_len_k = k.shape[1]
        if k.shape[2] != num_heads:
            f = num_heads // k.shape[2]
            k = k[:, :, :, None, :].expand(-1, -1, -1, f, -1).reshape(batch_size, seq_len_k, num_heads, head_dim)
            v = v[:, :, :, None, :].expand(-1, -1, -1, f, -1).reshape(batch_size, seq_len_k, num_heads, head_dim)
        qh = q.transpose(1, 2).contiguous().view(batch_size * num_heads, seq_len, head_dim)
        kh = k.transpose(1, 2).contiguous().view(batch_size * num_heads, seq_len_k, head_dim)
        vh = v.transpose(1, 2).contiguous().view(batch_size * num_heads, seq_len_k, head_dim)
        # k^T materialised: ROCm's batched bf16 GEMM with a transposed-view
        # right operand is a known GPU fault on this platform, so the eager
        # path only multiplies by a contiguous k^T; the products are the same.
        w = torch.bmm(qh, kh.transpose(-2, -1).contiguous()) * self.scale
        if self.causal:
            w.masked_fill_(torch.triu(torch.ones(seq_len, seq_len_k, device=q.device), diagonal=1).bool(),
                           float("-inf"))
        slopes = self._alibi_slopes()
        if slopes is not None:
            pos = torch.arange(seq_len_k, device=q.device).unsqueeze(0) - torch.arange(seq_len, device=q.device).unsqueeze(1)
            bias = -(pos.abs().unsqueeze(0) * slopes.to(q.device).view(-1, 1, 1))
            bias = bias.unsqueeze(0).expand(batch_size, -1, -1, -1)
            attn_mask = bias if attn_mask is None else attn_mask + bias
        if attn_mask is not None:
            m = attn_mask
            if m.dim() == 2:
                m = m[None, None]
            elif m.dim() == 3:
                m = m[:, None]
            w += m.expand(batch_size, num_heads, seq_len, seq_len_k).reshape(batch_size * num_heads, seq_len, seq_len_k)
        w = F.softmax(w, dim=-1)
        w = F.dropout(w, p=self.dropout, training=self.training)
        out = torch.bmm(w, vh)
        return out.reshape(batch_size, num_heads, seq_len, head_dim).transpose(1, 2)

    def _apply_triton_attention(self, q, k, v, attn_mask=None, rotary=None, q_norm=None):
        """HIP kernel backend (reference base.py:402-439), no fallback."""
        if not TritonAttentionKernel.is_available():
            raise RuntimeError("HIP attention kernel not available (build trinix_amd; needs a gfx950 GPU)")
        kw = {}
        if rotary is not None:
            kw = dict(rotary_cos=rotary[0], rotary_sin=rotary[1], rotary_k=False)
        if q_norm is not None:
            kw.update(q_norm_weight=q_norm.weight, q_norm_eps=q_norm.eps)
        return attention(
            q, k, v, attn_mask=attn_mask, causal=self.causal, scale=self.scale,
            dropout_p=self.dropout if self.training else 0.0, window_size=self._window_size(),
            alibi_slopes=self._alibi_slopes(), **kw)

    _apply_flash_attention = _apply_triton_attention

    def forward_attention(self, q, k, v, attn_mask=None):
        """q (B, Sq, H, D); k, v (B, Sk, Hkv, D) with Hkv dividing H."""
        if self._uses_kernel(q):
            return self._apply_triton_attention(q, k, v, attn_mask)
        if self.use_sliding_window and self.sliding_window_size is not None:
            attn_mask = self._apply_sliding_window_mask(attn_mask, k.shape[1], q.device, q.shape[1])
        return self._apply_pytorch_attention(q, k, v, attn_mask)

    def _fused_qk_norm_applies(self, q, k) -> bool:
        """qk-norm (+ RoPE) through the fused kernels (differentiable): GPU
        kernel path, a supported head_dim, RoPE / ALiBi / no position
        encoding; RMSNorm weights in the activations' 16-bit dtype (the eager
        module's output is then that dtype), LayerNorm weights of any float
        dtype (the eager module casts them to the activations' dtype)."""
        if not (self.qk_norm and self._uses_kernel(q)):
            return False
        if self.position_method not in ("rope", "alibi", "none"):
            return False
        from ...kernels.qk_norm_kernel import qk_norm_supported

        if isinstance(self.q_norm, _QKRMSNorm):
            return qk_norm_supported(q, self.q_norm.weight) and qk_norm_supported(k, self.k_norm.weight)
        if isinstance(self.q_norm, _QKLayerNorm):
            return (qk_norm_supported(q, self.q_norm.weight.detach().to(q.dtype))
                    and qk_norm_supported(k, self.k_norm.weight.detach().to(k.dtype)))
        return False

    def _fused_qk_norm(self, norm, x, cos, sin, position_ids):
        """The layer's q_norm / k_norm module applied (after RoPE when
        cos/sin are given) by the fused kernel."""
        from ...kernels.qk_norm_kernel import qk_layernorm, qk_rmsnorm

        if isinstance(norm, _QKLayerNorm):
            return qk_layernorm(x, norm.weight.to(x.dtype), norm.bias.to(x.dtype), norm.eps, cos, sin, position_ids)
        return qk_rmsnorm(x, norm.weight, norm.eps, cos, sin, position_ids)

    # -- shared layer body ------------------------------------------------------
    def _attend(self, q, k, v, attention_mask, position_ids, past_key_value, use_zero_attn):
        """q (B, Sq, H, D), k/v (B, Sk, Hkv, D) after projection.  Returns
        (out (B, Sq, H, D), k_cache, v_cache) with the caches in (B, Hkv, S, D)."""
        bs, seq_len_q = q.shape[0], q.shape[1]
        seq_len_k = k.shape[1]
        rotary = None
        fuse_rope = (self.position_method == "rope" and self.position_embedding is not None and q.is_cuda
                     and self._uses_kernel(q) and position_ids is None and not self.qk_norm
                     and past_key_value is None and not (use_zero_attn and self.add_zero_attn))
        fuse_norm = self._fused_qk_norm_applies(q, k)
        # q's RoPE + RMSNorm in the attention kernel's prologue (positions are
        # the query rows: no position_ids, no cache, no zero-attention row;
        # that kernel takes no mask and no dropout).  In training the kernel
        # also writes the normalised q for the backward, which then runs the
        # attention backward and the qk-norm backward.
        fuse_qnorm = (self.fuse_q_norm_in_attention and fuse_norm and isinstance(self.q_norm, _QKRMSNorm)
                      and position_ids is None and past_key_value is None
                      and not (use_zero_attn and self.add_zero_attn) and q.shape[-1] in (64, 128, 256)
                      and attention_mask is None and not (self.training and self.dropout > 0.0))
        if fuse_rope:
            # q is rotated inside the attention kernel; k by the RoPE kernel
            # (it is also the returned cache).
            cos, sin = self.position_embedding(q, max(seq_len_q, seq_len_k))
            from ...kernels.rope_kernel import rotate

            k = rotate(k, cos, sin)
            rotary = (cos, sin)
        elif fuse_norm:
            # RoPE (if any) and the qk-norm in one kernel pass per tensor
            # (the eager order: rotate, then normalise).
            cos = sin = None
            if self.position_method == "rope" and self.position_embedding is not None:
                cos, sin = self.position_embedding(q, max(seq_len_q, seq_len_k))
            if fuse_qnorm:
                rotary = (cos, sin) if cos is not None else None
            else:
                q = self._fused_qk_norm(self.q_norm, q, cos, sin, position_ids)
            k = self._fused_qk_norm(self.k_norm, k, cos, sin, position_ids)
            attention_mask = self._merge_position_bias(attention_mask, None)
        else:
            q, k, position_bias = self._apply_position_embedding(q, k, seq_len_q, seq_len_k, bs, position_ids)
            attention_mask = self._merge_position_bias(attention_mask, position_bias)
        q = q.transpose(1, 2)
        k = k.transpose(1, 2)
        v = v.transpose(1, 2)
        if self.qk_norm and not fuse_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)
        if past_key_value is not None:
            past_k, past_v = past_key_value
            k = torch.cat([past_k, k], dim=-2)
            v = torch.cat([past_v, v], dim=-2)
        k_cache, v_cache = k, v
        if use_zero_attn:
            k, v, attention_mask = self._add_zero_attention(k, v, attention_mask)
        q = q.transpose(1, 2)
        k = k.transpose(1, 2)
        v = v.transpose(1, 2)
        if self._uses_kernel(q):
            out = self._apply_triton_attention(q, k, v, attention_mask, rotary, self.q_norm if fuse_qnorm else None)
        else:
            out = self.forward_attention(q, k, v, attention_mask)
        return out, k_cache, v_cache
