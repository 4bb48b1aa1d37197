"""The five benchmark/parity workloads (BASELINE configs C1..C5) and their
seeded synthetic inputs.

Inputs are drawn in fp32 on the CPU from ``torch.Generator().manual_seed``
and then cast to the workload dtype, so every consumer (GPU kernel, CPU
oracle, benchmark) sees identical bits.  RoPE tables follow the reference
``FastRoPEPositionEmbedding`` (``trinix/layers/embeddings/rope.py:61,69-79``):
``inv_freq = 1 / base**(arange(0, D, 2)/D)`` in fp32, ``cos/sin`` of
``cat(t*inv_freq, t*inv_freq)`` cast to the input dtype.  ALiBi slopes follow
``FastALiBiPositionEmbedding._get_slopes`` (``trinix/layers/embeddings/alibi.py:47-63``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional, Sequence, Tuple

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    seqlen: int
    nheads: int
    nheads_kv: int
    head_dim: int
    dtype: torch.dtype
    causal: bool = False
    window: Optional[Tuple[int, int]] = None
    rope_base: Optional[float] = None
    alibi: bool = False
    block_mask: bool = False
    seed: int = 0
    description: str = ""


WORKLOADS = {
    "c1": Workload("c1", 2, 128, 8, 8, 64, torch.float32, seed=1,
                   description="fp32 MHA, non-causal (plumbing / fp32 parity)"),
    "c2": Workload("c2", 4, 1024, 12, 12, 64, torch.bfloat16, causal=True, seed=2,
                   description="GPT-2-small causal MHA, bf16"),
    "c3": Workload("c3", 1, 8192, 32, 8, 128, torch.bfloat16, causal=True, rope_base=500000.0, seed=3,
                   description="Llama-3-8B GQA 32q/8kv causal, RoPE base 5e5, bf16"),
    "c4": Workload("c4", 2, 16384, 32, 8, 128, torch.bfloat16, causal=True, window=(4096, 0),
                   rope_base=10000.0, seed=4,
                   description="Mistral sliding-window GQA 32q/8kv causal, window (4096,0), RoPE 1e4, bf16"),
    "c5a": Workload("c5a", 8, 2048, 16, 16, 64, torch.float16, alibi=True, block_mask=True, seed=5,
                    description="ALiBi + 10%-block -inf mask MHA, fp16"),
    "c5b": Workload("c5b", 8, 2048, 16, 1, 64, torch.float16, alibi=True, block_mask=True, seed=5,
                    description="ALiBi + 10%-block -inf mask MQA (1 KV head), fp16"),
}


def alibi_slopes(num_heads: int) -> torch.Tensor:
    """Per-head ALiBi slopes (reference ``alibi.py:47-63``), fp32."""

    def pow2(n):
        start = 2 ** (-(2 ** (-(math.log2(n) - 3))))
        return [start * start**i for i in range(n)]

    if math.log2(num_heads).is_integer():
        slopes = pow2(num_heads)
    else:
        c = 2 ** math.floor(math.log2(num_heads))
        slopes = pow2(c) + pow2(2 * c)[0::2][: num_heads - c]
    return torch.tensor(slopes, dtype=torch.float32)


def rope_tables(seqlen: int, head_dim: int, base: float, dtype: torch.dtype,
                device="cpu") -> Tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) of shape (seqlen, head_dim) in ``dtype``, reference rope.py:61,69-79."""
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim)
    t = torch.arange(seqlen, device=device, dtype=inv_freq.dtype)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def block_mask(seqlen: int, seed: int, frac: float = 0.10, block: int = 64) -> torch.Tensor:
    """[S, S] fp32 mask: 0, except -inf on a seeded ``frac`` of the
    ``block x block`` tiles; every block-row keeps at least one open tile."""
    nb = -(-seqlen // block)
    g = torch.Generator().manual_seed(seed + 1000)
    grid = torch.rand((nb, nb), generator=g) < frac
    for r in range(nb):
        if bool(grid[r].all()):
            grid[r, int(torch.randint(0, nb, (1,), generator=g))] = False
    full = grid.repeat_interleave(block, 0).repeat_interleave(block, 1)[:seqlen, :seqlen]
    m = torch.zeros((seqlen, seqlen), dtype=torch.float32)
    m[full] = float("-inf")
    return m


@dataclass
class Inputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    mask: Optional[torch.Tensor] = None
    alibi: Optional[torch.Tensor] = None
    cos: Optional[torch.Tensor] = None
    sin: Optional[torch.Tensor] = None
    extra: dict = field(default_factory=dict)


def make_inputs(w: Workload, device="cpu") -> Inputs:
    """Seeded q/k/v ~ N(0,1) (fp32 draw, cast to ``w.dtype``) plus the
    workload's mask / ALiBi slopes / RoPE tables.  q/k are NOT rotated."""
    g = torch.Generator().manual_seed(w.seed)
    shp_q = (w.batch, w.seqlen, w.nheads, w.head_dim)
    shp_kv = (w.batch, w.seqlen, w.nheads_kv, w.head_dim)
    q = torch.randn(shp_q, generator=g, dtype=torch.float32).to(w.dtype)
    k = torch.randn(shp_kv, generator=g, dtype=torch.float32).to(w.dtype)
    v = torch.randn(shp_kv, generator=g, dtype=torch.float32).to(w.dtype)
    inp = Inputs(q.to(device), k.to(device), v.to(device))
    if w.block_mask:
        inp.mask = block_mask(w.seqlen, w.seed).to(device)
    if w.alibi:
        inp.alibi = alibi_slopes(w.nheads).to(device)
    if w.rope_base is not None:
        c, s = rope_tables(w.seqlen, w.head_dim, w.rope_base, w.dtype)
        inp.cos, inp.sin = c.to(device), s.to(device)
    return inp


def flops(w: Workload, heads: Optional[Sequence[int]] = None, batches: Optional[Sequence[int]] = None) -> int:
    """Algorithmic FLOP = 4 * D * allowed pairs over (b, h).  Pairs removed by
    the -inf blocks of the mask are not counted either."""
    from .kernels.attention_kernel import allowed_pairs

    nh = w.nheads if heads is None else len(heads)
    nb = w.batch if batches is None else len(batches)
    if w.block_mask:
        m = block_mask(w.seqlen, w.seed)
        allowed = torch.isfinite(m)
        if w.causal:
            allowed &= torch.ones_like(allowed).tril()
        pairs = int(allowed.sum())
    else:
        pairs = allowed_pairs(w.seqlen, w.seqlen, w.causal, w.window)
    return 4 * w.head_dim * nb * nh * pairs
