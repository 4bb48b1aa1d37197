"""GPU tests of the forward paths under HIP graph capture (serving loops and
bench.py's kernel timing capture them).  The library launches kernels only:
no allocation, no memset, no host synchronisation.  Each test captures a few
calls into one graph and replays it several times, with eager work and
synchronisations between the replays.  Every replay's outputs must equal an
eager call's bit for bit (the kernels are deterministic).

Paths covered: the prefill kernel (plain causal GQA, fused RoPE), the
ALiBi + mask kernel with its block-map pre-pass, and the split-KV decode
kernels with their workspace."""
import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func
from test_attn_gpu import rand

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _replays_match_eager(fn, calls=3, replays=4):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [fn() for _ in range(calls)]
    for r in range(replays):
        # eager work between replays: overwrite the graph's outputs and
        # run the same op outside the graph
        for o in outs:
            o.fill_(float("nan"))
        again = fn()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(again, eager), f"eager call differs (replay {r})"
        for i, o in enumerate(outs):
            assert torch.equal(o, eager), f"replay {r}, call {i} differs from the eager output"


def test_graph_prefill_gqa_rope_causal():
    B, S, H, Hkv, D = 2, 700, 8, 2, 128
    q, k, v = rand((B, S, H, D), torch.bfloat16, 1), rand((B, S, Hkv, D), torch.bfloat16, 2), \
        rand((B, S, Hkv, D), torch.bfloat16, 3)
    pos = torch.arange(S, dtype=torch.float32)
    inv = 1.0 / 10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D)
    emb = torch.cat([torch.outer(pos, inv)] * 2, dim=-1)
    cos, sin = emb.cos().to(DEV, torch.bfloat16), emb.sin().to(DEV, torch.bfloat16)
    _replays_match_eager(lambda: triton_attn_func(q, k, v, causal=True, rotary_cos=cos, rotary_sin=sin))


def test_graph_alibi_block_mask_fp16():
    B, S, H, D = 2, 320, 4, 64
    q, k, v = (rand((B, S, H, D), torch.float16, s) for s in (4, 5, 6))
    mask = torch.zeros(S, S, device=DEV)
    mask[64:128, 128:192] = float("-inf")
    mask[200:260, :40] = float("-inf")
    slopes = orc.alibi_slopes(H).to(DEV)
    _replays_match_eager(lambda: triton_attn_func(q, k, v, attn_mask=mask, alibi_slopes=slopes))


def test_graph_splitkv_decode():
    B, Sk, H, Hkv, D = 3, 5000, 8, 2, 128
    q = rand((B, 1, H, D), torch.bfloat16, 7)
    k, v = rand((B, Sk, Hkv, D), torch.bfloat16, 8), rand((B, Sk, Hkv, D), torch.bfloat16, 9)
    _replays_match_eager(lambda: triton_attn_func(q, k, v))
