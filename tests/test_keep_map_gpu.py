"""GPU tests of the dropout keep map: a forward with dropout that keeps
state for the backward writes its keep decisions (one bit per (row, key),
``trinix_attn_fwd_args.dropout_keep_map``) and the 16-bit backward reads
them instead of regenerating the mask from Philox.

* The map decoded on the CPU by the layout the header states equals the
  oracle's keep mask (``oracle.dropout_keep``, the Philox stream pinned by
  Random123's known answers) at every allowed (row, key).
* Gradients through the map are bitwise those of the regenerating path
  (``TRINIX_DROPOUT_KEEP_MAP=0``): same keep decisions, same arithmetic.
  The gradients of both against eager autograd with the oracle's mask are
  checked in ``test_attn_bwd_gpu.py`` (``test_dropout_backward_matches_eager_with_philox_keep``
  runs both paths)."""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func
from trinix_amd.kernels import attention_kernel as ak

pytestmark = pytest.mark.gpu
DEV = "cuda"


def decode_keep_map(raw: np.ndarray, B: int, H: int, Sq: int, Sk: int) -> np.ndarray:
    """(B, H, Sq, Sk) keep mask from the map's bytes: per (b, h)
    2*ceil(Sq/64) x 4*ceil(Sk/128) blocks of 32 uint32 words, word r = row
    32*bi + r, bit 16h + 4q + e = key 32*bj + 8q + 4h + e."""
    nbi, nbj = 2 * -(-Sq // 64), 4 * -(-Sk // 128)
    words = raw.view(np.uint32).reshape(B, H, nbi, nbj, 32)
    bits = (words[..., None] >> np.arange(32, dtype=np.uint32)) & np.uint32(1)  # [b, h, bi, bj, r, c]
    c = np.arange(32)
    key = 8 * ((c % 16) // 4) + 4 * (c // 16) + c % 4
    ordered = np.empty_like(bits)
    ordered[..., key] = bits
    full = ordered.transpose(0, 1, 2, 4, 3, 5).reshape(B, H, nbi * 32, nbj * 32)
    return full[:, :, :Sq, :Sk].astype(bool)


def test_decode_layout_on_a_planted_block():
    """The decoder itself, on a hand-built block: row 5, key 13 of block
    (0, 1) is bit 16*1 + 4*1 + 1 of word 5 (13 = 8*1 + 4*1 + 1)."""
    B, H, Sq, Sk = 1, 1, 40, 70
    nbi, nbj = 2, 4
    words = np.zeros((B, H, nbi, nbj, 32), dtype=np.uint32)
    words[0, 0, 0, 1, 5] = np.uint32(1) << np.uint32(21)
    keep = decode_keep_map(words.view(np.uint8).ravel(), B, H, Sq, Sk)
    assert keep.sum() == 1 and keep[0, 0, 5, 32 + 13]


def _allowed(Sq, Sk, causal, window, mask):
    i = np.arange(Sq)[:, None]
    j = np.arange(Sk)[None, :]
    ok = np.ones((Sq, Sk), dtype=bool)
    if causal:
        ok &= j <= i
    if window is not None:
        ok &= (j - i >= -window[0]) & (j - i <= window[1])
    if mask is not None:
        ok &= np.isfinite(mask.numpy())
    return ok


def _mask(Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    blocks = torch.rand(-(-Sq // 32), -(-Sk // 32), generator=g) < 0.25
    blocks[:, 0] = False
    inf = blocks.repeat_interleave(32, 0).repeat_interleave(32, 1)[:Sq, :Sk]
    return torch.where(inf, float("-inf"), torch.randn(Sq, Sk, generator=g) * 0.5)


MAP_CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, p, causal, window, masked)
    (1, 160, 160, 4, 2, 64, torch.bfloat16, 0.1, True, None, False),
    (2, 96, 200, 2, 2, 128, torch.float16, 0.3, False, None, False),
    (1, 130, 200, 4, 1, 128, torch.bfloat16, 0.15, True, (50, 20), False),
    (1, 150, 150, 2, 2, 64, torch.float16, 0.5, False, None, True),
    (1, 17, 300, 1, 1, 128, torch.bfloat16, 0.2, False, None, False),
    (2, 300, 33, 3, 3, 64, torch.bfloat16, 0.05, True, None, False),
]


@pytest.mark.parametrize("case", range(len(MAP_CASES)))
def test_keep_map_equals_the_oracle_keep_mask(case, monkeypatch):
    B, Sq, Sk, H, Hkv, D, dtype, p, causal, window, masked = MAP_CASES[case]
    print(f"keep map case {MAP_CASES[case]}", flush=True)
    monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", "1")
    g = torch.Generator().manual_seed(900 + case)
    q = torch.randn(B, Sq, H, D, generator=g).to(DEV, dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(DEV, dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(DEV, dtype)
    mask = _mask(Sq, Sk, 77 + case) if masked else None
    torch.manual_seed(55 + case)
    _, _, state = ak._forward(q, k, v, None if mask is None else mask.to(DEV), causal, D ** -0.5, p, window, None,
                              None, None, True, False, True, keep_state=True)
    assert state["keep_map"] is not None
    torch.cuda.synchronize()
    raw = state["keep_map"].cpu().numpy()
    _, seed, offset = state["dropout"]
    got = decode_keep_map(raw, B, H, Sq, Sk)
    ref = orc.dropout_keep(B, H, Sq, Sk, p, seed, offset)
    ok = _allowed(Sq, Sk, causal, window, mask)
    assert ok.any()
    diff = (got != ref) & ok[None, None]
    assert not diff.any(), np.argwhere(diff)[:10]


BITWISE_CASES = [
    # (B, Sq, Sk, H, Hkv, D, dtype, p, kwargs): every 16-bit backward
    # variant reading the map (ALiBi, mask, both; head_dim 64 and 128;
    # 128-key dQ tiles at head_dim 128 without a mask)
    (1, 160, 160, 4, 2, 64, torch.bfloat16, 0.1, dict(causal=True)),
    (2, 96, 96, 2, 2, 128, torch.float16, 0.3, dict()),
    (1, 128, 128, 4, 1, 128, torch.bfloat16, 0.2, dict(alibi_slopes=orc.alibi_slopes(4), causal=True)),
    (1, 130, 200, 4, 2, 128, torch.bfloat16, 0.15, dict(window_size=(50, 20))),
    (2, 100, 100, 4, 4, 64, torch.float16, 0.5, dict(alibi_slopes=orc.alibi_slopes(4), attn_mask=_mask(100, 100, 3))),
    (1, 140, 140, 4, 2, 128, torch.float16, 0.2, dict(alibi_slopes=orc.alibi_slopes(4),
                                                      attn_mask=_mask(140, 140, 4), causal=True)),
    (1, 150, 150, 2, 1, 128, torch.bfloat16, 0.1, dict(attn_mask=_mask(150, 150, 5), causal=True)),
    (1, 2048, 2048, 8, 2, 128, torch.bfloat16, 0.1, dict(causal=True)),
    (2, 1024, 1024, 4, 4, 64, torch.bfloat16, 0.1, dict(causal=True)),
]


def _grads(q, k, v, do, p, seed, kw):
    ts = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    torch.manual_seed(seed)
    out = triton_attn_func(*ts, dropout_p=p, **kw)
    out.backward(do)
    return [out.detach()] + [t.grad for t in ts]


@pytest.mark.parametrize("case", range(len(BITWISE_CASES)))
def test_gradients_through_the_map_equal_the_regenerated_mask(case, monkeypatch):
    B, Sq, Sk, H, Hkv, D, dtype, p, kw = BITWISE_CASES[case]
    print(f"keep map bitwise case {BITWISE_CASES[case][:8]}", flush=True)
    g = torch.Generator().manual_seed(1000 + case)
    q = torch.randn(B, Sq, H, D, generator=g).to(DEV, dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(DEV, dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(DEV, dtype)
    do = torch.randn(B, Sq, H, D, generator=g).to(DEV, dtype)
    kw = {key: (val.to(DEV) if torch.is_tensor(val) else val) for key, val in kw.items()}
    used = []
    real = ak._keep_map_bytes

    def spy(*a):
        n = real(*a)
        used.append(n)
        return n

    monkeypatch.setattr(ak, "_keep_map_bytes", spy)
    monkeypatch.setattr(ak, "_TRAIN_LAUNCHES", {})  # the full host path, which sizes the map
    monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", "1")
    with_map = _grads(q, k, v, do, p, 31 + case, kw)
    assert used and used[-1] > 0  # the map was written and read
    monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", "0")
    regen = _grads(q, k, v, do, p, 31 + case, kw)
    assert used[-1] == 0
    for name, a, b in zip(("out", "dq", "dk", "dv"), with_map, regen):
        assert torch.equal(a, b), name


def test_a_forward_without_backward_frees_its_buffers_at_once():
    """Dropping the output of a differentiable call without running its
    backward frees the output, the lse and the keep map at once (no
    reference cycle through the autograd node), with the cycle collector
    off."""
    import gc

    q, k, v = (torch.randn(1, 1024, 4, 128, device=DEV, dtype=torch.bfloat16).requires_grad_(True) for _ in range(3))
    for p in (0.0, 0.1):  # warm-up: the launch caches and the device's dropout generator
        triton_attn_func(q, k, v, causal=True, dropout_p=p).sum().backward()
    q.grad = k.grad = v.grad = None
    torch.cuda.synchronize()
    gc.collect()
    gc.disable()
    try:
        base = torch.cuda.memory_allocated()
        for p in (0.0, 0.1):
            out = triton_attn_func(q, k, v, causal=True, dropout_p=p)
            held = torch.cuda.memory_allocated() - base
            assert held >= out.numel() * out.element_size()
            del out
            assert torch.cuda.memory_allocated() == base, (p, held)
    finally:
        gc.enable()
