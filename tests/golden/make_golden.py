"""Writes the committed attention fixtures of tests/golden/ (run from the
repository root: ``python tests/golden/make_golden.py``).

The reference ships no golden vectors (its tests compare against torch at
run time), so these are this build's own known answers, kept as data:

* ``cases.npz``: small attention problems covering the path's features
  (causal, sliding window, ALiBi, 2-D and 4-D masks, GQA, MQA, Sq != Sk,
  fp32 / bf16 / fp16, head_dim 64 / 128 / 256).  For each case the fixture
  holds the inputs (the exact bits) and the float64 closed form
  ``softmax(q k^T * scale + bias) v`` of those inputs (``expected``, stored
  as float32).
* ``c1_checksums.npz``: BASELINE config 1 (fp32 2x128x8x64) from the seeded
  workload inputs: checksums of q, k, v, and of the float64 closed-form
  output (sum, sum of |x|) plus 64 of its elements at fixed positions.

Masks are stored as float32 with -inf entries or as bool.  Everything is
stored with numpy (no pickling): ``np.load(..., allow_pickle=False)``.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention_oracle as orc  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# name, seed, B, Sq, Sk, H, Hkv, D, dtype, options
CASES = [
    ("fp32_plain", 11, 1, 33, 33, 4, 4, 64, torch.float32, {}),
    ("bf16_causal_gqa", 12, 1, 40, 40, 4, 2, 128, torch.bfloat16, {"causal": True}),
    ("fp16_window", 13, 1, 65, 65, 2, 2, 64, torch.float16, {"window_size": (9, 4)}),
    ("bf16_causal_window_sqsk", 14, 1, 40, 97, 2, 2, 64, torch.bfloat16, {"causal": True, "window_size": (20, 0)}),
    ("fp16_alibi_mask2d", 15, 1, 64, 64, 4, 4, 64, torch.float16, {"alibi": True, "mask": "2d"}),
    ("bf16_mqa_mask4d_bool", 16, 1, 48, 48, 4, 1, 128, torch.bfloat16, {"mask": "4d_bool"}),
    ("bf16_d256_alibi_causal", 17, 1, 40, 40, 2, 1, 256, torch.bfloat16, {"causal": True, "alibi": True}),
    ("fp16_short_q_long_k", 18, 1, 16, 300, 1, 1, 64, torch.float16, {"softmax_scale": 0.05}),
]

C1_SAMPLES = 64


def _bits(t: torch.Tensor) -> np.ndarray:
    """The tensor's exact bits (16-bit floats as int16, fp32 as float32)."""
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy()
    return t.contiguous().numpy()


def case_inputs(seed, B, Sq, Sk, H, Hkv, D, dtype, opts):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, H, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dtype)
    mask = None
    if opts.get("mask") == "2d":
        mask = torch.zeros(Sq, Sk)
        blocks = torch.rand(Sq // 16, Sk // 16, generator=g) < 0.2
        blocks[:, 0] = False  # every row keeps allowed keys
        mask[blocks.repeat_interleave(16, 0).repeat_interleave(16, 1)] = float("-inf")
    elif opts.get("mask") == "4d_bool":
        mask = torch.rand(B, H, Sq, Sk, generator=g) < 0.3
    slopes = orc.alibi_slopes(H) if opts.get("alibi") else None
    return q, k, v, mask, slopes


def main() -> None:
    arrays = {}
    for name, seed, B, Sq, Sk, H, Hkv, D, dtype, opts in CASES:
        q, k, v, mask, slopes = case_inputs(seed, B, Sq, Sk, H, Hkv, D, dtype, opts)
        kw = dict(causal=opts.get("causal", False), window_size=opts.get("window_size"),
                  softmax_scale=opts.get("softmax_scale"), alibi_slopes=slopes)
        expected = orc.closed_form(q, k, v, attn_mask=mask, **kw)
        arrays[f"{name}/q"], arrays[f"{name}/k"], arrays[f"{name}/v"] = _bits(q), _bits(k), _bits(v)
        if mask is not None:
            arrays[f"{name}/mask"] = mask.numpy()
        if slopes is not None:
            arrays[f"{name}/alibi"] = slopes.numpy().astype(np.float32)
        arrays[f"{name}/expected"] = expected.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "cases.npz"), **arrays)

    from trinix_amd.workloads import WORKLOADS, make_inputs

    w = WORKLOADS["c1"]
    inp = make_inputs(w)
    out = orc.closed_form(inp.q, inp.k, inp.v, causal=w.causal)
    flat = out.reshape(-1)
    idx = np.random.default_rng(1).choice(flat.size, C1_SAMPLES, replace=False)
    np.savez_compressed(
        os.path.join(HERE, "c1_checksums.npz"),
        input_sums=np.array([t.double().sum().item() for t in (inp.q, inp.k, inp.v)]),
        out_sum=np.array(flat.sum()), out_abs_sum=np.array(np.abs(flat).sum()),
        sample_index=idx.astype(np.int64), sample_value=flat[idx])
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
