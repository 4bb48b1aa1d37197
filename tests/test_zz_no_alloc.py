"""GPU test of ``trinix_attn_fwd_splitkv_noalloc``, the split-KV decode
forward that allocates nothing (its partial results live in the library's
static device scratch), called through the C ABI.

Its output and log-sum-exp must be bitwise those of
``trinix_attn_fwd_splitkv`` with a torch-allocated workspace on the same
inputs, over two calls in a row, the second with a smaller input (the
scratch keeps the first call's partials, which the second must not see),
and once more with a one-chunk plan that needs no scratch.
"""
import ctypes

import pytest
import torch

from trinix_amd import _native as nat
from trinix_amd.kernels.attention_kernel import current_stream_ptr

pytestmark = pytest.mark.gpu
DEV = "cuda"
CODES = {torch.bfloat16: nat.TRINIX_BF16, torch.float16: nat.TRINIX_F16}


def make_args(q, k, v, out, lse, causal=False, window=None):
    a = nat.AttnFwdArgs()
    a.q, a.k, a.v, a.out, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
    a.q_stride, a.k_stride = nat.int64x4(q.stride()), nat.int64x4(k.stride())
    a.v_stride, a.out_stride = nat.int64x4(v.stride()), nat.int64x4(out.stride())
    B, Sq, H, D = q.shape
    a.batch, a.seqlen_q, a.seqlen_k, a.nheads_q, a.nheads_kv, a.head_dim = B, Sq, k.shape[1], H, k.shape[2], D
    a.dtype = CODES[q.dtype]
    a.softmax_scale = D ** -0.5
    a.causal = 1 if causal else 0
    if window is not None:
        a.has_window = 1
        a.window_left, a.window_right = window
    return a


def run_pair(shape, dtype, seed, **kw):
    """(out, lse) of the workspace entry point and of the no-allocation one."""
    B, Sq, Sk, Hq, Hkv, D = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Sq, Hq, D), generator=g).to(dtype).to(DEV)
    k = torch.randn((B, Sk, Hkv, D), generator=g).to(dtype).to(DEV)
    v = torch.randn((B, Sk, Hkv, D), generator=g).to(dtype).to(DEV)
    lib = nat.load_library()
    stream = current_stream_ptr(q.device)
    res = []
    for noalloc in (False, True):
        out = torch.full((B, Sq, Hq, D), float("nan"), dtype=dtype, device=DEV)
        lse = torch.full((B, Hq, Sq), float("nan"), dtype=torch.float32, device=DEV)
        a = make_args(q, k, v, out, lse, **kw)
        ns, wb = ctypes.c_int32(), ctypes.c_int64()
        nat.check(lib.trinix_attn_fwd_splitkv_plan(ctypes.byref(a), ctypes.byref(ns), ctypes.byref(wb)), "plan")
        assert ns.value > 0
        if noalloc:
            assert wb.value <= nat.SPLITKV_SCRATCH_BYTES
            nat.check(lib.trinix_attn_fwd_splitkv_noalloc(ctypes.byref(a), stream), "noalloc")
        else:
            ws = torch.empty(max(wb.value, 16), dtype=torch.uint8, device=DEV)
            nat.check(lib.trinix_attn_fwd_splitkv(ctypes.byref(a), ws.data_ptr(), wb.value, stream), "splitkv")
        torch.cuda.synchronize()
        res.append((out.cpu(), lse.cpu(), ns.value))
    return res


def assert_same(res, what):
    (o1, l1, n1), (o2, l2, n2) = res
    assert n1 == n2
    assert not torch.isnan(o1).any() and not torch.isnan(l1).any(), what
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), what
    assert torch.equal(l1.view(torch.int32), l2.view(torch.int32)), what


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry_two_calls(dtype):
    # first call: Llama-3-8B-shaped decode step, 64 chunks (2.1 MB of partials)
    big = (2, 1, 8192, 32, 8, 128)
    print(f"noalloc call 1 {big} {dtype}", flush=True)
    res = run_pair(big, dtype, 11)
    assert res[0][2] > 1
    assert_same(res, "call 1")
    # second call, smaller: fewer rows, fewer chunks, D=64, a window that
    # bounds the visible keys to 0..902
    small = (1, 3, 1000, 8, 2, 64)
    print(f"noalloc call 2 {small} {dtype}", flush=True)
    res = run_pair(small, dtype, 12, window=(10, 900))
    assert res[0][2] > 1
    assert_same(res, "call 2")


def test_noalloc_single_chunk_needs_no_scratch():
    # >= 1024 work items: one chunk, the kernel writes the output directly
    shape = (160, 1, 256, 8, 8, 128)
    print(f"noalloc one chunk {shape}", flush=True)
    res = run_pair(shape, torch.bfloat16, 13)
    assert res[0][2] == 1
    assert_same(res, "one chunk")
