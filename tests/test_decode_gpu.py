"""GPU parity tests of the split-KV decode path (``trinix_attn_fwd_splitkv``):
seqlen_q <= 16 query rows against a long KV cache, bf16/fp16.

The oracle and the bar are those of the prefill tests: the restated eager
path (``oracle/attention_oracle.py``, reference base.py:347-400, top-left
causal), bf16/fp16 max abs <= 2e-2 and mean abs <= 2e-3, or, where the
oracle's own bf16 rounding of biased scores costs more than half of that,
the same bar against the fp64 closed form.  Each case also checks that the
split plan applies (so the split-KV kernel is what ran) and, for the larger
cases, that it used more than one chunk or exactly one, as stated.
"""
import ctypes

import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import _native as nat
from trinix_amd import triton_attn_func
from trinix_amd.kernels import attention_kernel as ak
from test_attn_gpu import assert_parity, assert_parity_or_more_accurate, oracle_on, rand

pytestmark = pytest.mark.gpu
DEV = "cuda"


def plan_of(q, k, **kw):
    """(num_splits, workspace bytes) the library plans for this call."""
    a = nat.AttnFwdArgs()
    B, Sq, H, D = q.shape
    a.q = a.k = a.v = a.out = 4096
    for name in ("q_stride", "k_stride", "v_stride", "out_stride"):
        setattr(a, name, nat.int64x4((8 * 1024, 1024, 128, 1)))
    a.batch, a.seqlen_q, a.seqlen_k, a.nheads_q, a.nheads_kv = B, Sq, k.shape[1], H, k.shape[2]
    a.head_dim = ak.kernel_head_dim(D)
    a.dtype = nat.TRINIX_BF16 if q.dtype == torch.bfloat16 else nat.TRINIX_F16
    a.causal = 1 if kw.get("causal") else 0
    if kw.get("window_size") is not None:
        a.has_window = 1
        a.window_left, a.window_right = kw["window_size"]
    ns, wb = ctypes.c_int32(), ctypes.c_int64()
    assert nat.load_library().trinix_attn_fwd_splitkv_plan(ctypes.byref(a), ctypes.byref(ns), ctypes.byref(wb)) == 0
    return ns.value, wb.value


def check(q, k, v, dtype, what, splits=None, **kw):
    ns, _ = plan_of(q, k, **kw)
    assert ns > 0, f"{what}: split-KV plan does not apply"
    if splits == "many":
        assert ns > 1, what
    elif splits is not None:
        assert ns == splits, (what, ns)
    out = triton_attn_func(q, k, v, **kw)
    ref = oracle_on(q, k, v, **kw)
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(), **kw)
    assert_parity_or_more_accurate(out, ref, x64, dtype, what)
    return out


CASES = [
    # (B, Sq, Sk, Hq, Hkv, D, splits)
    (1, 1, 8192, 32, 8, 128, "many"),   # Llama-3-8B decode step: 64 chunks of 128 keys
    (3, 1, 1000, 8, 2, 64, "many"),
    (2, 4, 777, 8, 2, 128, "many"),     # 16 packed rows = one full row group, ragged last chunk
    (1, 16, 300, 4, 1, 128, None),      # MQA, 64 packed rows = 4 row groups
    (1, 2, 65, 6, 2, 64, None),         # 6 packed rows, 65 keys: one partial 16-key step
    (2, 5, 5000, 3, 1, 64, "many"),     # G=3: 15 packed rows
    (160, 1, 256, 8, 8, 128, 1),        # >= 1024 work items: one chunk, direct output
    (1, 1, 1, 4, 4, 128, 1),            # a single key
    (1, 1, 131072, 32, 8, 128, "many"),  # a 128K-token cache (long context)
    (2, 3, 100000, 8, 1, 64, "many"),    # MQA over 100K keys, ragged last chunk
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", CASES, ids=[str(c[:6]) for c in CASES])
def test_decode_shapes(case, dtype):
    B, Sq, Sk, Hq, Hkv, D, splits = case
    print(f"decode case {case} {dtype}", flush=True)
    q = rand((B, Sq, Hq, D), dtype, 101)
    k = rand((B, Sk, Hkv, D), dtype, 102)
    v = rand((B, Sk, Hkv, D), dtype, 103)
    check(q, k, v, dtype, str(case), splits=splits)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("feat", ["causal", "window", "window_causal", "alibi", "pad_mask", "float_mask4d",
                                  "alibi_mask_scale"])
def test_decode_features(feat, dtype):
    B, Sq, Sk, Hq, Hkv, D = 2, 3, 1500, 8, 2, 128
    print(f"decode feature {feat} {dtype}", flush=True)
    q, k, v = rand((B, Sq, Hq, D), dtype, 111), rand((B, Sk, Hkv, D), dtype, 112), rand((B, Sk, Hkv, D), dtype, 113)
    g = torch.Generator().manual_seed(114)
    kw = {}
    if feat == "causal":
        kw = dict(causal=True)  # top-left: row i sees keys 0..i
    elif feat == "window":
        kw = dict(window_size=(40, 700))
    elif feat == "window_causal":
        kw = dict(window_size=(5, 1000), causal=True)
    elif feat == "alibi":
        kw = dict(alibi_slopes=orc.alibi_slopes(Hq))
    elif feat == "pad_mask":
        keep = torch.rand((B, Sk), generator=g) < 0.7  # padding mask of a batch of caches, as a bool (B,1,1,Sk)
        keep[:, 0] = True
        kw = dict(attn_mask=keep[:, None, None, :].expand(B, 1, Sq, Sk))
    elif feat == "float_mask4d":
        m = torch.randn((B, Hq, Sq, Sk), generator=g)
        m[torch.rand((B, Hq, Sq, Sk), generator=g) < 0.3] = float("-inf")
        m[..., 0] = 0
        kw = dict(attn_mask=m)
    else:
        m = torch.randn((Sq, Sk), generator=g)
        kw = dict(attn_mask=m, alibi_slopes=orc.alibi_slopes(Hq), softmax_scale=0.05)
    dev_kw = {k_: (v_.to(DEV) if torch.is_tensor(v_) else v_) for k_, v_ in kw.items()}
    ns, _ = plan_of(q, k, **kw)
    assert ns > 0
    out = triton_attn_func(q, k, v, **dev_kw)
    ref_kw = dict(kw)
    if "attn_mask" in ref_kw and ref_kw["attn_mask"].dtype == torch.bool:
        ref_kw["attn_mask"] = ref_kw["attn_mask"].to(torch.uint8)
    ref = oracle_on(q, k, v, **{k_: (v_.float() if k_ == "attn_mask" else v_) for k_, v_ in ref_kw.items()})
    x64 = orc.closed_form(q.cpu(), k.cpu(), v.cpu(),
                          **{k_: (v_.float() if k_ == "attn_mask" else v_) for k_, v_ in ref_kw.items()})
    assert_parity_or_more_accurate(out, ref, x64, dtype, feat)


def test_decode_matches_prefill_kernel_and_lse():
    """The split-KV result and log-sum-exp against the prefill kernel's on the
    same call (both within the bar of the fp64 closed form)."""
    B, Sq, Sk, Hq, Hkv, D = 2, 2, 3000, 16, 4, 128
    q, k, v = (rand((B, Sq, Hq, D), torch.bfloat16, 121), rand((B, Sk, Hkv, D), torch.bfloat16, 122),
               rand((B, Sk, Hkv, D), torch.bfloat16, 123))
    out_s, lse_s = triton_attn_func(q, k, v, return_lse=True)
    ak.SPLITKV_ENABLED = False
    try:
        out_p, lse_p = triton_attn_func(q, k, v, return_lse=True)
    finally:
        ak.SPLITKV_ENABLED = True
    x64 = torch.from_numpy(orc.closed_form(q.cpu(), k.cpu(), v.cpu()))
    assert_parity(out_s, x64, torch.bfloat16, "split vs fp64")
    assert_parity(out_p, x64, torch.bfloat16, "prefill vs fp64")
    qd, kd = q.cpu().double(), k.cpu().double().repeat_interleave(Hq // Hkv, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", qd, kd) * D ** -0.5
    lse64 = torch.logsumexp(s, dim=-1)
    assert torch.allclose(lse_s.cpu().double(), lse64, atol=2e-4, rtol=1e-5)
    assert torch.allclose(lse_s, lse_p, atol=2e-4, rtol=1e-5)


def test_decode_fully_masked_rows_are_nan_and_lse_minus_inf():
    B, Sq, Sk, H, D = 1, 4, 700, 4, 64
    q, k, v = rand((B, Sq, H, D), torch.float16, 131), rand((B, Sk, H, D), torch.float16, 132), rand((B, Sk, H, D), torch.float16, 133)
    m = torch.zeros(Sq, Sk)
    m[2] = float("-inf")
    out, lse = triton_attn_func(q, k, v, attn_mask=m.to(DEV), return_lse=True)
    ref = oracle_on(q, k, v, attn_mask=m)
    assert torch.isnan(ref[0, 2]).all()
    assert_parity(out, ref, torch.float16, "nan rows")
    assert torch.isneginf(lse[0, :, 2]).all() and torch.isfinite(lse[0, :, [0, 1, 3]]).all()


def test_decode_kv_cache_views_and_stride0_mqa():
    """A cache slice (non-contiguous batch stride) and an expand()ed single KV
    head are read in place; both layouts meet the bar against the oracle (they
    plan different chunkings: 8 KV heads of one row vs one of 8 rows)."""
    B, Sq, Smax, Sk, H, D = 2, 1, 4096, 2500, 8, 128
    cache_k = rand((B, Smax, 1, D), torch.bfloat16, 141)
    cache_v = rand((B, Smax, 1, D), torch.bfloat16, 142)
    q = rand((B, Sq, H, D), torch.bfloat16, 143)
    k, v = cache_k[:, :Sk].expand(-1, -1, H, -1), cache_v[:, :Sk].expand(-1, -1, H, -1)
    assert k.stride(2) == 0 and not k.is_contiguous()
    out = triton_attn_func(q, k, v)
    out1 = triton_attn_func(q, cache_k[:, :Sk].contiguous(), cache_v[:, :Sk].contiguous())
    ref = oracle_on(q, k.contiguous(), v.contiguous())
    assert_parity(out, ref, torch.bfloat16, "cache view, stride-0 heads")
    assert_parity(out1, ref, torch.bfloat16, "one KV head")


def test_decode_fused_rope_args_rotate_q_first():
    B, Sq, Sk, Hq, Hkv, D = 1, 3, 900, 8, 2, 128
    q, k, v = rand((B, Sq, Hq, D), torch.bfloat16, 151), rand((B, Sk, Hkv, D), torch.bfloat16, 152), rand((B, Sk, Hkv, D), torch.bfloat16, 153)
    cos, sin = orc.rope_tables(Sk, D, 500000.0, torch.bfloat16)
    out = triton_attn_func(q, k, v, rotary_cos=cos.to(DEV), rotary_sin=sin.to(DEV))
    qr, kr = orc.apply_rope(q.cpu(), cos[:Sq], sin[:Sq]), orc.apply_rope(k.cpu(), cos, sin)
    assert_parity(out, orc.functional_attention(qr, kr, v.cpu()), torch.bfloat16, "rope")


def test_decode_backward_through_split_path():
    """Gradients of a decode-shaped call (the forward runs split-KV, the
    backward uses its log-sum-exp) against eager autograd."""
    from test_attn_bwd_gpu import _check, _eager_grads, _hip_grads, _inputs

    q, k, v, do = _inputs(2, 3, 1200, 8, 2, 128, seed=161)
    _, truth = _eager_grads(q, k, v, do, torch.float64)
    _, eager = _eager_grads(q, k, v, do, torch.bfloat16)
    _, hip = _hip_grads(q, k, v, do, torch.bfloat16)
    _check(hip, eager, truth)


def test_gqa_layer_decode_steps_with_cache_match_eager():
    """A prompt, then three one-token steps through the layer's KV cache;
    every step's output against the eager layer on the same cache."""
    import trinix_amd as tx

    torch.manual_seed(171)
    E, H, HKV = 1024, 8, 2
    hip = tx.FastGroupedQueryAttention(E, H, HKV, causal=False, kernel_type="flash").cuda().to(torch.bfloat16)
    eager = tx.FastGroupedQueryAttention(E, H, HKV, causal=False, kernel_type="pytorch").cuda().to(torch.bfloat16)
    eager.load_state_dict(hip.state_dict())
    x = torch.randn(2, 200, E, device=DEV).to(torch.bfloat16)
    _, cache = hip(x, use_cache=True)
    for t in range(3):
        xt = torch.randn(2, 1, E, device=DEV).to(torch.bfloat16)
        o1, c1 = hip(xt, past_key_value=cache, use_cache=True)
        o2, c2 = eager(xt, past_key_value=cache, use_cache=True)
        assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
        d = (o1.float() - o2.float()).abs()
        scale = max(1.0, o2.float().abs().max().item())
        assert d.max().item() <= 2e-2 * scale and d.mean().item() <= 2e-3 * scale, (t, d.max().item())
        cache = c1
