"""CPU tests of the host launch cache (``kernels/attention_kernel.py``): a
call whose layout has run through the full host path once is launched from
a template of that call's argument struct.  The library is replaced by a
recording stub (compiled here with gcc) that keeps the last arguments of
each entry point and launches nothing, and CPU tensors stand in for device
ones, so the test compares, byte for byte, what the cached launch and the
full path hand to the C ABI."""
import ctypes
import os
import subprocess

import pytest
import torch

from trinix_amd import _native as nat
import trinix_amd.kernels.attention_kernel as ak
import trinix_amd.kernels.rope_kernel as rk

STUB = r"""
#include <stdint.h>
#include <string.h>
#include "trinix_attn.h"
static trinix_attn_fwd_args last_fwd, last_split;
static trinix_attn_bwd_args last_bwd;
static int n_fwd, n_split, n_rope, n_plan, n_bwd;
static int64_t last_rope[16];
static int64_t split_ws;
int trinix_abi_version(void) { return %(abi)d; }
int trinix_attn_is_available(void) { return 1; }
const char* trinix_status_string(int c) { (void)c; return "stub"; }
int trinix_attn_fwd(const trinix_attn_fwd_args* a, void* s) { (void)s; last_fwd = *a; ++n_fwd; return 0; }
int trinix_attn_fwd_splitkv_plan(const trinix_attn_fwd_args* a, int32_t* ns, int64_t* wb) {
  ++n_plan; *ns = a->seqlen_q <= 16 ? 3 : 0; *wb = a->seqlen_q <= 16 ? 4096 : 0; return 0; }
int trinix_attn_fwd_splitkv(const trinix_attn_fwd_args* a, void* ws, int64_t wb, void* s) {
  (void)ws; (void)s; last_split = *a; split_ws = wb; ++n_split; return 0; }
int trinix_rope_apply(const void* x, const int64_t* xs, void* out, const int64_t* os, int64_t B, int64_t S,
                      int64_t H, int64_t D, int32_t dt, const void* c, const void* sn, int64_t cst, int64_t rows,
                      const int64_t* pos, void* st) {
  (void)st;
  int64_t v[16] = {(int64_t)(intptr_t)x, xs[0], xs[1], xs[2], xs[3], (int64_t)(intptr_t)out, os[0], os[1], os[2],
                   os[3], B * 1000003 + S, H * 1000003 + D, dt, (int64_t)(intptr_t)c ^ (int64_t)(intptr_t)sn,
                   cst * 1000003 + rows, (int64_t)(intptr_t)pos};
  memcpy(last_rope, v, sizeof v); ++n_rope; return 0; }
int trinix_attn_bwd(const trinix_attn_bwd_args* a, void* s) { (void)s; last_bwd = *a; ++n_bwd; return 0; }
int trinix_dropout_keep_map_bytes(int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t* n) {
  *n = 128 * b * h * 2 * ((sq + 63) / 64) * 4 * ((sk + 127) / 128); return 0; }
int stub_counts(int* out) { out[0] = n_fwd; out[1] = n_split; out[2] = n_rope; out[3] = n_plan; out[4] = n_bwd;
  return 0; }
const trinix_attn_bwd_args* stub_last_bwd(void) { return &last_bwd; }
const trinix_attn_fwd_args* stub_last_fwd(void) { return &last_fwd; }
const trinix_attn_fwd_args* stub_last_split(void) { return &last_split; }
const int64_t* stub_last_rope(void) { return last_rope; }
int64_t stub_split_ws(void) { return split_ws; }
"""
# entry points the stub does not record: they only have to exist
OTHERS = [n for n in nat.SIGNATURES if n not in (
    "trinix_abi_version", "trinix_attn_is_available", "trinix_status_string", "trinix_attn_fwd",
    "trinix_attn_fwd_splitkv_plan", "trinix_attn_fwd_splitkv", "trinix_rope_apply", "trinix_attn_bwd",
    "trinix_dropout_keep_map_bytes")]


@pytest.fixture(scope="module")
def stub_path(tmp_path_factory):
    d = tmp_path_factory.mktemp("stub")
    src, rest = d / "stub.c", d / "others.c"
    src.write_text(STUB % {"abi": nat.ABI_VERSION})
    rest.write_text("".join(f"int {n}() {{ return 0; }}\n" for n in OTHERS))  # no header: any signature
    so = d / "libstub.so"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-w", "-I", inc, str(src), str(rest), "-o", str(so)],
                   check=True)
    return str(so)


@pytest.fixture
def stub(stub_path, monkeypatch):
    lib = ctypes.CDLL(stub_path)  # a fresh handle per test: counters start where the last test left them
    for name, (res, args) in nat.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    lib.stub_last_fwd.restype = ctypes.POINTER(nat.AttnFwdArgs)
    lib.stub_last_split.restype = ctypes.POINTER(nat.AttnFwdArgs)
    lib.stub_last_rope.restype = ctypes.POINTER(ctypes.c_int64 * 16)
    lib.stub_split_ws.restype = ctypes.c_int64
    lib.stub_last_bwd.restype = ctypes.POINTER(nat.AttnBwdArgs)
    monkeypatch.setattr(nat, "_lib", lib)
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(ak.TritonAttentionKernel, "_available", False)
    monkeypatch.setattr(ak, "current_stream_ptr", lambda dev: 0)
    monkeypatch.setattr(rk, "current_stream_ptr", lambda dev: 0)
    monkeypatch.setattr(ak, "_LAUNCHES", {})
    monkeypatch.setattr(ak, "_TRAIN_LAUNCHES", {})
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    return lib


def counts(lib):
    c = (ctypes.c_int * 5)()
    lib.stub_counts(c)
    return list(c)


def struct_bytes(a, zero=("q", "k", "v", "out", "rope_cos", "rope_sin")):
    b = nat.AttnFwdArgs.from_buffer_copy(a)
    for f in zero:
        setattr(b, f, None)
    return bytes(b)


def qkv(B=2, S=96, H=4, Hkv=2, D=64, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, S, H, D, generator=g).to(dtype), torch.randn(B, S, Hkv, D, generator=g).to(dtype),
            torch.randn(B, S, Hkv, D, generator=g).to(dtype))


def test_cached_launch_passes_the_full_paths_struct(stub):
    from trinix_amd import triton_attn_func

    q, k, v = qkv()
    triton_attn_func(q, k, v, causal=True, window_size=(40, 0))
    assert counts(stub)[0] == 1 and len(ak._LAUNCHES) == 1
    full = nat.AttnFwdArgs.from_buffer_copy(stub.stub_last_fwd().contents)
    q2, k2, v2 = qkv(seed=1)
    out = triton_attn_func(q2, k2, v2, causal=True, window_size=(40, 0))
    cached = stub.stub_last_fwd().contents
    assert counts(stub)[0] == 2 and len(ak._LAUNCHES) == 1
    assert struct_bytes(cached) == struct_bytes(full)
    assert (cached.q, cached.k, cached.v, cached.out) == (q2.data_ptr(), k2.data_ptr(), v2.data_ptr(),
                                                          out.data_ptr())
    assert out.shape == q2.shape and out.dtype == q2.dtype


@pytest.mark.parametrize("change", ["causal", "window", "scale", "stride", "dtype", "heads"])
def test_a_different_layout_takes_the_full_path(stub, change):
    from trinix_amd import triton_attn_func

    q, k, v = qkv()
    triton_attn_func(q, k, v, causal=True)
    kw = dict(causal=True)
    if change == "causal":
        kw["causal"] = False
    elif change == "window":
        kw["window_size"] = (8, 0)
    elif change == "scale":
        kw["softmax_scale"] = 0.5
    elif change == "stride":
        q = torch.randn(2, 4, 96, 64).to(torch.bfloat16).transpose(1, 2)  # (B, S, H, D) with other strides
    elif change == "dtype":
        q, k, v = qkv(dtype=torch.float16)
    elif change == "heads":
        q, k, v = qkv(Hkv=4)
    triton_attn_func(q, k, v, **kw)
    assert len(ak._LAUNCHES) == 2
    got = struct_bytes(stub.stub_last_fwd().contents)
    # the second layout's own cached launch reproduces its full-path struct
    triton_attn_func(*[t.clone() if t.is_contiguous() else t for t in (q, k, v)], **kw)
    assert struct_bytes(stub.stub_last_fwd().contents) == got and len(ak._LAUNCHES) == 2


def test_misaligned_operand_falls_back_to_the_full_path(stub):
    """The full path copies an operand whose rows are not 16-byte aligned;
    the cached launch must not hand it to the kernel as is."""
    from trinix_amd import triton_attn_func

    q, k, v = qkv()
    triton_attn_func(q, k, v)
    buf = torch.empty(q.numel() + 8, dtype=q.dtype)
    q_off = buf[4:4 + q.numel()].view(q.shape)  # same shape and strides, pointer 8 bytes off
    q_off.copy_(q)
    assert q_off.data_ptr() % 16
    triton_attn_func(q_off, k, v)
    a = stub.stub_last_fwd().contents
    assert a.q % 16 == 0 and a.q != q_off.data_ptr()  # a copy went to the kernel
    assert len(ak._LAUNCHES) == 1


def test_rope_pre_pass_is_cached_with_the_same_arguments(stub):
    from trinix_amd import triton_attn_func

    q, k, v = qkv(S=80, D=128)
    g = torch.Generator().manual_seed(5)
    cos, sin = torch.randn(80, 128, generator=g).to(q.dtype), torch.randn(80, 128, generator=g).to(q.dtype)
    triton_attn_func(q, k, v, causal=True, rotary_cos=cos, rotary_sin=sin)
    n0 = counts(stub)
    full, rope_full = struct_bytes(stub.stub_last_fwd().contents), list(stub.stub_last_rope().contents)
    assert len(ak._LAUNCHES) == 1 and ak._LAUNCHES[next(iter(ak._LAUNCHES))].rope is not None
    k2 = k.clone()
    out = triton_attn_func(q, k2, v, causal=True, rotary_cos=cos, rotary_sin=sin)
    n1 = counts(stub)
    assert n1[0] == n0[0] + 1 and n1[2] == n0[2] + 1  # one RoPE pre-pass, one attention launch
    a = stub.stub_last_fwd().contents
    rope = list(stub.stub_last_rope().contents)
    assert struct_bytes(a) == full
    assert (a.rope_cos, a.rope_sin) == (cos.data_ptr(), sin.data_ptr())
    assert rope[0] == k2.data_ptr() and a.k == rope[5]  # the kernel reads the rotated k
    # every RoPE argument but the input and output pointers is the full path's
    assert [rope[i] for i in range(16) if i not in (0, 5)] == [rope_full[i] for i in range(16) if i not in (0, 5)]
    assert out.shape == q.shape


def test_rope_tables_that_need_a_copy_are_not_cached(stub):
    from trinix_amd import triton_attn_func

    q, k, v = qkv(S=80, D=128)
    cos, sin = torch.randn(80, 128), torch.randn(80, 128)  # fp32 tables: converted to bf16 on every call
    triton_attn_func(q, k, v, rotary_cos=cos, rotary_sin=sin)
    assert len(ak._LAUNCHES) == 0


def test_decode_split_plan_is_cached(stub):
    from trinix_amd import triton_attn_func

    q = torch.randn(3, 1, 8, 128).to(torch.bfloat16)
    k = torch.randn(3, 500, 2, 128).to(torch.bfloat16)
    v = torch.randn_like(k)
    triton_attn_func(q, k, v)
    c0 = counts(stub)
    full = struct_bytes(stub.stub_last_split().contents)
    triton_attn_func(q.clone(), k, v)
    c1 = counts(stub)
    assert c1[1] == c0[1] + 1 and c1[3] == c0[3]  # launched again without a new plan call
    assert struct_bytes(stub.stub_last_split().contents) == full and stub.stub_split_ws() == 4096


@pytest.mark.parametrize("feature", ["mask", "alibi", "dropout", "lse", "grad"])
def test_calls_with_other_features_are_not_cached(stub, feature):
    from trinix_amd import triton_attn_func

    q, k, v = qkv()
    kw = {}
    if feature == "mask":
        kw["attn_mask"] = torch.zeros(96, 96)
    elif feature == "alibi":
        kw["alibi_slopes"] = torch.ones(4)
    elif feature == "dropout":
        kw["dropout_p"] = 0.1
    elif feature == "lse":
        kw["return_lse"] = True
    elif feature == "grad":
        q.requires_grad_(True)
        kw["dropout_p"] = 0.0
    if feature == "mask":
        pytest.importorskip("numpy")
    try:
        triton_attn_func(q, k, v, **kw)
    except Exception:
        pass  # the stub has no mask pre-pass output to return; only the cache matters here
    assert len(ak._LAUNCHES) == 0


BWD_PTRS = ("q", "k", "v", "out", "dout", "lse", "delta", "dq", "dk", "dv", "dropout_keep_map")


def bwd_bytes(a, zero=BWD_PTRS + ("dropout_seed",)):
    b = nat.AttnBwdArgs.from_buffer_copy(a)
    for f in zero:
        setattr(b, f, 0 if f == "dropout_seed" else None)
    return bytes(b)


def _train_step(q, k, v, do, **kw):
    from trinix_amd import triton_attn_func

    ts = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    out = triton_attn_func(*ts, **kw)
    out.backward(do)
    return ts, out


@pytest.mark.parametrize("dropout", [0.0, 0.2])
def test_training_launches_are_cached(stub, monkeypatch, dropout):
    """A differentiable call of a cached layout hands the forward and the
    backward the full path's structs, its own pointers and, with dropout, a
    fresh seed shared by its forward and backward (and its keep map)."""
    monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", "1")
    q, k, v = qkv(S=70, D=128)
    do = torch.randn_like(q)
    kw = dict(causal=True, dropout_p=dropout)
    c0 = counts(stub)
    _train_step(q, k, v, do, **kw)
    n0 = counts(stub)
    assert n0[0] == c0[0] + 1 and n0[4] == c0[4] + 1 and len(ak._TRAIN_LAUNCHES) == 1
    fwd_full = struct_bytes(stub.stub_last_fwd().contents, zero=("q", "k", "v", "out", "lse", "dropout_keep_map"))
    f_full = nat.AttnFwdArgs.from_buffer_copy(stub.stub_last_fwd().contents)
    b_full = nat.AttnBwdArgs.from_buffer_copy(stub.stub_last_bwd().contents)
    ent = ak._TRAIN_LAUNCHES[next(iter(ak._TRAIN_LAUNCHES))]
    assert ent.bwd is not None
    seeds = {f_full.dropout_seed}
    for rep in range(2):
        q2, k2, v2 = qkv(S=70, D=128, seed=10 + rep)
        ts, out = _train_step(q2, k2, v2, do, **kw)
        assert counts(stub)[0] == n0[0] + rep + 1 and counts(stub)[4] == n0[4] + rep + 1
        f = nat.AttnFwdArgs.from_buffer_copy(stub.stub_last_fwd().contents)
        b = nat.AttnBwdArgs.from_buffer_copy(stub.stub_last_bwd().contents)
        cmp = nat.AttnFwdArgs.from_buffer_copy(f)
        cmp.dropout_seed = f_full.dropout_seed
        assert struct_bytes(cmp, zero=("q", "k", "v", "out", "lse", "dropout_keep_map")) == fwd_full
        b_cmp = nat.AttnBwdArgs.from_buffer_copy(b)
        assert bwd_bytes(b_cmp) == bwd_bytes(b_full)
        assert (f.q, f.k, f.v) == tuple(t.data_ptr() for t in ts) and f.out == out.data_ptr()
        assert (b.q, b.k, b.v, b.out, b.lse) == (f.q, f.k, f.v, f.out, f.lse)
        assert b.dq == ts[0].grad.data_ptr() and b.dk == ts[1].grad.data_ptr() and b.dv == ts[2].grad.data_ptr()
        assert b.dropout_seed == f.dropout_seed and b.dropout_keep_map == f.dropout_keep_map
        if dropout:
            assert f.dropout_keep_map and f.dropout_p == pytest.approx(dropout)
            seeds.add(f.dropout_seed)
        else:
            assert not f.dropout_keep_map and f.dropout_seed == 0
    assert len(seeds) == (3 if dropout else 1)
    assert len(ak._TRAIN_LAUNCHES) == 1


def test_training_cache_follows_the_keep_map_switch(stub, monkeypatch):
    q, k, v = qkv(S=70, D=64)
    do = torch.randn_like(q)
    for mode, want in (("1", True), ("0", False), ("1", True), ("0", False)):
        monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", mode)
        _train_step(q, k, v, do, causal=True, dropout_p=0.1)
        f = stub.stub_last_fwd().contents
        b = stub.stub_last_bwd().contents
        assert bool(f.dropout_keep_map) == want and b.dropout_keep_map == f.dropout_keep_map
    assert len(ak._TRAIN_LAUNCHES) == 2


def test_training_with_alibi_or_mask_is_not_cached(stub, monkeypatch):
    q, k, v = qkv(S=70, D=64)
    do = torch.randn_like(q)
    c0 = counts(stub)
    _train_step(q, k, v, do, alibi_slopes=torch.ones(4))
    _train_step(q, k, v, do, attn_mask=torch.zeros(70, 70))
    assert len(ak._TRAIN_LAUNCHES) == 0 and counts(stub)[4] == c0[4] + 2
