"""CPU-only checks of the C ABI library and the host logic: the library
loads, exports every function ``include/trinix_attn.h`` declares, the ctypes
mirror of ``trinix_attn_fwd_args`` has the C layout, argument validation
returns the right status codes (no kernel is launched), and the Python layer
raises the reference's exception types."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

from trinix_amd import _native as nat
from trinix_amd.build import LIB_PATH, INCLUDE_DIR, build

HEADER = os.path.join(INCLUDE_DIR, "trinix_attn.h")


@pytest.fixture(scope="module")
def lib():
    if not LIB_PATH.exists():
        build()
    return nat.load_library()


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(trinix_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(nat.SIGNATURES), "ctypes signature table out of sync with the header"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True, text=True).stdout
    for n in names:
        assert re.search(rf"\bT {n}$", out, re.M), n


@pytest.mark.parametrize("cname,pyty", [("trinix_attn_fwd_args", "AttnFwdArgs"),
                                         ("trinix_attn_bwd_args", "AttnBwdArgs"),
                                         ("trinix_tile_cfg", "TileCfg")])
def test_struct_layout_matches_c(lib, cname, pyty):
    cls = getattr(nat, pyty)
    fields = [f for f, _ in cls._fields_]
    prog = ['#include <stdio.h>', '#include <stddef.h>', '#include "trinix_attn.h"', "int main(void){",
            f'printf("%zu\\n", sizeof({cname}));']
    prog += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    prog += ["return 0;}"]
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(src, "w").write("\n".join(prog))
        subprocess.run(["gcc", "-std=c99", "-I", str(INCLUDE_DIR), src, "-o", exe], check=True)
        vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(cls)
    for f, off in zip(fields, vals[1:]):
        assert getattr(cls, f).offset == off, f


def test_version_status_and_tiles(lib):
    assert lib.trinix_abi_version() == nat.ABI_VERSION
    for code in range(10):
        assert lib.trinix_status_string(code)
    cfg = nat.TileCfg()
    assert lib.trinix_attn_tile_config(128, nat.TRINIX_BF16, ctypes.byref(cfg)) == 0
    assert cfg.block_d == 128 and cfg.block_m % 32 == 0 and cfg.block_n % 64 == 0
    # large problems at head_dim 128: 8 wavefronts x 32 rows, 128-key tiles
    assert (cfg.block_m, cfg.block_n, cfg.waves, cfg.lds_bytes) == (256, 128, 8, 2 * 2 * 128 * 128 * 2)
    assert lib.trinix_attn_tile_config(96, nat.TRINIX_BF16, ctypes.byref(cfg)) == nat.TRINIX_ERR_BAD_HEAD_DIM
    assert lib.trinix_attn_tile_config(256, nat.TRINIX_BF16, ctypes.byref(cfg)) == 0
    assert cfg.block_d == 256 and cfg.lds_bytes == 4 * 64 * 256 * 2
    assert lib.trinix_attn_tile_config(64, 9, ctypes.byref(cfg)) == nat.TRINIX_ERR_BAD_DTYPE


def _args(**kw):
    a = nat.AttnFwdArgs()
    a.q = a.k = a.v = a.out = 4096
    for name in ("q_stride", "k_stride", "v_stride", "out_stride"):
        setattr(a, name, nat.int64x4((8 * 64 * 128, 8 * 128, 128, 1)))
    a.batch, a.seqlen_q, a.seqlen_k, a.nheads_q, a.nheads_kv, a.head_dim = 1, 64, 64, 8, 8, 128
    a.dtype = nat.TRINIX_BF16
    a.softmax_scale = 0.1
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=96), nat.TRINIX_ERR_BAD_HEAD_DIM),
    (dict(dtype=7), nat.TRINIX_ERR_BAD_DTYPE),
    (dict(nheads_kv=3), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(seqlen_q=0), nat.TRINIX_ERR_BAD_SHAPE),
    # every zero-sized dimension is rejected (no empty launch)
    (dict(seqlen_k=0), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(batch=0), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(nheads_q=0), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(q=None), nat.TRINIX_ERR_NULL_POINTER),
    (dict(q_stride=nat.int64x4((1, 1, 1, 2))), nat.TRINIX_ERR_BAD_STRIDE),
    (dict(k_stride=nat.int64x4((8 * 64 * 128, 8 * 128, 130, 1))), nat.TRINIX_ERR_BAD_STRIDE),
    # 16-bit K/V tiles are addressed with 32-bit in-tile offsets: key-row stride < 2^22 elements
    (dict(k_stride=nat.int64x4((1 << 30, 1 << 22, 128, 1))), nat.TRINIX_ERR_BAD_STRIDE),
    (dict(v_stride=nat.int64x4((1 << 30, 1 << 22, 128, 1))), nat.TRINIX_ERR_BAD_STRIDE),
    (dict(dropout_p=1.0), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(mask_blockmap=4096), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(dropout_p=0.1, dropout_state=4100), nat.TRINIX_ERR_BAD_ARGUMENT),  # {seed, offset}: 8-byte aligned
    # mask strides are non-negative, and the 32 rows of a query sub-tile sit
    # at 32-bit offsets from its first row: min(Sq - 1, 31) * row stride < 2^31
    (dict(mask=4096, mask_dtype=nat.TRINIX_F32, mask_stride=nat.int64x4((0, 0, -64, 1))), nat.TRINIX_ERR_BAD_STRIDE),
    (dict(mask=4096, mask_dtype=nat.TRINIX_F32, mask_stride=nat.int64x4((0, 0, 1 << 27, 1))),
     nat.TRINIX_ERR_BAD_STRIDE),
    # a dropout keep map: with dropout, 16-byte aligned, bf16/fp16 at head_dim 64/128
    (dict(dropout_keep_map=4096), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(dropout_p=0.1, dropout_keep_map=4104), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(dropout_p=0.1, dropout_keep_map=4096, dtype=nat.TRINIX_F32), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(dropout_p=0.1, dropout_keep_map=4096, head_dim=256,
          **{n: nat.int64x4((8 * 64 * 256, 8 * 256, 256, 1)) for n in ("q_stride", "k_stride", "v_stride",
                                                                       "out_stride")}),
     nat.TRINIX_ERR_BAD_ARGUMENT),
])
def test_validation_rejects_before_launch(lib, kw, code):
    a = _args(**kw)
    assert lib.trinix_attn_fwd(ctypes.byref(a), None) == code


def _bwd_args(**kw):
    a = nat.AttnBwdArgs()
    a.q = a.k = a.v = a.out = a.dout = a.lse = a.delta = a.dq = a.dk = a.dv = 4096
    for name in ("q", "k", "v", "out", "dout", "dq", "dk", "dv"):
        setattr(a, name + "_stride", nat.int64x4((8 * 64 * 128, 8 * 128, 128, 1)))
    a.batch, a.seqlen_q, a.seqlen_k, a.nheads_q, a.nheads_kv, a.head_dim = 1, 64, 64, 8, 8, 128
    a.dtype = nat.TRINIX_BF16
    a.softmax_scale = 0.1
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(dropout_p=1.0), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(lse=None), nat.TRINIX_ERR_NULL_POINTER),
    (dict(seqlen_q=0), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(seqlen_k=0), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(batch=0), nat.TRINIX_ERR_BAD_SHAPE),
    (dict(dropout_keep_map=4096), nat.TRINIX_ERR_BAD_ARGUMENT),  # a keep map without dropout
    (dict(dropout_p=0.1, dropout_keep_map=4100), nat.TRINIX_ERR_BAD_ARGUMENT),
    (dict(dropout_p=0.1, dropout_keep_map=4096, dtype=nat.TRINIX_F32), nat.TRINIX_ERR_BAD_ARGUMENT),
])
def test_backward_validation_rejects_before_launch(lib, kw, code):
    a = _bwd_args(**kw)
    assert lib.trinix_attn_bwd(ctypes.byref(a), None) == code


def test_dropout_keep_map_bytes(lib):
    """128 bytes per 32x32 block, 2*ceil(Sq/64) x 4*ceil(Sk/128) blocks per
    (batch, head): every 64-row item and 128-key group of the backward's
    tile copies lies inside the map."""
    n = ctypes.c_int64(0)
    for B, H, Sq, Sk in [(1, 1, 1, 1), (1, 32, 8192, 8192), (2, 3, 65, 129), (4, 12, 1024, 1024), (1, 1, 64, 128)]:
        assert lib.trinix_dropout_keep_map_bytes(B, H, Sq, Sk, ctypes.byref(n)) == 0
        nbi, nbj = 2 * -(-Sq // 64), 4 * -(-Sk // 128)
        assert n.value == 128 * B * H * nbi * nbj
        assert nbi * 32 >= Sq and nbj * 32 >= Sk and nbi % 2 == 0 and nbj % 4 == 0
    lib.trinix_dropout_keep_map_bytes(1, 32, 8192, 8192, ctypes.byref(n))
    assert n.value == 268435456  # 1/8 byte per (row, key) at full tiles
    assert lib.trinix_dropout_keep_map_bytes(0, 1, 1, 1, ctypes.byref(n)) == nat.TRINIX_ERR_BAD_SHAPE
    assert lib.trinix_dropout_keep_map_bytes(1, 1, 1 << 30, 1, ctypes.byref(n)) == nat.TRINIX_ERR_BAD_SHAPE
    assert lib.trinix_dropout_keep_map_bytes(1, 1, 1, 1, None) == nat.TRINIX_ERR_NULL_POINTER


def test_status_to_exception_types(lib):
    with pytest.raises(ValueError):
        nat.check(nat.TRINIX_ERR_BAD_SHAPE, "x")
    with pytest.raises(RuntimeError):
        nat.check(nat.TRINIX_ERR_LAUNCH, "x")
    nat.check(nat.TRINIX_OK, "x")


def test_functional_api_errors_match_reference():
    from trinix_amd import triton_attn_func
    from trinix_amd.kernels import TritonAttentionKernel

    q = torch.zeros(1, 4, 2, 64)
    with pytest.raises(ValueError, match="only supports CUDA tensors"):
        triton_attn_func(q, q, q)
    m4 = TritonAttentionKernel._prepare_mask(torch.zeros(4, 4), 2, 3, 4)
    assert m4.shape == (2, 3, 4, 4) and m4.stride()[:2] == (0, 0)
    m4 = TritonAttentionKernel._prepare_mask(torch.zeros(2, 4, 4), 2, 3, 4)
    assert m4.stride(1) == 0 and m4.stride(0) == 16
    m4 = TritonAttentionKernel._prepare_mask(torch.zeros(2, 1, 4, 6), 2, 3, 4, 6)
    assert m4.shape == (2, 3, 4, 6)
    with pytest.raises(ValueError, match="Unsupported mask shape"):
        TritonAttentionKernel._prepare_mask(torch.zeros(1, 1, 1, 4, 4), 1, 1, 4)
    with pytest.raises(ValueError):
        TritonAttentionKernel._prepare_mask(torch.zeros(5, 4), 1, 1, 4)
    assert not TritonAttentionKernel.is_available()  # no GPU in this process


def test_kernel_head_dim_padding_rule():
    from trinix_amd.kernels.attention_kernel import kernel_head_dim

    assert [kernel_head_dim(d) for d in (8, 32, 64, 65, 80, 128, 129, 192, 256, 257)] == \
        [64, 64, 64, 128, 128, 128, 256, 256, 256, None]


def _plan(lib, **kw):
    a = _args(**kw)
    ns, wb = ctypes.c_int32(-1), ctypes.c_int64(-1)
    assert lib.trinix_attn_fwd_splitkv_plan(ctypes.byref(a), ctypes.byref(ns), ctypes.byref(wb)) == nat.TRINIX_OK
    return ns.value, wb.value


def test_splitkv_plan(lib):
    """Host-only split plan of the decode kernel: rows of a KV head's q-heads
    packed 16 to a tile, the visible keys cut into chunks of >= 128 keys
    (multiples of 64) until about 1024 workgroups exist; fp32 partial O and
    lse per (row, chunk) when there is more than one chunk."""
    dec = dict(seqlen_q=1, seqlen_k=8192, nheads_q=32, nheads_kv=8)
    # 8 (batch, KV head) items -> 128 chunks wanted, capped at 8192/128 = 64
    assert _plan(lib, **dec) == (64, 8 * 4 * 64 * (128 + 1) * 4)
    # batch 8: 64 items -> 16 chunks of 512 keys; batch 64: 512 items -> 2 chunks
    assert _plan(lib, **dec, batch=8) == (16, 8 * 8 * 4 * 16 * 129 * 4)
    assert _plan(lib, **dec, batch=64) == (2, 64 * 8 * 4 * 2 * 129 * 4)
    # >= 1024 items: one chunk, the output is written directly (no workspace)
    assert _plan(lib, **dec, batch=128) == (1, 0)
    # 3 rows x G=4 = 12 packed rows, D=64, 1000 keys -> ceil(1000/128)=8 chunks of 128
    assert _plan(lib, seqlen_q=3, seqlen_k=1000, nheads_q=8, nheads_kv=2, head_dim=64) == (8, 2 * 12 * 8 * 65 * 4)
    # top-left causal with one query row sees key 0 only; a window bounds the span
    assert _plan(lib, **dec, causal=1) == (1, 0)
    assert _plan(lib, **dec, has_window=1, window_left=10, window_right=300) == (3, 8 * 4 * 3 * 129 * 4)
    # not applicable -> 0 chunks (trinix_attn_fwd is the path)
    assert _plan(lib, **dec, dtype=nat.TRINIX_F32)[0] == 0
    assert _plan(lib, **dec, dropout_p=0.1)[0] == 0
    assert _plan(lib, **dict(dec, seqlen_q=17))[0] == 0
    assert _plan(lib, **dec, rope_cos=4096, rope_sin=4096, rope_stride=64)[0] == 0
    assert _plan(lib, **dec, has_window=1, window_left=-10, window_right=-20)[0] == 0  # no visible key


def test_splitkv_rejects_before_launch(lib):
    a = _args(seqlen_q=1, seqlen_k=8192, nheads_q=32, nheads_kv=8)
    _, need = _plan(lib, seqlen_q=1, seqlen_k=8192, nheads_q=32, nheads_kv=8)
    assert lib.trinix_attn_fwd_splitkv(ctypes.byref(a), 4096, need - 4, None) == nat.TRINIX_ERR_BAD_ARGUMENT
    assert lib.trinix_attn_fwd_splitkv(ctypes.byref(a), None, need, None) == nat.TRINIX_ERR_BAD_ARGUMENT
    assert lib.trinix_attn_fwd_splitkv(ctypes.byref(a), 4100, need, None) == nat.TRINIX_ERR_BAD_ARGUMENT
    f32 = _args(seqlen_q=1, seqlen_k=8192, dtype=nat.TRINIX_F32)
    assert lib.trinix_attn_fwd_splitkv(ctypes.byref(f32), 4096, 1 << 30, None) == nat.TRINIX_ERR_BAD_ARGUMENT
    ns, wb = ctypes.c_int32(), ctypes.c_int64()
    assert lib.trinix_attn_fwd_splitkv_plan(ctypes.byref(_args(head_dim=96)), ctypes.byref(ns),
                                            ctypes.byref(wb)) == nat.TRINIX_ERR_BAD_HEAD_DIM
    assert lib.trinix_attn_fwd_splitkv_plan(ctypes.byref(a), None, ctypes.byref(wb)) == nat.TRINIX_ERR_NULL_POINTER


def test_splitkv_noalloc_rejects_before_launch(lib, monkeypatch):
    """The no-allocation entry point validates like trinix_attn_fwd_splitkv
    and refuses a plan whose workspace exceeds its static scratch, before
    touching the device (host-only paths)."""
    dec = dict(seqlen_q=1, seqlen_k=8192, nheads_q=32, nheads_kv=8)
    assert lib.trinix_attn_fwd_splitkv_noalloc(None, None) == nat.TRINIX_ERR_NULL_POINTER
    assert lib.trinix_attn_fwd_splitkv_noalloc(ctypes.byref(_args(**dec, head_dim=96)), None) == \
        nat.TRINIX_ERR_BAD_HEAD_DIM
    assert lib.trinix_attn_fwd_splitkv_noalloc(ctypes.byref(_args(**dec, dtype=nat.TRINIX_F32)), None) == \
        nat.TRINIX_ERR_BAD_ARGUMENT
    assert lib.trinix_attn_fwd_splitkv_noalloc(ctypes.byref(_args(**dict(dec, seqlen_q=17))), None) == \
        nat.TRINIX_ERR_BAD_ARGUMENT
    # a tuning override that asks for far more chunks than the default plan
    big = dict(batch=64, seqlen_q=16, seqlen_k=4096, nheads_q=32, nheads_kv=8)
    monkeypatch.setenv("TRINIX_SPLITKV_CFG", "65536,64")
    ns, need = _plan(lib, **big)
    assert need > nat.SPLITKV_SCRATCH_BYTES
    assert lib.trinix_attn_fwd_splitkv_noalloc(ctypes.byref(_args(**big)), None) == \
        nat.TRINIX_ERR_SCRATCH_TOO_SMALL
    with pytest.raises(ValueError, match="static buffer"):
        nat.check(nat.TRINIX_ERR_SCRATCH_TOO_SMALL, "trinix_attn_fwd_splitkv_noalloc")


def test_splitkv_default_plan_fits_static_scratch(lib):
    """The default plan never asks for more than the no-allocation entry
    point's scratch: the largest workspace comes from just under 1024
    (batch, KV head, 16-row) items, split in two, 16 rows each at D=128."""
    worst = 0
    for batch in (1, 2, 63, 64, 127, 128, 255, 511, 1023):
        for sq, hq, hkv in ((16, 8, 8), (16, 32, 8), (1, 32, 8), (4, 32, 8), (16, 4, 1)):
            for sk in (1 << 10, 1 << 14, 1 << 20):
                worst = max(worst, _plan(lib, batch=batch, seqlen_q=sq, seqlen_k=sk, nheads_q=hq, nheads_kv=hkv,
                                         head_dim=128)[1])
    assert 0 < worst <= 1023 * 16 * 2 * 129 * 4 < nat.SPLITKV_SCRATCH_BYTES


def test_qk_norm_rejects_before_launch(lib):
    st = (ctypes.c_int64 * 4)(8 * 64 * 128, 8 * 128, 128, 1)

    def call(x=4096, out=4096, w=4096, D=128, dtype=nat.TRINIX_BF16, stride=st, cos=None, sin=None):
        return lib.trinix_qk_norm(x, stride, out, stride, 1, 64, 8, D, dtype, w, 1e-6, cos, sin, 64, 64, None, None)

    assert call(D=96) == nat.TRINIX_ERR_BAD_HEAD_DIM
    assert call(dtype=nat.TRINIX_F32) == nat.TRINIX_ERR_BAD_DTYPE
    assert call(w=None) == nat.TRINIX_ERR_NULL_POINTER
    assert call(cos=4096) == nat.TRINIX_ERR_NULL_POINTER
    assert call(x=4100) == nat.TRINIX_ERR_BAD_STRIDE
    assert call(stride=(ctypes.c_int64 * 4)(8 * 64 * 128, 8 * 128, 130, 1)) == nat.TRINIX_ERR_BAD_STRIDE
    # tables shorter than the sequence (no position ids)
    assert lib.trinix_qk_norm(4096, st, 4096, st, 1, 64, 8, 128, nat.TRINIX_BF16, 4096, 1e-6, 4096, 4096, 64, 63,
                              None, None) == nat.TRINIX_ERR_BAD_SHAPE
    assert lib.trinix_rope_apply(4096, st, 4096, st, 1, 64, 8, 128, nat.TRINIX_BF16, 4096, 4096, 64, 63,
                                 None, None) == nat.TRINIX_ERR_BAD_SHAPE


def test_qk_layernorm_and_backward_reject_before_launch(lib):
    st = (ctypes.c_int64 * 4)(8 * 64 * 128, 8 * 128, 128, 1)

    def ln(x=4096, w=4096, b=4096, D=128, dtype=nat.TRINIX_BF16):
        return lib.trinix_qk_layernorm(x, st, 4096, st, 1, 64, 8, D, dtype, w, b, 1e-5, None, None, 0, 0, None,
                                       None)

    assert ln(b=None) == nat.TRINIX_ERR_NULL_POINTER  # LayerNorm needs its bias
    assert ln(D=48) == nat.TRINIX_ERR_BAD_HEAD_DIM
    assert ln(dtype=nat.TRINIX_F32) == nat.TRINIX_ERR_BAD_DTYPE
    assert ln(b=4100) == nat.TRINIX_ERR_BAD_STRIDE

    def bwd(norm=nat.TRINIX_NORM_RMS, dwp=4096, dbp=None, rows=16, dx=4096, dout=4096, cos=None):
        return lib.trinix_qk_norm_bwd(4096, st, dout, st, dx, st, 1, 64, 8, 128, nat.TRINIX_BF16, norm, 4096, 1e-6,
                                      cos, None, 64, 64, None, dwp, dbp, rows, None)

    assert bwd(norm=7) == nat.TRINIX_ERR_BAD_ARGUMENT
    assert bwd(dwp=None) == nat.TRINIX_ERR_NULL_POINTER
    assert bwd(norm=nat.TRINIX_NORM_LAYER) == nat.TRINIX_ERR_NULL_POINTER  # no dbias partials
    assert bwd(rows=0) == nat.TRINIX_ERR_BAD_SHAPE
    assert bwd(dx=None) == nat.TRINIX_ERR_NULL_POINTER
    assert bwd(dout=4104) == nat.TRINIX_ERR_BAD_STRIDE
    assert bwd(cos=4096) == nat.TRINIX_ERR_NULL_POINTER  # cos without sin


def test_qk_norm_backward_partial_rows():
    from trinix_amd.kernels.qk_norm_kernel import partial_rows

    assert partial_rows(1, 128) == 1
    assert partial_rows(32, 128) == 1 and partial_rows(33, 128) == 2  # 32 rows per pass at D = 128
    assert partial_rows(10 ** 7, 64) == 1024
    assert partial_rows(16, 16) == 1  # 256 rows per pass at D = 16


def test_splitkv_plan_invariants_random(lib):
    """For random decode shapes the plan's chunks tile the visible keys:
    chunk a multiple of 64 and >= 64, ceil(span / chunk) chunks, workspace =
    rows * chunks * (D + 1) * 4 bytes when there is more than one chunk."""
    import random

    r = random.Random(7)
    for _ in range(300):
        Hkv = r.choice([1, 2, 4, 8])
        kw = dict(batch=r.randint(1, 300), seqlen_q=r.randint(1, 16), seqlen_k=r.randint(1, 100000),
                  nheads_kv=Hkv, nheads_q=Hkv * r.choice([1, 2, 4, 8]), head_dim=r.choice([64, 128]))
        if r.random() < 0.3:
            kw["causal"] = 1
        if r.random() < 0.3:
            kw.update(has_window=1, window_left=r.randint(-50, 5000), window_right=r.randint(-50, 5000))
        ns, wb = _plan(lib, **kw)
        Sq, Sk = kw["seqlen_q"], kw["seqlen_k"]
        lo, hi = 0, Sk - 1
        if kw.get("causal"):
            hi = min(hi, Sq - 1)
        if kw.get("has_window"):
            lo = max(lo, -kw["window_left"])
            hi = min(hi, Sq - 1 + kw["window_right"])
        lo, khi = min(lo, Sk), max(0, min(Sk, hi + 1))
        span = khi - lo
        if span <= 0:
            assert ns == 0
            continue
        assert ns >= 1
        rows = kw["nheads_q"] // Hkv * Sq
        items = kw["batch"] * Hkv * ((rows + 15) // 16)
        chunk = -(-span // ns)
        assert ns == 1 or (ns - 1) * ((chunk + 63) // 64 * 64) < span
        assert items * ns < 2 ** 31
        assert wb == (0 if ns == 1 else kw["batch"] * Hkv * rows * ns * (kw["head_dim"] + 1) * 4)
        assert wb <= nat.SPLITKV_SCRATCH_BYTES
