"""Seeded random sweep of the differentiable API against the oracle: the
training-side complement of ``test_random_configs_gpu.py`` (forward and lse
over the dispatch paths and tile shapes).

Each seed draws one configuration: batch, lengths (including single rows,
single keys and decode-shaped calls against long key ranges), q/kv heads
(MHA, GQA, MQA), head_dim (32, 64, 96, 128, 256), dtype, causal, window,
ALiBi, an additive mask (fp32/bf16/bool, 2-D or 4-D, with -inf entries),
scale, ALiBi slopes per head or per (batch, head), dropout with and
without the keep map, the operands' layout (contiguous, (B, H, S, D)
transposed, head slices of one packed buffer, last-dim slices of one fused
projection output), the lse output, fused RoPE tables (the oracle rotates
q and k with the same tables, in the input dtype, as eager RoPE does), and
training or inference.
Output, lse and gradients are checked against fp64 autograd of the oracle
(``functional_attention``, with the kernel's Philox keep mask under
dropout) next to the same autograd in the input dtype ("eager"):

* output and each gradient: max error within twice eager's plus one unit
  roundoff of the input dtype (fp16: 2e-3, fp32: 1e-5) times the scale
  (output: its own; gradients: the largest gradient);
* a dq or dk whose fp64 value is exactly zero (every row it collects has a
  single allowed key, so the softmax backward vanishes): the kernels take
  delta = rowsum(dO * O) from their rounded output O_h, so for such a row
  dS = dO . (O - O_h) exactly, and dq_i = c dS k_j, dk_j = c sum_i dS q_i.
  The bar is twice that bound, with e_i = sum_d |dO_id| |O_id - O_h,id|:
  |c| max e max|k| for dq, |c| G n max e max|q| for dk (G q-heads per KV
  head, n rows per key allowed by the causal / window band), plus 4e-6 of
  the gradient scale;
* lse: within one unit roundoff of the fp64 log-sum-exp (the 16-bit
  kernels sum P as rounded for P @ V) plus fp32 slack.
"""
import random

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from trinix_amd import triton_attn_func

pytestmark = pytest.mark.gpu
DEV = "cuda"
UNIT = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
SLACK = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2.0 ** -8}


def draw(seed):
    r = random.Random(seed)
    D = r.choice([64, 64, 128, 128, 256, 96, 32])
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    B = r.choice([1, 2])
    Hkv = r.choice([1, 2, 4])
    H = Hkv * r.choice([1, 2, 4])
    Sq = r.choice([1, 5, 17, 64, 100, 128, 150, 257, 300])
    Sk = r.choice([Sq, Sq, 1, 33, 64, 200, 320])
    if Sq <= 17 and r.random() < 0.4:
        Sk = r.choice([700, 1500, 2049, 4096])
    layout = r.choice(["bshd", "bshd", "bhsd", "packed"])
    want_lse = r.random() < 0.3
    kw = {}
    if r.random() < 0.5:
        kw["causal"] = True
    if r.random() < 0.25:
        kw["window_size"] = (r.randint(0, 80), r.choice([0, r.randint(0, 50)]))
    if r.random() < 0.3:
        kw["alibi_slopes"] = orc.alibi_slopes(H)
    if r.random() < 0.3:
        g = torch.Generator().manual_seed(seed)
        kind = r.choice(["float", "bool", "bf16"])
        shape = r.choice([(Sq, Sk), (B, 1, Sq, Sk), (B, H, Sq, Sk)])
        if kind == "bool":  # additive 0 / 1, as the reference adds any mask
            m = torch.rand(*shape, generator=g) > 0.15
        else:
            m = torch.randn(*shape, generator=g) * 0.5
            m = m.masked_fill(torch.rand(*shape, generator=g) < 0.1, float("-inf"))
            m[..., 0] = 0.0
            if kind == "bf16":
                m = m.to(torch.bfloat16)
        kw["attn_mask"] = m
    if r.random() < 0.2:
        kw["softmax_scale"] = r.choice([0.05, 0.3, -0.1])
    # every row keeps an allowed key (the oracle's softmax of an empty row is
    # NaN and spreads NaN through its autograd; covered by its own tests)
    i, j = torch.arange(Sq)[:, None], torch.arange(Sk)[None, :]
    ok = torch.ones(Sq, Sk, dtype=torch.bool)
    if kw.get("causal"):
        ok &= j <= i
    if "window_size" in kw:
        ok &= (j - i >= -kw["window_size"][0]) & (j - i <= kw["window_size"][1])
    if "attn_mask" in kw and kw["attn_mask"].dtype != torch.bool:
        ok &= torch.isfinite(kw["attn_mask"].float()).reshape(-1, Sq, Sk).all(0)
    if not ok.any(1).all():
        kw.pop("window_size", None)
    p = r.choice([0.0, 0.0, 0.0, 0.1, 0.3])
    train = r.random() < (0.7 if Sk < 700 else 0.2) or p > 0
    keep_map = r.choice(["1", "0"])
    rope_base = r.choice([1e4, 5e5]) if r.random() < 0.2 else None  # fused RoPE (rotary_cos / rotary_sin)
    # ALiBi slopes as (H,), (1, H) or (B, H) (per-batch slopes)
    slope_shape = r.choice(["h", "1h", "bh"])
    if "alibi_slopes" in kw and slope_shape != "h":
        sl = kw["alibi_slopes"]
        kw["alibi_slopes"] = (sl[None] if slope_shape == "1h" else
                              torch.stack([sl * (1.0 + 0.5 * bb) for bb in range(B)]))
    # q, k, v as last-dim slices of one fused projection output (B, S, H, 3D + 8)
    if r.random() < 0.15 and H == Hkv and Sq == Sk and layout == "bshd":
        layout = "qkv_last"
    return dict(B=B, Sq=Sq, Sk=Sk, H=H, Hkv=Hkv, D=D, dtype=dtype, layout=layout, want_lse=want_lse, kw=kw, p=p,
                train=train, keep_map=keep_map, rope_base=rope_base)


def _rope_tables(c):
    """The RoPE tables in the input dtype (the kernel reads them so; the
    fp64 oracle takes the same rounded values), or None."""
    if c["rope_base"] is None:
        return None
    return orc.rope_tables(max(c["Sq"], c["Sk"]), c["D"], c["rope_base"], c["dtype"])


def _oracle(q, k, v, do, dt, c, keep):
    ts = [t.detach().to(dt).clone().requires_grad_(c["train"]) for t in (q, k, v)]
    extra = dict(keep=keep, dropout_p=c["p"]) if c["p"] > 0 else {}
    qa, ka = ts[0], ts[1]
    tables = _rope_tables(c)
    if tables is not None:
        cos, sin = (t.to(dt) for t in tables)
        qa, ka = orc.apply_rope(qa, cos, sin), orc.apply_rope(ka, cos, sin)
    out = orc.functional_attention(qa, ka, ts[2], **c["kw"], **extra)
    if not c["train"]:
        return out.detach().double(), []
    out.backward(do.to(dt))
    return out.detach().double(), [t.grad.double() for t in ts]


def _hip(q, k, v, do, c):
    B, Sq, Sk, H, Hkv, D, dtype = (c[n] for n in ("B", "Sq", "Sk", "H", "Hkv", "D", "dtype"))
    train = c["train"]
    ts = [t.to(DEV, dtype) for t in (q, k, v)]
    if c["layout"] == "qkv_last":  # one (B, S, H, 3D + 8) buffer, q / k / v side by side in the last dim
        buf = torch.zeros(B, Sq, H, 3 * D + 8, device=DEV, dtype=dtype)
        buf[..., :D], buf[..., D:2 * D], buf[..., 2 * D:3 * D] = ts
        buf.requires_grad_(train)
        xs = [buf[..., :D], buf[..., D:2 * D], buf[..., 2 * D:3 * D]]
    elif c["layout"] == "packed":  # one (B, S, H + 2 Hkv + 1, D) buffer, the extra head pads the row stride
        buf = torch.zeros(B, max(Sq, Sk), H + 2 * Hkv + 1, D, device=DEV, dtype=dtype)
        buf[:, :Sq, :H], buf[:, :Sk, H:H + Hkv], buf[:, :Sk, H + Hkv:H + 2 * Hkv] = ts
        buf.requires_grad_(train)
        xs = [buf[:, :Sq, :H], buf[:, :Sk, H:H + Hkv], buf[:, :Sk, H + Hkv:H + 2 * Hkv]]
    else:
        if c["layout"] == "bhsd":
            ts = [t.transpose(1, 2).contiguous().transpose(1, 2) for t in ts]
        xs = [t.requires_grad_(train) for t in ts]
    kw = {key: (val.to(DEV) if torch.is_tensor(val) else val) for key, val in c["kw"].items()}
    tables = _rope_tables(c)
    if tables is not None:
        kw["rotary_cos"], kw["rotary_sin"] = (t.to(DEV) for t in tables)
    torch.manual_seed(4321)  # the dropout seed comes from torch's CPU generator
    res = triton_attn_func(*xs, dropout_p=c["p"], return_lse=c["want_lse"], **kw)
    out, lse = res if c["want_lse"] else (res, None)
    grads = []
    if train:
        out.backward(do.to(DEV, dtype))
        if c["layout"] == "packed":
            gb = buf.grad
            grads = [gb[:, :Sq, :H], gb[:, :Sk, H:H + Hkv], gb[:, :Sk, H + Hkv:H + 2 * Hkv]]
        elif c["layout"] == "qkv_last":
            gb = buf.grad
            grads = [gb[..., :D], gb[..., D:2 * D], gb[..., 2 * D:3 * D]]
        else:
            grads = [t.grad for t in xs]
    return (out.detach().cpu().double(), [g.cpu().double() for g in grads],
            None if lse is None else lse.cpu().double())


@pytest.mark.parametrize("seed", range(200))
def test_random_configuration(seed, monkeypatch):
    c = draw(seed)
    print(f"seed {seed}: {({k: v for k, v in c.items() if k != 'kw'})} {sorted(c['kw'])}", flush=True)
    monkeypatch.setenv("TRINIX_DROPOUT_KEEP_MAP", c["keep_map"])
    B, Sq, Sk, H, Hkv, D, dtype = (c[n] for n in ("B", "Sq", "Sk", "H", "Hkv", "D", "dtype"))
    g = torch.Generator().manual_seed(10_000 + seed)
    q, k, v = (torch.randn(B, s, h, D, generator=g) for s, h in ((Sq, H), (Sk, Hkv), (Sk, Hkv)))
    do = torch.randn(B, Sq, H, D, generator=g)
    keep = None
    if c["p"] > 0:
        torch.manual_seed(4321)
        drop_seed = int(torch.randint(0, 2 ** 62, (1,)).item())
        keep = torch.from_numpy(orc.dropout_keep(B, H, Sq, Sk, c["p"], drop_seed))
    o64, g64 = _oracle(q, k, v, do, torch.float64, c, keep)
    oe, ge = _oracle(q, k, v, do, dtype, c, keep)
    oh, gh, lse = _hip(q, k, v, do, c)
    assert torch.equal(torch.isfinite(oh), torch.isfinite(o64))
    u, slack = UNIT[dtype], SLACK[dtype]
    gsc = max([t.abs().max().item() for t in g64] + [0.0])
    # bound of a single-key row's dS from the rounding of the output the
    # delta is taken from (see the module docstring)
    kw = c["kw"]
    i, j = torch.arange(Sq)[:, None], torch.arange(Sk)[None, :]
    band = torch.ones(Sq, Sk, dtype=torch.bool)
    if kw.get("causal"):
        band &= j <= i
    if "window_size" in kw:
        band &= (j - i >= -kw["window_size"][0]) & (j - i <= kw["window_size"][1])
    fin = torch.isfinite(o64)
    e_max = (do.to(dtype).double().abs() * (o64 - oh).abs()).masked_fill(~fin, 0).sum(-1).max().item()
    cs = abs(kw.get("softmax_scale", D ** -0.5))
    qx, kx = q.to(dtype), k.to(dtype)  # the operands the scores are taken of (rotated in the input dtype)
    tables = _rope_tables(c)
    if tables is not None:
        qx, kx = orc.apply_rope(qx, *tables), orc.apply_rope(kx, *tables)
    zero_bound = {"dq": cs * e_max * kx.abs().max().item(),
                  "dk": cs * (H // Hkv) * int(band.sum(0).max()) * e_max * qx.abs().max().item()}
    for name, h, e, t in [("out", oh, oe, o64)] + list(zip(("dq", "dk", "dv"), gh, ge, g64)):
        f = torch.isfinite(t)
        assert h.shape == t.shape, name
        sc = t[f].abs().max().item() if name == "out" else gsc
        eh = (h[f] - t[f]).abs().max().item()
        ee = (e[f] - t[f]).abs().max().item()
        if name in ("dq", "dk") and t.abs().max().item() == 0.0:
            assert eh <= 2 * zero_bound[name] + 4e-6 * sc, (name, "zero truth", eh, zero_bound[name], sc)
        else:
            assert eh <= 2 * ee + slack * sc, (name, eh, ee, sc)
    if lse is not None:
        s = torch.einsum("bihd,bjhd->bhij", qx.double(), kx.double().repeat_interleave(H // Hkv, 2))
        s = s * kw.get("softmax_scale", D ** -0.5) + torch.from_numpy(orc._bias64(
            Sq, Sk, H, B, kw.get("attn_mask"), kw.get("causal", False), kw.get("window_size"), kw.get("alibi_slopes")))
        ref = torch.logsumexp(s, -1)
        assert lse.shape == ref.shape
        err = (lse - ref).abs().max().item()
        assert err <= (0.0 if dtype == torch.float32 else u) + 2e-5 * (1 + ref.abs().max().item()), err
