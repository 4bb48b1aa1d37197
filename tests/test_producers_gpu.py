"""GPU tests of the producers either side of the attention call: the ALiBi
bias kernel (reference ``trinix/kernels/alibi_kernel.py``) against the eager
formula (``alibi.py:82-90``), and the RoPE autograd function (reference
``rope_kernel.py:134-177``) against eager autograd of the oracle rotation."""
import pytest
import torch

import trinix_amd as tx
from oracle import attention_oracle as orc
from trinix_amd.kernels import TritonALiBiKernel, TritonRoPEKernel

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("heads,seq,batch", [(8, 128, 2), (12, 100, 1), (3, 7, 3), (16, 2048, 1)])
def test_alibi_kernel_bitwise_equals_eager(heads, seq, batch):
    emb = tx.FastALiBiPositionEmbedding(heads).to(DEV)
    got = emb(seq, batch_size=batch)
    want = emb._compute_alibi_pytorch(seq, batch)
    assert got.shape == (batch, heads, seq, seq) and got.dtype == torch.float32
    assert torch.equal(got, want)
    # the same values as the oracle's closed form
    assert torch.equal(got[0].cpu(), orc.alibi_bias(seq, seq, orc.alibi_slopes(heads)))


def test_alibi_kernel_dtype_and_no_grad():
    sl = orc.alibi_slopes(8).to(DEV, torch.bfloat16).requires_grad_(True)
    b = TritonALiBiKernel.apply(sl, 2, 8, 33)
    assert b.dtype == torch.bfloat16 and b.shape == (2, 8, 33, 33)
    ref = -(sl.detach().float()[:, None, None] * (torch.arange(33, device=DEV)[None, :] -
                                                 torch.arange(33, device=DEV)[:, None]).abs().float())
    assert torch.equal(b[1], ref.to(torch.bfloat16))
    b.float().sum().backward()  # reference backward returns no gradient for the slopes
    assert sl.grad is None


def test_alibi_eager_and_kernel_paths_agree():
    emb = tx.FastALiBiPositionEmbedding(4).to(DEV)
    emb.use_triton = False
    assert torch.equal(emb(16), tx.FastALiBiPositionEmbedding(4).to(DEV)(16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rope_autograd_matches_eager_autograd(dtype):
    torch.manual_seed(7)
    B, S, H, D = 2, 40, 4, 64
    cos, sin = orc.rope_tables(S, D, 10000.0, dtype)
    q = torch.randn(B, S, H, D).to(dtype)
    k = torch.randn(B, S, 2, D).to(dtype)
    gq, gk = torch.randn(B, S, H, D).to(dtype), torch.randn(B, S, 2, D).to(dtype)
    # eager autograd of the oracle rotation (CPU)
    qe, ke = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    torch.autograd.backward([orc.apply_rope(qe, cos, sin), orc.apply_rope(ke, cos, sin)], [gq, gk])
    # HIP forward and backward
    qd, kd = q.to(DEV).requires_grad_(True), k.to(DEV).requires_grad_(True)
    oq, ok = TritonRoPEKernel.apply(qd, kd, cos.to(DEV), sin.to(DEV))
    assert torch.equal(oq.detach().cpu(), orc.apply_rope(q, cos, sin))
    torch.autograd.backward([oq, ok], [gq.to(DEV), gk.to(DEV)])
    assert torch.equal(qd.grad.cpu(), qe.grad) and torch.equal(kd.grad.cpu(), ke.grad)
