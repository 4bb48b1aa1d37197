"""HIP graph capture of the attention paths (serving loops capture decode
steps; training loops capture whole steps, backward included).  Every entry point enqueues its kernels on the caller's stream and
allocates nothing itself; the host layer's only device-to-host read (the
position_ids range check) is skipped while a stream is capturing, and the
kernels clamp ids to the tables instead.

Each captured graph is replayed several times with new input values copied
into its static inputs, eager work and synchronisations between replays, and
every replay is compared with the eager call on the same values (bitwise:
the same kernels run).
"""
import pytest
import torch

import trinix_amd as tx
from trinix_amd import triton_attn_func

pytestmark = pytest.mark.gpu
DEV = "cuda"


def capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def replay_and_check(g, static_out, inputs, fn, rounds=3):
    for rnd in range(rounds):
        gen = torch.Generator(device=DEV).manual_seed(1000 + rnd)
        for t in inputs:
            t.copy_(torch.randn(t.shape, device=DEV, generator=gen).to(t.dtype))
        torch.cuda.synchronize()
        g.replay()
        _ = torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)  # eager work between replays
        torch.cuda.synchronize()
        ref = fn()
        outs = static_out if isinstance(static_out, (tuple, list)) else (static_out,)
        refs = ref if isinstance(ref, (tuple, list)) else (ref,)
        for o, r in zip(outs, refs):
            assert torch.equal(o, r), f"replay {rnd} differs from eager"


def test_graph_prefill_gqa_fused_rope():
    B, S, H, HKV, D = 1, 512, 8, 2, 128
    q = torch.zeros(B, S, H, D, device=DEV, dtype=torch.bfloat16)
    k = torch.zeros(B, S, HKV, D, device=DEV, dtype=torch.bfloat16)
    v = torch.zeros(B, S, HKV, D, device=DEV, dtype=torch.bfloat16)
    emb = tx.FastRoPEPositionEmbedding(D, max_position_embeddings=S, base=500000.0).to(DEV)
    cos, sin = emb(q, S)

    def fn():
        return triton_attn_func(q, k, v, causal=True, rotary_cos=cos, rotary_sin=sin)

    g, out = capture(fn)
    replay_and_check(g, out, [q, k, v], fn)


def test_graph_alibi_block_mask_with_blockmap_prepass():
    # the mask path launches the block-map pre-pass and then the attention
    # kernel; the mask itself is a static input too
    B, S, H, D = 2, 320, 4, 64
    q = torch.zeros(B, S, H, D, device=DEV, dtype=torch.float16)
    k = torch.zeros(B, S, H, D, device=DEV, dtype=torch.float16)
    v = torch.zeros(B, S, H, D, device=DEV, dtype=torch.float16)
    mask = torch.zeros(S, S, device=DEV)
    mask[64:128, 128:192] = float("-inf")
    mask[200:260, :40] = float("-inf")
    slopes = torch.tensor([2.0 ** (-2 * (h + 1)) for h in range(H)], device=DEV)

    def fn():
        return triton_attn_func(q, k, v, attn_mask=mask, alibi_slopes=slopes)

    g, out = capture(fn)
    replay_and_check(g, out, [q, k, v], fn)


def test_graph_decode_split_kv_with_lse():
    B, Sk, H, HKV, D = 2, 3000, 16, 4, 128
    q = torch.zeros(B, 1, H, D, device=DEV, dtype=torch.bfloat16)
    k = torch.zeros(B, Sk, HKV, D, device=DEV, dtype=torch.bfloat16)
    v = torch.zeros(B, Sk, HKV, D, device=DEV, dtype=torch.bfloat16)

    def fn():
        return triton_attn_func(q, k, v, return_lse=True)

    g, out = capture(fn)
    replay_and_check(g, out, [q, k, v], fn)


def test_graph_layer_decode_step_with_cache_rope_and_qk_norm():
    torch.manual_seed(5)
    E, H, HKV, P = 1024, 8, 2, 100
    layer = tx.FastGroupedQueryAttention(E, H, HKV, position_method="rope", rope_base=10000.0, qk_norm=True,
                                         max_seq_len=256).to(DEV, torch.bfloat16).eval()
    D = E // H
    past_k = torch.zeros(1, HKV, P, D, device=DEV, dtype=torch.bfloat16)
    past_v = torch.zeros(1, HKV, P, D, device=DEV, dtype=torch.bfloat16)
    x = torch.zeros(1, 1, E, device=DEV, dtype=torch.bfloat16)
    # the layer's RoPE table covers this step's tokens only (reference
    # rope.py:69-79 builds it for seq_len rows), so a one-token step uses row 0
    pos = torch.zeros((1, 1), device=DEV, dtype=torch.int64)

    def fn():
        with torch.no_grad():
            out, (kc, vc) = layer(x, position_ids=pos, past_key_value=(past_k, past_v), use_cache=True)
        return out, kc, vc

    g, outs = capture(fn)
    replay_and_check(g, outs, [x, past_k, past_v], fn)


def test_graph_forward_backward():
    """A training step's attention (forward and backward to q, k, v through
    the MFMA backward kernels) captured whole, as PyTorch's whole-network
    capture does: every replay's gradients equal an eager step's."""
    B, S, H, HKV, D = 1, 320, 4, 2, 128
    dt = torch.bfloat16
    q = torch.zeros(B, S, H, D, device=DEV, dtype=dt, requires_grad=True)
    k = torch.zeros(B, S, HKV, D, device=DEV, dtype=dt, requires_grad=True)
    v = torch.zeros(B, S, HKV, D, device=DEV, dtype=dt, requires_grad=True)
    dout = torch.zeros(B, S, H, D, device=DEV, dtype=dt)

    def fn():
        q.grad = k.grad = v.grad = None
        out = triton_attn_func(q, k, v, causal=True)
        out.backward(dout)
        return out.detach(), q.grad, k.grad, v.grad

    g, static = capture(fn)
    for rnd in range(3):
        gen = torch.Generator(device=DEV).manual_seed(2000 + rnd)
        with torch.no_grad():
            for t in (q, k, v, dout):
                t.copy_(torch.randn(t.shape, device=DEV, generator=gen).to(dt))
        torch.cuda.synchronize()
        g.replay()
        _ = torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)  # eager work between replays
        torch.cuda.synchronize()
        replayed = [t.clone() for t in static]
        ref = fn()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dq", "dk", "dv"), replayed, ref):
            assert torch.equal(a, b), f"replay {rnd}: {name} differs from eager"


def test_dropout_state_advance_through_the_abi():
    """trinix_dropout_state_advance copies the generator {seed, offset} to the
    call's state and advances the generator's offset, on the stream."""
    import ctypes

    from trinix_amd import _native as nat
    from trinix_amd.kernels.attention_kernel import current_stream_ptr

    lib = nat.load_library()
    gen = torch.tensor([(1 << 62) + 12345, (7 << 32) + 5], dtype=torch.int64, device=DEV)
    call = torch.full((2,), -1, dtype=torch.int64, device=DEV)
    st = current_stream_ptr(gen.device)
    for n in range(3):
        assert lib.trinix_dropout_state_advance(gen.data_ptr(), call.data_ptr(), ctypes.c_uint64(3), st) == 0
        torch.cuda.synchronize()
        assert call.tolist() == [(1 << 62) + 12345, (7 << 32) + 5 + 3 * n]
        assert gen.tolist() == [(1 << 62) + 12345, (7 << 32) + 5 + 3 * (n + 1)]
    assert lib.trinix_dropout_state_advance(None, call.data_ptr(), 1, st) == nat.TRINIX_ERR_NULL_POINTER
    assert lib.trinix_dropout_state_advance(gen.data_ptr() + 4, call.data_ptr(), 1, st) == nat.TRINIX_ERR_BAD_ARGUMENT


def _max_err_rule(h, e, t, small):
    scale = t.abs().max().item()
    err_h, err_e = (h - t).abs().max().item(), (e - t).abs().max().item()
    return err_h <= 2 * err_e + small * scale, (err_h, err_e, scale)


@pytest.mark.parametrize("dtype,D,kw", [(torch.bfloat16, 128, dict(causal=True)),
                                        (torch.float16, 64, dict(window_size=(40, 10))),
                                        (torch.float32, 64, dict(causal=True))])
def test_graph_training_step_with_dropout_draws_a_new_mask_per_replay(dtype, D, kw):
    """A captured forward + backward with attention dropout.  A kernel of the
    graph copies the device's dropout generator to the call's {seed, offset}
    and advances it, so each replay drops a different set of weights; each
    replay's output and gradients are those of eager autograd of the oracle
    through the keep mask of that replay's {seed, offset} (the fp64 answer
    within twice the eager error in the same dtype)."""
    from oracle import attention_oracle as orc
    import trinix_amd.kernels.attention_kernel as ak

    B, S, H, HKV, p = 1, 112, 4, 2, 0.25
    g0 = torch.Generator().manual_seed(91)
    q0, k0, v0 = (torch.randn(B, S, h, D, generator=g0) for h in (H, HKV, HKV))
    do0 = torch.randn(B, S, H, D, generator=g0)
    q, k, v = (t.to(DEV, dtype).requires_grad_(True) for t in (q0, k0, v0))
    do = do0.to(DEV, dtype)

    def step():
        q.grad = k.grad = v.grad = None
        out = triton_attn_func(q, k, v, dropout_p=p, **kw)
        out.backward(do)
        return out

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    q.grad = k.grad = v.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = triton_attn_func(q, k, v, dropout_p=p, **kw)
        out.backward(do)
    gen = ak._DROPOUT_GENERATORS[q.device]
    small = 1e-5 if dtype == torch.float32 else 2e-3
    keeps = []
    for rnd in range(3):
        seed, off = (int(x) for x in gen.tolist())
        graph.replay()
        _ = torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)  # eager work between replays
        torch.cuda.synchronize()
        assert int(gen.tolist()[1]) == off + 1
        keep = torch.from_numpy(orc.dropout_keep(B, H, S, S, p, seed, off))
        keeps.append(keep)
        res = {}
        for name, dt in (("truth", torch.float64), ("eager", dtype)):
            ts = [t.detach().to(dt).clone().requires_grad_(True) for t in (q0, k0, v0)]
            o = orc.functional_attention(*ts, keep=keep, dropout_p=p, **kw)
            o.backward(do0.to(dt))
            res[name] = [o.detach().double()] + [t.grad.double() for t in ts]
        hip = [out.detach().cpu().double()] + [t.grad.cpu().double() for t in (q, k, v)]
        for name, h, e, t in zip(("out", "dq", "dk", "dv"), hip, res["eager"], res["truth"]):
            ok, info = _max_err_rule(h, e, t, small)
            assert ok, (rnd, name, info)
    assert not torch.equal(keeps[0], keeps[1]) and not torch.equal(keeps[1], keeps[2])
