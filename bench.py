#!/usr/bin/env python3
"""Attention-forward benchmark on one MI355X.

Workload (default ``c3``): the Llama-3-8B-shaped GQA causal config of
BASELINE.json -- B=1, S=8192, 32 query / 8 KV heads, D=128, bf16, RoPE base
5e5 on q and k.  One "step" = one ``triton_attn_func`` call on resident
inputs with the RoPE fused (q rotated inside the attention kernel, k by the
RoPE pre-pass kernel).

Printed as ONE JSON line:
  value        algorithmic TFLOP/s of the whole step (4*D*allowed pairs;
               masked pairs not counted) / measured step time;
  roofline     for the attention kernel alone: algorithmic flops per launch
               / its mean launch time (HIP events on the launch stream),
               against the dense bf16 MFMA peak of MI355X (2.5 PFLOP/s);
  cpu_baseline the CPU oracle (restated reference eager path) on a bounded
               sample of the same workload, on this host's cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attn fwd TFLOP/s + % of MI355X bf16 MFMA peak (1 GPU); vs CPU ref ms"
PEAK_TFLOPS = {"bf16": 2516.6, "fp16": 2516.6, "fp32": 157.3}
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
DTYPE_NAME = {"torch.bfloat16": "bf16", "torch.float16": "fp16", "torch.float32": "fp32"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c3")
    ap.add_argument("--cpu-sample-heads", type=int, default=32,
                    help="query heads of batch 0 timed on the CPU oracle")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="time the workload only: no MALL-flushed, forward+backward, decode or layer fields "
                         "(for profiler runs)")
    ap.add_argument("--all", action="store_true", help="also time every other workload (extra field)")
    ap.add_argument("--backward", action="store_true",
                    help="time forward + backward steps of the workload (its mask, ALiBi, window and RoPE "
                         "included) instead of the forward; with --counters, only W + K such steps")
    ap.add_argument("--counters", action="store_true",
                    help="for counter-collection profiler runs: W warm-up and K timed steps only (no clock "
                         "warm-up, no kernel timing blocks); prints the step time only")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (scale factor of the HBM byte counters)")
    return ap.parse_args()


def traffic_from_profile(workload):
    """HBM bytes per launch of the attention kernel, measured offline with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by a plain copy's
    counters) and recorded in profiles/attn_fwd_<workload>_traffic.txt."""
    path = os.path.join(ROOT, "profiles", f"attn_fwd_{workload}_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def calibrate_copy(torch):
    n = 256 * 1024 * 1024 // 2
    x = torch.ones(n, dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read_per_launch": n * 2, "copy_bytes_written_per_launch": n * 2}), flush=True)


def step_fn(w, inp, torch):
    from trinix_amd import triton_attn_func

    kw = dict(causal=w.causal)
    if w.window is not None:
        kw["window_size"] = w.window
    if inp.mask is not None:
        kw["attn_mask"] = inp.mask
    if inp.alibi is not None:
        kw["alibi_slopes"] = inp.alibi
    if inp.cos is not None:
        kw["rotary_cos"], kw["rotary_sin"] = inp.cos, inp.sin
    k, v = inp.k, inp.v
    if w.nheads_kv == 1:  # MQA: one KV head, expanded with stride 0 as the reference layer does
        k = k.expand(-1, -1, w.nheads, -1)
        v = v.expand(-1, -1, w.nheads, -1)
    return lambda: triton_attn_func(inp.q, k, v, **kw)


def kernel_only_fn(w, inp, torch):
    """The attention kernel alone: k pre-rotated once, q rotated in-kernel."""
    from trinix_amd.kernels import TritonAttentionKernel, rope_apply

    k, v = inp.k, inp.v
    kw = dict(causal=w.causal, window_size=w.window, attn_mask=inp.mask, alibi_slopes=inp.alibi)
    if inp.cos is not None:
        k = rope_apply(inp.k, inp.cos, inp.sin)
        kw.update(rotary_cos=inp.cos, rotary_sin=inp.sin, rotary_k=False)
    if w.nheads_kv == 1:
        k = k.expand(-1, -1, w.nheads, -1)
        v = v.expand(-1, -1, w.nheads, -1)
    return lambda: TritonAttentionKernel.apply(inp.q, k, v, **kw)


def time_events(fn, iters, torch):
    """Mean ms per call from HIP events on the current (launch) stream."""
    st = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(st)
    for _ in range(iters):
        fn()
    end.record(st)
    end.synchronize()
    return start.elapsed_time(end) / iters


def gpu_block_ms(fn, n, torch):
    """GPU ms per call of ``n`` back-to-back eager calls of ``fn``: HIP events
    on the launch stream (the stream every call launches on) before the
    first and after the last call.  The host enqueues faster than the GPU
    runs these kernels (the launch cache keeps a call at a few microseconds
    of host time), so the interval is GPU time."""
    st = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(st)
    for _ in range(n):
        fn()
    end.record(st)
    end.synchronize()
    return start.elapsed_time(end) / n


def interleaved_ms(step, kernel, per_call_s, torch, rounds=5, block_s=0.02):
    """(GPU ms per step, GPU ms per kernel-only call) from ``rounds``
    alternating blocks of back-to-back steps and kernel-only calls, each
    about ``block_s`` of GPU time, so both run in the same regime (eager
    launches, the output buffer reused by the allocator, the same clock
    state).  Medians over the rounds."""
    n = max(10, int(block_s / max(per_call_s, 1e-6)))
    steps, kern = [], []
    for _ in range(rounds):
        steps.append(gpu_block_ms(step, n, torch))
        kern.append(gpu_block_ms(kernel, n, torch))
    med = lambda xs: sorted(xs)[len(xs) // 2]
    return med(steps), med(kern), n


def cold_step_ms(fn, torch, iters=10):
    """Median ms of one step with the 256 MB MALL flushed first: a 512 MiB
    scratch buffer is written (untimed) before each step, and only the step
    is timed with HIP events on the launch stream."""
    scratch = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    times = []
    for _ in range(iters):
        scratch.fill_(1)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(st)
        fn()
        end.record(st)
        end.synchronize()
        times.append(start.elapsed_time(end))
    del scratch
    return sorted(times)[len(times) // 2]


def fwd_bwd_step(w, inp, torch, dropout_p=0.0):
    """One differentiable step on the workload: forward (with the workload's
    RoPE, window, ALiBi and mask) and backward to q, k, v through the HIP
    kernels, with attention dropout ``dropout_p``."""
    from trinix_amd import triton_attn_func

    q, k, v = (t.detach().clone().requires_grad_(True) for t in (inp.q, inp.k, inp.v))
    do = torch.randn_like(inp.q)
    kw = dict(causal=w.causal, window_size=w.window, dropout_p=dropout_p)
    if inp.cos is not None:
        kw.update(rotary_cos=inp.cos, rotary_sin=inp.sin)
    if inp.mask is not None:
        kw["attn_mask"] = inp.mask
    if inp.alibi is not None:
        kw["alibi_slopes"] = inp.alibi

    def step():
        # gradients start from None each step, as after optimizer.zero_grad()
        # (set_to_none=True, its default): no accumulation kernels are timed
        q.grad = k.grad = v.grad = None
        kk, vv = k, v
        if w.nheads_kv == 1:  # MQA: the layer's stride-0 expand
            kk, vv = k.expand(-1, -1, w.nheads, -1), v.expand(-1, -1, w.nheads, -1)
        triton_attn_func(q, kk, vv, **kw).backward(do)

    return step


def fwd_bwd_ms(w, inp, torch, iters=10, dropout_p=0.0, reps=3):
    """ms of one forward + backward step (fwd_bwd_step), host-timed over
    `iters` steps bracketed by synchronisations, median of `reps` such loops,
    after about 0.3 s of warm-up steps (the first loop after a short warm-up
    read up to 8% slow: clock ramp)."""
    step = fwd_bwd_step(w, inp, torch, dropout_p)
    t_warm, n = time.perf_counter(), 0
    while n < 3 or time.perf_counter() - t_warm < 0.3:
        step()
        n += 1
        torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for _ in range(iters):
            step()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3 / iters)
    return sorted(times)[len(times) // 2]


def measure(w, args, torch, cold=False, min_timed_s=0.0, strict=True):
    """(inputs, flop, step ms, kernel ms, cold-MALL ms, steps timed, GPU ms
    of a step, calls per interleaved block).
    The step loop times ``args.steps`` steps, or more when ``min_timed_s``
    asks for a longer timed region (the extra workloads of ``--all``: at
    C2's 16 us per step, 20 steps would be mostly the final synchronize)."""
    from trinix_amd.workloads import make_inputs, flops

    inp = make_inputs(w, device="cuda")
    fn = step_fn(w, inp, torch)
    # W warm-up steps, extended until the GPU has been busy for ~0.3 s so the
    # timed region runs at the steady-state clock (untimed).
    t_warm = time.perf_counter()
    n = 0
    while n < args.warmup or time.perf_counter() - t_warm < 0.3:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    steps = args.steps
    if min_timed_s > 0.0:
        per_step_s = (time.perf_counter() - t_warm) / n
        steps = max(steps, int(min_timed_s / per_step_s) + 1)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    fl = flops(w)
    # the attention kernel alone (k rotated once ahead), event-timed in
    # blocks that alternate with blocks of whole steps
    kfn = kernel_only_fn(w, inp, torch)
    ref = fn()
    if not torch.equal(kfn(), ref):
        raise RuntimeError("kernel-only call output differs from the step's")
    per_call_s = ms * 1e-3
    step_gpu, kms, n = interleaved_ms(fn, kfn, per_call_s, torch)
    if strict and (kms > ms or kms > step_gpu * 1.005):
        # a kernel-only call cannot take longer than a step holding the same
        # kernel: measure once more, then refuse to report
        step_gpu, kms, n = interleaved_ms(fn, kfn, per_call_s, torch)
        if kms > ms or kms > step_gpu * 1.005:
            raise SystemExit(f"inconsistent timing: kernel {kms:.4f} ms > step {ms:.4f} ms "
                             f"(GPU time of a step {step_gpu:.4f} ms)")
    cold_ms = cold_step_ms(fn, torch) if cold else None
    return inp, fl, ms, kms, cold_ms, steps, step_gpu, n


DECODE = dict(batch=16, seqlen_k=8192, nheads_q=32, nheads_kv=8, head_dim=128)


def decode_measure(torch, iters=30):
    """One decode step of the C3 model (Llama-3-8B GQA, bf16) against a KV
    cache: B=16 sequences, 1 query row each, 8192 cached keys.  The split-KV
    kernel and its merge are HBM-bound: the algorithmic bytes are the K and V
    caches read once (q and out are 0.1% of it).  Timed with HIP events on
    the launch stream over back-to-back calls (the GPU, not the host, is the
    bottleneck at this size)."""
    import ctypes
    from trinix_amd import triton_attn_func
    from trinix_amd import _native as nat

    c = DECODE
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(c["batch"], 1, c["nheads_q"], c["head_dim"], device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(c["batch"], c["seqlen_k"], c["nheads_kv"], c["head_dim"], device="cuda",
                    generator=g).to(torch.bfloat16)
    v = torch.randn_like(k)
    for _ in range(5):
        triton_attn_func(q, k, v)
    us = time_events(lambda: triton_attn_func(q, k, v), iters, torch) * 1e3
    kv_bytes = 2 * k.numel() * k.element_size()
    a = nat.AttnFwdArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), q.data_ptr()
    a.q_stride, a.k_stride = nat.int64x4(q.stride()), nat.int64x4(k.stride())
    a.v_stride, a.out_stride = nat.int64x4(v.stride()), nat.int64x4(q.stride())
    a.batch, a.seqlen_q, a.seqlen_k = c["batch"], 1, c["seqlen_k"]
    a.nheads_q, a.nheads_kv, a.head_dim, a.dtype = c["nheads_q"], c["nheads_kv"], c["head_dim"], nat.TRINIX_BF16
    ns, wb = ctypes.c_int32(), ctypes.c_int64()
    nat.check(nat.load_library().trinix_attn_fwd_splitkv_plan(ctypes.byref(a), ctypes.byref(ns), ctypes.byref(wb)),
              "plan")
    gbps = kv_bytes / (us * 1e-6) / 1e9
    # practical ceiling on this box: torch's device copy of the same bytes
    src = torch.cat([k.view(-1), v.view(-1)])
    dst = torch.empty_like(src)
    dst.copy_(src)
    cus = time_events(lambda: dst.copy_(src), 10, torch) * 1e3
    del src, dst
    return {"config": "Llama-3-8B decode step: B=16, seqlen_q=1, seqlen_k=8192, 32 q / 8 kv heads, D=128, bf16",
            "kernels": "attn_decode16 + attn_decode_combine", "num_splits": ns.value,
            "us_per_step": round(us, 2), "kv_bytes": kv_bytes, "achieved_gbps": round(gbps, 1),
            "peak_gbps": PEAK_HBM_GBPS, "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "copy_gbps_same_box": round(2 * kv_bytes / (cus * 1e-6) / 1e9, 1)}


def layer_measure(torch, iters=10):
    """The C3 model's attention layer forward (Llama-3-8B GQA: E=4096, 32 q /
    8 kv heads, RoPE 5e5, causal, qk_norm=True, B=1, S=8192, bf16, inference)
    three ways: q's RoPE + RMSNorm in the attention prologue and k's in the
    fused RoPE + qk RMSNorm kernel (the default); both through that kernel;
    the eager norm modules.  Plus that kernel alone on q (algorithmic bytes:
    q read and written once) and its backward on q (x and dout read, dx
    written), and a training step (forward + backward) of the layer with
    the fused and with the eager qk-norm.  The projections are torch Linear
    layers (hipBLASLt GEMMs)."""
    import trinix_amd as tx
    from trinix_amd.kernels import qk_rmsnorm

    B, S, H, HKV, D = 1, 8192, 32, 8, 128
    res = {"config": "GQA layer forward, E=4096, 32 q / 8 kv heads, D=128, B=1, S=8192, RoPE 5e5, causal, "
                     "qk_norm (RMSNorm), bf16, no grad"}
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(B, S, H * D, device="cuda", generator=g).to(torch.bfloat16)
    for mode in ("us_fused_qk_norm", "us_fused_qk_norm_q_separate", "us_eager_qk_norm"):
        fused = mode != "us_eager_qk_norm"
        layer = tx.FastGroupedQueryAttention(H * D, H, HKV, causal=True, position_method="rope", rope_base=500000.0,
                                             qk_norm=True, max_seq_len=S).to("cuda", torch.bfloat16)
        if not fused:
            layer._fused_qk_norm_applies = lambda q, k: False
        layer.fuse_q_norm_in_attention = mode == "us_fused_qk_norm"
        with torch.no_grad():
            for _ in range(3):
                layer(x)
            res[mode] = round(time_events(lambda: layer(x), iters, torch) * 1e3, 1)
        if mode == "us_fused_qk_norm":
            q = torch.randn(B, S, H, D, device="cuda", generator=g).to(torch.bfloat16)
            cos, sin = layer.position_embedding(q, S)
            w = layer.q_norm.weight.detach()
            with torch.no_grad():
                qk_rmsnorm(q, w, 1e-6, cos, sin)
                us = time_events(lambda: qk_rmsnorm(q, w, 1e-6, cos, sin), 20, torch) * 1e3
            res["qk_norm_kernel_q_us"] = round(us, 2)
            res["qk_norm_kernel_q_gbps"] = round(2 * q.numel() * 2 / (us * 1e-6) / 1e9, 1)
            # its backward on q (dx, and dweight from the per-workgroup
            # partial rows): x and dout read, dx written once
            from trinix_amd.kernels.qk_norm_kernel import NORM_RMS, _backward, _tables

            dout = torch.randn_like(q)
            c, s_, _ = _tables(q, cos, sin, None)
            _backward(q, dout, w, 1e-6, c, s_, None, NORM_RMS)
            us = time_events(lambda: _backward(q, dout, w, 1e-6, c, s_, None, NORM_RMS), 20, torch) * 1e3
            res["qk_norm_bwd_q_us"] = round(us, 2)
            res["qk_norm_bwd_q_gbps"] = round(3 * q.numel() * 2 / (us * 1e-6) / 1e9, 1)
        del layer
    # a training step of the layer (forward + backward to x and the
    # parameters): qk-norm through the fused kernels against the eager modules
    for mode in ("us_train_step_fused_qk_norm", "us_train_step_eager_qk_norm"):
        layer = tx.FastGroupedQueryAttention(H * D, H, HKV, causal=True, position_method="rope", rope_base=500000.0,
                                             qk_norm=True, max_seq_len=S).to("cuda", torch.bfloat16)
        if mode == "us_train_step_eager_qk_norm":
            layer._fused_qk_norm_applies = lambda q, k: False
        xg = x.detach().clone().requires_grad_(True)
        gy = torch.randn_like(x)

        def step():
            xg.grad = None
            for prm in layer.parameters():
                prm.grad = None
            layer(xg)[0].backward(gy)

        for _ in range(2):
            step()
        res[mode] = round(time_events(step, 5, torch) * 1e3, 1)
        del layer
    return res


def algo_bytes(w):
    """Minimum HBM bytes of one launch: q, k, v read once, out written once
    (+ the mask read once)."""
    esz = 4 if str(w.dtype) == "torch.float32" else 2
    n = (2 * w.batch * w.seqlen * w.nheads + 2 * w.batch * w.seqlen * w.nheads_kv) * w.head_dim * esz
    if w.block_mask:
        n += w.seqlen * w.seqlen * 4
    return n


def cpu_baseline(w, nheads, torch):
    """Oracle (restated reference eager path) on `nheads` query heads of
    batch 0, RoPE applied outside the timed region; 1 warm-up + median of 3
    (1 run if the sample takes > 20 s)."""
    from oracle.attention_oracle import apply_rope, functional_attention
    from trinix_amd.workloads import make_inputs, flops

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    inp = make_inputs(w)
    q, k = inp.q, inp.k
    if inp.cos is not None:
        q, k = apply_rope(q, inp.cos, inp.sin), apply_rope(k, inp.cos, inp.sin)
    heads = list(range(min(nheads, w.nheads)))
    kw = dict(attn_mask=inp.mask, causal=w.causal, window_size=w.window, alibi_slopes=inp.alibi,
              heads=heads, batches=[0])
    t0 = time.perf_counter()
    functional_attention(q, k, inp.v, **kw)
    first = time.perf_counter() - t0
    times = [first]
    if first < 20:
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            functional_attention(q, k, inp.v, **kw)
            times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    fl = flops(w, heads=heads, batches=[0])
    full_ms = t * 1e3 * (w.batch * w.nheads) / len(heads)
    return {
        "value": round(fl / t / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{len(heads)} of {w.batch * w.nheads} (batch, q-head) slices of {w.name}, "
                  f"eager bmm/softmax path in {DTYPE_NAME[str(w.dtype)]}, median of {len(times)}",
        "sample_ms": round(t * 1e3, 2),
        "full_config_ms_extrapolated": round(full_ms, 1),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); "
              "this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    from trinix_amd.workloads import WORKLOADS
    from trinix_amd import _native

    w = WORKLOADS[args.workload]
    dname = DTYPE_NAME[str(w.dtype)]
    if args.backward and not args.counters:
        from trinix_amd.workloads import make_inputs, flops
        inp = make_inputs(w, device="cuda")
        fb = fwd_bwd_ms(w, inp, torch, iters=max(args.steps, 10))
        fl = flops(w)
        print(json.dumps({"metric": "attn fwd+bwd TFLOP/s (3.5x the forward's algorithmic flop)", "workload": w.name,
                          "dtype": dname, "ms_per_step": round(fb, 4), "tflops": round(3.5 * fl / fb / 1e9, 2),
                          "steps": max(args.steps, 10)}), flush=True)
        return
    if args.counters:
        # each dispatch is serialised and its counters read out: keep the
        # run to a handful of dispatches of the step's kernels
        from trinix_amd.workloads import make_inputs
        inp = make_inputs(w, device="cuda")
        fn = fwd_bwd_step(w, inp, torch) if args.backward else step_fn(w, inp, torch)
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        print(json.dumps({"workload": w.name, "counters_run": True,
                          "ms_per_step": round((time.perf_counter() - t0) * 1e3 / args.steps, 4)}), flush=True)
        return
    inp, fl, ms, kms, cold_ms, _, step_gpu, nblk = measure(w, args, torch, cold=not args.no_extra)
    value = fl / (ms * 1e-3) / 1e12
    k_tflops = fl / (kms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[dname]
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic (seeded N(0,1) q/k/v)",
        "config": {
            "workload": f"{w.name}: {w.description}",
            "batch": w.batch, "seq_len": w.seqlen, "nheads_q": w.nheads, "nheads_kv": w.nheads_kv,
            "head_dim": w.head_dim, "causal": w.causal, "window": w.window, "rope_base": w.rope_base,
            "alibi": w.alibi, "block_mask": w.block_mask, "fused_rope": w.rope_base is not None,
            "algorithmic_flop": fl, "parallelism": "single GPU",
        },
        "pct_of_peak": round(100 * value / peak, 2),
        "roofline": {
            "bound": "mfma",
            # with a block mask the timed sequence is the block-map pre-pass
            # and the attention kernel (both in the rocprof summary)
            "kernel": ("blockmap_kernel + " if w.block_mask else "")
                      + ("attn_fwd_mfma16" if dname != "fp32" else "attn_fwd_f32"),
            "achieved": round(k_tflops, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(k_tflops / peak, 4),
            "kernel_ms": round(kms, 4),
            "kernel_timing": f"HIP events on the launch stream over blocks of {nblk} back-to-back eager "
                             f"kernel-only calls (k rotated ahead), alternating with blocks of whole steps; "
                             f"median of 5 blocks",
            "step_gpu_ms": round(step_gpu, 4),
            "traffic": traffic_from_profile(w.name),
            "traffic_unit": "bytes/launch",
            "algorithmic_bytes": algo_bytes(w),
        },
        "native_library": str(_native.LIB_PATH) if _native.library_loaded() else None,
    }
    if cold_ms is not None:
        # the same step with q/k/v evicted from the 256 MB MALL before each call
        rec["cold_mall"] = {"ms_per_step": round(cold_ms, 4), "tflops": round(fl / cold_ms / 1e9, 2)}
    if dname in ("bf16", "fp16") and not w.alibi and not w.block_mask and not args.no_extra:
        # forward + backward (3.5x the forward FLOP by the usual convention)
        fb = fwd_bwd_ms(w, inp, torch)
        rec["fwd_bwd"] = {"ms": round(fb, 4), "tflops": round(3.5 * fl / fb / 1e9, 2),
                          "bwd_ms": round(fb - ms, 4), "bwd_tflops": round(2.5 * fl / (fb - ms) / 1e9, 2)}
        # the same step with attention dropout 0.1 (keep masks regenerated
        # from the forward's Philox stream in both backward kernels)
        fbd = fwd_bwd_ms(w, inp, torch, dropout_p=0.1)
        rec["fwd_bwd_dropout"] = {"p": 0.1, "ms": round(fbd, 4), "tflops": round(3.5 * fl / fbd / 1e9, 2)}
    if dname in ("bf16", "fp16") and not args.no_extra:
        del inp
        torch.cuda.empty_cache()
        rec["decode"] = decode_measure(torch)
        torch.cuda.empty_cache()
        rec["layer"] = layer_measure(torch)
        torch.cuda.empty_cache()
        inp = None
    if args.all:
        extra = {}
        for name, wo in WORKLOADS.items():
            if name == w.name:
                continue
            # not strict: where a step is the kernel alone (no pre-pass), the
            # two figures are the same work and differ by the noise only
            _, f2, ms2, kms2, _, n2, sg2, _ = measure(wo, args, torch, min_timed_s=0.05, strict=False)
            pk = PEAK_TFLOPS[DTYPE_NAME[str(wo.dtype)]]
            extra[name] = {"ms": round(ms2, 4), "steps": n2, "step_gpu_ms": round(sg2, 4),
                           "tflops": round(f2 / ms2 / 1e9, 2),
                           "kernel_ms": round(kms2, 4), "kernel_tflops": round(f2 / kms2 / 1e9, 2),
                           "pct_of_peak": round(100 * f2 / ms2 / 1e9 / pk, 2),
                           "kernel_pct_of_peak": round(100 * f2 / kms2 / 1e9 / pk, 2)}
            torch.cuda.empty_cache()
        rec["other_workloads"] = extra
    if not args.no_cpu:
        inp = None
        torch.cuda.empty_cache()
        rec["cpu_baseline"] = cpu_baseline(w, args.cpu_sample_heads, torch)
        rec["speedup_vs_cpu_full_config"] = round(rec["cpu_baseline"]["full_config_ms_extrapolated"] / ms, 1)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
