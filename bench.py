"""Benchmark of the GLA inference path on one MI355X.

Headline (BASELINE.json metric): GLA prefill tokens/s at B=4, H=6, T=16384, Dk=Dv=64, bf16 I/O,
fp32 state (config 1), with the batched decode step at B=256 (config 2) reported alongside.

  step (prefill) = one fast_chunk_gla forward over the whole [4, 16384, 6, 64] batch, inputs
                   resident in HBM (two input sets used in turn, together larger than the 256 MB
                   MALL), bf16 outputs and fp32 final states written to HBM (three kernels; the
                   timed passes are one HIP-graph replay, the same passes as direct calls are
                   reported beside it).
  step (decode)  = one decode step for 256 sequences (H=6, D=64) on one of 12 rotating fp32
                   state buffers (302 MB in total, larger than the 256 MB MALL) with one of 12
                   rotating q/k/v/g/o sets; the 512-step loop is captured in a HIP graph and
                   replayed.  Also reported: the same loop with fresh inputs every step.

Prints ONE JSON line.  Roofline: HBM-bound (algorithmic bytes per pass / measured pass time vs
8 TB/s); MFMA fraction = algorithmic flops / time / 2.5 PFLOP/s (dense bf16).
cpu_baseline: the CPU restatement of the reference's PyTorch scan (oracle/ref_port.py) on a
bounded sample of the same workload, on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

from triune_amd._lib import check, lib

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "GLA prefill tok/s @B4 H6 T16k D64 (MFMA %); decode tok/s @B256 (HBM GB/s %)"


def _progress(msg):
    """One progress line on stderr as each leg ends (the JSON line stays the only stdout line)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def _events_time_ms(fn, iters, stream):
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def prefill_inputs(dev):
    """Config-1 inputs in HBM: two input sets used in turn (the second is the first rolled by one
    token), so 2 x 201 MB of q/k/v/g exceeds the 256 MB MALL and every pass reads its inputs from
    HBM; the initial state; an output buffer per set."""
    from triune_amd.workloads import config1

    q, k, v, g, s0 = config1(T=16384, B=4, H=6, D=64)
    sets = [[x.to(dev) for x in (q, k, v, g)], [x.roll(1, dims=1).to(dev) for x in (q, k, v, g)]]
    outs = [torch.empty_like(v, device=dev) for _ in sets]
    torch.cuda.synchronize()
    return sets, s0.to(dev), outs


def prefill_graph(steps, dev, inputs):
    """The headline's timed passes as one HIP graph: `steps` config-1 passes (the two input sets
    in turn), captured after one call outside the capture (library load, workspace sizes).  main()
    captures it before the secondary legs, so that nothing but the warm-up passes runs between the
    last leg's GPU work and the timed replay: the GPU's clocks drop within tens of milliseconds of
    idling (capture is host work), and after such a gap the replay read 125-132 us/pass against
    113-115 us/pass with the GPU kept busy."""
    from triune_amd import fast_chunk_gla

    sets, s0, outs = inputs
    turn = [0]

    def fn():
        i = turn[0] & 1
        turn[0] += 1
        fast_chunk_gla(*sets[i], initial_state=s0, out=outs[i])

    # The timed passes are one replay of the graph, not `steps` Python calls: host-side launch
    # jitter (a stalled Python loop left the GPU idle for a third of one 20-pass measurement) stays
    # out of the timed region, and the replay follows the warm-up passes with no idle gap.
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        fn()  # first call outside the capture (library load, workspace sizes)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            fn()
    torch.cuda.synchronize()
    return graph, fn


def bench_prefill(steps, warmup, dev, inputs=None, captured=None):
    from triune_amd.workloads import gla_algorithmic_bytes, gla_algorithmic_flops

    B, T, H, D = 4, 16384, 6, 64
    if inputs is None:
        inputs = prefill_inputs(dev)
    graph, fn = captured if captured is not None else prefill_graph(steps, dev, inputs)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = _events_time_ms(graph.replay, 1, stream) / steps
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the same passes as direct calls (host work plus three launches each), for reference
    eager_ms = _events_time_ms(fn, steps, stream)
    L = lib()
    # The roofline's kernel time, in a second loop of as many passes: one event pair per pass that
    # the library attaches to the output kernel's dispatch (the dominant of the pass's three
    # kernels).  HIP events include the dispatch latency, about 4 us per launch on MI355X, which
    # rocprofv3's kernel trace leaves out of a kernel's duration.
    k3 = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for b, e in k3:  # torch creates an event on its first record
        b.record(stream)
        e.record(stream)
    torch.cuda.synchronize()
    try:
        for b, e in k3:
            check(L.triune_hip_set_output_kernel_events(b._as_parameter_, e._as_parameter_), "arm events")
            fn()
    finally:
        L.triune_hip_set_output_kernel_events(None, None)
    torch.cuda.synchronize()
    k3_ms = sum(b.elapsed_time(e) for b, e in k3) / steps
    n_th = B * T * H
    k3_bytes = gla_algorithmic_bytes(n_th, D, D, 2, 2, 2)  # q, k, g, v read and o written once
    alg_bytes = k3_bytes + 2 * B * H * D * D * 4  # the pass also reads S0 and writes the final S
    alg_flops = gla_algorithmic_flops(n_th, D, D)
    return {
        "ms": ms,
        "eager_ms": eager_ms,
        "wall_s": wall,
        "tok_s": B * T / (ms * 1e-3),
        "alg_bytes": alg_bytes,
        "alg_flops": alg_flops,
        "gbs": alg_bytes / (ms * 1e-3) / 1e9,
        "tflops": alg_flops / (ms * 1e-3) / 1e12,
        "k3_ms": k3_ms,
        "k3_bytes": k3_bytes,
        "k3_gbs": k3_bytes / (k3_ms * 1e-3) / 1e9,
    }


def bench_decode(steps_total, dev, n_bufs=12):
    from triune_amd import gla_decode_step
    from triune_amd.workloads import config2

    B, H, D = 256, 6, 64
    q, k, v, g, s0 = config2(steps=steps_total, B=B, H=H, D=D)
    q, k, v, g = (x.to(dev) for x in (q, k, v, g))
    states = [s0.to(dev).clone() for _ in range(n_bufs)]
    outs = torch.empty(steps_total, B, 1, H, D, device=dev, dtype=torch.bfloat16)

    # Step t updates state buffer t % n_bufs.  Its q/k/v/g/o come from input set t % n_bufs (as in
    # a model, where the projection that feeds the step rewrites the same buffers every token);
    # the "cold" loop instead takes a fresh slice of [steps, ...] tensors every step, so the small
    # inputs also miss every cache and TLB.
    def loop(cold=False):
        for t in range(steps_total):
            i = t if cold else t % n_bufs
            gla_decode_step(q[i], k[i], v[i], g[i], states[t % n_bufs], inplace=True, out=outs[i])

    # A reference for the state traffic: torch's device copy moving the same bytes per step (one
    # state read, one written) over the same rotating buffers (run after the decode loops).
    def copy_loop(cold=False):
        for t in range(steps_total):
            states[(t - 1) % n_bufs].copy_(states[t % n_bufs])

    def graphed(cold, body=loop):
        # warm up on a side stream, then capture the whole loop in one graph
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            body(cold)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            body(cold)
        graph.replay()
        torch.cuda.synchronize()
        return graph

    stream = torch.cuda.current_stream()
    reps = 3
    ms_loop = _events_time_ms(graphed(False).replay, reps, stream)
    ms_cold = _events_time_ms(graphed(True).replay, reps, stream)
    eager_ms = _events_time_ms(loop, 1, stream)
    ms_copy = _events_time_ms(graphed(False, copy_loop).replay, reps, stream)
    step_us = ms_loop * 1e3 / steps_total
    state_bytes = B * H * D * D * 4
    step_bytes = 2 * state_bytes + B * H * D * 2 * 4 + B * H * D * 2  # state r+w; q,k,v,g read; o write
    copy_us = ms_copy * 1e3 / steps_total
    return {
        "step_us": step_us,
        "eager_step_us": eager_ms * 1e3 / steps_total,
        "cold_step_us": ms_cold * 1e3 / steps_total,
        "copy_step_us": copy_us,
        "copy_gbs": 2 * state_bytes / (copy_us * 1e-6) / 1e9,
        "tok_s": B / (step_us * 1e-6),
        "step_bytes": step_bytes,
        "gbs": step_bytes / (step_us * 1e-6) / 1e9,
        "state_buffers": n_bufs,
    }


def bench_gdn_decode(dev, steps=512, n_bufs=12):
    """Gated DeltaNet decode step (T == 1) at config 2's batch shape (B=256, H=6, D=64), beta per
    head, bf16 q/k/v/g/o, fp32 state, through the C-ABI entry the operator calls
    (triune_hip_gdn_prefill, which runs the decode kernel for T == 1).  `steps` steps in one HIP
    graph; step t reads state buffer t % n_bufs and writes buffer (t - 1) % n_bufs, which is read
    again n_bufs - 1 steps later (12 x 25 MB: more than the 256 MB MALL between a write and its
    read), and takes input set t % n_bufs."""
    from triune_amd._lib import check, dtype_code, lib, ptr, stream_of, strides

    B, H, D = 256, 6, 64
    gen = torch.Generator(device=dev).manual_seed(6)
    nq = lambda: torch.nn.functional.normalize(torch.randn(n_bufs, B, 1, H, D, device=dev, generator=gen), dim=-1)  # noqa: E731
    q, k = nq().bfloat16(), nq().bfloat16()
    v = torch.randn(n_bufs, B, 1, H, D, device=dev, generator=gen).bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(n_bufs, B, 1, H, D, device=dev, generator=gen)).bfloat16()
    beta = torch.sigmoid(torch.randn(n_bufs, B, 1, H, device=dev, generator=gen))
    states = [0.1 * torch.randn(B, H, D, D, device=dev, generator=gen) for _ in range(n_bufs)]
    outs = torch.empty(n_bufs, B, 1, H, D, device=dev, dtype=torch.bfloat16)
    tok3 = lambda x: (x.stride(0), x.stride(1), x.stride(2))  # noqa: E731
    st = strides(tok3(q[0]), tok3(k[0]), tok3(v[0]), tok3(g[0]), tok3(beta[0]), tok3(outs[0]))
    lb = lib()

    def loop():
        for t in range(steps):
            i = t % n_bufs
            rc = lb.triune_hip_gdn_prefill(ptr(q[i]), ptr(k[i]), ptr(v[i]), ptr(g[i]), dtype_code(q), dtype_code(g),
                                           ptr(beta[i]), dtype_code(beta), 1, st, ptr(states[i]), ptr(outs[i]),
                                           dtype_code(outs), ptr(states[(t - 1) % n_bufs]), B, 1, H, D, D,
                                           stream_of(q))
            check(rc, "triune_hip_gdn_prefill")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        loop()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loop()
    graph.replay()
    torch.cuda.synchronize()
    ms = _events_time_ms(graph.replay, 5, torch.cuda.current_stream())
    step_us = ms * 1e3 / steps
    # state read + written (fp32); q, k, v, g read and o written (bf16); beta read (fp32)
    step_bytes = 2 * B * H * D * D * 4 + B * H * D * 2 * 5 + B * H * 4
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    return {"workload": "Gated DeltaNet decode step (T == 1), config-2 shape (B=256, H=6, D=64), beta per head, "
                        f"{steps}-step graph, {n_bufs} rotating state buffers and input sets",
            "us_per_step": round(step_us, 3), "tok_s": round(B / (step_us * 1e-6), 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes_per_step": step_bytes}}


def bench_prep(dev, reps=10):
    """In-place GLA input pre-processing (ELU+1, L2 norm, RoPE on q and k; logsigmoid on g) at the
    config-1 shape: qkv [4, 16384, 3, 6, 64] and g [4, 16384, 6, 64] bf16, fp32 RoPE tables."""
    from triune_amd import fused_qkv_g_prep_inplace

    B, T, H, HD = 4, 16384, 6, 64
    gen = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, T, 3, H, HD, generator=gen).bfloat16().to(dev)
    g = torch.randn(B, T, H, HD, generator=gen).bfloat16().to(dev)
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    emb = torch.cat([torch.outer(torch.arange(T, dtype=torch.float32), inv)] * 2, dim=-1)
    cos, sin = emb.cos().to(dev), emb.sin().to(dev)
    fn = lambda: fused_qkv_g_prep_inplace(qkv, g, cos, sin)  # noqa: E731
    for _ in range(20):
        fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    alg = 6 * B * T * H * HD * 2  # q, k, g read and written once (v untouched)
    return {"workload": "VectorisedGLA pre-processing in place, config-1 shape (B=4, T=16384, H=6, HD=64, bf16, RoPE)",
            "us": round(ms * 1e3, 2), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "roofline": {"bound": "hbm", "achieved": round(alg / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def _graph_us_per_call(calls, restore=None, reps=5):
    """GPU time per call of `calls` (zero-argument callables) run back to back: they are captured
    in one HIP graph on a side stream (after a warm-up there), and the replay is timed with events;
    `restore` (not timed) runs before each replay, e.g. to give in-place operations their raw inputs
    back.  Median over `reps` replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        if restore:
            restore()
        for f in calls:
            f()
        if restore:
            restore()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for f in calls:
                f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps + 2):
        if restore:
            restore()
            torch.cuda.synchronize()
        b, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        b.record()
        graph.replay()
        e.record()
        e.synchronize()
        times.append(b.elapsed_time(e))
    times = sorted(times[2:])
    return times[len(times) // 2] * 1e3 / len(calls)


def bench_fused_prefill(dev, reps=20, T=16384):
    """VectorisedGLA's prefill from raw projections (qkv [4, T, 3, 6, 64] and gate logits
    g [4, T, 6, 64] bf16, fp32 RoPE tables, fp32 S0; T = 1024 is the tile VectorisedGLA runs every
    prefill in, attention.py:458-499): fused_qkv_g_prep_chunk_gla as dispatched (one launch where
    the call fits the single-launch prefill, as at T = 1024; otherwise the prep pass and then the
    prefill), the same entry with the single launch switched off, the two-step pipeline the
    reference launches (in-place pre-processing, then the three-launch prefill) called directly,
    and the entry with the pre-processing forced inside the segment-state kernel
    ("fused_in_state_kernel", gla_prep.FUSED_MAX_CHUNK_HEADS_PER_CU raised).  A warm-up of 60
    two-step calls precedes the legs, which are timed twice in turn and reported from the second
    round (in a single round the first leg ran up to 5 % slower than the same code timed later).  "us": GPU time per call, calls back to back in a replayed HIP graph, each on its own
    raw input set (restored before every replay, untimed); "eager_us": one Python call at a time
    between events, host work included."""
    import triune_amd.fast_gla as FG
    import triune_amd.gla_prep as GP
    from triune_amd import fast_chunk_gla, fused_qkv_g_prep_chunk_gla, fused_qkv_g_prep_inplace
    from triune_amd.workloads import gla_algorithmic_bytes

    B, H, HD = 4, 6, 64
    n_sets = 16 if T <= 2048 else 2
    gen = torch.Generator().manual_seed(15)
    raw_qkv = torch.randn(B, T, 3, H, HD, generator=gen).bfloat16().to(dev)
    # raw gate logits N(3, 1): logsigmoid of them decays about 0.05 nats per token, the scale of
    # config 1's logsigmoid(N(0, 1)) / 16
    raw_g = (torch.randn(B, T, H, HD, generator=gen) + 3.0).bfloat16().to(dev)
    s0 = (0.1 * torch.randn(B, H, HD, HD, generator=gen)).to(dev)
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    emb = torch.cat([torch.outer(torch.arange(T, dtype=torch.float32), inv)] * 2, dim=-1)
    cos, sin = emb.cos().to(dev), emb.sin().to(dev)
    sets = [(raw_qkv.clone(), raw_g.clone(), torch.empty(B, T, H, HD, device=dev, dtype=torch.bfloat16))
            for _ in range(n_sets)]

    def restore():
        for qkv, g, _ in sets:
            qkv.copy_(raw_qkv)
            g.copy_(raw_g)

    def fused(i):
        qkv, g, out = sets[i]
        fused_qkv_g_prep_chunk_gla(qkv, g, cos, sin, initial_state=s0, out=out)

    def two_step(i):
        qkv, g, out = sets[i]
        fused_qkv_g_prep_inplace(qkv, g, cos, sin)
        fast_chunk_gla(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], g, initial_state=s0, out=out)

    stream = torch.cuda.current_stream()
    # clocks up before the first timed leg (after an idle spell the first ~100 calls run slower)
    for i in range(60):
        if i % n_sets == 0:
            restore()
        two_step(i % n_sets)
    torch.cuda.synchronize()
    res, eager = {}, {}
    onepass0, fmax0 = FG.ONEPASS, GP.FUSED_MAX_CHUNK_HEADS_PER_CU
    from triune_amd._lib import lib as _l

    one = bool(_l().triune_hip_gla_prefill_onepass_supported(B, T, H, HD, 1, 1, 1, 0))
    in_state = not one and B * H * ((T + 63) // 64) <= fmax0 * torch.cuda.get_device_properties(dev).multi_processor_count
    legs = [("fused", fused, True, fmax0), ("fused_three_launch", fused, False, fmax0),
            ("prep_then_prefill", two_step, False, fmax0)]
    if not in_state:  # the entry does not take the pre-processing inside the segment-state kernel: time it too
        legs.append(("fused_in_state_kernel", fused, False, 1 << 30))
    try:
        for _round in range(2):  # every leg twice in turn, the second round kept (see the docstring)
            for name, fn, onepass, fmax in legs:
                FG.ONEPASS = onepass
                GP.FUSED_MAX_CHUNK_HEADS_PER_CU = fmax
                res[name] = _graph_us_per_call([lambda i=i: fn(i) for i in range(n_sets)], restore)
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
                for i in range(10 + reps):
                    restore()
                    if i >= 10:
                        ev[i - 10][0].record(stream)
                    fn(0)
                    if i >= 10:
                        ev[i - 10][1].record(stream)
                torch.cuda.synchronize()
                eager[name] = sorted(b.elapsed_time(e) for b, e in ev)[reps // 2] * 1e3  # median
    finally:
        FG.ONEPASS, GP.FUSED_MAX_CHUNK_HEADS_PER_CU = onepass0, fmax0
    alg = gla_algorithmic_bytes(B * T * H, HD, HD, 2, 2, 2) + 2 * B * H * HD * HD * 4
    gbs = alg / (res["fused"] * 1e-6) / 1e9
    return {"workload": f"VectorisedGLA prefill from raw projections (B=4, T={T}, H=6, HD=64, bf16, "
            "RoPE, gate logits N(3,1))",
            "path": "single launch (pre-processing, chunk states and outputs)" if one else
            ("pre-processing inside the segment-state kernel, then the carry scan and the output kernel"
             if in_state else "pre-processing pass, then the three-launch prefill"),
            "timing": f"GPU time per call: {n_sets} calls on their own input sets back to back in a replayed "
            "HIP graph; eager_*: one Python call between events",
            "us": round(res["fused"], 2), "tok_s": round(B * T / (res["fused"] * 1e-6), 1),
            "fused_three_launch_us": round(res["fused_three_launch"], 2),
            "prep_then_prefill_us": round(res["prep_then_prefill"], 2),
            "eager_us": round(eager["fused"], 2), "eager_fused_three_launch_us": round(eager["fused_three_launch"], 2),
            "eager_prep_then_prefill_us": round(eager["prep_then_prefill"], 2),
            **({"fused_in_state_kernel_us": round(res["fused_in_state_kernel"], 2),
                "eager_fused_in_state_kernel_us": round(eager["fused_in_state_kernel"], 2)}
               if "fused_in_state_kernel" in res else {}),
            "alg_bytes": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_tile_prefill(dev, reps=50, T=1024):
    """fast_chunk_gla on VectorisedGLA's prefill tile of already pre-processed inputs (B=4, T=1024,
    H=6, D=64, bf16, fp32 S0, bf16 outputs; the call attention.py:486-494 makes per tile): the
    single-launch prefill against the three-launch one on the same inputs, both timed twice in turn
    and reported from the second round.  "us": GPU time per call (16 calls on 8 rotating input sets
    back to back in a replayed HIP graph); "eager_us": one Python call between events."""
    import triune_amd.fast_gla as FG
    from triune_amd import fast_chunk_gla
    from triune_amd.workloads import gla_algorithmic_bytes, gla_inputs

    B, H, D = 4, 6, 64
    sets = []
    for i in range(8):
        q, k, v, g, s0 = (x.to(dev) for x in gla_inputs(B, T, H, D, seed=17 + i, dtype=torch.bfloat16,
                                                         init_std=0.1))
        sets.append((q, k, v, g, s0, torch.empty_like(v)))
    calls = [lambda i=i: fast_chunk_gla(*sets[i % 8][:4], initial_state=sets[i % 8][4], out=sets[i % 8][5])
             for i in range(16)]
    stream = torch.cuda.current_stream()
    res, eager = {}, {}
    onepass0 = FG.ONEPASS
    try:
        for _round in range(2):  # both legs twice in turn, the second round kept
            for name, onepass in (("onepass", True), ("three_launch", False)):
                FG.ONEPASS = onepass
                res[name] = _graph_us_per_call(calls)
                for _ in range(20):
                    calls[0]()
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
                for b, e in ev:
                    b.record(stream)
                    calls[0]()
                    e.record(stream)
                torch.cuda.synchronize()
                eager[name] = sorted(b.elapsed_time(e) for b, e in ev)[reps // 2] * 1e3
    finally:
        FG.ONEPASS = onepass0
    alg = gla_algorithmic_bytes(B * T * H, D, D, 2, 2, 2) + 2 * B * H * D * D * 4
    gbs = alg / (res["onepass"] * 1e-6) / 1e9
    return {"workload": f"GLA prefill tile (B=4, T={T}, H=6, D=64, bf16 I/O, fp32 S0), fast_chunk_gla",
            "timing": "GPU time per call: 16 calls back to back in a replayed HIP graph; eager_*: one Python "
            "call between events",
            "us": round(res["onepass"], 2), "tok_s": round(B * T / (res["onepass"] * 1e-6), 1),
            "three_launch_us": round(res["three_launch"], 2), "eager_us": round(eager["onepass"], 2),
            "eager_three_launch_us": round(eager["three_launch"], 2), "alg_bytes": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_fused_decode(steps_total, dev, n_bufs=12):
    """Decode step fused with the pre-processing at the config-2 shape (B=256, H=6, HD=64): raw
    qkvg [256, 4, 6, 64] bf16, fp32 state updated in place; 12 rotating state buffers and input
    sets, the loop captured in a graph."""
    from triune_amd import fused_qkvg_decode_step

    B, H, HD = 256, 6, 64
    gen = torch.Generator().manual_seed(6)
    xs = [torch.randn(B, 4, H, HD, generator=gen).bfloat16().to(dev) for _ in range(n_bufs)]
    states = [(0.1 * torch.randn(B, H, HD, HD, generator=gen)).to(dev) for _ in range(n_bufs)]
    outs = [torch.empty(B, 1, H, HD, device=dev, dtype=torch.bfloat16) for _ in range(n_bufs)]
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    emb = torch.cat([torch.outer(torch.arange(steps_total, dtype=torch.float32), inv)] * 2, dim=-1)
    cos, sin = emb.cos().to(dev), emb.sin().to(dev)

    def loop():
        for t in range(steps_total):
            i = t % n_bufs
            fused_qkvg_decode_step(xs[i], cos[t], sin[t], initial_state=states[i], out=outs[i], inplace=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        loop()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loop()
    graph.replay()
    torch.cuda.synchronize()
    ms = _events_time_ms(graph.replay, 3, torch.cuda.current_stream())
    step_us = ms * 1e3 / steps_total
    step_bytes = 2 * B * H * HD * HD * 4 + B * 4 * H * HD * 2 + B * H * HD * 2
    return {"workload": "decode step fused with the pre-processing, config-2 shape (B=256, H=6, HD=64), "
            f"{steps_total}-step graph, {n_bufs} rotating fp32 state buffers and input sets",
            "us_per_step": round(step_us, 3), "tok_s": round(B / (step_us * 1e-6), 1),
            "roofline": {"bound": "hbm", "achieved": round(step_bytes / (step_us * 1e-6) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(step_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "alg_bytes_per_step": step_bytes}}


def bench_gdn(dev, reps=20):
    """Gated DeltaNet prefill, config 3 (B=4, H=6, T=8192, D=64, bf16, per-head beta, one decay per
    token and head).  The gate reaches the operator as config 3 states it, broadcast over D (a
    stride-0 view: the scalar-decay kernels); the same pass with the gate copied out to a full
    [B, T, H, D] tensor (the per-key-dim kernels) is reported beside it."""
    from triune_amd import fast_chunk_gated_deltanet
    from triune_amd.workloads import config3, to_device

    q, k, v, g, beta = config3()
    q, k, v, beta = (x.to(dev) for x in (q, k, v, beta))
    gv = to_device(g, dev)
    gm = gv.contiguous()
    B, T, H, D = q.shape

    def timed(gate):
        fn = lambda: fast_chunk_gated_deltanet(q, k, v, gate, beta=beta)  # noqa: E731
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        return _events_time_ms(fn, reps, torch.cuda.current_stream())

    ms = timed(gv)
    ms_dim = timed(gm)
    # the operator's tensors: q, k, v read, o written (bf16), one gate and one beta per
    # (token, head) read (bf16); zero initial state, fp32 final state written
    alg = B * T * H * (4 * D * 2 + 2 + 2) + B * H * D * D * 4
    # with the gate materialised per key dim it is read as a [B, T, H, D] bf16 tensor
    alg_dim = B * T * H * (5 * D * 2 + 2) + B * H * D * D * 4
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "Gated DeltaNet prefill, config 3 (B=4, H=6, T=8192, D=64, bf16, scalar decay)",
            "ms": round(ms, 4), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "kernels": "gdn_sg_seg_mn + gdn_seg_scan + gdn_sg_seg_out",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "per_dim_gate": {"ms": round(ms_dim, 4), "tok_s": round(B * T / (ms_dim * 1e-3), 1),
                             "alg_bytes": alg_dim,
                             "kernels": "gdn_seg_mn + gdn_seg_scan + gdn_seg_out",
                             "frac": round(alg_dim / (ms_dim * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def bench_gdn_bwd(dev, reps=3):
    """Gated DeltaNet backward, config 3 (B=4, H=6, T=8192, D=64, bf16, per-head beta, one decay
    per token and head, zero initial state): the gradients of q, k, v, g and beta for an upstream
    gradient of o, as fast_chunk_gated_deltanet's autograd returns them (the reference
    differentiates its PyTorch recurrence, fast_gla.py:885-904)."""
    from triune_amd import _lib
    from triune_amd.fast_gla import _gdn_bwd
    from triune_amd.workloads import config3, to_device

    q, k, v, g, beta = config3()
    q, k, v, beta = (x.to(dev) for x in (q, k, v, beta))
    g = to_device(g, dev)
    B, T, H, D = q.shape
    do = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(dev)
    fn = lambda: _gdn_bwd(q, k, v, g, beta, None, _lib.BETA_HEAD, do, None)  # noqa: E731
    fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    # q, k, v, do read and dq, dk, dv, dg written ([B, T, H, D] bf16), the gate read per (token,
    # head) and materialised per key dim by the call, beta read and its gradient written
    alg = B * T * H * (8 * D * 2 + D * 2 + 2 + 2)
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "Gated DeltaNet backward, config 3 (B=4, H=6, T=8192, D=64, bf16, per-head beta)",
            "ms": round(ms, 3), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "kernels": "gdn_segmap + gdn_carry + gdn_ckpt + gdn_dloc + gdn_carry + gdn_bwd + gdn_slice_sum (token-serial inside segments walked in parallel, states recomputed from checkpoints)",
            "roofline": {"bound": "latency (token-serial)", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_gdn_bwd128(dev, reps=3):
    """Gated DeltaNet backward at the reference model's head dim (B=4, T=8192, H=12, D=128, bf16,
    q, k = normalize(elu(x) + 1), logsigmoid gates per key dim, no beta, zero initial state): the
    gradients of q, k, v and g for an upstream gradient of o."""
    from triune_amd import _lib
    from triune_amd.fast_gla import _gdn_bwd

    B, T, H, D = 4, 8192, 12, 128
    gen = torch.Generator(device=dev).manual_seed(13)
    qk = torch.randn(B, T, 2, H, D, device=dev, generator=gen)
    qk = torch.nn.functional.normalize(torch.nn.functional.elu(qk) + 1.0, dim=-1).bfloat16()
    q, k = qk[:, :, 0].contiguous(), qk[:, :, 1].contiguous()
    v = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, device=dev, generator=gen)).bfloat16()
    do = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    fn = lambda: _gdn_bwd(q, k, v, g, None, None, _lib.BETA_NONE, do, None)  # noqa: E731
    fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    alg = B * T * H * (9 * D * 2)  # q, k, v, g, do read; dq, dk, dv, dg written (bf16)
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "Gated DeltaNet backward at head dim 128 (B=4, H=12, T=8192, D=128, bf16, "
                        "per-key-dim logsigmoid gate, no beta)",
            "ms": round(ms, 3), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "roofline": {"bound": "latency (token-serial)", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_gdn128(dev, reps=10):
    """Gated DeltaNet prefill as the reference model calls it at its default head dim
    (triune/model/attention.py:509-536, config.py GLA_HEAD_DIM = 128): q, k = normalize(elu(x) + 1),
    g = logsigmoid(x) per key dim, no beta, zero initial state; B=4, T=8192, H=12 (d_model 1536),
    bf16 (the per-key-dim chunked kernels at D = 128)."""
    from triune_amd import fast_chunk_gated_deltanet

    B, T, H, D = 4, 8192, 12, 128
    gen = torch.Generator(device=dev).manual_seed(3)
    qk = torch.randn(B, T, 2, H, D, device=dev, generator=gen)
    qk = torch.nn.functional.normalize(torch.nn.functional.elu(qk) + 1.0, dim=-1).bfloat16()
    q, k = qk[:, :, 0], qk[:, :, 1]
    v = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, device=dev, generator=gen)).bfloat16()
    fn = lambda: fast_chunk_gated_deltanet(q, k, v, g)  # noqa: E731
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    # q, k, v, g read and o written (bf16), the fp32 final state written
    alg = B * T * H * 5 * D * 2 + B * H * D * D * 4
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "Gated DeltaNet prefill, model call at head dim 128 (B=4, H=12, T=8192, D=128, bf16, "
                        "per-key-dim logsigmoid gate, no beta)",
            "ms": round(ms, 4), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "kernels": "gdn_seg_mn + gdn_seg_scan + gdn_seg_out (D=128)",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_gdn_vbeta(dev, reps=10):
    """Gated DeltaNet prefill with beta per value column (the reference's Triton orientation,
    fast_gla.py:464-465; [B, T, H, D] beta through fast_chunk_gated_deltanet): config 3's shape
    (B=4, H=6, T=8192, D=64) and the model's head dim (B=4, H=12, T=8192, D=128), bf16, q and k
    L2-normalised, g = logsigmoid(x) per key dim, beta = sigmoid(x).  Each sequence is one segment
    (the per-column segment maps differ), walked by the output kernel."""
    from triune_amd import fast_chunk_gated_deltanet

    out = {"workload": "Gated DeltaNet prefill, beta per value column (bf16, per-key-dim logsigmoid gates)"}
    for key, (B, T, H, D) in (("d64", (4, 8192, 6, 64)), ("d128", (4, 8192, 12, 128))):
        gen = torch.Generator(device=dev).manual_seed(5)
        qk = torch.nn.functional.normalize(torch.randn(B, T, 2, H, D, device=dev, generator=gen), dim=-1).bfloat16()
        q, k = qk[:, :, 0], qk[:, :, 1]
        v = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
        g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, device=dev, generator=gen)).bfloat16()
        beta = torch.sigmoid(torch.randn(B, T, H, D, device=dev, generator=gen))
        fn = lambda: fast_chunk_gated_deltanet(q, k, v, g, beta=beta)  # noqa: E731
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
        # q, k, v, g read and o written (bf16), beta read (fp32), the fp32 final state written
        alg = B * T * H * D * (5 * 2 + 4) + B * H * D * D * 4
        gbs = alg / (ms * 1e-3) / 1e9
        out[key] = {"shape": f"B={B}, H={H}, T={T}, D={D}", "ms": round(ms, 4), "tok_s": round(B * T / (ms * 1e-3), 1),
                    "alg_bytes": alg, "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                                   "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    return out


def bench_varlen(dev, reps=5):
    """Packed ragged GLA prefill, config 4 (32 sequences of 128..8192 tokens, H=12, D=128, bf16)."""
    from triune_amd import fast_chunk_gla_varlen
    from triune_amd.workloads import config4

    q, k, v, g, cu, s0 = config4()
    q, k, v, g, cu, s0 = (x.to(dev) for x in (q, k, v, g, cu, s0))
    out = torch.empty_like(v)
    fn = lambda: fast_chunk_gla_varlen(q, k, v, g, cu, initial_state=s0, out=out)  # noqa: E731
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    n_tok, H, D = q.shape[1], q.shape[2], q.shape[3]
    from triune_amd.workloads import gla_algorithmic_bytes

    alg = gla_algorithmic_bytes(n_tok * H, D, D, 2, 2, 2) + 2 * s0.numel() * 4
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": f"varlen GLA prefill, config 4 ({cu.numel() - 1} sequences, {n_tok} tokens, H=12, D=128, bf16)",
            "ms": round(ms, 4), "tok_s": round(n_tok / (ms * 1e-3), 1), "alg_bytes": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_scan(dev, reps=10):
    """FusedRecurrentScan forward and backward at the chunk-state shape of config 1 (B=4, H=6,
    N=256 chunks, Dk=Dv=64, fp32 kv and upstream gradients, as in the reference's own check)."""
    from triune_amd import FusedRecurrentScan
    from triune_amd._lib import dtype_code, lib, ptr, stream_of

    B, H, N, D = 4, 6, 256, 64
    gen = torch.Generator().manual_seed(13)
    kv = torch.randn(B, H, N, D, D, generator=gen).to(dev)
    dec = torch.rand(B, H, N, D, 1, generator=gen).to(dev)
    init = torch.randn(B, H, D, D, generator=gen).to(dev)
    with torch.no_grad():
        fwd = lambda: FusedRecurrentScan.apply(kv, dec, init)  # noqa: E731
        fwd()
        torch.cuda.synchronize()
        ms_f = _events_time_ms(fwd, reps, torch.cuda.current_stream())
        s_all, _ = fwd()
    d_s = torch.randn(B, H, N, D, D, generator=gen).to(dev)
    d_f = torch.randn(B, H, D, D, generator=gen).to(dev)
    dec4 = dec[..., 0].contiguous()
    d_kv, d_init = torch.empty_like(kv), torch.empty_like(init)
    d_dec = torch.empty(B, H, N, D, device=dev)

    def bwd():
        lib().triune_hip_recurrent_scan_bwd(ptr(d_s), dtype_code(d_s), ptr(d_f), dtype_code(d_f), ptr(dec4),
                                            dtype_code(dec4), ptr(s_all), ptr(d_kv), ptr(d_dec), ptr(d_init),
                                            dtype_code(d_kv), B, H, N, D, D, stream_of(kv))

    bwd()
    torch.cuda.synchronize()
    ms_b = _events_time_ms(bwd, reps, torch.cuda.current_stream())
    big, small = kv.numel() * 4, dec4.numel() * 4
    alg_f = 2 * big + small + 2 * init.numel() * 4  # kv read, s_all written, decay, init and final
    alg_b = 3 * big + 2 * small + 2 * init.numel() * 4  # d_s_all, s_all read, d_kv written; decay, d_decay
    out = {"workload": f"FusedRecurrentScan, B={B}, H={H}, N={N}, Dk=Dv={D}, fp32"}
    for name, ms, alg in (("forward", ms_f, alg_f), ("backward", ms_b, alg_b)):
        gbs = alg / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "alg_bytes": alg,
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    return out


def bench_bwd(dev, reps=10):
    """Chunked GLA backward at the config-1 shape (B=4, T=16384, H=6, D=64): bf16 inputs and
    upstream gradient of o, fp32 initial state and final-state gradient, bf16 dq/dk/dv/dg and fp32
    dS0 (the whole launch sequence: segment states, forward scan, chunk states, reverse scan,
    gradient kernel)."""
    from triune_amd.fast_gla import _prefill_bwd
    from triune_amd.workloads import config1

    q, k, v, g, s0 = (x.to(dev) for x in config1(T=16384, B=4, H=6, D=64))
    gen = torch.Generator().manual_seed(11)
    do = torch.randn(q.shape, generator=gen).bfloat16().to(dev)
    ds = torch.randn(s0.shape, generator=gen).to(dev)
    fn = lambda: _prefill_bwd(q, k, v, g, s0, do, ds, 0)  # noqa: E731
    for _ in range(10):
        fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    B, T, H, D = q.shape
    alg = 9 * B * T * H * D * 2 + 3 * B * H * D * D * 4  # q,k,v,g,do read; dq,dk,dv,dg written; states
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "GLA prefill backward, config-1 shape (B=4, T=16384, H=6, D=64, bf16, fp32 states)",
            "ms": round(ms, 4), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_bwd128(dev, reps=5):
    """Chunked GLA backward at the config-4 head size (H=12, Dk=Dv=128) on one dense sequence
    (B=1, T=16384, bf16, config-1 distributions): the gradient kernels hold 64-wide heads, so this
    runs as four (key block, value block) sub-problems whose gradients are summed."""
    from triune_amd.fast_gla import _prefill_bwd
    from triune_amd.workloads import gla_inputs

    q, k, v, g, s0 = (x.to(dev) for x in gla_inputs(1, 16384, 12, 128, seed=128, dtype=torch.bfloat16,
                                                     init_std=0.1))
    gen = torch.Generator().manual_seed(12)
    do = torch.randn(q.shape, generator=gen).bfloat16().to(dev)
    ds = torch.randn(s0.shape, generator=gen).to(dev)
    fn = lambda: _prefill_bwd(q, k, v, g, s0, do, ds, 0)  # noqa: E731
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    ms = _events_time_ms(fn, reps, torch.cuda.current_stream())
    B, T, H, D = q.shape
    alg = 9 * B * T * H * D * 2 + 3 * B * H * D * D * 4
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "GLA prefill backward, config-4 head size (B=1, T=16384, H=12, D=128, bf16, fp32 states)",
            "ms": round(ms, 4), "tok_s": round(B * T / (ms * 1e-3), 1), "alg_bytes": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def cpu_baseline(budget_s=12.0):
    """The reference's PyTorch CPU scan, restated (oracle/ref_port.py), on the config-1 workload
    itself (B=4, H=6, T=16384, D=64; bf16 inputs widened to fp32, as the CPU path computes in
    the input dtype), repeated for about budget_s seconds on all host cores."""
    from oracle.ref_port import fast_chunk_gla_cpu
    from triune_amd.workloads import config1

    torch.set_num_threads(os.cpu_count() or 1)
    q, k, v, g, s0 = config1(T=16384, B=4, H=6, D=64)
    q, k, v, g = (x.float() for x in (q, k, v, g))
    fast_chunk_gla_cpu(q[:, :1024], k[:, :1024], v[:, :1024], g[:, :1024], s0)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fast_chunk_gla_cpu(q, k, v, g, s0)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": 4 * 16384 / med,
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"full config-1 pass (B=4, H=6, T=16384, D=64, fp32 math), median of {len(times)} runs, "
        f"{med:.3f} s each; os.cpu_count()={os.cpu_count()}; cpu={cpu_model or platform.processor()}",
    }


def cpu_baseline_decode(budget_s=5.0, steps=8):
    """The reference's T == 1 op sequence on CPU (fast_gla.py:746-753: S <- e^g S + k v^T, o = q S),
    restated in oracle/ref_port.py, on the config-2 shapes (B=256, H=6, D=64, fp32: the reference
    computes in q.dtype, and its CPU path is run here in fp32), the state carried from step to step
    as the reference's decode loop does; repeated for about budget_s seconds on all host cores."""
    from oracle.ref_port import decode_step_cpu
    from triune_amd.workloads import config2

    torch.set_num_threads(os.cpu_count() or 1)
    B, H, D = 256, 6, 64
    q, k, v, g, s0 = config2(steps=steps, B=B, H=H, D=D)
    q, k, v, g = (x.float() for x in (q, k, v, g))
    with torch.no_grad():
        decode_step_cpu(q[0], k[0], v[0], g[0], s0)  # warm-up
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < 3 or time.perf_counter() < t_end:
            S = s0
            t0 = time.perf_counter()
            for t in range(steps):
                _, S = decode_step_cpu(q[t], k[t], v[t], g[t], S)
            times.append((time.perf_counter() - t0) / steps)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": B / med,
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"config-2 decode (B=256, H=6, D=64, fp32 math, state carried), {steps}-step loops, median "
        f"of {len(times)} loops, {med * 1e3:.2f} ms per step; os.cpu_count()={os.cpu_count()}",
    }


def _traffic_from_profiles(key="output_kernel_bytes_per_launch"):
    """A figure of the config-1 prefill measured with rocprofv3 counters on this build
    (profiles/prefill_traffic.json, written from those runs): HBM bytes per output-kernel launch
    or per pass (FETCH_SIZE / WRITE_SIZE scaled by the same counters on a copy of known size), or
    the MFMA busy fraction of a kernel (the MfmaUtil counter: SQ_VALU_MFMA_BUSY_CYCLES over
    GRBM_GUI_ACTIVE x SIMDs); None when nothing is recorded."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "prefill_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--decode-steps", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary workload lines (GDN, varlen, pre-processing, fused decode, backward)")
    ap.add_argument("--fused-prefill-t", type=int, default=1024, metavar="T",
                    help="sequence length of the fused pre-processing prefill leg (default 1024, the tile "
                    "VectorisedGLA prefills in)")
    ap.add_argument(
        "--copy-probe",
        type=int,
        default=0,
        metavar="MIB",
        help="only run a plain device copy of MIB MiB (steps times): the known-size reference used to "
        "scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings",
    )
    ap.add_argument(
        "--only",
        choices=("decode", "gdn", "gdn128", "gdn_vbeta", "gdn_decode", "gdn_bwd", "gdn_bwd128", "varlen", "prep", "fused_prefill", "fused_decode", "bwd", "bwd128", "scan", "tile_prefill"),
        default=None,
        help="profiling aid: run one secondary workload alone and print its own JSON line",
    )
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build has no multi-GPU path (the (b, h) recurrences "
            "shard across GPUs with no exchange). Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.copy_probe:
        n = args.copy_probe << 18  # fp32 elements
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_mib": args.copy_probe, "launches": args.steps}), flush=True)
        return
    if args.only:
        if args.only == "decode":
            res = bench_decode(args.decode_steps, dev)
        elif args.only == "fused_decode":
            res = bench_fused_decode(args.decode_steps, dev)
        else:
            res = {"gdn": bench_gdn, "gdn128": bench_gdn128, "gdn_vbeta": bench_gdn_vbeta, "gdn_decode": bench_gdn_decode,
                   "gdn_bwd": bench_gdn_bwd, "gdn_bwd128": bench_gdn_bwd128,
                   "varlen": bench_varlen, "prep": bench_prep, "bwd": bench_bwd, "bwd128": bench_bwd128,
                   "scan": bench_scan, "tile_prefill": bench_tile_prefill,
                   "fused_prefill": lambda d: bench_fused_prefill(d, T=args.fused_prefill_t)}[args.only](dev)
        print(json.dumps({"only": args.only, **res}), flush=True)
        return
    # Order: the CPU baselines and the headline's input generation first (the GPU idles
    # meanwhile), then the secondary GPU legs, the last of them a replayed graph with no host gaps,
    # then the headline prefill, so no leg is timed right after the GPU sat idle (clocks ramp down
    # when idle: after a 2 s idle gap the first hundred passes run up to 25 % slower, and even
    # right after other GPU work the first ten run about 6 % slower than the steady state).  The
    # headline itself does exactly `warmup` untimed passes before its `steps` timed ones.
    def leg(name, fn, *fa):
        # each leg allocates its own buffers from a clean caching allocator (the previous legs'
        # blocks returned to the device first)
        import gc

        gc.collect()
        if torch.cuda.is_available():
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        r = fn(*fa)
        _progress(f"{name} done")
        return r

    cpu = None if args.no_cpu else leg("cpu baseline (prefill)", cpu_baseline)
    cpu_dec = None if args.no_cpu or args.no_decode else leg("cpu baseline (decode)", cpu_baseline_decode)
    pre_in = prefill_inputs(dev)
    pre_graph = prefill_graph(args.steps, dev, pre_in)  # captured now: see prefill_graph
    dec = None if args.no_decode else leg("decode", bench_decode, args.decode_steps, dev)
    extra = {}
    if not args.no_extra:
        legs = (("gdn", bench_gdn, dev), ("gdn128", bench_gdn128, dev), ("gdn_vbeta", bench_gdn_vbeta, dev),
                ("gdn_decode", bench_gdn_decode, dev), ("gdn_bwd", bench_gdn_bwd, dev),
                ("gdn_bwd128", bench_gdn_bwd128, dev), ("varlen", bench_varlen, dev), ("prep", bench_prep, dev),
                ("fused_prefill", lambda d: bench_fused_prefill(d, T=args.fused_prefill_t), dev),
                ("fused_prefill_t16k", lambda d: bench_fused_prefill(d, T=16384), dev),
                ("tile_prefill", bench_tile_prefill, dev), ("bwd", bench_bwd, dev),
                ("bwd128", bench_bwd128, dev), ("scan", bench_scan, dev),
                ("fused_decode", bench_fused_decode, args.decode_steps, dev))
        for name, fn, *fa in legs:
            extra[name] = leg(name, fn, *fa)
    pre = bench_prefill(args.steps, args.warmup, dev, pre_in, captured=pre_graph)
    _progress("headline prefill done")
    line = {
        "metric": METRIC,
        "value": round(pre["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms"], 4),
        "timing": "one HIP-graph replay of the `steps` passes (events around it; the graph captured before the "
        "secondary legs), right after `warmup` direct calls, which follow the last leg's GPU work; "
        f"the same passes as direct calls: {pre['eager_ms']:.4f} ms/pass",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE config 1 distributions)",
        "config": {
            "workload": "GLA chunked prefill, config 1",
            "B": 4,
            "T": 16384,
            "H": 6,
            "Dk": 64,
            "Dv": 64,
            "chunk": 64,
            "io": "bf16",
            "state": "fp32",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(pre["k3_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(pre["k3_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": _traffic_from_profiles(),
            "kernel": "gla_seg_output_kernel<bf16,bf16,64,64> (HIP events on its dispatch, one pair per pass)",
            "kernel_us": round(pre["k3_ms"] * 1e3, 2),
            "alg_bytes_per_launch": pre["k3_bytes"],
            "pass": {
                "kernels": "gla_seg_state + seg_scan_f32 + gla_seg_output",
                "alg_bytes": pre["alg_bytes"],
                "achieved_gbs": round(pre["gbs"], 1),
                "frac": round(pre["gbs"] / HBM_PEAK_GBS, 4),
                "traffic": _traffic_from_profiles("bytes_per_pass"),
            },
            "mfma_alg_tflops": round(pre["tflops"], 2),
            "mfma_alg_frac": round(pre["tflops"] / BF16_PEAK_TFLOPS, 4),
            "mfma_busy": _traffic_from_profiles("mfma_busy_output_kernel"),
            "mfma_busy_state_kernel": _traffic_from_profiles("mfma_busy_state_kernel"),
        },
        "cpu_baseline": cpu,
    }
    if dec is not None:
        line["decode"] = {
            "workload": "batched decode step, config 2 (B=256, H=6, D=64, fp32 state, bf16 q/k/v/g/o), "
            f"{args.decode_steps}-step graph, {dec['state_buffers']} rotating state buffers and input sets",
            "tok_s": round(dec["tok_s"], 1),
            "us_per_step": round(dec["step_us"], 3),
            "eager_us_per_step": round(dec["eager_step_us"], 3),
            "cold_inputs_us_per_step": round(dec["cold_step_us"], 3),
            "torch_copy_same_state_bytes": {"us_per_step": round(dec["copy_step_us"], 3),
                                            "achieved": round(dec["copy_gbs"], 1), "unit": "GB/s"},
            "roofline": {
                "bound": "hbm",
                "achieved": round(dec["gbs"], 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
                "alg_bytes_per_step": dec["step_bytes"],
            },
            "cpu_baseline": cpu_dec,
        }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
