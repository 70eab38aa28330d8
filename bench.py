#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (one JSON line on stdout).

Headline workload (the decode GEMV configuration): W4A16 decode GEMV, M=1, K=4096, N=11008, int4 group
128 with fp16 scales, fp16 activations N(0,1), weights N(0, 0.02), seeded CPU generator.
A "step" is one decode call over one activation row, made as ``QuantLinear`` makes it: the
prepared strip GEMV (``_pk.PreparedStrips`` over ``pk_w4a16_strips_run``) on the layer's
decode copy of the weights (the strip layout: each 16-column strip's K rows contiguous, one
workgroup per strip over the whole of K, one launch). The same kernel through the generic
binding (``pk_w4a16_gemm_strips``), and the same call on ``QuantLinear``'s block layout
(``pk_w4a16_gemm_tiled``, 128 x 256 blocks: the split-K GEMV, slices added in L2) and on
``pack_int4_n``'s row layout (``pk_w4a16_gemm``), are timed beside it. ``value`` is the
whole-op HBM throughput (algorithmic bytes / step time), inputs resident in HBM. 40 distinct
copies of the packed weights and scales (932 MB, more than twice the 256 MB Infinity Cache)
are rotated: the W warm-up calls read copies 0..W-1, the timed calls start at copy W.

Timing (``eager_ms``): W eager warm-up steps, then eager steps for 250 ms (the clocks settle
under load); then 5 repetitions of exactly K steps. Before each repetition, 15 untimed calls
read the 15 copies before the first timed one (350 MB, as the layers before it would in a
decode loop), so a repetition never starts on weights its predecessor left in the caches,
however small K is; then a spin kernel keeps the GPU busy while the host enqueues the timed
calls (4.3 us of host time per call against 6.3 us of kernel), so they run back to back.
The timed region runs from the first timed kernel's start to the last one's end: HIP events
on the calls' stream that the first and last dispatches record themselves
(``pk_w4a16_strips_run_events``), so no event packet sits inside it. The median repetition
gives ``ms_per_step``; the best, the same K steps between two event packets on the stream
(~4.5 us more per repetition), and the same K steps replayed as one HIP graph (which adds
the graph's launch bubble, ~7 us per replay) are reported beside it. The strip GEMV is one kernel launch, so
the op is the dominant kernel and the roofline fraction uses its time. The other lines
replay HIP graphs (``GraphTimer``) after the same settling time.

Correctness comes first: before any timing each GPU line checks its own output against the
reference's test-path expression in fp32 torch on the GPU (unpack, multiply by the repeated
group scales, ``a.float() @ deq``; for fp8 ``(a8.float() @ b8.float()) * out_scale`` and the
fp32 product) and runs the call twice to check that the two outputs are bitwise equal.

The same JSON line carries the split-K sweep of the config, the Llama-3-8B layer sweep
(config 5), the W4A16 GEMM (prefill 2048x4096x4096 and 4096^3) and fp8 GEMM (4096^3) lines the
metric also names, split-KV decode attention, GPTQ of one layer, the eager host time of one
``w4a16_gemm`` call, and the reference's CPU path (the torch expression above on the host
cores: dequantize, then matmul, each the median of 5 runs after a warm-up).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-sweep]
       python bench.py --only {gemv,prefill,gemm4096,fp8,fp8_2048,flash_decode,gptq,sweep}
       [--no-row-layout: time the W4A16 lines on the block layout only, for kernel traces]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "pico-kernels_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2516.6  # dense fp16 (256 CU x 2.4 GHz x 4096 FLOP/clk)
MFMA_F8_PEAK_TFLOPS = 5033.2   # dense fp8
N_ROTATE = 40
# Time the row layout (pack_int4_n order, pk_w4a16_gemm) beside QuantLinear's block layout;
# --no-row-layout turns it off, so a kernel trace holds the block layout's launches alone
# (both layouts run the same kernels).
ROW_LAYOUT = True
WARM_MS = 250.0  # untimed graph replays before each timed measurement (GraphTimer.run)
SPIN_CYCLES = 500_000  # spin ahead of each timed repetition: ~0.2 ms at the shader clock
PREROLL = 15  # untimed calls on other weight copies ahead of each timed GEMV replay (350 MB)
KERNEL_NAMES = {1: "w4a16_gemv_mfma_kernel", 2: "gemm_v3_f16_kernel", 3: "w4a16_skinny_kernel",
                4: "w4a16_tr4_kernel", "strips": "w4a16_strip_kernel"}


def _gen(seed: int):
    import torch

    g = torch.Generator()
    g.manual_seed(seed)
    return g


def w4a16_bytes(M: int, K: int, N: int, group: int = 128) -> int:
    """Algorithmic HBM bytes of one W4A16 matmul: packed weights, fp16 scales, fp16
    activations in, fp16 output."""
    return K * N // 2 + (K // group) * N * 2 + M * K * 2 + M * N * 2


class GraphTimer:
    """Capture `steps` calls fn(warmup + i) in one HIP graph on a private stream, after the
    eager warm-up calls fn(0 .. warmup-1); time replays. With fn rotating over buffer copies
    by index, the graph starts on the copy after the last one the warm-up read."""

    def __init__(self, fn, steps: int, warmup: int):
        import torch

        self.stream = torch.cuda.Stream()
        self.steps = steps
        self.fn = fn
        self.start = max(warmup, 1)
        with torch.cuda.stream(self.stream):
            for i in range(max(warmup, 1)):
                fn(i)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        start = max(warmup, 1)
        with torch.cuda.graph(self.graph, stream=self.stream):
            for i in range(steps):
                fn(start + i)
        torch.cuda.synchronize()

    def run(self, reps: int = 1, warm_ms: float = WARM_MS, preroll: int = 0) -> float:
        """Milliseconds per step (median of `reps` replays; the best is kept in `self.best`),
        after untimed replays for at least `warm_ms` of wall time: the GPU's clocks settle
        under load over a few hundred milliseconds, and without this the first configuration
        timed reads ~3% slow. With `preroll` > 0, the calls fn(start - preroll .. start - 1)
        run eagerly (untimed) before every timed replay, as the calls before it in a decode
        loop would: with fn rotating over weight copies by index modulo their count, these
        are the copies just before the graph's first, so the replay starts with other weights
        in the caches rather than the tail of its own previous replay. A short spin kernel
        ahead of the start event keeps the GPU busy while the host enqueues the replay, so a
        graph of a few calls is not timed with its launch latency."""
        import statistics

        import torch

        times = []
        with torch.cuda.stream(self.stream):
            t_end = time.perf_counter() + warm_ms * 1e-3
            while time.perf_counter() < t_end:
                self.graph.replay()
                torch.cuda.synchronize()
            for _ in range(reps):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                for j in range(preroll):
                    self.fn(self.start - preroll + j)
                torch.cuda._sleep(SPIN_CYCLES)
                e0.record(self.stream)
                self.graph.replay()
                e1.record(self.stream)
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1) / self.steps)
        self.best = min(times)
        return statistics.median(times)


def eager_ms(fn, steps: int, warmup: int, reps: int = 5, preroll: int = PREROLL,
             warm_ms: float = WARM_MS, fn_timed=None) -> dict:
    """Milliseconds per step of exactly `steps` eager calls fn(start .. start + steps - 1)
    (start = max(warmup, 1)) between two HIP events on a private stream: (median, best) of
    `reps` repetitions. Before the timing: the warm-up calls fn(0 .. warmup - 1), then calls
    for `warm_ms` of wall time (the clocks settle under load). Before each repetition: the
    calls fn(start - preroll .. start - 1), untimed, as the calls before them in a decode loop
    would (with fn rotating over weight copies by index modulo their count, the copies just
    before the timed ones), then a spin kernel of SPIN_CYCLES, during which the host enqueues
    the timed calls ahead of the GPU. For a call whose host cost is below its kernel time
    the GPU then runs the timed calls back to back; a graph replay would add its launch
    bubble (~7 us here) to every repetition.

    Returns the median and best milliseconds per step between two event packets recorded on
    the stream around the calls ("markers": they add ~4.5 us per repetition, 0.22 us per step
    at K = 20). With ``fn_timed(i, start, stop)`` -- fn(i) with the dispatch itself recording
    the events as its kernel starts and ends -- each repetition is also run with the first
    call recording its kernel's start and the last its kernel's end ("kernels": the GPU time
    from the first timed kernel's start to the last one's end, the launches between them
    back to back as before)."""
    import statistics

    import torch

    stream = torch.cuda.Stream()
    start = max(warmup, 1)
    times = []
    with torch.cuda.stream(stream):
        for i in range(start):
            fn(i)
        torch.cuda.synchronize()
        t_end = time.perf_counter() + warm_ms * 1e-3
        i = start
        while time.perf_counter() < t_end:
            for _ in range(64):
                fn(i)
                i += 1
            torch.cuda.synchronize()
        times_k = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            for j in range(preroll):
                fn(start - preroll + j)
            torch.cuda._sleep(SPIN_CYCLES)
            e0.record(stream)
            for j in range(steps):
                fn(start + j)
            e1.record(stream)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / steps)
            if fn_timed is None:
                continue
            k0 = torch.cuda.Event(enable_timing=True)
            k1 = torch.cuda.Event(enable_timing=True)
            k0.record(stream)  # creates both events before the dispatches record them
            k1.record(stream)
            torch.cuda.synchronize()
            for j in range(preroll):
                fn(start - preroll + j)
            torch.cuda._sleep(SPIN_CYCLES)
            for j in range(steps):
                if j == 0 or j == steps - 1:
                    fn_timed(start + j, k0 if j == 0 else None, k1 if j == steps - 1 else None)
                else:
                    fn(start + j)
            torch.cuda.synchronize()
            times_k.append(k0.elapsed_time(k1) / steps)
    res = {"markers": statistics.median(times), "markers_best": min(times)}
    if times_k:
        res.update(kernels=statistics.median(times_k), kernels_best=min(times_k))
    return res


def per_launch_ms(fn, n: int) -> float:
    """Mean duration of single launches: a HIP event pair around each fn(i) on one
    stream (fn launches on the current stream), after a warm-up."""
    import torch

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(10):
            fn(i)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(n)]
        for i, (e0, e1) in enumerate(ev):
            e0.record(stream)
            fn(i)
            e1.record(stream)
        torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) / n


def gemv_inputs(M: int, K: int, N: int, nrot: int, dev):
    import torch

    import gemm_int4

    a = torch.randn(M, K, generator=_gen(0)).half()
    w = (torch.randn(K, N, generator=_gen(1)) * 0.02).half()
    qw, sc = gemm_int4.quantize_int4_group(w.to(dev), 128)
    qws = [qw] + [qw.clone() for _ in range(nrot - 1)]
    scs = [sc] + [sc.clone() for _ in range(nrot - 1)]
    return a, w, qws, scs


def tiled_copies(qws: list) -> list:
    """The weight copies in QuantLinear's in-memory layout (128 x 256 blocks)."""
    import _pk

    return [_pk.tile_weights(q) for q in qws]


def strip_copies(qws: list, scs: list) -> tuple[list, list]:
    """The weight and scale copies in QuantLinear's decode layout (16-column strips)."""
    import _pk

    return [_pk.strip_weights(q) for q in qws], [_pk.strip_scales(s) for s in scs]


def unpack_codes(qw):
    """``(K, N//8)`` int32 words holding pack_int4_n bytes -> ``(K, N)`` int8 codes in [-8, 7],
    with plain torch ops (the reference's unpack, tests/test_gemm_int4.py:36-41)."""
    import torch

    b = qw.contiguous().view(torch.uint8)
    lo = (b & 0x0F).to(torch.int8)
    hi = (b >> 4).to(torch.int8)
    q = torch.stack((lo, hi), dim=2).reshape(b.shape[0], -1)
    return torch.where(q >= 8, q - 16, q)


def dequant_expr(qw, sc, group: int = 128):
    """fp32 weights of the group format: codes times the scales repeated over each group."""
    return unpack_codes(qw).float() * sc.float().repeat_interleave(group, 0)[: qw.shape[0]]


def rel_fro(x, ref) -> float:
    import torch

    return (torch.linalg.norm(x.float() - ref) / torch.linalg.norm(ref)).item()


def check_w4a16(call, a, qw, sc, group: int = 128) -> dict:
    """Correctness of a W4A16 call before it is timed: relative Frobenius error against the
    reference's test-path expression in fp32 torch on the GPU (``a.float() @ deq``,
    tests/test_gemm_int4.py:26), and a bitwise repeat of the call."""
    import torch

    y1 = call().clone()
    y2 = call().clone()
    torch.cuda.synchronize()
    ref = a.float() @ dequant_expr(qw, sc, group)
    rel = rel_fro(y1, ref)
    ok = bool(torch.equal(y1, y2))
    if not (rel <= 1e-3 and ok):
        raise RuntimeError(f"W4A16 output check failed before timing: rel_fro={rel:.3e} "
                           f"bitwise_repeat={ok}")
    return {"rel_fro_vs_fp32_expr": float(f"{rel:.3e}"), "tolerance": 1e-3,
            "bitwise_repeat": ok}


def host_overhead(step, n: int = 1000) -> dict:
    """Eager cost of one call from Python: ``wall`` = n back-to-back calls then one device
    synchronisation, per call; ``enqueue`` = median host time inside one call (argument
    checks, plan, ctypes marshalling, launch)."""
    import statistics

    import torch

    for i in range(20):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        step(i)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / n
    ts = []
    for i in range(200):
        t = time.perf_counter()
        step(i)
        ts.append(time.perf_counter() - t)
        if i % 16 == 15:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return {"eager_wall_us_per_call": round(wall * 1e6, 2),
            "host_enqueue_us_median": round(statistics.median(ts) * 1e6, 2)}


def bench_gemv(args, dev) -> dict:
    import torch

    import _pk

    M, K, N = 1, 4096, 11008
    a, w, qws, scs = gemv_inputs(M, K, N, N_ROTATE, dev)
    qts = tiled_copies(qws)
    qss, sss = strip_copies(qws, scs)
    ag = a.to(dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    nbytes = w4a16_bytes(M, K, N)
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)

    # QuantLinear's decode call: a prepared strip GEMV per layer (here per weight copy)
    calls = [_pk.PreparedStrips(q, sc, 128, 1.0, torch.float16) for q, sc in zip(qss, sss)]

    def step(i):
        calls[i % N_ROTATE](ag, out)

    def step_timed(i, start, stop):  # the same call, its dispatch recording start / stop
        calls[i % N_ROTATE].timed(ag, out, start, stop)

    def step_binding(i):  # the same kernel through the generic binding
        _pk.w4a16_gemm_strips(ag, qss[i % N_ROTATE], sss[i % N_ROTATE], 128, 1.0,
                              torch.float16, out=out)

    def step_blocks(i):  # QuantLinear's layout above its decode rows: blocks
        _pk.w4a16_gemm(ag, qts[i % N_ROTATE], scs[i % N_ROTATE], 128, 1.0, torch.float16,
                       split_k=0, out=out, tiled=True)

    def step_rows(i):  # pack_int4_n's row layout
        _pk.w4a16_gemm(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 1.0, torch.float16,
                       split_k=0, out=out)

    def once(fn):
        def call():
            fn(0)
            return out
        return call

    check = check_w4a16(once(step), ag, qws[0], scs[0])
    y_strips = out.clone()
    check_w4a16(once(step_binding), ag, qws[0], scs[0])
    check["bitwise_equal_to_binding"] = bool(torch.equal(y_strips, out))
    if not check["bitwise_equal_to_binding"]:
        raise RuntimeError("W4A16 GEMV: prepared call and binding disagree")
    check_blocks = check_w4a16(once(step_blocks), ag, qws[0], scs[0])
    y_blocks = out.clone()
    check_rows = check_w4a16(once(step_rows), ag, qws[0], scs[0])
    check_blocks["bitwise_equal_to_row_layout"] = bool(torch.equal(y_blocks, out))
    if not check_blocks["bitwise_equal_to_row_layout"]:
        raise RuntimeError("W4A16 GEMV: block and row layouts disagree")
    timed = args.steps  # exactly K steps per repetition
    em = eager_ms(step, timed, args.warmup, fn_timed=step_timed)
    ms, ms_best = em["kernels"], em["kernels_best"]
    ms_markers = em["markers"]
    ms_graph = GraphTimer(step, timed, args.warmup).run(reps=5, preroll=PREROLL)
    ms_blocks = (GraphTimer(step_blocks, timed, args.warmup).run(reps=5, preroll=PREROLL)
                 if ROW_LAYOUT else None)
    ms_rows = (GraphTimer(step_rows, timed, args.warmup).run(reps=5, preroll=PREROLL)
               if ROW_LAYOUT else None)

    # The op is one launch of the strip kernel: the timed calls' per-step time is that kernel's
    # average launch duration (from the first timed kernel's start to the last one's end, on
    # the launch stream). Single launches bracketed by their own event packets read ~2.5 us
    # longer and are reported beside it.
    ms_kernel = ms
    ms_kernel_events = per_launch_ms(step, min(timed, 500))

    sweep = {}
    for s in ((1, 2, 4, 8, 16) if getattr(args, "split_sweep", True) else ()):
        def step_s(i, s=s):
            _pk.w4a16_gemm(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 1.0, torch.float16,
                           split_k=s, out=out)

        check_w4a16(once(step_s), ag, qws[0], scs[0])
        ms_s = GraphTimer(step_s, max(min(args.steps, 400), 2 * N_ROTATE), 2).run(reps=3)
        sweep[str(s)] = round(nbytes / (ms_s * 1e-3) / 1e9, 1)
    return {
        "M": M, "K": K, "N": N, "split": 1, "kernel_id": "strips", "launches": 1,
        "blocks_layout_plan": {"kernel_id": kid, "split": split,
                               "launches": _pk.w4a16_launches(M, N, K, 128, 0)},
        "bytes": nbytes, "steps_timed": timed, "check": check, "check_blocks": check_blocks,
        "check_rows": check_rows, "ms_per_step": ms, "ms_per_step_best": ms_best,
        "ms_graph": ms_graph, "ms_markers": ms_markers,
        "ms_blocks": ms_blocks, "ms_rows": ms_rows,
        "ms_kernel": ms_kernel, "ms_kernel_events": ms_kernel_events,
        "split_sweep_GBs": sweep,
        "host": host_times(ag, qws[0], scs[0], qss[0], sss[0], out, step_binding),
        "inputs": (ag, qws[0], scs[0]),
    }


def host_times(ag, qw, sc, qs, ss, out, step) -> dict:
    """Eager host cost of one decode call at M = 1 (see host_overhead), three ways: the generic
    binding (``_pk.w4a16_gemm_strips``), the prepared call QuantLinear keeps per layer
    (``_pk.PreparedStrips``, output given: the timed step), and ``QuantLinear.forward`` itself
    (its output allocated per call)."""
    import _pk
    import quant_linear

    K, N = qw.shape[0], qw.shape[1] * 8
    call = _pk.PreparedStrips(qs, ss, 128, 1.0, out.dtype)
    layer = quant_linear.QuantLinear(K, N, bias=False, group_size=128, device=ag.device)
    layer.set_codes(qw)
    layer.scales.copy_(sc)
    layer._refresh()
    return {"binding": host_overhead(step), "prepared_call": host_overhead(lambda i: call(ag, out)),
            "quant_linear_forward": host_overhead(lambda i: layer(ag))}


def bench_prefill(dev, iters: int = 50, M: int = 2048) -> dict:
    """W4A16 GEMM (group 128, fp16 out) at M x 4096 x 4096: M = 2048 is the prefill config,
    M = 4096 the 4096^3 shape the metric also names. Checked, then a graph of `iters` calls
    replayed 5 times (best replay)."""
    import torch

    import _pk
    import gemm_int4

    K, N = 4096, 4096
    a = torch.randn(M, K, generator=_gen(2)).half().to(dev)
    w = (torch.randn(K, N, generator=_gen(3)) * 0.02).half().to(dev)
    qw, sc = gemm_int4.quantize_int4_group(w, 128)
    qt = _pk.tile_weights(qw)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)

    def once():  # QuantLinear's layout: blocks
        _pk.w4a16_gemm(a, qt, sc, 128, 1.0, torch.float16, out=out, tiled=True)
        return out

    def once_rows():
        _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16, out=out)
        return out

    check = check_w4a16(once, a, qw, sc)
    y_tiles = out.clone()
    check_w4a16(once_rows, a, qw, sc)
    check["bitwise_equal_to_row_layout"] = bool(torch.equal(y_tiles, out))
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)
    ms = GraphTimer(lambda i: once(), iters, 2).run(reps=5)
    ms_rows = GraphTimer(lambda i: once_rows(), iters, 2).run(reps=5) if ROW_LAYOUT else None
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"workload": "w4a16_prefill_gemm" if M == 2048 else "w4a16_gemm_4096^3", "M": M, "K": K,
            "N": N, "ms": round(ms, 4), "kernel_id": kid, "split": split,
            "value": round(tflops, 1), "unit": "TFLOP/s", "dtype": "fp16 MFMA, fp32 acc",
            "weights": "128x256 blocks (QuantLinear's layout, pk_w4a16_gemm_tiled)",
            "row_layout_TFLOP/s": round(2.0 * M * N * K / (ms_rows * 1e-3) / 1e12, 1) if ms_rows else None,
            "check": check,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}}


def bench_fp8(dev, iters: int = 50, M: int = 4096) -> dict:
    """fp8 e4m3 GEMM at M x 4096 x 4096 (fp16 out). Checked first: relative Frobenius error of
    this output against the fp32 product (the reference test's comparison,
    tests/test_gemm_fp8.py:24), beside the same error of the reference kernel's arithmetic in
    fp32 torch, ``(a8.float() @ b8.float()) * out_scale`` with out_scale = 1 / (a_scale *
    b_scale) (gemm_fp8.py:98-117), and a bitwise repeat."""
    import torch

    import _pk
    import gemm_fp8

    N = K = 4096
    a = torch.randn(M, K, generator=_gen(4)).half().to(dev)
    b = torch.randn(K, N, generator=_gen(5)).half().to(dev)
    a8, sa = gemm_fp8.quantize(a)
    b8, sb = gemm_fp8.quantize(b)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    scale = 1.0 / (sa * sb)

    def once():
        _pk.fp8_gemm(a8, b8, scale, torch.float16, out=out)
        return out

    y1 = once().clone()
    y2 = once().clone()
    ref = a.float() @ b.float()
    rel = rel_fro(y1, ref)
    rel_expr = rel_fro((a8.float() @ b8.float()) * scale, ref)
    ok = bool(torch.equal(y1, y2))
    if not (abs(rel - rel_expr) <= 1e-3 and ok):
        raise RuntimeError(f"fp8 output check failed before timing: rel={rel:.5f} "
                           f"reference expression {rel_expr:.5f} bitwise_repeat={ok}")
    del y1, y2, ref
    ms = GraphTimer(lambda i: once(), iters, 2).run(reps=5)
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"workload": "fp8_e4m3_gemm" if M == 4096 else "fp8_e4m3_gemm_2048x4096x4096",
            "M": M, "K": K, "N": N, "ms": round(ms, 4),
            "value": round(tflops, 1), "unit": "TFLOP/s", "dtype": "e4m3 MFMA, fp32 acc",
            "rel_fro_vs_fp32": round(rel, 5),
            "check": {"rel_fro_vs_fp32": round(rel, 5),
                      "reference_expr_rel_fro_vs_fp32": round(rel_expr, 5),
                      "diff_pp": round(100 * (rel - rel_expr), 4), "tolerance_pp": 0.1,
                      "bitwise_repeat": ok},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1),
                         "peak": MFMA_F8_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_F8_PEAK_TFLOPS, 4)}}


SWEEP_LAYERS = (("qkv", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up", 4096, 14336),
                ("down", 14336, 4096))


def bench_llama_sweep(dev, iters: int = 50) -> list:
    """Llama-3-8B layer sweep: each layer at M = 1, 8, 32, 128, checked,
    then timed over rotating weight copies (more than 600 MB per layer, at most 40 copies):
    a graph of max(iters, 2 x copies) calls starting after the warm-up's copies, best of 3
    replays. ``frac`` is the applicable roof (slower of streaming the bytes at 8 TB/s and
    issuing the MFMAs at the dense fp16 peak) over the measured time."""
    import torch

    import _pk
    import gemm_int4
    import quant_linear

    rows = []
    for name, K, N in SWEEP_LAYERS:
        w = (torch.randn(K, N, generator=_gen(6)) * 0.02).half().to(dev)
        qw, sc = gemm_int4.quantize_int4_group(w, 128)
        del w
        nrot = max(2, min(N_ROTATE, (600 << 20) // (K * N // 2) + 1))
        qws = [qw] + [qw.clone() for _ in range(nrot - 1)]
        qts = tiled_copies(qws)
        scs = [sc] + [sc.clone() for _ in range(nrot - 1)]
        qss, sss = strip_copies(qws, scs)
        for M in (1, 8, 32, 128):
            a = torch.randn(M, K, generator=_gen(7)).half().to(dev)
            out = torch.empty((M, N), dtype=torch.float16, device=dev)
            strips = M <= quant_linear.decode_rows(K, N)

            def step(i):  # what QuantLinear runs: the strip copy for decode rows, else blocks
                if strips:
                    _pk.w4a16_gemm_strips(a, qss[i % nrot], sss[i % nrot], 128, 1.0,
                                          torch.float16, out=out)
                else:
                    _pk.w4a16_gemm(a, qts[i % nrot], scs[i % nrot], 128, 1.0, torch.float16,
                                   out=out, tiled=True)

            def step_rows(i):
                _pk.w4a16_gemm(a, qws[i % nrot], scs[i % nrot], 128, 1.0, torch.float16,
                               out=out)

            def once():
                step(0)
                return out

            check = check_w4a16(once, a, qw, sc)
            ms = GraphTimer(step, max(iters, 2 * nrot), 2).run(reps=3)
            ms_rows = GraphTimer(step_rows, max(iters, 2 * nrot), 2).run(reps=3) if ROW_LAYOUT else None
            by = w4a16_bytes(M, K, N)
            flop = 2.0 * M * N * K
            t_hbm = by / (HBM_PEAK_GBS * 1e9)
            t_mfma = flop / (MFMA_F16_PEAK_TFLOPS * 1e12)
            kid, split = _pk.w4a16_plan(M, N, K, 128, 0)
            rows.append({"layer": name, "M": M, "K": K, "N": N, "us": round(ms * 1e3, 2),
                         "us_row_layout": round(ms_rows * 1e3, 2) if ms_rows else None,
                         "GB/s": round(by / (ms * 1e-3) / 1e9, 1),
                         "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 2),
                         "bound": "hbm" if t_hbm >= t_mfma else "mfma",
                         "frac": round(max(t_hbm, t_mfma) / (ms * 1e-3), 4),
                         "layout": "strips" if strips else "blocks",
                         "kernel_id": "strips" if strips else kid, "split": 1 if strips else split,
                         "launches": 1 if strips else _pk.w4a16_launches(M, N, K, 128, 0),
                         "copies": nrot,
                         "rel_fro": check["rel_fro_vs_fp32_expr"]})
        del qws, qts, scs, qss, sss
    return rows


def flash_decode_bytes(B: int, H: int, N: int, D: int) -> int:
    """Algorithmic HBM bytes of one decode-attention call: fp16 K and V once, fp16 q in,
    fp32 out (the per-split partials stay in L2)."""
    return 2 * B * H * N * D * 2 + B * H * D * 2 + B * H * D * 4


def bench_flash_decode(dev, iters: int = 50) -> dict:
    """Split-KV decode attention (flash_decoding.flash_decoding). The reference's own benchmark
    shapes (flash_decoding.py:141-152: B=2, H=4, D=64, split 256) against its eager_decode on
    this GPU, plus one HBM-bound shape (B=8, H=32, N=8192, D=128: 1.07 GB of K/V, more than
    the Infinity Cache) with its roofline fraction."""
    import math

    import torch

    import _pk
    import flash_decoding

    def qkv(B, H, N, D, seed):
        q = torch.randn(B, H, 1, D, generator=_gen(seed)).half().to(dev)
        k = torch.randn(B, H, N, D, generator=_gen(seed + 1)).half().to(dev)
        v = torch.randn(B, H, N, D, generator=_gen(seed + 2)).half().to(dev)
        return q, k, v

    rows = []
    for N in (1024, 2048, 4096, 8192):
        q, k, v = qkv(2, 4, N, 64, 20)
        ms = GraphTimer(lambda i: flash_decoding.flash_decoding(q, k, v, split_size=256), iters, 2).run(reps=3)
        ms_eager = GraphTimer(lambda i: flash_decoding.eager_decode(q, k, v), iters, 2).run(reps=3)
        rows.append({"B": 2, "H": 4, "N": N, "D": 64, "split": 256, "us": round(ms * 1e3, 2),
                     "us_eager": round(ms_eager * 1e3, 2), "vs_eager": round(ms_eager / ms, 2)})
    B, H, N, D, split = 8, 32, 8192, 128, 256
    q, k, v = qkv(B, H, N, D, 30)
    q3 = q[:, :, 0]
    scale = 1.0 / math.sqrt(D)
    ms = GraphTimer(lambda i: _pk.flash_decode(q3, k, v, split, scale), 20, 2).run(reps=3)
    ms_eager = GraphTimer(lambda i: flash_decoding.eager_decode(q, k, v), 10, 2).run(reps=3)
    by = flash_decode_bytes(B, H, N, D)
    gbs = by / (ms * 1e-3) / 1e9
    return {"workload": "split_kv_decode_attention", "B": B, "H": H, "N": N, "D": D,
            "split": split, "launches": _pk.flash_decode_launches(B, H, N, D, split),
            "us": round(ms * 1e3, 2), "value": round(gbs, 1), "unit": "GB/s",
            "us_eager": round(ms_eager * 1e3, 2), "vs_eager": round(ms_eager / ms, 2),
            "dtype": "fp16 K/V, fp32 softmax and accumulate",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": by},
            "reference_bench_shapes": rows}


def bench_gptq(dev) -> dict:
    """GPTQ of one 4096 x 4096 layer (quantize.gptq_layer, quantize.py:71-115) from 2048
    calibration rows, 4-bit, groups of 128 rows: the Hessian GEMM, its inverse, the blocked
    column sweep (pk_gptq_block) and the GEMM updates between blocks, end to end."""
    import time

    import torch

    import quantize

    W = (torch.randn(4096, 4096, generator=_gen(40)) * 0.02).to(dev)
    X = torch.randn(2048, 4096, generator=_gen(41)).to(dev)
    quantize.gptq_layer(W, X, 4, group_size=128)
    best = float("inf")
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        quantize.gptq_layer(W, X, 4, group_size=128)
        torch.cuda.synchronize()
        best = min(best, time.perf_counter() - t0)
    return {"workload": "gptq_layer", "out": 4096, "in": 4096, "calib_rows": 2048, "bits": 4,
            "group_size": 128, "value": round(best * 1e3, 2), "unit": "ms per layer",
            "higher_is_better": False, "dtype": "fp32"}


def cpu_setup() -> dict:
    """Host threads for the CPU baseline: every core os.cpu_count() reports, capped by
    OMP_NUM_THREADS where the environment sets one (a shared GPU box's CPU share)."""
    import torch

    n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    torch.set_num_threads(n)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "affinity_cpus": len(os.sched_getaffinity(0)), "cpu_model": model}


def median_ms(fn, runs: int = 5):
    """One warm-up call, then the median of `runs` timed calls (ms) and the last result."""
    import statistics

    fn()
    ts, r = [], None
    for _ in range(runs):
        t0 = time.perf_counter()
        r = fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e3, r


def cpu_w4a16(a, qw, sc, y_gpu=None, group: int = 128, runs: int = 5) -> dict:
    """The reference's CPU path for one W4A16 call, in torch on the host: dequantize
    (unpack, multiply by the scales repeated over each group), then ``a.float() @ deq``
    (tests/test_gemm_int4.py:26). Dequant, matmul and the two together are each the median
    of `runs` after a warm-up. With `y_gpu`, also the GPU output's error against this one."""
    ac, qc, scc = a.cpu(), qw.cpu(), sc.cpu()
    M, K = ac.shape
    N = qc.shape[1] * 8
    t_deq, deq = median_ms(lambda: dequant_expr(qc, scc, group), runs)
    t_mm, y = median_ms(lambda: ac.float() @ deq, runs)
    t_tot, _ = median_ms(lambda: ac.float() @ dequant_expr(qc, scc, group), runs)
    row = {"M": M, "K": K, "N": N, "dequant_ms": round(t_deq, 3), "matmul_ms": round(t_mm, 3),
           "total_ms": round(t_tot, 3), "GFLOP/s": round(2.0 * M * N * K / (t_tot * 1e-3) / 1e9, 2),
           "GB/s": round(w4a16_bytes(M, K, N, group) / (t_tot * 1e-3) / 1e9, 3)}
    if y_gpu is not None:
        row["gpu_rel_fro_vs_cpu"] = float(f"{rel_fro(y_gpu.cpu(), y):.3e}")
    return row


def cpu_fp8(a8, b8, scale: float, runs: int = 5) -> dict:
    """The fp8 call on the host in torch (the reference has no CPU fp8 path; its test compares
    with the fp16 product, tests/test_gemm_fp8.py:24): e4m3 bytes to fp32, fp32 matmul,
    times the output scale; timed like cpu_w4a16."""
    ac, bc = a8.cpu(), b8.cpu()
    M, K = ac.shape
    N = bc.shape[1]
    t_deq, (af, bf) = median_ms(lambda: (ac.float(), bc.float()), runs)
    t_mm, _ = median_ms(lambda: (af @ bf) * scale, runs)
    t_tot, _ = median_ms(lambda: (ac.float() @ bc.float()) * scale, runs)
    return {"M": M, "K": K, "N": N, "dequant_ms": round(t_deq, 3), "matmul_ms": round(t_mm, 3),
            "total_ms": round(t_tot, 3),
            "GFLOP/s": round(2.0 * M * N * K / (t_tot * 1e-3) / 1e9, 2)}


def cpu_baseline_table(dev, gemv_inputs_dev) -> dict:
    """The four rows of the CPU baseline table: W4A16 16x1024x1024 (the reference's CPU
    plumbing config), 1x4096x11008 (the headline's own inputs), 2048x4096x4096 (the prefill
    line's seeds) and fp8 4096^3 (the fp8 line's seeds). Codes and scales come from this
    library's quantization on the GPU, copied to the host; only dequant + matmul is timed."""
    import torch

    import _pk
    import gemm_fp8
    import gemm_int4

    info = cpu_setup()
    rows = {}
    a = torch.randn(16, 1024, generator=_gen(0)).half().to(dev)
    w = (torch.randn(1024, 1024, generator=_gen(1)) * 0.02).half().to(dev)
    qw, sc = gemm_int4.quantize_int4_group(w, 128)
    y = _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16)
    rows["w4a16_16x1024x1024"] = cpu_w4a16(a, qw, sc, y)
    ag, qw, sc = gemv_inputs_dev
    y = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float16)
    rows["w4a16_1x4096x11008"] = cpu_w4a16(ag, qw, sc, y)
    a = torch.randn(2048, 4096, generator=_gen(2)).half().to(dev)
    w = (torch.randn(4096, 4096, generator=_gen(3)) * 0.02).half().to(dev)
    qw, sc = gemm_int4.quantize_int4_group(w, 128)
    y = _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16)
    rows["w4a16_2048x4096x4096"] = cpu_w4a16(a, qw, sc, y)
    a8, sa = gemm_fp8.quantize(torch.randn(4096, 4096, generator=_gen(4)).half().to(dev))
    b8, sb = gemm_fp8.quantize(torch.randn(4096, 4096, generator=_gen(5)).half().to(dev))
    rows["fp8_4096^3"] = cpu_fp8(a8, b8, 1.0 / (sa * sb))
    return {**info, "rows": rows}


def cpu_baseline_decode() -> dict:
    """The reference's single-query attention (eager_decode, flash_decoding.py:118-125) in
    torch on the host, on 8 of the 256 (b, h) pairs of the bench shape (N = 8192, D = 128);
    GB/s of fp16 K/V those pairs hold, median of 5 after a warm-up."""
    import torch

    import flash_decoding

    H, N, D = 8, 8192, 128
    q = torch.randn(1, H, 1, D, generator=_gen(30)).half()
    k = torch.randn(1, H, N, D, generator=_gen(31)).half()
    v = torch.randn(1, H, N, D, generator=_gen(32)).half()
    ms, _ = median_ms(lambda: flash_decoding.eager_decode(q, k, v))
    return {"value": round(flash_decode_bytes(1, H, N, D) / (ms * 1e-3) / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"eager_decode on 1x{H}x{N}x{D} (8 of the 256 heads): median of 5, {ms:.2f} ms"}


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return int(max((p.get("num_threads", 1) for p in threadpool_info()
                        if p.get("user_api") == "blas"), default=1))
    except Exception:  # threadpoolctl missing: numpy's BLAS default
        return os.cpu_count() or 1


def cpu_baseline_gptq(seconds: float) -> dict:
    """The reference's gptq_layer column loop on the host through the oracle (fp32, one column
    at a time, quantize.py:71-115), on a 1024 x 1024 layer (a 4096 x 4096 one is ~64x the
    work); milliseconds per 1024 x 1024 layer."""
    import numpy as np
    import torch

    import oracle

    W = (torch.randn(1024, 1024, generator=_gen(42)) * 0.02).numpy()
    X = torch.randn(512, 1024, generator=_gen(43)).numpy()
    t0 = time.perf_counter()
    reps = 0
    while True:
        q = oracle.gptq_layer(W, X, 4, group_size=128)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(el / reps * 1e3, 1), "unit": "ms per 1024x1024 layer", "cores": _blas_threads(),
            "kind": "port", "sample": f"{reps} layers of 1024x1024 (512 calibration rows, group 128) in {el:.1f} s",
            "check": float(np.abs(q).sum())}


TRAFFIC_PROFILE = ROOT / "profiles" / "w4a16_gemv_decode_traffic.md"
COPY_PROBE_BYTES = 256 << 20


def traffic_probe(dev) -> int:
    """Short run for the rocprofv3 --pmc passes: 50 launches of the headline's kernel (the
    strip GEMV, the whole op) on rotating weights, then 10 device copies of COPY_PROBE_BYTES
    (the calibration kernel: it must read and write exactly that many bytes)."""
    import torch

    import _pk

    M, K, N = 1, 4096, 11008
    a, w, qws, scs = gemv_inputs(M, K, N, N_ROTATE, dev)
    qss, sss = strip_copies(qws, scs)
    ag = a.to(dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    for i in range(50):
        _pk.w4a16_gemm_strips(ag, qss[i % N_ROTATE], sss[i % N_ROTATE], 128, 1.0,
                              torch.float16, out=out)
    torch.cuda.synchronize()
    src = torch.empty(COPY_PROBE_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"traffic probe done: launches=50 copy_bytes={COPY_PROBE_BYTES}", flush=True)
    return 0


def mfma_probe(dev) -> int:
    """Eager launches (no graph) of the GEMMs whose MFMA utilisation is read with rocprofv3
    --pmc: W4A16 and fp8 GEMMs (fp16 out) at 2048x4096x4096 and 4096^3, 5 calls each."""
    import torch

    import _pk
    import gemm_fp8
    import gemm_int4

    for M in (2048, 4096):
        a = torch.randn(M, 4096, generator=_gen(2)).half().to(dev)
        w = (torch.randn(4096, 4096, generator=_gen(3)) * 0.02).half().to(dev)
        qw, sc = gemm_int4.quantize_int4_group(w, 128)
        out = torch.empty((M, 4096), dtype=torch.float16, device=dev)
        for _ in range(5):
            _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16, out=out)
    for M in (2048, 4096):
        a = torch.randn(M, 4096, generator=_gen(4)).half().to(dev)
        b = torch.randn(4096, 4096, generator=_gen(5)).half().to(dev)
        a8, sa = gemm_fp8.quantize(a)
        b8, sb = gemm_fp8.quantize(b)
        out = torch.empty((M, 4096), dtype=torch.float16, device=dev)
        for _ in range(5):
            _pk.fp8_gemm(a8, b8, 1.0 / (sa * sb), torch.float16, out=out)
    torch.cuda.synchronize()
    print("mfma probe done", flush=True)
    return 0


def mfma_ceiling(dev) -> dict:
    """What the matrix cores sustain with no memory traffic (pkb_mfma_probe): 256 workgroups of
    8 waves issuing independent MFMAs on constant or pseudo-random operands, timed with HIP
    events on the launch stream, against MI355X's published dense peaks."""
    import torch

    import _probes

    grid, iters = 256, 4000
    out = torch.empty(grid * 512, dtype=torch.float32, device=dev)
    rows = []
    for fp8, peak in ((True, MFMA_F8_PEAK_TFLOPS), (False, MFMA_F16_PEAK_TFLOPS)):
        flops = grid * 8 * iters * 8 * (131072 if fp8 else 32768)
        for random in (False, True):
            _probes.mfma_probe(fp8, random, grid, iters, out)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                _probes.mfma_probe(fp8, random, grid, iters, out)
            e1.record()
            e1.synchronize()
            tf = 5 * flops / (e0.elapsed_time(e1) * 1e-3) / 1e12
            rows.append({"dtype": "e4m3" if fp8 else "fp16", "operands": "random" if random else "constant",
                         "TFLOP/s": round(tf, 1), "frac_of_dense_peak": round(tf / peak, 4)})
    return {"mfma_ceiling": rows, "grid": grid, "waves_per_workgroup": 8, "mfmas_per_wave": iters * 8}


def vendor_compare(dev) -> dict:
    """This library's GEMMs beside the vendor library's (hipBLASLt through torch) on the same
    GPU and inputs: fp16 GEMMs with B row-major (NN) and transposed (NT) against the W4A16
    GEMM, torch._scaled_mm against the fp8 GEMM; graph-timed like the bench lines."""
    import torch

    import _pk
    import gemm_fp8
    import gemm_int4

    rows = []
    for (M, N, K) in ((2048, 4096, 4096), (4096, 4096, 4096), (8192, 8192, 8192)):
        a = torch.randn(M, K, generator=_gen(4)).half().to(dev)
        b = torch.randn(K, N, generator=_gen(5)).half().to(dev)
        bt = b.t().contiguous()
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        w = (torch.randn(K, N, generator=_gen(6)) * 0.02).half().to(dev)
        qw, sc = gemm_int4.quantize_int4_group(w, 128)
        qt = _pk.tile_weights(qw)
        a8, sa = gemm_fp8.quantize(a)
        b8, sb = gemm_fp8.quantize(b)
        b8t = b8.t().contiguous().t()
        one = torch.tensor(1.0, device=dev)

        def tf(fn):
            ms = GraphTimer(fn, 20, 2).run(reps=3)
            return round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)

        rows.append({"M": M, "N": N, "K": K,
                     "hipblaslt_f16_nn": tf(lambda i: torch.matmul(a, b, out=out)),
                     "hipblaslt_f16_nt": tf(lambda i: torch.matmul(a, bt.t(), out=out)),
                     "pk_w4a16_g128": tf(lambda i: _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16, out=out)),
                     "pk_w4a16_g128_blocks": tf(lambda i: _pk.w4a16_gemm(a, qt, sc, 128, 1.0, torch.float16,
                                                                       out=out, tiled=True)),
                     "hipblaslt_fp8_scaled_mm": tf(lambda i: torch._scaled_mm(a8, b8t, one, one, out_dtype=torch.float16)),
                     "pk_fp8": tf(lambda i: _pk.fp8_gemm(a8, b8, 1.0, torch.float16, out=out)),
                     "unit": "TFLOP/s"})
        del a, b, bt, out, w, qw, qt, sc, a8, b8, b8t
    return {"vendor_compare": rows}


def hbm_ceiling(dev) -> dict:
    """What one launch that only reads achieves (pkb_read_probe), timed like the GEMV: a graph of
    back-to-back launches over rotating buffers (more than the 256 MB Infinity Cache). At the
    GEMV's 23,279,104 bytes it is the ceiling the headline's fraction is read against; 256 MiB
    and 1 GiB show the asymptotic rate."""
    import torch

    import _probes

    rows = []
    for nbytes, nrot, steps in ((23279104, N_ROTATE, 2000), (256 << 20, 4, 40), (1 << 30, 2, 20)):
        bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(nrot)]
        best = None
        for grid in (256, 512, 768, 1024, 2048, 4096):
            out = torch.empty(grid, dtype=torch.int32, device=dev)
            ms = GraphTimer(lambda i: _probes.read_probe(bufs[i % nrot], out, grid), steps, 2).run(reps=3)
            tbs = nbytes / (ms * 1e-3) / 1e12
            if best is None or tbs > best["TB/s"]:
                best = {"bytes": nbytes, "grid": grid, "us": round(ms * 1e3, 3), "TB/s": round(tbs, 3),
                        "frac_of_8TBs": round(tbs / (HBM_PEAK_GBS / 1000), 4)}
        rows.append(best)
        del bufs
    # The headline GEMV's own read pattern (688 strips of 32 KB, one workgroup of 8 waves per
    # strip, U blocks of 1 KB per wave) with no other work, over 40 rotating copies of the
    # packed weights (22,544,384 B; the GEMV also reads 704,512 B of scales and the activations).
    strips, strip_bytes = 11008 // 16, 4096 // 2 * 16
    nbytes = strips * strip_bytes
    bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(N_ROTATE)]
    out = torch.empty(64 * -(-strips // 8), dtype=torch.int32, device=dev)
    pattern = []
    for u in (2, 4, 8):
        ms = GraphTimer(lambda i: _probes.strip_read_probe(bufs[i % N_ROTATE], strips, u, out),
                        2000, 2).run(reps=3, preroll=PREROLL)
        tbs = nbytes / (ms * 1e-3) / 1e12
        pattern.append({"bytes": nbytes, "blocks_per_wave": u, "us": round(ms * 1e3, 3),
                        "TB/s": round(tbs, 3), "frac_of_8TBs": round(tbs / (HBM_PEAK_GBS / 1000), 4)})
    del bufs
    return {"hbm_read_ceiling": rows, "strip_read_pattern": pattern}


def measured_traffic():
    """HBM bytes per slice-kernel launch from the committed --pmc summary, or None."""
    import re

    try:
        m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", TRAFFIC_PROFILE.read_text())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true", help="skip the GEMM lines")
    ap.add_argument("--no-sweep", action="store_true", help="skip the Llama-3-8B layer sweep")
    ap.add_argument("--no-row-layout", action="store_true",
                    help="time the W4A16 lines on QuantLinear's block layout only (for kernel traces)")
    ap.add_argument("--only", choices=("gemv", "prefill", "gemm4096", "fp8", "fp8_2048",
                                       "flash_decode", "gptq", "sweep"),
                    help="run one secondary workload alone and print its JSON (for profiling)")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only run eager GEMM calls for rocprofv3 --pmc MFMA utilisation")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only measure the matrix cores' sustained rate with no memory traffic")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only measure what a read-only launch of the GEMV's bytes achieves")
    ap.add_argument("--vendor", action="store_true",
                    help="only time hipBLASLt's fp16 / fp8 GEMMs beside this library's")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the short kernel + copy sequence profiled with --pmc")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the kernel is "
              "benchmarked at its single-GPU shape, one GPU's share of a sharded layer).",
              file=sys.stderr)
        return 2

    import torch

    import _pk

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    _pk.lib()
    dev = torch.device("cuda", 0)
    global ROW_LAYOUT
    ROW_LAYOUT = not args.no_row_layout
    if args.traffic_probe:
        return traffic_probe(dev)
    if args.mfma_probe:
        return mfma_probe(dev)
    if args.mfma_ceiling:
        print(json.dumps(mfma_ceiling(dev)), flush=True)
        return 0
    if args.vendor:
        print(json.dumps(vendor_compare(dev)), flush=True)
        return 0
    if args.hbm_ceiling:
        print(json.dumps(hbm_ceiling(dev)), flush=True)
        return 0
    if args.only == "gemv":  # the headline call alone: its timing, no split sweep
        args.split_sweep = False
        g = bench_gemv(args, dev)
        g.pop("inputs")
        g["GB/s"] = round(g["bytes"] / (g["ms_per_step"] * 1e-3) / 1e9, 1)
        print(json.dumps(g), flush=True)
        return 0
    if args.only:
        fn = {"prefill": bench_prefill, "gemm4096": lambda d: bench_prefill(d, M=4096),
              "fp8": bench_fp8, "fp8_2048": lambda d: bench_fp8(d, M=2048),
              "flash_decode": bench_flash_decode, "gptq": bench_gptq,
              "sweep": lambda d: {"llama3_8b_sweep": bench_llama_sweep(d)}}[args.only]
        print(json.dumps(fn(dev)), flush=True)
        return 0

    g = bench_gemv(args, dev)
    gbs = g["bytes"] / (g["ms_per_step"] * 1e-3) / 1e9
    kern_gbs = g["bytes"] / (g["ms_kernel"] * 1e-3) / 1e9
    result = {
        "metric": "W4A16 GEMV HBM GB/s (M=1, 4096x11008)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 5),
        "ms_per_step_best": round(g["ms_per_step_best"], 5),
        "ms_per_step_graph": round(g["ms_graph"], 5),
        "ms_per_step_event_packets": round(g["ms_markers"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights (group 128, fp16 scales) x fp16 activations, fp32 accumulate",
        "data": "synthetic: seeded CPU generator, A ~ N(0,1) fp16, W ~ N(0,0.02) int4-quantized "
                "(group 128), the codes in QuantLinear's decode layout (16-column strips, each "
                "strip's K rows contiguous); "
                f"{N_ROTATE} copies of the packed weights and scales rotated "
                f"({N_ROTATE * g['bytes'] / 1e6:.0f} MB > 2x the 256 MB Infinity Cache): warm-up "
                f"reads copies 0..{args.warmup - 1}, the timed {g['steps_timed']} calls start "
                f"at copy {max(args.warmup, 1) % N_ROTATE}, each timed repetition after "
                f"{PREROLL} untimed calls on the copies before it, median of 5 repetitions",
        "config": {"workload": "w4a16_decode_gemv", "M": g["M"], "K": g["K"], "N": g["N"],
                   "group_size": 128, "split_k": 1, "out_dtype": "fp16",
                   "weights": "16-column strips (QuantLinear's decode copy, pk_w4a16_gemm_strips): "
                              "one workgroup per strip over the whole of K, one launch",
                   "blocks_layout_GBs": (round(g["bytes"] / (g["ms_blocks"] * 1e-3) / 1e9, 1)
                                         if g["ms_blocks"] else None),
                   "blocks_layout_plan": g["blocks_layout_plan"],
                   "row_layout_GBs": (round(g["bytes"] / (g["ms_rows"] * 1e-3) / 1e9, 1)
                                      if g["ms_rows"] else None),
                   "split_k_sweep_GBs": g["split_sweep_GBs"],
                   "split_k_sweep_weights": "row layout (pk_w4a16_gemm; splits 1, 2, 4 run the "
                                            "VALU GEMV, which reads rows only)"},
        "steps_timed": g["steps_timed"],
        "check": g["check"],
        "host": g["host"],
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": KERNEL_NAMES[g["kernel_id"]] + " (one launch: the whole op)",
                     "kernel_us": round(g["ms_kernel"] * 1e3, 3),
                     "kernel_us_single_launch_events": round(g["ms_kernel_events"] * 1e3, 3),
                     "bytes_per_launch": g["bytes"]},
    }
    if not args.no_secondary:
        result["secondary"] = [bench_prefill(dev), bench_prefill(dev, M=4096), bench_fp8(dev),
                               bench_fp8(dev, M=2048), bench_flash_decode(dev), bench_gptq(dev)]
    if not args.no_sweep:
        result["llama3_8b_sweep"] = bench_llama_sweep(dev)
    if not args.no_cpu_baseline:
        table = cpu_baseline_table(dev, g["inputs"])
        head = table["rows"]["w4a16_1x4096x11008"]
        result["cpu_baseline"] = {
            "value": head["GB/s"], "unit": "GB/s", "cores": table["torch_threads"],
            "kind": "reference",
            "sample": "the reference's own CPU path, its tests' torch expression (unpack + group "
                      "dequant, then a.float() @ deq, tests/test_gemm_int4.py:26) run by torch on "
                      "the host, on the headline's own inputs: median of 5 after a warm-up, "
                      f"dequant {head['dequant_ms']} ms + matmul {head['matmul_ms']} ms, "
                      f"together {head['total_ms']} ms",
            "ms_per_step": head["total_ms"], "table": table}
        if not args.no_secondary:  # the reference's CPU path beside the GEMM lines too
            for entry in result["secondary"]:
                if entry["workload"] == "w4a16_prefill_gemm":
                    r = table["rows"]["w4a16_2048x4096x4096"]
                    entry["cpu_baseline"] = {"value": round(r["GFLOP/s"] / 1e3, 4), "unit": "TFLOP/s",
                                             "cores": table["torch_threads"], "kind": "reference",
                                             "sample": "the reference's test expression "
                                                       "(tests/test_gemm_int4.py:26) in torch on "
                                                       "the host: dequant + fp32 matmul, median "
                                                       f"of 5: {r['total_ms']} ms"}
                elif entry["workload"] == "fp8_e4m3_gemm":
                    r = table["rows"]["fp8_4096^3"]
                    entry["cpu_baseline"] = {"value": round(r["GFLOP/s"] / 1e3, 4), "unit": "TFLOP/s",
                                             "cores": table["torch_threads"], "kind": "port",
                                             "sample": "the fp8 call's own semantics in torch on "
                                                       "the host (the reference has no CPU fp8 "
                                                       "path): e4m3->fp32, fp32 matmul, times the "
                                                       f"output scale, median of 5: {r['total_ms']} ms"}
                elif entry["workload"] == "split_kv_decode_attention":
                    entry["cpu_baseline"] = cpu_baseline_decode()
                elif entry["workload"] == "gptq_layer":
                    entry["cpu_baseline"] = cpu_baseline_gptq(args.cpu_seconds / 6)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
