#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (one JSON line on stdout).

Headline workload: W4A16 decode GEMV, M=1, K=4096, N=11008, int4 group
128 with fp16 scales, fp16 activations N(0,1), weights N(0, 0.02), seeded CPU generator.
A "step" is one ``w4a16_gemm`` call over one activation row. ``value`` is the whole-op HBM
throughput (algorithmic bytes / step time), inputs resident in HBM, with 40 distinct weight
buffers rotated (932 MB, more than twice the 256 MB Infinity Cache) so every step streams
its weights from HBM.

Timing: W eager warmup steps, then exactly K steps captured in one HIP graph and replayed
once between HIP events (bracketed by device synchronisation). On MI355X the GEMV's split-K
slices add up in L2 inside the one kernel, so the op is the dominant kernel and the
roofline fraction uses its time; where a second (reduce) launch is needed, the slice kernel
is timed on its own through ``pk_w4a16_gemm_partials``. The same JSON line carries the split-K sweep of the config, the
W4A16 GEMM (prefill 2048x4096x4096 and 4096^3) and fp8 GEMM (4096^3) throughputs the
metric also names, split-KV decode attention (the reference's benchmark shapes against its eager path,
and one HBM-bound shape), and the reference's CPU path (dequantize + matmul, numpy oracle) on
a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--sweep]
       python bench.py --only {prefill,gemm4096,fp8,flash_decode,gptq}   (one secondary line)
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
KERNEL_NAMES = {1: "w4a16_gemv_mfma_kernel", 2: "gemm_v3_f16_kernel", 3: "w4a16_skinny_kernel"}


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
    """Capture `steps` calls of fn(i) in one HIP graph on a private stream; time a replay."""

    def __init__(self, fn, steps: int, warmup: int):
        import torch

        self.stream = torch.cuda.Stream()
        self.steps = steps
        with torch.cuda.stream(self.stream):
            for i in range(max(warmup, 1)):
                fn(i)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            for i in range(steps):
                fn(i)
        torch.cuda.synchronize()

    def run(self, reps: int = 1) -> float:
        """Milliseconds per step (best of `reps` replays)."""
        import torch

        best = float("inf")
        with torch.cuda.stream(self.stream):
            for _ in range(reps):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record(self.stream)
                self.graph.replay()
                e1.record(self.stream)
                torch.cuda.synchronize()
                best = min(best, e0.elapsed_time(e1) / self.steps)
        return best


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


def bench_gemv(args, dev) -> dict:
    import torch

    import _pk

    M, K, N = 1, 4096, 11008
    a, w, qws, scs = gemv_inputs(M, K, N, N_ROTATE, dev)
    ag = a.to(dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    nbytes = w4a16_bytes(M, K, N)
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)

    def step(i):
        _pk.w4a16_gemm(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 1.0, torch.float16,
                       split_k=0, out=out)

    ms = GraphTimer(step, args.steps, args.warmup).run()
    launches = _pk.w4a16_launches(M, N, K, 128, 0)

    # The dominant kernel's average launch: K launches back to back in one graph, HIP events
    # around the replay on the launch stream (agrees with rocprof's kernel-trace average);
    # single launches bracketed by their own events read ~1.5 us longer (event overhead).
    # With the slices added in L2 the op is that one kernel; otherwise time the slice kernel
    # alone (it writes the fp32 partials that a second launch adds).
    if launches == 1:
        ms_kernel = ms
        ms_kernel_events = per_launch_ms(step, min(args.steps, 500))
    else:
        parts = torch.empty((split, M, N), dtype=torch.float32, device=dev)

        def step_partials(i):
            _pk.w4a16_gemm_partials(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 0, parts)

        ms_kernel = GraphTimer(step_partials, args.steps, args.warmup).run()
        ms_kernel_events = per_launch_ms(step_partials, min(args.steps, 500))

    sweep = {}
    for s in (1, 2, 4, 8, 16):
        def step_s(i, s=s):
            _pk.w4a16_gemm(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 1.0, torch.float16,
                           split_k=s, out=out)

        ms_s = GraphTimer(step_s, min(args.steps, 400), 2).run()
        sweep[str(s)] = round(nbytes / (ms_s * 1e-3) / 1e9, 1)
    return {
        "M": M, "K": K, "N": N, "split": split, "kernel_id": kid, "launches": launches,
        "bytes": nbytes,
        "ms_per_step": ms, "ms_kernel": ms_kernel, "ms_kernel_events": ms_kernel_events,
        "split_sweep_GBs": sweep,
        "inputs": (a, w),
    }


def bench_prefill(dev, iters: int = 50, M: int = 2048) -> dict:
    """W4A16 GEMM (group 128, fp16 out) at M x 4096 x 4096: M = 2048 is the prefill config,
    M = 4096 the 4096^3 shape the metric also names."""
    import torch

    import _pk
    import gemm_int4

    K, N = 4096, 4096
    a = torch.randn(M, K, generator=_gen(2)).half().to(dev)
    w = (torch.randn(K, N, generator=_gen(3)) * 0.02).half().to(dev)
    qw, sc = gemm_int4.quantize_int4_group(w, 128)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    ms = GraphTimer(lambda i: _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16, out=out),
                    iters, 2).run(reps=5)
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"workload": "w4a16_prefill_gemm" if M == 2048 else "w4a16_gemm_4096^3", "M": M, "K": K,
            "N": N, "ms": round(ms, 4),
            "value": round(tflops, 1), "unit": "TFLOP/s", "dtype": "fp16 MFMA, fp32 acc",
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}}


def bench_fp8(dev, iters: int = 50) -> dict:
    import torch

    import _pk
    import gemm_fp8

    M = N = K = 4096
    a = torch.randn(M, K, generator=_gen(4)).half().to(dev)
    b = torch.randn(K, N, generator=_gen(5)).half().to(dev)
    a8, sa = gemm_fp8.quantize(a)
    b8, sb = gemm_fp8.quantize(b)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    scale = 1.0 / (sa * sb)
    ms = GraphTimer(lambda i: _pk.fp8_gemm(a8, b8, scale, torch.float16, out=out), iters, 2).run(reps=5)
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    # accuracy of this very output vs fp32 (the reference's own metric)
    ref = a.float() @ b.float()
    rel = (torch.linalg.norm(out.float() - ref) / torch.linalg.norm(ref)).item()
    return {"workload": "fp8_e4m3_gemm", "M": M, "K": K, "N": N, "ms": round(ms, 4),
            "value": round(tflops, 1), "unit": "TFLOP/s", "dtype": "e4m3 MFMA, fp32 acc",
            "rel_fro_vs_fp32": round(rel, 5),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1),
                         "peak": MFMA_F8_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_F8_PEAK_TFLOPS, 4)}}


def bench_llama_sweep(dev, iters: int = 50) -> list:
    import torch

    import _pk
    import gemm_int4

    rows = []
    for name, K, N in (("qkv", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up", 4096, 14336),
                       ("down", 14336, 4096)):
        w = (torch.randn(K, N, generator=_gen(6)) * 0.02).half().to(dev)
        qw, sc = gemm_int4.quantize_int4_group(w, 128)
        nrot = max(2, min(N_ROTATE, (600 << 20) // (K * N // 2) + 1))
        qws = [qw] + [qw.clone() for _ in range(nrot - 1)]
        scs = [sc] + [sc.clone() for _ in range(nrot - 1)]
        for M in (1, 8, 32, 128):
            a = torch.randn(M, K, generator=_gen(7)).half().to(dev)
            out = torch.empty((M, N), dtype=torch.float16, device=dev)
            ms = GraphTimer(lambda i: _pk.w4a16_gemm(a, qws[i % nrot], scs[i % nrot], 128, 1.0,
                                                     torch.float16, out=out), iters, 2).run()
            by = w4a16_bytes(M, K, N)
            flop = 2.0 * M * N * K
            # the applicable roof: the slower of streaming the bytes and issuing the MFMAs
            t_hbm = by / (HBM_PEAK_GBS * 1e9)
            t_mfma = flop / (MFMA_F16_PEAK_TFLOPS * 1e12)
            rows.append({"layer": name, "M": M, "K": K, "N": N, "us": round(ms * 1e3, 2),
                         "GB/s": round(by / (ms * 1e-3) / 1e9, 1),
                         "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 2),
                         "bound": "hbm" if t_hbm >= t_mfma else "mfma",
                         "frac": round(max(t_hbm, t_mfma) / (ms * 1e-3), 4)})
        del qws, scs
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


def cpu_baseline(a, w, seconds: float) -> dict:
    """The reference's CPU path for the same GEMV (dequantize with the group scales, then an
    fp32 matmul), run through the numpy oracle on the host cores for a bounded sample."""
    import numpy as np

    import oracle

    threads = _blas_threads()
    an = a.numpy()
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, 128)
    packed = oracle.pack_int4_n(codes)
    K, N = codes.shape
    nbytes = w4a16_bytes(an.shape[0], K, N)
    t0 = time.perf_counter()
    reps = 0
    while True:
        q = oracle.unpack_int4_n(packed)         # dequantize: unpack ...
        y = oracle.w4a16_ref(an, q, s16, 128)    # ... scale and fp32 matmul
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(nbytes * reps / el / 1e9, 3), "unit": "GB/s", "cores": int(threads),
            "kind": "port", "sample": f"{reps} full GEMVs (M=1, K=4096, N=11008: unpack + "
            f"group dequant + fp32 matmul) in {el:.1f} s", "ms_per_step": round(el / reps * 1e3, 2),
            "check": float(np.abs(y).sum())}


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return int(max((p.get("num_threads", 1) for p in threadpool_info()
                        if p.get("user_api") == "blas"), default=1))
    except Exception:  # threadpoolctl missing: numpy's BLAS default
        return os.cpu_count() or 1


def cpu_baseline_gemm(kind: str, seconds: float) -> dict:
    """The reference's CPU path for the GEMM lines, full size, through the numpy oracle:
    W4A16 2048x4096x4096 = unpack + group dequantize + fp32 matmul of the same seeded inputs
    as bench_prefill; fp8 4096^3 = the e4m3 bytes decoded to fp32, fp32 matmul, out_scale
    (the test-path oracle, tests/test_gemm_fp8.py:24). Repeated for about `seconds`."""
    import numpy as np
    import torch

    import oracle

    if kind == "w4a16":
        M, K, N = 2048, 4096, 4096
        a = torch.randn(M, K, generator=_gen(2)).half().numpy()
        w = (torch.randn(K, N, generator=_gen(3)) * 0.02).half().numpy()
        codes, _, s16 = oracle.rtn_group_codes(w, 4, 128)
        packed = oracle.pack_int4_n(codes)

        def run():
            return oracle.w4a16_ref(a, oracle.unpack_int4_n(packed), s16, 128)
    else:
        M = N = K = 4096
        a8, sa = oracle.fp8_quantize(torch.randn(M, K, generator=_gen(4)).half().numpy())
        b8, sb = oracle.fp8_quantize(torch.randn(K, N, generator=_gen(5)).half().numpy())

        def run():
            return oracle.fp8_gemm_ref(a8, sa, b8, sb)
    t0 = time.perf_counter()
    reps = 0
    while True:
        y = run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    flop = 2.0 * M * N * K
    return {"value": round(flop * reps / el / 1e12, 4), "unit": "TFLOP/s", "cores": _blas_threads(),
            "kind": "port", "sample": f"{reps} full {M}x{K}x{N} products ({'unpack + group dequant' if kind == 'w4a16' else 'e4m3 decode'} + fp32 matmul) in {el:.1f} s",
            "ms_per_step": round(el / reps * 1e3, 1), "check": float(np.abs(y).sum())}


def cpu_baseline_decode(seconds: float) -> dict:
    """The reference's single-query attention (eager_decode, flash_decoding.py:126-133) on the
    host through the float64 oracle, on 8 of the 256 (b, h) pairs of the bench shape
    (N = 8192, D = 128); GB/s of fp16 K/V those pairs hold."""
    import numpy as np
    import torch

    import oracle

    H, N, D = 8, 8192, 128
    q = torch.randn(1, H, 1, D, generator=_gen(30)).half().numpy()
    k = torch.randn(1, H, N, D, generator=_gen(31)).half().numpy()
    v = torch.randn(1, H, N, D, generator=_gen(32)).half().numpy()
    t0 = time.perf_counter()
    reps = 0
    while True:
        y = oracle.decode_attention_ref(q, k, v)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(flash_decode_bytes(1, H, N, D) * reps / el / 1e9, 3), "unit": "GB/s",
            "cores": _blas_threads(), "kind": "port",
            "sample": f"{reps} calls of 1x{H}x{N}x{D} (8 of the 256 heads) in {el:.1f} s",
            "check": float(np.abs(y).sum())}


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
    """Short run for the rocprofv3 --pmc passes: 50 launches of the GEMV's dominant kernel
    on rotating weights (the whole op when its slices add up in L2, else the slice kernel),
    then 10 device copies of COPY_PROBE_BYTES (the calibration kernel: it must read and
    write exactly that many bytes)."""
    import torch

    import _pk

    M, K, N = 1, 4096, 11008
    a, w, qws, scs = gemv_inputs(M, K, N, N_ROTATE, dev)
    ag = a.to(dev)
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)
    if _pk.w4a16_launches(M, N, K, 128, 0) == 1:
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        for i in range(50):
            _pk.w4a16_gemm(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 1.0, torch.float16,
                           out=out)
    else:
        parts = torch.empty((split, M, N), dtype=torch.float32, device=dev)
        for i in range(50):
            _pk.w4a16_gemm_partials(ag, qws[i % N_ROTATE], scs[i % N_ROTATE], 128, 0, parts)
    torch.cuda.synchronize()
    src = torch.empty(COPY_PROBE_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"traffic probe done: split={split} copy_bytes={COPY_PROBE_BYTES}", flush=True)
    return 0


def mfma_probe(dev) -> int:
    """Eager launches (no graph) of the GEMMs whose MFMA utilisation is read with rocprofv3
    --pmc: W4A16 prefill 2048x4096x4096 and 4096^3, fp8 4096^3 (fp16 out), 5 calls each."""
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
    a = torch.randn(4096, 4096, generator=_gen(4)).half().to(dev)
    b = torch.randn(4096, 4096, generator=_gen(5)).half().to(dev)
    a8, sa = gemm_fp8.quantize(a)
    b8, sb = gemm_fp8.quantize(b)
    out = torch.empty((4096, 4096), dtype=torch.float16, device=dev)
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
                     "hipblaslt_fp8_scaled_mm": tf(lambda i: torch._scaled_mm(a8, b8t, one, one, out_dtype=torch.float16)),
                     "pk_fp8": tf(lambda i: _pk.fp8_gemm(a8, b8, 1.0, torch.float16, out=out)),
                     "unit": "TFLOP/s"})
        del a, b, bt, out, w, qw, sc, a8, b8, b8t
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
    return {"hbm_read_ceiling": rows}


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
    ap.add_argument("--sweep", action="store_true", help="add the Llama-3-8B layer sweep")
    ap.add_argument("--only", choices=("prefill", "gemm4096", "fp8", "flash_decode", "gptq"),
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
              "benchmarked at its single-GPU shape; see the sharding notes in DESIGN.md).",
              file=sys.stderr)
        return 2

    import torch

    import _pk

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    _pk.lib()
    dev = torch.device("cuda", 0)
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
    if args.only:
        fn = {"prefill": bench_prefill, "gemm4096": lambda d: bench_prefill(d, M=4096),
              "fp8": bench_fp8, "flash_decode": bench_flash_decode, "gptq": bench_gptq}[args.only]
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
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights (group 128, fp16 scales) x fp16 activations, fp32 accumulate",
        "data": "synthetic: seeded CPU generator, A ~ N(0,1) fp16, W ~ N(0,0.02) int4-quantized; "
                f"{N_ROTATE} rotating weight copies (> 2x Infinity Cache)",
        "config": {"workload": "w4a16_decode_gemv", "M": g["M"], "K": g["K"], "N": g["N"],
                   "group_size": 128, "split_k": g["split"], "out_dtype": "fp16",
                   "split_k_sweep_GBs": g["split_sweep_GBs"]},
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": KERNEL_NAMES.get(g["kernel_id"], "?") + (
                         " (split-K slices added in L2: the whole op)" if g["launches"] == 1
                         else " (split-K slices)"),
                     "kernel_us": round(g["ms_kernel"] * 1e3, 3),
                     "kernel_us_single_launch_events": round(g["ms_kernel_events"] * 1e3, 3),
                     "bytes_per_launch": g["bytes"]},
    }
    if not args.no_secondary:
        result["secondary"] = [bench_prefill(dev), bench_prefill(dev, M=4096), bench_fp8(dev),
                               bench_flash_decode(dev), bench_gptq(dev)]
    if args.sweep:
        result["llama3_8b_sweep"] = bench_llama_sweep(dev)
    if not args.no_cpu_baseline:
        a, w = g["inputs"]
        result["cpu_baseline"] = cpu_baseline(a, w, args.cpu_seconds)
        if not args.no_secondary:  # the reference's CPU path beside the GEMM lines too
            for entry in result["secondary"]:
                if entry["workload"] == "w4a16_prefill_gemm":
                    entry["cpu_baseline"] = cpu_baseline_gemm("w4a16", args.cpu_seconds / 3)
                elif entry["workload"] == "fp8_e4m3_gemm":
                    entry["cpu_baseline"] = cpu_baseline_gemm("fp8", args.cpu_seconds / 3)
                elif entry["workload"] == "split_kv_decode_attention":
                    entry["cpu_baseline"] = cpu_baseline_decode(args.cpu_seconds / 6)
                elif entry["workload"] == "gptq_layer":
                    entry["cpu_baseline"] = cpu_baseline_gptq(args.cpu_seconds / 6)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
