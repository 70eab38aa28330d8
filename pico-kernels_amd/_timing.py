"""Timing helper of the drop-in modules' ``bench()`` functions (the role ``triton.testing.do_bench``
plays in the reference's modules, e.g. gemm_int4.py:121-122): the median of HIP-event timed
calls on the current stream after a warm-up, in milliseconds."""

from __future__ import annotations

import statistics

import torch


def do_bench(fn, warmup_ms: float = 25.0, rep_ms: float = 100.0) -> float:
    """Median milliseconds of ``fn()``: calls for about ``warmup_ms``, then about ``rep_ms`` of
    individually event-timed calls (at least 5)."""
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        fn()
    e1.record()
    e1.synchronize()
    est = max(e0.elapsed_time(e1) / 5, 1e-3)
    for _ in range(max(1, int(warmup_ms / est))):
        fn()
    n = max(5, int(rep_ms / est))
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for s, e in zip(starts, ends):
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return statistics.median(s.elapsed_time(e) for s, e in zip(starts, ends))


def banner() -> str:
    import _pk

    return (f"device: {torch.cuda.get_device_name(0)} | hip {torch.version.hip} | "
            f"{_pk.LIB_PATH.name} v{_pk.lib().pk_version()}")
