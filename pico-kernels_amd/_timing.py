"""Timing and self-check harness of the drop-in modules (``gemm_int4``, ``gemm_fp8``,
``gemm_splitk``, ``flash_decoding``).

The reference gives each of those modules a ``check_correctness()`` / ``bench()`` pair and a
``__main__`` that prints them (e.g. gemm_int4.py:95-137, timed with
``triton.testing.do_bench``); its top-level bench.py runs every module as a subprocess and
prints what it writes (bench.py:29-53). Here each module only *declares* its self-checks and
its timing rows as data (:class:`Check`, :class:`Row`); this one harness runs them, times
every candidate with HIP events (:func:`do_bench`) and prints one ``key=value`` line per check
or row, so any caller that captures stdout reads it and a test can parse it.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass, field
from typing import Callable

import torch


def do_bench(fn, warmup_ms: float = 25.0, rep_ms: float = 100.0) -> float:
    """Median milliseconds of ``fn()`` on the current stream: calls for about ``warmup_ms``,
    then about ``rep_ms`` of individually event-timed calls (at least 5)."""
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

    return (f"device={torch.cuda.get_device_name(0)!r} hip={torch.version.hip} "
            f"lib={_pk.LIB_PATH.name} v{_pk.lib().pk_version()}")


@dataclass
class Check:
    """A self-check: ``measure()`` returns ``{metric: value}``; ``bars`` maps a metric to its
    accepted ``(low, high)`` interval (either end None for open)."""

    name: str
    measure: Callable[[], dict]
    bars: dict = field(default_factory=dict)


@dataclass
class Row:
    """A timing row: ``build()`` returns ``{candidate: zero-argument callable}`` (inputs made
    once, outside the timed region); ``work`` is the row's FLOP count (rates in TFLOP/s) or
    None (times in milliseconds); the first candidate is the baseline of the ratios."""

    label: str
    build: Callable[[], dict]
    work: float | None = None
    note: str = ""


def _fmt(v) -> str:
    if isinstance(v, bool):
        return "yes" if v else "no"
    if isinstance(v, float):
        return f"{v:.4g}"
    return str(v)


def run_checks(module: str, checks: list[Check]) -> bool:
    """Print ``check <module>.<name> <metric>=<value> ... verdict=pass|FAIL``; True if all pass."""
    all_ok = True
    for c in checks:
        got = c.measure()
        ok = True
        for metric, (lo, hi) in c.bars.items():
            v = got[metric]
            ok &= (lo is None or v >= lo) and (hi is None or v <= hi)
        all_ok &= ok
        fields = " ".join(f"{k}={_fmt(v)}" for k, v in got.items())
        bars = " ".join(f"bar[{k}]=[{_fmt(lo)},{_fmt(hi)}]" for k, (lo, hi) in c.bars.items())
        print(f"check {module}.{c.name} {fields} {bars} verdict={'pass' if ok else 'FAIL'}",
              flush=True)
    return all_ok


def run_rows(module: str, rows: list[Row]) -> None:
    """Print ``time <module> <label> <candidate>=<rate or ms> ... ratio[<c>/<base>]=x``."""
    for r in rows:
        cands = r.build()
        ms = {name: do_bench(fn) for name, fn in cands.items()}
        base = next(iter(ms))
        if r.work is None:
            vals = " ".join(f"{n}_ms={m:.4f}" for n, m in ms.items())
            ratios = " ".join(f"speedup[{n}/{base}]={ms[base] / m:.3f}"
                              for n, m in ms.items() if n != base)
        else:
            tf = {n: r.work / (m * 1e-3) / 1e12 for n, m in ms.items()}
            vals = " ".join(f"{n}_tflops={t:.2f}" for n, t in tf.items())
            ratios = " ".join(f"speedup[{n}/{base}]={tf[n] / tf[base]:.3f}"
                              for n in tf if n != base)
        note = f" note={r.note!r}" if r.note else ""
        print(f"time {module} {r.label} {vals} {ratios}{note}", flush=True)
        del cands
        torch.cuda.empty_cache()


def main(module: str, checks: list[Check], rows: list[Row]) -> int:
    """The ``__main__`` of a drop-in module: banner, self-checks, timing rows."""
    print(f"harness module={module} {banner()}", flush=True)
    ok = run_checks(module, checks)
    run_rows(module, rows)
    return 0 if ok else 1
