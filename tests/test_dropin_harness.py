"""The drop-in modules' own harness, run the way the reference's bench.py runs its modules
(bench.py:29-53: ``python <module>.py`` as a subprocess, stdout kept). gemm_int4, gemm_fp8,
gemm_splitk and flash_decoding each declare a self-check and timing rows at the reference's
shapes (gemm_int4.py:95-130, gemm_fp8.py:127-156, gemm_splitk.py:83-113,
flash_decoding.py:128-152), which ``_timing.main`` runs and prints as ``key=value`` lines. The
self-check figures must be within the reference's own bars."""

from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

PKG = Path(__file__).resolve().parents[1] / "pico-kernels_amd"


def _run(module: str) -> str:
    r = subprocess.run([sys.executable, str(PKG / module)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return r.stdout


def _checks(out: str) -> list[str]:
    lines = [l for l in out.splitlines() if l.startswith("check ")]
    assert lines and all(l.endswith("verdict=pass") for l in lines), lines
    return lines


def _field(line: str, key: str) -> str:
    return re.search(rf"\b{re.escape(key)}=(\S+)", line).group(1)


def _rows(out: str, module: str) -> list[str]:
    return [l for l in out.splitlines() if l.startswith(f"time {module} ")]


def test_gemm_int4_main():
    out = _run("gemm_int4.py")
    (line,) = _checks(out)
    assert float(_field(line, "rel_fro")) < 1e-4  # the fused kernel reproduces the product
    rows = _rows(out, "gemm_int4")
    assert len(rows) == 4 and all("int4_gemm_tflops=" in r for r in rows)


def test_gemm_fp8_main():
    out = _run("gemm_fp8.py")
    (line,) = _checks(out)
    assert 0.02 < float(_field(line, "rel_fro")) < 0.06  # fp8-accurate: the reference's ~3.7%
    rows = _rows(out, "gemm_fp8")
    assert len(rows) == 4 and all("fp8_gemm_precast_tflops=" in r for r in rows)


def test_gemm_splitk_main():
    out = _run("gemm_splitk.py")
    (line,) = _checks(out)
    assert _field(line, "allclose_1e-2") == "yes"
    rows = _rows(out, "gemm_splitk")
    assert len(rows) == 4 and all(re.search(r"split\d+_tflops=", r) for r in rows)


def test_flash_decoding_main():
    out = _run("flash_decoding.py")
    (line,) = _checks(out)
    assert _field(line, "allclose_1e-2") == "yes"
    rows = _rows(out, "flash_decoding")
    assert len(rows) == 4 and all("flash_decoding_ms=" in r for r in rows)
