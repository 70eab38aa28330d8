"""The drop-in modules' own harness, run the way the reference's bench.py runs its modules
(bench.py:29-53: ``python <module>.py`` as a subprocess, stdout kept): gemm_int4, gemm_fp8,
gemm_splitk and flash_decoding each print their correctness line and benchmark table
(check_correctness / bench / __main__, as gemm_int4.py:95-137, gemm_fp8.py:127-163,
gemm_splitk.py:83-120 and flash_decoding.py:128-159). The correctness figures printed must
be within the reference's own bars."""

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
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout


def test_gemm_int4_main():
    out = _run("gemm_int4.py")
    rel = float(re.search(r"rel Frobenius err ([0-9.]+)%", out).group(1))
    assert rel < 0.01  # the per-tensor kernel reproduces the quantized product
    assert len(re.findall(r"^\s*\(\d+, \d+, \d+\)\s+\d+ G\s+\d+ G", out, re.M)) == 4


def test_gemm_fp8_main():
    out = _run("gemm_fp8.py")
    rel = float(re.search(r"rel Frobenius err ([0-9.]+)%", out).group(1))
    assert 2.0 < rel < 6.0  # fp8-accurate: the ~3.7% the reference reports
    assert len(re.findall(r"^\s*\d+\s+\d+ G\s+\d+ G", out, re.M)) == 4


def test_gemm_splitk_main():
    out = _run("gemm_splitk.py")
    assert "allclose True" in out
    assert len(re.findall(r"^\s*\(\d+, \d+, \d+\)(\s+\d+ G){3}", out, re.M)) == 4


def test_flash_decoding_main():
    out = _run("flash_decoding.py")
    assert "allclose True" in out
    assert len(re.findall(r"^\s*\d+\s+[0-9.]+m\s+[0-9.]+m", out, re.M)) == 4
