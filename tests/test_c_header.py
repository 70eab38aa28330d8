"""The boundary as a C caller sees it (no GPU needed): include/pico_kernels_amd.h compiles as
strict C99 with every warning an error, a C program links against the built library, and the
host-only entry points answer through the C ABI -- the version, a W4A16 plan, and an invalid
plan that returns an error code with a message in pk_last_error()."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB_DIR = ROOT / "pico-kernels_amd"

C_SRC = r"""
#include <stdio.h>
#include <string.h>
#include "pico_kernels_amd.h"

int main(void) {
  int kid = 0, split = 0;
  if (pk_version() <= 0) return 1;
  if (pk_w4a16_plan(1, 11008, 4096, 128, 0, &kid, &split) != PK_OK) return 2;
  printf("plan %d %d\n", kid, split);
  if (pk_w4a16_plan(1, 11008, 4096, 128, 3, &kid, &split) == PK_OK) return 3; /* 4096 % 3 */
  if (strlen(pk_last_error()) == 0) return 4;
  printf("error %s\n", pk_last_error());
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_header_is_c99_and_the_library_links(tmp_path):
    lib = LIB_DIR / "libpico_kernels_amd.so"
    if not lib.exists():
        pytest.skip("library not built (python pico-kernels_amd/build.py)")
    src = tmp_path / "caller.c"
    src.write_text(C_SRC)
    exe = tmp_path / "caller"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{ROOT / 'include'}",
           str(src), f"-L{LIB_DIR}", "-lpico_kernels_amd", f"-Wl,-rpath,{LIB_DIR}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    lines = run.stdout.splitlines()
    assert lines[0] == "plan 1 16"  # the decode GEMV, 16 slices of 256 rows
    assert lines[1].startswith("error pk_w4a16_plan")
