"""Build the HIP library ``libpico_kernels_amd.so`` for gfx950, in-tree.

Usage: ``python pico-kernels_amd/build.py [-j N] [--verbose]``.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only and linked into one shared
library next to this file. The library exposes the C ABI declared in
``include/pico_kernels_amd.h``; the Python modules in this directory load it with ctypes.
The measurement probes bench.py uses (``csrc/bench/*.hip``) go into a second library,
``libpk_bench_probes.so``, so they stay outside the product library and its header.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB_NAME = "libpico_kernels_amd.so"
PROBES_LIB_NAME = "libpk_bench_probes.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-pass-failed",
    # Never let the compiler form packed-fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return cand


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the gfx950 target feature; that warning is harmless.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err)


def _link(objs: list[Path], out: Path, verbose: bool) -> None:
    tmp = out.with_name(out.name + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    # Resolve every symbol now (a kernel whose host stub was dropped shows up here, not at
    # the first test on a GPU box).
    import ctypes

    try:
        ctypes.CDLL(str(tmp), mode=os.RTLD_NOW)
    except OSError as e:
        raise RuntimeError(f"built library {out.name} does not load: {e}") from None
    os.replace(tmp, out)


def _build_pkcall(lib: Path, verbose: bool) -> Path:
    """The CPython module ``_pkcall`` (csrc/pkcall.c: the prepared decode call without ctypes),
    linked against ``lib`` by path (rpath $ORIGIN)."""
    import sysconfig

    src = CSRC / "pkcall.c"
    out = HERE / ("_pkcall" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = [shutil.which("gcc") or "gcc", "-O2", "-shared", "-fPIC", "-Wall", "-Werror",
           f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}", str(src), "-o", str(tmp),
           f"-L{lib.parent}", "-l:" + lib.name, "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed for {src.name}:\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all HIP sources and link the product library and the bench probes library;
    returns the product library's path."""
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    probe_sources = sorted((CSRC / "bench").glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in sources]
    probe_objs = [objdir / ("bench_" + s.stem + ".o") for s in probe_sources]
    jobs = jobs or min(len(sources) + len(probe_sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose)
                for s, o in zip(sources + probe_sources, objs + probe_objs)]
        for f in futs:
            f.result()
    out = HERE / LIB_NAME
    _link(objs, out, verbose)
    _build_pkcall(out, verbose)
    if probe_objs:
        _link(probe_objs, HERE / PROBES_LIB_NAME, verbose)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    path = build(args.jobs, args.verbose)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
