"""ctypes binding to ``libpk_bench_probes.so``: the ceiling probes behind ``bench.py
--mfma-ceiling`` and ``--hbm-ceiling`` and the workgroup-placement probe of the tests
(declared in ``csrc/bench/pk_bench_probes.h``). They are measurement tools, kept outside the
product library; no product module imports this one."""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libpk_bench_probes.so"

_lib = None
_lock = threading.Lock()
_vp, _i32, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_SIGNATURES = {
    "pkb_mfma_probe": (_i32, [_i32, _i32, _i32, _i32, _vp, _vp]),
    "pkb_read_probe": (_i32, [_vp, _sz, _vp, _i32, _vp]),
    "pkb_strip_read_probe": (_i32, [_vp, _i32, ctypes.c_int64, _i32, _vp, _vp]),
    "pkb_xcc_count": (_i32, []),
    "pkb_xcc_probe": (_i32, [_i32, _i32, _i32, _i32, _vp, _vp]),
}


class ProbeError(RuntimeError):
    """A probe call returned a non-zero status."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise ImportError(f"{LIB_PATH} is missing: build it with `python pico-kernels_amd/build.py`")
                h = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in _SIGNATURES.items():
                    fn = getattr(h, name)
                    fn.restype, fn.argtypes = res, args
                _lib = h
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ProbeError(f"{what} failed (status {rc})")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def mfma_probe(fp8: bool, random: bool, grid: int, iters: int, out: torch.Tensor) -> None:
    """Pure-MFMA throughput probe on the current stream; ``out`` holds ``grid * 512`` fp32
    values."""
    assert out.dtype == torch.float32 and out.numel() >= grid * 512 and out.is_cuda
    _check(lib().pkb_mfma_probe(int(fp8), int(random), int(grid), int(iters), out.data_ptr(),
                                _stream(out)), "pkb_mfma_probe")


def read_probe(src: torch.Tensor, out: torch.Tensor, grid: int) -> None:
    """Streaming read of ``src``'s bytes on the current stream; ``out`` holds ``grid`` int32
    words."""
    assert out.dtype == torch.int32 and out.numel() >= grid and out.is_cuda and src.is_cuda
    _check(lib().pkb_read_probe(src.data_ptr(), src.numel() * src.element_size(), out.data_ptr(),
                                int(grid), _stream(src)), "pkb_read_probe")


def xcc_count() -> int:
    """The current device's XCD count in its partition."""
    n = lib().pkb_xcc_count()
    if n < 1:
        raise ProbeError("pkb_xcc_count failed")
    return n


def xcc_probe(grid: int, threads: int, lds_bytes: int, spin: int, out: torch.Tensor) -> None:
    """out[b] = the XCC id workgroup b of a (grid, threads, lds_bytes) launch ran on."""
    assert out.dtype == torch.int32 and out.numel() >= grid and out.is_cuda
    _check(lib().pkb_xcc_probe(int(grid), int(threads), int(lds_bytes), int(spin), out.data_ptr(),
                               _stream(out)), "pkb_xcc_probe")


def strip_read_probe(src: torch.Tensor, strips: int, u: int, out: torch.Tensor) -> None:
    """The strip GEMV's read pattern alone on the current stream: ``src`` holds ``strips``
    contiguous strips of equal size (a multiple of 1 KB); ``out`` holds at least
    ``64 * ceil(strips / 8)`` int32 words."""
    nbytes = src.numel() * src.element_size()
    assert out.dtype == torch.int32 and out.numel() >= 64 * -(-strips // 8) and out.is_cuda
    assert nbytes % strips == 0
    _check(lib().pkb_strip_read_probe(src.data_ptr(), int(strips), nbytes // strips, int(u),
                                      out.data_ptr(), _stream(src)), "pkb_strip_read_probe")
