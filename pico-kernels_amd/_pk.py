"""ctypes binding to ``libpico_kernels_amd.so`` (the C ABI in ``include/pico_kernels_amd.h``).

This module is the only place that touches the shared library. It turns torch tensors into
(pointer, shape, stride, stream) arguments, owns the per-stream workspaces and raises on any
non-zero status. It never computes anything itself: if the library or a GPU is missing it
raises instead of falling back to another implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_NAME = "libpico_kernels_amd.so"
LIB_PATH = Path(os.environ.get("PICO_KERNELS_AMD_LIB", str(HERE / LIB_NAME)))

# dtype codes (include/pico_kernels_amd.h)
PK_F32, PK_F16, PK_BF16, PK_E4M3, PK_I8, PK_U8, PK_I32 = range(7)
_TORCH_TO_PK = {torch.float32: PK_F32, torch.float16: PK_F16, torch.bfloat16: PK_BF16}

PK_OK, PK_EINVAL, PK_EUNSUPPORTED, PK_EWORKSPACE, PK_EHIP = 0, -1, -2, -3, -4

KERNEL_GEMV, KERNEL_GEMM, KERNEL_SKINNY, KERNEL_GEMM_TR4 = 1, 2, 3, 4  # pk_w4a16_plan kernel ids


class PicoKernelsError(RuntimeError):
    """A library call returned a non-zero status."""


_lib = None
_lib_lock = threading.Lock()

_vp, _i32, _i64, _f32, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
_SIGNATURES = {
    "pk_version": (_i32, []),
    "pk_last_error": (ctypes.c_char_p, []),
    "pk_absmax_workspace_bytes": (_sz, [_i64]),
    "pk_absmax": (_i32, [_vp, _i32, _i64, _vp, _vp, _sz, _vp]),
    "pk_quantize_int4": (_i32, [_vp, _i32, _i64, _f32, _vp, _vp]),
    "pk_pack_int4": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "pk_unpack_int4": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "pk_quantize_group": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _i32,
                                 _vp, _i32, _vp]),
    "pk_cast_e4m3": (_i32, [_vp, _i32, _i64, _f32, _vp, _vp]),
    "pk_w4a16_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "pk_w4a16_launches": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "pk_w4a16_plan": (_i32, [_i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i32),
                             ctypes.POINTER(_i32)]),
    "pk_w4a16_gemm": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _f32, _vp, _i32, _i64, _i32, _i32,
                             _i32, _i32, _vp, _sz, _vp]),
    "pk_w4a16_gemm_bias": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _f32, _vp, _i32, _vp, _i32,
                                  _i64, _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
    "pk_w4a16_gemm_tiled": (_i32, [_vp, _i64, _vp, _vp, _i32, _f32, _vp, _i32, _vp, _i32, _i64,
                                   _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
    "pk_w4a16_noalloc_scratch_bytes": (_sz, []),
    "pk_w4a16_tiled_rows_per_call": (_i64, [_i64, _i64]),
    "pk_w4a16_gemm_strips": (_i32, [_vp, _i64, _vp, _vp, _i32, _f32, _vp, _i32, _vp, _i32, _i64,
                                    _i32, _i32, _i32, _vp]),
    "pk_w4a16_strips_config": (_i32, [_i32]),
    "pk_w4a16_strips_plan": (_i32, [_i32, _i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                                    ctypes.POINTER(_i32)]),
    "pk_w4a16_strips_prepare": (_vp, [_vp, _vp, _i32, _f32, _vp, _i32, _i32, _i32, _i32, _i64]),
    "pk_w4a16_strips_run": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp]),
    "pk_w4a16_strips_run_events": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp]),
    "pk_w4a16_strips_release": (None, [_vp]),
    "pk_w4a16_skinny_layout": (_i32, [_i32, _i32]),
    "pk_w4a16_prep_activations": (_i32, [_vp, _i32, _i64, _vp, _f32, _vp, _i64, _i32, _i32, _vp]),
    "pk_w4a16_gemm_noalloc": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _f32, _vp, _i32, _i64, _i32, _i32,
                                     _i32, _i32, _vp]),
    "pk_w4a16_gemm_partials": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _vp, _sz, _i32, _i32, _i32,
                                      _i32, _vp]),
    "pk_splitk_reduce": (_i32, [_vp, _i32, _i32, _i32, _f32, _vp, _i32, _i64, _vp]),
    "pk_gemm_f16_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "pk_gemm_f16": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp,
                           _sz, _vp]),
    "pk_gemm_bf16": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp,
                           _sz, _vp]),
    "pk_fp8_gemm": (_i32, [_vp, _i64, _vp, _i64, _i32, _f32, _vp, _i32, _i64, _i32, _i32, _i32,
                           _vp]),
    "pk_gptq_block_cols": (_i32, [_i32, _i32]),
    "pk_gptq_block": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "pk_flash_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "pk_flash_decode_launches": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "pk_flash_decode": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                               _i32, _i32, _i32, _i32, _i32, _f32, _vp, _vp, _sz, _vp]),
}
EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Load the shared library once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise ImportError(
                        f"{LIB_PATH} is missing: build it with `python pico-kernels_amd/build.py`"
                    )
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in _SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


_strips_run_fast = None  # _pkcall.strips_run once probed, False when unavailable


def strips_run_entry():
    """``pk_w4a16_strips_run`` as the CPython module ``_pkcall`` exposes it (built beside the
    library by build.py: six integers in, the status out, no ctypes conversion), when that
    module is there and the library was loaded from its default path (the one ``_pkcall`` is
    linked against); else the ctypes function. Both launch the same kernel."""
    global _strips_run_fast
    L = lib()
    if _strips_run_fast is None:
        _strips_run_fast = False
        if LIB_PATH.resolve() == (HERE / LIB_NAME).resolve():
            try:
                import _pkcall

                _strips_run_fast = _pkcall.strips_run
            except ImportError:
                pass
    return _strips_run_fast or L.pk_w4a16_strips_run


def _check(rc: int, what: str) -> None:
    if rc != PK_OK:
        msg = lib().pk_last_error().decode(errors="replace")
        raise PicoKernelsError(f"{what} failed (status {rc}): {msg}")


def gpu_device() -> torch.device:
    """The GPU the kernels run on; raises when no ROCm GPU is visible."""
    if not torch.cuda.is_available():
        raise RuntimeError("pico-kernels_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def to_gpu(t: torch.Tensor) -> torch.Tensor:
    """Tensors on the host are staged through the current GPU (results go back to the host)."""
    return t if t.is_cuda else t.to(gpu_device())


def _gpu_args(what: str, first: torch.Tensor, *others: torch.Tensor | None) -> None:
    """Raise unless every tensor given (None skipped) lives on the GPU of ``first``: a host or
    other-device pointer handed to a kernel would fault the device instead of failing the call."""
    dev = first.get_device() if first.is_cuda else -1
    if dev < 0 or any(t is not None and (not t.is_cuda or t.get_device() != dev) for t in others):
        raise ValueError(f"{what}: every tensor must be on one GPU (got "
                         + ", ".join(str(t.device) for t in (first, *others) if t is not None) + ")")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def pk_dtype(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_PK[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------------------
# Workspaces: one byte buffer per (device, stream), grown on demand and reused. It holds the
# split-K arrival counters (zero-filled here once, at allocation; every call leaves them zero)
# and the fp32 partials of split-K slices. Calls on one stream are ordered, so they never
# overlap on it.
# ---------------------------------------------------------------------------------------
_workspaces: dict[tuple[int, int], torch.Tensor] = {}


# Workspaces a larger one replaced. A captured HIP graph keeps using the address it recorded,
# so a replaced workspace is never handed back to the allocator.
_retired_workspaces: list[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor | None:
    """The zero-initialised workspace of (device, stream -- the current one by default), grown
    to `nbytes` on demand (the split-K counters at its head are left zero by every call)."""
    if nbytes <= 0:
        return None
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        old = 0
        if ws is not None:
            _retired_workspaces.append(ws)
            old = ws.numel()
        # at least double: growing shapes retire O(log) buffers, at most ~2x the final size
        size = max(nbytes, 1 << 20, 2 * old)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


# ---------------------------------------------------------------------------------------
# Thin wrappers (one per C entry point). Inputs must already be on the GPU.
# ---------------------------------------------------------------------------------------
def absmax(x: torch.Tensor) -> torch.Tensor:
    """max|x| as a 0-d fp32 device tensor."""
    _gpu_args("absmax", x)
    x = x.contiguous()
    n = x.numel()
    out = torch.empty((), dtype=torch.float32, device=x.device)
    nb = lib().pk_absmax_workspace_bytes(n)
    ws = torch.empty(max(nb, 4), dtype=torch.uint8, device=x.device)
    _check(lib().pk_absmax(x.data_ptr(), pk_dtype(x.dtype), n, out.data_ptr(), ws.data_ptr(), ws.numel(),
                           stream_of(x)), "pk_absmax")
    return out


def quantize_int4(w: torch.Tensor, scale: float) -> torch.Tensor:
    _gpu_args("quantize_int4", w)
    w = w.contiguous()
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    _check(lib().pk_quantize_int4(w.data_ptr(), pk_dtype(w.dtype), w.numel(), float(scale),
                                  q.data_ptr(), stream_of(w)), "pk_quantize_int4")
    return q


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    _gpu_args("pack_int4", q)
    assert q.dim() == 2 and q.dtype == torch.int8
    if q.stride(1) != 1:
        q = q.contiguous()
    rows, cols = q.shape
    out = torch.empty((rows, cols // 2), dtype=torch.uint8, device=q.device)
    _check(lib().pk_pack_int4(q.data_ptr(), rows, cols, max(q.stride(0), cols), out.data_ptr(),
                              stream_of(q)), "pk_pack_int4")
    return out


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    _gpu_args("unpack_int4", packed)
    assert packed.dim() == 2 and packed.dtype == torch.uint8
    packed = packed.contiguous()
    rows, half = packed.shape
    q = torch.empty((rows, 2 * half), dtype=torch.int8, device=packed.device)
    _check(lib().pk_unpack_int4(packed.data_ptr(), rows, 2 * half, q.data_ptr(), stream_of(packed)),
           "pk_unpack_int4")
    return q


def quantize_group(w: torch.Tensor, bits: int, group_size: int | None, *, half_math: bool,
                   want_qweight: bool, want_scales: bool, want_fake: bool,
                   scale_dtype: torch.dtype = torch.float16,
                   fake_dtype: torch.dtype | None = None):
    """Group RTN along dim 0 of a 2-D (K, N) tensor. Returns (qweight, scales, fake)."""
    _gpu_args("quantize_group", w)
    assert w.dim() == 2
    if w.stride(1) != 1:
        w = w.contiguous()
    K, N = w.shape
    g = int(group_size) if group_size else 0
    ngroups = -(-K // g) if g else 1
    qweight = torch.empty((K, N // 8), dtype=torch.int32, device=w.device) if want_qweight else None
    scales = torch.empty((ngroups, N), dtype=scale_dtype, device=w.device) if want_scales else None
    fdt = fake_dtype or w.dtype
    fake = torch.empty((K, N), dtype=fdt, device=w.device) if want_fake else None
    _check(lib().pk_quantize_group(
        w.data_ptr(), pk_dtype(w.dtype), K, N, max(w.stride(0), N), int(bits), g, int(half_math),
        ptr(qweight), ptr(scales), pk_dtype(scale_dtype), ptr(fake), pk_dtype(fdt), stream_of(w)),
        "pk_quantize_group")
    return qweight, scales, fake


def cast_e4m3(x: torch.Tensor, scale: float) -> torch.Tensor:
    _gpu_args("cast_e4m3", x)
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    _check(lib().pk_cast_e4m3(x.data_ptr(), pk_dtype(x.dtype), x.numel(), float(scale),
                              out.data_ptr(), stream_of(x)), "pk_cast_e4m3")
    return out


def w4a16_plan(M: int, N: int, K: int, group_size: int, split_k: int) -> tuple[int, int]:
    kid, spl = ctypes.c_int(0), ctypes.c_int(0)
    _check(lib().pk_w4a16_plan(M, N, K, group_size, split_k, ctypes.byref(kid), ctypes.byref(spl)),
           "pk_w4a16_plan")
    return kid.value, spl.value


def w4a16_prep_activations(x: torch.Tensor, in_scale: torch.Tensor | None, mul: float,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 ``x * in_scale[k] * mul`` for (M, K) activations of any float dtype (no scale:
    the cast alone)."""
    _gpu_args("w4a16_prep_activations", x, in_scale, out)
    M, K = x.shape
    if x.stride(1) != 1:
        x = x.contiguous()
    if in_scale is not None:
        assert in_scale.dtype == torch.float32 and in_scale.is_contiguous() and in_scale.numel() == K
    if out is None:
        out = torch.empty((M, K), dtype=torch.float16, device=x.device)
    _check(lib().pk_w4a16_prep_activations(x.data_ptr(), pk_dtype(x.dtype), x.stride(0),
                                           None if in_scale is None else in_scale.data_ptr(),
                                           float(mul), out.data_ptr(), out.stride(0), M, K,
                                           stream_of(x)), "pk_w4a16_prep_activations")
    return out


def w4a16_skinny_layout(cols_per_lane: int, waves: int) -> None:
    """Fix the register-dequant kernel's layout for later plans ((0, 0): automatic)."""
    _check(lib().pk_w4a16_skinny_layout(int(cols_per_lane), int(waves)), "pk_w4a16_skinny_layout")
    _ws_bytes.clear()


def w4a16_launches(M: int, N: int, K: int, group_size: int, split_k: int) -> int:
    """Kernel launches one pk_w4a16_gemm call makes (1 when split-K slices add up in L2)."""
    n = lib().pk_w4a16_launches(M, N, K, group_size, split_k)
    _check(min(n, 0), "pk_w4a16_launches")
    return n


FP16_MAX = 65504.0


def check_fp16_range(x: torch.Tensor, what: str, converted: torch.Tensor | None = None) -> None:
    """Raise ``ValueError`` when a finite element of ``x`` (bf16 / fp32 activations the W4A16
    kernels take as fp16) lies beyond fp16's largest finite value 65504, where the fp16 cast
    would turn it into an infinity -- or, given ``converted`` (the fp16 tensor made from
    ``x``), when a finite element of ``x`` became infinite in it. One device reduction and a
    synchronisation; skipped while the stream is being captured into a graph (no
    synchronisation is allowed there)."""
    if x.dtype == torch.float16 or (x.is_cuda and torch.cuda.is_current_stream_capturing()):
        return
    bad = torch.isinf(converted) if converted is not None else x.abs() > FP16_MAX
    if bool((bad & torch.isfinite(x)).any()):
        big = x[torch.isfinite(x)].abs().max().item()
        raise ValueError(f"{what}: {x.dtype} activations up to |x| = {big:g} exceed fp16's range "
                         f"(65504); the W4A16 kernels compute in fp16")


def _rows_ok(t: torch.Tensor) -> torch.Tensor:
    """Row-major with unit inner stride and 16-byte aligned rows, else a contiguous copy."""
    es = t.element_size()
    if (t.stride(-1) != 1 or (t.stride(0) * es) % 16 or t.data_ptr() % 16):
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


# Workspace bytes per W4A16 shape (a pure function of the plan; cleared when the plan rules
# change through w4a16_skinny_layout), so an eager call makes one C call, not two.
_ws_bytes: dict[tuple[int, int, int, int, int], int] = {}


def tiles_ok(K: int, N: int, group_size: int) -> bool:
    """Shapes whose weights pk_w4a16_gemm_tiled reads in blocks (group 0: per-tensor)."""
    return N % 256 == 0 and K % 256 == 0 and group_size % 64 == 0


def tile_weights(qweight: torch.Tensor) -> torch.Tensor:
    """(K, N/8) int32 words in pack_int4_n order -> the same codes in 128 x 256 blocks: each
    block's 128 rows of 32 words contiguous (16 KB), the blocks ordered by row block and then
    column tile (still shaped (K, N/8))."""
    K, W = qweight.shape
    if W % 32 or K % 128:
        raise ValueError(f"tile_weights: K = {K} must be a multiple of 128 and N = {8 * W} of 256")
    return (qweight.reshape(K // 128, 128, W // 32, 32).permute(0, 2, 1, 3).contiguous()
            .view(K, W))


def untile_weights(qtiled: torch.Tensor) -> torch.Tensor:
    """Inverse of tile_weights: blocks -> (K, N/8) words in pack_int4_n order."""
    K, W = qtiled.shape
    if W % 32 or K % 128:
        raise ValueError(f"untile_weights: K = {K} must be a multiple of 128 and N = {8 * W} of 256")
    return (qtiled.contiguous().view(K // 128, W // 32, 128, 32).permute(0, 2, 1, 3)
            .contiguous().view(K, W))


def strips_ok(K: int, N: int, group_size: int) -> bool:
    """Shapes pk_w4a16_gemm_strips takes (group 0: per-tensor): N % 16 == 0, K % 128 == 0, and
    a group of a multiple of 32 that divides 128 or is a multiple of it."""
    if N % 16 or K % 128 or K < 128:
        return False
    g = int(group_size)
    return g == 0 or (g % 32 == 0 and K % g == 0 and (128 % g == 0 or g % 128 == 0))


def strip_weights(qweight: torch.Tensor) -> torch.Tensor:
    """(K, N/8) int32 words in pack_int4_n order -> the same bytes in the strip layout of
    pk_w4a16_gemm_strips (still shaped (K, N/8) int32): byte (k, c) of the (K, N/2) packed
    bytes, k = 128b + 32rs + 8g + e and c = 8s + 2cps + h, moves to
    ((((s * K/128 + b) * 4 + g) * 4 + rs) * 4 + cps) * 16 + 8h + e, with both nibbles XOR 8
    (u = v + 8, the code biased to 0..15)."""
    K, W = qweight.shape
    N = 8 * W
    if N % 16 or K % 128:
        raise ValueError(f"strip_weights: K = {K} must be a multiple of 128 and N = {N} of 16")
    b = qweight.contiguous().view(torch.uint8).view(K // 128, 4, 4, 8, N // 16, 4, 2)
    return (b.permute(4, 0, 2, 1, 5, 6, 3).contiguous() ^ 0x88).view(torch.int32).view(K, W)


def unstrip_weights(qstrips: torch.Tensor) -> torch.Tensor:
    """Inverse of strip_weights: the strip layout -> (K, N/8) words in pack_int4_n order."""
    K, W = qstrips.shape
    N = 8 * W
    if N % 16 or K % 128:
        raise ValueError(f"unstrip_weights: K = {K} must be a multiple of 128 and N = {N} of 16")
    b = qstrips.contiguous().view(torch.uint8).view(N // 16, K // 128, 4, 4, 4, 2, 8) ^ 0x88
    return b.permute(1, 3, 2, 6, 0, 4, 5).contiguous().view(K, N // 2).view(torch.int32)


def strip_scales(scales: torch.Tensor) -> torch.Tensor:
    """(K/G, N) group scales -> (N/16, K/G, 16), each strip's scales contiguous (still
    shaped (K/G, N))."""
    KG, N = scales.shape
    return scales.contiguous().view(KG, N // 16, 16).permute(1, 0, 2).contiguous().view(KG, N)


def unstrip_scales(sstrips: torch.Tensor) -> torch.Tensor:
    """Inverse of strip_scales."""
    KG, N = sstrips.shape
    return sstrips.contiguous().view(N // 16, KG, 16).permute(1, 0, 2).contiguous().view(KG, N)


def w4a16_gemm_strips(a: torch.Tensor, qstrips: torch.Tensor, sstrips: torch.Tensor | None,
                      group_size: int, tensor_scale: float, out_dtype: torch.dtype,
                      out: torch.Tensor | None = None,
                      bias: torch.Tensor | None = None) -> torch.Tensor:
    """out = tensor_scale * (a @ dequant(q, s)) (+ bias) for 1..8 rows of fp16 activations on
    strip-layout codes and scales (strip_weights / strip_scales; pk_w4a16_gemm_strips)."""
    _gpu_args("w4a16_gemm_strips", a, qstrips, sstrips, out, bias)
    M, K = a.shape
    N = qstrips.shape[1] * 8
    a = _rows_ok(a)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    g = int(group_size) if sstrips is not None else 0
    L = _lib if _lib is not None else lib()
    rc = L.pk_w4a16_gemm_strips(
        a.data_ptr(), a.stride(0), qstrips.data_ptr(),
        None if sstrips is None else sstrips.data_ptr(), g, float(tensor_scale),
        None if bias is None else bias.data_ptr(),
        _TORCH_TO_PK[bias.dtype] if bias is not None else PK_F16, out.data_ptr(),
        _TORCH_TO_PK[out.dtype], out.stride(0), M, N, K,
        torch.cuda.current_stream(a.device).cuda_stream)
    if rc != PK_OK:
        _check(rc, "pk_w4a16_gemm_strips")
    return out


class PreparedStrips:
    """``pk_w4a16_gemm_strips`` bound to one strip-layout weight copy through
    ``pk_w4a16_strips_prepare``: the fixed arguments are checked and the launches for 1..8 rows
    planned once, so a call passes only the activations, the output, the row count and the
    stream (what an eager decode loop pays per layer). Activations must be 16-byte aligned with
    row stride ``lda`` (elements; default K). The tensors stay referenced here, and must stay
    in place, while the object lives (QuantLinear drops it when its buffers move or change)."""

    __slots__ = ("h", "N", "K", "lda", "out_dtype", "dev", "run", "run_events", "release", "_keep")

    def __init__(self, qstrips: torch.Tensor, sstrips: torch.Tensor | None, group_size: int,
                 tensor_scale: float, out_dtype: torch.dtype, bias: torch.Tensor | None = None,
                 lda: int | None = None):
        L = lib()
        self.K, W = qstrips.shape
        self.N = 8 * W
        self.lda = self.K if lda is None else int(lda)
        self.out_dtype = out_dtype
        self.dev = qstrips.device.index
        self._keep = (qstrips, sstrips, bias)
        self.h = L.pk_w4a16_strips_prepare(
            qstrips.data_ptr(), None if sstrips is None else sstrips.data_ptr(),
            int(group_size) if sstrips is not None else 0, float(tensor_scale),
            None if bias is None else bias.data_ptr(),
            _TORCH_TO_PK[bias.dtype] if bias is not None else PK_F16, _TORCH_TO_PK[out_dtype],
            self.N, self.K, self.lda)
        if not self.h:
            raise PicoKernelsError("pk_w4a16_strips_prepare failed: "
                                   + L.pk_last_error().decode(errors="replace"))
        self.run, self.release = strips_run_entry(), L.pk_w4a16_strips_release
        self.run_events = L.pk_w4a16_strips_run_events

    def __del__(self):
        h = getattr(self, "h", None)
        if h:
            self.release(h)
            self.h = None

    def __call__(self, a: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        if (a.dtype != torch.float16 or a.dim() != 2 or a.shape[1] != self.K or not a.is_cuda
                or a.get_device() != self.dev):
            raise ValueError(f"PreparedStrips: activations must be (M, {self.K}) fp16 on "
                             f"cuda:{self.dev} (got {tuple(a.shape)} {a.dtype} on {a.device})")
        M = a.shape[0]
        if a.stride(0) != self.lda or a.stride(1) != 1 or a.data_ptr() % 16:
            a = a.contiguous() if self.lda == self.K else _rows_ok(a)
            if a.stride(0) != self.lda or a.data_ptr() % 16:
                raise ValueError(f"PreparedStrips: activations need row stride {self.lda}, "
                                 "16-byte aligned")
        if out is None:
            out = a.new_empty((M, self.N), dtype=self.out_dtype)
        elif (out.dtype != self.out_dtype or out.dim() != 2 or out.shape[0] != M
              or out.shape[1] != self.N or out.stride(1) != 1 or not out.is_cuda
              or out.get_device() != self.dev):
            raise ValueError(f"PreparedStrips: out must be ({M}, {self.N}) {self.out_dtype} with "
                             f"unit column stride on cuda:{self.dev}")
        rc = self.run(self.h, a.data_ptr(), out.data_ptr(), out.stride(0), M,
                      torch._C._cuda_getCurrentRawStream(self.dev))
        if rc != PK_OK:
            _check(rc, "pk_w4a16_strips_run")
        return out

    def timed(self, a: torch.Tensor, out: torch.Tensor, start=None, stop=None) -> None:
        """The call above (activations as the prepared stride wants them, output given), with
        ``torch.cuda.Event`` ``start`` recorded as its kernel starts and ``stop`` as it ends, by
        the dispatch itself (``pk_w4a16_strips_run_events``). Each event is recorded once on
        the current stream first if it has no HIP event yet."""
        if (a.dtype != torch.float16 or a.dim() != 2 or a.shape[1] != self.K or not a.is_cuda
                or a.get_device() != self.dev or out.dtype != self.out_dtype
                or tuple(out.shape) != (a.shape[0], self.N) or out.stride(1) != 1
                or out.get_device() != self.dev):
            raise ValueError("PreparedStrips.timed: (M, K) fp16 activations and an (M, N) output "
                             "of the prepared dtype, both on the prepared device")
        if a.stride(0) != self.lda or a.stride(1) != 1 or a.data_ptr() % 16:
            raise ValueError(f"PreparedStrips.timed: activations need row stride {self.lda}, "
                             "16-byte aligned")
        handles = []
        for ev in (start, stop):
            if ev is not None and not ev.cuda_event:
                ev.record()
            handles.append(None if ev is None else ev.cuda_event)
        rc = self.run_events(self.h, a.data_ptr(), out.data_ptr(), out.stride(0), a.shape[0],
                             torch._C._cuda_getCurrentRawStream(self.dev), *handles)
        if rc != PK_OK:
            _check(rc, "pk_w4a16_strips_run_events")


def w4a16_strips_config(blocks_per_wave: int) -> None:
    """Fix the strip GEMV's 1 KB blocks per wave (2, 4 or 8; 0: automatic)."""
    _check(lib().pk_w4a16_strips_config(int(blocks_per_wave)), "pk_w4a16_strips_config")


def w4a16_strips_plan(M: int, N: int, K: int) -> tuple[int, int, int]:
    """(strips per workgroup, 1 KB blocks per wave, waves per workgroup) of the strip GEMV's
    launch for M rows of an (N, K) layer."""
    ns, u, nw = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    _check(lib().pk_w4a16_strips_plan(M, N, K, ctypes.byref(ns), ctypes.byref(u), ctypes.byref(nw)),
           "pk_w4a16_strips_plan")
    return ns.value, u.value, nw.value


def w4a16_gemm(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor | None,
               group_size: int, tensor_scale: float, out_dtype: torch.dtype,
               split_k: int = 0, out: torch.Tensor | None = None,
               bias: torch.Tensor | None = None, tiled: bool = False) -> torch.Tensor:
    """out = tensor_scale * (a @ dequant(qweight, scales)) (+ bias, N values of fp32 / fp16 /
    bf16 added in the kernels' epilogue: pk_w4a16_gemm_bias). ``tiled``: qweight holds the
    codes in 128 x 256 blocks (tile_weights; pk_w4a16_gemm_tiled)."""
    _gpu_args("w4a16_gemm", a, qweight, scales, out, bias)
    M, K = a.shape
    N = qweight.shape[1] * 8
    if bias is not None and (bias.numel() != N or bias.dtype not in _TORCH_TO_PK
                             or not bias.is_contiguous()):
        raise ValueError(f"w4a16_gemm: bias must be {N} contiguous fp32 / fp16 / bf16 values, "
                         f"got {tuple(bias.shape)} {bias.dtype}")
    a = _rows_ok(a)
    if qweight.stride(1) != 1:
        qweight = qweight.contiguous()
    if scales is not None and not scales.is_contiguous():
        scales = scales.contiguous()
    dev = a.device
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    g = int(group_size) if scales is not None else 0
    split_k = int(split_k)
    key = (M, N, K, g, split_k)
    nbytes = _ws_bytes.get(key)
    L = _lib if _lib is not None else lib()
    if nbytes is None:
        nbytes = L.pk_w4a16_workspace_bytes(M, N, K, g, split_k)
        if len(_ws_bytes) > 4096:
            _ws_bytes.clear()
        _ws_bytes[key] = nbytes
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = workspace(dev, nbytes, stream) if nbytes else None
    if tiled:
        if not qweight.is_contiguous():
            raise ValueError("w4a16_gemm: block-layout weights must be contiguous")
        rc = L.pk_w4a16_gemm_tiled(
            a.data_ptr(), a.stride(0), qweight.data_ptr(),
            None if scales is None else scales.data_ptr(), g, float(tensor_scale),
            None if bias is None else bias.data_ptr(),
            _TORCH_TO_PK[bias.dtype] if bias is not None else PK_F16, out.data_ptr(),
            _TORCH_TO_PK[out.dtype], out.stride(0), M, N, K, split_k,
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), stream)
        if rc != PK_OK:
            _check(rc, "pk_w4a16_gemm_tiled")
        return out
    if bias is None:
        rc = L.pk_w4a16_gemm(
            a.data_ptr(), a.stride(0), qweight.data_ptr(), qweight.stride(0),
            None if scales is None else scales.data_ptr(), g, float(tensor_scale), out.data_ptr(),
            _TORCH_TO_PK[out.dtype], out.stride(0), M, N, K, split_k,
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), stream)
        if rc != PK_OK:
            _check(rc, "pk_w4a16_gemm")
        return out
    rc = L.pk_w4a16_gemm_bias(
        a.data_ptr(), a.stride(0), qweight.data_ptr(), qweight.stride(0),
        None if scales is None else scales.data_ptr(), g, float(tensor_scale), bias.data_ptr(),
        _TORCH_TO_PK[bias.dtype], out.data_ptr(), _TORCH_TO_PK[out.dtype], out.stride(0), M, N,
        K, split_k, None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
        stream)
    if rc != PK_OK:
        _check(rc, "pk_w4a16_gemm_bias")
    return out


def w4a16_gemm_partials(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor | None,
                        group_size: int, split_k: int, partials: torch.Tensor | None = None
                        ) -> torch.Tensor:
    """Per-slice fp32 partial sums (split, M, N) of a split-K W4A16 matmul."""
    _gpu_args("w4a16_gemm_partials", a, qweight, scales, partials)
    M, K = a.shape
    N = qweight.shape[1] * 8
    g = int(group_size) if scales is not None else 0
    kid, split = w4a16_plan(M, N, K, g, int(split_k))
    if partials is None:
        partials = torch.empty((split, M, N), dtype=torch.float32, device=a.device)
    _check(lib().pk_w4a16_gemm_partials(
        a.data_ptr(), a.stride(0), qweight.data_ptr(), qweight.stride(0), ptr(scales), g,
        partials.data_ptr(), partials.numel() * 4, M, N, K, int(split_k), stream_of(a)),
        "pk_w4a16_gemm_partials")
    return partials


def splitk_reduce(partials: torch.Tensor, scale: float, out: torch.Tensor) -> torch.Tensor:
    _gpu_args("splitk_reduce", partials, out)
    split, M, N = partials.shape
    _check(lib().pk_splitk_reduce(partials.data_ptr(), split, M, N, float(scale), out.data_ptr(),
                                  pk_dtype(out.dtype), out.stride(0), stream_of(partials)),
           "pk_splitk_reduce")
    return out


def gemm_dense(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype, split_k: int) -> torch.Tensor:
    """C = A @ B for fp16 or bf16 A and B (same dtype), fp32 accumulate (pk_gemm_f16 /
    pk_gemm_bf16)."""
    _gpu_args("gemm_dense", a, b)
    M, K = a.shape
    N = b.shape[1]
    a, b = _rows_ok(a), _rows_ok(b)
    out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    nbytes = lib().pk_gemm_f16_workspace_bytes(M, N, K, int(split_k))
    ws = workspace(a.device, nbytes)
    name = "pk_gemm_bf16" if a.dtype == torch.bfloat16 else "pk_gemm_f16"
    _check(getattr(lib(), name)(a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
                                out.data_ptr(), pk_dtype(out_dtype), out.stride(0), M, N, K,
                                int(split_k), ptr(ws), 0 if ws is None else ws.numel(),
                                stream_of(a)), name)
    return out


gemm_f16 = gemm_dense  # the fp16 name used by earlier callers


def fp8_gemm(a8: torch.Tensor, b8: torch.Tensor, out_scale: float, out_dtype: torch.dtype,
             out: torch.Tensor | None = None) -> torch.Tensor:
    _gpu_args("fp8_gemm", a8, b8, out)
    M, K = a8.shape
    N = b8.shape[1]
    a8 = _rows_ok(a8)
    # b8 is (K, N). A transposed view of a row-major (N, K) buffer is consumed in place.
    if b8.stride(0) == 1 and b8.stride(1) >= K and (b8.stride(1) % 16 == 0) and b8.data_ptr() % 16 == 0:
        b_layout, b_buf, ldb = 1, b8, b8.stride(1)
    else:
        b_buf = b8 if (b8.stride(1) == 1 and b8.stride(0) % 8 == 0 and b8.data_ptr() % 8 == 0) else b8.contiguous()
        b_layout, ldb = 0, b_buf.stride(0)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a8.device)
    _check(lib().pk_fp8_gemm(a8.data_ptr(), a8.stride(0), b_buf.data_ptr(), ldb, b_layout,
                             float(out_scale), out.data_ptr(), pk_dtype(out.dtype), out.stride(0),
                             M, N, K, stream_of(a8)), "pk_fp8_gemm")
    return out


def gptq_block_cols(out: int, group: int) -> int:
    """Columns the GPTQ sweep kernel takes per launch for `out` rows and scale group `group`
    (0: one scale per column)."""
    return int(lib().pk_gptq_block_cols(out, group))


def gptq_block(q: torch.Tensor, ratio: torch.Tensor, err: torch.Tensor, b0: int, nb: int, bits: int,
               group: int) -> None:
    """Sweep columns [b0, b0 + nb) of q (fp32 [out, in], row stride q.stride(0)) in place;
    err[:, :nb] receives the quantization errors (pk_gptq_block)."""
    _gpu_args("gptq_block", q, ratio, err)
    assert q.dtype == ratio.dtype == err.dtype == torch.float32
    assert q.stride(1) == 1 and ratio.stride(1) == 1 and err.stride(1) == 1
    out, n_in = q.shape
    _check(lib().pk_gptq_block(q.data_ptr(), q.stride(0), ratio.data_ptr(), ratio.stride(0),
                               err.data_ptr(), err.stride(0), out, n_in, int(b0), int(nb), int(bits),
                               int(group), stream_of(q)), "pk_gptq_block")


def flash_decode_launches(B: int, H: int, N: int, D: int, split: int) -> int:
    """Kernel launches one pk_flash_decode call makes (1: combined in the split kernel)."""
    return int(lib().pk_flash_decode_launches(B, H, N, D, int(split)))


def flash_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, split: int,
                 sm_scale: float) -> torch.Tensor:
    """(B, H, D) fp32 single-query attention of q (B, H, D) over k, v (B, H, N, D), all fp16
    with unit stride along D (pk_flash_decode)."""
    _gpu_args("flash_decode", q, k, v)
    B, H, N, D = k.shape

    def _d_unit(t: torch.Tensor) -> torch.Tensor:
        ok = t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1]) and t.data_ptr() % 16 == 0
        return t if ok else t.contiguous()

    q, k, v = _d_unit(q), _d_unit(k), _d_unit(v)
    out = torch.empty((B, H, D), dtype=torch.float32, device=q.device)
    nbytes = lib().pk_flash_decode_workspace_bytes(B, H, N, D, int(split))
    ws = workspace(q.device, nbytes)  # zero-filled counters, shared with the GEMMs
    _check(lib().pk_flash_decode(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
                                 k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1),
                                 v.stride(2), B, H, N, D, int(split), float(sm_scale),
                                 out.data_ptr(), 0 if ws is None else ws.data_ptr(),
                                 0 if ws is None else ws.numel(), stream_of(q)),
           "pk_flash_decode")
    return out
