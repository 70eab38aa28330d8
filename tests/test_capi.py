"""C-ABI boundary checks that need no GPU: the library loads, exports every declared symbol,
plans the right kernels, and rejects bad arguments before launching anything."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import _pk

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pico_kernels_amd.h"


def _declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(pk_\w+)\s*\(", text, re.M)))


def test_header_declares_the_boundary():
    syms = _declared_symbols()
    for name in ("pk_w4a16_gemm", "pk_fp8_gemm", "pk_quantize_group", "pk_cast_e4m3", "pk_absmax",
                 "pk_pack_int4", "pk_unpack_int4", "pk_quantize_int4", "pk_gemm_f16"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = _pk.lib()
    for name in _declared_symbols():
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(_declared_symbols()) == set(_pk.EXPORTED_SYMBOLS)


def test_version_and_error_string():
    lib = _pk.lib()
    assert lib.pk_version() >= 100
    assert isinstance(lib.pk_last_error(), bytes)


def test_w4a16_plans():
    # headline decode shape: skinny GEMV, split chosen to fill the chip
    kid, split = _pk.w4a16_plan(1, 11008, 4096, 128, 0)
    assert kid == _pk.KERNEL_GEMV and split >= 4
    for s in (1, 2, 4, 8, 16):
        assert _pk.w4a16_plan(1, 11008, 4096, 128, s) == (_pk.KERNEL_GEMV, s)
    # prefill: the MFMA GEMM that keeps B packed in LDS, no split needed at 2048 rows
    assert _pk.w4a16_plan(2048, 4096, 4096, 128, 0) == (_pk.KERNEL_GEMM_TR4, 1)
    # 64-row tiles (chosen by the tile-height cost model) take the k-split the model prices
    # lowest within 256 workgroups: 2 x 24 tiles x 4 for qkv at 128 rows, 2 x 16 x 8 at K =
    # 14336 and at K = 12288, 3 x 16 x 4 at 129 rows, 3 x 8 x 8 at N = 2048
    assert _pk.w4a16_plan(128, 6144, 4096, 128, 0) == (_pk.KERNEL_GEMM_TR4, 4)
    assert _pk.w4a16_plan(128, 4096, 14336, 128, 0) == (_pk.KERNEL_GEMM_TR4, 8)
    assert _pk.w4a16_plan(128, 4096, 12288, 128, 0) == (_pk.KERNEL_GEMM_TR4, 8)
    assert _pk.w4a16_plan(129, 4096, 14336, 128, 0) == (_pk.KERNEL_GEMM_TR4, 4)
    assert _pk.w4a16_plan(129, 2048, 14336, 128, 0) == (_pk.KERNEL_GEMM_TR4, 8)
    # 128-row tiles take a power of two when it reaches half the most slices: 4, not 7, for
    # 2 x 16 tiles at K = 14336
    assert _pk.w4a16_plan(256, 4096, 14336, 128, 0) == (_pk.KERNEL_GEMM_TR4, 4)
    # per-tensor mode (group_size 0) for the drop-in int4_gemm
    assert _pk.w4a16_plan(256, 512, 256, 0, 0)[0] == _pk.KERNEL_GEMM_TR4
    assert _pk.w4a16_plan(256, 520, 256, 0, 0)[0] == _pk.KERNEL_GEMM   # N % 256 != 0
    assert _pk.w4a16_plan(256, 512, 192, 0, 0)[0] == _pk.KERNEL_GEMM   # K % 128 != 0
    assert _pk.w4a16_plan(128, 512, 256, 0, 0) == (_pk.KERNEL_GEMM_TR4, 1)  # two k-tiles: unsplit
    assert _pk.w4a16_plan(64, 512, 256, 0, 0)[0] == _pk.KERNEL_SKINNY
    # slices may cut a group (scales are applied per 16-row chunk) ...
    assert _pk.w4a16_plan(1, 4096, 4096, 128, 64) == (_pk.KERNEL_GEMV, 64)
    # ... but a split must divide K into multiples of the row chunk
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_plan(1, 4096, 4096, 128, 3)
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_plan(64, 4096, 4096, 128, 128)


def test_w4a16_plans_by_row_count():
    """The kernel each row count gets, and its split (host planning only)."""
    G, C = _pk.KERNEL_GEMV, _pk.KERNEL_GEMM
    S = _pk.KERNEL_SKINNY
    # M <= 4: the GEMV's 256-row slices (16 for K = 4096); 512-row slices (two 64-row blocks
    # per wave) where 256 would make more than 32: 28 for K = 14336
    assert _pk.w4a16_plan(4, 4096, 4096, 128, 0) == (G, 16)
    assert _pk.w4a16_plan(1, 4096, 14336, 128, 0) == (G, 28)
    assert _pk.w4a16_plan(1, 4096, 14336, 128, 56) == (G, 56)
    # 5 <= M <= 64: register-dequant kernel, 8 waves per workgroup (wave rows of at most one
    # group: slices of at most 1024 rows), the fewest slices reaching 1536 waves: 256-column
    # tiles where they reach it without extra slices, else 128-column tiles
    for M in (5, 8, 16, 17, 32, 33, 64):
        assert _pk.w4a16_plan(M, 6144, 4096, 128, 0) == (S, 4)       # 48 tiles x 4 x 8 waves
    assert _pk.w4a16_plan(8, 4096, 4096, 128, 0) == (S, 8)           # 32 tiles x 8 x 8
    assert _pk.w4a16_plan(8, 4096, 14336, 128, 0) == (S, 14)         # 16 wide tiles x 14 x 8
    # 33..64 rows of layers of more than 4096 x 8192 weights: the packed-B GEMM
    assert _pk.w4a16_plan(48, 4096, 14336, 128, 0) == (_pk.KERNEL_GEMM_TR4, 16)  # 64-row tiles
    assert _pk.w4a16_plan(40, 11008, 4096, 128, 0) == (_pk.KERNEL_GEMM_TR4, 4)
    assert _pk.w4a16_plan(64, 8192, 4096, 128, 0) == (S, 4)
    assert _pk.w4a16_plan(48, 4096, 14336, 128, 14) == (S, 14)      # explicit split
    # short K: 384 rows fit no 8-wave slice -> 4 waves, 3 slices of one 32-row k-step each
    assert _pk.w4a16_plan(8, 528, 384, 128, 0) == (S, 3)
    # explicit splits whose wave rows exceed a group go to the GEMM
    assert _pk.w4a16_plan(8, 1024, 2048, 128, 1)[0] == C
    assert _pk.w4a16_plan(8, 1024, 2048, 128, 2) == (S, 2)
    # ineligible shapes (N % 16, K % 128) stay on the GEMM
    assert _pk.w4a16_plan(8, 520, 1024, 32, 0)[0] == C
    assert _pk.w4a16_plan(8, 512, 1056, 32, 0)[0] == C
    # 65 <= M <= 128 on layers of 1024^2 .. 4096^2 weights: two row parts of the
    # register-dequant kernel when its automatic plan needs at most 8 slices
    T = _pk.KERNEL_GEMM_TR4
    assert _pk.w4a16_plan(128, 4096, 4096, 128, 0) == (S, 4)      # 32 tiles x 2 parts x 4
    assert _pk.w4a16_plan(96, 4096, 4096, 128, 0) == (S, 4)
    assert _pk.w4a16_plan(72, 1024, 1024, 128, 0) == (S, 4)
    assert _pk.w4a16_plan(128, 1024, 4096, 128, 0) == (T, 8)      # its plan would need 16
    assert _pk.w4a16_plan(128, 768, 1024, 128, 0) == (T, 4)       # below 1024^2 weights
    # otherwise above 64 rows: the GEMM that keeps B packed in LDS where its shape rules hold
    # (N % 256, K % 128, group % 64) with the most equal k-slices (at most 16) that keep
    # tiles x slices <= 224, unsplit where the tiles alone reach that: 64 x 256 or 128 x 256
    # tiles by the tile-height cost model (128-row ones take a power of two when one reaches
    # half the most slices)
    assert _pk.w4a16_plan(128, 6144, 4096, 128, 0) == (T, 4)      # 2 x 24 tiles x 4
    assert _pk.w4a16_plan(128, 14336, 4096, 128, 0) == (T, 2)     # 2 x 56 tiles x 2
    assert _pk.w4a16_plan(128, 4096, 14336, 128, 0) == (T, 8)     # 2 x 16 tiles x 8 (112 k-tiles)
    assert _pk.w4a16_plan(256, 6144, 4096, 128, 0) == (T, 2)      # 4 x 24 tiles of 64 rows x 2
    assert _pk.w4a16_plan(1024, 4096, 4096, 128, 0) == (T, 1)     # 128 tiles (x 2 > 224)
    assert _pk.w4a16_plan(2048, 4096, 4096, 128, 0) == (T, 1)
    assert _pk.w4a16_plan(4096, 4096, 4096, 128, 0) == (T, 1)
    assert _pk.w4a16_plan(128, 4096, 4096, 128, 4) == (T, 4)      # explicit split
    # other shapes: two row parts of the register-dequant kernel up to 128 rows of layers of at
    # most 4096 x 4096 weights, else the LDS-tiled GEMM (most slices fitting 256 workgroups)
    assert _pk.w4a16_plan(128, 4000, 4096, 128, 0) == (S, 4)      # N % 256 != 0
    assert _pk.w4a16_plan(128, 6160, 4096, 128, 0) == (C, 4)      # 49 tiles x 4
    assert _pk.w4a16_plan(2048, 4096, 4096, 32, 0) == (C, 1)      # group % 64 != 0
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_plan(128, 4096, 4096, 128, 3)                    # 32 k-tiles, 3 slices


def test_workspace_sizes():
    """Workspaces start with 64 KiB of split-K arrival counters, then the fp32 partials
    (tile-padded for the GEMV's one-launch form)."""
    lib = _pk.lib()
    counters = 64 << 10
    assert lib.pk_w4a16_workspace_bytes(2048, 4096, 4096, 128, 1) == 0
    assert lib.pk_w4a16_workspace_bytes(1, 11008, 4096, 128, 16) == counters + 16 * 11008 * 4
    # N = 11000: 43 column tiles of 256, partial rows padded to 11008
    assert lib.pk_w4a16_workspace_bytes(1, 11000, 4096, 128, 16) == counters + 16 * 11008 * 4
    assert lib.pk_w4a16_workspace_bytes(8, 6144, 4096, 128, 0) == counters + 4 * 8 * 6144 * 4
    assert lib.pk_gemm_f16_workspace_bytes(512, 512, 1024, 4) == counters + 4 * 512 * 512 * 4


@pytest.mark.parametrize("args,code", [
    # N not a multiple of 8
    (dict(M=1, N=12, K=64), _pk.PK_EINVAL),
    # K not a multiple of 32
    (dict(M=1, N=64, K=48), _pk.PK_EINVAL),
    # null A
    (dict(M=1, N=64, K=64, a=0), _pk.PK_EINVAL),
])
def test_w4a16_argument_errors(args, code):
    lib = _pk.lib()
    M, N, K = args["M"], args["N"], args["K"]
    a = args.get("a", 256)  # a fake, aligned, never-dereferenced address
    rc = lib.pk_w4a16_gemm(a, K, 256, N // 8 or 1, None, 0, 1.0, 256, _pk.PK_F32, N, M, N, K, 0,
                           None, 0, None)
    assert rc == code
    assert lib.pk_last_error()


def test_fp8_argument_errors():
    lib = _pk.lib()
    rc = lib.pk_fp8_gemm(256, 104, 256, 104, 0, 1.0, 256, _pk.PK_F32, 104, 4, 104, 100, None)
    assert rc == _pk.PK_EINVAL and b"multiple of 16" in lib.pk_last_error()


def test_flash_decode_workspace_and_errors():
    """Split-KV decode: counters, then per-(b, h) partial regions of S records of 2 + D floats
    rounded up to 128-byte lines; shape errors are reported before any launch."""
    lib = _pk.lib()
    counters = 64 << 10
    # B=2, H=4, N=1024, D=64, split 256: S = 4 records of 66 floats = 264 -> 288 floats
    assert lib.pk_flash_decode_workspace_bytes(2, 4, 1024, 64, 256) == counters + 8 * 288 * 4
    assert lib.pk_flash_decode_workspace_bytes(1, 1, 512, 32, 128) == counters + 160 * 4
    assert lib.pk_flash_decode_workspace_bytes(1, 1, 1000, 64, 256) == 0
    assert lib.pk_flash_decode_launches(1, 1, 1000, 64, 256) == 0
    assert lib.pk_flash_decode_launches(2, 4, 1024, 64, 256) in (1, 2)
    assert lib.pk_flash_decode_launches(8, 128, 1024, 64, 256) == 2  # B*H > 512 counters
    fake = 256  # aligned, never dereferenced
    args = (fake, 64, 64, fake, 64 * 1024, 64 * 1024, 64, fake, 64 * 1024, 64 * 1024, 64)
    rc = lib.pk_flash_decode(*args, 1, 1, 1000, 64, 256, 0.125, fake, None, 0, None)
    assert rc == _pk.PK_EINVAL and b"multiple of split" in lib.pk_last_error()
    rc = lib.pk_flash_decode(*args, 1, 1, 1024, 48, 256, 0.125, fake, None, 0, None)
    assert rc == _pk.PK_EINVAL and b"D=48" in lib.pk_last_error()
    rc = lib.pk_flash_decode(*args, 1, 1, 1024, 64, 256, 0.125, fake, None, 0, None)
    assert rc == _pk.PK_EWORKSPACE


def test_product_modules_never_import_the_oracle():
    for f in (ROOT / "pico-kernels_amd").glob("*.py"):
        src = f.read_text()
        assert not re.search(r"^\s*(import|from)\s+oracle\b", src, re.M), f.name


def test_tiled_rows_per_call():
    """Block-layout calls whose activations span 2 GiB or more (the packed-B GEMM's 32-bit
    buffer offsets) run as equal chunks of whole 128-row multiples below that limit."""
    f = _pk.lib().pk_w4a16_tiled_rows_per_call
    assert f(2048, 4096) == 2048
    assert f(262143, 4096) == 262143                    # 2 GiB - 8 KB: one call
    for M, lda in ((262144, 4096), (75000, 14336), (131072, 14336), (1 << 20, 4096),
                   (300000, 8192)):
        rows = f(M, lda)
        chunks = -(-M // rows)
        assert rows % 128 == 0 and rows * lda * 2 < 2 ** 31, (M, lda, rows)
        assert (chunks - 1) * rows < M <= chunks * rows
        assert rows - M / chunks < 128                   # equal chunks, no small tail call
    assert f(75000, 14336) == 37504
    assert f(100, 1 << 24) == 0                          # even 128 rows exceed 2 GiB


def test_pkcall_module_shares_the_library():
    """The CPython fast-call module that build.py links beside the library: it is the entry
    PreparedStrips uses, it reaches the very library _pk loaded (a null handle's error shows up
    in that library's pk_last_error) and it checks its argument count. No device work."""
    import _pkcall

    assert _pk.strips_run_entry() is _pkcall.strips_run
    assert _pkcall.strips_run(0, 0, 0, 16, 1, 0) == _pk.PK_EINVAL
    assert b"null pointer" in _pk.lib().pk_last_error()
    with pytest.raises(TypeError):
        _pkcall.strips_run(1, 2, 3)
    with pytest.raises(OverflowError):
        _pkcall.strips_run(0, 0, 0, 16, 1 << 40, 0)
