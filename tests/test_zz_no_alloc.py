"""pk_w4a16_gemm_noalloc (the W4A16 entry point that allocates nothing: its split-K scratch is a
fixed device array in the library) against pk_w4a16_gemm with a caller workspace, through the
C ABI: bitwise equal on two calls in a row, the second smaller, for the GEMV (split-K counters
and partials in the scratch), the register-dequant kernel with its reduce launch, the packed-B
and LDS-tiled GEMMs and an unsplit shape; an automatic split too large for the array is
lowered, an explicit one rejected."""

from __future__ import annotations

import ctypes

import pytest
import torch

import _pk
import gemm_int4

pytestmark = pytest.mark.gpu


def _inputs(M, K, N, seed, cuda):
    g = torch.Generator()
    g.manual_seed(seed)
    a = torch.randn(M, K, generator=g).half().to(cuda)
    w = (torch.randn(K, N, generator=g) * 0.02).half().to(cuda)
    qw, sc = gemm_int4.quantize_int4_group(w, 128)
    return a, qw, sc


def _noalloc(a, qw, sc, split, out):
    M, K = a.shape
    N = qw.shape[1] * 8
    rc = _pk.lib().pk_w4a16_gemm_noalloc(
        a.data_ptr(), a.stride(0), qw.data_ptr(), qw.stride(0), sc.data_ptr(), 128, 1.0,
        out.data_ptr(), _pk.pk_dtype(out.dtype), out.stride(0), M, N, K, split,
        _pk.stream_of(a))
    return rc


@pytest.mark.parametrize("shapes", [
    [(1, 4096, 11008, 0), (1, 1024, 512, 4)],       # GEMV, slices added through the scratch
    [(4, 4096, 4096, 16), (2, 2048, 1024, 8)],
    [(32, 4096, 6144, 0), (8, 1024, 2048, 2)],      # register-dequant kernel + reduce launch
    [(32, 14336, 4096, 0), (24, 4096, 1024, 2)],    # group-spanning waves, slices in L2
    [(256, 4096, 1024, 4), (128, 2048, 512, 2)],    # packed-B GEMM, split-K + reduce launch
    [(256, 4096, 1152, 4), (128, 2048, 520, 2)],    # LDS-tiled GEMM, split-K
    [(2048, 512, 2048, 0), (256, 512, 512, 1)],     # unsplit: no scratch used
])
def test_noalloc_matches_workspace_entry_point(shapes, cuda):
    assert _pk.lib().pk_w4a16_noalloc_scratch_bytes() == 16 << 20
    for i, (M, K, N, split) in enumerate(shapes):
        a, qw, sc = _inputs(M, K, N, 100 + i, cuda)
        want = _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16, split_k=split)
        got = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)
        assert _noalloc(a, qw, sc, split, got) == _pk.PK_OK, _pk.lib().pk_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i} {M}x{K}x{N} split {split}"


def test_noalloc_smaller_automatic_split(cuda):
    """An automatic packed-B split whose partials exceed the scratch (4 slices of 256 x 4096
    fp32 at K = 14336, 16.8 MB) runs the largest smaller split that fits (2): the same bits as
    the workspace entry point at that split."""
    M, K, N = 256, 14336, 4096
    assert _pk.w4a16_plan(M, N, K, 128, 0) == (_pk.KERNEL_GEMM_TR4, 4)
    assert _pk.lib().pk_w4a16_workspace_bytes(M, N, K, 128, 4) > 16 << 20
    assert _pk.lib().pk_w4a16_workspace_bytes(M, N, K, 128, 2) <= 16 << 20
    a, qw, sc = _inputs(M, K, N, 11, cuda)
    want = _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float16, split_k=2)
    got = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)
    assert _noalloc(a, qw, sc, 0, got) == _pk.PK_OK, _pk.lib().pk_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_noalloc_rejects_oversized_plan(cuda):
    M, K, N = 64, 4096, 14336
    need = _pk.lib().pk_w4a16_workspace_bytes(M, N, K, 128, 8)
    assert need > _pk.lib().pk_w4a16_noalloc_scratch_bytes()
    a, qw, sc = _inputs(M, K, N, 7, cuda)
    out = torch.empty((M, N), dtype=torch.float16, device=cuda)
    assert _noalloc(a, qw, sc, 8, out) == _pk.PK_EWORKSPACE
    assert b"scratch" in _pk.lib().pk_last_error()
