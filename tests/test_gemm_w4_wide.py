"""The 256 x 256 W4A16 kernel (gemm_w4_wide.hip), forced with PK_W4_WIDE=1 so that shapes the
oracle finishes quickly reach it: parity with the CPU oracle (dequantize + fp32 matmul,
relative Frobenius error <= 1e-3 for fp32 output) on full-size and ragged shapes, every k-tile
count class of its four-stage pipeline, group sizes 32..128 and the per-tensor scale, strided
operands and every output dtype; results bitwise reproducible and equal to the 256 x 128
kernel's (PK_W4_WIDE=0): both sum each output's k in the same order. The automatic choice
(two rounds of 256 x 256 tiles or more, e.g. 8192^3) is exercised at full size."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gemm_int4
import oracle

pytestmark = pytest.mark.gpu

W4A16_TOL = 1e-3


@pytest.fixture(autouse=True)
def _force_wide(monkeypatch):
    monkeypatch.setenv("PK_W4_WIDE", "1")


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(M, K, N, G, seed, cuda):
    a = torch.randn(M, K, generator=_gen(seed)).half()
    w = (torch.randn(K, N, generator=_gen(seed + 1)) * 0.02).half()
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), G)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    return a, qw, sc, codes, s16


# K / 32 k-tiles: 1, 3, 5 and 14 exercise the prologue and the three remainder steps of the
# four-stage loop; (4000, 4104) has a partial last tile row and column.
@pytest.mark.parametrize("M,K,N,G", [(4096, 256, 4096, 128), (4096, 32, 4096, 32),
                                     (4096, 96, 4096, 32), (4000, 160, 4104, 32),
                                     (4352, 448, 4096, 64), (4096, 4096, 4096, 128)])
def test_wide_gemm_matches_oracle(M, K, N, G, cuda):
    a, qw, sc, codes, s16 = _case(M, K, N, G, M + K + N, cuda)
    ag = a.to(cuda)
    out = gemm_int4.w4a16_gemm(ag, qw, sc, G, out_dtype=torch.float32)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    err = oracle.rel_fro(out.cpu().numpy(), ref)
    assert err <= W4A16_TOL, f"{M}x{K}x{N} g{G}: rel err {err:.3e}"
    again = gemm_int4.w4a16_gemm(ag, qw, sc, G, out_dtype=torch.float32)
    assert torch.equal(out, again), "not bitwise reproducible"


def test_wide_gemm_per_tensor_scale(cuda):
    """The reference's int4_gemm (one scale for the tensor) at a shape the wide kernel takes."""
    M, K, N = 4096, 256, 4096
    a = torch.randn(M, K, generator=_gen(3)).half()
    w = torch.randn(K, N, generator=_gen(4)).half()
    w_q, scale = gemm_int4.quantize_int4(w.to(cuda))
    c = gemm_int4.int4_gemm(a.to(cuda), gemm_int4.pack_int4_n(w_q), scale)
    ref = a.float().numpy() @ (w_q.cpu().float().numpy() * scale)
    assert oracle.rel_fro(c.cpu().numpy(), ref) < 1e-5  # exact products, fp32 sums


@pytest.mark.parametrize("out_dtype,tol", [(torch.float16, 2e-3), (torch.bfloat16, 1e-2),
                                           (torch.float32, W4A16_TOL)])
def test_wide_gemm_output_dtypes(out_dtype, tol, cuda):
    a, qw, sc, codes, s16 = _case(4096, 128, 4096, 128, 11, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=out_dtype)
    assert out.dtype == out_dtype
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(out.float().cpu().numpy(), ref) <= tol


@pytest.mark.parametrize("pad", [4, 2])
def test_wide_gemm_strided_operands(pad, cuda):
    """A with a row stride above K, and C rows that are not 16-byte aligned (the epilogue's
    direct-store path: 8-byte stores for pad 4, element stores for pad 2)."""
    import _pk

    M, K, N, G = 4096, 128, 4096, 64
    a, qw, sc, codes, s16 = _case(M, K, N, G, 21, cuda)
    abig = torch.zeros(M, K + 64, dtype=torch.float16, device=cuda)
    abig[:, :K] = a.to(cuda)
    cbig = torch.full((M, N + pad), -1.0, dtype=torch.float16, device=cuda)
    out = _pk.w4a16_gemm(abig[:, :K], qw, sc, G, 1.0, torch.float16, out=cbig[:, :N])
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    assert oracle.rel_fro(out.float().cpu().numpy(), ref) <= 2e-3
    assert torch.all(cbig[:, N:] == -1.0), "stores past the row"
    dense = _pk.w4a16_gemm(a.to(cuda), qw, sc, G, 1.0, torch.float16)
    assert torch.equal(out, dense), "strided and contiguous operands give different bits"


@pytest.mark.parametrize("M,K,N,G", [(4096, 256, 4096, 128), (4000, 160, 4104, 32)])
def test_wide_gemm_equals_256x128_kernel(M, K, N, G, monkeypatch, cuda):
    a, qw, sc, codes, s16 = _case(M, K, N, G, 7 * M + K, cuda)
    ag = a.to(cuda)
    wide = gemm_int4.w4a16_gemm(ag, qw, sc, G, out_dtype=torch.float32)
    monkeypatch.setenv("PK_W4_WIDE", "0")
    narrow = gemm_int4.w4a16_gemm(ag, qw, sc, G, out_dtype=torch.float32)
    assert torch.equal(wide, narrow)


def test_wide_gemm_automatic_at_8192(monkeypatch, cuda):
    """8192^3 (1024 tiles of 256 x 256: four full rounds) takes the 256 x 256 kernel without
    the override; checked against the oracle on a 512-row band of the output."""
    monkeypatch.delenv("PK_W4_WIDE")
    M = K = N = 8192
    a, qw, sc, codes, s16 = _case(M, K, N, 128, 31, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    rows = slice(3000, 3512)
    ref = oracle.w4a16_ref(a[rows].numpy(), codes, s16, 128)
    assert oracle.rel_fro(out[rows].cpu().numpy(), ref) <= W4A16_TOL
    monkeypatch.setenv("PK_W4_WIDE", "0")
    narrow = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    assert torch.equal(out, narrow)
