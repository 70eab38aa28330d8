"""Dense split-K parity on the GPU (drop-in gemm_splitk.triton_gemm_splitk)."""

from __future__ import annotations

import pytest
import torch

import gemm_splitk
import oracle

pytestmark = pytest.mark.gpu


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def test_splitk_matches_fp32(cuda):
    """The reference's test (tests/test_gemm_splitk.py:19-27) with CPU-seeded inputs."""
    a = torch.randn(512, 1024, generator=_gen(0)).half()
    b = torch.randn(1024, 512, generator=_gen(1)).half()
    c = gemm_splitk.triton_gemm_splitk(a.to(cuda), b.to(cuda), split_k=4)
    assert c.dtype == torch.float32
    ref = a.float() @ b.float()
    assert torch.allclose(c.cpu(), ref, atol=1e-2, rtol=1e-2), (c.cpu() - ref).abs().max()


def test_splitk_matches_non_split(cuda):
    """The reference's test (tests/test_gemm_splitk.py:30-38): split-K against the dense
    ``gemm.triton_gemm`` drop-in."""
    import gemm

    a = torch.randn(512, 512, generator=_gen(1)).half().to(cuda)
    b = torch.randn(512, 512, generator=_gen(2)).half().to(cuda)
    c_split = gemm_splitk.triton_gemm_splitk(a, b, split_k=4)
    c_plain = gemm.triton_gemm(a, b)
    assert torch.allclose(c_split, c_plain, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("split_k", [1, 2, 4, 8])
def test_splitk_closed_form_and_determinism(split_k, cuda):
    M, K, N = 300, 2048, 264
    a = torch.randn(M, K, generator=_gen(3)).half()
    b = torch.randn(K, N, generator=_gen(4)).half()
    c1 = gemm_splitk.triton_gemm_splitk(a.to(cuda), b.to(cuda), split_k=split_k)
    c2 = gemm_splitk.triton_gemm_splitk(a.to(cuda), b.to(cuda), split_k=split_k)
    assert torch.equal(c1, c2), "split-K result must be bitwise reproducible"
    ref = oracle.splitk_ref(a.numpy(), b.numpy(), split_k)
    assert oracle.rel_fro(c1.cpu().numpy(), ref) < 1e-6


def test_splitk_divisibility_contract(cuda):
    a = torch.randn(64, 192, generator=_gen(5)).half().to(cuda)
    b = torch.randn(192, 64, generator=_gen(6)).half().to(cuda)
    with pytest.raises(AssertionError):
        gemm_splitk.triton_gemm_splitk(a, b, split_k=4)  # 192 % (4 * 64) != 0


@pytest.mark.parametrize("M,K,N", [(256, 192, 256), (300, 320, 528), (128, 448, 384)])
def test_dense_odd_k_tile_counts(M, K, N, cuda):
    """Odd numbers of 64-wide K tiles through the large-tile MFMA kernel, against fp32."""
    a = torch.randn(M, K, generator=_gen(M + K)).half()
    b = torch.randn(K, N, generator=_gen(M + N)).half()
    c = gemm_splitk.triton_gemm_splitk(a.to(cuda), b.to(cuda), split_k=1)
    ref = (a.float() @ b.float()).numpy()
    assert oracle.rel_fro(c.cpu().numpy(), ref) < 1e-5
