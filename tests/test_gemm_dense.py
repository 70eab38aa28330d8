"""Dense fp16 / bf16 matmul (drop-in ``gemm.triton_gemm``, gemm.py:103-128, and bf16 through
``gemm_splitk.triton_gemm_splitk``): parity with an fp32 CPU matmul of the same inputs. Both
input types multiply exactly (fp16 11-bit and bf16 8-bit significands) and accumulate in fp32,
so only the summation order differs from the closed form."""

from __future__ import annotations

import pytest
import torch

import gemm
import gemm_splitk
import oracle

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(M, K, N, dtype, seed):
    a = torch.randn(M, K, generator=_gen(seed)).to(dtype)
    b = torch.randn(K, N, generator=_gen(seed + 1)).to(dtype)
    return a, b, (a.float() @ b.float()).numpy()


@pytest.mark.parametrize("dtype", DTYPES)
def test_check_correctness(dtype, cuda):
    """The reference's check_correctness (gemm.py:134-142): 1024^3, allclose 1e-2."""
    a, b, ref = _case(1024, 1024, 1024, dtype, 0)
    c = gemm.triton_gemm(a.to(cuda), b.to(cuda))
    assert c.dtype == torch.float32 and c.shape == (1024, 1024)
    assert torch.allclose(c.cpu(), torch.from_numpy(ref), atol=1e-2, rtol=1e-2)
    assert oracle.rel_fro(c.cpu().numpy(), ref) < 1e-5


# 256-row tiles (M >= 256), the reference's benchmark shapes included
@pytest.mark.parametrize("M,N,K", [(256, 512, 1024), (512, 2048, 1024), (1024, 256, 2048),
                                   (256, 1024, 4096), (2048, 4096, 4096)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_triton_gemm_shapes(M, N, K, dtype, cuda):
    a, b, ref = _case(M, K, N, dtype, M + N + K)
    c = gemm.triton_gemm(a.to(cuda), b.to(cuda))
    assert oracle.rel_fro(c.cpu().numpy(), ref) < 1e-5


# split-K and the 128-row (64 <= M <= 128) and small-M (M < 64) kernels, bf16 and fp16
@pytest.mark.parametrize("M,K,N,split", [(100, 1024, 264, 4), (64, 512, 512, 1), (32, 1024, 256, 2),
                                         (8, 512, 128, 1), (300, 2048, 264, 8)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_splitk_dtypes(M, K, N, split, dtype, cuda):
    a, b, ref = _case(M, K, N, dtype, 7 * M + K)
    c1 = gemm_splitk.triton_gemm_splitk(a.to(cuda), b.to(cuda), split_k=split)
    c2 = gemm_splitk.triton_gemm_splitk(a.to(cuda), b.to(cuda), split_k=split)
    assert torch.equal(c1, c2)
    assert oracle.rel_fro(c1.cpu().numpy(), ref) < 1e-5


def test_triton_gemm_asserts_like_the_reference(cuda):
    a = torch.randn(300, 256, generator=_gen(9)).half().to(cuda)
    b = torch.randn(256, 256, generator=_gen(10)).half().to(cuda)
    with pytest.raises(AssertionError):
        gemm.triton_gemm(a, b)  # M not a multiple of 256
    with pytest.raises(AssertionError):
        gemm.triton_gemm(b, b.to(torch.bfloat16))  # mixed dtypes
    with pytest.raises(AssertionError):
        gemm.triton_gemm(b, a[:, :200].contiguous())  # inner dims differ
