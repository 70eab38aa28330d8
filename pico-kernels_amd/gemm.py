"""Dense fp16 / bf16 matmul on MI355X -- drop-in for the reference's ``gemm`` module.

Reference entry point kept with its signature and checks (gemm.py:103-128):
  ``triton_gemm(a, b) -> (M, N) fp32``

It asserts what the reference asserts: both inputs on the GPU with one dtype, matching inner
dimensions, and ``M, N`` multiples of 256 with ``K`` a multiple of 64 (the reference kernel
is mask-free and autotunes tiles up to 256). The matmul is the hand-written MFMA GEMM behind
``pk_gemm_f16`` / ``pk_gemm_bf16`` (fp32 accumulate, no split-K); the name keeps
``triton_`` only for drop-in compatibility. The reference's split-K test uses it as the
comparator of ``gemm_splitk.triton_gemm_splitk`` (tests/test_gemm_splitk.py:30-38).
"""

from __future__ import annotations

import torch

import _pk

__all__ = ["triton_gemm"]


def triton_gemm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    assert a.is_cuda and b.is_cuda and a.dtype == b.dtype
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, "inner dims must match"
    assert M % 256 == 0 and N % 256 == 0 and K % 64 == 0, (
        f"mask-free kernel needs M,N divisible by 256 and K by 64 (got {M},{N},{K})"
    )
    assert a.dtype in (torch.float16, torch.bfloat16), "fp16 or bf16 inputs expected"
    return _pk.gemm_dense(a, b, torch.float32, 1)
