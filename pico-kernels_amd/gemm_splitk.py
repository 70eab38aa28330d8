"""Split-K fp16 matmul on MI355X -- drop-in for the reference's ``gemm_splitk`` module.

Reference entry point kept with its signature (gemm_splitk.py:67-80):
  ``triton_gemm_splitk(a, b, split_k=4, BLOCK_M=128, BLOCK_N=128, BLOCK_K=64) -> (M, N) fp32``

K is split into ``split_k`` contiguous slices of ``K // split_k`` rows (gemm_splitk.py:49-53)
and the same divisibility contract is asserted (gemm_splitk.py:71). fp16 and bf16 inputs are
served (the reference's ``tl.dot`` takes either). The reference adds the slices with fp32
atomics; here each slice writes an fp32 partial tile and a second launch adds them in slice
order, so the output is reproducible bit for bit. The name keeps ``triton_`` only for
drop-in compatibility: the kernel is hand-written HIP (MFMA).
"""

from __future__ import annotations

import torch

import _pk

__all__ = ["triton_gemm_splitk", "check_correctness", "bench"]


def triton_gemm_splitk(a: torch.Tensor, b: torch.Tensor, split_k: int = 4,
                       BLOCK_M: int = 128, BLOCK_N: int = 128, BLOCK_K: int = 64) -> torch.Tensor:
    M, K = a.shape
    K2, N = b.shape
    assert K == K2 and K % (split_k * BLOCK_K) == 0, "K must divide split_k * BLOCK_K"
    assert a.is_cuda and b.is_cuda, "triton_gemm_splitk: inputs must be on the GPU"
    assert a.dtype == b.dtype and a.dtype in (torch.float16, torch.bfloat16), \
        "fp16 or bf16 inputs expected"
    return _pk.gemm_dense(a, b, torch.float32, split_k)


def _harness_checks() -> list:
    """Self-check at the reference's check shape (gemm_splitk.py:83-91: 1024^3, split 4):
    the split-K product against the fp32 product, max absolute error and torch.allclose at
    atol = rtol = 1e-2."""
    from _timing import Check

    def measure():
        g = torch.Generator(device="cuda").manual_seed(0)
        a = torch.randn(1024, 1024, device="cuda", dtype=torch.float16, generator=g)
        b = torch.randn(1024, 1024, device="cuda", dtype=torch.float16, generator=g)
        y = triton_gemm_splitk(a, b, split_k=4)
        exact = a.float() @ b.float()
        return {"max_abs_err": (y - exact).abs().max().item(),
                "allclose_1e-2": bool(torch.allclose(y, exact, atol=1e-2, rtol=1e-2))}

    return [Check("splitk4_1024^3", measure, {"allclose_1e-2": (True, True)})]


def _harness_rows() -> list:
    """The reference's benchmark shapes and splits (gemm_splitk.py:94-113): torch's fp16
    matmul (hipBLASLt), the unsplit ``gemm.triton_gemm`` and ``triton_gemm_splitk``."""
    from _timing import Row

    def build(M, N, K, sk):
        def make():
            import gemm

            a = torch.randn(M, K, device="cuda", dtype=torch.float16)
            b = torch.randn(K, N, device="cuda", dtype=torch.float16)
            return {"torch_fp16": lambda: a @ b, "unsplit": lambda: gemm.triton_gemm(a, b),
                    f"split{sk}": lambda: triton_gemm_splitk(a, b, split_k=sk)}
        return make

    shapes = ((512, 512, 8192, 4, "tall-skinny"), (512, 512, 16384, 8, "tall-skinny"),
              (1024, 1024, 4096, 4, "square"), (4096, 4096, 4096, 4, "square"))
    return [Row(f"M={M},N={N},K={K}", build(M, N, K, sk), 2.0 * M * N * K, note)
            for M, N, K, sk, note in shapes]


def check_correctness() -> bool:
    """Run and print the module's self-check (see ``_harness_checks``)."""
    from _timing import run_checks

    return run_checks("gemm_splitk", _harness_checks())


def bench() -> None:
    """Time and print the module's benchmark rows (see ``_harness_rows``)."""
    from _timing import run_rows

    run_rows("gemm_splitk", _harness_rows())


if __name__ == "__main__":
    import sys

    from _timing import main

    sys.exit(main("gemm_splitk", _harness_checks(), _harness_rows()))
