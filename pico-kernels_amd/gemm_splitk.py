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


def check_correctness(M: int = 1024, K: int = 1024, N: int = 1024) -> None:
    """The reference's self-check (gemm_splitk.py:83-91): split-K 4 against the fp32 product."""
    torch.manual_seed(0)
    a = torch.randn(M, K, device="cuda", dtype=torch.float16)
    b = torch.randn(K, N, device="cuda", dtype=torch.float16)
    c = triton_gemm_splitk(a, b, split_k=4)
    ref = a.float() @ b.float()
    print(f"split-K vs fp32: max abs err {(c - ref).abs().max().item():.3e} | "
          f"allclose {torch.allclose(c, ref, atol=1e-2, rtol=1e-2)}")


def bench() -> None:
    """The reference's benchmark table (gemm_splitk.py:94-113): GFLOPS of the fp16 matmul
    (hipBLASLt through torch), the unsplit GEMM (gemm.triton_gemm) and split-K."""
    import gemm
    from _timing import do_bench

    print(f"{'shape (M,N,K)':>16} {'hipBLASLt':>10} {'unsplit':>10} {'split-K':>10}  note")
    print("-" * 64)
    cases = [
        (512, 512, 8192, 4, "tall-skinny"),
        (512, 512, 16384, 8, "tall-skinny"),
        (1024, 1024, 4096, 4, "square"),
        (4096, 4096, 4096, 4, "square"),
    ]
    for M, N, K, sk, note in cases:
        a = torch.randn(M, K, device="cuda", dtype=torch.float16)
        b = torch.randn(K, N, device="cuda", dtype=torch.float16)
        flops = 2 * M * N * K / 1e9
        ms_blas = do_bench(lambda: a @ b)
        ms_auto = do_bench(lambda: gemm.triton_gemm(a, b))
        ms_split = do_bench(lambda: triton_gemm_splitk(a, b, split_k=sk))
        fmt = lambda ms: f"{flops / (ms / 1e3):>7.0f} G"
        print(f"{(M, N, K)!s:>16} {fmt(ms_blas):>10} {fmt(ms_auto):>10} {fmt(ms_split):>10}  {note}")


if __name__ == "__main__":
    from _timing import banner

    print(banner())
    print("=== correctness ===")
    check_correctness()
    print("=== benchmark (GFLOPS) ===")
    bench()
