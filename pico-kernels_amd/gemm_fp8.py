"""Per-tensor-scaled fp8 (OCP e4m3) matmul on MI355X -- drop-in for the reference's
``gemm_fp8`` module.

Reference entry points kept with their signatures (file:line in the reference repository):
  * ``_E4M3_MAX``                                   gemm_fp8.py:24 (448.0)
  * ``quantize(x) -> (x_fp8, scale)``               gemm_fp8.py:89-95, ``x ~= x_fp8 / scale``
  * ``fp8_gemm_precast(a8, a_scale, b8, b_scale)``  gemm_fp8.py:98-117 -> (M, N) fp32
  * ``fp8_gemm(a, b)``                              gemm_fp8.py:120-124 -> (M, N) fp32

The matmul runs on the gfx950 fp8 matrix cores (v_mfma_f32_16x16x128_f8f6f4, e4m3 x e4m3,
fp32 accumulate) and applies ``1 / (a_scale * b_scale)`` once in the epilogue. The cast is a
HIP kernel reproducing torch's rounding chain bit for bit: ``x * scale`` is rounded to ``x``'s
dtype first, then to e4m3 with round-to-nearest-even and NaN on overflow.
"""

from __future__ import annotations

import torch

import _pk

__all__ = ["_E4M3_MAX", "quantize", "fp8_gemm_precast", "fp8_gemm", "check_correctness", "bench"]

_E4M3_MAX = float(torch.finfo(torch.float8_e4m3fn).max)


def quantize(x: torch.Tensor) -> tuple[torch.Tensor, float]:
    """Cast ``x`` to e4m3, scaled so ``max|x|`` maps to the e4m3 max.

    Returns ``(x_fp8, scale)`` where ``x ~= x_fp8 / scale`` (gemm_fp8.py:89-95).
    """
    xg = _pk.to_gpu(x)
    scale = _E4M3_MAX / _pk.absmax(xg).item()
    x8 = _pk.cast_e4m3(xg, scale)
    return (x8 if x.is_cuda else x8.to(x.device)), scale


def fp8_gemm_precast(a8: torch.Tensor, a_scale: float, b8: torch.Tensor, b_scale: float,
                     *, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Kernel-only fp8 matmul on already-cast ``a8 (M, K)``, ``b8 (K, N)``.

    Output fp32 by default (the reference's dtype); ``out_dtype`` may be fp16/bf16. A ``b8``
    that is the transposed view of a row-major ``(N, K)`` buffer is read in place.
    """
    M, K = a8.shape
    K2, N = b8.shape
    assert K == K2
    assert a8.is_cuda and b8.is_cuda, "fp8_gemm_precast: inputs must be on the GPU"
    assert a8.dtype == torch.float8_e4m3fn and b8.dtype == torch.float8_e4m3fn
    out_scale = 1.0 / (a_scale * b_scale)
    return _pk.fp8_gemm(a8, b8, out_scale, out_dtype)


def fp8_gemm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Convenience: quantize then matmul (the full fp8 path, gemm_fp8.py:120-124)."""
    a8, a_scale = quantize(a)
    b8, b_scale = quantize(b)
    return fp8_gemm_precast(a8, a_scale, b8, b_scale)


def _harness_checks() -> list:
    """Self-check at the reference's check shape (gemm_fp8.py:127-136: 1024^3, N(0,1) fp16):
    ``fp8_gemm`` against the fp32 product. Its relative Frobenius error is the e4m3 rounding
    of both operands, ~3.7% for N(0,1) data (the reference reports 3.74%)."""
    from _timing import Check

    def measure():
        g = torch.Generator(device="cuda").manual_seed(0)
        a = torch.randn(1024, 1024, device="cuda", dtype=torch.float16, generator=g)
        b = torch.randn(1024, 1024, device="cuda", dtype=torch.float16, generator=g)
        y = fp8_gemm(a, b)
        exact = a.float() @ b.float()
        return {"rel_fro": (torch.linalg.norm(y - exact) / torch.linalg.norm(exact)).item(),
                "max_abs_err": (y - exact).abs().max().item()}

    return [Check("fp8_gemm_1024^3", measure, {"rel_fro": (0.02, 0.06)})]


def _harness_rows() -> list:
    """The reference's benchmark sizes (gemm_fp8.py:139-156): square fp16 matmul through torch
    (hipBLASLt) against ``fp8_gemm_precast`` on operands cast once, outside the timing."""
    from _timing import Row

    def build(n):
        def make():
            a = torch.randn(n, n, device="cuda", dtype=torch.float16)
            b = torch.randn(n, n, device="cuda", dtype=torch.float16)
            (a8, sa), (b8, sb) = quantize(a), quantize(b)
            return {"torch_fp16": lambda: a @ b,
                    "fp8_gemm_precast": lambda: fp8_gemm_precast(a8, sa, b8, sb)}
        return make

    return [Row(f"M=N=K={n}", build(n), 2.0 * n ** 3) for n in (512, 1024, 2048, 4096)]


def check_correctness() -> bool:
    """Run and print the module's self-check (see ``_harness_checks``)."""
    from _timing import run_checks

    return run_checks("gemm_fp8", _harness_checks())


def bench() -> None:
    """Time and print the module's benchmark rows (see ``_harness_rows``)."""
    from _timing import run_rows

    run_rows("gemm_fp8", _harness_rows())


if __name__ == "__main__":
    import sys

    from _timing import main

    sys.exit(main("gemm_fp8", _harness_checks(), _harness_rows()))
