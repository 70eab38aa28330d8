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


def check_correctness(M: int = 1024, K: int = 1024, N: int = 1024) -> None:
    """The reference's self-check (gemm_fp8.py:127-136): fp8_gemm against the fp32 product."""
    torch.manual_seed(0)
    a = torch.randn(M, K, device="cuda", dtype=torch.float16)
    b = torch.randn(K, N, device="cuda", dtype=torch.float16)
    c = fp8_gemm(a, b)
    ref = a.float() @ b.float()
    rel_fro = torch.norm(c - ref) / torch.norm(ref)
    print(f"fp8 vs fp32: rel Frobenius err {rel_fro.item():.4%} | "
          f"max abs err {(c - ref).abs().max().item():.3e}")


def bench() -> None:
    """The reference's benchmark table (gemm_fp8.py:139-156): GFLOPS of the fp16 matmul
    (hipBLASLt through torch) and of fp8_gemm_precast (cast done once, untimed)."""
    from _timing import do_bench

    print(f"{'size':>7} {'fp16 hipBLASLt':>14} {'fp8 HIP':>12} {'speedup':>8}")
    print("-" * 46)
    for size in (512, 1024, 2048, 4096):
        a = torch.randn(size, size, device="cuda", dtype=torch.float16)
        b = torch.randn(size, size, device="cuda", dtype=torch.float16)
        a8, a_scale = quantize(a)
        b8, b_scale = quantize(b)
        flops = 2 * size**3 / 1e9
        ms_fp16 = do_bench(lambda: a @ b)
        ms_fp8 = do_bench(lambda: fp8_gemm_precast(a8, a_scale, b8, b_scale))
        g_fp16 = flops / (ms_fp16 / 1e3)
        g_fp8 = flops / (ms_fp8 / 1e3)
        print(f"{size:>7} {g_fp16:>11.0f} G {g_fp8:>9.0f} G {g_fp8 / g_fp16:>7.2f}x")


if __name__ == "__main__":
    from _timing import banner

    print(banner())
    print("=== correctness (fp8 vs fp32 reference) ===")
    check_correctness()
    print("=== benchmark (GFLOPS - higher is better; cast is pre-done) ===")
    bench()
