"""Packed INT4 (W4A16) matmul on MI355X -- drop-in for the reference's ``gemm_int4`` module.

Reference entry points kept with their signatures (file:line in the reference repository):
  * ``quantize_int4(w)``      gemm_int4.py:58-62  -> (int8 codes, Python float scale)
  * ``pack_int4_n(w_q)``      gemm_int4.py:65-72  -> (K, N//2) uint8, low nibble = even column
  * ``int4_gemm(a, w_packed, scale, BLOCK_M=64, BLOCK_N=64, BLOCK_K=64)``
                              gemm_int4.py:75-92  -> (M, N) fp32 = a @ (W_int4 * scale)

Additions of this build (the group-128 W4A16 path):
  * ``unpack_int4_n(w_packed)``            inverse of pack_int4_n (the kernel's unpack,
                                           gemm_int4.py:44-49)
  * ``quantize_int4_group(w, group_size)`` RTN codes + fp16 scales with quantize.rtn_layer
                                           semantics (quantize.py:42-68), packed as int32
  * ``w4a16_gemm(a, qweight, scales, ...)`` fused-dequant matmul with deterministic split-K

All compute runs in the HIP library (``libpico_kernels_amd.so``); there is no Triton and no
CPU fallback. Host tensors given to the quantization helpers are staged through the GPU.
"""

from __future__ import annotations

import torch

import _pk

__all__ = [
    "quantize_int4",
    "pack_int4_n",
    "unpack_int4_n",
    "int4_gemm",
    "quantize_int4_group",
    "dequantize_int4_group",
    "w4a16_gemm",
    "check_correctness",
    "bench",
]


def quantize_int4(w: torch.Tensor) -> tuple[torch.Tensor, float]:
    """Per-tensor symmetric int4 quantization of ``w`` (fp16/bf16/fp32).

    Same numbers as the reference (gemm_int4.py:58-62): ``scale = max|w| / 7.0`` in Python
    double; codes ``round(w / scale).clamp(-8, 7)`` where the quotient is rounded to ``w``'s
    dtype before the round-half-even, exactly as the torch expression does on a CPU tensor.
    """
    wg = _pk.to_gpu(w)
    absmax = _pk.absmax(wg).item()
    scale = absmax / 7.0
    q = _pk.quantize_int4(wg, scale)
    return (q if w.is_cuda else q.to(w.device)), scale


def pack_int4_n(w_q: torch.Tensor) -> torch.Tensor:
    """Pack signed int4 weights 2-per-byte along N -> (K, N//2) uint8 (gemm_int4.py:65-72)."""
    K, N = w_q.shape
    assert N % 2 == 0
    q = _pk.to_gpu(w_q)
    if q.dtype != torch.int8:
        q = q.to(torch.int8)
    out = _pk.pack_int4(q)
    return out if w_q.is_cuda else out.to(w_q.device)


def unpack_int4_n(w_packed: torch.Tensor) -> torch.Tensor:
    """(K, N//2) uint8 -> (K, N) int8 codes in [-8, 7] (sign-extended nibbles)."""
    assert w_packed.dtype == torch.uint8 and w_packed.dim() == 2
    out = _pk.unpack_int4(_pk.to_gpu(w_packed))
    return out if w_packed.is_cuda else out.to(w_packed.device)


def int4_gemm(a: torch.Tensor, w_packed: torch.Tensor, scale: float,
              BLOCK_M: int = 64, BLOCK_N: int = 64, BLOCK_K: int = 64) -> torch.Tensor:
    """``a @ (W_int4 * scale)`` where ``w_packed`` is ``(K, N//2)`` uint8 (gemm_int4.py:75-92).

    Returns a new fp32 ``(M, N)`` tensor. The ``BLOCK_*`` arguments are accepted for
    signature compatibility; tiles are chosen by the library. Unlike the reference kernel,
    any M is valid (no out-of-bounds rows); N must be a multiple of 8 and K of 32.

    bf16 activations (admitted by the reference wrapper, gemm_int4.py:78) are converted to
    fp16 in one pass (``pk_w4a16_prep_activations``) and run on the fp16 kernels: the
    conversion is exact for 2^-17 <= |x| <= 65504 (and 0), so there the products with the
    exact integer codes, and the fp32 sums, are those of a bf16 dot; smaller magnitudes keep
    fp16's subnormal precision. A finite bf16 activation above 65504 raises ``ValueError``
    (checked with one device reduction, except while a graph is being captured).
    """
    assert a.is_cuda and a.dtype in (torch.float16, torch.bfloat16)
    M, K = a.shape
    K2, N_half = w_packed.shape
    assert K2 == K, "int4_gemm: w_packed must be (K, N//2) for a of shape (M, K)"
    if a.dtype == torch.bfloat16:
        _pk.check_fp16_range(a, "int4_gemm")
        a = _pk.w4a16_prep_activations(a, None, 1.0)
    N = N_half * 2
    assert N % 8 == 0, "int4_gemm: N must be a multiple of 8 (whole int32 words)"
    wp = w_packed if w_packed.is_cuda else w_packed.to(a.device)
    if not wp.is_contiguous():
        wp = wp.contiguous()
    qweight = wp.view(torch.int32)  # (K, N//8): pack_int4_n bytes are the int32 words
    return _pk.w4a16_gemm(a, qweight, None, 0, float(scale), torch.float32)


def quantize_int4_group(w: torch.Tensor, group_size: int = 128
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """Group-wise int4 quantization of a ``(K, N)`` weight along K.

    Codes and scales follow ``quantize.rtn_layer(w, 4, group_size)`` (quantize.py:42-68):
    per column and per group of ``group_size`` consecutive k, ``s = max|w|.clamp_min(1e-12)/7``
    in fp32 and ``q = clamp(round(w / s), -7, 7)``. Returns
      * ``qweight``: ``(K, N//8)`` int32, byte-identical to ``pack_int4_n(q)``,
      * ``scales``:  ``(ceil(K/group_size), N)`` fp16 (``s`` rounded to nearest even).
    """
    assert w.dim() == 2
    K, N = w.shape
    assert N % 8 == 0, "quantize_int4_group: N must be a multiple of 8"
    wg = _pk.to_gpu(w)
    qweight, scales, _ = _pk.quantize_group(wg, 4, group_size, half_math=False, want_qweight=True,
                                            want_scales=True, want_fake=False)
    if not w.is_cuda:
        qweight, scales = qweight.to(w.device), scales.to(w.device)
    return qweight, scales


def dequantize_int4_group(qweight: torch.Tensor, scales: torch.Tensor, group_size: int = 128
                          ) -> torch.Tensor:
    """``(K, N)`` fp32 weights ``q * scale`` of the packed group format (for inspection)."""
    q = unpack_int4_n(qweight.contiguous().view(torch.uint8)).float()
    s = scales.float().repeat_interleave(group_size, 0)[: q.shape[0]]
    return q * s.to(q.device)


def w4a16_gemm(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
               group_size: int = 128, split_k: int | None = None,
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """``a @ (q * scales)`` for the packed group format, fp32 accumulation.

    ``a``: (M, K) fp16 on the GPU; ``qweight``: (K, N//8) int32; ``scales``: (K//group, N)
    fp16. ``split_k=None`` lets the library choose; an explicit ``split_k`` splits K into
    that many contiguous slices (each a whole number of groups) reduced in a fixed order, so
    the result is reproducible bit for bit. ``out_dtype`` is fp16 (default), bf16 or fp32.
    """
    assert a.is_cuda and a.dtype == torch.float16, "w4a16_gemm: a must be fp16 on the GPU"
    assert qweight.dtype == torch.int32 and qweight.dim() == 2
    M, K = a.shape
    assert qweight.shape[0] == K, "w4a16_gemm: qweight must be (K, N//8)"
    N = qweight.shape[1] * 8
    assert scales.dtype == torch.float16 and tuple(scales.shape) == (K // group_size, N), (
        "w4a16_gemm: scales must be fp16 (K//group_size, N)")
    return _pk.w4a16_gemm(a, qweight, scales, group_size, 1.0, out_dtype,
                          split_k=0 if split_k is None else int(split_k))


def _harness_checks() -> list:
    """Self-check of the per-tensor path at the reference's check shape (gemm_int4.py:95-104:
    128 x 256 x 256, N(0,1) fp16): the relative Frobenius error of ``int4_gemm`` against the
    fp32 product of the dequantised weights, which the fused kernel reproduces to fp32
    rounding."""
    from _timing import Check

    def measure():
        g = torch.Generator(device="cuda").manual_seed(0)
        a = torch.randn(128, 256, device="cuda", dtype=torch.float16, generator=g)
        w = torch.randn(256, 256, device="cuda", dtype=torch.float16, generator=g)
        codes, s = quantize_int4(w)
        y = int4_gemm(a, pack_int4_n(codes), s)
        exact = a.float() @ (codes.float() * s)
        return {"rel_fro": (torch.linalg.norm(y - exact) / torch.linalg.norm(exact)).item()}

    return [Check("int4_gemm_per_tensor_128x256x256", measure, {"rel_fro": (None, 1e-4)})]


def _harness_rows() -> list:
    """The reference's four benchmark shapes (gemm_int4.py:107-130), rates of torch's fp16
    matmul (hipBLASLt) and of ``int4_gemm`` on the same operands."""
    from _timing import Row

    def build(M, N, K):
        def make():
            a = torch.randn(M, K, device="cuda", dtype=torch.float16)
            codes, s = quantize_int4(torch.randn(K, N, device="cuda", dtype=torch.float16))
            wp = pack_int4_n(codes)
            wd = codes.half() * s
            return {"torch_fp16": lambda: a @ wd, "int4_gemm": lambda: int4_gemm(a, wp, s)}
        return make

    shapes = ((16, 4096, 4096, "decode"), (16, 8192, 8192, "decode"),
              (1024, 4096, 4096, "mixed"), (4096, 4096, 4096, "compute"))
    return [Row(f"M={M},N={N},K={K}", build(M, N, K), 2.0 * M * N * K, note)
            for M, N, K, note in shapes]


def check_correctness() -> bool:
    """Run and print the module's self-check (see ``_harness_checks``)."""
    from _timing import run_checks

    return run_checks("gemm_int4", _harness_checks())


def bench() -> None:
    """Time and print the module's benchmark rows (see ``_harness_rows``)."""
    from _timing import run_rows

    run_rows("gemm_int4", _harness_rows())


if __name__ == "__main__":
    import sys

    from _timing import main

    sys.exit(main("gemm_int4", _harness_checks(), _harness_rows()))
