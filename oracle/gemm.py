"""numpy GEMM references of the reference's own tests -- TEST INFRASTRUCTURE ONLY.

These are the closed forms the reference checks its kernels against; they are what the HIP
GEMMs are compared with (within tolerance, since fp32 summation order differs).
"""

from __future__ import annotations

import numpy as np

from .quant import e4m3_to_f32


def rel_fro(x: np.ndarray, ref: np.ndarray) -> float:
    """||x - ref||_F / ||ref||_F in float64 (gemm_int4.py:103, tests/test_gemm_fp8.py:25)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / np.linalg.norm(ref))


def int4_gemm_ref(a: np.ndarray, codes: np.ndarray, scale: float) -> np.ndarray:
    """``a.float() @ (w_q.float() * scale)`` (tests/test_gemm_int4.py:26, gemm_int4.py:102)."""
    return np.asarray(a, dtype=np.float32) @ (np.asarray(codes, dtype=np.float32) * np.float32(scale))


def w4a16_ref(a: np.ndarray, codes: np.ndarray, scales: np.ndarray, group_size: int = 128,
              tensor_scale: float = 1.0) -> np.ndarray:
    """Dequantize + fp32 matmul for the group format:
    ``a.float() @ (q.float() * scales.float().repeat_interleave(G, 0))`` -- the W4A16 bar of
    the path (test closed form of tests/test_gemm_int4.py:26 with group scales)."""
    K = codes.shape[0]
    s = np.repeat(np.asarray(scales, dtype=np.float32), group_size, axis=0)[:K]
    w = np.asarray(codes, dtype=np.float32) * s
    out = np.asarray(a, dtype=np.float32) @ w
    return out * np.float32(tensor_scale) if tensor_scale != 1.0 else out


def fp8_gemm_ref(a8: np.ndarray, a_scale: float, b8: np.ndarray, b_scale: float) -> np.ndarray:
    """``(a8.float() @ b8.float()) * out_scale`` with out_scale = 1/(a_scale*b_scale)
    narrowed to fp32 (gemm_fp8.py:86, 106)."""
    out_scale = np.float32(1.0 / (a_scale * b_scale))
    return (e4m3_to_f32(a8) @ e4m3_to_f32(b8)) * out_scale


def splitk_ref(a: np.ndarray, b: np.ndarray, split_k: int) -> np.ndarray:
    """Split-K semantics of gemm_splitk.py:49-53, 64: K cut into split_k contiguous slices of
    K // split_k rows, fp32 partial products summed (in slice order here)."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    K = a.shape[1]
    ks = K // split_k
    out = np.zeros((a.shape[0], b.shape[1]), dtype=np.float32)
    for s in range(split_k):
        out += a[:, s * ks:(s + 1) * ks] @ b[s * ks:(s + 1) * ks]
    return out
