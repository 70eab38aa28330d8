"""The benchmark's plumbing configuration (W4A16, M=16, K=1024, N=1024, group 128 along K, fp16
scales, fp16 output with fp32 accumulation, seeded): the oracle against an independent
float64 dequantize-and-multiply on the CPU, and the HIP path against the oracle on the GPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

M, K, N, G = 16, 1024, 1024, 128


def _inputs():
    g = torch.Generator()
    g.manual_seed(0)
    a = torch.randn(M, K, generator=g).half()
    w = (torch.randn(K, N, generator=g) * 0.02).half()
    return a, w


def test_oracle_at_plumbing_config():
    """Codes in [-7, 7] with per-(group, column) scales max|w| / 7 in fp16; the oracle's
    product equals float64 arithmetic on the same codes and scales to fp32 rounding."""
    a, w = _inputs()
    codes, s32, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    assert codes.shape == (K, N) and s16.shape == (K // G, N)
    assert codes.min() >= -7 and codes.max() <= 7
    wf = w.numpy().astype(np.float64).reshape(K // G, G, N)
    np.testing.assert_allclose(s32, np.abs(wf).max(axis=1) / 7, rtol=1e-6)
    ref64 = a.numpy().astype(np.float64) @ (codes.astype(np.float64) *
                                            np.repeat(s16.astype(np.float64), G, axis=0))
    got = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    assert oracle.rel_fro(got, ref64) < 1e-6
    # codes are round-to-nearest against the fp32 scale (half a step from the weights); the
    # stored scale is that fp32 scale rounded to fp16
    step = np.repeat(s32.astype(np.float64), G, axis=0)
    deq = codes.astype(np.float64) * step
    assert np.all(np.abs(deq - w.numpy().astype(np.float64)) <= 0.5 * step * (1 + 1e-6))
    assert np.array_equal(s16, s32.astype(np.float16))


@pytest.mark.gpu
def test_hip_path_at_plumbing_config(cuda):
    import gemm_int4

    a, w = _inputs()
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), G)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    assert np.array_equal(qw.cpu().numpy().view(np.uint8), oracle.pack_int4_n(codes))
    assert np.array_equal(sc.cpu().numpy(), s16)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, G, out_dtype=torch.float16)
    assert out.dtype == torch.float16 and out.shape == (M, N)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    assert oracle.rel_fro(out.float().cpu().numpy(), ref) <= 1e-3
