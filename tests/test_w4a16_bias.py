"""pk_w4a16_gemm_bias: the bias added where each W4A16 kernel stores its output (GEMV epilogue
and its in-L2 split-K handoff, the register-dequant kernel's epilogue and handoff, the
packed-B GEMM unsplit and through the reduce launch, the LDS-tiled GEMMs). The fused result
is tensor_scale * (A @ W) + bias in fp32, rounded once: bitwise what adding the bias to the
fp32 output of pk_w4a16_gemm and rounding gives, and within the oracle's tolerance of the
reference linear layer (x @ w + b)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import _pk
import gemm_int4
import oracle


def _case(M, K, N, seed, cuda):
    g = torch.Generator()
    g.manual_seed(seed)
    a = torch.randn(M, K, generator=g).half()
    w = (torch.randn(K, N, generator=g) * 0.02).half()
    bias = torch.randn(N, generator=g) * 0.5
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), 128)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, 128)
    return a, qw, sc, bias, codes, s16


# (M, K, N, split_k, kernel id): every output path of the W4A16 dispatch
PATHS = [
    (1, 4096, 4096, 0, _pk.KERNEL_GEMV),      # MFMA GEMV, slices added in L2
    (3, 1024, 1032, 0, _pk.KERNEL_GEMV),      # VALU GEMV (N % 32 != 0) + reduce launch
    (2, 2048, 1024, 1, _pk.KERNEL_GEMV),      # GEMV unsplit
    (8, 4096, 2048, 0, _pk.KERNEL_SKINNY),    # register-dequant, slices added in L2
    (32, 4096, 2048, 0, _pk.KERNEL_SKINNY),   # register-dequant + reduce launch
    (100, 2048, 1040, 0, _pk.KERNEL_SKINNY),  # two row parts
    (128, 1024, 768, 0, _pk.KERNEL_GEMM_TR4),  # packed-B split-K + reduce launch
    (256, 512, 512, 1, _pk.KERNEL_GEMM_TR4),  # packed-B unsplit (staged epilogue)
    (256, 1024, 1152, 0, _pk.KERNEL_GEMM),    # LDS-dequant large tiles, split-K
    (300, 512, 1160, 1, _pk.KERNEL_GEMM),     # LDS-dequant large tiles, unsplit, ragged
    (40, 1024, 520, 0, _pk.KERNEL_GEMM),      # small-tile GEMM (N % 16 != 0)
    (24, 4096, 3072, 1, _pk.KERNEL_SKINNY),   # group-spanning waves (4 groups), unsplit
    (32, 8192, 1280, 4, _pk.KERNEL_SKINNY),   # group-spanning waves, slices added in L2
    (40, 4096, 11008, 0, _pk.KERNEL_GEMM_TR4),  # 33..64 rows of a large layer: packed-B
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,split,kid", PATHS)
def test_bias_fused_on_every_path(M, K, N, split, kid, cuda):
    a, qw, sc, bias, codes, s16 = _case(M, K, N, 900 + M + N, cuda)
    assert _pk.w4a16_plan(M, N, K, 128, split)[0] == kid
    ag = a.to(cuda)
    f32 = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32, split_k=split)
    for bdt in (torch.float32, torch.float16, torch.bfloat16):
        b = bias.to(bdt).to(cuda)
        for out_dtype in (torch.float32, torch.float16, torch.bfloat16):
            got = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, out_dtype, split_k=split, bias=b)
            want = (f32 + b.float()).to(out_dtype)
            assert torch.equal(got, want), (bdt, out_dtype)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128) + bias.numpy()
    got = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32, split_k=split, bias=bias.to(cuda))
    assert oracle.rel_fro(got.cpu().numpy(), ref) < 1e-3


@pytest.mark.gpu
def test_bias_with_tensor_scale_and_out_view(cuda):
    """Per-tensor mode: the tensor scale multiplies the product, not the bias; an output view
    wider than N keeps its margins."""
    g = torch.Generator()
    g.manual_seed(31)
    M, K, N = 4, 1024, 512
    a = torch.randn(M, K, generator=g).half()
    q = torch.randint(-8, 8, (K, N), generator=g, dtype=torch.int8)
    packed = torch.from_numpy(oracle.pack_int4_n(q.numpy()).view(np.int32).copy()).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.25).to(cuda)
    ag = a.to(cuda)
    got = _pk.w4a16_gemm(ag, packed, None, 0, 0.037, torch.float32, bias=bias)
    ref = (a.double().numpy() @ q.double().numpy()) * 0.037 + bias.double().cpu().numpy()
    assert oracle.rel_fro(got.cpu().numpy(), ref) < 1e-5
    big = torch.full((M, N + 256), 9.0, dtype=torch.float16, device=cuda)
    _pk.w4a16_gemm(ag, packed, None, 0, 0.037, torch.float16, out=big[:, 128:128 + N], bias=bias)
    assert torch.equal(big[:, 128:128 + N], got.half())
    assert torch.all(big[:, :128] == 9.0) and torch.all(big[:, 128 + N:] == 9.0)


def test_bias_argument_errors():
    """A bias dtype code other than fp32 / fp16 / bf16 is rejected before any GPU work; the
    Python wrapper checks the bias length and dtype."""
    lib = _pk.lib()
    rc = lib.pk_w4a16_gemm_bias(ctypes.c_void_p(16), 64, ctypes.c_void_p(16), 8, None, 0, 1.0,
                                ctypes.c_void_p(16), 7, ctypes.c_void_p(16), _pk.PK_F16, 64,
                                1, 64, 64, 0, None, 0, None)
    assert rc == _pk.PK_EINVAL
    assert b"bias dtype" in lib.pk_last_error()
    with pytest.raises(ValueError):
        _pk.w4a16_gemm(torch.zeros(1, 64, dtype=torch.float16),
                       torch.zeros(64, 8, dtype=torch.int32), None, 0, 1.0, torch.float16,
                       bias=torch.zeros(32, dtype=torch.float16))
