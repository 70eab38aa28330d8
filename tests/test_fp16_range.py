"""bf16 / fp32 activations beyond fp16's range. The W4A16 kernels take their activations as
fp16 (the reference wrapper admits bf16, gemm_int4.py:78); a finite value above 65504 would
become an infinity in that cast, so ``int4_gemm`` and ``QuantLinear`` raise ``ValueError``
instead (``QuantLinear.range_check = False`` keeps torch's own cast semantics: infinities)."""

from __future__ import annotations

import pytest
import torch

import _pk


def test_range_check_host_logic():
    ok = torch.tensor([65504.0, -65504.0, 1e-30, float("inf"), float("nan")])
    _pk.check_fp16_range(ok, "t")                       # the edge itself, non-finite inputs
    _pk.check_fp16_range(ok.to(torch.bfloat16), "t")
    with pytest.raises(ValueError, match="exceed fp16's range"):
        _pk.check_fp16_range(torch.tensor([1.0, 70000.0]), "t")
    with pytest.raises(ValueError):
        _pk.check_fp16_range(torch.tensor([-1e5], dtype=torch.bfloat16), "t")
    # given the converted tensor, only finite inputs that turned infinite count
    x = torch.tensor([1e5, 2.0])
    _pk.check_fp16_range(x, "t", torch.tensor([1.0, 2.0], dtype=torch.float16))
    with pytest.raises(ValueError):
        _pk.check_fp16_range(x, "t", x.half())
    _pk.check_fp16_range(torch.tensor([7e4]).half(), "t")  # already fp16: nothing to check


@pytest.mark.gpu
def test_int4_gemm_bf16_overflow_raises(cuda):
    import gemm_int4

    g = torch.Generator().manual_seed(0)
    w = torch.randn(256, 64, generator=g).half()
    codes, s = gemm_int4.quantize_int4(w.to(cuda))
    wp = gemm_int4.pack_int4_n(codes)
    a = torch.randn(4, 256, generator=g).to(torch.bfloat16).to(cuda)
    y = gemm_int4.int4_gemm(a, wp, s)                    # in range: computed
    ref = a.float() @ (codes.float() * s)
    assert torch.linalg.norm(y - ref) / torch.linalg.norm(ref) < 1e-3
    a[2, 17] = 1.0e5
    with pytest.raises(ValueError, match="exceed fp16's range"):
        gemm_int4.int4_gemm(a, wp, s)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quant_linear_overflow(dtype, cuda):
    from torch import nn

    import quant_linear as ql

    lin = nn.Linear(256, 256, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(256, 256, generator=torch.Generator().manual_seed(1)) * 0.02)
    q = ql.QuantLinear.from_linear(lin.to(cuda), 128)
    x = torch.ones(2, 256, device=cuda, dtype=dtype)
    assert torch.isfinite(q(x)).all()
    x[1, 5] = 2.0e5
    with pytest.raises(ValueError, match="exceed fp16's range"):
        q(x)
    q.range_check = False
    y = q(x)
    assert torch.isfinite(y[0]).all() and not torch.isfinite(y[1]).all()
